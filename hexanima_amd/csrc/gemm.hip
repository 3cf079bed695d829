// Weight-only-quantised / fp16 GEMM for gfx950: O[M][N] = A[M][K] . W[N][K]^T with fused epilogues.
//
// Replaces the reference's HMX GEMM engine (hexagon/mega/gemm2.c:96-137, gemm_run_geo) including its q8 tile
// dequantisation (gemm2.c:19-35 dq_tile), the MOSS q4a dequantisation (moss/hexagon/mega/gemm2.c:39-56) and the
// flush epilogues (gemm2.c:58-82: gated residual, GELU, split-K residual partial; moss mode 5 SiTU).
//
// Design (CDNA4, 64-wide waves):
//  * 256 threads = 4 waves in a 2x2 grid; each wave owns a (BM/2)x(BN/2) sub-tile computed with
//    v_mfma_f32_32x32x16_f16 (fp32 accumulate).
//  * K is consumed in steps of 32 (one quantisation group). A and W k-tiles go from global memory straight into a
//    4-stage LDS ring (global_load_lds_dwordx4, no VGPR staging), 3 steps ahead of the MFMAs; one s_barrier per
//    step, with explicit vmcnt waits so the prefetches stay in flight. 16-byte LDS chunks are XOR-swizzled per row
//    so the fragment reads of 32 consecutive rows hit distinct banks.
//  * int8 / int4 weights stay raw in LDS and are dequantised into the B fragments in registers with the fp16
//    exponent-bias trick: a byte u placed under the exponent 0x64 is the fp16 value 1024+u, so (1024+u) - 1152 = q
//    exactly, then one fp16 multiply by the group scale gives f16(q*s) -- the reference's exact dequantised value
//    (gemm2.c:19-22).
//  * The fp16-rounded output tile is staged through LDS for a coalesced epilogue (16-byte loads / stores).
//  * The block index is remapped so each of the 8 XCDs (own L2) works on a contiguous range of output tiles.
#include <mutex>
#include <type_traits>

#include "hxa_common.h"
#include "kernels.h"

namespace {


struct GemmParams {
  const hxa_h *A;
  long lda;
  const void *W;
  const hxa_h *S, *Z;
  // W element (fp16 / int8; q4: byte) offset of row n, k group g: n * w_rs + g * w_gs. Row-major [N][K]: w_rs = K
  // (q4: K/2), w_gs = 32 (16); k-tiled [K/32][N][32] (q4: [K/32][N][16 bytes]): w_rs = 32 (16), w_gs = 32 N (16 N)
  long w_rs, w_gs;
  int M, N, Kslice, Ktot;
  int epi;
  hxa_h *out;
  long ldo, out_zstride;
  float *out32;  // PARTIAL_F32: slice z's fp32 sums at out32[z * out_zstride + m * ldo + n]
  float *x;
  long ldx;
  const float *gate;
  hxa_h *out_t;  // columns >= split_col go transposed to out_t[n - split_col][m]
  long ldo_t;
  int split_col;
  int tiles_m, tiles_n;
  // XCD placement: workgroup b runs on XCD b % 8. xcd_gm > 0: the tile grid is cut into 8 equal rectangles, xcd_gm
  // along M, and XCD x takes rectangle x (M-fastest inside); 0: XCD x takes the x-th eighth of the M-fastest order
  int xcd_gm;
  // head norm (STORE epilogue): columns [0, hn_cols), in whole heads of 128, get RMSNorm * gain and optional RoPE
  int hn_cols, hn_gsplit, hn_ttab;
  const float *hn_g0, *hn_g1, *hn_cos, *hn_sin;
  const uint8_t *pf;  // bytes to touch after the main loop (HxaGemm::pf)
  long pf_bytes;
  HxaClk clk;  // shader-clock record (hxa_clock_record), indexed by the launch's flat workgroup id
  const hxa_h *erf_t2;  // GELU-erf: T2 of every non-negative fp16 bit pattern (null: evaluated in the epilogue)
  int erf_lds;          // > 0: byte offset in LDS where the epilogue copies the table's first ERF_T2_LDS_N values
  // fused cross attention (gemm_xattn_kernel): the tile's queries attend to image (m0 / xa_T)'s keys
  // xa_k [NKV][xa_ldk] (+ image * xa_kb), V^T xa_vt [D][xa_ldvt] (+ image * xa_vb); O to xa_o [M][xa_ldo]
  const hxa_h *xa_k, *xa_vt;
  hxa_h *xa_o;
  long xa_ldk, xa_ldvt, xa_ldo, xa_kb, xa_vb;
  int xa_nkv, xa_nvalid, xa_T;
  // side_wgs > 0 (ping-pong kernel, one K slice): workgroups past the tile grid run side's GEMV rows
  HxaSideGemv side;
  int side_wgs;
};

// Touch this workgroup's share of [p.pf, p.pf + p.pf_bytes), one 4-byte load per 128-byte line: the lines come into
// L2 / MALL for the next kernel while this one runs its epilogue. The loads go straight to LDS (no register is
// written behind the compiler's back) into `sink`, PF_LDS bytes past everything the kernel uses, whose contents are
// never read; the workgroup drains them (vmcnt 0) before it ends, as every LDS DMA must.
HXA_DEV void prefetch_share(const GemmParams &p, int wg, int nwg, int tid, int nt, const uint8_t *sink) {
  const long lines = (p.pf_bytes + 127) >> 7;
  const long per = (lines + nwg - 1) / nwg;
  const long l0 = (long)wg * per, l1 = min(lines, l0 + per);
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)sink);
  for (long l = l0 + tid; l < l1; l += nt) {
    const uint8_t *a = p.pf + min(l << 7, p.pf_bytes - 4);  // pf_bytes >= 4 (checked on the host)
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(a), "s"(la) : "memory", "m0");
  }
}

// tile (tm, tn) of workgroup bid
// Byte offsets of one lane's 16-byte load chunks from the tile corner (row m0 of A / row n0 of W, k group 0). They
// are the same for every k tile, so the loaders compute them once and then issue each load as a wave-uniform base
// (moved per k tile, in SGPRs) plus this offset: no per-lane 64-bit address arithmetic in the k loop. Rows past
// the end are clamped to the last row. A chunk: 16 rows x 64 B per 1 KB block, swizzle c ^ ((row >> 2) & 3).
HXA_DEV uint32_t a_lane_off(const GemmParams &p, int blk, int lane, int m0) {
  const int row = blk * 16 + (lane >> 2), cl = (lane & 3) ^ ((row >> 2) & 3);
  return ((uint32_t)(min(m0 + row, p.M - 1) - m0) * (uint32_t)p.lda + cl * 8) * 2u;
}
// q8 rows of a stage are 32 B: chunk c of row r sits at 16-byte unit 2 r + (c ^ q8_swz(r))
HXA_DEV int q8_swz(int row) { return (row >> 3) & 1; }
// W chunk c of a stage: fp16 rows of 64 B (4 chunks), q8 rows of 32 B (2 chunks), q4 rows of 16 B (1 chunk)
template <int FMT>
HXA_DEV uint32_t w_lane_off(const GemmParams &p, int chunk, int n0) {
  if constexpr (FMT == HXA_W_F16) {
    const int row = chunk >> 2, cl = (chunk & 3) ^ ((row >> 2) & 3);
    return ((uint32_t)(min(n0 + row, p.N - 1) - n0) * (uint32_t)p.w_rs + cl * 8) * 2u;
  } else if constexpr (FMT == HXA_W_Q8) {
    const int row = chunk >> 1, cl = (chunk & 1) ^ q8_swz(row);
    return (uint32_t)(min(n0 + row, p.N - 1) - n0) * (uint32_t)p.w_rs + cl * 16;
  } else {
    return (uint32_t)(min(n0 + chunk, p.N - 1) - n0) * (uint32_t)p.w_rs;
  }
}
// the k tile's A / W corners: A row m0, column k0; W row n0, k group k0 / 32
HXA_DEV const uint8_t *a_tile_base(const GemmParams &p, int m0, int k0) {
  return (const uint8_t *)(p.A + (long)m0 * p.lda + k0);
}
template <int FMT>
HXA_DEV const uint8_t *w_tile_base(const GemmParams &p, int n0, int k0) {
  constexpr long ES = FMT == HXA_W_F16 ? 2 : 1;
  return (const uint8_t *)p.W + ((long)n0 * p.w_rs + (long)(k0 >> 5) * p.w_gs) * ES;
}

HXA_DEV void tile_coords(const GemmParams &p, int bid, int &tm, int &tn) {
  const int ntiles = p.tiles_m * p.tiles_n;
  if (p.xcd_gm > 0) {
    const int x = bid & 7, i = bid >> 3;
    const int xm = p.tiles_m / p.xcd_gm, xn = p.tiles_n * p.xcd_gm / 8;
    tm = (x % p.xcd_gm) * xm + i % xm;
    tn = (x / p.xcd_gm) * xn + i / xm;
    return;
  }
  const int tile = (ntiles % 8 == 0) ? (bid % 8) * (ntiles / 8) + bid / 8 : bid;
  tm = tile % p.tiles_m;
  tn = tile / p.tiles_m;
}

// the gains of head-normed columns n .. n+7 and a row's RoPE coefficients of dims (n & 63) .. +7
HXA_DEV void hn_gains(const GemmParams &p, int n, float (&g)[8]) {
  const float *gp = (n < p.hn_gsplit ? p.hn_g0 : p.hn_g1) + (n & 127);
  const float4_t a = *(const float4_t *)gp, b = *(const float4_t *)(gp + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    g[e] = a[e];
    g[e + 4] = b[e];
  }
}
HXA_DEV void hn_rope_t(const GemmParams &p, int tt, int n, float (&cs)[8], float (&sn)[8]) {
  const long o = (long)tt * 64 + (n & 63);
  const float4_t c0 = *(const float4_t *)(p.hn_cos + o), c1 = *(const float4_t *)(p.hn_cos + o + 4);
  const float4_t s0 = *(const float4_t *)(p.hn_sin + o), s1 = *(const float4_t *)(p.hn_sin + o + 4);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    cs[e] = c0[e];
    cs[e + 4] = c1[e];
    sn[e] = s0[e];
    sn[e + 4] = s1[e];
  }
}

HXA_DEV half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
HXA_DEV uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// 4 int8 (two's complement, k-consecutive) -> 2 x half2 of f16(q*s)
HXA_DEV void dq8_word(uint32_t d, half2_t s2, uint32_t &o0, uint32_t &o1) {
  const uint32_t x = d ^ 0x80808080u;                         // offset binary u = q + 128
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);  // (0x64|u0, 0x64|u1) = 1024+u
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
  const half2_t c = {(hxa_h)1152.0f, (hxa_h)1152.0f};
  o0 = as_u((as_h2(lo) - c) * s2);
  o1 = as_u((as_h2(hi) - c) * s2);
}

// 8 int4 of one 32-bit word -> 4 x half2
template <bool ASYM>
HXA_DEV void dq4_word(uint32_t d, half2_t s2, half2_t z2, uint32_t *o) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t v = ((d >> (4 * j)) & 0x000F000Fu) | 0x64006400u;  // (1024+n_{2j}, 1024+n_{2j+1})
    if (ASYM) {
      const half2_t c = {(hxa_h)1024.0f, (hxa_h)1024.0f};
      o[j] = as_u(__builtin_elementwise_fma(as_h2(v) - c, s2, z2));
    } else {
      const half2_t c = {(hxa_h)1032.0f, (hxa_h)1032.0f};
      o[j] = as_u((as_h2(v) - c) * s2);
    }
  }
}

// The k order of the fragments. In v_mfma_f32_32x32x16_f16 lane half h = lane >> 5 supplies the 8 k values
// 8h .. 8h+7 of the instruction's 16 for both operands. Slice ks of a 32-deep stage gives lane half h the stage's
// k values 16h + 8ks .. +7, the same for A and W (the sum over the stage is unchanged): fp16 16-byte chunk 2h + ks
// of a row, bytes 8ks .. 8ks+7 of q8 chunk h, 4-byte q4 slot 2h + ks. A lane's two q8 slices then come from one
// 16-byte chunk of the row (measured 3-4% faster on the large ping-pong tiles than slices 2ks + h). Every kernel
// uses this order, so a product's fp32 sums are the same whatever the tile.
HXA_DEV constexpr int kslot(int ks, int h) { return 2 * h + ks; }
// the raw quantised W of slice ks of a row for lane half h
HXA_DEV uint2_t read_wq8(const uint8_t *ws, int row, int h, int ks) {
  return *(const uint2_t *)(ws + row * 32 + ((h ^ q8_swz(row)) << 4) + (ks << 3));
}
HXA_DEV uint32_t read_wq4(const uint8_t *ws, int row, int h, int ks) {
  return *(const uint32_t *)(ws + row * 16 + (kslot(ks, h) << 2));
}

HXA_DEV float gelu_tanh_f(float t) {
  // 0.5 t (1 + tanh u) written as t / (1 + exp(-2u)) (kern.c:116-132): no cancellation for negative t. With
  // u = sqrt(2/pi) (t + 0.044715 t^3), exp(-2u) = 2^(t (K1 + K3 t^2)): the constants folded, three VALU operations
  // for the exponent instead of six (the MLP-up epilogue runs this on every output)
  constexpr float K1 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654);
  constexpr float K3 = (float)(-2.0 * 1.4426950408889634 * 0.7978845608028654 * 0.044715);
  const float e = __builtin_amdgcn_exp2f(t * fmaf(K3, t * t, K1));
  return t * __builtin_amdgcn_rcpf(1.0f + e);  // v_rcp_f32 (1 ulp): far below the fp16 rounding
}
HXA_DEV float gelu_erf_f(float t) {
  // kern.c:248-260: f16(max(t,0) - T2(|t|)), T2 = f16(|t| * 0.5 * erfc(|t|/sqrt 2))
  const float a = fabsf(t);
  const float t2 = (float)(hxa_h)(a * 0.5f * erfcf(a * 0.7071067811865476f));
  return fmaxf(t, 0.0f) - t2;
}
// T2(a) = f16(a * 0.5 * erfc(a / sqrt 2)) of gelu_erf_f for every non-negative fp16 bit pattern b (a = |t|; NaN and
// inf patterns included): the GELU-erf epilogue looks its values up instead of evaluating erfcf per output. Filled
// once per device by erf_t2_kernel with gelu_erf_f's own expression, so a lookup returns the same bits.
constexpr int ERF_T2_N = 0x8000;
// the part of the table a GELU-erf epilogue copies into LDS where its tile leaves room: |t| < 6 (bit patterns below
// 0x4600), 35840 bytes = 35 wave-wide 16-byte copies; larger |t| (rare) is looked up in the global table
constexpr int ERF_T2_LDS_N = 0x4600, ERF_T2_LDS_BYTES = ERF_T2_LDS_N * 2;
__device__ __align__(16) hxa_h g_erf_t2[ERF_T2_N];
__global__ __launch_bounds__(256) void erf_t2_kernel(hxa_h *t) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= ERF_T2_N) return;
  const float a = (float)__builtin_bit_cast(hxa_h, (uint16_t)b);
  t[b] = (hxa_h)(a * 0.5f * erfcf(a * 0.7071067811865476f));
}
HXA_DEV float gelu_erf_tab(float t, const hxa_h *__restrict__ t2tab) {
  const uint32_t b = __builtin_bit_cast(uint16_t, (hxa_h)t) & 0x7fffu;
  return fmaxf(t, 0.0f) - (float)t2tab[b];
}
HXA_DEV float situ_f(float u, float g) {
  // moss kern.c:376-405: f16(f16(25 tanh(u/25)) * f16(4 tanh(g/4) sigmoid(g)))
  const float tu = (float)(hxa_h)(25.0f * tanhf(u * 0.04f));
  const float gs = (float)(hxa_h)(4.0f * tanhf(g * 0.25f) / (1.0f + __expf(-g)));
  return tu * gs;
}

template <int BM, int BN, int FMT>
struct GemmGeo {
  static constexpr int BK = 32;                                      // k per stage (one quantisation group)
  static constexpr int RB = FMT == HXA_W_F16 ? 64 : FMT == HXA_W_Q8 ? 32 : 16;  // W bytes per row per stage
  static constexpr int NS = 4, PD = NS - 1;  // LDS ring stages, prefetch distance
  static constexpr int A_BYTES = BM * 64;
  static constexpr int W_BYTES = BN * RB;
  static constexpr int S_BYTES = FMT == HXA_W_F16 ? 0 : (BN * 2 + 15) / 16 * 16;
  static constexpr int STAGE = A_BYTES + W_BYTES + 2 * S_BYTES;     // scale + optional offset vectors
  static constexpr int CROW = BN + 8;
  static constexpr int C_BYTES = BM * CROW * 2;
  static constexpr int PF_LDS = 256;                                 // prefetch_share's sink (64 lanes x 4 B)
  static constexpr int LDS = (NS * STAGE > C_BYTES ? NS * STAGE : C_BYTES) + PF_LDS;
  // a GELU-erf launch's LDS with the T2 table past everything above, where that fits the CU's 160 KB
  static constexpr bool ERF_FITS = LDS + ERF_T2_LDS_BYTES <= 160 * 1024;
  static constexpr int NA = BM / 64;                                 // A load instructions per wave per stage
  static constexpr int TW = (W_BYTES / 16 + 63) / 64;                // W load instructions per stage (all waves)
};

// Per-wave number of direct-to-LDS instructions issued for one stage (A and W instructions dealt round-robin over
// the NW waves; every wave loads its share of the scale / offset vectors).
template <int BM, int BN, int FMT, bool ASYM, int NW>
HXA_DEV constexpr int loads_per_stage(int wave) {
  using G = GemmGeo<BM, BN, FMT>;
  constexpr int NA = BM / 16;
  return NA / NW + (wave < NA % NW ? 1 : 0) + G::TW / NW + (wave < G::TW % NW ? 1 : 0) +
         (FMT != HXA_W_F16 ? (ASYM ? 2 : 1) : 0);
}
// Wait until at most LATER further stages of this wave's loads are outstanding, with one wave-uniform count: the
// fewest loads any wave issues per stage. A wave that issues more waits for a few of its newest loads too, never for
// fewer than its own older stages. (A count chosen per wave branches on the wave index inside the main loop, and the
// register allocator then copied the live accumulators between AGPRs and VGPRs around that branch every k step.)
template <int BM, int BN, int FMT, bool ASYM, int NW, int LATER>
HXA_DEV void wait_stage(int) {
  constexpr int lmin = [] {
    int m = loads_per_stage<BM, BN, FMT, ASYM, NW>(0);
    for (int w = 1; w < NW; w++) m = loads_per_stage<BM, BN, FMT, ASYM, NW>(w) < m ? loads_per_stage<BM, BN, FMT, ASYM, NW>(w) : m;
    return m;
  }();
  wait_vm<LATER * lmin>();
}

// ---- epilogue after f16(acc) is staged in LDS as a row-major [BM][BN + 8] tile (and, for SPLIT2, the first K
// half's tile after it): cooperative passes over 8-column chunks, coalesced 16-byte loads / stores.
// PARTIAL_F32: the K slice's fp32 sums straight from the accumulators (no fp16 rounding, no LDS staging). For block
// (j, i) the lane holds row mrow + i*32 and columns ncol + j*32 + 8q + 0..3 (q = 0..3): one 16-byte store each, so
// the four q stores of a wave fill 32 rows x 128 contiguous bytes. N % 8 == 0, so a chunk is inside N or past it.
template <int MI, int NI>
HXA_DEV void store_partial_f32(const GemmParams &p, const float16_t (&acc)[NI][MI], int mrow, int ncol, int z) {
  float *base = p.out32 + (long)z * p.out_zstride;
#pragma unroll
  for (int i = 0; i < MI; i++) {
    const int m = mrow + i * 32;
    if (m >= p.M) continue;
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int n = ncol + j * 32 + 8 * q;
        if (n < p.N)
          *(float4_t *)(base + (long)m * p.ldo + n) =
              (float4_t){acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2], acc[j][i][4 * q + 3]};
      }
  }
}

template <int BM, int BN, int NT, bool SPLIT2>
HXA_DEV void gemm_epilogue(const GemmParams &p, const hxa_h *Cs, int m0, int n0, int tid, int z) {
  constexpr int CROW = BN + 8;
  constexpr int C8 = BN / 8;
  if (p.epi == HXA_EPI_SITU) {
    // columns interleaved per 32 (up_j, gate_j): output column (n0/2) + p*32 + c
    for (int c = tid; c < BM * (C8 / 2); c += NT) {
      const int ml = c / (C8 / 2), oc = (c % (C8 / 2)) * 8;
      const int m = m0 + ml, on = n0 / 2 + oc;
      if (m >= p.M || on * 2 >= p.N) continue;
      const int pr = oc / 32, cc = oc % 32;
      const half8_t u = *(const half8_t *)(Cs + ml * CROW + pr * 64 + cc);
      const half8_t g = *(const half8_t *)(Cs + ml * CROW + pr * 64 + 32 + cc);
      half8_t o;
#pragma unroll
      for (int e = 0; e < 8; e++) o[e] = (hxa_h)situ_f((float)u[e], (float)g[e]);
      *(half8_t *)(p.out + (long)m * p.ldo + on) = o;
    }
    return;
  }
  // local columns [0, nsplit) row-major, [nsplit, BN) transposed into out_t. Without out_t the chunk count per row
  // is the compile-time BN / 8 (no runtime division in the loop).
  const int nsplit = p.out_t == nullptr ? BN : min(max(p.split_col - n0, 0), BN);
  if (p.epi == HXA_EPI_RESADD) {
    // x += gate * t: the x / gate loads of RB chunks are issued together before any of them is used, so a thread
    // waits one memory latency per batch instead of one per chunk (x stores may alias later x loads otherwise)
    constexpr int NC8 = BN / 8, ITERS = BM * NC8 / NT, RB = ITERS % 4 == 0 ? 4 : ITERS % 3 == 0 ? 3 : ITERS % 2 == 0 ? 2 : 1;
    static_assert(BM * NC8 % NT == 0 && ITERS % RB == 0, "whole chunk passes");
#pragma unroll
    for (int b0 = 0; b0 < ITERS; b0 += RB) {
      float4_t xv[RB][2], gv[RB][2];
      float t[RB][8];
      bool ok[RB];
#pragma unroll
      for (int u = 0; u < RB; u++) {
        const int c = tid + (b0 + u) * NT, ml = c / NC8, nl = (c % NC8) * 8, m = m0 + ml, n = n0 + nl;
        ok[u] = m < p.M && n < p.N;
        if (ok[u]) {
          const float4_t *xp = (const float4_t *)(p.x + (long)m * p.ldx + n);
          xv[u][0] = xp[0];
          xv[u][1] = xp[1];
          gv[u][0] = *(const float4_t *)(p.gate + n);
          gv[u][1] = *(const float4_t *)(p.gate + n + 4);
          const half8_t v = *(const half8_t *)(Cs + ml * CROW + nl);
#pragma unroll
          for (int e = 0; e < 8; e++) t[u][e] = (float)v[e];
          if constexpr (SPLIT2) {
            const half8_t v1 = *(const half8_t *)(Cs + BM * CROW + ml * CROW + nl);
#pragma unroll
            for (int e = 0; e < 8; e++) t[u][e] = (float)v1[e] + t[u][e];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < RB; u++) {
        if (!ok[u]) continue;
        const int c = tid + (b0 + u) * NT, ml = c / NC8, nl = (c % NC8) * 8;
        float4_t *xp = (float4_t *)(p.x + (long)(m0 + ml) * p.ldx + n0 + nl);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          xv[u][0][e] = fmaf(gv[u][0][e], t[u][e], xv[u][0][e]);
          xv[u][1][e] = fmaf(gv[u][1][e], t[u][e + 4], xv[u][1][e]);
        }
        xp[0] = xv[u][0];
        xp[1] = xv[u][1];
      }
    }
    return;
  }
  if constexpr (BN % 128 == 0) {
  if (p.hn_cols > 0 && (n0 + BN <= p.hn_cols || p.hn_cols >= p.N)) {
    // every (valid) column of this tile is head-normed. Thread (row group r0, jj) owns dims [8jj, 8jj+8) and
    // [64+8jj, 64+8jj+8) of every head of the tile on its rows: the gains are loaded once, the RoPE coefficients once
    // per row for all heads (fetched one pass ahead), and the rotation partners sit in the same thread.
    constexpr int HT = BN / 128, RP = NT / 8;  // heads per tile, rows per pass
    static_assert(BM % RP == 0, "whole passes");
    const int jj = tid & 7, r0 = tid >> 3;
    const bool rope = p.hn_cos != nullptr;
    float glo[HT][8], ghi[HT][8], cs[8] = {}, sn[8] = {}, csn[8] = {}, snn[8] = {};
#pragma unroll
    for (int hh = 0; hh < HT; hh++) {
      hn_gains(p, n0 + hh * 128 + 8 * jj, glo[hh]);
      hn_gains(p, n0 + hh * 128 + 64 + 8 * jj, ghi[hh]);
    }
    // RoPE table row of the next pass's row, stepped by RP rows without a division (rows past M are not stored)
    int tt = rope ? min(m0 + r0, p.M - 1) % p.hn_ttab : 0;
    if (rope) hn_rope_t(p, tt, 8 * jj, cs, sn);
    for (int it = 0; it < BM / RP; it++) {
      const int ml = r0 + it * RP, m = m0 + ml;
      if (rope && it + 1 < BM / RP) {
        if (m + RP < p.M) {
          tt += RP;
          while (tt >= p.hn_ttab) tt -= p.hn_ttab;
        }
        hn_rope_t(p, tt, 8 * jj, csn, snn);
      }
      if (m < p.M) {  // whole 8-lane groups share m
#pragma unroll
        for (int hh = 0; hh < HT; hh++) {
          const int nl = hh * 128 + 8 * jj;
          if (n0 + nl >= p.N) break;
          half8_t lo = *(const half8_t *)(Cs + ml * CROW + nl), hi = *(const half8_t *)(Cs + ml * CROW + nl + 64);
          head_norm2(lo, hi, glo[hh], ghi[hh], rope, cs, sn);
          *(half8_t *)(p.out + (long)m * p.ldo + n0 + nl) = lo;
          *(half8_t *)(p.out + (long)m * p.ldo + n0 + nl + 64) = hi;
        }
      }
      if (rope) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          cs[e] = csn[e];
          sn[e] = snn[e];
        }
      }
    }
    return;
  }
  }
  if (p.epi == HXA_EPI_GELU_ERF && p.erf_t2 != nullptr && nsplit == BN) {
    // GELU-erf through the T2 table: the LDS reads and table lookups of RB chunks are issued together before any
    // of them is used, so a thread waits one lookup latency per batch instead of one per chunk. With erf_lds the
    // table's |t| < 6 part is first copied into LDS past the staged tile (LDS gathers, where global ones issue at
    // a few lanes per clock)
    constexpr int ITERS = BM * C8 / NT, RB = ITERS % 4 == 0 ? 4 : ITERS % 3 == 0 ? 3 : ITERS % 2 == 0 ? 2 : 1;
    static_assert(BM * C8 % NT == 0 && ITERS % RB == 0, "whole chunk passes");
    static_assert(ERF_T2_LDS_BYTES % 1024 == 0, "whole wave-wide copies");
    const hxa_h *tl = nullptr;
    if (p.erf_lds > 0) {
      uint8_t *dst = (uint8_t *)Cs + p.erf_lds;
      const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
      for (int c0 = wave * 64; c0 < ERF_T2_LDS_BYTES / 16; c0 += NT) {
        const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)(dst + c0 * 16));
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(p.erf_t2 + (c0 + lane) * 8), "s"(la)
                     : "memory", "m0");
      }
      wait_vm<0>();
      __syncthreads();
      tl = (const hxa_h *)dst;
    }
#pragma unroll
    for (int b0 = 0; b0 < ITERS; b0 += RB) {
      half8_t v[RB];
      hxa_h t2[RB][8];
      bool ok[RB];
#pragma unroll
      for (int u = 0; u < RB; u++) {
        const int c = tid + (b0 + u) * NT, ml = c / C8, nl = (c % C8) * 8;
        ok[u] = m0 + ml < p.M && n0 + nl < p.N;
        v[u] = *(const half8_t *)(Cs + ml * CROW + nl);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const hxa_h x = v[u][e];  // (a scalar copy: bit_cast of a vector element itself read element 0 only)
          const uint32_t b = __builtin_bit_cast(uint16_t, x) & 0x7fffu;
          t2[u][e] = tl != nullptr && b < (uint32_t)ERF_T2_LDS_N ? tl[b] : p.erf_t2[b];
        }
      }
#pragma unroll
      for (int u = 0; u < RB; u++) {
        if (!ok[u]) continue;
        const int c = tid + (b0 + u) * NT, ml = c / C8, nl = (c % C8) * 8;
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (hxa_h)(fmaxf((float)v[u][e], 0.0f) - (float)t2[u][e]);
        *(half8_t *)(p.out + (long)(m0 + ml) * p.ldo + n0 + nl) = o;
      }
    }
    return;
  }
  auto rows_pass = [&](auto ncols_c) {
  const int nc8 = ncols_c / 8;
  for (int c = tid; c < BM * nc8; c += NT) {
    const int ml = c / nc8, nl = (c % nc8) * 8;
    const int m = m0 + ml, n = n0 + nl;
    if (m >= p.M || n >= p.N) continue;
    half8_t v = *(const half8_t *)(Cs + ml * CROW + nl);
    const long o = (long)m * p.ldo + n;
    if (p.epi == HXA_EPI_PARTIAL) {
      *(half8_t *)(p.out + (long)z * p.out_zstride + o) = v;
    } else {
      if (p.epi == HXA_EPI_GELU_TANH) {  // (head-normed tiles never get here: whole tiles take the path above)
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (hxa_h)gelu_tanh_f((float)v[e]);
      } else if (p.epi == HXA_EPI_GELU_ERF) {  // (without the T2 table, or with transposed columns)
        if (p.erf_t2) {
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = (hxa_h)gelu_erf_tab((float)v[e], p.erf_t2);
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = (hxa_h)gelu_erf_f((float)v[e]);
        }
      }
      *(half8_t *)(p.out + o) = v;
    }
  }
  };
  if (p.out_t == nullptr)
    rows_pass(std::integral_constant<int, BN>{});
  else
    rows_pass(nsplit);
  if (nsplit < BN) {
    // transposed columns (a multiple of 32: split_col % 32 == 0): a thread takes 4 adjacent columns x 8 rows, read as
    // 8-byte LDS words, and writes four 16-byte runs of 8 rows, one per output row n of out_t. Four consecutive
    // threads take consecutive 8-row chunks of the same columns, so each store instruction writes 64-byte runs
    // (16 rows of out_t per wave) rather than 64 scattered 16-byte pieces; the LDS reads of those four threads are 8
    // rows apart (two-way bank conflicts).
    static_assert(BM % 32 == 0, "8-row chunks in fours");
    const int ngrp = (BN - nsplit) / 4;
    for (int c = tid; c < ngrp * (BM / 8); c += NT) {
      const int rest = c >> 2;
      const int nl = nsplit + (rest % ngrp) * 4, ml = ((rest / ngrp) * 4 + (c & 3)) * 8;
      const int m = m0 + ml;
      if (m >= p.M) continue;
      uint2_t w[8];
#pragma unroll
      for (int e = 0; e < 8; e++) w[e] = *(const uint2_t *)(Cs + (ml + e) * CROW + nl);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int n = n0 + nl + q;
        if (n >= p.N) break;
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {  // rows 2k, 2k+1 of column q: halves (q & 1) of word (q >> 1)
          const uint32_t a = (q >> 1) ? w[2 * k].y : w[2 * k].x, b = (q >> 1) ? w[2 * k + 1].y : w[2 * k + 1].x;
          o[k] = __builtin_amdgcn_perm(b, a, (q & 1) ? 0x07060302u : 0x05040100u);
        }
        hxa_h *dst = p.out_t + (long)(n - p.split_col) * p.ldo_t + m;
        if (m + 7 < p.M) {
          *(uint4_t *)dst = (uint4_t){o[0], o[1], o[2], o[3]};
        } else {
          const half8_t v = __builtin_bit_cast(half8_t, (uint4_t){o[0], o[1], o[2], o[3]});
          for (int e = 0; e < 8 && m + e < p.M; e++) dst[e] = v[e];
        }
      }
    }
  }
}

// ---- fused cross attention (blk.c:163-169 in one kernel) ----
// After the main loop of a 128 x 128 fp16 tile of the cross-q projection (one head: the tile's 128 columns), the
// tile becomes that head's 128 queries: f16(acc) is staged in LDS and RMSNorm * gain is applied in place (kern.c:163-197,
// the head-norm epilogue's arithmetic), each of the 4 waves takes 32 queries as MFMA fragments, and the head's text
// keys are swept in 64-key tiles of K and V^T, double-buffered in LDS behind the query tile (the attention kernel's
// layouts: K rows in krow_key order, chunks XOR-swizzled), with the exact online softmax in fp32; O = f16(P V / l).
// LDS: the GEMM's ring (64 KB, then the query tile [128][136] fp16 in its place), then K, K, V^T, V^T (64 KB): the
// first two key tiles are loaded when the workgroup starts and arrive during the main loop.
// LDS of the fused kernel: the 128x128 fp16 ring [0, 64 KB) (later the query staging and the V^T tiles 2, 3 of the
// two-pass form), K / V^T tiles 0, 1 at XA_KV_OFF, K tiles 2, 3 at XA_K23_OFF: 160 KB. The ring's prefetch sink is
// not needed (the fused kernel prefetches nothing).
constexpr int XA_KV_OFF = 4 * 16384;
constexpr int XA_K23_OFF = XA_KV_OFF + 4 * 16384;
constexpr int XA_LDS = XA_K23_OFF + 2 * 16384;
static_assert(XA_KV_OFF >= GemmGeo<128, 128, HXA_W_F16>::NS * GemmGeo<128, 128, HXA_W_F16>::STAGE &&
                  XA_KV_OFF >= GemmGeo<128, 128, HXA_W_F16>::C_BYTES && XA_LDS <= 160 * 1024,
              "fused cross-attention LDS layout");
// key tile i of the tile's head into LDS buffer i & 1: 16 KB of K (rows in krow_key order, 256 B each, chunk c at
// c ^ (row & 15)) and 16 KB of V^T (128 rows of 64 keys, chunk c at c ^ ((d >> 1) & 7)); keys past NKV read a valid
// row (probability 0). 8 loads per wave of the 4.
// key tile i of the workgroup's head and image -> K tile at kb, V^T tile at vb (16 KB each, the attention kernel's
// swizzled layout); keys past NKV read a valid row
HXA_DEV void xattn_load_tile(const GemmParams &p, int m0, int n0, int i, int wave, int lane, uint8_t *kb, uint8_t *vb,
                             bool with_k = true, bool with_v = true) {
  const int img = m0 / p.xa_T, h = n0 >> 7, key0 = i * 64, NKV = p.xa_nkv;
  const hxa_h *kh = p.xa_k + (long)img * p.xa_kb + h * 128;
  const hxa_h *vh = p.xa_vt + (long)img * p.xa_vb + (long)h * 128 * p.xa_ldvt;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (!with_k) break;
    const int blk = j * 4 + wave;
    const int row = 4 * blk + (lane >> 4), c = (lane & 15) ^ (row & 15);
    const int key = min(key0 + krow_key(row), NKV - 1);
    g2l16_opaque(kh + (long)key * p.xa_ldk + c * 8, kb + blk * 1024);
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (!with_v) break;
    const int blk = j * 4 + wave;
    const int d = 8 * blk + (lane >> 3), c = (lane & 7) ^ ((d >> 1) & 7);
    int key = key0 + c * 8;
    if (key >= NKV) key = 0;
    g2l16_opaque(vh + (long)d * p.xa_ldvt + key, vb + blk * 1024);
  }
}
// tiles 0 and 1 (and, for the online form, every later tile in turn) at the K / V^T buffers past the GEMM's ring
HXA_DEV void xattn_load_kv(const GemmParams &p, int m0, int n0, int i, int wave, int lane, uint8_t *lds8) {
  xattn_load_tile(p, m0, n0, i, wave, lane, lds8 + XA_KV_OFF + (i & 1) * 16384, lds8 + XA_KV_OFF + (2 + (i & 1)) * 16384);
}
template <int MI, int NI, int WTM, int WTN>
HXA_DEV void xattn_tail(const GemmParams &p, float16_t (&acc)[NI][MI], int m0, int n0, int tid, int lane, int wave, int wm,
                        int wn, uint8_t *lds8) {
  constexpr float L2E = 1.4426950408889634f, RESCALE_TH = 5.5f;
  constexpr int CROW = 136;
  const int g = lane >> 5, ql = lane & 31;
  const int h = n0 >> 7, ntiles = (p.xa_nvalid + 63) / 64;
  auto kbuf = [&](int i) { return lds8 + XA_KV_OFF + (i & 1) * 16384; };
  auto vbuf = [&](int i) { return lds8 + XA_KV_OFF + (2 + (i & 1)) * 16384; };
  // the head's gains (key tiles 0 and 1 were loaded when the workgroup started and have landed: the main loop's
  // waits covered every older load)
  const int jj = tid & 7, r0 = tid >> 3;
  float glo[8], ghi[8];
  hn_gains(p, n0 + 8 * jj, glo);
  hn_gains(p, n0 + 64 + 8 * jj, ghi);
  wait_vm<0>();  // (and the main loop's trailing loads must land before its LDS ring is reused)
  __syncthreads();
  // stage f16(acc) as the row-major query tile
  hxa_h *Cs = (hxa_h *)lds8;
  {
    const int ml = wm * WTM + (lane & 31), nl = wn * WTN + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const half4_t v = {(hxa_h)acc[j][i][4 * q], (hxa_h)acc[j][i][4 * q + 1], (hxa_h)acc[j][i][4 * q + 2],
                             (hxa_h)acc[j][i][4 * q + 3]};
          *(half4_t *)(Cs + (ml + i * 32) * CROW + nl + j * 32 + 8 * q) = v;
        }
  }
  __syncthreads();
  // RMSNorm * gain per query row, in place: 8 lanes per row (lane jj owns dims [8jj, 8jj+8) and [64+8jj, 64+8jj+8))
  {
    const float z8[8] = {};
#pragma unroll
    for (int it = 0; it < 4; it++) {
      hxa_h *row = Cs + (r0 + it * 32) * CROW;
      half8_t lo = *(const half8_t *)(row + 8 * jj), hi = *(const half8_t *)(row + 64 + 8 * jj);
      head_norm2(lo, hi, glo, ghi, false, z8, z8);
      *(half8_t *)(row + 8 * jj) = lo;
      *(half8_t *)(row + 64 + 8 * jj) = hi;
    }
  }
  __syncthreads();
  half8_t qf[8];
#pragma unroll
  for (int sd = 0; sd < 8; sd++) qf[sd] = *(const half8_t *)(Cs + (wave * 32 + ql) * CROW + sd * 16 + 8 * g);
  float16_t o[4];
#pragma unroll
  for (int d = 0; d < 4; d++) o[d] = (float16_t){};
  float mrun = -INFINITY, lsum = 0.0f;
  if (ntiles <= 4) {
    // Up to 256 keys: every tile stays in LDS (tiles 2 and 3 in the staging region, free once every wave holds its
    // q fragments), so the scores of all tiles are formed first and the row max is exact: no running rescale, and
    // the exponentials of tile t + 1 run between the P V MFMAs of tile t.
    // (K of tiles 2 and 3 was loaded with tiles 0 and 1 and has landed; their V^T goes to the staging region)
    __syncthreads();
    auto kt = [&](int t) -> const uint8_t * {
      return t < 2 ? lds8 + XA_KV_OFF + t * 16384 : lds8 + XA_K23_OFF + (t - 2) * 16384;
    };
    auto vt = [&](int t) -> const uint8_t * {
      return t < 2 ? lds8 + XA_KV_OFF + (2 + t) * 16384 : lds8 + (t - 2) * 16384;
    };
    if (ntiles > 2) xattn_load_tile(p, m0, n0, 2, wave, lane, nullptr, lds8, false, true);
    if (ntiles > 3) xattn_load_tile(p, m0, n0, 3, wave, lane, nullptr, lds8 + 16384, false, true);
    const uint8_t *const kts[4] = {kt(0), kt(1), kt(2), kt(3)}, *const vts[4] = {vt(0), vt(1), vt(2), vt(3)};
    attn_two_pass(qf, kts, vts, ntiles, p.xa_nvalid, true, lane, o, lsum);
  } else {
  for (int i = 0; i < ntiles; i++) {
    if (i + 1 < ntiles) wait_vm<8>();  // tile i landed (tile i + 1 may still fly)
    else wait_vm<0>();
    // a plain barrier (no fence): tile i + 1's loads stay in flight
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint8_t *kb = kbuf(i), *vb = vbuf(i);
    // every K fragment of the tile, then the V^T fragments, read ahead of the MFMAs that use them (the V^T reads
    // land during the QK MFMAs and the softmax)
    half8_t kf[8][2], vf[16];
#pragma unroll
    for (int ds = 0; ds < 8; ds++)
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++) {
        const int row = kb2 * 32 + ql, c = 2 * ds + g;
        kf[ds][kb2] = *(const half8_t *)(kb + row * 256 + ((c ^ (row & 15)) << 4));
      }
#pragma unroll
    for (int j = 0; j < 16; j++) {  // j = (kb2 * 2 + ks) * 4 + dblk
      const int dblk = j & 3, kk = j >> 2, d = dblk * 32 + ql, c = 2 * kk + g;
      vf[j] = *(const half8_t *)(vb + d * 128 + ((c ^ ((d >> 1) & 7)) << 4));
    }
    float16_t S[2];
    S[0] = (float16_t){};
    S[1] = (float16_t){};
#pragma unroll
    for (int ds = 0; ds < 8; ds++)
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++) S[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[ds][kb2], qf[ds], S[kb2], 0, 0, 0);
    const int key0 = i * 64;
    if (key0 + 64 > p.xa_nvalid) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (key0 + kb2 * 32 + 16 * (r >> 3) + 8 * g + (r & 7) >= p.xa_nvalid) S[kb2][r] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
      for (int r = 0; r < 16; r++) mt = fmaxf(mt, S[kb2][r]);
    {
      float lo, hi;
      halves(mt, lo, hi);
      mt = fmaxf(lo, hi);
    }
    const bool need = mt > mrun + RESCALE_TH;  // also while mrun is -inf
    if (__any(need)) {
      const float alpha = need ? __builtin_amdgcn_exp2f((mrun - mt) * L2E) : 1.0f;
      if (need) mrun = mt;
      lsum *= alpha;
#pragma unroll
      for (int d = 0; d < 4; d++) o[d] *= alpha;
    }
    const float mb = (mrun == -INFINITY ? 0.0f : mrun) * L2E;
    half8_t pf[2][2];
    float ls[2] = {0.0f, 0.0f};
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {  // fp16 pairs, summed by v_dot2 (the row sum of the fp16 P)
        const float p0 = __builtin_amdgcn_exp2f(fmaf(S[kb2][r], L2E, -mb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(S[kb2][r + 1], L2E, -mb));
        const half2_t h2 = {(hxa_h)p0, (hxa_h)p1};
        pf[kb2][r >> 3][r & 7] = h2[0];
        pf[kb2][r >> 3][(r & 7) + 1] = h2[1];
        ls[(r >> 1) & 1] = __builtin_amdgcn_fdot2(h2, (half2_t){(hxa_h)1.0f, (hxa_h)1.0f}, ls[(r >> 1) & 1], false);
      }
    lsum += ls[0] + ls[1];
#pragma unroll
    for (int j = 0; j < 16; j++)
      o[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[j], pf[j >> 3][(j >> 2) & 1], o[j & 3], 0, 0, 0);
    if (i + 2 < ntiles) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();  // every wave's reads of buffer i & 1 are in registers (the MFMAs used them)
      asm volatile("" ::: "memory");
      xattn_load_kv(p, m0, n0, i + 2, wave, lane, lds8);
    }
  }
  }
  float llo, lhi;
  halves(lsum, llo, lhi);
  const float ltot = llo + lhi;
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  half4_t v[4][4];
#pragma unroll
  for (int d = 0; d < 4; d++)
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++)
#pragma unroll
      for (int e = 0; e < 4; e++) v[d][r4][e] = (hxa_h)(o[d][4 * r4 + e] * inv);
  // whole output rows, staged in the K-tile 2 / 3 region: unused with at most two key tiles, and with more every
  // wave has passed the barrier before tile 2's P V, so every QK pass is done (the online form never uses it)
  store_rows32(lds8 + XA_K23_OFF + wave * 8192, v, lane, p.xa_o + (long)(m0 + wave * 32) * p.xa_ldo + h * 128, p.xa_ldo,
               32);
}

// SPLIT2: the first and second halves of K are rounded to fp16 separately and combined in the residual epilogue,
// x += gate * (f16(first half) + f16(second half)) (blk.c:172-174 + kern.c:330-339 in one kernel): the first half's
// f16 accumulators are kept in registers while the second half accumulates.
// NW = 4 waves (2 x 2 grid, one wave per SIMD) or 8 waves (2 x 4 grid, two waves per SIMD: one wave's waits are
// covered by the other's MFMAs).
template <int BM, int BN, int FMT, bool ASYM, bool SPLIT2, int NW, bool XATTN = false>
HXA_DEV void gemm_body(const GemmParams &p, const int bid, const int z) {
  using G = GemmGeo<BM, BN, FMT>;
  constexpr int NT = 64 * NW;
  // waves along M: 2 (a 2 x NW/2 wave grid), or 1 for int8 / int4 weights where BN splits into 32-column strips (a
  // 1 x NW grid): every W fragment then belongs to one wave and is dequantised once per workgroup, at the price of
  // each wave reading all BM rows of A
  constexpr int WMW = (FMT != HXA_W_F16 && !XATTN && BN % (32 * NW) == 0) ? 1 : 2;
  constexpr int WTM = BM / WMW, WTN = BN / (NW / WMW), MI = WTM / 32, NI = WTN / 32;
  constexpr int BK = G::BK, NS = G::NS, PD = G::PD;
  static_assert(BM % 64 == 0 && WTN % 32 == 0 && (NW == 4 || NW == 8), "tile shape");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];

  int tm, tn;
  tile_coords(p, bid, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int kbase = z * p.Kslice;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = WMW == 2 ? (wave & 1) : 0, wn = WMW == 2 ? (wave >> 1) : wave;
  const HxaClkMark clk0 = clk_mark(p.clk);
  if constexpr (XATTN) {  // the first two key tiles of the fused attention, into LDS past the ring
    xattn_load_kv(p, m0, n0, 0, wave, lane, lds8);
    if (p.xa_nvalid > 64) xattn_load_kv(p, m0, n0, 1, wave, lane, lds8);
    if (p.xa_nvalid > 128 && p.xa_nvalid <= 256) {  // the two-pass form: K of tiles 2 and 3 as well
      xattn_load_tile(p, m0, n0, 2, wave, lane, lds8 + XA_K23_OFF, nullptr, true, false);
      if (p.xa_nvalid > 192) xattn_load_tile(p, m0, n0, 3, wave, lane, lds8 + XA_K23_OFF + 16384, nullptr, true, false);
    }
  }

  // ---- loader: stage s <- k tile kt. A and fp16 W rows are 64 B (4 chunks of 16 B) stored with the chunk swizzle
  // c ^ ((row >> 2) & 3); q8 rows are 32 B with chunk swizzle c ^ q8_swz(row); q4 rows are 16 B.
  constexpr int NAI = BM / 16;  // 1 KB A instructions (16 rows) per stage
  constexpr int NAL = (NAI + NW - 1) / NW, NWL = (G::TW + NW - 1) / NW;  // this wave's A / W loads per stage
  uint32_t aoff[NAL], woff[NWL];
#pragma unroll
  for (int a = 0; a < NAL; a++) aoff[a] = a_lane_off(p, min(a * NW + wave, NAI - 1), lane, m0);
#pragma unroll
  for (int t = 0; t < NWL; t++) woff[t] = w_lane_off<FMT>(p, min((t * NW + wave) * 64 + lane, G::W_BYTES / 16 - 1), n0);
  // between(q) runs before load slot q (q < NAL + NWL) in a region of its own: the scheduler does not see these asm
  // loads as memory instructions, so only such fences keep them spread over the MFMAs instead of in one burst
  auto issue = [&](int s, int kt, auto between) {
    uint8_t *st = lds8 + s * G::STAGE;
    const int k0 = kbase + min(kt, p.Kslice / BK - 1) * BK;  // tiles past the end reload the last one (never read)
    const uint8_t *ab = a_tile_base(p, m0, k0), *wb = w_tile_base<FMT>(p, n0, k0);
#pragma unroll
    for (int a0 = 0; a0 < NAI; a0 += NW) {
      const int a = a0 + wave;
      between(a0 / NW);
      if (NAI % NW == 0 || a < NAI) g2l16_sbase(ab, aoff[a0 / NW], st + a * 1024);
      __builtin_amdgcn_sched_barrier(0);
    }
    uint8_t *ws = st + G::A_BYTES;
#pragma unroll
    for (int t0 = 0; t0 < G::TW; t0 += NW) {
      const int t = t0 + wave;
      between(NAL + t0 / NW);
      if (G::TW % NW == 0 || t < G::TW) {
        const int chunk = t * 64 + lane;
        if ((G::W_BYTES / 16) % 64 == 0 || chunk < G::W_BYTES / 16) g2l16_sbase(wb, woff[t0 / NW], ws + t * 1024);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (FMT != HXA_W_F16) {  // the stage's scale (and offset) vector, 16-byte chunks spread over the waves
      constexpr int CPW = (BN / 8 + NW - 1) / NW;  // chunks per wave
      const int g = k0 >> 5, c = wave * CPW + lane;
      const int nn = min(n0 + c * 8, p.N - 8);
      if (lane < CPW && c < BN / 8) g2l16_opaque(p.S + (long)g * p.N + nn, ws + G::W_BYTES + 16 * wave * CPW);
      if (ASYM && lane < CPW && c < BN / 8)
        g2l16_opaque(p.Z + (long)g * p.N + nn, ws + G::W_BYTES + G::S_BYTES + 16 * wave * CPW);
    }
  };

  float16_t acc[NI][MI];
#pragma unroll
  for (int j = 0; j < NI; j++)
#pragma unroll
    for (int i = 0; i < MI; i++) acc[j][i] = (float16_t){};

  // Fragments of one stage: A rows fa[ks][i]; W rows fb[ks][j]. fp16 W fragments are read directly; quantised W
  // is read raw (wq, scale ws_, offset wz) and dequantised ahead of the MFMAs that need it: the second slice under
  // the first slice's MFMAs, the first slice of the next stage at the end of a step, under its last MFMAs.
  typedef typename std::conditional<FMT == HXA_W_Q8, uint2_t, uint32_t>::type raw_t;
  raw_t wq0[2][NI], wq1[2][NI];
  hxa_h sc0[NI], sc1[NI], zc0[NI], zc1[NI];
  auto read_frags = [&](int s, half8_t (&fa)[2][MI], half8_t (&fb)[2][NI], raw_t (&wq)[2][NI], hxa_h (&sc)[NI],
                        hxa_h (&zc)[NI]) {
    const uint8_t *st = lds8 + s * G::STAGE;
    const uint8_t *ws = st + G::A_BYTES;
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
      const int cl = kslot(ks, h);
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int row = wm * WTM + i * 32 + (lane & 31);
        fa[ks][i] = *(const half8_t *)(st + row * 64 + ((cl ^ ((row >> 2) & 3)) << 4));
      }
#pragma unroll
      for (int j = 0; j < NI; j++) {
        const int row = wn * WTN + j * 32 + (lane & 31);
        if constexpr (FMT == HXA_W_F16) {
          fb[ks][j] = *(const half8_t *)(ws + row * 64 + ((cl ^ ((row >> 2) & 3)) << 4));
        } else if constexpr (FMT == HXA_W_Q8) {
          wq[ks][j] = read_wq8(ws, row, h, ks);
        } else {
          wq[ks][j] = read_wq4(ws, row, h, ks);
        }
      }
    }
    if constexpr (FMT != HXA_W_F16) {
#pragma unroll
      for (int j = 0; j < NI; j++) {
        const int row = wn * WTN + j * 32 + (lane & 31);
        sc[j] = *(const hxa_h *)(ws + G::W_BYTES + row * 2);
        zc[j] = ASYM ? *(const hxa_h *)(ws + G::W_BYTES + G::S_BYTES + row * 2) : (hxa_h)0.0f;
      }
    }
  };
  auto dequant = [&](int ks, half8_t (&fb)[2][NI], const raw_t (&wq)[2][NI], const hxa_h (&sc)[NI], const hxa_h (&zc)[NI]) {
    if constexpr (FMT != HXA_W_F16) {
#pragma unroll
      for (int j = 0; j < NI; j++) {
        const half2_t s2 = {sc[j], sc[j]};
        uint32_t o[4];
        if constexpr (FMT == HXA_W_Q8) {
          dq8_word(wq[ks][j].x, s2, o[0], o[1]);
          dq8_word(wq[ks][j].y, s2, o[2], o[3]);
        } else {
          const half2_t z2 = {zc[j], zc[j]};
          dq4_word<ASYM>(wq[ks][j], s2, z2, o);
        }
        fb[ks][j] = __builtin_bit_cast(half8_t, (uint4_t){o[0], o[1], o[2], o[3]});
      }
    }
  };
  auto mfma_range = [&](const half8_t (&fa)[MI], const half8_t (&fb)[NI], int from, int to) {
#pragma unroll
    for (int q = 0; q < NI * MI; q++) {
      if (q >= from && q < to) {
        const int j = q / MI, i = q % MI;
        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[j], fa[i], acc[j][i], 0, 0, 0);
      }
    }
  };
  constexpr int NMF = NI * MI;  // MFMAs per 16-k slice
  const int nk = p.Kslice / BK;
  // One k step with register-double-buffered fragments. After the first two MFMAs of stage kt this wave waits for
  // stage kt+1, passes the barrier, then interleaves the remaining MFMAs of stage kt one-to-one with the prefetch of
  // tile kt+NS (into stage kt's LDS, whose fragments are already in registers) and the fragment reads of stage kt+1.
  // Every load is unconditional (past the end: clamped dummy loads), so the vmcnt accounting is constant.
  auto step = [&](int kt, half8_t (&ca)[2][MI], half8_t (&cb)[2][NI], half8_t (&na)[2][MI], half8_t (&nb)[2][NI],
                  raw_t (&cq)[2][NI], hxa_h (&cs)[NI], hxa_h (&cz)[NI], raw_t (&nq)[2][NI], hxa_h (&ns)[NI],
                  hxa_h (&nz)[NI]) {
    mfma_range(ca[0], cb[0], 0, 2);
    __builtin_amdgcn_sched_barrier(0);
    wait_stage<BM, BN, FMT, ASYM, NW, NS - 2>(wave);  // tile kt+1 complete; tiles kt+2 .. kt+NS-1 may still fly
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();             // stage kt+1 visible; every wave holds its stage kt fragments
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // the remaining slice-0 MFMAs one per load slot, then the rest with the fragment reads of stage kt+1
    issue(kt % NS, kt + NS, [&](int q) { mfma_range(ca[0], cb[0], 2 + q, 3 + q); });
    mfma_range(ca[0], cb[0], 2 + NAL + NWL, NMF);
    dequant(1, cb, cq, cs, cz);
    read_frags((kt + 1) % NS, na, nb, nq, ns, nz);
    mfma_range(ca[1], cb[1], 0, NMF);
#pragma unroll
    for (int q = 0; q < 2 * (MI + NI); q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    // stage kt+1's first slice, under this stage's last MFMAs: the next step starts with MFMAs
    dequant(0, nb, nq, ns, nz);
  };

  // prologue: fill all NS stages (tiles 0..NS-1); step kt then refills stage kt % NS with tile kt + NS
  static_assert(NS == PD + 1, "ring of PD + 1 stages");
  half8_t fa0[2][MI], fb0[2][NI], fa1[2][MI], fb1[2][NI];
#pragma unroll
  for (int s = 0; s < NS; s++) issue(s, s, [](int) {});
  wait_stage<BM, BN, FMT, ASYM, NW, NS - 2>(wave);  // tiles 0 and 1 complete
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  read_frags(0, fa0, fb0, wq0, sc0, zc0);
  dequant(0, fb0, wq0, sc0, zc0);
  [[maybe_unused]] half4_t first[SPLIT2 ? NI : 1][SPLIT2 ? MI : 1][4];
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, fa0, fb0, fa1, fb1, wq0, sc0, zc0, wq1, sc1, zc1);
    if (kt + 1 < nk) step(kt + 1, fa1, fb1, fa0, fb0, wq1, sc1, zc1, wq0, sc0, zc0);
    if constexpr (SPLIT2) {
      if (kt + 2 == nk / 2) {  // first half of K done: keep its fp16 rounding, restart the accumulators
#pragma unroll
        for (int j = 0; j < NI; j++)
#pragma unroll
          for (int i = 0; i < MI; i++) {
#pragma unroll
            for (int q = 0; q < 4; q++)
              first[j][i][q] = (half4_t){(hxa_h)acc[j][i][4 * q], (hxa_h)acc[j][i][4 * q + 1], (hxa_h)acc[j][i][4 * q + 2],
                                         (hxa_h)acc[j][i][4 * q + 3]};
            acc[j][i] = (float16_t){};
          }
      }
    }
  }
  clk_store(p.clk, (int)(blockIdx.x + blockIdx.z * gridDim.x), tid, clk0);
  if constexpr (XATTN) {
    xattn_tail<MI, NI, WTM, WTN>(p, acc, m0, n0, tid, lane, wave, wm, wn, lds8);
    return;
  }
  wait_vm<0>();  // the trailing (dummy) tile loads must land before the epilogue reuses the LDS ring
  if constexpr (!SPLIT2) {
    if (p.epi == HXA_EPI_PARTIAL_F32) {  // no LDS staging and no prefetch (gemm_prepare rejects pf with it)
      store_partial_f32<MI, NI>(p, acc, m0 + wm * WTM + (lane & 31), n0 + wn * WTN + 4 * (lane >> 5), z);
      return;
    }
  }
  __syncthreads();
  if (p.pf_bytes > 0)
    prefetch_share(p, bid + z * p.tiles_m * p.tiles_n, p.tiles_m * p.tiles_n * (int)gridDim.z, tid, NT,
                   lds8 + G::LDS - G::PF_LDS);

  // ---- epilogue. Stage f16(acc) through LDS as a row-major [BM][CROW] tile: lane holds, for block (j, i),
  // row i*32 + (lane & 31) and columns j*32 + 8q + 4*(lane/32) + 0..3 (q = 0..3) -> one 8-byte write each.
  constexpr int CROW = G::CROW;
  hxa_h *Cs = (hxa_h *)lds8;
  {
    const int ml = wm * WTM + (lane & 31), nl = wn * WTN + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const half4_t v = {(hxa_h)acc[j][i][4 * q], (hxa_h)acc[j][i][4 * q + 1], (hxa_h)acc[j][i][4 * q + 2],
                             (hxa_h)acc[j][i][4 * q + 3]};
          *(half4_t *)(Cs + (ml + i * 32) * CROW + nl + j * 32 + 8 * q) = v;
          if constexpr (SPLIT2) *(half4_t *)(Cs + BM * CROW + (ml + i * 32) * CROW + nl + j * 32 + 8 * q) = first[j][i][q];
        }
  }
  __syncthreads();
  gemm_epilogue<BM, BN, NT, SPLIT2>(p, Cs, m0, n0, tid, z);
  if (p.pf_bytes > 0) wait_vm<0>();
}

template <int BM, int BN, int FMT, bool ASYM, bool SPLIT2 = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) void gemm_kernel(GemmParams p) {
  gemm_body<BM, BN, FMT, ASYM, SPLIT2, NW>(p, blockIdx.x, blockIdx.z);
}
// the cross-q projection with its attention (xattn_tail): 128 x 128 fp16 tiles, 4 waves
__global__ __launch_bounds__(256) void gemm_xattn_kernel(GemmParams p) {
  gemm_body<128, 128, HXA_W_F16, false, false, 4, true>(p, blockIdx.x, 0);
}
// two independent GEMMs of the same tile shape and weight format in one launch: workgroups [0, nwg0) run p0,
// the rest p1 (nwg0 a multiple of 8 keeps each GEMM's XCD placement)
template <int BM, int BN, int FMT, bool ASYM, int NW = 4>
__global__ __launch_bounds__(64 * NW) void gemm_pair_kernel(GemmParams p0, GemmParams p1, int nwg0) {
  if ((int)blockIdx.x < nwg0) gemm_body<BM, BN, FMT, ASYM, false, NW>(p0, blockIdx.x, 0);
  else gemm_body<BM, BN, FMT, ASYM, false, NW>(p1, blockIdx.x - nwg0, 0);
}

// Ping-pong GEMM, fp16 weights, 8 waves: two groups of 4 (one wave of each per SIMD). Group g owns columns
// [g BN/2, (g+1) BN/2) of the tile, its waves split them 2 x 2 (wave tile BM/2 x BN/4). The main loop runs in
// phases separated by one s_barrier: in each phase one group issues the MFMAs of a stage on fragments already in
// registers (s_setprio 1) while the other group reads the next stage's fragments from LDS -- group 1 also issues
// the global -> LDS loads, three stages ahead -- so one wave per SIMD keeps the matrix core fed while its partner
// waits on memory. Stage j: group 1 reads it in phase 2j and computes it in 2j+1; group 0 reads it in 2j+1 and
// computes it in 2j+2. The LDS ring, stage layout and epilogue are those of gemm_kernel.
// int8 / int4 weights: the memory phase also reads the raw weights and their scales (and offsets) and dequantises
// them into the fp16 fragments, so the compute phase is MFMAs only.
// PAIRED: the workgroup index within its GEMM is `bid` (the pair kernel); otherwise blockIdx.x (bid unused)
template <int BM, int BN, int FMT, bool ASYM, bool PAIRED>
HXA_DEV void gemm_pp_body(const GemmParams &p, const int bid_arg) {
  const int bid = PAIRED ? bid_arg : (int)blockIdx.x;
  if (!PAIRED && bid >= p.tiles_m * p.tiles_n) {  // an appended workgroup: side GEMV rows, no LDS and no barrier
    side_gemv<2>(p.side, (bid - p.tiles_m * p.tiles_n) * 8 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
              p.side_wgs * 8, threadIdx.x & 63);
    return;
  }
  using G = GemmGeo<BM, BN, FMT>;
  constexpr int NT = 512, NWG = 4;  // threads, waves per group
  // each group's 4 waves cover its BN / 2 columns as a 2 x 2 grid, or, for int8 / int4 weights on 256-wide tiles, as
  // 1 x 4 strips of 32 columns over all BM rows, so that no two waves of a group dequantise the same W fragment
  constexpr int WMW = (FMT != HXA_W_F16 && BN >= 256) ? 1 : 2;
  constexpr int WTM = BM / WMW, WTN = BN / 2 / (4 / WMW), MI = WTM / 32, NI = WTN / 32;
  constexpr int BK = G::BK, NS = G::NS;
  constexpr int NAI = BM / 16, TW = G::W_BYTES / 1024;       // 1 KB load instructions per stage (A, W)
  constexpr int LPS = (NAI + TW) / NWG;                     // per group-1 wave and stage (+ the vectors for wave 0)
  constexpr int NVEC = FMT == HXA_W_F16 ? 0 : (ASYM ? 2 : 1);
  static_assert(BM % 64 == 0 && WTN % 32 == 0 && NS == 4 && (NAI + TW) % NWG == 0 && NAI % NWG == 0 &&
                    G::W_BYTES % 1024 == 0 && (BN / 8) % NWG == 0,
                "tile shape");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds8[];

  int tm, tn;
  tile_coords(p, bid, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int z = blockIdx.z;
  const int kbase = z * p.Kslice;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, wl = wave & 3, wm = WMW == 2 ? (wl & 1) : 0, wn = WMW == 2 ? (wl >> 1) : wl;
  const int nk = p.Kslice / BK;
  const HxaClkMark clk0 = clk_mark(p.clk);

  // group 1: stage s <- k tile kt (clamped past the end: dummy reloads keep the vmcnt accounting constant)
  // per-lane offsets from the tile corner, fixed over the k loop (only group 1 issues loads)
  constexpr int NLP = (NAI + TW) / NWG;
  uint32_t loff[NLP];
#pragma unroll
  for (int j = 0; j < NLP; j++) {
    const int t = j * NWG + wl;
    loff[j] = t < NAI ? a_lane_off(p, t, lane, m0) : w_lane_off<FMT>(p, (t - NAI) * 64 + lane, n0);
  }
  auto issue = [&](int s, int kt) {
    uint8_t *st = lds8 + s * G::STAGE;
    const int k0 = kbase + min(kt, nk - 1) * BK;
    const uint8_t *ab = a_tile_base(p, m0, k0), *wb = w_tile_base<FMT>(p, n0, k0);
#pragma unroll
    for (int t0 = 0; t0 < NAI + TW; t0 += NWG) {
      const int t = t0 + wl;
      if (t < NAI) g2l16_sbase(ab, loff[t0 / NWG], st + t * 1024);
      else g2l16_sbase(wb, loff[t0 / NWG], st + G::A_BYTES + (t - NAI) * 1024);
    }
    if constexpr (NVEC > 0) {  // scale (and offset) vector of the stage's k group, 16-byte chunks over the 4 waves
      constexpr int CPW = BN / 8 / NWG;
      const int g = k0 >> 5, c = wl * CPW + lane, nn = min(n0 + c * 8, p.N - 8);
      uint8_t *ws = st + G::A_BYTES;
      if (lane < CPW) g2l16_opaque(p.S + (long)g * p.N + nn, ws + G::W_BYTES + 16 * wl * CPW);
      if (ASYM && lane < CPW) g2l16_opaque(p.Z + (long)g * p.N + nn, ws + G::W_BYTES + G::S_BYTES + 16 * wl * CPW);
    }
  };
  // wait until at most `later` further stages of this group-1 wave's loads are in flight (the same count in every
  // wave: no branch on the wave index in the loop)
  auto wait_later = [&](auto later_c) {
    constexpr int L = decltype(later_c)::value;
    wait_vm<L * (LPS + NVEC)>();
  };
  // Quantised W is read raw in the memory phase (wq, scale sc, offset zc). The first 16-deep slice is dequantised at
  // the end of the memory phase, once the reads have landed (the other group's MFMAs run meanwhile), so the compute
  // phase starts with MFMAs; the second slice's dequantisation issues under the first slice's MFMAs.
  typedef typename std::conditional<FMT == HXA_W_Q8, uint2_t, uint32_t>::type raw_t;
  [[maybe_unused]] raw_t wq[2][NI];
  [[maybe_unused]] hxa_h sc[NI], zc[NI];
  auto read_frags = [&](int s, half8_t (&fa)[2][MI], half8_t (&fb)[2][NI]) {
    const uint8_t *st = lds8 + s * G::STAGE;
    const uint8_t *ws = st + G::A_BYTES;
    const int h = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const int cl = kslot(ks, h);
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int row = wm * WTM + i * 32 + (lane & 31);
        fa[ks][i] = *(const half8_t *)(st + row * 64 + ((cl ^ ((row >> 2) & 3)) << 4));
      }
      if constexpr (FMT == HXA_W_F16) {
#pragma unroll
        for (int j = 0; j < NI; j++) {
          const int row = grp * (BN / 2) + wn * WTN + j * 32 + (lane & 31);
          fb[ks][j] = *(const half8_t *)(ws + row * 64 + ((cl ^ ((row >> 2) & 3)) << 4));
        }
      }
    }
    if constexpr (FMT != HXA_W_F16) {
#pragma unroll
      for (int j = 0; j < NI; j++) {
        const int row = grp * (BN / 2) + wn * WTN + j * 32 + (lane & 31);
        if constexpr (FMT == HXA_W_Q8) {
          wq[0][j] = read_wq8(ws, row, h, 0);
          wq[1][j] = read_wq8(ws, row, h, 1);
        } else {
          wq[0][j] = read_wq4(ws, row, h, 0);
          wq[1][j] = read_wq4(ws, row, h, 1);
        }
        sc[j] = *(const hxa_h *)(ws + G::W_BYTES + row * 2);
        zc[j] = ASYM ? *(const hxa_h *)(ws + G::W_BYTES + G::S_BYTES + row * 2) : (hxa_h)0.0f;
      }
    }
  };
  auto dequant = [&](int ks, int j, half8_t (&fb)[2][NI]) {
    if constexpr (FMT != HXA_W_F16) {
      const half2_t s2 = {sc[j], sc[j]};
      uint32_t o[4];
      if constexpr (FMT == HXA_W_Q8) {
        dq8_word(wq[ks][j].x, s2, o[0], o[1]);
        dq8_word(wq[ks][j].y, s2, o[2], o[3]);
      } else {
        const half2_t z2 = {zc[j], zc[j]};
        dq4_word<ASYM>(wq[ks][j], s2, z2, o);
      }
      fb[ks][j] = __builtin_bit_cast(half8_t, (uint4_t){o[0], o[1], o[2], o[3]});
    }
  };
  float16_t acc[NI][MI];
#pragma unroll
  for (int j = 0; j < NI; j++)
#pragma unroll
    for (int i = 0; i < MI; i++) acc[j][i] = (float16_t){};
  auto dequant0 = [&](half8_t (&fb)[2][NI]) {
    if constexpr (FMT != HXA_W_F16) {
#pragma unroll
      for (int j = 0; j < NI; j++) dequant(0, j, fb);
    }
  };
  auto mfmas = [&](const half8_t (&fa)[2][MI], half8_t (&fb)[2][NI]) {
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int j = 0; j < NI; j++) {
        if (ks == 0) dequant(1, j, fb);  // slice 1's fragment j, under slice 0's MFMAs
#pragma unroll
        for (int i = 0; i < MI; i++) acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fb[ks][j], fa[ks][i], acc[j][i], 0, 0, 0);
      }
  };
  auto bar = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // each group runs its own loop (one fragment buffer: read in one phase, consumed in the next); both loops pass
  // the same barriers, two per stage
  half8_t fa[2][MI], fb[2][NI];
  if (grp == 1) {
#pragma unroll
    for (int s = 0; s < NS; s++) issue(s, s);
    wait_later(std::integral_constant<int, NS - 1>{});  // stage 0 landed
    bar();
    for (int j = 0; j < nk; j++) {
      // phase 2j: read stage j, load stage j+3 into the buffer of stage j-1 (read by both groups by now)
      read_frags(j % NS, fa, fb);
      if (j >= 1) issue((j + NS - 1) % NS, j + NS - 1);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the fragments are in registers
      dequant0(fb);
      bar();
      // phase 2j+1: compute stage j, then wait for stage j+1 (stages j+2, j+3 may still fly)
      __builtin_amdgcn_s_setprio(1);
      mfmas(fa, fb);
      __builtin_amdgcn_s_setprio(0);
      wait_later(std::integral_constant<int, 2>{});
      bar();
    }
  } else {
    bar();
    for (int j = 0; j < nk; j++) {
      // phase 2j: compute stage j-1
      if (j >= 1) {
        __builtin_amdgcn_s_setprio(1);
        mfmas(fa, fb);
        __builtin_amdgcn_s_setprio(0);
      }
      bar();
      // phase 2j+1: read stage j
      read_frags(j % NS, fa, fb);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      dequant0(fb);
      bar();
    }
    // phase 2 nk: compute stage nk-1
    mfmas(fa, fb);
  }
  clk_store(p.clk, (int)(blockIdx.x + blockIdx.z * gridDim.x), tid, clk0);
  wait_vm<0>();  // the trailing (dummy) tile loads must land before the epilogue reuses the LDS ring
  if (p.epi == HXA_EPI_PARTIAL_F32) {  // no LDS staging and no prefetch (gemm_prepare rejects pf with it)
    store_partial_f32<MI, NI>(p, acc, m0 + wm * WTM + (lane & 31), n0 + grp * (BN / 2) + wn * WTN + 4 * (lane >> 5), z);
    return;
  }
  __syncthreads();
  if (p.pf_bytes > 0)
    prefetch_share(p, bid + z * p.tiles_m * p.tiles_n, p.tiles_m * p.tiles_n * (int)gridDim.z, tid, NT,
                   lds8 + G::LDS - G::PF_LDS);

  constexpr int CROW = G::CROW;
  hxa_h *Cs = (hxa_h *)lds8;
  {
    const int ml = wm * WTM + (lane & 31), nl = grp * (BN / 2) + wn * WTN + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < NI; j++)
#pragma unroll
      for (int i = 0; i < MI; i++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const half4_t v = {(hxa_h)acc[j][i][4 * q], (hxa_h)acc[j][i][4 * q + 1], (hxa_h)acc[j][i][4 * q + 2],
                             (hxa_h)acc[j][i][4 * q + 3]};
          *(half4_t *)(Cs + (ml + i * 32) * CROW + nl + j * 32 + 8 * q) = v;
        }
  }
  __syncthreads();
  gemm_epilogue<BM, BN, NT, false>(p, Cs, m0, n0, tid, z);
  if (p.pf_bytes > 0) wait_vm<0>();
}
template <int BM, int BN, int FMT = HXA_W_F16, bool ASYM = false>
__global__ __launch_bounds__(512) void gemm_pp_kernel(GemmParams p) {
  gemm_pp_body<BM, BN, FMT, ASYM, false>(p, 0);
}
// two independent GEMMs on the ping-pong kernel in one grid: workgroups [0, nwg0) run p0, the rest p1
template <int BM, int BN, int FMT, bool ASYM>
__global__ __launch_bounds__(512) void gemm_pp_pair_kernel(GemmParams p0, GemmParams p1, int nwg0) {
  if ((int)blockIdx.x < nwg0) gemm_pp_body<BM, BN, FMT, ASYM, true>(p0, blockIdx.x);
  else gemm_pp_body<BM, BN, FMT, ASYM, true>(p1, blockIdx.x - nwg0);
}
// G independent GEMMs of one tile shape and weight format on the ping-pong kernel, each with its own parameters
// (a device array): workgroup (x, y) runs tile x of GEMM y
template <int BM, int BN, int FMT, bool ASYM>
__global__ __launch_bounds__(512) void gemm_pp_group_kernel(const GemmParams *__restrict__ ps) {
  gemm_pp_body<BM, BN, FMT, ASYM, true>(ps[blockIdx.y], blockIdx.x);
}

// Tile cost model, per weight format (fp16, int8, int4): a launch of `waves` rounds of workgroups over the CUs takes
// about waves * (a * BM * BN * Kslice / 1e6 + b) + c microseconds. a, b, c >= 0 were fitted by least squares on the
// relative error to every tile timed on 78 projection shapes on a 256-CU MI355X: the qkv, attention-output, MLP-up
// and MLP-down projections of the 2B (hidden 2048), 2.9B-class (2560) and MOSS-class (3072, up-gate 16384) blocks
// at 384, 512, 1536 and 6656 rows, split-K 1 and 2 (and 4 at 1536 rows); a = 0 marks a tile that format does not
// use. nw 4: one wave per SIMD; nw 8: two (int8 / int4 dequantisation overlaps the other wave's MFMAs); nw 9: the
// ping-pong kernel. Over those shapes the picks came within 0.3% (fp16), 0.5% (int8) and 0.6% (int4) of the fastest
// tile's summed time; with the int8 / int4 wave strips (gemm_body, gemm_pp_body) within 1.3% and 2.7%.
struct TileCost {
  int bm, bn, nw;
  float a[3], b[3], c[3];
};
constexpr TileCost kTiles[] = {
    {192, 256, 4, {0.2807f, 0.4725f, 0.5084f}, {11.50f, 10.83f, 10.16f}, {0.00f, 0.00f, 0.00f}},
    {192, 192, 4, {0.3052f, 0.5077f, 0.5578f}, {10.33f, 8.85f, 8.12f}, {0.00f, 0.00f, 0.00f}},
    {256, 128, 4, {0.3446f, 0.4439f, 0.5133f}, {8.80f, 8.45f, 7.53f}, {0.00f, 0.00f, 0.00f}},
    {128, 256, 4, {0.3213f, 0.5315f, 0.6355f}, {8.75f, 7.92f, 7.10f}, {0.00f, 0.00f, 0.00f}},
    {192, 128, 4, {0.3855f, 0.5336f, 0.5665f}, {7.27f, 2.45f, 0.18f}, {0.00f, 4.06f, 7.37f}},
    {128, 128, 4, {0.4574f, 0.5958f, 0.5965f}, {2.89f, 0.00f, 0.00f}, {1.77f, 9.34f, 9.38f}},
    {128, 64, 4, {0.7533f, 0.7707f, 0.0000f}, {0.99f, 0.00f, 0.00f}, {1.63f, 6.60f, 0.00f}},
    {64, 128, 4, {0.6581f, 0.8466f, 0.8716f}, {0.49f, 0.00f, 0.00f}, {3.68f, 10.92f, 11.58f}},
    {192, 256, 8, {0.3002f, 0.3773f, 0.4420f}, {9.65f, 8.92f, 8.16f}, {0.00f, 0.00f, 0.00f}},
    {128, 256, 8, {0.3256f, 0.4574f, 0.5409f}, {7.24f, 6.43f, 5.79f}, {0.00f, 0.00f, 0.00f}},
    {192, 128, 8, {0.4581f, 0.6220f, 0.5743f}, {6.41f, 5.54f, 1.68f}, {0.00f, 0.00f, 3.79f}},
    {128, 128, 8, {0.4755f, 0.6311f, 0.6435f}, {2.77f, 0.81f, 0.10f}, {1.43f, 5.34f, 6.45f}},
    {256, 256, 9, {0.2712f, 0.3157f, 0.3321f}, {10.91f, 9.85f, 9.27f}, {0.00f, 0.00f, 0.00f}},
    {192, 256, 9, {0.3042f, 0.3781f, 0.4006f}, {8.70f, 7.83f, 7.13f}, {0.00f, 0.00f, 0.00f}},
    {128, 256, 9, {0.3726f, 0.5011f, 0.5641f}, {6.15f, 0.66f, 0.00f}, {0.00f, 5.56f, 7.60f}},
    {128, 128, 9, {0.5054f, 0.6590f, 0.0000f}, {1.74f, 0.00f, 0.00f}, {3.42f, 9.07f, 0.00f}},
    {192, 128, 9, {0.4632f, 0.5685f, 0.0000f}, {5.52f, 0.82f, 0.00f}, {0.00f, 4.96f, 0.00f}},
    {256, 128, 9, {0.3952f, 0.4634f, 0.0000f}, {6.39f, 6.27f, 0.00f}, {0.00f, 0.00f, 0.00f}},
};

template <int BM, int BN, int FMT, bool ASYM, bool SPLIT2 = false, int NW = 4>
hipError_t launch_t(const GemmParams &p, int ksplit, hipStream_t st) {
  auto kern = gemm_kernel<BM, BN, FMT, ASYM, SPLIT2, NW>;
  using G = GemmGeo<BM, BN, FMT>;
  const int lds = SPLIT2 && 2 * G::C_BYTES > G::LDS ? 2 * G::C_BYTES : G::LDS;
  constexpr bool erf_ok = !SPLIT2 && G::ERF_FITS;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       erf_ok ? G::LDS + ERF_T2_LDS_BYTES : lds);
    if (e != hipSuccess) return e;
    attr = true;
  }
  dim3 grid(p.tiles_m * p.tiles_n, 1, ksplit);
  if (erf_ok && p.epi == HXA_EPI_GELU_ERF && p.erf_t2 != nullptr) {  // the T2 table past the kernel's own LDS
    GemmParams pe = p;
    pe.erf_lds = G::LDS;
    hxa_launch(kern, grid, dim3(64 * NW), G::LDS + ERF_T2_LDS_BYTES, st, pe);
  } else {
    hxa_launch(kern, grid, dim3(64 * NW), lds, st, p);
  }
  return hipGetLastError();
}

template <int FMT, bool ASYM>
hipError_t launch_split2(int bm, int bn, const GemmParams &p, hipStream_t st) {
  if (bm == 128 && bn == 128) return launch_t<128, 128, FMT, ASYM, true>(p, 1, st);
  if (bm == 64 && bn == 128) return launch_t<64, 128, FMT, ASYM, true>(p, 1, st);
  return hipErrorInvalidValue;
}

template <int BM, int BN, int FMT, bool ASYM>
hipError_t launch_pp(const GemmParams &p, int ksplit, hipStream_t st) {
  auto kern = gemm_pp_kernel<BM, BN, FMT, ASYM>;
  using G = GemmGeo<BM, BN, FMT>;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       G::ERF_FITS ? G::LDS + ERF_T2_LDS_BYTES : G::LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  dim3 grid(p.tiles_m * p.tiles_n + (ksplit == 1 ? p.side_wgs : 0), 1, ksplit);
  if (G::ERF_FITS && p.epi == HXA_EPI_GELU_ERF && p.erf_t2 != nullptr) {  // the T2 table past the kernel's own LDS
    GemmParams pe = p;
    pe.erf_lds = G::LDS;
    hxa_launch(kern, grid, dim3(512), G::LDS + ERF_T2_LDS_BYTES, st, pe);
  } else {
    hxa_launch(kern, grid, dim3(512), G::LDS, st, p);
  }
  return hipGetLastError();
}

template <int FMT, bool ASYM>
hipError_t launch_fmt(int bm, int bn, int nw, const GemmParams &p, int ksplit, hipStream_t st) {
  if (nw == 9) {  // ping-pong 8 waves
    if (bm == 192 && bn == 256) return launch_pp<192, 256, FMT, ASYM>(p, ksplit, st);
    if (bm == 256 && bn == 256) return launch_pp<256, 256, FMT, ASYM>(p, ksplit, st);
    if (bm == 128 && bn == 256) return launch_pp<128, 256, FMT, ASYM>(p, ksplit, st);
    if constexpr (FMT != HXA_W_Q4) {
      if (bm == 128 && bn == 128) return launch_pp<128, 128, FMT, ASYM>(p, ksplit, st);
      if (bm == 192 && bn == 128) return launch_pp<192, 128, FMT, ASYM>(p, ksplit, st);
      if (bm == 256 && bn == 128) return launch_pp<256, 128, FMT, ASYM>(p, ksplit, st);
    }
    return hipErrorInvalidValue;
  }
  if (nw == 8) {
    if (bm == 192 && bn == 256) return launch_t<192, 256, FMT, ASYM, false, 8>(p, ksplit, st);
    if (bm == 192 && bn == 128) return launch_t<192, 128, FMT, ASYM, false, 8>(p, ksplit, st);
    if (bm == 128 && bn == 256) return launch_t<128, 256, FMT, ASYM, false, 8>(p, ksplit, st);
    if (bm == 128 && bn == 128) return launch_t<128, 128, FMT, ASYM, false, 8>(p, ksplit, st);
    return hipErrorInvalidValue;  // (kTiles lists the shapes instantiated here)
  }
  if (bm == 192 && bn == 256) return launch_t<192, 256, FMT, ASYM>(p, ksplit, st);
  if (bm == 192 && bn == 192) return launch_t<192, 192, FMT, ASYM>(p, ksplit, st);
  if (bm == 192 && bn == 128) return launch_t<192, 128, FMT, ASYM>(p, ksplit, st);
  if (bm == 256 && bn == 128) return launch_t<256, 128, FMT, ASYM>(p, ksplit, st);
  if (bm == 128 && bn == 256) return launch_t<128, 256, FMT, ASYM>(p, ksplit, st);
  if (bm == 128 && bn == 128) return launch_t<128, 128, FMT, ASYM>(p, ksplit, st);
  if (bm == 64 && bn == 128) return launch_t<64, 128, FMT, ASYM>(p, ksplit, st);
  if constexpr (FMT != HXA_W_Q4) {
    if (bm == 128 && bn == 64) return launch_t<128, 64, FMT, ASYM>(p, ksplit, st);
  }
  return hipErrorInvalidValue;
}

// CUs of the device current at the first call (read once, thread-safe; 256 when the query fails)
int num_cu() {
  static const int n = [] {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    return hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0 ? c : 256;
  }();
  return n;
}

}  // namespace

// Choose the tile of least modelled time (kTiles). HXA_EPI_RESADD_SPLIT2 keeps both K halves' accumulators in
// registers and runs on the 4-wave 128x128 / 64x128 tiles only (ranked with the fp16 costs).
static void pick_tile(int M, int N, int K, int ksplit, int fmt, int epi, int hn_cols, int *bm, int *bn, int *nw) {
  const bool headnorm = hn_cols > 0;
  const bool split2 = epi == HXA_EPI_RESADD_SPLIT2;
  const int ncu = num_cu();
  const int f = split2 ? 0 : fmt;
  double best = -1.0;
  for (const TileCost &c : kTiles) {
    if (c.a[f] == 0.0f) continue;
    if (split2 && !(c.bn == 128 && (c.bm == 128 || c.bm == 64) && c.nw == 4)) continue;  // register budget
    if (fmt == HXA_W_Q4 && c.bn < 128) continue;
    if (epi == HXA_EPI_SITU && c.bn % 128 != 0) continue;  // each wave needs whole (up, gate) block pairs
    if (headnorm && (c.bn % 128 != 0 || (hn_cols % c.bn != 0 && hn_cols < N))) continue;  // whole head-normed tiles
    const long tiles = (long)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * ksplit;
    const long waves = (tiles + ncu - 1) / ncu;
    const double t = (double)waves * (c.a[f] * 1e-6 * c.bm * c.bn * (double)(K / ksplit) + c.b[f]) + c.c[f];
    if (best < 0.0 || t < best - 1e-9) {
      best = t;
      *bm = c.bm;
      *bn = c.bn;
      *nw = c.nw;
    }
  }
}

// the modelled time (us) of the tile pick_tile chooses for a plain-store GEMM with ksplit slices
static double tile_time(int M, int N, int K, int ksplit, int fmt) {
  int bm = 128, bn = 128, nw = 4;
  pick_tile(M, N, K, ksplit, fmt, HXA_EPI_STORE, 0, &bm, &bn, &nw);
  const int ncu = num_cu();
  for (const TileCost &c : kTiles) {
    if (c.bm != bm || c.bn != bn || c.nw != nw) continue;
    const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * ksplit;
    return (double)((tiles + ncu - 1) / ncu) * (c.a[fmt] * 1e-6 * bm * bn * (double)(K / ksplit) + c.b[fmt]) + c.c[fmt];
  }
  return 1e30;
}
// split-K linear cost terms: the sum kernel's launch and kernel boundary (us), the bytes per us of the slices' round
// trip through L2 / MALL, and the factor by which a split form must beat the one-launch model
constexpr double kSumLaunchUs = 4.0, kSumBytesPerUs = 8.0e6, kSplitGain = 0.95;

// the tiles launch_fmt has kernels for (split2: launch_split2's)
static bool tile_built(int bm, int bn, int nw, int fmt, bool split2) {
  if (split2) return nw == 4 && bn == 128 && (bm == 128 || bm == 64);
  const bool q4 = fmt == HXA_W_Q4;
  if (nw == 9) return (bn == 256 && (bm == 256 || bm == 192 || bm == 128)) || ((bm == 128 || bm == 192 || bm == 256) && bn == 128 && !q4);
  if (nw == 8) return (bm == 192 || bm == 128) && (bn == 256 || bn == 128);
  if (nw != 4) return false;
  if (bm == 128 && bn == 64) return !q4;
  return (bm == 192 && (bn == 256 || bn == 192 || bn == 128)) || (bm == 256 && bn == 128) ||
         (bm == 128 && (bn == 256 || bn == 128)) || (bm == 64 && bn == 128);
}

// The device address of the GELU-erf T2 table on the current device, filled on first use there (a launch of
// erf_t2_kernel on `st`, waited for, so the table is complete for every later launch on any stream). Under stream
// capture an unfilled table is not filled (the epilogue then evaluates erfcf): null.
const hxa_h *erf_table(hipStream_t st) {
  static const hxa_h *tab[HXA_MAX_DEVICES];
  static std::mutex mu;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= HXA_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lk(mu);
  if (tab[dev]) return tab[dev];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
  void *ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(g_erf_t2)) != hipSuccess || ptr == nullptr) return nullptr;
  hxa_launch(erf_t2_kernel, dim3(ERF_T2_N / 256), dim3(256), 0, st, (hxa_h *)ptr);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) return nullptr;
  tab[dev] = (const hxa_h *)ptr;
  return tab[dev];
}

// validate a GEMM description, fill its kernel parameters and choose (or take the forced) tile
static int gemm_prepare(const HxaGemm &g, GemmParams &p, int &bm, int &bn, int &nw, HxaWeight &w, bool &split2) {
  w = *g.w;
  const int wkt = (w.fmt & HXA_W_KTILED) ? 1 : 0;
  w.fmt &= ~HXA_W_KTILED;
  if (g.M <= 0 || w.N <= 0 || w.K <= 0 || g.ksplit < 1) return HXA_E_ARG;
  if (w.K % (32 * g.ksplit) != 0) return HXA_E_ARG;
  if (w.fmt != HXA_W_F16 && w.s == nullptr) return HXA_E_ARG;
  if (g.epi == HXA_EPI_SITU && (w.N % 64) != 0) return HXA_E_ARG;
  if ((g.lda % 8) != 0 || ((uintptr_t)g.A % 16) != 0 || ((uintptr_t)w.w % 16) != 0) return HXA_E_ARG;
  if (w.N % 8 != 0) return HXA_E_ARG;  // 16-byte epilogue chunks
  split2 = g.epi == HXA_EPI_RESADD_SPLIT2;
  if (split2 && (g.ksplit != 1 || w.K % 128 != 0)) return HXA_E_ARG;  // two halves of whole k-step pairs
  if (g.epi == HXA_EPI_RESADD || split2
          ? ((g.ldx % 8) != 0 || ((uintptr_t)g.x % 32) != 0 || ((uintptr_t)g.gate % 32) != 0)
          : ((g.ldo % (g.epi == HXA_EPI_PARTIAL_F32 ? 4 : 8)) != 0 || ((uintptr_t)g.out % 16) != 0))
    return HXA_E_ARG;
  const bool f32 = g.epi == HXA_EPI_PARTIAL_F32;
  if (f32 && (g.out_t != nullptr || g.hn_cols > 0 || g.pf_bytes > 0 || g.side != nullptr)) return HXA_E_ARG;
  p = GemmParams{};
  if (g.epi == HXA_EPI_STORE_T) {  // all columns transposed
    p.out_t = g.out;
    p.ldo_t = g.ldo;
    p.split_col = 0;
  } else if (g.epi == HXA_EPI_STORE && g.out_t != nullptr) {  // fused projections: the tail columns transposed
    if (g.split_col % 32 != 0 || g.split_col < 0 || g.split_col > w.N) return HXA_E_ARG;
    p.out_t = g.out_t;
    p.ldo_t = g.ldo_t;
    p.split_col = g.split_col;
  }
  if (p.out_t != nullptr && ((p.ldo_t % 8) != 0 || ((uintptr_t)p.out_t % 16) != 0)) return HXA_E_ARG;
  p.A = g.A;
  p.lda = g.lda;
  p.W = w.w;
  p.S = w.s;
  p.Z = w.z;
  {
    const long cb = w.fmt == HXA_W_Q4 ? 16 : 32;  // elements (q4: bytes) of one row's k group
    p.w_rs = wkt ? cb : (long)w.K / 32 * cb;
    p.w_gs = wkt ? cb * w.N : cb;
  }
  // the loaders' per-lane offsets within a tile (up to 256 rows) are 32-bit: keep them below 2^31
  if (g.lda >= (1L << 22) || p.w_rs * (w.fmt == HXA_W_F16 ? 2 : 1) >= (1L << 23)) return HXA_E_ARG;
  p.M = g.M;
  p.N = w.N;
  p.Ktot = w.K;
  p.Kslice = w.K / g.ksplit;
  p.epi = split2 ? HXA_EPI_RESADD : g.epi;
  p.out = g.epi == HXA_EPI_STORE_T || f32 ? nullptr : g.out;
  p.out32 = f32 ? (float *)g.out : nullptr;
  p.ldo = g.ldo;
  p.out_zstride = g.out_zstride;
  p.x = g.x;
  p.ldx = g.ldx;
  p.gate = g.gate;
  const bool headnorm = g.hn_cols > 0;
  if (headnorm) {
    if (g.epi != HXA_EPI_STORE || g.ksplit != 1 || g.hn_cols % 128 || w.N % 128 || !g.hn_g0 || !g.hn_g1 ||
        (g.hn_cos && (!g.hn_sin || g.hn_ttab <= 0)) || ((uintptr_t)g.hn_g0 | (uintptr_t)g.hn_g1) % 16 ||
        (g.out_t && (g.split_col % 128 || g.split_col < g.hn_cols)))
      return HXA_E_ARG;
  }
  p.hn_cols = headnorm ? min(g.hn_cols, w.N) : 0;
  p.hn_gsplit = g.hn_gsplit;
  p.hn_ttab = g.hn_ttab;
  p.hn_g0 = g.hn_g0;
  p.hn_g1 = g.hn_g1;
  p.hn_cos = g.hn_cos;
  p.hn_sin = g.hn_sin;
  // the prefetch rides on epilogues that issue no loads of their own (their waits would wait for it too)
  if (g.pf_bytes > 0 && (g.pf == nullptr || g.pf_bytes < 4 || ((uintptr_t)g.pf & 3) || headnorm ||
                         g.epi == HXA_EPI_RESADD || split2))
    return HXA_E_ARG;
  p.pf = (const uint8_t *)g.pf;
  p.pf_bytes = g.pf_bytes > 0 ? g.pf_bytes : 0;
  p.clk = g_hxa_clk_gemm;
  bm = 128;
  bn = 128;
  nw = 4;
  pick_tile(g.M, w.N, w.K, g.ksplit, w.fmt, g.epi, headnorm ? min(g.hn_cols, w.N) : 0, &bm, &bn, &nw);
  if (g.force_bm) {
    bm = g.force_bm;
    bn = g.force_bn;
    nw = g.force_nw ? g.force_nw : 4;
    if (!tile_built(bm, bn, nw, w.fmt, split2)) return HXA_E_ARG;
    if ((g.epi == HXA_EPI_SITU && bn % 128 != 0) || (w.fmt == HXA_W_Q4 && bn < 128)) return HXA_E_ARG;
    if (headnorm && (bn % 128 != 0 || (p.hn_cols % bn != 0 && p.hn_cols < w.N))) return HXA_E_ARG;
  }
  p.tiles_m = (g.M + bm - 1) / bm;
  p.tiles_n = (w.N + bn - 1) / bn;
  // 8 XCD rectangles of the fewest A + W bytes per k step (each XCD's L2 then serves its CUs' shared rows)
  p.xcd_gm = 0;
  {
    const long wrow = w.fmt == HXA_W_F16 ? 64 : (w.fmt == HXA_W_Q8 ? 32 : 16);
    long best = -1;
    for (int gm = 1; gm <= 8; gm *= 2) {
      if (p.tiles_m % gm || p.tiles_n % (8 / gm)) continue;
      const long bytes = (long)(p.tiles_m / gm) * bm * 64 + (long)(p.tiles_n / (8 / gm)) * bn * wrow;
      if (best < 0 || bytes < best) {
        best = bytes;
        p.xcd_gm = gm;
      }
    }
  }
  return HXA_OK;
}

int hxa_gemm_launch(const HxaGemm &g, hipStream_t st) {
  GemmParams p;
  int bm, bn, nw;
  HxaWeight w;
  bool split2;
  const int r = gemm_prepare(g, p, bm, bn, nw, w, split2);
  if (r != HXA_OK) return r;
  if (g.epi == HXA_EPI_GELU_ERF) p.erf_t2 = erf_table(st);
  hipError_t e;
  if (split2) {
    if (w.fmt == HXA_W_F16) e = launch_split2<HXA_W_F16, false>(bm, bn, p, st);
    else if (w.fmt == HXA_W_Q8) e = launch_split2<HXA_W_Q8, false>(bm, bn, p, st);
    else if (w.z) e = launch_split2<HXA_W_Q4, true>(bm, bn, p, st);
    else e = launch_split2<HXA_W_Q4, false>(bm, bn, p, st);
    return e == hipSuccess ? HXA_OK : HXA_E_HIP;
  }
  // a side GEMV rides in the CUs the ping-pong grid leaves idle in its last round (at least 16 of them), else it
  // runs as its own launch after the GEMM
  bool side_after = false;
  if (g.side != nullptr) {
    const HxaSideGemv &sg = *g.side;
    if (!hxa_side_k_ok(sg.K) || sg.N <= 0 || sg.per <= 0 || !sg.x || !sg.W || !sg.y ||
        ((uintptr_t)sg.x | (uintptr_t)sg.W) % 16)
      return HXA_E_ARG;
    const int ncu = num_cu(), tiles = p.tiles_m * p.tiles_n, idle = (tiles + ncu - 1) / ncu * ncu - tiles;
    if (nw == 9 && g.ksplit == 1 && idle >= 16) {
      p.side = sg;
      p.side_wgs = idle;
    } else {
      side_after = true;
    }
  }
  if (w.fmt == HXA_W_F16) e = launch_fmt<HXA_W_F16, false>(bm, bn, nw, p, g.ksplit, st);
  else if (w.fmt == HXA_W_Q8) e = launch_fmt<HXA_W_Q8, false>(bm, bn, nw, p, g.ksplit, st);
  else if (w.z) e = launch_fmt<HXA_W_Q4, true>(bm, bn, nw, p, g.ksplit, st);
  else e = launch_fmt<HXA_W_Q4, false>(bm, bn, nw, p, g.ksplit, st);
  if (e != hipSuccess) return HXA_E_HIP;
  if (side_after) {
    const HxaSideGemv &sg = *g.side;
    return hxa_modgemv_launch(sg.x, sg.K, sg.W, sg.N, sg.y, sg.per, sg.ostride, sg.split, sg.gap, sg.act, st);
  }
  return HXA_OK;
}

template <int BM, int BN, int FMT, bool ASYM, int NW>
hipError_t launch_pair_t(const GemmParams &p0, const GemmParams &p1, hipStream_t st) {
  auto kern = gemm_pair_kernel<BM, BN, FMT, ASYM, NW>;
  using G = GemmGeo<BM, BN, FMT>;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const int n0 = p0.tiles_m * p0.tiles_n;
  hxa_launch(kern, dim3(n0 + p1.tiles_m * p1.tiles_n), dim3(64 * NW), G::LDS, st, p0, p1, n0);
  return hipGetLastError();
}
template <int BM, int BN, int FMT, bool ASYM>
hipError_t launch_pp_pair_t(const GemmParams &p0, const GemmParams &p1, hipStream_t st) {
  auto kern = gemm_pp_pair_kernel<BM, BN, FMT, ASYM>;
  using G = GemmGeo<BM, BN, FMT>;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  const int n0 = p0.tiles_m * p0.tiles_n;
  hxa_launch(kern, dim3(n0 + p1.tiles_m * p1.tiles_n), dim3(512), G::LDS, st, p0, p1, n0);
  return hipGetLastError();
}
template <int FMT, bool ASYM>
hipError_t launch_pair_fmt(int bm, int bn, int nw, const GemmParams &p0, const GemmParams &p1, hipStream_t st) {
  if (bm == 128 && bn == 128 && nw == 4) return launch_pair_t<128, 128, FMT, ASYM, 4>(p0, p1, st);
  if (bm == 128 && bn == 128 && nw == 8) return launch_pair_t<128, 128, FMT, ASYM, 8>(p0, p1, st);
  if (bm == 192 && bn == 256 && nw == 9) return launch_pp_pair_t<192, 256, FMT, ASYM>(p0, p1, st);
  return hipErrorInvalidValue;
}

long hxa_gemm_group_param_bytes(int G) { return (long)G * (long)sizeof(GemmParams); }

int hxa_gemm_group_prepare(const HxaGemm *g, int G, void *params_host, int *tiles, int *fmt) {
  if (G < 1 || !g || !params_host || !tiles || !fmt) return HXA_E_ARG;
  GemmParams *ps = (GemmParams *)params_host;
  for (int i = 0; i < G; i++) {
    if (g[i].ksplit != 1 || g[i].pf_bytes > 0 || g[i].M != g[0].M || !g[i].w || !g[0].w || g[i].w->N != g[0].w->N ||
        g[i].w->K != g[0].w->K || (g[i].w->fmt & ~HXA_W_KTILED) != (g[0].w->fmt & ~HXA_W_KTILED) ||
        (g[i].w->z != nullptr) != (g[0].w->z != nullptr))
      return HXA_E_ARG;
    HxaGemm gf = g[i];
    gf.force_bm = 192;
    gf.force_bn = 256;
    gf.force_nw = 9;
    int bm, bn, nw;
    HxaWeight w;
    bool split2;
    const int r = gemm_prepare(gf, ps[i], bm, bn, nw, w, split2);
    if (r != HXA_OK) return r;
    if (split2 || bm != 192 || bn != 256 || nw != 9) return HXA_E_ARG;
    ps[i].clk = HxaClk{nullptr, 0};  // the parameters outlive any clock record
    *fmt = w.fmt | (w.z ? 0x100 : 0);
  }
  *tiles = ps[0].tiles_m * ps[0].tiles_n;
  return HXA_OK;
}

namespace {
template <int FMT, bool ASYM>
hipError_t launch_group_t(const GemmParams *ps, int G, int tiles, hipStream_t st) {
  auto kern = gemm_pp_group_kernel<192, 256, FMT, ASYM>;
  using Geo = GemmGeo<192, 256, FMT>;
  static bool attr = false;
  if (!attr) {
    hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, Geo::LDS);
    if (e != hipSuccess) return e;
    attr = true;
  }
  hxa_launch(kern, dim3(tiles, G), dim3(512), Geo::LDS, st, ps);
  return hipGetLastError();
}
}  // namespace

int hxa_gemm_group_launch(const void *params_dev, int G, int tiles, int fmt, hipStream_t st) {
  if (!params_dev || G < 1 || G > 65535 || tiles < 1) return HXA_E_ARG;
  const GemmParams *ps = (const GemmParams *)params_dev;
  hipError_t e;
  switch (fmt) {
    case HXA_W_F16: e = launch_group_t<HXA_W_F16, false>(ps, G, tiles, st); break;
    case HXA_W_Q8: e = launch_group_t<HXA_W_Q8, false>(ps, G, tiles, st); break;
    case HXA_W_Q4: e = launch_group_t<HXA_W_Q4, false>(ps, G, tiles, st); break;
    case HXA_W_Q4 | 0x100: e = launch_group_t<HXA_W_Q4, true>(ps, G, tiles, st); break;
    default: return HXA_E_ARG;
  }
  return e == hipSuccess ? HXA_OK : HXA_E_HIP;
}

bool hxa_gemm_pair_fits(const HxaGemm &g0, const HxaGemm &g1) {
  GemmParams p0, p1;
  int bm, bn, nw, bm1, bn1, nw1;
  HxaWeight w0, w1;
  bool s0, s1;
  if (gemm_prepare(g0, p0, bm, bn, nw, w0, s0) != HXA_OK || s0 || g0.ksplit != 1 || g1.ksplit != 1) return false;
  if (!((bm == 128 && bn == 128 && nw != 9) || (bm == 192 && bn == 256 && nw == 9)) || (p0.tiles_m * p0.tiles_n) % 8)
    return false;
  HxaGemm g1f = g1;
  g1f.force_bm = bm;
  g1f.force_bn = bn;
  g1f.force_nw = nw;
  if (gemm_prepare(g1f, p1, bm1, bn1, nw1, w1, s1) != HXA_OK || s1 || w0.fmt != w1.fmt || (w0.z != nullptr) != (w1.z != nullptr))
    return false;
  const long n0 = (long)p0.tiles_m * p0.tiles_n, n1 = (long)p1.tiles_m * p1.tiles_n;
  const long c = num_cu();
  return (n0 + n1 + c - 1) / c == (n0 + c - 1) / c;
}

bool hxa_gemm_xattn_fits(int M, int N) {
  return (long)((M + 127) / 128) * ((N + 127) / 128) <= num_cu();
}

int hxa_gemm_xattn_launch(const HxaGemm &g, const HxaXAttn &a, hipStream_t st) {
  if (g.side != nullptr) return HXA_E_ARG;  // (no side GEMV: only hxa_gemm_launch hosts one)
  if (g.w == nullptr || (g.w->fmt & ~HXA_W_KTILED) != HXA_W_F16 || g.epi != HXA_EPI_STORE || g.ksplit != 1 ||
      g.hn_cols < g.w->N || g.hn_cos != nullptr || g.out_t != nullptr || g.pf_bytes > 0)
    return HXA_E_ARG;
  // (NKV % 8: a V^T chunk of 8 keys that starts below NKV ends within it)
  if (a.T <= 0 || a.T % 128 || g.M % a.T || g.w->N % 128 || a.NKV < 1 || a.NKV % 8 || a.nvalid < 1 || a.nvalid > a.NKV ||
      !a.k || !a.vt || !a.o)
    return HXA_E_ARG;
  if ((a.ldk % 8) || (a.ldvt % 8) || (a.ldo % 4) || a.ldvt < a.NKV || (((uintptr_t)a.k | (uintptr_t)a.vt) % 16) ||
      ((uintptr_t)a.o % 8) || (a.kb % 8) || (a.vb % 8) || a.ldk >= (1L << 24) || a.ldvt >= (1L << 23))
    return HXA_E_ARG;
  HxaGemm gf = g;
  gf.force_bm = 128;
  gf.force_bn = 128;
  gf.force_nw = 4;
  GemmParams p;
  int bm, bn, nw;
  HxaWeight w;
  bool split2;
  const int r = gemm_prepare(gf, p, bm, bn, nw, w, split2);
  if (r != HXA_OK) return r;
  p.xa_k = a.k;
  p.xa_vt = a.vt;
  p.xa_o = a.o;
  p.xa_ldk = a.ldk;
  p.xa_ldvt = a.ldvt;
  p.xa_ldo = a.ldo;
  p.xa_kb = a.kb;
  p.xa_vb = a.vb;
  p.xa_nkv = a.NKV;
  p.xa_nvalid = a.nvalid;
  p.xa_T = a.T;
  constexpr int LDS = GemmGeo<128, 128, HXA_W_F16>::LDS > XA_LDS ? GemmGeo<128, 128, HXA_W_F16>::LDS : XA_LDS;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void *)gemm_xattn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, LDS) != hipSuccess)
      return HXA_E_HIP;
    attr = true;
  }
  hxa_launch(gemm_xattn_kernel, dim3(p.tiles_m * p.tiles_n), dim3(256), LDS, st, p);
  return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
}

int hxa_gemm_plan(const HxaGemm &g, int *bm, int *bn, int *nw, int *rounds) {
  GemmParams p;
  HxaWeight w;
  bool split2;
  const int r = gemm_prepare(g, p, *bm, *bn, *nw, w, split2);
  if (r != HXA_OK) return r;
  const long n = (long)p.tiles_m * p.tiles_n * g.ksplit;
  *rounds = (int)((n + num_cu() - 1) / num_cu());
  return HXA_OK;
}

int hxa_gemm_pair_launch(const HxaGemm &g0, const HxaGemm &g1, hipStream_t st) {
  if (g0.side != nullptr || g1.side != nullptr) return HXA_E_ARG;  // (only hxa_gemm_launch hosts a side GEMV)
  GemmParams p0, p1;
  int bm, bn, nw, bm1, bn1, nw1;
  HxaWeight w0, w1;
  bool s0, s1;
  int r = gemm_prepare(g0, p0, bm, bn, nw, w0, s0);
  if (r != HXA_OK) return r;
  hipError_t e = hipErrorInvalidValue;
  // paired on the 128x128 4- / 8-wave tiles and the 192x256 ping-pong tile; the second GEMM then takes the first
  // one's tile. The ping-pong pair only where the second GEMM's tiles fit in the CUs the first leaves idle: a
  // further round of 192x256 tiles is slower than the second GEMM's own launch (6144 x 2048 cross q + 512-row text
  // k / v: 79 us paired, 70 us as two launches)
  if (((bm == 128 && bn == 128 && nw != 9) || (bm == 192 && bn == 256 && nw == 9)) && !s0 && g0.ksplit == 1 &&
      g1.ksplit == 1 && (p0.tiles_m * p0.tiles_n) % 8 == 0) {
    HxaGemm g1f = g1;
    g1f.force_bm = bm;
    g1f.force_bn = bn;
    g1f.force_nw = nw;
    r = gemm_prepare(g1f, p1, bm1, bn1, nw1, w1, s1);
    if (r != HXA_OK) return r;
    if (g0.epi == HXA_EPI_GELU_ERF) p0.erf_t2 = erf_table(st);
    if (g1.epi == HXA_EPI_GELU_ERF) p1.erf_t2 = erf_table(st);
    const long n0 = (long)p0.tiles_m * p0.tiles_n, n1 = (long)p1.tiles_m * p1.tiles_n;
    const long c = num_cu();
    const bool extra_round = (n0 + n1 + c - 1) / c > (n0 + c - 1) / c;
    if (w0.fmt == w1.fmt && (w0.z != nullptr) == (w1.z != nullptr) && !s1 && !(nw == 9 && extra_round)) {
      if (w0.fmt == HXA_W_F16) e = launch_pair_fmt<HXA_W_F16, false>(bm, bn, nw, p0, p1, st);
      else if (w0.fmt == HXA_W_Q8) e = launch_pair_fmt<HXA_W_Q8, false>(bm, bn, nw, p0, p1, st);
      else if (w0.z) e = launch_pair_fmt<HXA_W_Q4, true>(bm, bn, nw, p0, p1, st);
      else e = launch_pair_fmt<HXA_W_Q4, false>(bm, bn, nw, p0, p1, st);
    }
  }
  if (e == hipErrorInvalidValue) {  // not pairable: two launches, each on its own tile
    r = hxa_gemm_launch(g0, st);
    return r != HXA_OK ? r : hxa_gemm_launch(g1, st);
  }
  return e == hipSuccess ? HXA_OK : HXA_E_HIP;
}

// ---- int8 / int4 weights -> fp16, k-tiled [K/32][N][32] (the layout the fp16 kernels read) ----
// One 8-k slot of one row per thread (the 16-byte fragment unit of the main loops), dequantised with their own
// dq8_word / dq4_word, so the values are the same f16(q * s) (+ z) bits the fused path feeds its MFMAs. Reads
// w.w / w.s / w.z once (the weights with non-temporal loads), writes 2 N K bytes.
namespace {
template <int FMT, bool ASYM>
__global__ __launch_bounds__(256) void dequant_kernel(GemmParams p, hxa_h *out) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;  // 8-k slot c = t % 4 of group i = t / 4 (g = i / N, n = i % N)
  const long i = t >> 2;
  const int c = (int)(t & 3);
  if (i >= (long)(p.Ktot / 32) * p.N) return;
  const long g = i / p.N, n = i % p.N;
  const hxa_h s = p.S[i];
  const half2_t s2 = {s, s};
  const hxa_h z = ASYM ? p.Z[i] : (hxa_h)0.0f;
  const half2_t z2 = {z, z};
  const uint8_t *src = (const uint8_t *)p.W + n * p.w_rs + g * p.w_gs;
  uint32_t o[4];
  if constexpr (FMT == HXA_W_Q8) {
    const uint2_t v = __builtin_nontemporal_load((const uint2_t *)(src + 8 * c));
    dq8_word(v.x, s2, o[0], o[1]);
    dq8_word(v.y, s2, o[2], o[3]);
  } else {
    dq4_word<ASYM>(__builtin_nontemporal_load((const uint32_t *)(src + 4 * c)), s2, z2, o);
  }
  // lanes write consecutive 16-byte chunks: 1 KB per wave store
  *(uint4_t *)(out + i * 32 + c * 8) = (uint4_t){o[0], o[1], o[2], o[3]};
}
}  // namespace

int hxa_dequant_launch(const HxaWeight &w0, hxa_h *out, hipStream_t st) {
  HxaWeight w = w0;
  const int wkt = (w.fmt & HXA_W_KTILED) ? 1 : 0;
  w.fmt &= ~HXA_W_KTILED;
  if ((w.fmt != HXA_W_Q8 && w.fmt != HXA_W_Q4) || w.s == nullptr || w.N <= 0 || w.K <= 0 || w.K % 32 != 0)
    return HXA_E_ARG;
  if (((uintptr_t)w.w % 16) != 0 || ((uintptr_t)out % 16) != 0) return HXA_E_ARG;
  GemmParams p{};
  p.W = w.w;
  p.S = w.s;
  p.Z = w.z;
  p.N = w.N;
  p.Ktot = w.K;
  const long cb = w.fmt == HXA_W_Q4 ? 16 : 32;
  p.w_rs = wkt ? cb : (long)w.K / 32 * cb;
  p.w_gs = wkt ? cb * w.N : cb;
  const long slots = (long)(w.K / 32) * w.N * 4;
  const dim3 grid((unsigned)((slots + 255) / 256));
  if (w.fmt == HXA_W_Q8) hxa_launch((dequant_kernel<HXA_W_Q8, false>), grid, dim3(256), 0, st, p, out);
  else if (w.z) hxa_launch((dequant_kernel<HXA_W_Q4, true>), grid, dim3(256), 0, st, p, out);
  else hxa_launch((dequant_kernel<HXA_W_Q4, false>), grid, dim3(256), 0, st, p, out);
  return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
}

// ---- split-K linear: fp32 slice sums added in order and rounded once
// out[m][n] = f16(p[0] + p[1] + ... + p[S-1]) at element (m, n) of each slice; one thread per 8 columns of a row
__global__ __launch_bounds__(256) void sum_partials_kernel(const float *__restrict__ p, int S, long zstride, long ldp,
                                                           int M, int N, hxa_h *__restrict__ out, long ldo) {
  const int c8 = N / 8;
  const long c = (long)blockIdx.x * 256 + threadIdx.x;
  if (c >= (long)M * c8) return;
  const int m = (int)(c / c8), n = (int)(c % c8) * 8;
  const float *src = p + (long)m * ldp + n;
  float4_t a0 = *(const float4_t *)src, a1 = *(const float4_t *)(src + 4);
  for (int z = 1; z < S; z++) {
    const float *q = src + (long)z * zstride;
    a0 += *(const float4_t *)q;
    a1 += *(const float4_t *)(q + 4);
  }
  const half8_t o = {(hxa_h)a0[0], (hxa_h)a0[1], (hxa_h)a0[2], (hxa_h)a0[3],
                     (hxa_h)a1[0], (hxa_h)a1[1], (hxa_h)a1[2], (hxa_h)a1[3]};
  *(half8_t *)(out + (long)m * ldo + n) = o;
}

int hxa_sum_partials_launch(const float *p, int S, long zstride, long ldp, int M, int N, hxa_h *out, long ldo,
                            hipStream_t st) {
  if (!p || !out || S < 1 || M <= 0 || N <= 0 || N % 8 || ldp < N || ldo < N || ldp % 4 || ldo % 8 ||
      (S > 1 && zstride < (long)M * ldp) || zstride % 4 || ((uintptr_t)p | (uintptr_t)out) % 16)
    return HXA_E_ARG;
  const long chunks = (long)M * (N / 8);
  hxa_launch(sum_partials_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, p, S, zstride, ldp, M, N,
             out, ldo);
  return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
}

// The K slices hxa_linear runs a linear in: 1 (one launch, fp16 store) or S in {2, 4} (fp32 slices, then their sum)
// when the tile model's time for S slices plus the slices' round trip through memory is below the one-launch time.
int hxa_linear_split(int M, int N, int K, int fmt) {
  fmt &= ~HXA_W_KTILED;
  if (M <= 0 || N <= 0 || K <= 0 || N % 8 || fmt < 0 || fmt > HXA_W_Q4) return 1;
  const double t1 = tile_time(M, N, K, 1, fmt);
  int best = 1;
  double tb = t1;
  for (int S = 2; S <= 4; S *= 2) {
    if (K % (32 * S) != 0) continue;
    // slices written by the GEMM and read back by the sum, fp16 out, and the second launch
    const double bytes = 2.0 * S * M * (double)N * 4.0 + 2.0 * M * (double)N;
    const double t = tile_time(M, N, K, S, fmt) + kSumLaunchUs + bytes / kSumBytesPerUs;
    if (t < tb * kSplitGain) {
      tb = t;
      best = S;
    }
  }
  return best;
}
