// Shared definitions for the MI355X (gfx950) kernels of the DiT block runner.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include <type_traits>

typedef _Float16 hxa_h;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

#define HXA_DEV __device__ __forceinline__

// Stage timing of a block run (host side, per thread). While hxa_t_stage_event is set, every launch binds it as its
// stop event (hipExtLaunchKernel), so the event completes with the last kernel of the stage; hxa_t_start_event, when
// set, is bound as the start event of the next launch only (the start of the first stage). No marker packet sits
// between the kernels. hxa_t_stage_launches counts the launches since the stage event was set.
extern thread_local hipEvent_t hxa_t_stage_event, hxa_t_start_event;
extern thread_local int hxa_t_stage_launches;
template <typename F, typename... Args>
inline void hxa_launch(F kernel, const dim3 &grid, const dim3 &block, uint32_t shmem, hipStream_t st, Args... args) {
  if (hxa_t_stage_event != nullptr || hxa_t_start_event != nullptr) {
    ++hxa_t_stage_launches;
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, hxa_t_start_event, hxa_t_stage_event, 0, args...);
    hxa_t_start_event = nullptr;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, st, args...);
  }
}

// devices with per-device host-side state (the no-allocation scratch address, the stage-timing events)
constexpr int HXA_MAX_DEVICES = 64;

// status codes, weight formats (HXA_W_*) and GEMM epilogues (HXA_EPI_*) are those of the public C-ABI
#include "../../include/hexanima_hip.h"

struct HxaWeight {
  int fmt;            // HXA_W_*
  int N, K;
  const void *w;      // fp16 [N][K] | int8 [N][K] | packed int4 [N][K/2]
  const hxa_h *s;     // [K/32][N] scales (q8, q4)
  const hxa_h *z;     // [K/32][N] q4 offsets (optional)
};

// ---- shader-clock record (hxa_clock_record) ----
// A kernel given a record writes, per workgroup w < n, four 64-bit counters at rec[4 w .. 4 w + 3]: s_memtime and
// s_memrealtime when its work starts, and both again when its main loop ends. s_memtime counts shader-clock cycles,
// s_memrealtime a constant 100 MHz clock, so (c1 - c0) / (r1 - r0) * 100 MHz is the clock the workgroup ran at and
// c1 - c0 its main loop's length in cycles. rec == nullptr: nothing is read or written.
struct HxaClk {
  unsigned long long *rec;
  int n;
};
// the record the GEMM and attention launches copy into their parameters (set by hxa_clock_record; host side)
extern HxaClk g_hxa_clk_gemm, g_hxa_clk_attn;
struct HxaClkMark {
  unsigned long long c, r;
};
HXA_DEV HxaClkMark clk_mark(const HxaClk &k) {
  if (k.rec == nullptr) return {0, 0};
  return {__builtin_amdgcn_s_memtime(), __builtin_amdgcn_s_memrealtime()};
}
// lanes 0-3 of the calling threads write the record (a per-lane address: vector stores)
HXA_DEV void clk_store(const HxaClk &k, int wg, int tid, HxaClkMark s) {
  if (k.rec == nullptr) return;
  const HxaClkMark e = clk_mark(k);
  if (tid < 4 && wg < k.n) k.rec[4L * wg + tid] = tid == 0 ? s.c : tid == 1 ? s.r : tid == 2 ? e.c : e.r;
}

// ---- attention tile layout (shared by the attention kernel and the fused cross-attention tail) ----
// key (within a 64-key tile) held by LDS row i of a K tile: rows 4-7 and 8-11 of each 16-row group are swapped, which
// makes the S^T = K Q^T scores of a lane exactly the B operand of O^T += V^T P^T
HXA_DEV int krow_key(int i) {
  const int b = i & 15, q4 = b >> 2;
  return (i & ~15) + (q4 == 1 ? b + 4 : q4 == 2 ? b - 4 : b);
}
// every lane l gets the values of lanes l % 32 (lo) and l % 32 + 32 (hi): one v_permlane32_swap, no LDS round trip.
// Combining lo and hi gives lanes l and l ^ 32 bit-identical results.
HXA_DEV void halves(float v, float &lo, float &hi) {
  const int x = __builtin_bit_cast(int, v);
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  lo = __builtin_bit_cast(float, (int)r[0]);
  hi = __builtin_bit_cast(float, (int)r[1]);
}

// A wave's 32 x 128 fp16 output block of attention -- lane (g = lane / 32, r = lane % 32) holds row r, columns
// 32 d + 8 i + 4 g .. + 3 as v[d][i] -- written as whole 256-byte rows: staged through 8 KB of LDS at `stage` (row
// r's 8-byte unit u at r * 256 + 8 (u ^ r): conflict-free both ways), then each row by 32 lanes at out + r * ldo.
// Rows >= nrows are not written. Only this wave touches `stage`; its LDS accesses complete in order.
HXA_DEV void store_rows32(uint8_t *stage, const half4_t (&v)[4][4], int lane, hxa_h *out, long ldo, int nrows) {
  const int g = lane >> 5, r = lane & 31;
#pragma unroll
  for (int d = 0; d < 4; d++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int u = d * 8 + 2 * i + g;
      *(half4_t *)(stage + r * 256 + ((u ^ r) << 3)) = v[d][i];
    }
#pragma unroll
  for (int it = 0; it < 16; it++) {
    const int row = 2 * it + g;
    const half4_t x = *(const half4_t *)(stage + row * 256 + ((r ^ row) << 3));
    if (row < nrows) *(half4_t *)(out + (long)row * ldo + 4 * r) = x;
  }
}

// ---- direct-to-LDS loads and VMEM waits (gfx950) ----
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gmem_void_t;

// s_waitcnt vmcnt(N) only (expcnt / lgkmcnt left at their maxima); encoding of gfx9: vmcnt[3:0] | vmcnt_hi[15:14]
template <int N>
HXA_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// 16 bytes per lane from global memory straight into LDS: lane l writes lds_base + 16 l
HXA_DEV void g2l16(const void *g, void *lds_base) {
  __builtin_amdgcn_global_load_lds((gmem_void_t *)g, (lds_void_t *)lds_base, 16, 0, 0);
}

// global_load_lds_dwordx4 issued from inline asm: lane l's 16 bytes land at LDS byte address lds_addr + 16 l (M0).
// The compiler does not see this as an LDS write, so it keeps exact lgkmcnt waits for the fragment reads around it
// (it falls back to lgkmcnt(0) while a visible LDS DMA is in flight). Completion is awaited explicitly (vmcnt(0) and
// a barrier) before any wave reads the tile; LDS reads complete in order, so these loads can only lengthen an
// lgkmcnt wait, never satisfy one early.
HXA_DEV void g2l16_opaque(const void *g, const void *lds_ptr) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void_t *)lds_ptr;
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}

// The same load in the scalar-base form: a wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane byte offset
// (unsigned; keep it below 2^31), so a loop that moves only the base does no per-lane 64-bit address arithmetic.
HXA_DEV void g2l16_sbase(const void *sbase, uint32_t off, const void *lds_ptr) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void_t *)lds_ptr;
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(sbase), "s"(la) : "memory", "m0");
}

// Cross-lane moves inside a 16-lane DPP row (VALU, no LDS round trip).
template <int CTRL>
HXA_DEV float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over the aligned 8-lane group (pairs i^1, i^2 within quads, then quad with quad by the half-row mirror
// i^7): every lane of the group gets the bit-identical total.
HXA_DEV float sum8(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  return v;
}
// sum over the 64 lanes, all in VALU cross-lane moves: the 16-lane row sums (sum8 + row mirror), then row 0 -> 1
// and row 2 -> 3 (row_bcast:15), rows 0+1 -> 3 (row_bcast:31); lane 63 holds the total, read into a scalar
HXA_DEV float wave_sum(float v) {
  v = sum8(v);
  v += dpp_f<0x140>(v);  // row_mirror: every lane of a row holds the row sum
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Modulation GEMV rows (megarun.cpp:156-171 role: adaLN rows from one embedding vector), shared by modgemv_kernel
// and the workgroups an attention launch lends to it. K = KC chunks of 64*EPL; lane l keeps act(x[k]) for
// k = c*64*EPL + EPL*l + e in xr (act 1: SiLU). Row n = sum_k xr * W[n][k] is one fmaf chain per lane in (c, e)
// order, then wave_sum, so a row's bits do not depend on which wave computes it or how many rows it has in flight.
// Row n goes to y[(n / per) * ostride + r + (r >= split ? gap : 0)], r = n % per. Weights are read once per call:
// non-temporal loads (modulation of 28 2B blocks, 1.41 GB: 249 -> 212 us).
template <int KC, int EPL>
HXA_DEV void modgemv_x(const float *__restrict__ x, int act, int lane, float (&xr)[KC][EPL]) {
  constexpr int CH = 64 * EPL;
#pragma unroll
  for (int c = 0; c < KC; c++)
#pragma unroll
    for (int e4 = 0; e4 < EPL; e4 += 4) {
      const float4_t a = *(const float4_t *)(x + c * CH + lane * EPL + e4);
#pragma unroll
      for (int e = 0; e < 4; e++) xr[c][e4 + e] = act == 1 ? a[e] / (1.0f + __expf(-a[e])) : a[e];
    }
}
// rows [n0, n1), R of them in flight
template <int KC, int EPL, int R>
HXA_DEV void modgemv_rows(const float (&xr)[KC][EPL], const hxa_h *__restrict__ W, long n0, long n1,
                          float *__restrict__ y, int per, long ostride, int split, int gap, int lane) {
  constexpr int CH = 64 * EPL, K = KC * CH;
  using wvec = typename std::conditional<EPL == 8, half8_t, half4_t>::type;
  for (long n = n0; n < n1; n += R) {
    wvec w[R][KC];
#pragma unroll
    for (int j = 0; j < R; j++)
      if (n + j < n1) {
#pragma unroll
        for (int c = 0; c < KC; c++)
          w[j][c] = __builtin_nontemporal_load((const wvec *)(W + (n + j) * K + c * CH + lane * EPL));
      }
    float a[R];
#pragma unroll
    for (int j = 0; j < R; j++) a[j] = 0.0f;
#pragma unroll
    for (int c = 0; c < KC; c++)
#pragma unroll
      for (int e = 0; e < EPL; e++)
#pragma unroll
        for (int j = 0; j < R; j++)
          if (n + j < n1) a[j] = fmaf(xr[c][e], (float)w[j][c][e], a[j]);
#pragma unroll
    for (int j = 0; j < R; j++) {
      if (n + j < n1) {
        const float v = wave_sum(a[j]);
        const long m = n + j;
        const int r = (int)(m % per);
        if (lane == 0) y[(m / per) * ostride + r + (r >= split ? gap : 0)] = v;
      }
    }
  }
}

// A modulation GEMV (the rows hxa_modgemv_launch computes, with the same bits) that a launch runs in extra
// workgroups appended to its grid, on the CUs its own tiles leave idle: y rows [0, N) of act(x) . W^T, K (the
// embedding width) 2048, 2560 or 3072
struct HxaSideGemv {
  const float *x = nullptr;
  const hxa_h *W = nullptr;
  long N = 0;
  float *y = nullptr;
  int per = 1;
  long ostride = 0;
  int split = 0, gap = 0, act = 0, K = 0;
};
// the widths the hosting kernels are built for
inline bool hxa_side_k_ok(int K) { return K == 2048 || K == 2560 || K == 3072; }
// Wave gw of the nw waves in the appended workgroups: an equal run of the side GEMV's rows, R in flight (R = 2 in the
// GEMM kernels, where more would raise the kernel's register count for its tiles)
template <int R = 4>
HXA_DEV void side_gemv(const HxaSideGemv &s, int gw, int nw, int lane) {
  const long rpw = (s.N + nw - 1) / nw, n0 = (long)gw * rpw, n1 = n0 + rpw < s.N ? n0 + rpw : s.N;
  if (n0 >= s.N) return;
  auto run = [&](auto kc) {
    constexpr int KC = decltype(kc)::value;
    float xr[KC][8];
    modgemv_x<KC, 8>(s.x, s.act, lane, xr);
    modgemv_rows<KC, 8, R>(xr, s.W, n0, n1, s.y, s.per, s.ostride, s.split, s.gap, lane);
  };
  if (s.K == 2048) run(std::integral_constant<int, 4>{});
  else if (s.K == 2560) run(std::integral_constant<int, 5>{});
  else if (s.K == 3072) run(std::integral_constant<int, 6>{});
}

// Per-head RMSNorm * gain + split-half RoPE (kern.c:163-197) on the 8 lanes holding one head of 128: lane jj owns
// dims [8jj, 8jj+8) (lo) and their RoPE partners [64+8jj, 64+8jj+8) (hi), so the rotation needs no exchange:
//   y[d] = x[d] c_d - x[d+64] s_d,  y[d+64] = x[d] s_d + x[d+64] c_d  (d < 64).
// Shared by the GEMM's head-norm epilogue and the standalone kernel, which therefore give the same bits.
HXA_DEV void head_norm2(half8_t &lo, half8_t &hi, const float (&glo)[8], const float (&ghi)[8], bool rope,
                        const float (&cs)[8], const float (&sn)[8]) {
  float a[8], b[8], ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    a[e] = (float)lo[e];
    ss = fmaf(a[e], a[e], ss);
  }
#pragma unroll
  for (int e = 0; e < 8; e++) {
    b[e] = (float)hi[e];
    ss = fmaf(b[e], b[e], ss);
  }
  ss = sum8(ss);
  const float r = rsqrtf(fmaf(ss, 1.0f / 128.0f, 1e-6f));
#pragma unroll
  for (int e = 0; e < 8; e++) {
    a[e] = a[e] * r * glo[e];
    b[e] = b[e] * r * ghi[e];
  }
  if (rope) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = a[e], y = b[e];
      a[e] = fmaf(x, cs[e], -(y * sn[e]));
      b[e] = fmaf(x, sn[e], y * cs[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) {
    lo[e] = (hxa_h)a[e];
    hi[e] = (hxa_h)b[e];
  }
}

// Attention of one wave's 32 queries over at most 4 key tiles of 64 resident in LDS, two-pass: the scores of every
// tile first (64 MFMAs, K fragments read 8 ahead), the exact row max, then P V of tile t with the exponentials of tile
// t + 1 between its MFMAs (V^T fragments read 4 ahead). qf: the Q^T operand (lane (g, ql) holds query ql, dims
// 16 sd + 8 g .. + 7 in qf[sd]); K tile t at kt[t], V^T tile t at vt[t] in the attention kernel's layouts. Keys at or
// past nvalid get probability 0; tiles >= ntiles (ntiles = ceil(nvalid / 64)) are not touched except that their
// K is read and its scores discarded. v2_wait: before tile 2's P V, wait for this wave's outstanding loads and pass a
// workgroup barrier (V^T of tiles 2 and 3 still landing). Out: o = O^T unnormalised, lsum = this lane's half of the
// row sum (add the other half with halves()).
HXA_DEV void attn_two_pass(const half8_t (&qf)[8], const uint8_t *const (&kt)[4], const uint8_t *const (&vt)[4],
                           int ntiles, int nvalid, bool v2_wait, int lane, float16_t (&o)[4], float &lsum) {
  constexpr float L2E = 1.4426950408889634f;
  const int g = lane >> 5, ql = lane & 31;
  float16_t S[4][2];
#pragma unroll
  for (int t = 0; t < 4; t++) S[t][0] = S[t][1] = (float16_t){};
  auto kfrag = [&](int i) {  // i = (t * 8 + ds) * 2 + kb2
    const int t = i >> 4, ds = (i >> 1) & 7, kb2 = i & 1, row = kb2 * 32 + ql, c = 2 * ds + g;
    return *(const half8_t *)(kt[t] + row * 256 + ((c ^ (row & 15)) << 4));
  };
  constexpr int KA = 8;
  half8_t kr[KA];
#pragma unroll
  for (int i = 0; i < KA; i++) kr[i] = kfrag(i);
#pragma unroll
  for (int i = 0; i < 64; i++) {
    __builtin_amdgcn_sched_barrier(0);
    const half8_t cur = kr[i % KA];
    if (i + KA < 64) kr[i % KA] = kfrag(i + KA);
    __builtin_amdgcn_sched_barrier(0);
    S[i >> 4][i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur, qf[(i >> 1) & 7], S[i >> 4][i & 1], 0, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < 4; t++) {
    if (t >= ntiles) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int r = 0; r < 16; r++) S[t][kb2][r] = -INFINITY;
    } else if (t == ntiles - 1 && t * 64 + 64 > nvalid) {  // keys past nvalid in the last tile
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (t * 64 + kb2 * 32 + 16 * (r >> 3) + 8 * g + (r & 7) >= nvalid) S[t][kb2][r] = -INFINITY;
    }
  }
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
      for (int r = 0; r < 16; r++) m = fmaxf(m, S[t][kb2][r]);
  {
    float lo, hi;
    halves(m, lo, hi);
    m = fmaxf(lo, hi);  // finite: nvalid >= 1
  }
  const float mb = m * L2E;
  float ls[2] = {0.0f, 0.0f};
  half8_t pf[2][2][2];
  // probabilities of scores idx, idx + 1 (idx even) of tile t (0 for masked keys and absent tiles): one fp16 pair,
  // summed by one v_dot2 (the row sum of the fp16 P the P V MFMAs use)
  auto expo2 = [&](int t, int idx) {
    const int kb2 = idx >> 4, r = idx & 15;
    const float p0 = __builtin_amdgcn_exp2f(fmaf(S[t][kb2][r], L2E, -mb));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(S[t][kb2][r + 1], L2E, -mb));
    const half2_t h2 = {(hxa_h)p0, (hxa_h)p1};
    pf[t & 1][kb2][r >> 3][r & 7] = h2[0];
    pf[t & 1][kb2][r >> 3][(r & 7) + 1] = h2[1];
    ls[(idx >> 1) & 1] = __builtin_amdgcn_fdot2(h2, (half2_t){(hxa_h)1.0f, (hxa_h)1.0f}, ls[(idx >> 1) & 1], false);
  };
#pragma unroll
  for (int idx = 0; idx < 32; idx += 2) expo2(0, idx);
#pragma unroll
  for (int t = 0; t < 4; t++) {
    if (t == 2 && v2_wait && ntiles > 2) {
      wait_vm<0>();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    if (t < ntiles) {
      const uint8_t *vb = vt[t];
      auto vfrag = [&](int j) {  // j = (kb2 * 2 + ks) * 4 + dblk
        const int dblk = j & 3, kk = j >> 2, d = dblk * 32 + ql, c = 2 * kk + g;
        return *(const half8_t *)(vb + d * 128 + ((c ^ ((d >> 1) & 7)) << 4));
      };
      constexpr int VA = 4;
      half8_t vr[VA];
#pragma unroll
      for (int j = 0; j < VA; j++) vr[j] = vfrag(j);
#pragma unroll
      for (int j = 0; j < 16; j++) {
        __builtin_amdgcn_sched_barrier(0);
        const half8_t cur = vr[j % VA];
        if (j + VA < 16) vr[j % VA] = vfrag(j + VA);
        __builtin_amdgcn_sched_barrier(0);
        o[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur, pf[t & 1][j >> 3][(j >> 2) & 1], o[j & 3], 0, 0, 0);
        if (t + 1 < 4) expo2(t + 1, 2 * j);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  lsum = ls[0] + ls[1];
}

#define HXA_CHECK(x)                                  \
  do {                                                \
    hipError_t e_ = (x);                              \
    if (e_ != hipSuccess) return HXA_E_HIP;           \
  } while (0)
