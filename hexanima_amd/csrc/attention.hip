// Flash attention for gfx950 (head dim 128, fp16 in/out, fp32 online softmax).
//
// Replaces the reference's slab-wise attention driver (hexagon/mega/blk.c:54-91 attn_run with p_attn_setup,
// k_transpose_tile, k_softmax2p and k_rowscale_sum from kern.c:261-318) and its MOSS joint-attention key mask
// (moss/hexagon/mega/blk.c:56-58). No 1/sqrt(d) is applied: it is folded into the q RMSNorm gain
// (export_all.py:31-32). Keys >= nvalid get probability 0.
//
// Work split: a workgroup of 2 x NWH waves (NWH = 4: 8 waves) owns 32 NWH = 128 queries of one head. Waves [0, NWH)
// take the first half of the key tiles, the others the second half (two waves per SIMD, one of each half); the
// halves are merged through LDS at the end. (96 queries on 6 waves would fill 256 CUs at 1536 queries x 16 heads,
// but waves are dealt to the SIMDs round-robin, two SIMDs then run two waves, and the workgroup takes as long as
// the 128-query one: 29.5 against 29.0 us on MI355X.) Each wave owns 32
// queries and keeps Q in registers. Two schedules of the key loop: lock-step (one barrier per tile for both halves)
// and, for whole tiles in a multiple of 4, ping-pong (each tile split into a VALU phase, the softmax, and an MFMA
// phase, PV with the next QK; the halves one phase apart, so the two waves of a SIMD alternate between the two
// kinds of work: 5-6% faster at 1536 and 6656 keys on MI355X).
//
// Per 64-key tile a wave computes S^T = K . Q^T (v_mfma_f32_32x32x16_f16), so a lane holds 16 scores of ONE query
// and the row max needs a single exchange between the wave's two halves (v_permlane32_swap). K rows are stored in LDS with rows 4-7 and 8-11 of every 16 swapped,
// which makes the scores of lane l (keys 8*(l/32)+0..7 of each 16-key slice) exactly the B operand of
// O^T += V^T . P^T: P goes from the accumulator to the PV MFMA with one fp16 conversion, and each V^T fragment is one
// 16-byte LDS read. K and V^T tiles move global -> LDS directly (global_load_lds_dwordx4), XOR-swizzled so the
// fragment reads are bank-conflict free, double buffered, one barrier per tile. The QK MFMAs of tile j+1 are issued
// before the softmax of tile j so the exponentials overlap them. exp(s - m) is exp2(s*log2e - m*log2e) (one FMA +
// v_exp_f32). O and the row sum are rescaled only when the running max grows by more than 5.5 (P <= e^5.5 in fp16
// otherwise), which keeps the result exact up to rounding while skipping most rescales.
#include <cstdlib>
#include <type_traits>

#include "hxa_common.h"
#include "kernels.h"

namespace {

constexpr int KT = 64;                        // keys per tile
constexpr int TILE_BYTES = KT * 128 * 2;      // K tile [64 keys][128] = V^T tile [128][64 keys] = 16 KB
constexpr int HALF_BYTES = 4 * TILE_BYTES;    // K[2] | V[2]
constexpr int LDS_BYTES = 2 * HALF_BYTES;     // 128 KB
constexpr int SINK_BYTES = 256;               // past the tiles: where the weight touch loads land (never read)
constexpr float L2E = 1.4426950408889634f;
constexpr float RESCALE_TH = 5.5f;

HXA_DEV float16_t mfma(half8_t a, half8_t b, float16_t c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }

// NWH waves per key half (4: 128 queries per workgroup, 8 waves). FULL: every key tile lies wholly below nvalid and
// NKV (nvalid % 64 == 0: 1536 image tokens, 6144 + 512 joint tokens, 256 text tokens), so the loop carries no key
// masking and no clamped per-lane tile addresses. PF: the launch touches weights for the next kernel (p.pf_bytes > 0). Both are compile-time so that the
// main loop holds only the code it runs: the general form kept 44 - 62 scalar registers spilled to VGPR lanes and
// their v_readlane / v_writelane in the loop.
template <int NWH, bool FULL, bool PF, bool PP = false>
__global__ __launch_bounds__(2 * NWH * 64) void attn_kernel(HxaAttn p, int nqb) {
  static_assert(!PP || FULL, "the ping-pong form runs whole tiles only");
  constexpr int QB = NWH * 32;  // queries per workgroup
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // waves w and w + NWH share a SIMD (waves are dealt to the SIMDs round-robin): one wave of each key half
  const int half = wave / NWH, wq = wave % NWH, g = lane >> 5, ql = lane & 31;
  // XCD-aware order: the query blocks of one head run on one XCD (its L2 keeps that head's K / V^T)
  const int ntot = nqb * p.H, bid = blockIdx.x;
  if (bid >= ntot) {  // a workgroup past the tiles (side_wgs): GEMV rows, no LDS and no barrier
    side_gemv(p.side, (bid - ntot) * 2 * NWH + wave, (gridDim.x - ntot) * 2 * NWH, lane);
    return;
  }
  const int tile = (ntot % 8 == 0) ? (bid % 8) * (ntot / 8) + bid / 8 : bid;
  const int h = tile / nqb, qb = tile % nqb, b = blockIdx.y;
  const hxa_h *q = p.q + (long)b * p.q_bstride + h * 128;
  const hxa_h *k = p.k + (long)b * p.k_bstride + h * 128;
  const hxa_h *vt = p.vt + (long)b * p.vt_bstride + (long)h * 128 * p.ldvt;
  hxa_h *o = p.o + (long)b * p.o_bstride + h * 128;
  const HxaClkMark clk0 = clk_mark(p.clk);

  const int qrow = qb * QB + wq * 32 + ql;
  const bool qok = qrow < p.T;
  half8_t qf[8];
#pragma unroll
  for (int s = 0; s < 8; s++) qf[s] = qok ? *(const half8_t *)(q + (long)qrow * p.ldq + s * 16 + 8 * g) : (half8_t){};

  // key tiles covering [0, nvalid); half 0 takes [0, nh), half 1 takes [nh, ntiles)
  const int ntiles = (p.nvalid + KT - 1) / KT, nh = (ntiles + 1) / 2;
  const int t0 = half * nh, nmine = min(nh, ntiles - t0);
  uint8_t *const hb = lds + half * HALF_BYTES;
  auto kbuf = [&](int i) { return hb + (i & 1) * TILE_BYTES; };
  auto vbuf = [&](int i) { return hb + (2 + (i & 1)) * TILE_BYTES; };

  // local tile i -> LDS: 16 KB of K (rows of 256 B, 16 chunks, chunk c at c ^ (row & 15)) and 16 KB of V^T (rows of
  // 128 B, 8 chunks, chunk c at c ^ ((row >> 1) & 7)); the 16 + 16 blocks of 1 KB are dealt round-robin over the NWH
  // waves of the half. Keys past NKV read a valid row (their probability is 0).
  // A tile that lies wholly below NKV moves only a wave-uniform base: each lane's byte offsets within the tile are
  // fixed (koff / voff, computed once), so those loads take the scalar-base form with no per-lane address math.
  constexpr int NLD = (16 + NWH - 1) / NWH;
  uint32_t koff[NLD], voff[NLD];
#pragma unroll
  for (int j = 0; j < NLD; j++) {
    const int blk = min(j * NWH + wq, 15);
    const int row = 4 * blk + (lane >> 4), c = (lane & 15) ^ (row & 15);
    koff[j] = ((uint32_t)krow_key(row) * (uint32_t)p.ldk + c * 8) * 2u;
    const int d = 8 * blk + (lane >> 3), cv = (lane & 7) ^ ((d >> 1) & 7);
    voff[j] = ((uint32_t)d * (uint32_t)p.ldvt + cv * 8) * 2u;
  }
  // tile i of this half into buffer (i & 1); src >= 0: the half's tile src into that buffer instead (the ping-pong
  // form's loads past the last tile, into a buffer that is never read again)
  auto load_kv = [&](int i, bool with_k, bool with_v, int src = -1) {
    const int key0 = (t0 + (src >= 0 ? src : i)) * KT;
    if (FULL || key0 + KT <= p.NKV) {
      if (with_k) {
        const hxa_h *kt = k + (long)key0 * p.ldk;
#pragma unroll
        for (int j = 0; j < NLD; j++) {
          const int blk = j * NWH + wq;
          if (16 % NWH == 0 || blk < 16) g2l16_sbase(kt, koff[j], kbuf(i) + blk * 1024);
        }
      }
      if (with_v) {
        const hxa_h *vtt = vt + key0;
#pragma unroll
        for (int j = 0; j < NLD; j++) {
          const int blk = j * NWH + wq;
          if (16 % NWH == 0 || blk < 16) g2l16_sbase(vtt, voff[j], vbuf(i) + blk * 1024);
        }
      }
      return;
    }
    if constexpr (FULL) return;
    if (with_k) {
      uint8_t *dst = kbuf(i);
#pragma unroll
      for (int j = 0; j < (16 + NWH - 1) / NWH; j++) {
        const int blk = j * NWH + wq;
        if (16 % NWH == 0 || blk < 16) {
          const int row = 4 * blk + (lane >> 4), c = (lane & 15) ^ (row & 15);
          const int key = min(key0 + krow_key(row), p.NKV - 1);
          g2l16_opaque(k + (long)key * p.ldk + c * 8, dst + blk * 1024);
        }
      }
    }
    if (with_v) {
      uint8_t *dst = vbuf(i);
#pragma unroll
      for (int j = 0; j < (16 + NWH - 1) / NWH; j++) {
        const int blk = j * NWH + wq;
        if (16 % NWH == 0 || blk < 16) {
          const int d = 8 * blk + (lane >> 3), c = (lane & 7) ^ ((d >> 1) & 7);
          int key = key0 + c * 8;
          if (key >= p.NKV) key = 0;
          g2l16_opaque(vt + (long)d * p.ldvt + key, dst + blk * 1024);
        }
      }
    }
  };

  // the weight touch: this workgroup's share of the 128-byte lines of [p.pf, p.pf + p.pf_bytes) (a whole number of
  // lines, checked on the host), spread evenly over the steps but the last, so that the touch's HBM reads stay a
  // small fraction of the bandwidth; each line a 4-byte direct-to-LDS load into the sink (no register is written;
  // the next step's vmcnt(0) wait drains it)
  constexpr int NT = 2 * NWH * 64;
  const uint8_t *pf_base = nullptr;
  uint32_t pf_lines = 0;  // of this workgroup
  if constexpr (PF) {
    const uint32_t lines = (uint32_t)(p.pf_bytes >> 7), nwg = ntot * gridDim.y;  // the attention workgroups
    const uint32_t per = (lines + nwg - 1) / nwg, l0 = min((blockIdx.x + blockIdx.y * ntot) * per, lines);
    pf_base = p.pf + ((long)l0 << 7);
    pf_lines = min(lines, l0 + per) - l0;
  }
  const int pf_steps = max(nh - 1, 1);
  const uint32_t pf_per_step = (pf_lines + pf_steps - 1) / pf_steps;
  auto touch = [&](int i) {  // one line per thread and step at most (lines past NT a step are left untouched)
    const uint32_t line = i * pf_per_step + tid;
    if (PF && tid < pf_per_step && line < pf_lines) {
      const uint32_t la = (uint32_t)(uintptr_t)(lds_void_t *)(lds + LDS_BYTES);
      asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(line << 7), "s"(pf_base), "s"(la)
                   : "memory", "m0");
    }
  };

  float16_t acc[4];
#pragma unroll
  for (int d = 0; d < 4; d++) acc[d] = (float16_t){};
  float mrun = -INFINITY, lsum = 0.0f;

  auto qk = [&](int i, float16_t(&S)[2]) {
    const uint8_t *kb = kbuf(i);
    S[0] = (float16_t){};
    S[1] = (float16_t){};
#pragma unroll
    for (int ds = 0; ds < 8; ds++)
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++) {
        const int row = kb2 * 32 + ql, c = 2 * ds + g;
        const half8_t kf = *(const half8_t *)(kb + row * 256 + ((c ^ (row & 15)) << 4));
        S[kb2] = mfma(kf, qf[ds], S[kb2]);
      }
  };

  // (mask, max, rescale) of tile i, then QK of tile i+1 (Sn) overlapped with the exponentials of tile i (pf)
  auto softmax_qk = [&](int i, float16_t(&Sc)[2], float16_t(&Sn)[2], half8_t(&pf)[2][2]) {
    const bool nxt = i + 1 < nmine;
    const int key0 = (t0 + i) * KT;
    if (!FULL && key0 + KT > p.nvalid) {
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (key0 + kb2 * 32 + 16 * (r >> 3) + 8 * g + (r & 7) >= p.nvalid) Sc[kb2][r] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
      for (int r = 0; r < 16; r++) mt = fmaxf(mt, Sc[kb2][r]);
    {
      float lo, hi;
      halves(mt, lo, hi);
      mt = fmaxf(lo, hi);
    }
    const bool need = mt > mrun + RESCALE_TH;  // also when mrun is still -inf
    if (__any(need)) {
      const float alpha = need ? __builtin_amdgcn_exp2f((mrun - mt) * L2E) : 1.0f;
      if (need) mrun = mt;
      lsum *= alpha;
#pragma unroll
      for (int d = 0; d < 4; d++) acc[d] *= alpha;
    }
    const float mb = (mrun == -INFINITY ? 0.0f : mrun) * L2E;
    // One straight-line block: QK of tile i+1 (clamped: the last tile recomputes its own, unused scores) with the
    // K fragments read one step ahead, the exponentials of tile i between its MFMAs, then PV of tile i.
    const uint8_t *kb = kbuf(nxt ? i + 1 : i);
    auto kfrag = [&](int ds, int kb2) {
      const int row = kb2 * 32 + ql, c = 2 * ds + g;
      return *(const half8_t *)(kb + row * 256 + ((c ^ (row & 15)) << 4));
    };
    Sn[0] = (float16_t){};
    Sn[1] = (float16_t){};
    float ls[2] = {0.0f, 0.0f};
    // sched_barrier(0) fences keep each fragment read one stage ahead of the MFMA that consumes it (the scheduler
    // would otherwise sink the reads next to their uses under this register pressure)
    half8_t kf[2][2];
    kf[0][0] = kfrag(0, 0);
    kf[0][1] = kfrag(0, 1);
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
      __builtin_amdgcn_sched_barrier(0);
      if (ds + 1 < 8) {
        kf[(ds + 1) & 1][0] = kfrag(ds + 1, 0);
        kf[(ds + 1) & 1][1] = kfrag(ds + 1, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      Sn[0] = mfma(kf[ds & 1][0], qf[ds], Sn[0]);
      Sn[1] = mfma(kf[ds & 1][1], qf[ds], Sn[1]);
#pragma unroll
      for (int u = 0; u < 4; u += 2) {  // two probabilities at a time: one fp16 pair, summed by one v_dot2
        const int idx = ds * 4 + u, kb2 = idx >> 4, r = idx & 15;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(Sc[kb2][r], L2E, -mb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(Sc[kb2][r + 1], L2E, -mb));
        const half2_t h2 = {(hxa_h)p0, (hxa_h)p1};
        pf[kb2][r >> 3][r & 7] = h2[0];
        pf[kb2][r >> 3][(r & 7) + 1] = h2[1];
        ls[u >> 1] = __builtin_amdgcn_fdot2(h2, (half2_t){(hxa_h)1.0f, (hxa_h)1.0f}, ls[u >> 1], false);
      }
    }
    lsum += ls[0] + ls[1];
  };
  // O^T += V^T P^T for tile i
  auto pv = [&](int i, const half8_t(&pf)[2][2]) {
    const uint8_t *vb = vbuf(i);
    auto vfrag = [&](int j) {  // j = (kb2 * 2 + ks) * 4 + dblk
      const int dblk = j & 3, kk = j >> 2, d = dblk * 32 + ql, c = 2 * kk + g;
      return *(const half8_t *)(vb + d * 128 + ((c ^ ((d >> 1) & 7)) << 4));
    };
    half8_t va[2];
    __builtin_amdgcn_sched_barrier(0);
    va[0] = vfrag(0);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < 16) va[(j + 1) & 1] = vfrag(j + 1);
      __builtin_amdgcn_sched_barrier(0);
      acc[j & 3] = mfma(va[j & 1], pf[j >> 3][(j >> 2) & 1], acc[j & 3]);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // lock-step form: one key tile per step, one barrier per step for both halves
  auto step = [&](int i, float16_t(&Sc)[2], float16_t(&Sn)[2]) {
    wait_vm<0>();
    __builtin_amdgcn_s_barrier();  // tile i V^T and tile i+1 K landed; every wave is done with tiles i-1 / i reads
    asm volatile("" ::: "memory");
    if (i >= nmine) {
      if (i + 2 < nmine) load_kv(i + 2, true, false);
      if (i + 1 < nmine) load_kv(i + 1, false, true);
      return;
    }
    half8_t pf[2][2];
    softmax_qk(i, Sc, Sn, pf);
    // the next tiles' loads after the QK / exponential block, not ahead of it (their issue would delay the softmax)
    if (i + 2 < nmine) load_kv(i + 2, true, false);
    if (i + 1 < nmine) load_kv(i + 1, false, true);
    if (PF && i < pf_steps) touch(i);
    pv(i, pf);
  };

  if (nmine > 0) load_kv(0, true, true);
  if (nmine > 1) load_kv(1, true, false);
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  float16_t Sa[2], Sb[2];
  if (nmine > 0) qk(0, Sa);
  if constexpr (PP) {
    // Ping-pong form (both halves hold nh tiles, whole tiles): each tile is two phases, V(i) = the softmax of tile i
    // (VALU only: max, rescale, exponentials -> P(i)) and M(i) = its PV with the QK of tile i+1 (MFMA only), and
    // half 1 runs one phase behind half 0. The waves of a SIMD belong to different halves (waves w and w + NWH), so
    // in every phase one of them keeps the matrix core busy while the other computes exponentials. One workgroup
    // barrier per phase (2 nh + 1 for either half).
    //  V(i) issues V(i+1) (its buffer held V(i-1), read in M(i-1)) and, from i = 1, K(i+2) (its buffer held K(i),
    //  read in M(i-1)); K(2) is issued in M(0), since half 0's QK of tile 0 has no barrier before V(0). Loads past
    //  the half's last tile reload that tile into the free buffer (M of the last tile skips its QK), so every V
    //  phase issues the same loads and M(i), i >= 1, waits until at most that many are in flight: K(i+1) and V(i),
    //  issued one V phase earlier, have landed.
    half8_t pf[2][2];
    constexpr int NLDMIN = 16 / NWH;  // the fewest K (or V) tile loads a wave issues
    auto bar = [&]() {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    };
    // O^T += V^T P^T of tile i with, when qk, S = K Q^T of tile i+1: 16 + 16 MFMAs, the fragments read two ahead
    auto mphase = [&](int i, auto qk_next) {
      constexpr int nm = decltype(qk_next)::value ? 32 : 16;
      const uint8_t *vb = vbuf(i), *kb = kbuf(i + 1);
      auto frag = [&](int j) {
        if (j < 16) {  // V^T: j = (kb2 * 2 + ks) * 4 + dblk
          const int dblk = j & 3, kk = j >> 2, d = dblk * 32 + ql, c = 2 * kk + g;
          return *(const half8_t *)(vb + d * 128 + ((c ^ ((d >> 1) & 7)) << 4));
        }
        const int q = j - 16, ds = q >> 1, kb2 = q & 1, row = kb2 * 32 + ql, c = 2 * ds + g;
        return *(const half8_t *)(kb + row * 256 + ((c ^ (row & 15)) << 4));
      };
      if constexpr (nm == 32) {
        Sa[0] = (float16_t){};
        Sa[1] = (float16_t){};
      }
      constexpr int AH = 2;  // fragment reads in flight ahead of the MFMA stream (4 or 6: no faster)
      half8_t fr[AH + 1];
#pragma unroll
      for (int j = 0; j < AH; j++) fr[j] = frag(j);
#pragma unroll
      for (int j = 0; j < nm; j++) {
        __builtin_amdgcn_sched_barrier(0);
        if (j + AH < nm) fr[(j + AH) % (AH + 1)] = frag(j + AH);
        __builtin_amdgcn_sched_barrier(0);
        if (j < 16) {
          acc[j & 3] = mfma(fr[j % (AH + 1)], pf[j >> 3][(j >> 2) & 1], acc[j & 3]);
        } else {
          const int q = j - 16;
          Sa[q & 1] = mfma(fr[j % (AH + 1)], qf[q >> 1], Sa[q & 1]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // max, rescale and exponentials of tile i (scores in Sa) -> pf, row sums into lsum
    auto vphase = [&](int i) {
      // the row max as four independent chains (one wave issues this phase alone: latency, not throughput)
      float m4[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
      for (int kb2 = 0; kb2 < 2; kb2++)
#pragma unroll
        for (int r = 0; r < 16; r++) m4[r & 3] = fmaxf(m4[r & 3], Sa[kb2][r]);
      float mt = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
      {
        float lo, hi;
        halves(mt, lo, hi);
        mt = fmaxf(lo, hi);
      }
      const bool need = mt > mrun + RESCALE_TH;  // also when mrun is still -inf
      if (__any(need)) {
        const float alpha = need ? __builtin_amdgcn_exp2f((mrun - mt) * L2E) : 1.0f;
        if (need) mrun = mt;
        lsum *= alpha;
#pragma unroll
        for (int d = 0; d < 4; d++) acc[d] *= alpha;
      }
      const float mb = (mrun == -INFINITY ? 0.0f : mrun) * L2E;
      float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int idx = 0; idx < 32; idx += 2) {
        const int kb2 = idx >> 4, r = idx & 15;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(Sa[kb2][r], L2E, -mb));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(Sa[kb2][r + 1], L2E, -mb));
        const half2_t h2 = {(hxa_h)p0, (hxa_h)p1};
        pf[kb2][r >> 3][r & 7] = h2[0];
        pf[kb2][r >> 3][(r & 7) + 1] = h2[1];
        ls[(idx >> 1) & 3] = __builtin_amdgcn_fdot2(h2, (half2_t){(hxa_h)1.0f, (hxa_h)1.0f}, ls[(idx >> 1) & 3], false);
      }
      lsum += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    auto vstep = [&](int i) {
      if (i > 0) load_kv(i + 2, true, false, min(i + 2, nmine - 1));
      load_kv(i + 1, false, true, min(i + 1, nmine - 1));
      if (PF && i < pf_steps) touch(i);
      vphase(i);
      if (i > 0) wait_vm<2 * NLDMIN>();
      bar();
      if (i == 0) load_kv(2, true, false, min(2, nmine - 1));
    };
    if (half == 1) bar();  // phase 0: half 1 has done its QK of tile 0 (half 0 its QK and V(0))
    for (int i = 0; i < nh - 1; i++) {
      vstep(i);
      mphase(i, std::true_type{});
      bar();
    }
    vstep(nh - 1);
    mphase(nh - 1, std::false_type{});  // the last tile: no next QK
    bar();
    if (half == 0) bar();  // the last phase: half 1's M(nh - 1)
  } else {
    for (int i = 0; i < nh; i += 2) {
      step(i, Sa, Sb);
      if (i + 1 < nh) step(i + 1, Sb, Sa);
    }
  }

  // merge the two key halves: half 1 publishes (m, l, O) per lane, half 0 combines and stores
  clk_store(p.clk, (int)(blockIdx.x + blockIdx.y * gridDim.x), tid, clk0);
  wait_vm<0>();  // no tile load may still be writing the LDS reused below
  __syncthreads();
  float *xch = (float *)lds + wq * 66 * 64;
  if (half == 1) {
    xch[lane] = mrun;
    xch[64 + lane] = lsum;
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int r = 0; r < 16; r++) xch[(2 + d * 16 + r) * 64 + lane] = acc[d][r];
  }
  __syncthreads();
  if (half == 1) return;
  const float m2 = xch[lane], l2 = xch[64 + lane];
  const float m = fmaxf(mrun, m2);
  const float a1 = mrun == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mrun - m) * L2E);
  const float a2 = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m2 - m) * L2E);
  const float lp = lsum * a1 + l2 * a2;
  float llo, lhi;
  halves(lp, llo, lhi);
  const float ltot = llo + lhi;
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  half4_t v[4][4];
#pragma unroll
  for (int d = 0; d < 4; d++)
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int r = 4 * r4 + e;
        v[d][r4][e] = (hxa_h)((acc[d][r] * a1 + xch[(2 + d * 16 + r) * 64 + lane] * a2) * inv);
      }
  // whole output rows, staged past the exchange area (every wave is done with the K / V tiles)
  const int row0 = qb * QB + wq * 32;
  store_rows32(lds + NWH * 66 * 64 * 4 + wq * 8192, v, lane, o + (long)row0 * p.ldo, p.ldo, p.T - row0);
}

// ---- short key ranges (at most 256 valid keys) ----
// A workgroup of 4 waves owns 128 queries of one head, and every wave takes all (at most 4) key tiles, resident in
// LDS together: the two-pass form (attn_two_pass: the exact row max, no running rescale, no key-half merge). The
// output staging (4 x 8 KB) lies past the tiles (4 x 32 KB), so a wave done early never writes where another still
// reads K.
constexpr int SK_LDS = 4 * 2 * TILE_BYTES + 4 * 8192;  // 160 KB

__global__ __launch_bounds__(256) void attn_short_kernel(HxaAttn p, int nqb) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, ql = lane & 31;
  // XCD-aware order: the query blocks of one head run on one XCD
  const int ntot = nqb * p.H, bid = blockIdx.x;
  const int tile = (ntot % 8 == 0) ? (bid % 8) * (ntot / 8) + bid / 8 : bid;
  const int h = tile / nqb, qb = tile % nqb, b = blockIdx.y;
  const hxa_h *q = p.q + (long)b * p.q_bstride + h * 128;
  const hxa_h *k = p.k + (long)b * p.k_bstride + h * 128;
  const hxa_h *vt = p.vt + (long)b * p.vt_bstride + (long)h * 128 * p.ldvt;
  hxa_h *o = p.o + (long)b * p.o_bstride + h * 128;
  const HxaClkMark clk0 = clk_mark(p.clk);

  const int ntiles = (p.nvalid + KT - 1) / KT;  // 1 .. 4
  // every tile: K at 32 KB t, V^T at 32 KB t + 16 KB; this wave's blocks wave, wave + 4, wave + 8, wave + 12
  for (int t = 0; t < ntiles; t++) {
    uint8_t *kd = lds + t * 2 * TILE_BYTES, *vd = kd + TILE_BYTES;
    const int key0 = t * KT;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int blk = j * 4 + wave;
      const int row = 4 * blk + (lane >> 4), c = (lane & 15) ^ (row & 15);
      const int key = min(key0 + krow_key(row), p.NKV - 1);
      g2l16_opaque(k + (long)key * p.ldk + c * 8, kd + blk * 1024);
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int blk = j * 4 + wave;
      const int d = 8 * blk + (lane >> 3), c = (lane & 7) ^ ((d >> 1) & 7);
      int key = key0 + c * 8;
      if (key >= p.NKV) key = 0;
      g2l16_opaque(vt + (long)d * p.ldvt + key, vd + blk * 1024);
    }
  }
  const int row0 = qb * 128 + wave * 32, qrow = row0 + ql;
  half8_t qf[8];
#pragma unroll
  for (int s = 0; s < 8; s++)
    qf[s] = qrow < p.T ? *(const half8_t *)(q + (long)qrow * p.ldq + s * 16 + 8 * g) : (half8_t){};
  wait_vm<0>();
  __syncthreads();

  const uint8_t *const kts[4] = {lds, lds + 2 * TILE_BYTES, lds + 4 * TILE_BYTES, lds + 6 * TILE_BYTES};
  const uint8_t *const vts[4] = {lds + TILE_BYTES, lds + 3 * TILE_BYTES, lds + 5 * TILE_BYTES, lds + 7 * TILE_BYTES};
  float16_t acc[4];
#pragma unroll
  for (int d = 0; d < 4; d++) acc[d] = (float16_t){};
  float lsum;
  attn_two_pass(qf, kts, vts, ntiles, p.nvalid, false, lane, acc, lsum);
  clk_store(p.clk, (int)(blockIdx.x + blockIdx.y * gridDim.x), tid, clk0);
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
      for (int e = 0; e < 4; e++) v[d][r4][e] = (hxa_h)(acc[d][4 * r4 + e] * inv);
  store_rows32(lds + 8 * TILE_BYTES + wave * 8192, v, lane, o + (long)row0 * p.ldo, p.ldo, p.T - row0);
}

}  // namespace

int hxa_attn_launch(const HxaAttn &p, hipStream_t st) {
  if (p.T <= 0 || p.NKV <= 0 || p.H <= 0 || p.batch <= 0) return HXA_E_ARG;
  if (p.nvalid < 1 || p.nvalid > p.NKV) return HXA_E_ARG;
  if ((p.NKV % 8) || (p.ldq % 8) || (p.ldk % 8) || (p.ldvt % 8) || (p.ldo % 4) || p.ldvt < p.NKV) return HXA_E_ARG;
  // per-lane byte offsets within a K / V^T tile are 32-bit: 64 key rows of K and 128 rows of V^T stay below 2^31
  if (p.ldk >= (1 << 24) || p.ldvt >= (1 << 23)) return HXA_E_ARG;
  if (((uintptr_t)p.q | (uintptr_t)p.k | (uintptr_t)p.vt) % 16 || (uintptr_t)p.o % 8) return HXA_E_ARG;
  if (p.q_bstride % 8 || p.k_bstride % 8 || p.vt_bstride % 8 || p.o_bstride % 4) return HXA_E_ARG;
  // the weight touch: whole 128-byte lines, below 2 GB (the per-lane byte offsets are unsigned 32-bit)
  if (p.pf_bytes < 0 || p.pf_bytes % 128 || p.pf_bytes >= (1L << 31) || (p.pf_bytes > 0 && (p.pf == nullptr || (uintptr_t)p.pf % 4)))
    return HXA_E_ARG;
  if (p.side_wgs < 0 || p.side_wgs > 4096) return HXA_E_ARG;
  if (p.side_wgs > 0) {
    const HxaSideGemv &g = p.side;
    if (p.batch != 1 || !hxa_side_k_ok(g.K) || g.N <= 0 || g.per <= 0 || g.split < 0 ||
        g.gap < 0 || !g.y || ((uintptr_t)g.x | (uintptr_t)g.W) % 16 || !g.x || !g.W)
      return HXA_E_ARG;
  }
  // the side GEMV as its own launch, where the attention kernel does not host it
  auto side_alone = [&]() -> int {
    if (p.side_wgs == 0) return HXA_OK;
    const HxaSideGemv &g = p.side;
    return hxa_modgemv_launch(g.x, g.K, g.W, g.N, g.y, g.per, g.ostride, g.split, g.gap, g.act, st);
  };
  static bool attr = false;
  if (!attr) {
    const void *kerns[] = {(const void *)attn_kernel<4, false, false>,      (const void *)attn_kernel<4, false, true>,
                           (const void *)attn_kernel<4, true, false>,       (const void *)attn_kernel<4, true, true>,
                           (const void *)attn_kernel<4, true, false, true>, (const void *)attn_kernel<4, true, true, true>};
    for (const void *kf : kerns)
      if (hipFuncSetAttribute(kf, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES + SINK_BYTES) != hipSuccess)
        return HXA_E_HIP;
    if (hipFuncSetAttribute((const void *)attn_short_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, SK_LDS) !=
        hipSuccess)
      return HXA_E_HIP;
    attr = true;
  }
  HxaAttn pk = p;
  pk.clk = g_hxa_clk_attn;
#ifndef HXA_ATTN_SHORT
#define HXA_ATTN_SHORT 1
#endif
  if (HXA_ATTN_SHORT && p.nvalid <= 4 * KT) {  // every key tile resident: the two-pass kernel
    const int nqb = (p.T + 127) / 128;
    hxa_launch(attn_short_kernel, dim3(nqb * p.H, p.batch), dim3(256), SK_LDS, st, pk, nqb);
    if (hipGetLastError() != hipSuccess) return HXA_E_HIP;
    return side_alone();
  }
  const int nqb = (p.T + 127) / 128;
  const bool full = p.nvalid % KT == 0, pf = p.pf_bytes > 0;
  dim3 grid(nqb * p.H + p.side_wgs, p.batch);
  const int lds = LDS_BYTES + SINK_BYTES;
  // the ping-pong form: whole tiles, the same even number of tiles in both halves (HXA_ATTN_PP=0: lock-step form)
  static const int pp_env = [] {
    const char *e = getenv("HXA_ATTN_PP");
    return e ? atoi(e) : 1;
  }();
  if (pp_env && full && (p.nvalid / KT) % 4 == 0) {
    pf ? hxa_launch(attn_kernel<4, true, true, true>, grid, dim3(512), lds, st, pk, nqb)
       : hxa_launch(attn_kernel<4, true, false, true>, grid, dim3(512), lds, st, pk, nqb);
    return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
  }
  if (full) pf ? hxa_launch(attn_kernel<4, true, true>, grid, dim3(512), lds, st, pk, nqb)
            : hxa_launch(attn_kernel<4, true, false>, grid, dim3(512), lds, st, pk, nqb);
  else pf ? hxa_launch(attn_kernel<4, false, true>, grid, dim3(512), lds, st, pk, nqb)
          : hxa_launch(attn_kernel<4, false, false>, grid, dim3(512), lds, st, pk, nqb);
  return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
}

int hxa_attn_idle_wgs(int T, int H, int batch) {
  if (batch != 1 || T <= 0 || H <= 0) return 0;
  static const int ncu = [] {  // CUs of the device current at the first call (0: unknown, no side GEMV)
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    return n > 0 ? n : 0;
  }();
  if (ncu == 0) return 0;
  const int ntot = (T + 127) / 128 * H, rem = ntot % ncu, idle = rem == 0 ? 0 : ncu - rem;
  return idle >= ncu / 4 ? idle : 0;
}
