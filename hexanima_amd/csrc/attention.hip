// Flash attention for gfx950 (head dim 128, fp16 in/out, fp32 online softmax).
//
// Replaces the reference's slab-wise attention driver (hexagon/mega/blk.c:54-91 attn_run with p_attn_setup,
// k_transpose_tile, k_softmax2p and k_rowscale_sum from kern.c:261-318) and its MOSS joint-attention key mask
// (moss/hexagon/mega/blk.c:56-58). No 1/sqrt(d) is applied: it is folded into the q RMSNorm gain
// (export_all.py:31-32). Keys >= nvalid get probability 0.
//
// Each wave owns 32 queries of one head. It computes S^T = K . Q^T with v_mfma_f32_32x32x16_f16, so every lane
// holds 16 scores of ONE query (its partner lane l^32 holds the other 16 of the 32-key block): the row max and
// row sum need only one cross-lane exchange, and the fp16 probabilities already sit in the B-operand layout of
// O^T += V^T . P^T. V is consumed transposed (V^T [H*128][keys]), which the V projection writes directly.
// K / V^T tiles of 64 keys are staged in LDS (double buffered) and shared by the 4 waves of a workgroup.
#include "hxa_common.h"
#include "kernels.h"

namespace {

constexpr int KT = 64;          // keys per tile
constexpr int KROW = 128 + 8;   // K tile row (halves)
constexpr int VROW = KT + 8;    // V^T tile row (halves)
constexpr int NW = 4;           // waves per workgroup
constexpr int NT = NW * 64;
constexpr int K_STAGE = KT * KROW, V_STAGE = 128 * VROW;
constexpr int LDS_BYTES = 2 * (K_STAGE + V_STAGE) * (int)sizeof(hxa_h);
constexpr int KCH = KT * 16 / NT;   // 16-byte K chunks per thread
constexpr int VCH = 128 * 8 / NT;   // 16-byte V^T chunks per thread

__global__ __launch_bounds__(NT) void attn_kernel(HxaAttn p) {
  extern __shared__ __attribute__((aligned(16))) hxa_h lds[];
  hxa_h *const Ks0 = lds, *const Vs0 = lds + 2 * K_STAGE;
  const int h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, ql = lane & 31;
  const hxa_h *q = p.q + (long)b * p.q_bstride + h * 128;
  const hxa_h *k = p.k + (long)b * p.k_bstride + h * 128;
  const hxa_h *vt = p.vt + (long)b * p.vt_bstride + (long)h * 128 * p.ldvt;
  hxa_h *o = p.o + (long)b * p.o_bstride + h * 128;

  const int qrow = blockIdx.x * (NW * 32) + wave * 32 + ql;
  const bool qok = qrow < p.T;
  half8_t qf[8];
#pragma unroll
  for (int s = 0; s < 8; s++)
    qf[s] = qok ? *(const half8_t *)(q + (long)qrow * p.ldq + s * 16 + 8 * g) : (half8_t){};

  float16_t acc[4];
#pragma unroll
  for (int d = 0; d < 4; d++) acc[d] = (float16_t){};
  float mrun = -INFINITY, lsum = 0.0f;

  uint4_t rk[KCH], rv[VCH];
  auto load = [&](int t) {
    const int key0 = t * KT;
#pragma unroll
    for (int i = 0; i < KCH; i++) {
      const int c = tid + i * NT, r = c >> 4, cc = c & 15, key = key0 + r;
      rk[i] = key < p.NKV ? *(const uint4_t *)(k + (long)key * p.ldk + cc * 8) : (uint4_t){0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VCH; i++) {
      const int c = tid + i * NT, r = c >> 3, cc = c & 7, key = key0 + cc * 8;
      rv[i] = key < p.NKV ? *(const uint4_t *)(vt + (long)r * p.ldvt + key) : (uint4_t){0, 0, 0, 0};
    }
  };
  auto store = [&](int buf) {
    hxa_h *Ks = Ks0 + buf * K_STAGE, *Vs = Vs0 + buf * V_STAGE;
#pragma unroll
    for (int i = 0; i < KCH; i++) {
      const int c = tid + i * NT, r = c >> 4, cc = c & 15;
      *(uint4_t *)(Ks + r * KROW + cc * 8) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < VCH; i++) {
      const int c = tid + i * NT, r = c >> 3, cc = c & 7;
      *(uint4_t *)(Vs + r * VROW + cc * 8) = rv[i];
    }
  };

  const int ntiles = (p.NKV + KT - 1) / KT;
  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < ntiles; t++) {
    const int cur = t & 1;
    if (t + 1 < ntiles) load(t + 1);
    const hxa_h *Ks = Ks0 + cur * K_STAGE, *Vs = Vs0 + cur * V_STAGE;

    // S^T for two 32-key blocks: lane holds keys 8*(r/4) + 4*g + (r%4) of query ql
    float16_t sc[2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++) {
      sc[kb] = (float16_t){};
#pragma unroll
      for (int ds = 0; ds < 8; ds++) {
        const half8_t kf = *(const half8_t *)(Ks + (kb * 32 + ql) * KROW + ds * 16 + 8 * g);
        sc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[ds], sc[kb], 0, 0, 0);
      }
    }
    // mask keys >= nvalid and take the tile max
    float mt = -INFINITY;
    const int key0 = t * KT;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        if (key >= p.nvalid) sc[kb][r] = -INFINITY;
        mt = fmaxf(mt, sc[kb][r]);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mnew = fmaxf(mrun, mt);
    const float alpha = mnew == -INFINITY ? 1.0f : __expf(mrun - mnew);
    const float mref = mnew == -INFINITY ? 0.0f : mnew;
    mrun = mnew;
    lsum *= alpha;
#pragma unroll
    for (int d = 0; d < 4; d++) acc[d] *= alpha;

    half8_t pf[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const hxa_h ph = (hxa_h)__expf(sc[kb][8 * ks + e] - mref);
          pf[kb][ks][e] = ph;
          lsum += (float)ph;
        }
    // O^T += V^T . P^T ; B operand keys of slice ks: {16ks + 4g + 0..3, 16ks + 8 + 4g + 0..3}
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int d = 0; d < 4; d++) {
          const hxa_h *vr = Vs + (d * 32 + ql) * VROW + kb * 32 + ks * 16 + 4 * g;
          const half4_t v0 = *(const half4_t *)vr, v1 = *(const half4_t *)(vr + 8);
          const half8_t va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pf[kb][ks], acc[d], 0, 0, 0);
        }
    if (t + 1 < ntiles) store(cur ^ 1);
    __syncthreads();
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  const float inv = ltot > 0.0f ? 1.0f / ltot : 0.0f;
  if (qok) {
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const int dim = d * 32 + 8 * r4 + 4 * g;
        const half4_t v = {(hxa_h)(acc[d][4 * r4] * inv), (hxa_h)(acc[d][4 * r4 + 1] * inv), (hxa_h)(acc[d][4 * r4 + 2] * inv),
                           (hxa_h)(acc[d][4 * r4 + 3] * inv)};
        *(half4_t *)(o + (long)qrow * p.ldo + dim) = v;
      }
  }
}

}  // namespace

int hxa_attn_launch(const HxaAttn &p, hipStream_t st) {
  if (p.T <= 0 || p.NKV <= 0 || p.H <= 0 || p.batch <= 0) return HXA_E_ARG;
  if (p.nvalid < 1 || p.nvalid > p.NKV) return HXA_E_ARG;
  if ((p.NKV % 8) || (p.ldq % 8) || (p.ldk % 8) || (p.ldvt % 8) || (p.ldo % 4) || p.ldvt < p.NKV) return HXA_E_ARG;
  if (((uintptr_t)p.q | (uintptr_t)p.k | (uintptr_t)p.vt) % 16 || (uintptr_t)p.o % 8) return HXA_E_ARG;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void *)attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES) != hipSuccess)
      return HXA_E_HIP;
    attr = true;
  }
  dim3 grid((p.T + NW * 32 - 1) / (NW * 32), p.H, p.batch);
  hipLaunchKernelGGL(attn_kernel, grid, dim3(NT), LDS_BYTES, st, p);
  return hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP;
}
