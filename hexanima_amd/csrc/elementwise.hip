// Bandwidth-bound kernels of the DiT block runner for gfx950: modulated LayerNorm / RMSNorm, per-head
// RMSNorm + RoPE, the split-K gated residual, the reference crouton-layout conversions used at the C-ABI
// boundary, synthetic-data fills and the caller-side glue (patch embed, timestep sinusoid, final layer + Euler).
//
// Row kernels use one 64-lane wave per row with 16-byte vector loads (fully coalesced); reductions stay inside
// the wave (no LDS, no barriers).
#include <algorithm>
#include <type_traits>

#include "hxa_common.h"
#include "kernels.h"

namespace {

// ---------------------------------------------------------------------------------------------------------------
// modulated norm (kern.c:31-65 LN-mod; moss kern.c:345-375 RMS-mod)
// ---------------------------------------------------------------------------------------------------------------
// With NP > 0 pending fp16 partials t_j = t + j tz the gated residual of the previous site is applied first:
// x += gate * t (NP 1, kern.c:320-328, the same fma as the GEMM residual epilogue), x += gate * (t0 + t1) (NP 2,
// kern.c:330-339) or x += gate * ((t0 + t1) + (t2 + t3)) (NP 4, the K-quarter partials), the same sums as
// resaddn_kernel; x is written back, and the norm is taken of the updated row.
// A 256-thread workgroup per group of rows (row = blockIdx.x + j gridDim.x; a float4 of every 1024 columns per
// thread). The column vectors (gate, 1 + scale [* w], shift) are read once per workgroup, and the next row's x and
// pending terms are loaded while the current row is reduced and stored, so loads and stores of the grid overlap.
// The row sums are wave DPP sums combined through LDS in a fixed order (the same bits for any grid).
// NP pending fp16 terms (0, 1, 2 or 4; term j at t + j tz) are summed in a fixed order, ((t0 + t1) + (t2 + t3)).
template <int NV, int NP>
__global__ __launch_bounds__(256) void normrow_kernel(float *__restrict__ x, long ldx, int D, int T,
                                                      const hxa_h *__restrict__ t, long tz, long ldt,
                                                      const float *__restrict__ gate, const float *__restrict__ shift,
                                                      const float *__restrict__ scale, const float *__restrict__ w,
                                                      float eps, hxa_h *__restrict__ h, long ldh) {
  constexpr int NT = NP > 0 ? NP : 1;
  __shared__ float red[2][8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int row = blockIdx.x;
  float4_t xv[NV];
  half4_t ta[NT][NV];
  auto load = [&](int r) {
    const float4_t *xr = (const float4_t *)(x + (long)r * ldx);
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int c = (tid + 256 * k) * 4;
      xv[k] = c < D ? xr[tid + 256 * k] : (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
      if (NP > 0 && c < D) {
#pragma unroll
        for (int j = 0; j < NP; j++) ta[j][k] = *(const half4_t *)(t + j * tz + (long)r * ldt + c);
      }
    }
  };
  load(row);
  // the column vectors, formed while the first row is in flight: multiplier (1 + scale) [* w] (k_rms_prep), shift
  float4_t g[NV], mul[NV], sh[NV];
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const int c = (tid + 256 * k) * 4;
    if (c < D) {
      if (NP > 0) g[k] = *(const float4_t *)(gate + c);
      mul[k] = *(const float4_t *)(scale + c) + 1.0f;
      if (w != nullptr) mul[k] *= *(const float4_t *)(w + c);
      sh[k] = *(const float4_t *)(shift + c);
    }
  }
  const float inv = 1.0f / (float)D;
  for (int par = 0; row < T; row += gridDim.x, par ^= 1) {
    float4_t v[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
      v[k] = xv[k];
      if (NP > 0 && (tid + 256 * k) * 4 < D) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          float sum = (float)ta[0][k][e];
          if (NP == 2) sum += (float)ta[NT > 1 ? 1 : 0][k][e];
          if (NP == 4)
            sum = (sum + (float)ta[NT > 1 ? 1 : 0][k][e]) + ((float)ta[NT > 2 ? 2 : 0][k][e] + (float)ta[NT > 3 ? 3 : 0][k][e]);
          v[k][e] = fmaf(g[k][e], sum, v[k][e]);
        }
      }
    }
    if (row + (int)gridDim.x < T) load(row + gridDim.x);  // in flight during this row's reduction and stores
    float4_t *xr = (float4_t *)(x + (long)row * ldx);
    if (NP > 0) {
#pragma unroll
      for (int k = 0; k < NV; k++)
        if ((tid + 256 * k) * 4 < D) xr[tid + 256 * k] = v[k];
    }
    float s = 0.0f, q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
      s += (v[k][0] + v[k][1]) + (v[k][2] + v[k][3]);
      q += (v[k][0] * v[k][0] + v[k][1] * v[k][1]) + (v[k][2] * v[k][2] + v[k][3] * v[k][3]);
    }
    s = wave_sum(s);
    q = wave_sum(q);
    // red[par]: the previous row's values (red[par ^ 1]) may still be read by a slower wave; the row before that is
    // past everyone's barrier of the previous row
    if (lane == 0) {
      red[par][2 * wave] = s;
      red[par][2 * wave + 1] = q;
    }
    __syncthreads();
    s = (red[par][0] + red[par][2]) + (red[par][4] + red[par][6]);
    q = (red[par][1] + red[par][3]) + (red[par][5] + red[par][7]);
    float mu, r;
    if (w == nullptr) {
      mu = s * inv;
      r = rsqrtf(q * inv - mu * mu + eps);  // var = E[x^2] - mu^2 (kern.c:52-53)
    } else {
      mu = 0.0f;
      r = rsqrtf(q * inv + eps);
    }
#pragma unroll
    for (int k = 0; k < NV; k++) {
      const int c = (tid + 256 * k) * 4;
      if (c < D) {
        half4_t o;
#pragma unroll
        for (int e = 0; e < 4; e++) o[e] = (hxa_h)((v[k][e] - mu) * r * mul[k][e] + sh[k][e]);
        *(half4_t *)(h + (long)row * ldh + c) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// per-head RMSNorm * gain + split-half RoPE (kern.c:163-197). 8 lanes per (token, head); lane jj owns dims
// [8jj, 8jj+8) and [64+8jj, 64+8jj+8) (two 16-byte loads / stores), see head_norm2.
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rmsrope_kernel(hxa_h *q0, hxa_h *q1, const float *g0, const float *g1, long ldq,
                                                      int T, int H, const float *__restrict__ cosT,
                                                      const float *__restrict__ sinT, int ttab) {
  const long gid = (long)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int jj = threadIdx.x & 7;
  if (gid >= (long)T * H) return;  // whole 8-lane groups leave together; the cross-lane sum stays inside a group
  const int t = (int)(gid / H), hd = (int)(gid % H);
  hxa_h *q = blockIdx.y ? q1 : q0;
  const float *g = blockIdx.y ? g1 : g0;
  hxa_h *p = q + (long)t * ldq + hd * 128 + 8 * jj;
  half8_t lo = *(const half8_t *)p, hi = *(const half8_t *)(p + 64);
  float glo[8], ghi[8], cs[8] = {}, sn[8] = {};
  {
    const float4_t a0 = *(const float4_t *)(g + 8 * jj), a1 = *(const float4_t *)(g + 8 * jj + 4);
    const float4_t b0 = *(const float4_t *)(g + 64 + 8 * jj), b1 = *(const float4_t *)(g + 64 + 8 * jj + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      glo[e] = a0[e];
      glo[e + 4] = a1[e];
      ghi[e] = b0[e];
      ghi[e + 4] = b1[e];
    }
  }
  if (cosT != nullptr) {
    const long o = (long)(t % ttab) * 64 + 8 * jj;
    const float4_t c0 = *(const float4_t *)(cosT + o), c1 = *(const float4_t *)(cosT + o + 4);
    const float4_t s0 = *(const float4_t *)(sinT + o), s1 = *(const float4_t *)(sinT + o + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      cs[e] = c0[e];
      cs[e + 4] = c1[e];
      sn[e] = s0[e];
      sn[e + 4] = s1[e];
    }
  }
  head_norm2(lo, hi, glo, ghi, cosT != nullptr, cs, sn);
  *(half8_t *)p = lo;
  *(half8_t *)(p + 64) = hi;
}

// ---------------------------------------------------------------------------------------------------------------
// x += gate * (t1 + t2)   (kern.c:330-339, split-K down projection); NP = 4: x += gate * ((t1 + t2) + (t3 + t4)),
// term j at t + j tz
// ---------------------------------------------------------------------------------------------------------------
template <int NP>
__global__ __launch_bounds__(256) void resaddn_kernel(float *x, long ldx, const hxa_h *__restrict__ t, long tz, long ldt,
                                                      int T, int D, const float *__restrict__ gate) {
  const long i4 = (long)blockIdx.x * 256 + threadIdx.x;
  const int per_row = D / 4;
  if (i4 >= (long)T * per_row) return;
  const int row = (int)(i4 / per_row), c = (int)(i4 % per_row) * 4;
  float4_t *xp = (float4_t *)(x + (long)row * ldx + c);
  half4_t a[NP];
#pragma unroll
  for (int j = 0; j < NP; j++) a[j] = *(const half4_t *)(t + j * tz + (long)row * ldt + c);
  const float4_t g = *(const float4_t *)(gate + c);
  float4_t xv = *xp;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const float sum = NP == 2 ? (float)a[0][e] + (float)a[NP > 1 ? 1 : 0][e]
                              : ((float)a[0][e] + (float)a[NP > 1 ? 1 : 0][e]) +
                                    ((float)a[NP > 2 ? 2 : 0][e] + (float)a[NP > 3 ? 3 : 0][e]);
    xv[e] = fmaf(g[e], sum, xv[e]);
  }
  *xp = xv;
}

// ---------------------------------------------------------------------------------------------------------------
// crouton layout conversions (kern.h:5-8): x32 float(r,c) = r*32+c; h16 halfword(r,c) = (r/2)*64 + c*2 + (r&1)
// ---------------------------------------------------------------------------------------------------------------
__global__ void x32_to_rows_kernel(const float *tiles, float *x, int R, int C) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)R * C) return;
  const int r = (int)(i / C), c = (int)(i % C);
  x[i] = tiles[((long)(r >> 5) * (C >> 5) + (c >> 5)) * 1024 + (r & 31) * 32 + (c & 31)];
}
__global__ void rows_to_x32_kernel(const float *x, float *tiles, int R, int C) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)R * C) return;
  const int r = (int)(i / C), c = (int)(i % C);
  tiles[((long)(r >> 5) * (C >> 5) + (c >> 5)) * 1024 + (r & 31) * 32 + (c & 31)] = x[i];
}
__global__ void h16_to_rows_kernel(const hxa_h *tiles, hxa_h *a, long lda, int R, int C) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)R * C) return;
  const int r = (int)(i / C), c = (int)(i % C);
  a[(long)r * lda + c] = tiles[((long)(r >> 5) * (C >> 5) + (c >> 5)) * 1024 + ((r & 31) >> 1) * 64 + (c & 31) * 2 + (r & 1)];
}
__global__ void rows_to_h16_kernel(const hxa_h *a, long lda, hxa_h *tiles, int R, int C, int transposed) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)R * C) return;
  const int r = (int)(i / C), c = (int)(i % C);
  const hxa_h v = transposed ? a[(long)c * lda + r] : a[(long)r * lda + c];
  tiles[((long)(r >> 5) * (C >> 5) + (c >> 5)) * 1024 + ((r & 31) >> 1) * 64 + (c & 31) * 2 + (r & 1)] = v;
}
__global__ void cs_to_rows_kernel(const float *tiles, float *rows, int T) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * 64) return;
  const int tk = (int)(i / 64), d = (int)(i % 64);
  rows[i] = tiles[((long)(tk >> 5) * 2 + (d >> 5)) * 1024 + (tk & 31) * 32 + (d & 31)];
}

// ---------------------------------------------------------------------------------------------------------------
// synthetic data: counter-based hash (splitmix64 finaliser) -> uniform / Box-Muller normal
// ---------------------------------------------------------------------------------------------------------------
HXA_DEV uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__global__ void fill_normal_kernel(void *dst, int dtype, size_t n, uint64_t seed, float mean, float std) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t h = mix64(seed * 0xD1B54A32D192ED03ull + i);
  const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
  const float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
  const float z = sqrtf(-2.0f * __logf(u1)) * __cosf(6.283185307179586f * u2);
  const float v = mean + std * z;
  if (dtype == 0) ((float *)dst)[i] = v;
  else ((hxa_h *)dst)[i] = (hxa_h)v;
}
__global__ void fill_uniform_int_kernel(void *dst, int bits, size_t n, uint64_t seed, int lo, int hi) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t h = mix64(seed * 0xD1B54A32D192ED03ull + i);
  const uint32_t span = (uint32_t)(hi - lo + 1);
  if (bits == 8) {
    ((int8_t *)dst)[i] = (int8_t)(lo + (int)((h >> 32) % span));
  } else {  // one byte = two int4 nibbles (value + 8)
    const int a = lo + (int)((h >> 32) % span) + 8, b = lo + (int)((h & 0xFFFFFFFFull) % span) + 8;
    ((uint8_t *)dst)[i] = (uint8_t)(a | (b << 4));
  }
}
__global__ void fill_const_kernel(void *dst, int dtype, size_t n, float v) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  if (dtype == 0) ((float *)dst)[i] = v;
  else ((hxa_h *)dst)[i] = (hxa_h)v;
}

// ---------------------------------------------------------------------------------------------------------------
// caller-side glue (phone/animad.cpp)
// ---------------------------------------------------------------------------------------------------------------
// patchify (animad.cpp:447-450): lat [B][C][H][W] -> tok [B*T][C*4], feature (c, ph, pw)
__global__ void patchify_kernel(const float *lat, int B, int Cc, int H, int W, float *tok) {
  const int gh = H / 2, gw = W / 2, F = Cc * 4;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * gh * gw * F) return;
  const int f = (int)(i % F);
  const long tkb = i / F;
  const int tk = (int)(tkb % (gh * gw)), b = (int)(tkb / (gh * gw));
  const int gy = tk / gw, gx = tk % gw, c = f / 4, a = (f / 2) & 1, bb = f & 1;
  tok[i] = lat[(((long)b * Cc + c) * H + gy * 2 + a) * W + gx * 2 + bb];
}

// angle of frequency j of the timestep sinusoid (animad.cpp:425): t * 10000^(-j / half)
HXA_DEV float sinusoid_angle(float t, int j, int half) { return t * expf(-logf(10000.0f) * (float)j / (float)half); }

// y[m][n] = act(sum_k x[m][k] * W[n][k] (+ bias[n])); act 0 none, 1 SiLU on the input (x -> x sigmoid(x)), 2 the
// input row is the timestep sinusoid of t = x[0] at width K (the values sinusoid_kernel stores; one row).
// One wave per output feature n, lanes stride K (coalesced weight reads), up to 8 input rows.
// two adjacent weights as fp32: fp16 storage (most glue) or fp32 storage (the MOSS time MLP, video embedding and
// head, kept fp32 as the reference keeps them, moss/export_glue.py:7-12)
__device__ inline float2_t wpair(const hxa_h *p) {
  const half2_t h = *(const half2_t *)p;
  return (float2_t){(float)h[0], (float)h[1]};
}
__device__ inline float2_t wpair(const float *p) { return *(const float2_t *)p; }
template <typename WT>
__global__ __launch_bounds__(256) void gemv_kernel(const float *__restrict__ x, long ldx, int M, int K,
                                                   const WT *__restrict__ W, int N, float *__restrict__ y, long ldy,
                                                   int act, const float *__restrict__ bias, int split, int gap) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (n >= N) return;
  float accm[8];
#pragma unroll
  for (int m = 0; m < 8; m++) accm[m] = 0.0f;
  const WT *wr = W + (long)n * K;
  for (int k = lane * 2; k < K; k += 128) {
    const float2_t wv = wpair(wr + k);
#pragma unroll
    for (int m = 0; m < 8; m++) {
      if (m < M) {
        float x0, x1;
        if (act == 2) {  // the sinusoid of t = x[0] at width K (sinusoid_kernel's values), one row
          const int half = K / 2, j0 = k < half ? k : k - half;  // k even, half even: k and k + 1 on one side
          const float a0 = sinusoid_angle(x[0], j0, half), a1 = sinusoid_angle(x[0], j0 + 1, half);
          x0 = k < half ? cosf(a0) : sinf(a0);
          x1 = k < half ? cosf(a1) : sinf(a1);
        } else {
          x0 = x[(long)m * ldx + k];
          x1 = x[(long)m * ldx + k + 1];
        }
        if (act == 1) {
          x0 = x0 / (1.0f + __expf(-x0));
          x1 = x1 / (1.0f + __expf(-x1));
        }
        accm[m] = fmaf(x0, wv[0], fmaf(x1, wv[1], accm[m]));
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 8; m++) {
    if (m < M) {
      const float v = wave_sum(accm[m]);
      if (lane == 0) y[(long)m * ldy + n + (n >= split ? gap : 0)] = v + (bias ? bias[n] : 0.0f);
    }
  }
}

// Modulation GEMV over stacked weight matrices (megarun.cpp:156-171 role: every block's adaLN rows from one
// embedding vector): rows of W [N][K] as modgemv_rows (hxa_common.h) computes and places them; each wave streams
// RPW rows, two in flight.
template <int KC, int EPL>
__global__ __launch_bounds__(256) void modgemv_kernel(const float *__restrict__ x, const hxa_h *__restrict__ W, long N,
                                                      float *__restrict__ y, int per, long ostride, int split, int gap,
                                                      int act, int rpw) {
  const int lane = threadIdx.x & 63;
  const long row0 = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw;
  if (row0 >= N) return;
  float xr[KC][EPL];
  modgemv_x<KC, EPL>(x, act, lane, xr);
  modgemv_rows<KC, EPL, 2>(xr, W, row0, row0 + rpw < N ? row0 + rpw : N, y, per, ostride, split, gap, lane);
}

// patch embed (animad.cpp:440-446): x[b][tk][n] = sum_f tok[b tk][f] * Wemb[n][f], f = 4 c + 2 a + bb over the
// Cc channels and the 2 x 2 patch (a, bb) of token tk = (gy, gx), read straight from the latent lat [B][Cc][H][W]
// (the patchified token rows are never stored). A 64-token x 64-column tile per workgroup over the B * T tokens, 4 x 4
// outputs per thread. K = 4 Cc is staged in chunks of 64 in LDS as fp32 rows of float4 (feature float4 c = the
// 2 x 2 patch of channel c: two float2 loads of the latent; W as one half4), read back as float4 along k; every
// output accumulates its products in ascending k (one fma chain). Image b's rows go to x + b * xrows * D.
// Workgroups with blockIdx.x >= tiles_n (side_cols columns appended to the grid) run the side GEMV instead.
__global__ __launch_bounds__(256) void patch_embed_kernel(const float *__restrict__ lat, int B, int Cc, int H, int W,
                                                          const hxa_h *__restrict__ Wemb, int N, float *__restrict__ x,
                                                          int xrows, HxaSideGemv side, int tiles_n, int side_cols) {
  if ((int)blockIdx.x >= tiles_n) {  // an appended workgroup: side GEMV rows, before any barrier
    side_gemv<2>(side, (((int)blockIdx.x - tiles_n) * (int)gridDim.y + (int)blockIdx.y) * 4 +
                        __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
              side_cols * (int)gridDim.y * 4, threadIdx.x & 63);
    return;
  }
  __shared__ float4_t xs[64][17];  // [token][k / 4], one float4 of padding per row
  __shared__ float4_t ws[64][17];
  const int gw = W / 2, T = (H / 2) * gw, M = B * T, K = 4 * Cc;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64, tid = threadIdx.x;
  const int tr = tid / 16, tc = tid % 16;  // tokens tr*4 + i, columns tc + 16 j
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 64) {
    const int kc4 = min(64, K - k0) / 4;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int i = tid + 256 * u, r = i >> 4, k4 = i & 15;
      float4_t xv = {0.0f, 0.0f, 0.0f, 0.0f}, wv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (k4 < kc4) {
        const int m = m0 + r;
        if (m < M) {
          const int b = m / T, tk = m % T, gy = tk / gw, gx = tk % gw, c = k0 / 4 + k4;
          const float *p = lat + (((long)b * Cc + c) * H + 2 * gy) * W + 2 * gx;
          const float2_t top = *(const float2_t *)p, bot = *(const float2_t *)(p + W);
          xv = (float4_t){top[0], top[1], bot[0], bot[1]};
        }
        if (n0 + r < N) {
          const half4_t h = *(const half4_t *)(Wemb + (long)(n0 + r) * K + k0 + 4 * k4);
          wv = (float4_t){(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        }
      }
      xs[r][k4] = xv;
      ws[r][k4] = wv;
    }
    __syncthreads();
    for (int k4 = 0; k4 < kc4; k4++) {
      float4_t a[4], bq[4];
#pragma unroll
      for (int i = 0; i < 4; i++) a[i] = xs[tr * 4 + i][k4];
#pragma unroll
      for (int j = 0; j < 4; j++) bq[j] = ws[tc + 16 * j][k4];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int e = 0; e < 4; e++) acc[i][j] = fmaf(a[i][e], bq[j][e], acc[i][j]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + tr * 4 + i;
    if (m >= M) continue;
    float *y = x + ((long)(m / T) * xrows + m % T) * N;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = n0 + tc + 16 * j;
      if (n < N) y[n] = acc[i][j];
    }
  }
}

// timestep sinusoid (animad.cpp:425): out[i] = cos(t w_i), out[half+i] = sin(t w_i), w_i = 10000^(-i/half)
__global__ void sinusoid_kernel(const float *t, int n, int dim, float *out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int half = dim / 2;
  if (i >= n * half) return;
  const int b = i / half, j = i % half;
  const float a = sinusoid_angle(t[b], j, half);
  out[(long)b * dim + j] = cosf(a);
  out[(long)b * dim + half + j] = sinf(a);
}

// final layer (animad.cpp:474-492): per token LN (eps 1e-6, two-pass) * (1 + scale) + shift, linear D -> 4C,
// unpatchify (ph, pw, c) into lat; when dt != 0 the Euler update lat += dt * v is applied instead of storing v.
// With normw the norm is the MOSS head's RMSNorm * normw (mossrun.cpp:331-332), and with x0rows the 4C outputs v of
// token t go to x0rows[t][o] = zrows[t][o] - v, the rapid-moss estimate x0 = z - v (mossrun.cpp:333-334).
// FT = 16 tokens per workgroup of NW waves (16; 8 for 256 outputs):
// (1) statistics: wave w takes tokens w, w + NW (all its rows in flight together) and leaves (mu, 1/sigma) in LDS;
// (2) the linear: wave w takes the k range [w D/NW, (w+1) D/NW). Per 16-deep k step each lane normalises its 4
//     values of the A fragment (token lane % 16, k 4 (lane / 16) .. +3; the same fp32 expression as the
//     reference's normalised row), splits each into f16 hi = f16(a) and lo = f16(a - hi) (22 significant bits
//     together), and v_mfma_f32_16x16x16_f16 multiplies both by the f16 weights for the NOB = 4C / 16 output blocks
//     (the products are exact, the sums fp32). The weights come k-tiled by 4, Wf4 [D/4][4C][4], so a step reads one
//     contiguous block; row-major weights (64 rows 4 KB apart per step) made this phase 1.7x slower;
// (3) the NW partial sums of each output meet in LDS and are added in wave order; each thread then finishes its
//     outputs, reading every value it updates before it writes any.
// One wave per SIMD (96 workgroups of 4 waves at 1536 tokens) left every load and MFMA latency exposed (45 us);
// the 16-wave workgroup overlaps them.
// W32: fp32 weights (the MOSS head, final_linear_video, kept fp32 as the reference keeps it), Wf4 [D/4][4C][4] fp32;
// the products then go through v_mfma_f32_16x16x4_f32, four per 16-deep k step, with the normalised value unsplit.
constexpr int FT = 16;
template <int NOB, int NW, bool W32>
__global__ __launch_bounds__(64 * NW) void final_kernel(const float *__restrict__ x, int T, int xrows, int D,
                                                        const float *__restrict__ shift, const float *__restrict__ scale,
                                                        const void *__restrict__ Wf4, int Cc, int H, int W, float *lat,
                                                        const float *__restrict__ dtp, int ntok,
                                                        const float *__restrict__ normw, float *__restrict__ x0rows,
                                                        const float *__restrict__ zrows) {
  constexpr int NO = 16 * NOB, NT = 64 * NW;
  extern __shared__ float fsh[];  // [NW][FT][NO] partial sums, then [FT][2] statistics
  float *stat = fsh + NW * FT * NO;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok0 = blockIdx.x * FT;
  const int nv = D / 256;  // float4 per lane of a row (D % 256 == 0, D <= 4096)
  {
    constexpr int R = FT / NW;  // rows per wave: 1 or 2
    float4_t v[R][16];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int tok = min(tok0 + wave + NW * r, ntok - 1);
      const float4_t *xr = (const float4_t *)(x + ((long)(tok / T) * xrows + tok % T) * D);
#pragma unroll
      for (int i = 0; i < 16; i++)
        if (i < nv) v[r][i] = xr[lane + 64 * i];
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      float s = 0.0f;
      if (normw == nullptr) {
#pragma unroll
        for (int i = 0; i < 16; i++)
          if (i < nv) s += (v[r][i][0] + v[r][i][1]) + (v[r][i][2] + v[r][i][3]);
      }
      const float mu = normw == nullptr ? wave_sum(s) / (float)D : 0.0f;  // RMS: no centring
      float q = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++)
        if (i < nv) {
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const float d = v[r][i][e] - mu;
            q = fmaf(d, d, q);
          }
        }
      const float rs = 1.0f / sqrtf(wave_sum(q) / (float)D + 1e-6f);
      if (lane == 0) {
        stat[2 * (wave + NW * r)] = mu;
        stat[2 * (wave + NW * r) + 1] = rs;
      }
    }
  }
  __syncthreads();
  const int row = lane & 15, kk = 4 * (lane >> 4);
  const int tok = tok0 + row;
  const bool ok = tok < ntok;
  const float mu = stat[2 * row], rs = stat[2 * row + 1];
  const float *xr = x + ((long)(min(tok, ntok - 1) / T) * xrows + min(tok, ntok - 1) % T) * D;
  float4_t acc[NOB];
#pragma unroll
  for (int b = 0; b < NOB; b++) acc[b] = (float4_t){0.0f, 0.0f, 0.0f, 0.0f};
  // U k steps per round, their loads issued before the first use. The range D / NW is a multiple of 16 but not
  // always of 16 U (D 2560: 10 steps): past its end a round reloads the range's last step and skips its MFMAs.
  constexpr int U = NOB == 16 ? 1 : 2;
  const int kw = D / NW, kend = (wave + 1) * kw;
  for (int k0 = wave * kw; k0 < kend; k0 += 16 * U) {
    float4_t xv[U], sc[U], sh[U], nw[U];
    half4_t wv[U][W32 ? 1 : NOB];
    float4_t wf[U][W32 ? NOB : 1];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int c = min(k0 + 16 * u, kend - 16) + kk;
      xv[u] = *(const float4_t *)(xr + c);
      sc[u] = *(const float4_t *)(scale + c);
      sh[u] = *(const float4_t *)(shift + c);
      nw[u] = normw != nullptr ? *(const float4_t *)(normw + c) : (float4_t){1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
      for (int b = 0; b < NOB; b++) {
        const long wi = ((long)(c >> 2) * NO + 16 * b + row) * 4;
        if constexpr (W32) wf[u][b] = *(const float4_t *)((const float *)Wf4 + wi);
        else wv[u][b] = *(const half4_t *)((const hxa_h *)Wf4 + wi);
      }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (k0 + 16 * u >= kend) break;
      float4_t a4;
#pragma unroll
      for (int e = 0; e < 4; e++) a4[e] = ok ? (xv[u][e] - mu) * rs * nw[u][e] * (1.0f + sc[u][e]) + sh[u][e] : 0.0f;
      if constexpr (W32) {
        // instruction e takes k = 4 (lane / 16) + e of each lane's four: A[token][k] B[k][output] over the 16-deep step
#pragma unroll
        for (int b = 0; b < NOB; b++)
#pragma unroll
          for (int e = 0; e < 4; e++) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[e], wf[u][b][e], acc[b], 0, 0, 0);
      } else {
        half4_t hi, lo;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          hi[e] = (hxa_h)a4[e];
          lo[e] = (hxa_h)(a4[e] - (float)hi[e]);
        }
#pragma unroll
        for (int b = 0; b < NOB; b++) {
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(hi, wv[u][b], acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x16f16(lo, wv[u][b], acc[b], 0, 0, 0);
        }
      }
    }
  }
  // lane holds tokens 4 (lane / 16) + i, output 16 b + lane % 16
#pragma unroll
  for (int b = 0; b < NOB; b++)
#pragma unroll
    for (int i = 0; i < 4; i++) fsh[(wave * FT + 4 * (lane >> 4) + i) * NO + 16 * b + row] = acc[b][i];
  __syncthreads();
  constexpr int PER = FT * NO / NT;  // outputs per thread
  const float dt = dtp != nullptr ? *dtp : 0.0f;
  const int gw = W / 2;
  float val[PER], cur[PER];
  float *dst[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int idx = tid + NT * j, t = idx / NO, o = idx % NO, tk0 = tok0 + t;
    const float *ps = fsh + t * NO + o;
    float sum = ps[0];
#pragma unroll
    for (int w = 1; w < NW; w++) sum += ps[w * FT * NO];
    val[j] = sum;
    dst[j] = nullptr;
    cur[j] = 0.0f;
    if (tk0 >= ntok) continue;
    if (x0rows != nullptr) {
      dst[j] = x0rows + (long)tk0 * NO + o;
      cur[j] = zrows[(long)tk0 * NO + o];
    } else {
      const int bi = tk0 / T, tk = tk0 % T, gy = tk / gw, gx = tk % gw;
      const int ab = o / Cc, c = o % Cc, a = ab >> 1, bb = ab & 1;
      dst[j] = lat + (((long)bi * Cc + c) * H + gy * 2 + a) * W + gx * 2 + bb;
      if (dtp != nullptr) cur[j] = *dst[j];
    }
  }
#pragma unroll
  for (int j = 0; j < PER; j++) {
    if (dst[j] == nullptr) continue;
    if (x0rows != nullptr) *dst[j] = cur[j] - val[j];
    else *dst[j] = dtp != nullptr ? cur[j] + dt * val[j] : val[j];
  }
}

// W [N][K] fp16 or fp32 -> Wk [K/4][N][4] (k-tiled by 4: the final layer's weight layout)
template <typename V, typename T>
__global__ void ktile4_kernel(const T *__restrict__ W, int N, int K, T *__restrict__ Wk) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // one 4-k chunk of one row
  if (i >= (long)N * (K / 4)) return;
  const int n = (int)(i % N), g = (int)(i / N);
  *(V *)(Wk + i * 4) = *(const V *)(W + (long)n * K + 4 * g);
}

// q8 / q4 quantisation of W[N][K] fp32, one thread per (column n, 32-group g): amax of the fp16-rounded weights,
// s = f16(max(amax / qmax, 6.2e-5)), q = clip(rint(f16(w) / s)) (export_all.py:10-18, moss/export_all_q8.py:13)
__global__ void quantize_kernel(const float *W, int N, int K, int fmt, int kt, void *q, hxa_h *s) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int G = K / 32;
  if (i >= (long)N * G) return;
  const int n = (int)(i / G), g = (int)(i % G);
  const float *wr = W + (long)n * K + g * 32;
  float a[32], amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 32; j++) {
    a[j] = (float)(hxa_h)wr[j];
    amax = fmaxf(amax, fabsf(a[j]));
  }
  const float qmax = fmt == HXA_W_Q8 ? 127.0f : 7.0f, qmin = fmt == HXA_W_Q8 ? -127.0f : -8.0f;
  float sc = amax / qmax;
  if (sc < 6.2e-5f) sc = 6.2e-5f;
  const hxa_h sh = (hxa_h)sc;
  const float sf = (float)sh;
  s[(long)g * N + n] = sh;
  if (fmt == HXA_W_Q8) {
    int8_t *qr = (int8_t *)q + (kt ? ((long)g * N + n) * 32 : (long)n * K + g * 32);
#pragma unroll
    for (int j = 0; j < 32; j++) qr[j] = (int8_t)fminf(fmaxf(rintf(a[j] / sf), qmin), qmax);
  } else {
    uint32_t *qw = (uint32_t *)((uint8_t *)q + (kt ? ((long)g * N + n) * 16 : (long)n * (K / 2) + g * 16));
#pragma unroll
    for (int w8 = 0; w8 < 4; w8++) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int v = (int)fminf(fmaxf(rintf(a[w8 * 8 + j] / sf), qmin), qmax) + 8;
        word |= (uint32_t)v << ((j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1));
      }
      qw[w8] = word;
    }
  }
}

#ifndef HXA_NORM_WPC
#define HXA_NORM_WPC 4
#endif

inline unsigned nblk(long n, int per = 256) { return (unsigned)((n + per - 1) / per); }

}  // namespace

#define LAUNCH_OK() (hipGetLastError() == hipSuccess ? HXA_OK : HXA_E_HIP)

int hxa_resid_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, long ldt, const float *gate,
                              const float *shift, const float *scale, const float *w, float eps, hxa_h *h, long ldh,
                              hipStream_t st) {
  return hxa_residn_norm_mod_launch(x, ldx, T, D, t, t ? 1 : 0, 0, ldt, gate, shift, scale, w, eps, h, ldh, st);
}
int hxa_resid2_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, const hxa_h *t2, long ldt,
                               const float *gate, const float *shift, const float *scale, const float *w, float eps,
                               hxa_h *h, long ldh, hipStream_t st) {
  if (t2 && !t) return HXA_E_ARG;
  return hxa_residn_norm_mod_launch(x, ldx, T, D, t, t2 ? 2 : t ? 1 : 0, t2 ? (long)(t2 - t) : 0, ldt, gate, shift,
                                    scale, w, eps, h, ldh, st);
}
int hxa_residn_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, int np, long tz, long ldt,
                               const float *gate, const float *shift, const float *scale, const float *w, float eps,
                               hxa_h *h, long ldh, hipStream_t st) {
  if (T <= 0 || D % 256 != 0 || ldx % 4 || ldh % 4 || (np > 0 && (!t || ldt % 4 || tz % 4 || !gate))) return HXA_E_ARG;
  if (D > 4096 || !(np == 0 || np == 1 || np == 2 || np == 4)) return HXA_E_ARG;
  // HXA_NORM_WPC workgroups per CU, each taking every grid-th row
  static int num_cu = 0;
  if (num_cu == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&num_cu, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess)
      num_cu = 256;
  }
  const int grid = (int)std::min<long>(T, (long)HXA_NORM_WPC * num_cu);
  const int nv = (D + 1023) / 1024;
#define HXA_NORMROW(V, P)                                                                                         \
  if (nv == V && np == P)                                                                                          \
    hxa_launch(normrow_kernel<V, P>, dim3(grid), dim3(256), 0, st, x, ldx, D, T, t, tz, ldt, gate, shift, scale, w, \
               eps, h, ldh);
#define HXA_NORMROW_P(V) HXA_NORMROW(V, 0) HXA_NORMROW(V, 1) HXA_NORMROW(V, 2) HXA_NORMROW(V, 4)
  HXA_NORMROW_P(1) HXA_NORMROW_P(2) HXA_NORMROW_P(3) HXA_NORMROW_P(4)
#undef HXA_NORMROW_P
#undef HXA_NORMROW
  return LAUNCH_OK();
}

int hxa_norm_mod_launch(const float *x, long ldx, int T, int D, const float *shift, const float *scale, const float *w,
                        float eps, hxa_h *h, long ldh, hipStream_t st) {
  return hxa_resid_norm_mod_launch((float *)x, ldx, T, D, nullptr, 0, nullptr, shift, scale, w, eps, h, ldh, st);
}

int hxa_rmsrope_launch(hxa_h *q0, hxa_h *q1, const float *g0, const float *g1, long ldq, int T, int H, const float *cosT,
                       const float *sinT, int ttab, hipStream_t st) {
  if (T <= 0 || H <= 0 || (cosT && ttab <= 0) || ldq % 8 || (uintptr_t)q0 % 16 || (uintptr_t)q1 % 16) return HXA_E_ARG;
  dim3 g(nblk((long)T * H, 32), q1 ? 2 : 1);
  hxa_launch(rmsrope_kernel, g, dim3(256), 0, st, q0, q1, g0, g1, ldq, T, H, cosT, sinT, ttab > 0 ? ttab : 1);
  return LAUNCH_OK();
}

int hxa_resadd2_launch(float *x, long ldx, const hxa_h *t1, const hxa_h *t2, long ldt, int T, int D, const float *gate,
                       hipStream_t st) {
  return hxa_resaddn_launch(x, ldx, t1, 2, (long)(t2 - t1), ldt, T, D, gate, st);
}
int hxa_resaddn_launch(float *x, long ldx, const hxa_h *t, int np, long tz, long ldt, int T, int D, const float *gate,
                       hipStream_t st) {
  if (D % 4 || ldx % 4 || ldt % 4 || tz % 4 || !(np == 2 || np == 4)) return HXA_E_ARG;
  if (np == 2)
    hxa_launch(resaddn_kernel<2>, dim3(nblk((long)T * D / 4)), dim3(256), 0, st, x, ldx, t, tz, ldt, T, D, gate);
  else
    hxa_launch(resaddn_kernel<4>, dim3(nblk((long)T * D / 4)), dim3(256), 0, st, x, ldx, t, tz, ldt, T, D, gate);
  return LAUNCH_OK();
}

int hxa_x32_to_rows_launch(const float *tiles, float *x, int R, int C, hipStream_t st) {
  if (R % 32 || C % 32) return HXA_E_ARG;
  hxa_launch(x32_to_rows_kernel, dim3(nblk((long)R * C)), dim3(256), 0, st, tiles, x, R, C);
  return LAUNCH_OK();
}
int hxa_rows_to_x32_launch(const float *x, float *tiles, int R, int C, hipStream_t st) {
  if (R % 32 || C % 32) return HXA_E_ARG;
  hxa_launch(rows_to_x32_kernel, dim3(nblk((long)R * C)), dim3(256), 0, st, x, tiles, R, C);
  return LAUNCH_OK();
}
int hxa_h16_to_rows_launch(const hxa_h *tiles, hxa_h *a, long lda, int R, int C, hipStream_t st) {
  if (R % 32 || C % 32) return HXA_E_ARG;
  hxa_launch(h16_to_rows_kernel, dim3(nblk((long)R * C)), dim3(256), 0, st, tiles, a, lda, R, C);
  return LAUNCH_OK();
}
int hxa_rows_to_h16_launch(const hxa_h *a, long lda, hxa_h *tiles, int R, int C, int transposed, hipStream_t st) {
  if (R % 32 || C % 32) return HXA_E_ARG;
  hxa_launch(rows_to_h16_kernel, dim3(nblk((long)R * C)), dim3(256), 0, st, a, lda, tiles, R, C, transposed);
  return LAUNCH_OK();
}
int hxa_cs_to_rows_launch(const float *tiles, float *rows, int T, hipStream_t st) {
  if (T % 32) return HXA_E_ARG;
  hxa_launch(cs_to_rows_kernel, dim3(nblk((long)T * 64)), dim3(256), 0, st, tiles, rows, T);
  return LAUNCH_OK();
}

int hxa_fill_normal_launch(void *dst, int dtype, size_t n, uint64_t seed, float mean, float std, hipStream_t st) {
  if (n == 0) return HXA_OK;
  hxa_launch(fill_normal_kernel, dim3(nblk((long)n)), dim3(256), 0, st, dst, dtype, n, seed, mean, std);
  return LAUNCH_OK();
}
int hxa_fill_uniform_int_launch(void *dst, int bits, size_t n, uint64_t seed, int lo, int hi, hipStream_t st) {
  if (n == 0) return HXA_OK;
  if (hi < lo || (bits != 8 && bits != 4)) return HXA_E_ARG;
  hxa_launch(fill_uniform_int_kernel, dim3(nblk((long)n)), dim3(256), 0, st, dst, bits, n, seed, lo, hi);
  return LAUNCH_OK();
}
int hxa_fill_const_launch(void *dst, int dtype, size_t n, float v, hipStream_t st) {
  if (n == 0) return HXA_OK;
  hxa_launch(fill_const_kernel, dim3(nblk((long)n)), dim3(256), 0, st, dst, dtype, n, v);
  return LAUNCH_OK();
}

int hxa_patchify_launch(const float *lat, int B, int Cc, int H, int W, float *tok, hipStream_t st) {
  if (H % 2 || W % 2) return HXA_E_ARG;
  hxa_launch(patchify_kernel, dim3(nblk((long)B * Cc * H * W)), dim3(256), 0, st, lat, B, Cc, H, W, tok);
  return LAUNCH_OK();
}

int hxa_patch_embed_launch(const float *lat, int B, int Cc, int H, int W, const hxa_h *Wemb, int N, float *x, int xrows,
                           hipStream_t st, const HxaSideGemv *side) {
  if (B < 1 || Cc < 1 || H % 2 || W % 2 || H < 2 || W < 2 || N < 1 || xrows < (H / 2) * (W / 2)) return HXA_E_ARG;
  if ((uintptr_t)lat % 8 || (uintptr_t)Wemb % 8) return HXA_E_ARG;  // float2 latent pairs (W even), half4 weights
  if (side && (!hxa_side_k_ok(side->K) || side->N <= 0 || side->per <= 0 || !side->x || !side->W || !side->y ||
               ((uintptr_t)side->x | (uintptr_t)side->W) % 16))
    return HXA_E_ARG;
  const int M = B * (H / 2) * (W / 2), gx = (int)nblk(N, 64), gy = (int)nblk(M, 64);
  // the side GEMV: enough appended columns for ~16 rows per wave (the embedding itself is latency-bound, so the
  // GEMV's weight stream runs beside it)
  const int cols = side ? (int)std::min<long>(std::max<long>((side->N + 16 * 4 * gy - 1) / (16 * 4 * gy), 1), 64) : 0;
  hxa_launch(patch_embed_kernel, dim3(gx + cols, gy), dim3(256), 0, st, lat, B, Cc, H, W, Wemb, N, x, xrows,
             side ? *side : HxaSideGemv{}, gx, cols);
  return LAUNCH_OK();
}

template <typename WT>
static int linear_launch(const float *x, long ldx, int M, int K, const WT *W, int N, float *y, long ldy, int act,
                         const float *bias, int split, int gap, hipStream_t st) {
  if (M <= 0 || K <= 0 || N <= 0 || (uintptr_t)W % (2 * sizeof(WT))) return HXA_E_ARG;
  if (M <= 8) {
    if (K % 2 || (act == 2 && (M != 1 || K % 4))) return HXA_E_ARG;
    hxa_launch(gemv_kernel<WT>, dim3(nblk(N, 4)), dim3(256), 0, st, x, ldx, M, K, W, N, y, ldy, act, bias,
               split > 0 ? split : N, gap);
  } else {
    return HXA_E_ARG;  // more than 8 rows: the patch embed has its own kernel (hxa_patch_embed_launch)
  }
  return LAUNCH_OK();
}
int hxa_linear_f32_launch(const float *x, long ldx, int M, int K, const hxa_h *W, int N, float *y, long ldy, int act,
                          const float *bias, int split, int gap, hipStream_t st) {
  return linear_launch(x, ldx, M, K, W, N, y, ldy, act, bias, split, gap, st);
}
int hxa_linear_w32_launch(const float *x, long ldx, int M, int K, const float *W, int N, float *y, long ldy, int act,
                          const float *bias, int split, int gap, hipStream_t st) {
  return linear_launch(x, ldx, M, K, W, N, y, ldy, act, bias, split, gap, st);
}

int hxa_modgemv_launch(const float *x, int K, const hxa_h *W, long N, float *y, int per, long ostride, int split, int gap,
                       int act, hipStream_t st) {
  if (N <= 0 || per <= 0 || K % 256 || K < 256 || K > 4096 || split < 0 || gap < 0) return HXA_E_ARG;
  if ((uintptr_t)x % 16 || (uintptr_t)W % 16) return HXA_E_ARG;
  // rows per wave: 8 for the modulation of all blocks (344K rows at 2048), 2 for short matrices (the final layer's
  // 4096 rows: 128 workgroups of 8 rows per wave left half the SIMDs idle, 10.6 us for 16.8 MB), 4 between (one
  // block's 6D rows: every wave first loads and activates the whole input vector, which 2 rows do not amortise)
  const int RPW = N >= 65536 ? 8 : N >= 8192 ? 4 : 2;
  const dim3 grid((unsigned)((N + 4 * RPW - 1) / (4 * RPW)));
#define HXA_MODGEMV(KC, EPL)                                                                                       \
  hxa_launch((modgemv_kernel<KC, EPL>), grid, dim3(256), 0, st, x, W, N, y, per, ostride, split, gap, act, RPW)
  if (K % 512) {
    switch (K / 256) {
      case 1: HXA_MODGEMV(1, 4); break;
      case 3: HXA_MODGEMV(3, 4); break;
      case 5: HXA_MODGEMV(5, 4); break;
      case 7: HXA_MODGEMV(7, 4); break;
      default: return HXA_E_ARG;
    }
  } else {
    switch (K / 512) {
      case 1: HXA_MODGEMV(1, 8); break;
      case 2: HXA_MODGEMV(2, 8); break;
      case 3: HXA_MODGEMV(3, 8); break;
      case 4: HXA_MODGEMV(4, 8); break;
      case 5: HXA_MODGEMV(5, 8); break;
      case 6: HXA_MODGEMV(6, 8); break;
      case 7: HXA_MODGEMV(7, 8); break;
      case 8: HXA_MODGEMV(8, 8); break;
      default: return HXA_E_ARG;
    }
  }
#undef HXA_MODGEMV
  return LAUNCH_OK();
}


int hxa_ktile4_launch(const hxa_h *W, int N, int K, hxa_h *Wk, hipStream_t st) {
  if (N <= 0 || K <= 0 || K % 4 || (uintptr_t)W % 8 || (uintptr_t)Wk % 8) return HXA_E_ARG;
  hxa_launch((ktile4_kernel<half4_t, hxa_h>), dim3(nblk((long)N * (K / 4))), dim3(256), 0, st, W, N, K, Wk);
  return LAUNCH_OK();
}
int hxa_ktile4_f32_launch(const float *W, int N, int K, float *Wk, hipStream_t st) {
  if (N <= 0 || K <= 0 || K % 4 || (uintptr_t)W % 16 || (uintptr_t)Wk % 16) return HXA_E_ARG;
  hxa_launch((ktile4_kernel<float4_t, float>), dim3(nblk((long)N * (K / 4))), dim3(256), 0, st, W, N, K, Wk);
  return LAUNCH_OK();
}

namespace {
template <bool W32>
int final_launch(const float *x, int B, int T, int xrows, int D, const float *shift, const float *scale, const void *Wf4,
                 int Cc, int H, int W, float *lat, const float *dtp, hipStream_t st, const float *normw, float *x0rows,
                 const float *zrows) {
  if ((x0rows == nullptr) != (zrows == nullptr) || (normw && (uintptr_t)normw % 16)) return HXA_E_ARG;
  const int NO = 4 * Cc;
  if ((NO != 64 && NO != 128 && NO != 256) || (H / 2) * (W / 2) != T || xrows < T || D % 256 || D > 4096 || B * T < 1)
    return HXA_E_ARG;
  if ((uintptr_t)x % 16 || (uintptr_t)shift % 16 || (uintptr_t)scale % 16 || (uintptr_t)Wf4 % (W32 ? 16 : 8))
    return HXA_E_ARG;
  // partial sums + statistics: 16 x 16 x 64, 16 x 16 x 128 or 8 x 16 x 256 floats (64 / 128 / 128 KB)
  auto bytes = [](int nw, int no) { return (int)sizeof(float) * (nw * FT * no + 2 * FT); };
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void *)final_kernel<4, 16, W32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            bytes(16, 64)) != hipSuccess ||
        hipFuncSetAttribute((const void *)final_kernel<8, 16, W32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            bytes(16, 128)) != hipSuccess ||
        hipFuncSetAttribute((const void *)final_kernel<16, 8, W32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            bytes(8, 256)) != hipSuccess)
      return HXA_E_HIP;
    attr = true;
  }
  const int ntok = B * T;
  const dim3 grid((ntok + FT - 1) / FT);
  if (NO == 64)
    hxa_launch(final_kernel<4, 16, W32>, grid, dim3(1024), bytes(16, 64), st, x, T, xrows, D, shift, scale, Wf4, Cc, H,
               W, lat, dtp, ntok, normw, x0rows, zrows);
  else if (NO == 128)
    hxa_launch(final_kernel<8, 16, W32>, grid, dim3(1024), bytes(16, 128), st, x, T, xrows, D, shift, scale, Wf4, Cc,
               H, W, lat, dtp, ntok, normw, x0rows, zrows);
  else
    hxa_launch(final_kernel<16, 8, W32>, grid, dim3(512), bytes(8, 256), st, x, T, xrows, D, shift, scale, Wf4, Cc, H,
               W, lat, dtp, ntok, normw, x0rows, zrows);
  return LAUNCH_OK();
}
}  // namespace

int hxa_final_launch(const float *x, int B, int T, int xrows, int D, const float *shift, const float *scale,
                     const void *Wf4, int Cc, int H, int W, float *lat, const float *dtp, hipStream_t st,
                     const float *normw, float *x0rows, const float *zrows, int w32) {
  return w32 ? final_launch<true>(x, B, T, xrows, D, shift, scale, Wf4, Cc, H, W, lat, dtp, st, normw, x0rows, zrows)
             : final_launch<false>(x, B, T, xrows, D, shift, scale, Wf4, Cc, H, W, lat, dtp, st, normw, x0rows, zrows);
}



// ---- the reference's own DiT glue (phone/animad.cpp:424-492, moss/mossrun/mossrun.cpp:255-343) ----
// y = x * rsqrt(mean(x^2) + eps) * w, one vector of n <= 4096 (animad.cpp:115-123 rms_rows on the t-embedding)
__global__ __launch_bounds__(256) void rmsvec_kernel(const float *__restrict__ x, int n, const hxa_h *__restrict__ w,
                                                     float eps, float *__restrict__ y) {
  __shared__ float part[4];
  float q = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) q = fmaf(x[i], x[i], q);
  q = wave_sum(q);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = q;
  __syncthreads();
  const float r = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
  for (int i = threadIdx.x; i < n; i += 256) y[i] = x[i] * r * (float)w[i];
}
// G independent GEMVs in one launch: y[g * ldy + n] = bias[n] + sum_k W[g][n][k] x[g * ldx + k] (W fp16
// [G][N][K]); one wave per output row. The per-block, per-site B matrices of the Anima modulation (megarun.cpp:166-167)
__global__ __launch_bounds__(256) void grouped_gemv_kernel(const float *__restrict__ x, long ldx, const hxa_h *__restrict__ W,
                                                           int N, int K, const float *__restrict__ bias, float *__restrict__ y,
                                                           long ldy) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63, g = blockIdx.y;
  if (n >= N) return;
  const hxa_h *wr = W + ((long)g * N + n) * K;
  const float *xg = x + (long)g * ldx;
  float acc = 0.0f;
  for (int k = lane * 2; k < K; k += 128) {
    const half2_t wv = *(const half2_t *)(wr + k);
    acc = fmaf(xg[k], (float)wv[0], fmaf(xg[k + 1], (float)wv[1], acc));
  }
  acc = wave_sum(acc);
  if (lane == 0) y[(long)g * ldy + n] = acc + (bias ? bias[n] : 0.0f);
}
// Groups of GEMV rows whose weights sit in separate allocations: group g reads x + g * x_gs (SiLU applied on load
// when act == 1), weight rows Wp[g / gpp] + w_off + (g % gpp) * w_gs ([N][K] fp16) and writes y + g * y_gs [N],
// plus bias. Same per-lane order of the products as gemv_kernel, so the same sums.
__global__ __launch_bounds__(256) void ptr_gemv_kernel(const float *__restrict__ x, long x_gs, int act,
                                                       const hxa_h *const *__restrict__ Wp, int gpp, long w_off, long w_gs,
                                                       int N, int K, const float *__restrict__ bias, float *__restrict__ y,
                                                       long y_gs) {
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63, g = blockIdx.y;
  if (n >= N) return;
  const hxa_h *wr = Wp[g / gpp] + w_off + (long)(g % gpp) * w_gs + (long)n * K;
  const float *xg = x + (long)g * x_gs;
  float acc = 0.0f;
  for (int k = lane * 2; k < K; k += 128) {
    const half2_t wv = *(const half2_t *)(wr + k);
    float x0 = xg[k], x1 = xg[k + 1];
    if (act == 1) {
      x0 = x0 / (1.0f + __expf(-x0));
      x1 = x1 / (1.0f + __expf(-x1));
    }
    acc = fmaf(x0, (float)wv[0], fmaf(x1, (float)wv[1], acc));
  }
  acc = wave_sum(acc);
  if (lane == 0) y[(long)g * y_gs + n] = acc + (bias ? bias[n] : 0.0f);
}
// rapid-moss input (mossrun.cpp:316-320): per image token t, xin = z_t + Q x0_t (Q fp32 [C4][C4]) and the token's
// row x = Wv xin + bv (Wv [D][C4], fp32 or fp16); FT tokens per workgroup, their xin in LDS, each weight row read once
template <typename WT>
__global__ __launch_bounds__(256) void moss_embed_kernel(const float *__restrict__ z, const float *__restrict__ x0,
                                                         const float *__restrict__ Q, const WT *__restrict__ Wv,
                                                         const float *__restrict__ bv, float *__restrict__ x, int T,
                                                         int xrows, int D, int C4, int ntok) {
  extern __shared__ float xin[];  // [FT][C4]
  const int tok0 = blockIdx.x * FT;
  for (int i = threadIdx.x; i < FT * C4; i += 256) {
    const int tl = i / C4, o = i % C4, tok = tok0 + tl;
    float a = 0.0f;
    if (tok < ntok) {
      a = z[(long)tok * C4 + o];
      const float *xr = x0 + (long)tok * C4;
      for (int c = 0; c < C4; c++) a = fmaf(Q[o * C4 + c], xr[c], a);
    }
    xin[i] = a;
  }
  __syncthreads();
  for (int n = threadIdx.x; n < D; n += 256) {
    float acc[FT];
#pragma unroll
    for (int t = 0; t < FT; t++) acc[t] = bv[n];
    const WT *wr = Wv + (long)n * C4;
    for (int c = 0; c < C4; c += 2) {
      const float2_t wv = wpair(wr + c);
#pragma unroll
      for (int t = 0; t < FT; t++) acc[t] = fmaf(xin[t * C4 + c], wv[0], fmaf(xin[t * C4 + c + 1], wv[1], acc[t]));
    }
#pragma unroll
    for (int t = 0; t < FT; t++) {
      const int tok = tok0 + t;
      if (tok < ntok) x[((long)(tok / T) * xrows + tok % T) * D + n] = acc[t];
    }
  }
}
// BN denorm + unpatchify (mossrun.cpp:339-343): x0 token rows [B*T][4C] (feature c*4 + ph*2 + pw) ->
// lat [B][C][H][W] = x0 * sqrt(var + 1e-4) + mean, per feature
__global__ void bn_unpatchify_kernel(const float *__restrict__ x0, const float *__restrict__ mean,
                                     const float *__restrict__ var, int B, int Cc, int H, int W, float *__restrict__ lat) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  const int C4 = 4 * Cc, gh = H / 2, gw = W / 2;
  if (i >= (long)B * gh * gw * C4) return;
  const int f = (int)(i % C4);
  const long tb = i / C4;
  const int tk = (int)(tb % (gh * gw)), b = (int)(tb / (gh * gw));
  const int gy = tk / gw, gx = tk % gw, c = f / 4, ph = (f / 2) & 1, pw = f & 1;
  lat[(((long)b * Cc + c) * H + 2 * gy + ph) * W + 2 * gx + pw] = x0[i] * sqrtf(var[f] + 1e-4f) + mean[f];
}

// ---- low-res first steps (phone/animad.cpp:392-503, moss/mossrun/mossrun.cpp:278-313). Round-to-nearest
// operations in the reference's order, no contraction: the results are the reference's fp32 / double values.
// t = sig[0], tn = sig[1], sig[2] = tn - t (the runner's sigma vector in device memory).
// x_low [BC][H/f][W/f] = (1 - t) mean_fxf(dhat) + t sum_fxf(noise) / f, the sums in double (animad.cpp:429-437)
__global__ void lowres_pool_kernel(const float *__restrict__ nfull, const float *__restrict__ dhat, long BC, int H, int W,
                                   int f, const float *__restrict__ sig, float *__restrict__ xlow) {
  const int Hl = H / f, Wl = W / f;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= BC * Hl * Wl) return;
  const int x = (int)(i % Wl), y = (int)((i / Wl) % Hl);
  const long c = i / ((long)Wl * Hl);
  double sn = 0.0, sd = 0.0;
  for (int a = 0; a < f; a++)
    for (int b = 0; b < f; b++) {
      const long j = (c * H + (long)y * f + a) * W + (long)x * f + b;
      sn = __dadd_rn(sn, (double)nfull[j]);
      sd = __dadd_rn(sd, (double)dhat[j]);
    }
  const float t = sig[0];  // (1 - t) is a float expression in the reference, the rest double
  xlow[i] = (float)__dadd_rn(__ddiv_rn(__dmul_rn((double)__fsub_rn(1.0f, t), sd), (double)(f * f)),
                             __ddiv_rn(__dmul_rn((double)t, sn), (double)f));
}
// dl = x_low - t v_low bilinearly upsampled (half-pixel centres, clamped) into dhat; x_next = (1 - tn) dhat + tn noise;
// v = (x - x_next) / (t - tn) (0 when t - tn <= 1e-6); then the Euler step x += (tn - t) v in place (animad.cpp:486-503
// and the sampler's update)
__global__ void lowres_velocity_kernel(const float *__restrict__ xlow, const float *__restrict__ vlow, float *__restrict__ lat,
                                       const float *__restrict__ nfull, float *__restrict__ dhat, long BC, int H, int W,
                                       int f, const float *__restrict__ sig) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= BC * H * W) return;
  const int Hl = H / f, Wl = W / f;
  const int x = (int)(i % W), y = (int)((i / W) % H);
  const long c = i / ((long)W * H);
  const float t = sig[0];
  const double tn = (double)sig[1], dt = __dsub_rn((double)t, tn);
  const float fy = __fsub_rn(__fdiv_rn(__fadd_rn((float)y, 0.5f), (float)f), 0.5f);
  const float fx = __fsub_rn(__fdiv_rn(__fadd_rn((float)x, 0.5f), (float)f), 0.5f);
  int y0 = (int)floorf(fy), x0 = (int)floorf(fx);
  const float wy = __fsub_rn(fy, (float)y0), wx = __fsub_rn(fx, (float)x0);
  const int y1 = min(max(y0 + 1, 0), Hl - 1), x1 = min(max(x0 + 1, 0), Wl - 1);
  y0 = min(max(y0, 0), Hl - 1);
  x0 = min(max(x0, 0), Wl - 1);
  const long base = c * Hl * Wl;
  auto dl = [&](int yy, int xx) {
    const long j = base + (long)yy * Wl + xx;
    return __fsub_rn(xlow[j], __fmul_rn(t, vlow[j]));
  };
  const float owy = __fsub_rn(1.0f, wy), owx = __fsub_rn(1.0f, wx);
  const float top = __fadd_rn(__fmul_rn(owx, dl(y0, x0)), __fmul_rn(wx, dl(y0, x1)));
  const float bot = __fadd_rn(__fmul_rn(owx, dl(y1, x0)), __fmul_rn(wx, dl(y1, x1)));
  const float up = __fadd_rn(__fmul_rn(owy, top), __fmul_rn(wy, bot));
  dhat[i] = up;
  const float xnext = __fadd_rn(__fmul_rn((float)__dsub_rn(1.0, tn), up), __fmul_rn((float)tn, nfull[i]));
  const float xf = lat[i];
  const float v = dt > 1e-6 ? __fdiv_rn(__fsub_rn(xf, xnext), (float)dt) : 0.0f;
  lat[i] = __fadd_rn(xf, __fmul_rn(sig[2], v));
}
// token rows [B][H*W][C4] -> 2 x the 2x2 mean, [B][(H/2)*(W/2)][C4] (mossrun.cpp:291)
__global__ void moss_pool2_kernel(const float *__restrict__ z, int B, int H, int W, int C4, float *__restrict__ zl) {
  const int Wl = W / 2, Tl = (H / 2) * Wl;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * Tl * C4) return;
  const int cc = (int)(i % C4), tk = (int)((i / C4) % Tl);
  const long b = i / ((long)C4 * Tl);
  const int ii = tk / Wl, jj = tk % Wl;
  const float *zb = z + b * H * W * C4;
  auto at = [&](int r, int q) { return zb[((long)r * W + q) * C4 + cc]; };
  const float sum = __fadd_rn(__fadd_rn(__fadd_rn(at(2 * ii, 2 * jj), at(2 * ii, 2 * jj + 1)), at(2 * ii + 1, 2 * jj)),
                              at(2 * ii + 1, 2 * jj + 1));
  zl[i] = __fmul_rn(0.5f, sum);
}
// token rows [B][h*w][C4] -> bilinear 2x with half-pixel centres, clamped, [B][(2h)*(2w)][C4] (mossrun.cpp:278-282)
__global__ void upsample2_rows_kernel(const float *__restrict__ src, int B, int h, int w, int C4, float *__restrict__ dst) {
  const int Tn = 4 * h * w;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)B * Tn * C4) return;
  const int cc = (int)(i % C4), tk = (int)((i / C4) % Tn);
  const long b = i / ((long)C4 * Tn);
  const int y = tk / (2 * w), x = tk % (2 * w);
  const float fy = __fsub_rn(__fdiv_rn(__fadd_rn((float)y, 0.5f), 2.0f), 0.5f);
  const float fx = __fsub_rn(__fdiv_rn(__fadd_rn((float)x, 0.5f), 2.0f), 0.5f);
  const int y0 = (int)floorf(fy), x0 = (int)floorf(fx);
  const float ty = __fsub_rn(fy, (float)y0), tx = __fsub_rn(fx, (float)x0);
  const int ya = min(max(y0, 0), h - 1), yb = min(max(y0 + 1, 0), h - 1);
  const int xa = min(max(x0, 0), w - 1), xb = min(max(x0 + 1, 0), w - 1);
  const float *sb = src + b * h * w * C4;
  auto at = [&](int r, int q) { return sb[((long)r * w + q) * C4 + cc]; };
  const float otx = __fsub_rn(1.0f, tx), oty = __fsub_rn(1.0f, ty);
  const float top = __fadd_rn(__fmul_rn(otx, at(ya, xa)), __fmul_rn(tx, at(ya, xb)));
  const float bot = __fadd_rn(__fmul_rn(otx, at(yb, xa)), __fmul_rn(tx, at(yb, xb)));
  dst[i] = __fadd_rn(__fmul_rn(oty, top), __fmul_rn(ty, bot));
}

// ---- weight-file import: the reference's on-disk tiles (already in device memory) -> k-tiled pack matrices.
// fp16 crouton tiles of a [K][N] matrix, [N/32][K/32] tiles of 1024 halves with k pairs interleaved (export_all.py:7-8)
// -> rows row0 .. row0 + N of a k-tiled [K/32][ldn][32] fp16 matrix; one thread per output element, k fastest
__global__ void crouton_to_ktiled_kernel(const uint16_t *__restrict__ src, int N, int K, uint16_t *__restrict__ dst,
                                         int row0, int ldn) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)N * K) return;
  const int r = (int)(i & 31), n = (int)((i >> 5) % N);
  const long g = (i >> 5) / N;
  dst[(g * ldn + row0 + n) * 32 + r] = src[((long)(n >> 5) * (K / 32) + g) * 1024 + (r >> 1) * 64 + (n & 31) * 2 + (r & 1)];
}
// q8 records of a [K][N] matrix, [N/32][kbt] records of 1152 bytes: 64 fp16 scales (each stored twice) and 1024
// offset-binary bytes u = q + 128 with k pairs interleaved (export_all.py:10-18) -> int8 rows row0 .. row0 + N of a
// k-tiled [Kt/32][ldn][32] matrix and scales s[Kt/32][ldn]. Record k-block ib < nkb_main is k group ib, the others
// (the rapid-moss LoRA's B rows, moss/export_moss.py:40-46) group lora_g + ib - nkb_main.
__global__ void q8rec_to_ktiled_kernel(const uint8_t *__restrict__ rec, int N, int nkb, int kbt, uint8_t *__restrict__ q,
                                       uint16_t *__restrict__ s, int row0, int ldn, int nkb_main, int lora_g) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)N * nkb * 32) return;
  const int r = (int)(i & 31), n = (int)((i >> 5) % N), ib = (int)((i >> 5) / N);
  const int c = n & 31;
  const uint8_t *R = rec + ((long)(n >> 5) * kbt + ib) * 1152;
  const long g = ib < nkb_main ? ib : lora_g + (ib - nkb_main);
  q[(g * ldn + row0 + n) * 32 + r] = (uint8_t)(R[128 + (r >> 1) * 64 + c * 2 + (r & 1)] ^ 0x80);
  if (r == 0) s[g * ldn + row0 + n] = ((const uint16_t *)R)[2 * c];
}

int hxa_rmsvec_launch(const float *x, int n, const hxa_h *w, float eps, float *y, hipStream_t st) {
  if (n <= 0 || n > 4096) return HXA_E_ARG;
  hxa_launch(rmsvec_kernel, dim3(1), dim3(256), 0, st, x, n, w, eps, y);
  return LAUNCH_OK();
}
int hxa_grouped_gemv_launch(const float *x, long ldx, const hxa_h *W, int G, int N, int K, const float *bias, float *y,
                            long ldy, hipStream_t st) {
  if (G <= 0 || N <= 0 || K <= 0 || K % 2 || G > 65535) return HXA_E_ARG;
  hxa_launch(grouped_gemv_kernel, dim3(nblk(N, 4), G), dim3(256), 0, st, x, ldx, W, N, K, bias, y, ldy);
  return LAUNCH_OK();
}
int hxa_ptr_gemv_launch(const float *x, long x_gs, int act, const hxa_h *const *Wp, int G, int gpp, long w_off, long w_gs,
                        int N, int K, const float *bias, float *y, long y_gs, hipStream_t st) {
  if (G <= 0 || gpp <= 0 || N <= 0 || K <= 0 || K % 2 || G > 65535 || !Wp) return HXA_E_ARG;
  hxa_launch(ptr_gemv_kernel, dim3(nblk(N, 4), G), dim3(256), 0, st, x, x_gs, act, Wp, gpp, w_off, w_gs, N, K, bias, y,
             y_gs);
  return LAUNCH_OK();
}
int hxa_moss_embed_launch(const float *z, const float *x0, const float *Q, const void *Wv, int w32, const float *bv,
                          float *x, int B, int T, int xrows, int D, int C4, hipStream_t st) {
  if (C4 % 2 || C4 > 512 || B <= 0 || T <= 0 || xrows < T || (uintptr_t)Wv % (w32 ? 8 : 4)) return HXA_E_ARG;
  const int ntok = B * T;
  if (w32)
    hxa_launch(moss_embed_kernel<float>, dim3((ntok + FT - 1) / FT), dim3(256), sizeof(float) * FT * C4, st, z, x0, Q,
               (const float *)Wv, bv, x, T, xrows, D, C4, ntok);
  else
    hxa_launch(moss_embed_kernel<hxa_h>, dim3((ntok + FT - 1) / FT), dim3(256), sizeof(float) * FT * C4, st, z, x0, Q,
               (const hxa_h *)Wv, bv, x, T, xrows, D, C4, ntok);
  return LAUNCH_OK();
}
int hxa_bn_unpatchify_launch(const float *x0, const float *mean, const float *var, int B, int Cc, int H, int W, float *lat,
                             hipStream_t st) {
  hxa_launch(bn_unpatchify_kernel, dim3(nblk((long)B * Cc * H * W)), dim3(256), 0, st, x0, mean, var, B, Cc, H, W,
                     lat);
  return LAUNCH_OK();
}

int hxa_lowres_pool_launch(const float *nfull, const float *dhat, long BC, int H, int W, int f, const float *sig,
                           float *xlow, hipStream_t st) {
  if (f < 2 || H % f || W % f || BC <= 0) return HXA_E_ARG;
  hxa_launch(lowres_pool_kernel, dim3(nblk(BC * (H / f) * (W / f))), dim3(256), 0, st, nfull, dhat, BC, H, W, f, sig, xlow);
  return LAUNCH_OK();
}
int hxa_lowres_velocity_launch(const float *xlow, const float *vlow, float *lat, const float *nfull, float *dhat, long BC,
                               int H, int W, int f, const float *sig, hipStream_t st) {
  if (f < 2 || H % f || W % f || BC <= 0) return HXA_E_ARG;
  hxa_launch(lowres_velocity_kernel, dim3(nblk(BC * H * W)), dim3(256), 0, st, xlow, vlow, lat, nfull, dhat, BC, H, W, f,
             sig);
  return LAUNCH_OK();
}
int hxa_moss_pool2_launch(const float *z, int B, int H, int W, int C4, float *zl, hipStream_t st) {
  if (H % 2 || W % 2 || B <= 0 || C4 <= 0) return HXA_E_ARG;
  hxa_launch(moss_pool2_kernel, dim3(nblk((long)B * (H / 2) * (W / 2) * C4)), dim3(256), 0, st, z, B, H, W, C4, zl);
  return LAUNCH_OK();
}
int hxa_upsample2_rows_launch(const float *src, int B, int h, int w, int C4, float *dst, hipStream_t st) {
  if (h <= 0 || w <= 0 || B <= 0 || C4 <= 0) return HXA_E_ARG;
  hxa_launch(upsample2_rows_kernel, dim3(nblk((long)B * 4 * h * w * C4)), dim3(256), 0, st, src, B, h, w, C4, dst);
  return LAUNCH_OK();
}

int hxa_crouton_to_ktiled_launch(const void *src, int N, int K, void *dst, int row0, int ldn, hipStream_t st) {
  if (N % 32 || K % 32 || row0 < 0 || row0 + N > ldn) return HXA_E_ARG;
  hxa_launch(crouton_to_ktiled_kernel, dim3(nblk((long)N * K)), dim3(256), 0, st, (const uint16_t *)src, N, K,
             (uint16_t *)dst, row0, ldn);
  return LAUNCH_OK();
}
int hxa_q8rec_to_ktiled_launch(const void *rec, int N, int nkb, int kbt, void *q, void *s, int row0, int ldn, int nkb_main,
                               int lora_g, hipStream_t st) {
  if (N % 32 || nkb <= 0 || nkb > kbt || row0 < 0 || row0 + N > ldn) return HXA_E_ARG;
  hxa_launch(q8rec_to_ktiled_kernel, dim3(nblk((long)N * nkb * 32)), dim3(256), 0, st, (const uint8_t *)rec, N, nkb, kbt,
             (uint8_t *)q, (uint16_t *)s, row0, ldn, nkb_main, lora_g);
  return LAUNCH_OK();
}

// the per-step sigma values: sig[0..3] = {s0, s1, s1 - s0, 0}, one value per lane (vector stores)
__global__ void set_sigma_kernel(float *sig, float s0, float s1) {
  const int i = threadIdx.x;
  if (i < 4) sig[i] = i == 0 ? s0 : i == 1 ? s1 : i == 2 ? s1 - s0 : 0.0f;
}
int hxa_set_sigma_launch(float *sig, float s0, float s1, hipStream_t st) {
  hxa_launch(set_sigma_kernel, dim3(1), dim3(64), 0, st, sig, s0, s1);
  return LAUNCH_OK();
}
// n floats from host-mapped pinned memory into device memory on the compute queue (16 bytes per thread; n % 4 == 0)
__global__ void copy_f4_kernel(const float4_t *__restrict__ src, float4_t *__restrict__ dst, int n4) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n4) dst[i] = src[i];
}
int hxa_copy_f32_launch(const float *src, float *dst, int n, hipStream_t st) {
  if (n % 4) return HXA_E_ARG;
  hxa_launch(copy_f4_kernel, dim3((n / 4 + 255) / 256), dim3(256), 0, st, (const float4_t *)src, (float4_t *)dst, n / 4);
  return LAUNCH_OK();
}
int hxa_sinusoid_launch(const float *t, int n, int dim, float *out, hipStream_t st) {
  hxa_launch(sinusoid_kernel, dim3(nblk((long)n * dim / 2)), dim3(256), 0, st, t, n, dim, out);
  return LAUNCH_OK();
}
int hxa_quantize_launch(const float *W, int N, int K, int fmt, void *q, hxa_h *s, hipStream_t st) {
  const int kt = (fmt & HXA_W_KTILED) ? 1 : 0;
  fmt &= ~HXA_W_KTILED;
  if (K % 32 || (fmt != HXA_W_Q8 && fmt != HXA_W_Q4)) return HXA_E_ARG;
  hxa_launch(quantize_kernel, dim3(nblk((long)N * (K / 32))), dim3(256), 0, st, W, N, K, fmt, kt, q, s);
  return LAUNCH_OK();
}
