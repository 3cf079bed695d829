/* hxo — CPU oracle for the HexAnima DiT block runner. TEST INFRASTRUCTURE ONLY (see hxo.h).
 *
 * Block semantics restated (Anima structure, hexagon/mega/blk.c:149-176):
 *   site s in {0 self-attn, 1 cross-attn, 2 MLP}; shift = mod[3s], scale = mod[3s+1], gate = mod[3s+2] (blk.c:150)
 *   h   = f16(LN(x) * (1 + scale) + shift)                         kern.c:38-65   (var = E[x^2] - mu^2, eps 1e-6)
 *   s0: q,k,v = f16(h Wq,k,v); q,k = f16(RoPE(RMS(.) * gain))       blk.c:158-160, kern.c:163-197
 *       o = attention(q, k, v); x += gate * f16(o Wo)               blk.c:161-162, kern.c:320-328
 *   s1: q = f16(h Wcq); ck,cv = f16(ctx Wck,cv); q,ck = f16(RMS(.) * gain)   blk.c:164-167
 *       o = attention(q, ck, cv); x += gate * f16(o Wco)             blk.c:168-169
 *   s2: mid = f16(GELU(f16(h W1)))                                   blk.c:171, gemm2.c:74
 *       x += gate * (f16(mid[:, :F/2] W2[:F/2]) + f16(mid[:, F/2:] W2[F/2:]))   blk.c:172-174, kern.c:330-339
 * Arithmetic between storage points is carried in double (the reference uses Hexagon qf32, i.e. ~fp32); the
 * storage points themselves are rounded exactly as the reference stores them.
 */
#include "hxo.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------------ */
/* fp16                                                                                              */
/* ------------------------------------------------------------------------------------------------ */
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t hxo_f2h(float f) {
  uint32_t x = fbits(f);
  const uint32_t s = (x >> 16) & 0x8000u;
  x &= 0x7fffffffu;
  if (x > 0x7f800000u) return (uint16_t)(s | 0x7e00u);     /* NaN */
  if (x >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);    /* >= 65520 rounds to inf */
  if (x >= 0x38800000u) {                                  /* normal half */
    const uint32_t mant = x & 0x7fffffu, e = (x >> 23) - 112u;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(s | h);
  }
  if (x < 0x33000000u) return (uint16_t)s;                 /* < 2^-25 (and the tie at 2^-25) -> 0 */
  const uint32_t e = x >> 23, mant = (x & 0x7fffffu) | 0x800000u;
  const int sh = 126 - (int)e;                             /* 14..24 */
  uint32_t h = mant >> sh;
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
  if (rem > half || (rem == half && (h & 1u))) h++;
  return (uint16_t)(s | h);
}

float hxo_h2f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) { const float v = (float)m * (1.0f / 16777216.0f); return s ? -v : v; }
  if (e == 31) return bitsf(s | 0x7f800000u | (m << 13));
  return bitsf(s | ((e + 112u) << 23) | (m << 13));
}

/* double -> fp16 with a single rounding (the exact value of a double is rounded directly) */
static uint16_t d2h(double d) {
  if (d != d) return 0x7e00u;
  const uint16_t s = signbit(d) ? 0x8000u : 0;
  double a = fabs(d);
  if (a >= 65520.0) return s | 0x7c00u;
  if (a < 6.103515625e-05) {                               /* subnormal range: units of 2^-24 */
    double u = a * 16777216.0, f = floor(u), r = u - f;
    uint32_t h = (uint32_t)f;
    if (r > 0.5 || (r == 0.5 && (h & 1u))) h++;
    return s | (uint16_t)h;                                /* h == 1024 is the smallest normal: bit pattern matches */
  }
  int e;
  double m = frexp(a, &e);                                 /* a = m 2^e, m in [0.5,1) */
  double u = m * 2048.0, f = floor(u), r = u - f;          /* 11 significant bits */
  uint32_t q = (uint32_t)f;
  if (r > 0.5 || (r == 0.5 && (q & 1u))) q++;
  if (q == 2048u) { q = 1024u; e++; }
  const int he = e - 1 + 15;                               /* biased exponent of 1.xxx 2^(e-1) */
  if (he >= 31) return s | 0x7c00u;
  return (uint16_t)(s | ((uint32_t)he << 10) | (q - 1024u));
}

static float g_h2f[65536];
static int g_tab_ready;
static void tab_init(void) {
  if (g_tab_ready) return;
  for (int i = 0; i < 65536; i++) g_h2f[i] = hxo_h2f((uint16_t)i);
  g_tab_ready = 1;
}
__attribute__((constructor)) static void hxo_ctor(void) { tab_init(); }
#define H2F(h) (g_h2f[(uint16_t)(h)])

void hxo_f2h_n(const float *src, uint16_t *dst, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; i++) dst[i] = hxo_f2h(src[i]);
}
void hxo_h2f_n(const uint16_t *src, float *dst, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; i++) dst[i] = H2F(src[i]);
}
int hxo_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
  return omp_get_max_threads();
#else
  (void)n;
  return 1;
#endif
}

/* ------------------------------------------------------------------------------------------------ */
/* GEMM (packed panels, double accumulation)                                                        */
/* ------------------------------------------------------------------------------------------------ */
typedef double v4d __attribute__((vector_size(32)));
#define MR 4
#define NR 8
#define KC 256
#define MC 96
#define NC 256

static void pack_a(const uint16_t *A, long lda, int m0, int mc, int k0, int kc, double *pa) {
  for (int i = 0; i < MC; i += MR)
    for (int r = 0; r < MR; r++) {
      const int m = i + r;
      double *dst = pa + (size_t)(i / MR) * KC * MR + r;
      if (m < mc) {
        const uint16_t *src = A + (long)(m0 + m) * lda + k0;
        for (int k = 0; k < kc; k++) dst[(size_t)k * MR] = H2F(src[k]);
      } else {
        for (int k = 0; k < kc; k++) dst[(size_t)k * MR] = 0.0;
      }
    }
}
static void pack_w(const uint16_t *W, long ldw, int n0, int nc, int k0, int kc, double *pb) {
  for (int j = 0; j < NC; j += NR)
    for (int c = 0; c < NR; c++) {
      const int n = j + c;
      double *dst = pb + (size_t)(j / NR) * KC * NR + c;
      if (n < nc) {
        const uint16_t *src = W + (long)(n0 + n) * ldw + k0;
        for (int k = 0; k < kc; k++) dst[(size_t)k * NR] = H2F(src[k]);
      } else {
        for (int k = 0; k < kc; k++) dst[(size_t)k * NR] = 0.0;
      }
    }
}
static void ukernel(int kc, const double *pa, const double *pb, double *c, int ldc) {
  v4d c00 = {0}, c01 = {0}, c10 = {0}, c11 = {0}, c20 = {0}, c21 = {0}, c30 = {0}, c31 = {0};
  for (int k = 0; k < kc; k++) {
    v4d b0, b1;
    memcpy(&b0, pb + (size_t)k * NR, 32);
    memcpy(&b1, pb + (size_t)k * NR + 4, 32);
    const double *a = pa + (size_t)k * MR;
    c00 += a[0] * b0; c01 += a[0] * b1;
    c10 += a[1] * b0; c11 += a[1] * b1;
    c20 += a[2] * b0; c21 += a[2] * b1;
    c30 += a[3] * b0; c31 += a[3] * b1;
  }
  v4d acc[8] = {c00, c01, c10, c11, c20, c21, c30, c31};
  for (int r = 0; r < MR; r++)
    for (int h = 0; h < 2; h++) {
      double *dst = c + (size_t)r * ldc + h * 4;
      for (int e = 0; e < 4; e++) dst[e] += acc[r * 2 + h][e];
    }
}

void hxo_gemm(const uint16_t *A, long lda, const uint16_t *W, long ldw, float *C, long ldc, int M, int N, int K) {
  const int nmb = (M + MC - 1) / MC, nnb = (N + NC - 1) / NC;
#pragma omp parallel
  {
    double *pa = (double *)aligned_alloc(64, sizeof(double) * MC * KC);
    double *pb = (double *)aligned_alloc(64, sizeof(double) * NC * KC);
    double *cb = (double *)aligned_alloc(64, sizeof(double) * MC * NC);
#pragma omp for collapse(2) schedule(dynamic)
    for (int ib = 0; ib < nmb; ib++)
      for (int jb = 0; jb < nnb; jb++) {
        const int m0 = ib * MC, mc = M - m0 < MC ? M - m0 : MC, n0 = jb * NC, nc = N - n0 < NC ? N - n0 : NC;
        memset(cb, 0, sizeof(double) * MC * NC);
        for (int k0 = 0; k0 < K; k0 += KC) {
          const int kc = K - k0 < KC ? K - k0 : KC;
          pack_a(A, lda, m0, mc, k0, kc, pa);
          pack_w(W, ldw, n0, nc, k0, kc, pb);
          for (int jr = 0; jr < nc; jr += NR)
            for (int ir = 0; ir < mc; ir += MR)
              ukernel(kc, pa + (size_t)(ir / MR) * KC * MR, pb + (size_t)(jr / NR) * KC * NR, cb + (size_t)ir * NC + jr, NC);
        }
        for (int i = 0; i < mc; i++)
          for (int j = 0; j < nc; j++) C[(long)(m0 + i) * ldc + n0 + j] = (float)cb[(size_t)i * NC + j];
      }
    free(pa); free(pb); free(cb);
  }
}

void hxo_gemm_naive(const uint16_t *A, long lda, const uint16_t *W, long ldw, float *C, long ldc, int M, int N, int K) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double acc = 0.0;
      for (int k = 0; k < K; k++) acc += (double)H2F(A[(long)m * lda + k]) * (double)H2F(W[(long)n * ldw + k]);
      C[(long)m * ldc + n] = (float)acc;
    }
}

void hxo_linear_f32(const float *x, long ldx, const uint16_t *W, long ldw, float *y, long ldy, int M, int N, int K) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; m++)
    for (int n = 0; n < N; n++) {
      double acc = 0.0;
      const float *xr = x + (long)m * ldx;
      const uint16_t *wr = W + (long)n * ldw;
      for (int k = 0; k < K; k++) acc += (double)xr[k] * (double)H2F(wr[k]);
      y[(long)m * ldy + n] = (float)acc;
    }
}

/* round a float GEMM result buffer to fp16 storage */
static void f2h_rows(const float *src, long lds, uint16_t *dst, long ldd, int R, int C) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < R; r++)
    for (int c = 0; c < C; c++) dst[(long)r * ldd + c] = hxo_f2h(src[(long)r * lds + c]);
}

/* ------------------------------------------------------------------------------------------------ */
/* norms                                                                                             */
/* ------------------------------------------------------------------------------------------------ */
void hxo_lnmod(const float *x, int T, int D, const float *shift, const float *scale, float eps, uint16_t *h) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) {
    const float *xr = x + (long)t * D;
    double s = 0.0, q = 0.0;
    for (int c = 0; c < D; c++) { s += xr[c]; q += (double)xr[c] * xr[c]; }
    const double mu = s / D, var = q / D - mu * mu, r = 1.0 / sqrt(var + (double)eps);
    for (int c = 0; c < D; c++) h[(long)t * D + c] = d2h(((double)xr[c] - mu) * r * (1.0 + (double)scale[c]) + shift[c]);
  }
}

void hxo_rmsmod(const float *x, int T, int D, const float *w, const float *shift, const float *scale, float eps, uint16_t *h) {
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) {
    const float *xr = x + (long)t * D;
    double q = 0.0;
    for (int c = 0; c < D; c++) q += (double)xr[c] * xr[c];
    const double r = 1.0 / sqrt(q / D + (double)eps);
    for (int c = 0; c < D; c++) {
      const float m = (1.0f + scale[c]) * w[c]; /* k_rms_prep: M = (1 + scale) * w, formed in fp32 */
      h[(long)t * D + c] = d2h((double)xr[c] * r * (double)m + shift[c]);
    }
  }
}

void hxo_rmsrope(uint16_t *q, int T, long ldq, int H, const float *gain, const float *cosT, const float *sinT, int rope) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int t = 0; t < T; t++)
    for (int hd = 0; hd < H; hd++) {
      uint16_t *p = q + (long)t * ldq + (long)hd * 128;
      double u[128], ss = 0.0;
      for (int d = 0; d < 128; d++) { u[d] = H2F(p[d]); ss += u[d] * u[d]; }
      const double r = 1.0 / sqrt(ss / 128.0 + 1e-6);
      for (int d = 0; d < 128; d++) u[d] = u[d] * r * (double)gain[d];
      if (rope) {
        for (int d = 0; d < 64; d++) {
          const double a = u[d], b = u[d + 64], c = cosT[(long)t * 64 + d], s = sinT[(long)t * 64 + d];
          u[d] = a * c - b * s;
          u[d + 64] = a * s + b * c;
        }
      }
      for (int d = 0; d < 128; d++) p[d] = d2h(u[d]);
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* attention                                                                                         */
/* ------------------------------------------------------------------------------------------------ */
#define ATT_RB 256
void hxo_attention(const uint16_t *q, long ldq, const uint16_t *k, long ldk, const uint16_t *v, long ldv, uint16_t *o,
                   long ldo, int T, int NKV, int nvalid, int H, int mode) {
  float *S = (float *)malloc(sizeof(float) * (size_t)ATT_RB * NKV);
  uint16_t *P = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)ATT_RB * NKV);
  double *Pd = mode ? (double *)malloc(sizeof(double) * (size_t)ATT_RB * NKV) : NULL;
  uint16_t *VT = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)128 * NKV);
  float *Ou = (float *)malloc(sizeof(float) * (size_t)ATT_RB * 128);
  uint16_t *L = (uint16_t *)malloc(sizeof(uint16_t) * ATT_RB);
  double *Ld = (double *)malloc(sizeof(double) * ATT_RB);
  for (int hd = 0; hd < H; hd++) {
    for (int j = 0; j < NKV; j++)
      for (int d = 0; d < 128; d++) VT[(size_t)d * NKV + j] = v[(long)j * ldv + (long)hd * 128 + d];
    for (int r0 = 0; r0 < T; r0 += ATT_RB) {
      const int rb = T - r0 < ATT_RB ? T - r0 : ATT_RB;
      hxo_gemm(q + (long)r0 * ldq + (long)hd * 128, ldq, k + (long)hd * 128, ldk, S, NKV, rb, NKV, 128);
      if (mode == 0) {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < rb; i++) {
          const float *Si = S + (size_t)i * NKV;
          uint16_t *Pi = P + (size_t)i * NKV;
          /* S = f16(q.k); padded keys hold -65504 (0xFBFF, moss kern.c:268) */
          double m = -65504.0;
          for (int j = 0; j < NKV; j++) {
            const uint16_t sh = j < nvalid ? hxo_f2h(Si[j]) : 0xFBFFu;
            Pi[j] = sh;
            const double sv = H2F(sh);
            if (sv > m) m = sv;
          }
          /* P = table exp(-|f16(S - m)|) (kern.c:235-243, 272-273); l = f16(sum P) (the ones column of blk.c:59) */
          double l = 0.0;
          for (int j = 0; j < NKV; j++) {
            const uint16_t dh = d2h((double)H2F(Pi[j]) - m);
            const uint16_t mag = dh & 0x7fffu;
            const uint16_t p = mag >= 0x7c00u ? 0 : d2h(exp(-(double)H2F(mag)));
            Pi[j] = p;
            l += H2F(p);
          }
          L[i] = d2h(l);
        }
        /* O = f16(P V) then f16(O * (1/l)) (blk.c:78-83, kern.c:285-295) */
        hxo_gemm(P, NKV, VT, NKV, Ou, 128, rb, 128, NKV);
#pragma omp parallel for schedule(static)
        for (int i = 0; i < rb; i++) {
          const double rl = 1.0 / (double)H2F(L[i]);
          for (int d = 0; d < 128; d++)
            o[(long)(r0 + i) * ldo + (long)hd * 128 + d] = d2h((double)H2F(hxo_f2h(Ou[(size_t)i * 128 + d])) * rl);
        }
      } else {
#pragma omp parallel for schedule(static)
        for (int i = 0; i < rb; i++) {
          const float *Si = S + (size_t)i * NKV;
          double *Pi = Pd + (size_t)i * NKV, m = -1e300, l = 0.0;
          for (int j = 0; j < nvalid; j++) if (Si[j] > m) m = Si[j];
          for (int j = 0; j < NKV; j++) { Pi[j] = j < nvalid ? exp((double)Si[j] - m) : 0.0; l += Pi[j]; }
          Ld[i] = l;
          double acc[128];
          for (int d = 0; d < 128; d++) acc[d] = 0.0;
          for (int j = 0; j < nvalid; j++) {
            const double p = Pi[j];
            const uint16_t *vr = VT + j; /* VT[d][j] */
            for (int d = 0; d < 128; d++) acc[d] += p * (double)H2F(vr[(size_t)d * NKV]);
          }
          for (int d = 0; d < 128; d++) o[(long)(r0 + i) * ldo + (long)hd * 128 + d] = d2h(acc[d] / Ld[i]);
        }
      }
    }
  }
  free(S); free(P); free(Pd); free(VT); free(Ou); free(L); free(Ld);
}

/* ------------------------------------------------------------------------------------------------ */
/* activations                                                                                       */
/* ------------------------------------------------------------------------------------------------ */
uint16_t hxo_gelu_erf_h(uint16_t t) {
  const uint16_t mag = t & 0x7fffu;
  /* t2 table: fp16(|x| * 0.5 * erfc(|x|/sqrt 2)), 0 for inf/NaN magnitudes (kern.c:238-240) */
  const double a = H2F(mag);
  const uint16_t t2 = mag >= 0x7c00u ? 0 : d2h(a * 0.5 * erfc(a / sqrt(2.0)));
  const double xv = H2F(t), pos = xv > 0.0 ? xv : 0.0; /* vmax(x, 0) */
  return d2h(pos - (double)H2F(t2));
}
uint16_t hxo_gelu_tanh_h(uint16_t t) {
  const double x = H2F(t);
  return d2h(0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))));
}
uint16_t hxo_situ_h(uint16_t up, uint16_t gate) {
  /* three fp16 tables indexed by magnitude (moss kern.c:376-386): 25 tanh(a/25); 4 tanh(a/4) sigmoid(a); 4 tanh(a/4) sigmoid(-a) */
  const uint16_t mu = up & 0x7fffu, mg = gate & 0x7fffu;
  const double au = H2F(mu), ag = H2F(mg);
  const uint16_t t25 = mu >= 0x7c00u ? 0 : d2h(25.0 * tanh(au / 25.0));
  const uint16_t gp = mg >= 0x7c00u ? 0 : d2h(4.0 * tanh(ag / 4.0) / (1.0 + exp(-ag)));
  const uint16_t gn = mg >= 0x7c00u ? 0 : d2h(4.0 * tanh(ag / 4.0) / (1.0 + exp(ag)));
  const uint16_t tu = t25 | (up & 0x8000u);                    /* odd: sign of u */
  const uint16_t gs = (gate & 0x8000u) ? (uint16_t)(gn | 0x8000u) : gp; /* g < 0: -Gn(|g|) */
  return d2h((double)H2F(tu) * (double)H2F(gs));
}
void hxo_gelu_n(uint16_t *t, size_t n, int mode) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; i++) t[i] = mode ? hxo_gelu_tanh_h(t[i]) : hxo_gelu_erf_h(t[i]);
}
void hxo_situ_n(const uint16_t *up, const uint16_t *gate, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; i++) out[i] = hxo_situ_h(up[i], gate[i]);
}

/* ------------------------------------------------------------------------------------------------ */
/* residuals                                                                                         */
/* ------------------------------------------------------------------------------------------------ */
void hxo_resadd(float *x, int T, int D, const uint16_t *t, const float *gate) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)T * D; i++) x[i] = (float)((double)x[i] + (double)gate[i % D] * (double)H2F(t[i]));
}
void hxo_resadd2(float *x, int T, int D, const uint16_t *t1, const uint16_t *t2, const float *gate) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)T * D; i++) {
    const float s = H2F(t1[i]) + H2F(t2[i]); /* qf32 sum of the two fp16 partials, converted to sf */
    x[i] = (float)((double)x[i] + (double)gate[i % D] * (double)s);
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* quantisation                                                                                      */
/* ------------------------------------------------------------------------------------------------ */
static uint16_t q_scale(float amax, float div) {
  float s = amax / div;
  if (s < 6.2e-5f) s = 6.2e-5f;
  return hxo_f2h(s);
}
void hxo_q8_quantize(const float *W, int N, int K, int8_t *q, uint16_t *s) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++)
    for (int g = 0; g < K / 32; g++) {
      float a[32], amax = 0.0f;
      for (int i = 0; i < 32; i++) { a[i] = H2F(hxo_f2h(W[(long)n * K + g * 32 + i])); if (fabsf(a[i]) > amax) amax = fabsf(a[i]); }
      const uint16_t sh = q_scale(amax, 127.0f);
      const float sf = H2F(sh);
      s[(long)g * N + n] = sh;
      for (int i = 0; i < 32; i++) {
        float r = rintf(a[i] / sf);
        r = r < -127.0f ? -127.0f : r > 127.0f ? 127.0f : r;
        q[(long)n * K + g * 32 + i] = (int8_t)r;
      }
    }
}
void hxo_q8_dequant(const int8_t *q, const uint16_t *s, int N, int K, uint16_t *w16) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) w16[(long)n * K + k] = hxo_f2h((float)q[(long)n * K + k] * H2F(s[(long)(k / 32) * N + n]));
}
static inline int q4_shift(int k) { const int j = k & 7; return (j & 1) ? 16 + 4 * (j >> 1) : 4 * (j >> 1); }
void hxo_q4_quantize(const float *W, int N, int K, uint8_t *q, uint16_t *s) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    uint32_t *wq = (uint32_t *)(q + (long)n * (K / 2));
    for (int i = 0; i < K / 8; i++) wq[i] = 0;
    for (int g = 0; g < K / 32; g++) {
      float a[32], amax = 0.0f;
      for (int i = 0; i < 32; i++) { a[i] = H2F(hxo_f2h(W[(long)n * K + g * 32 + i])); if (fabsf(a[i]) > amax) amax = fabsf(a[i]); }
      const uint16_t sh = q_scale(amax, 7.0f);
      const float sf = H2F(sh);
      s[(long)g * N + n] = sh;
      for (int i = 0; i < 32; i++) {
        float r = rintf(a[i] / sf);
        r = r < -8.0f ? -8.0f : r > 7.0f ? 7.0f : r;
        const int k = g * 32 + i;
        wq[k / 8] |= (uint32_t)((int)r + 8) << q4_shift(k);
      }
    }
  }
}
void hxo_q4_dequant(const uint8_t *q, const uint16_t *s, const uint16_t *z, int N, int K, uint16_t *w16) {
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; n++) {
    const uint32_t *wq = (const uint32_t *)(q + (long)n * (K / 2));
    for (int k = 0; k < K; k++) {
      const int nib = (int)((wq[k / 8] >> q4_shift(k)) & 15u);
      const double sc = H2F(s[(long)(k / 32) * N + n]);
      const double v = z ? (double)nib * sc + (double)H2F(z[(long)(k / 32) * N + n]) : (double)(nib - 8) * sc;
      w16[(long)n * K + k] = d2h(v);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* reference tile formats                                                                            */
/* ------------------------------------------------------------------------------------------------ */
static inline size_t hw_idx(int r, int c) { return (size_t)(r >> 1) * 64 + (size_t)c * 2 + (size_t)(r & 1); }

void hxo_h16_tile(const uint16_t *a, int R, int C, uint16_t *tiles) {
  const int ncb = C / 32;
  for (int r = 0; r < R; r++)
    for (int c = 0; c < C; c++) tiles[((size_t)(r / 32) * ncb + c / 32) * 1024 + hw_idx(r & 31, c & 31)] = a[(size_t)r * C + c];
}
void hxo_h16_untile(const uint16_t *tiles, int R, int C, uint16_t *a) {
  const int ncb = C / 32;
  for (int r = 0; r < R; r++)
    for (int c = 0; c < C; c++) a[(size_t)r * C + c] = tiles[((size_t)(r / 32) * ncb + c / 32) * 1024 + hw_idx(r & 31, c & 31)];
}
void hxo_x32_tile(const float *a, int R, int C, float *tiles) {
  const int ncb = C / 32;
  for (int r = 0; r < R; r++)
    for (int c = 0; c < C; c++) tiles[((size_t)(r / 32) * ncb + c / 32) * 1024 + (size_t)(r & 31) * 32 + (c & 31)] = a[(size_t)r * C + c];
}
void hxo_x32_untile(const float *tiles, int R, int C, float *a) {
  const int ncb = C / 32;
  for (int r = 0; r < R; r++)
    for (int c = 0; c < C; c++) a[(size_t)r * C + c] = tiles[((size_t)(r / 32) * ncb + c / 32) * 1024 + (size_t)(r & 31) * 32 + (c & 31)];
}
/* weight matrix M[K][N] = W[N][K]^T tiled [n block][k block], tile rows = k (export_all.py:7-8) */
void hxo_wt16_pack(const uint16_t *wNK, int N, int K, uint16_t *tiles) {
  const int kb = K / 32;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) tiles[((size_t)(n / 32) * kb + k / 32) * 1024 + hw_idx(k & 31, n & 31)] = wNK[(size_t)n * K + k];
}
void hxo_wt16_unpack(const uint16_t *tiles, int N, int K, uint16_t *wNK) {
  const int kb = K / 32;
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) wNK[(size_t)n * K + k] = tiles[((size_t)(n / 32) * kb + k / 32) * 1024 + hw_idx(k & 31, n & 31)];
}
void hxo_q8rec_pack(const uint16_t *wNK, int N, int K, uint8_t *rec, int floor_mode) {
  const int kb = K / 32, nb = N / 32;
#pragma omp parallel for schedule(static)
  for (int jb = 0; jb < nb; jb++)
    for (int ib = 0; ib < kb; ib++) {
      uint8_t *R = rec + ((size_t)jb * kb + ib) * 1152;
      uint16_t *sv = (uint16_t *)R;
      for (int c = 0; c < 32; c++) {
        float amax = 0.0f;
        for (int r = 0; r < 32; r++) { const float a = fabsf(H2F(wNK[(size_t)(jb * 32 + c) * K + ib * 32 + r])); if (a > amax) amax = a; }
        float s = amax / 127.0f;
        if (floor_mode) { if (s < 6.2e-5f) s = 6.2e-5f; }
        else if (s == 0.0f) s = 1.0f;
        const uint16_t sh = hxo_f2h(s);
        const float sf = H2F(sh);
        sv[2 * c] = sv[2 * c + 1] = sh;
        for (int r = 0; r < 32; r++) {
          float q = rintf(H2F(wNK[(size_t)(jb * 32 + c) * K + ib * 32 + r]) / sf);
          q = q < -127.0f ? -127.0f : q > 127.0f ? 127.0f : q;
          R[128 + hw_idx(r, c)] = (uint8_t)((int)q + 128);
        }
      }
    }
}
void hxo_q8rec_unpack(const uint8_t *rec, int N, int K, uint16_t *wNK) {
  const int kb = K / 32, nb = N / 32;
#pragma omp parallel for schedule(static)
  for (int jb = 0; jb < nb; jb++)
    for (int ib = 0; ib < kb; ib++) {
      const uint8_t *R = rec + ((size_t)jb * kb + ib) * 1152;
      const uint16_t *sv = (const uint16_t *)R;
      for (int c = 0; c < 32; c++)
        for (int r = 0; r < 32; r++) {
          const int q = (int)R[128 + hw_idx(r, c)] - 128;
          wNK[(size_t)(jb * 32 + c) * K + ib * 32 + r] = hxo_f2h((float)q * H2F(sv[2 * c]));
        }
    }
}
void hxo_q4arec_unpack(const uint8_t *rec, int N, int K, uint16_t *wNK) {
  const int kb = K / 32, nb = N / 32;
  for (int jb = 0; jb < nb; jb++)
    for (int ib = 0; ib < kb; ib++) {
      const uint8_t *R = rec + ((size_t)jb * kb + ib) * 768;
      const uint16_t *sv = (const uint16_t *)R, *mv = (const uint16_t *)(R + 128);
      const uint8_t *nb8 = R + 256;
      for (int hw = 0; hw < 1024; hw++) {
        const int m = hw / 256, b = hw % 256;
        const int nib = b < 128 ? (nb8[m * 128 + b] & 15) : (nb8[m * 128 + b - 128] >> 4);
        const int r = (hw / 64) * 2 + (hw & 1), c = (hw % 64) / 2;
        wNK[(size_t)(jb * 32 + c) * K + ib * 32 + r] = d2h((double)nib * H2F(sv[2 * c]) + H2F(mv[2 * c]));
      }
    }
}

/* ------------------------------------------------------------------------------------------------ */
/* RoPE tables                                                                                       */
/* ------------------------------------------------------------------------------------------------ */
void hxo_rope_anima(int gh, int gw, float *cosT, float *sinT) {
  const int dim_h = 128 / 6 * 2, dim_t = 128 - 2 * dim_h, nt = dim_t / 2, nh = dim_h / 2;
  double fh[64];
  for (int i = 0; i < nh; i++) fh[i] = 1.0 / pow(10000.0, (2.0 * i) / dim_h);
  for (int tk = 0; tk < gh * gw; tk++) {
    const int hh = tk / gw, ww = tk % gw;
    for (int d = 0; d < 64; d++) {
      const double ang = d < nt ? 0.0 : d < nt + nh ? hh * fh[d - nt] : ww * fh[d - nt - nh];
      cosT[(size_t)tk * 64 + d] = (float)cos(ang);
      sinT[(size_t)tk * 64 + d] = (float)sin(ang);
    }
  }
}
void hxo_rope_moss(int H, int W, int ntxt, const float *bands16, float *cosT, float *sinT) {
  hxo_rope_moss_scaled(H, W, ntxt, bands16, 1.0, cosT, sinT);
}
/* moss/mossrun/mossrun.cpp:190-201 with its position scale: image positions (row, column) times `scale` (the
 * low-res steps' MOSS_LOWSCALE, 2 by default: mossrun.cpp:288, :313) */
void hxo_rope_moss_scaled(int H, int W, int ntxt, const float *bands16, double scale, float *cosT, float *sinT) {
  const int nimg = H * W;
  for (int tk = 0; tk < nimg + ntxt; tk++) {
    double pos[4];
    if (tk < nimg) {
      pos[0] = 0; pos[1] = ntxt; pos[2] = ((tk / W) - (H - 1) / 2.0) * scale; pos[3] = ((tk % W) - (W - 1) / 2.0) * scale;
    }
    else { pos[0] = 0; pos[1] = tk - nimg; pos[2] = 0; pos[3] = 0; }
    for (int d = 0; d < 64; d++) {
      const double ph = pos[d / 16] * (double)bands16[d % 16];
      cosT[(size_t)tk * 64 + d] = (float)cos(ph);
      sinT[(size_t)tk * 64 + d] = (float)sin(ph);
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* low-res first steps (no fp contraction: the expressions are rounded as written)                  */
/* ------------------------------------------------------------------------------------------------ */
/* phone/animad.cpp:429-437: the latent of a step run at 1/f resolution, [C][H/f][W/f] from the full-res noise of the
 * first step and the previous full-res clean estimate: x_low = (1 - t) mean_fxf(dhat) + t sum_fxf(noise) / f (the
 * noise mean times f keeps unit variance), both sums in double in (a, b) order */
__attribute__((optimize("fp-contract=off")))
void hxo_lowres_pool(const float *nfull, const float *dhat, int C, int H, int W, int f, float t, float *xlow) {
  const int Hl = H / f, Wl = W / f;
  for (int c = 0; c < C; c++)
    for (int y = 0; y < Hl; y++)
      for (int x = 0; x < Wl; x++) {
        double sn = 0, sd = 0;
        for (int a = 0; a < f; a++)
          for (int b = 0; b < f; b++) {
            const size_t i = ((size_t)c * H + y * f + a) * W + x * f + b;
            sn += nfull[i];
            sd += dhat[i];
          }
        xlow[((size_t)c * Hl + y) * Wl + x] = (float)((1 - t) * sd / (f * f) + t * sn / f);  /* 1 - t in float */
      }
}
/* phone/animad.cpp:486-503: from the low-res velocity, the low-res clean estimate dl = x_low - t v_low, bilinearly
 * upsampled with half-pixel centres (clamped at the edges) into dhat, the full-res state it implies at tn,
 * x_next = (1 - tn) dhat + tn noise, and the velocity that lands sd.cpp's Euler step there, (x_full - x_next) / (t - tn)
 * (0 when t - tn <= 1e-6). tn and t - tn in double as in the reference. */
__attribute__((optimize("fp-contract=off")))
void hxo_lowres_velocity(const float *xlow, const float *vlow, const float *xfull, const float *nfull, int C, int H, int W,
                         int f, float t, double tn, float *dhat, float *vf) {
  const int Hl = H / f, Wl = W / f;
  const double dt = t - tn;
  float *dl = (float *)malloc(sizeof(float) * (size_t)C * Hl * Wl);
  for (size_t i = 0; i < (size_t)C * Hl * Wl; i++) dl[i] = xlow[i] - t * vlow[i];
  for (int c = 0; c < C; c++)
    for (int y = 0; y < H; y++) {
      const float fy = (y + 0.5f) / f - 0.5f;
      int y0 = (int)floorf(fy);
      const float wy = fy - y0;
      const int y1 = y0 + 1 < 0 ? 0 : (y0 + 1 > Hl - 1 ? Hl - 1 : y0 + 1);
      y0 = y0 < 0 ? 0 : (y0 > Hl - 1 ? Hl - 1 : y0);
      for (int x = 0; x < W; x++) {
        const float fx = (x + 0.5f) / f - 0.5f;
        int x0 = (int)floorf(fx);
        const float wx = fx - x0;
        const int x1 = x0 + 1 < 0 ? 0 : (x0 + 1 > Wl - 1 ? Wl - 1 : x0 + 1);
        x0 = x0 < 0 ? 0 : (x0 > Wl - 1 ? Wl - 1 : x0);
        const float *b = dl + (size_t)c * Hl * Wl;
        const float up = (1 - wy) * ((1 - wx) * b[y0 * Wl + x0] + wx * b[y0 * Wl + x1]) +
                         wy * ((1 - wx) * b[y1 * Wl + x0] + wx * b[y1 * Wl + x1]);
        const size_t i = ((size_t)c * H + y) * W + x;
        dhat[i] = up;
        const float xnext = (float)(1 - tn) * up + (float)tn * nfull[i];
        vf[i] = dt > 1e-6 ? (xfull[i] - xnext) / (float)dt : 0.f;
      }
    }
  free(dl);
}
/* moss/mossrun/mossrun.cpp:291: the low-res noise of the MOSS steps, 2 x the mean of each 2x2 block of the token grid
 * (unit variance), on token rows: z [H*W][C4] -> zl [(H/2)*(W/2)][C4] */
__attribute__((optimize("fp-contract=off")))
void hxo_moss_pool2(const float *z, int H, int W, int C4, float *zl) {
  const int Wl = W / 2;
  for (int i = 0; i < H / 2; i++)
    for (int j = 0; j < Wl; j++)
      for (int c = 0; c < C4; c++) {
        const float p0 = z[((size_t)(2 * i) * W + 2 * j) * C4 + c], p1 = z[((size_t)(2 * i) * W + 2 * j + 1) * C4 + c];
        const float p2 = z[((size_t)(2 * i + 1) * W + 2 * j) * C4 + c], p3 = z[((size_t)(2 * i + 1) * W + 2 * j + 1) * C4 + c];
        zl[((size_t)i * Wl + j) * C4 + c] = 0.5f * (p0 + p1 + p2 + p3);
      }
}
/* moss/mossrun/mossrun.cpp:278-282 upsample2: bilinear 2x with half-pixel centres, clamped, on token rows
 * [h*w][C4] -> [(2h)*(2w)][C4] (the low-res clean estimate seeding the first full-res step, :311) */
__attribute__((optimize("fp-contract=off")))
void hxo_upsample2_rows(const float *src, int h, int w, int C4, float *dst) {
  for (int y = 0; y < 2 * h; y++) {
    const float fy = (y + 0.5f) / 2 - 0.5f;
    const int y0 = (int)floorf(fy);
    const float ty = fy - y0;
    const int ya = y0 < 0 ? 0 : (y0 > h - 1 ? h - 1 : y0), yb = y0 + 1 < 0 ? 0 : (y0 + 1 > h - 1 ? h - 1 : y0 + 1);
    for (int x = 0; x < 2 * w; x++) {
      const float fx = (x + 0.5f) / 2 - 0.5f;
      const int x0 = (int)floorf(fx);
      const float tx = fx - x0;
      const int xa = x0 < 0 ? 0 : (x0 > w - 1 ? w - 1 : x0), xb = x0 + 1 < 0 ? 0 : (x0 + 1 > w - 1 ? w - 1 : x0 + 1);
      for (int c = 0; c < C4; c++) {
        const float a = src[((size_t)ya * w + xa) * C4 + c], b = src[((size_t)ya * w + xb) * C4 + c];
        const float cc = src[((size_t)yb * w + xa) * C4 + c], d = src[((size_t)yb * w + xb) * C4 + c];
        dst[((size_t)y * 2 * w + x) * C4 + c] = (1 - ty) * ((1 - tx) * a + tx * b) + ty * ((1 - tx) * cc + tx * d);
      }
    }
  }
}

/* ------------------------------------------------------------------------------------------------ */
/* blocks                                                                                            */
/* ------------------------------------------------------------------------------------------------ */
#define TICK() do { stage++; if (cfg->stop && stage >= cfg->stop) goto done; } while (0)

int hxo_anima_block(const hxo_anima_cfg *cfg, const hxo_anima_w *w, float *x, const uint16_t *ctx, const float *mod9,
                    const float *cosT, const float *sinT, hxo_anima_buf *b) {
  const int T = cfg->T, D = cfg->D, H = cfg->H, C = cfg->C, DC = cfg->DC, F = cfg->F;
  const long big = (long)T * (F > D ? F : D);
  float *tmp = (float *)malloc(sizeof(float) * (size_t)(big > (long)C * D ? big : (long)C * D));
  uint16_t *t2 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * D);
  int stage = 0;
  for (int site = 0; site < 3; site++) {
    const float *sh = mod9 + (size_t)(site * 3 + 0) * D, *sc = mod9 + (size_t)(site * 3 + 1) * D, *gt = mod9 + (size_t)(site * 3 + 2) * D;
    hxo_lnmod(x, T, D, sh, sc, 1e-6f, b->h);
    TICK();
    if (site == 0) {
      hxo_gemm(b->h, D, w->wq, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->q, D, T, D);
      hxo_gemm(b->h, D, w->wk, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->k, D, T, D);
      hxo_gemm(b->h, D, w->wv, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->v, D, T, D);
      TICK();
      hxo_rmsrope(b->q, T, D, H, w->gain, cosT, sinT, 1);
      hxo_rmsrope(b->k, T, D, H, w->gain + 128, cosT, sinT, 1);
      TICK();
      hxo_attention(b->q, D, b->k, D, b->v, D, b->o, D, T, T, T, H, cfg->attn_mode);
      TICK();
      hxo_gemm(b->o, D, w->wo, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->t, D, T, D);
      hxo_resadd(x, T, D, b->t, gt);
      TICK();
    } else if (site == 1) {
      hxo_gemm(b->h, D, w->wcq, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->q, D, T, D);
      hxo_gemm(ctx, DC, w->wck, DC, tmp, D, C, D, DC); f2h_rows(tmp, D, b->ck, D, C, D);
      hxo_gemm(ctx, DC, w->wcv, DC, tmp, D, C, D, DC); f2h_rows(tmp, D, b->cv, D, C, D);
      TICK();
      hxo_rmsrope(b->q, T, D, H, w->gain + 256, NULL, NULL, 0);
      hxo_rmsrope(b->ck, C, D, H, w->gain + 384, NULL, NULL, 0);
      TICK();
      hxo_attention(b->q, D, b->ck, D, b->cv, D, b->o, D, T, C, C, H, cfg->attn_mode);
      TICK();
      hxo_gemm(b->o, D, w->wco, D, tmp, D, T, D, D); f2h_rows(tmp, D, b->t, D, T, D);
      hxo_resadd(x, T, D, b->t, gt);
      TICK();
    } else {
      hxo_gemm(b->h, D, w->w1, D, tmp, F, T, F, D); f2h_rows(tmp, F, b->mid, F, T, F);
      hxo_gelu_n(b->mid, (size_t)T * F, cfg->gelu);
      TICK();
      const int F2 = F / 2;
      hxo_gemm(b->mid, F, w->w2, F, tmp, D, T, D, F2); f2h_rows(tmp, D, b->t, D, T, D);
      hxo_gemm(b->mid + F2, F, w->w2 + F2, F, tmp, D, T, D, F2); f2h_rows(tmp, D, t2, D, T, D);
      hxo_resadd2(x, T, D, b->t, t2, gt);
      TICK();
    }
  }
done:
  free(tmp); free(t2);
  return stage;
}

#define LORA_R 128
/* C[T][N] = [a | l] . W^T with a [T][Ka] (row stride lda), the LoRA columns l [T][r] (ldl; NULL: none) and
   W[N][Ka + r] (ldw): the K range of the reference's gemm_geo_t A2 tiles (moss/hexagon/mega/gemm2.c:125-133) */
static void gemm_cat(const uint16_t *a, long lda, int Ka, const uint16_t *l, long ldl, int r, const uint16_t *W, long ldw,
                     float *C, int T, int N, uint16_t *cat) {
  if (!l) { hxo_gemm(a, lda, W, ldw, C, N, T, N, Ka); return; }
#pragma omp parallel for schedule(static)
  for (int t = 0; t < T; t++) {
    memcpy(cat + (size_t)t * (Ka + r), a + (size_t)t * lda, sizeof(uint16_t) * Ka);
    memcpy(cat + (size_t)t * (Ka + r) + Ka, l + (size_t)t * ldl, sizeof(uint16_t) * r);
  }
  hxo_gemm(cat, Ka + r, W, ldw, C, N, T, N, Ka + r);
}

int hxo_moss_block(const hxo_moss_cfg *cfg, const hxo_moss_w *w, float *x, const float *mod6, const float *cosT,
                   const float *sinT, hxo_moss_buf *b) {
  const int T = cfg->T, D = cfg->D, H = cfg->H, F = cfg->F;
  const int lora = w->aqkv != NULL, R = lora ? LORA_R : 0;
  const float *sha = mod6, *sca = mod6 + D, *ga = mod6 + 2 * D, *shf = mod6 + 3 * D, *scf = mod6 + 4 * D, *gf = mod6 + 5 * D;
  /* widest GEMM output: D, F or (with the LoRA) the 3R columns of L_qkv */
  const int tw = F > D ? F : D;
  float *tmp = (float *)malloc(sizeof(float) * (size_t)T * (tw > 3 * R ? tw : 3 * R));
  uint16_t *t2 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * D);
  uint16_t *cat = lora ? (uint16_t *)malloc(sizeof(uint16_t) * (size_t)T * ((F / 2 > D ? F / 2 : D) + R)) : NULL;
  int stage = 0;
  hxo_rmsmod(x, T, D, w->n1, sha, sca, 1e-6f, b->h);
  TICK();
  if (lora) { /* L = f16(h . A_qkv) (blk.c:238) */
    hxo_gemm(b->h, D, w->aqkv, D, tmp, 3 * R, T, 3 * R, D); f2h_rows(tmp, 3 * R, b->lqkv, 3 * R, T, 3 * R);
  }
  TICK(); /* the LoRA-A GEMM stage (blk.c:238) */
  gemm_cat(b->h, D, D, lora ? b->lqkv : NULL, 3 * R, R, w->wq, D + R, tmp, T, D, cat); f2h_rows(tmp, D, b->q, D, T, D);
  gemm_cat(b->h, D, D, lora ? b->lqkv + R : NULL, 3 * R, R, w->wk, D + R, tmp, T, D, cat); f2h_rows(tmp, D, b->k, D, T, D);
  gemm_cat(b->h, D, D, lora ? b->lqkv + 2 * R : NULL, 3 * R, R, w->wv, D + R, tmp, T, D, cat); f2h_rows(tmp, D, b->v, D, T, D);
  hxo_rmsrope(b->q, T, D, H, w->gq, cosT, sinT, 1);
  hxo_rmsrope(b->k, T, D, H, w->gk, cosT, sinT, 1);
  TICK();
  hxo_attention(b->q, D, b->k, D, b->v, D, b->o, D, T, T, cfg->nvalid, H, cfg->attn_mode);
  TICK();
  if (lora) { hxo_gemm(b->o, D, w->ao, D, tmp, R, T, R, D); f2h_rows(tmp, R, b->lo, R, T, R); } /* blk.c:244 */
  gemm_cat(b->o, D, D, lora ? b->lo : NULL, R, R, w->wo, D + R, tmp, T, D, cat); f2h_rows(tmp, D, b->t, D, T, D);
  hxo_resadd(x, T, D, b->t, ga);
  TICK();
  hxo_rmsmod(x, T, D, w->n2, shf, scf, 1e-6f, b->h);
  TICK();
  if (lora) { hxo_gemm(b->h, D, w->aug, D, tmp, R, T, R, D); f2h_rows(tmp, R, b->lu, R, T, R); } /* blk.c:251 */
  gemm_cat(b->h, D, D, lora ? b->lu : NULL, R, R, w->wup, D + R, tmp, T, F, cat); f2h_rows(tmp, F, b->up, F, T, F);
  gemm_cat(b->h, D, D, lora ? b->lu : NULL, R, R, w->wgate, D + R, tmp, T, F, cat); f2h_rows(tmp, F, b->gate, F, T, F);
  hxo_situ_n(b->up, b->gate, b->mid, (size_t)T * F);
  TICK();
  {
    const int F2 = F / 2;
    if (lora) { hxo_gemm(b->mid, F, w->adn, F, tmp, R, T, R, F); f2h_rows(tmp, R, b->ld, R, T, R); } /* blk.c:255 */
    /* first K half without, second K half with the LoRA columns (blk.c:256-259) */
    hxo_gemm(b->mid, F, w->wdown, F + R, tmp, D, T, D, F2); f2h_rows(tmp, D, b->t, D, T, D);
    gemm_cat(b->mid + F2, F, F2, lora ? b->ld : NULL, R, R, w->wdown + F2, F + R, tmp, T, D, cat);
    f2h_rows(tmp, D, t2, D, T, D);
    hxo_resadd2(x, T, D, b->t, t2, gf);
  }
  TICK();
done:
  free(tmp); free(t2); free(cat);
  return stage;
}

/* ------------------------------------------------------------------------------------------------ */
/* caller-side glue                                                                                  */
/* ------------------------------------------------------------------------------------------------ */
void hxo_sinusoid(float t, int dim, float *out) {
  const int half = dim / 2;
  for (int i = 0; i < half; i++) {
    const float a = t * expf(-logf(10000.0f) * (float)i / (float)half);
    out[i] = cosf(a);
    out[i + half] = sinf(a);
  }
}
void hxo_patchify(const float *lat, int C, int H, int W, float *tok) {
  const int gh = H / 2, gw = W / 2;
  for (int gy = 0; gy < gh; gy++)
    for (int gx = 0; gx < gw; gx++)
      for (int c = 0; c < C; c++)
        for (int a = 0; a < 2; a++)
          for (int bb = 0; bb < 2; bb++)
            tok[(size_t)(gy * gw + gx) * (C * 4) + c * 4 + a * 2 + bb] = lat[((size_t)c * H + gy * 2 + a) * W + gx * 2 + bb];
}
void hxo_unpatchify(const float *y, int C, int H, int W, float *lat) {
  const int gh = H / 2, gw = W / 2;
  for (int gy = 0; gy < gh; gy++)
    for (int gx = 0; gx < gw; gx++)
      for (int a = 0; a < 2; a++)
        for (int bb = 0; bb < 2; bb++)
          for (int c = 0; c < C; c++)
            lat[((size_t)c * H + gy * 2 + a) * W + gx * 2 + bb] = y[(size_t)(gy * gw + gx) * (C * 4) + (a * 2 + bb) * C + c];
}
void hxo_final_norm(float *x, int T, int D, const float *shift, const float *scale) {
#pragma omp parallel for schedule(static)
  for (int i = 0; i < T; i++) {
    float *v = x + (size_t)i * D;
    double mu = 0, var = 0;
    for (int c = 0; c < D; c++) mu += v[c];
    mu /= D;
    for (int c = 0; c < D; c++) var += (v[c] - mu) * (v[c] - mu);
    const float rs = 1.0f / sqrtf((float)(var / D) + 1e-6f);
    for (int c = 0; c < D; c++) v[c] = (v[c] - (float)mu) * rs * (1.0f + scale[c]) + shift[c];
  }
}
