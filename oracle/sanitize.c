/* Sanitizer driver of the oracle (test infrastructure only, like hxo.c): every hxo_* function on small seeded inputs
 * in buffers of exactly the size each function's contract allows, built with -fsanitize=address,undefined by
 * `make -C oracle sanitize` and run there, so that an out-of-bounds access, a use of uninitialised-size memory or
 * undefined arithmetic in the oracle aborts the run. It also checks a few closed forms on the way (the fp16 round trip,
 * zero-gate identity of both blocks, softmax rows of one key), so a broken build does not pass silently. Exit 0: clean. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hxo.h"

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static double urand(void) { /* xorshift64*, [0, 1) */
  g_rng ^= g_rng >> 12;
  g_rng ^= g_rng << 25;
  g_rng ^= g_rng >> 27;
  return (double)((g_rng * 2685821657736338717ull) >> 11) * (1.0 / 9007199254740992.0);
}
static double nrand(void) {
  const double u = urand() + 1e-300, v = urand();
  return sqrt(-2.0 * log(u)) * cos(6.283185307179586 * v);
}
static float *fvec(size_t n, double sd) {
  float *p = malloc(n * sizeof(float));
  for (size_t i = 0; i < n; i++) p[i] = (float)(nrand() * sd);
  return p;
}
static uint16_t *hvec(size_t n, double sd) {
  uint16_t *p = malloc(n * sizeof(uint16_t));
  for (size_t i = 0; i < n; i++) p[i] = hxo_f2h((float)(nrand() * sd));
  return p;
}
static uint16_t *hzero(size_t n) { return calloc(n, sizeof(uint16_t)); }

static int g_fail = 0;
static void check(int ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "sanitize: check failed: %s\n", what);
    g_fail = 1;
  }
}

static void primitives(void) {
  /* fp16 conversions: every half round-trips */
  for (uint32_t h = 0; h < 65536; h++) {
    if ((h & 0x7c00) == 0x7c00 && (h & 0x3ff)) continue; /* NaN payloads */
    const float f = hxo_h2f((uint16_t)h);
    check(hxo_f2h(f) == (uint16_t)h || (h == 0x8000 && hxo_f2h(f) == 0x8000), "fp16 round trip");
  }
  const int M = 37, N = 64, K = 96; /* M not a multiple of anything */
  uint16_t *A = hvec((size_t)M * K, 1.0), *W = hvec((size_t)N * K, 0.05);
  float *C = malloc(sizeof(float) * M * N), *C2 = malloc(sizeof(float) * M * N);
  hxo_gemm(A, K, W, K, C, N, M, N, K);
  hxo_gemm_naive(A, K, W, K, C2, N, M, N, K);
  for (int i = 0; i < M * N; i++) check(fabsf(C[i] - C2[i]) <= 1e-5f * (1.0f + fabsf(C2[i])), "gemm vs naive");
  float *xf = fvec((size_t)M * K, 1.0), *yf = malloc(sizeof(float) * M * N);
  hxo_linear_f32(xf, K, W, K, yf, N, M, N, K);
  /* norms */
  const int T = 33, D = 256;
  float *x = fvec((size_t)T * D, 1.0), *sh = fvec(D, 0.1), *scl = fvec(D, 0.1), *wn = fvec(D, 1.0);
  uint16_t *h = hzero((size_t)T * D);
  hxo_lnmod(x, T, D, sh, scl, 1e-6f, h);
  hxo_rmsmod(x, T, D, wn, sh, scl, 1e-6f, h);
  /* head norm + RoPE */
  float *gain = fvec(128, 1.0), *cs = malloc(sizeof(float) * T * 64), *sn = malloc(sizeof(float) * T * 64);
  for (int i = 0; i < T * 64; i++) {
    const double a = nrand();
    cs[i] = (float)cos(a);
    sn[i] = (float)sin(a);
  }
  uint16_t *q = hvec((size_t)T * D, 1.0);
  hxo_rmsrope(q, T, D, 2, gain, cs, sn, 1);
  hxo_rmsrope(q, T, D, 2, gain, NULL, NULL, 0);
  /* attention, both modes, masked keys, a single valid key */
  const int NKV = 45;
  uint16_t *k = hvec((size_t)NKV * D, 1.0), *v = hvec((size_t)NKV * D, 1.0), *o = hzero((size_t)T * D);
  for (int mode = 0; mode < 2; mode++) {
    hxo_attention(q, D, k, D, v, D, o, D, T, NKV, NKV, 2, mode);
    hxo_attention(q, D, k, D, v, D, o, D, T, NKV, 29, 2, mode);
    hxo_attention(q, D, k, D, v, D, o, D, T, NKV, 1, 2, mode);
    /* one valid key: every output row is that key's v (to fp16) */
    check(o[5 * D + 7] == v[7] || fabsf(hxo_h2f(o[5 * D + 7]) - hxo_h2f(v[7])) <= 1e-3f * (1 + fabsf(hxo_h2f(v[7]))),
          "attention over one key");
  }
  /* activations and residuals */
  for (uint32_t t = 0; t < 65536; t += 7) {
    (void)hxo_gelu_erf_h((uint16_t)t);
    (void)hxo_gelu_tanh_h((uint16_t)t);
    (void)hxo_situ_h((uint16_t)t, (uint16_t)(t * 31u));
  }
  uint16_t *t1 = hvec((size_t)T * D, 1.0), *t2 = hvec((size_t)T * D, 1.0), *so = hzero((size_t)T * D);
  hxo_gelu_n(t1, (size_t)T * D, 0);
  hxo_gelu_n(t2, (size_t)T * D, 1);
  hxo_situ_n(t1, t2, so, (size_t)T * D);
  hxo_resadd(x, T, D, t1, sh);
  hxo_resadd2(x, T, D, t1, t2, sh);
  /* codecs and layouts (sizes multiples of the 32 x 32 tiles) */
  const int QN = 64, QK = 128;
  float *Wq = fvec((size_t)QN * QK, 0.02);
  int8_t *q8 = malloc((size_t)QN * QK);
  uint8_t *q4 = malloc((size_t)QN * QK / 2);
  uint16_t *s = malloc(sizeof(uint16_t) * (QK / 32) * QN), *w16 = malloc(sizeof(uint16_t) * QN * QK);
  uint16_t *z = hvec((size_t)(QK / 32) * QN, 0.01);
  hxo_q8_quantize(Wq, QN, QK, q8, s);
  hxo_q8_dequant(q8, s, QN, QK, w16);
  hxo_q4_quantize(Wq, QN, QK, q4, s);
  hxo_q4_dequant(q4, s, NULL, QN, QK, w16);
  hxo_q4_dequant(q4, s, z, QN, QK, w16);
  uint16_t *tiles = malloc(sizeof(uint16_t) * QN * QK), *back = malloc(sizeof(uint16_t) * QN * QK);
  hxo_h16_tile(w16, QN, QK, tiles);
  hxo_h16_untile(tiles, QN, QK, back);
  check(memcmp(back, w16, sizeof(uint16_t) * QN * QK) == 0, "h16 tile round trip");
  float *xt = malloc(sizeof(float) * QN * QK), *xb = malloc(sizeof(float) * QN * QK);
  hxo_x32_tile(Wq, QN, QK, xt);
  hxo_x32_untile(xt, QN, QK, xb);
  check(memcmp(xb, Wq, sizeof(float) * QN * QK) == 0, "x32 tile round trip");
  hxo_wt16_pack(w16, QN, QK, tiles);
  hxo_wt16_unpack(tiles, QN, QK, back);
  check(memcmp(back, w16, sizeof(uint16_t) * QN * QK) == 0, "weight tile round trip");
  uint8_t *rec = malloc((size_t)QN * QK / 1024 * 1152);
  hxo_q8rec_pack(w16, QN, QK, rec, 0);
  hxo_q8rec_unpack(rec, QN, QK, back);
  hxo_q8rec_pack(w16, QN, QK, rec, 1);
  hxo_q8rec_unpack(rec, QN, QK, back);
  uint8_t *rec4 = malloc((size_t)QN * QK / 1024 * 768);
  for (size_t i = 0; i < (size_t)QN * QK / 1024 * 768; i++) rec4[i] = (uint8_t)(urand() * 256);
  for (size_t r = 0; r < (size_t)QN * QK / 1024; r++) /* finite scales and mins */
    for (int m = 0; m < 128; m++) {
      const uint16_t hv = hxo_f2h((float)(nrand() * 0.01));
      memcpy(rec4 + r * 768 + 2 * m, &hv, 2);
    }
  hxo_q4arec_unpack(rec4, QN, QK, back);
  /* RoPE tables, low-res glue */
  float *rc = malloc(sizeof(float) * 12 * 8 * 64), *rs = malloc(sizeof(float) * 12 * 8 * 64);
  hxo_rope_anima(12, 8, rc, rs);
  float *bands = fvec(16, 0.1), *mc = malloc(sizeof(float) * (6 * 4 + 5) * 64), *ms = malloc(sizeof(float) * (6 * 4 + 5) * 64);
  hxo_rope_moss(6, 4, 5, bands, mc, ms);
  hxo_rope_moss_scaled(6, 4, 5, bands, 2.0, mc, ms);
  const int LC = 4, LH = 16, LW = 12, f = 2;
  float *nf = fvec((size_t)LC * LH * LW, 1.0), *dh = fvec((size_t)LC * LH * LW, 1.0);
  float *xl = malloc(sizeof(float) * LC * (LH / f) * (LW / f)), *vl = fvec((size_t)LC * (LH / f) * (LW / f), 1.0);
  float *dh2 = malloc(sizeof(float) * LC * LH * LW), *vf = malloc(sizeof(float) * LC * LH * LW);
  hxo_lowres_pool(nf, dh, LC, LH, LW, f, 0.75f, xl);
  hxo_lowres_velocity(xl, vl, nf, nf, LC, LH, LW, f, 0.75f, 0.5, dh2, vf);
  float *zr = fvec((size_t)6 * 4 * 16, 1.0), *zl = malloc(sizeof(float) * 3 * 2 * 16), *up = malloc(sizeof(float) * 6 * 4 * 16);
  hxo_moss_pool2(zr, 6, 4, 16, zl);
  hxo_upsample2_rows(zl, 3, 2, 16, up);
  float *sinus = malloc(sizeof(float) * 256), *tok = malloc(sizeof(float) * (LH / 2) * (LW / 2) * LC * 4);
  float *lat = malloc(sizeof(float) * LC * LH * LW);
  hxo_sinusoid(0.75f, 256, sinus);
  hxo_patchify(nf, LC, LH, LW, tok);
  hxo_unpatchify(tok, LC, LH, LW, lat);
  float *fx = fvec((size_t)T * D, 1.0);
  hxo_final_norm(fx, T, D, sh, scl);
  void *ps[] = {A, W, C, C2, xf, yf, x, sh, scl, wn, h, gain, cs, sn, q, k, v, o, t1, t2, so, Wq, q8, q4, s, w16, z, tiles, back,
                xt, xb, rec, rec4, rc, rs, bands, mc, ms, nf, dh, xl, vl, dh2, vf, zr, zl, up, sinus, tok, lat, fx};
  for (size_t i = 0; i < sizeof ps / sizeof ps[0]; i++) free(ps[i]);
}

static void anima_block(int stop) {
  const int T = 64, D = 256, H = 2, Cn = 32, DC = 128, F = 512;
  hxo_anima_cfg cfg = {T, D, H, Cn, DC, F, 0, stop, 0};
  uint16_t *wq = hvec((size_t)D * D, 0.02), *wk = hvec((size_t)D * D, 0.02), *wv = hvec((size_t)D * D, 0.02),
           *wo = hvec((size_t)D * D, 0.02), *wcq = hvec((size_t)D * D, 0.02), *wck = hvec((size_t)D * DC, 0.02),
           *wcv = hvec((size_t)D * DC, 0.02), *wco = hvec((size_t)D * D, 0.02), *w1 = hvec((size_t)F * D, 0.02),
           *w2 = hvec((size_t)D * F, 0.02);
  float *gain = fvec(512, 0.1);
  for (int i = 0; i < 512; i++) gain[i] += 1.0f;
  hxo_anima_w w = {wq, wk, wv, wo, wcq, wck, wcv, wco, w1, w2, gain};
  float *x = fvec((size_t)T * D, 1.0), *x0 = malloc(sizeof(float) * T * D);
  memcpy(x0, x, sizeof(float) * T * D);
  uint16_t *ctx = hvec((size_t)Cn * DC, 1.0);
  float *mod = fvec((size_t)9 * D, 0.2), *cs = malloc(sizeof(float) * T * 64), *sn = malloc(sizeof(float) * T * 64);
  hxo_rope_anima(8, 8, cs, sn);
  hxo_anima_buf b = {hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * D),
                     hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * F), hzero((size_t)Cn * D),
                     hzero((size_t)Cn * D)};
  (void)hxo_anima_block(&cfg, &w, x, ctx, mod, cs, sn, &b);
  if (stop == 0) { /* zero gates: the block is the identity on x */
    memcpy(x, x0, sizeof(float) * T * D);
    for (int s = 0; s < 3; s++) memset(mod + (3 * s + 2) * D, 0, sizeof(float) * D);
    (void)hxo_anima_block(&cfg, &w, x, ctx, mod, cs, sn, &b);
    check(memcmp(x, x0, sizeof(float) * T * D) == 0, "anima block with zero gates is the identity");
  }
  void *ps[] = {wq, wk, wv, wo, wcq, wck, wcv, wco, w1, w2, gain, x, x0, ctx, mod, cs, sn, b.h, b.q, b.k, b.v, b.o, b.t, b.mid,
                b.ck, b.cv};
  for (size_t i = 0; i < sizeof ps / sizeof ps[0]; i++) free(ps[i]);
}

static void moss_block(int lora, int stop) {
  const int T = 96, nvalid = 83, D = 256, H = 2, F = 256, r = lora ? 128 : 0;
  hxo_moss_cfg cfg = {T, nvalid, D, H, F, stop, 0};
  const size_t KD = (size_t)D + r, KF = (size_t)F + r;
  uint16_t *wq = hvec(D * KD, 0.02), *wk = hvec(D * KD, 0.02), *wv = hvec(D * KD, 0.02), *wo = hvec(D * KD, 0.02),
           *wup = hvec(F * KD, 0.02), *wgate = hvec(F * KD, 0.02), *wdown = hvec(D * KF, 0.02);
  uint16_t *aqkv = lora ? hvec((size_t)3 * r * D, 0.02) : NULL, *ao = lora ? hvec((size_t)r * D, 0.02) : NULL,
           *aug = lora ? hvec((size_t)r * D, 0.02) : NULL, *adn = lora ? hvec((size_t)r * F, 0.02) : NULL;
  float *gq = fvec(128, 0.1), *gk = fvec(128, 0.1), *n1 = fvec(D, 0.1), *n2 = fvec(D, 0.1);
  hxo_moss_w w = {wq, wk, wv, wo, wup, wgate, wdown, gq, gk, n1, n2, aqkv, ao, aug, adn};
  float *x = fvec((size_t)T * D, 1.0), *x0 = malloc(sizeof(float) * T * D);
  memcpy(x0, x, sizeof(float) * T * D);
  float *mod = fvec((size_t)6 * D, 0.2), *cs = malloc(sizeof(float) * T * 64), *sn = malloc(sizeof(float) * T * 64);
  for (int i = 0; i < T * 64; i++) {
    cs[i] = 1.0f;
    sn[i] = 0.0f;
  }
  const size_t rr = lora ? (size_t)r : 1;
  hxo_moss_buf b = {hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * D),
                    hzero((size_t)T * D), hzero((size_t)T * D), hzero((size_t)T * F), hzero((size_t)T * F),
                    hzero((size_t)T * F), hzero((size_t)T * 3 * rr), hzero((size_t)T * rr), hzero((size_t)T * rr),
                    hzero((size_t)T * rr)};
  (void)hxo_moss_block(&cfg, &w, x, mod, cs, sn, &b);
  if (stop == 0) {
    memcpy(x, x0, sizeof(float) * T * D);
    memset(mod + 2 * D, 0, sizeof(float) * D);
    memset(mod + 5 * D, 0, sizeof(float) * D);
    (void)hxo_moss_block(&cfg, &w, x, mod, cs, sn, &b);
    check(memcmp(x, x0, sizeof(float) * T * D) == 0, "moss block with zero gates is the identity");
  }
  void *ps[] = {wq, wk, wv, wo, wup, wgate, wdown, aqkv, ao, aug, adn, gq, gk, n1, n2, x, x0, mod, cs, sn, b.h, b.q, b.k,
                b.v, b.o, b.t, b.up, b.gate, b.mid, b.lqkv, b.lo, b.lu, b.ld};
  for (size_t i = 0; i < sizeof ps / sizeof ps[0]; i++) free(ps[i]);
}

int main(void) {
  hxo_set_threads(2);
  primitives();
  for (int stop = 0; stop <= 13; stop += 13) anima_block(stop);
  anima_block(5);
  for (int lora = 0; lora < 2; lora++) {
    moss_block(lora, 0);
    moss_block(lora, 4);
  }
  printf("sanitize: %s\n", g_fail ? "FAILED" : "clean");
  return g_fail;
}
