/* hxo — CPU oracle for the HexAnima DiT block runner.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (hexanima_amd/, include/) links or calls this code;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker.
 *
 * It restates, in plain C with double-precision arithmetic, the block semantics of the reference's
 * Hexagon mega-kernel (hexagon/mega/blk.c:149-176, kern.c, gemm2.c) and of the MOSS variant
 * (moss/hexagon/mega/blk.c:234-259, moss/moss_ref.py:21-67), honouring every point where the reference
 * stores fp16 (activations h/q/k/v/o/t/mid, attention S/P/rowsum) and keeping the residual stream fp32.
 *
 * Layouts are the math layouts, not the reference's crouton tiles:
 *   activations [rows][cols] row-major; weights W[N][K] (row n = output feature, K contiguous), so a
 *   linear is y[m][n] = sum_k x[m][k] * W[n][k]. Crouton / q8-record converters for the reference's
 *   on-disk formats are provided separately (hxo_h16tile_*, hxo_q8rec_*, hxo_q4arec_*).
 *
 * Parity pinning of every function is done in tests/test_oracle_*.py (closed forms, invariants, numpy
 * float64 / float16 library routines, brute force, the reference's own integer-hash KAT generator).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 (IEEE binary16, round-to-nearest-even) ---- */
uint16_t hxo_f2h(float f);
float hxo_h2f(uint16_t h);
void hxo_f2h_n(const float *src, uint16_t *dst, size_t n);
void hxo_h2f_n(const uint16_t *src, float *dst, size_t n);
int hxo_set_threads(int n); /* <=0: leave as is; returns the thread count in use */

/* ---- GEMM: C[m][n] = sum_k A[m][k] * W[n][k]  (fp16 operands, double accumulation, fp32 result) ----
   reference: gemm2.c:96-137 (O = A*W on HMX; fp16 in, fp16 out; the caller rounds C to fp16 where the
   reference stores fp16) */
void hxo_gemm(const uint16_t *A, long lda, const uint16_t *W, long ldw, float *C, long ldc, int M, int N, int K);
void hxo_gemm_naive(const uint16_t *A, long lda, const uint16_t *W, long ldw, float *C, long ldc, int M, int N, int K);
/* fp32-activation linear (used by the caller-side glue: patch embed, t-embedding MLPs, final layer) */
void hxo_linear_f32(const float *x, long ldx, const uint16_t *W, long ldw, float *y, long ldy, int M, int N, int K);

/* ---- row norms with adaLN modulation (x fp32 [T][D] -> h fp16 [T][D]) ----
   lnmod: kern.c:31-65   y = (x - mu) * rsqrt(E[x^2] - mu^2 + eps) * (1 + scale) + shift
   rmsmod: moss kern.c:345-375   y = x * rsqrt(mean(x^2) + eps) * (w * (1 + scale)) + shift */
void hxo_lnmod(const float *x, int T, int D, const float *shift, const float *scale, float eps, uint16_t *h);
void hxo_rmsmod(const float *x, int T, int D, const float *w, const float *shift, const float *scale, float eps, uint16_t *h);

/* ---- per-head RMSNorm * gain, then split-half RoPE on pairs (d, d+64) (kern.c:163-197) ----
   q fp16 [T][ldq], H heads of 128; gain[128]; cos/sin [T][64] (NULL when rope == 0). In place. */
void hxo_rmsrope(uint16_t *q, int T, long ldq, int H, const float *gain, const float *cosT, const float *sinT, int rope);

/* ---- attention, per head of 128, no 1/sqrt(d) (folded into the q gain, export_all.py:31-32) ----
   q [T][ldq], k [NKV][ldk], v [NKV][ldv] fp16; o [T][ldo] fp16. Keys >= nvalid are masked (moss blk.c:56-58).
   mode 0 = reference rounding (blk.c:54-91, kern.c:261-295):
     S = f16(q.k), m = rowmax S, P = f16(exp(-|f16(S - m)|)), l = f16(sum P), O = f16(f16(P.v) * (1/l))
   mode 1 = exact softmax in double, one final fp16 rounding of O (calibration of the tolerance budget) */
void hxo_attention(const uint16_t *q, long ldq, const uint16_t *k, long ldk, const uint16_t *v, long ldv, uint16_t *o,
                   long ldo, int T, int NKV, int nvalid, int H, int mode);

/* ---- activations on fp16 values ---- */
uint16_t hxo_gelu_erf_h(uint16_t t);  /* kern.c:235-260: f16(max(t,0) - f16(|t| Phi(-|t|))) */
uint16_t hxo_gelu_tanh_h(uint16_t t); /* f16(0.5 t (1 + tanh(sqrt(2/pi)(t + 0.044715 t^3)))) */
uint16_t hxo_situ_h(uint16_t up, uint16_t gate); /* moss kern.c:376-405: f16(f16(25 tanh(u/25)) * f16(4 tanh(g/4) sigmoid(g))) */
void hxo_gelu_n(uint16_t *t, size_t n, int mode); /* mode 0 erf (reference table), 1 tanh */
void hxo_situ_n(const uint16_t *up, const uint16_t *gate, uint16_t *out, size_t n);

/* ---- gated residuals (x fp32 [T][D]; t fp16) ----
   resadd:  x += gate * t          (kern.c:320-328)
   resadd2: x += gate * (t1 + t2)  (kern.c:330-339, the split-K down projection) */
void hxo_resadd(float *x, int T, int D, const uint16_t *t, const float *gate);
void hxo_resadd2(float *x, int T, int D, const uint16_t *t1, const uint16_t *t2, const float *gate);

/* ---- weight-only quantisation (GPU-native layout) ----
   q8 (export_all.py:10-18, moss/export_all_q8.py:13): per (column n, 32-row K group g):
     s = f16(max|f16(w)| / 127), floored at 6.2e-5; q = clip(rint(f16(w) / s), -127, 127); value = f16(q * s)
   layout: q [N][K] int8, s [K/32][N] fp16.
   q4 symmetric: s = f16(max|f16(w)| / 7) (floored at 6.2e-5), q = clip(rint(w/s), -8, 7), value = f16(q * s).
   q4 asymmetric (q4a, moss/export_te.py:1-3): value = f16(nibble * s + z) with nibble in [0,15].
   q4 layout: [N][K/2] bytes; each 32-bit word holds 8 consecutive k (k0..k0+7): k0+2j at bits [4j,4j+4),
   k0+2j+1 at bits [16+4j, 20+4j); symmetric nibble = q + 8. s, z: [K/32][N] fp16. */
void hxo_q8_quantize(const float *W, int N, int K, int8_t *q, uint16_t *s);
void hxo_q8_dequant(const int8_t *q, const uint16_t *s, int N, int K, uint16_t *w16);
void hxo_q4_quantize(const float *W, int N, int K, uint8_t *q, uint16_t *s);
void hxo_q4_dequant(const uint8_t *q, const uint16_t *s, const uint16_t *z, int N, int K, uint16_t *w16);

/* ---- the reference's on-disk tile formats (boundary compatibility) ----
   h16 tile (kern.h:5-8): 32x32 fp16, halfword(r,c) = (r/2)*64 + c*2 + (r&1); matrices [row slab][col block].
   weights are tiled as the matrix [K][N] with tiles [n block][k block] (export_all.py:7-8).
   q8 record (export_all.py:10-18): 64 fp16 (halfword l = scale of column l/2) + 1024 B offset-binary int8.
   q4a record (moss/export_te.py:1-3): 64 fp16 scales, 64 fp16 mins, 512 B nibbles (byte b of vector m:
   low nibble = halfword 256m+b, high nibble = halfword 256m+128+b). */
void hxo_h16_tile(const uint16_t *a, int R, int C, uint16_t *tiles);   /* a [R][C] -> [R/32][C/32] tiles */
void hxo_h16_untile(const uint16_t *tiles, int R, int C, uint16_t *a);
void hxo_x32_tile(const float *a, int R, int C, float *tiles);         /* x32: float(r,c) = r*32 + c */
void hxo_x32_untile(const float *tiles, int R, int C, float *a);
void hxo_wt16_pack(const uint16_t *wNK, int N, int K, uint16_t *tiles);  /* W[N][K] -> matrix [K][N] tiles [nb][kb] */
void hxo_wt16_unpack(const uint16_t *tiles, int N, int K, uint16_t *wNK);
void hxo_q8rec_pack(const uint16_t *wNK, int N, int K, uint8_t *rec, int floor_mode); /* floor_mode 0: s==0 -> 1; 1: floor 6.2e-5 */
void hxo_q8rec_unpack(const uint8_t *rec, int N, int K, uint16_t *wNK);   /* dequantised f16(q*s) as W[N][K] */
void hxo_q4arec_unpack(const uint8_t *rec, int N, int K, uint16_t *wNK);

/* ---- RoPE tables [T][64] ----
   anima: megarun.cpp:77-90 (3-axis split: 22 zero t-angles, 21 h, 21 w; theta 10000; dim_h 42)
   moss:  moss_ref.py:27-35 (4 axes x 16 bands; image tokens (0, ntxt, h-(H-1)/2, w-(W-1)/2), text (0, i, 0, 0)) */
void hxo_rope_anima(int gh, int gw, float *cosT, float *sinT);
void hxo_rope_moss(int H, int W, int ntxt, const float *bands16, float *cosT, float *sinT);
void hxo_rope_moss_scaled(int H, int W, int ntxt, const float *bands16, double scale, float *cosT, float *sinT);
/* low-res first steps: phone/animad.cpp:429-437, :486-503; moss/mossrun/mossrun.cpp:278-282, :291 */
void hxo_lowres_pool(const float *nfull, const float *dhat, int C, int H, int W, int f, float t, float *xlow);
void hxo_lowres_velocity(const float *xlow, const float *vlow, const float *xfull, const float *nfull, int C, int H, int W,
                         int f, float t, double tn, float *dhat, float *vf);
void hxo_moss_pool2(const float *z, int H, int W, int C4, float *zl);
void hxo_upsample2_rows(const float *src, int h, int w, int C4, float *dst);

/* ---- one Anima-structure DiT block (blk.c:149-176; appendix semantics in the header comment of hxo.c) ---- */
typedef struct {
  int T, D, H, C, DC, F; /* image tokens, width, heads (x128), context tokens, context width, MLP width */
  int gelu;              /* 0 erf table (the reference block), 1 tanh */
  int stop;              /* stop after this many stages (meta[M_STOP]); 0 = run all 13 */
  int attn_mode;         /* hxo_attention mode */
} hxo_anima_cfg;
typedef struct {
  const uint16_t *wq, *wk, *wv, *wo, *wcq, *wck, *wcv, *wco, *w1, *w2; /* W[N][K] fp16 */
  const float *gain; /* [4][128]: q/sqrt(128), k, cross q/sqrt(128), cross k (export_all.py:31-32) */
} hxo_anima_w;
typedef struct {
  uint16_t *h, *q, *k, *v, *o, *t; /* [T][D] */
  uint16_t *mid;                   /* [T][F] */
  uint16_t *ck, *cv;               /* [C][D] */
} hxo_anima_buf;
int hxo_anima_block(const hxo_anima_cfg *cfg, const hxo_anima_w *w, float *x, const uint16_t *ctx, const float *mod9,
                    const float *cosT, const float *sinT, hxo_anima_buf *b);

/* ---- one MOSS-class block (moss/hexagon/mega/blk.c:234-259, moss_ref.py:56-67), joint attention ---- */
typedef struct {
  int T, nvalid, D, H, F; /* padded tokens, valid tokens, width, heads, FFN width (up and gate each F) */
  int stop, attn_mode;
} hxo_moss_cfg;
/* rapid-moss LoRA (moss/hexagon/mega/blk.c:238-259, packed by moss/export_moss.py:34-47): with aqkv != NULL every
   projection runs on [x | L] . [W ; s B] where L = f16(x . A) is rank r = 128 and the scaled B rows are appended
   along K. The matrices are then W[N][K + r]: wq / wk / wv / wo / wup / wgate [.][D + r], wdown [D][F + r]; the
   A matrices (as W[N][K]): aqkv [3r][D] (q, k, v parts), ao [r][D], aug [r][D], adn [r][F]. The down projection's
   two K halves are [0, F/2) and [F/2, F) + the r LoRA columns (blk.c:256-259). */
typedef struct {
  const uint16_t *wq, *wk, *wv, *wo; /* [D][D] ([D][D + r] with LoRA) */
  const uint16_t *wup, *wgate;       /* [F][D] ([F][D + r]) */
  const uint16_t *wdown;             /* [D][F] ([D][F + r]) */
  const float *gq, *gk;              /* [128]; gq pre-scaled by 1/sqrt(128) */
  const float *n1, *n2;              /* [D] RMSNorm weights */
  const uint16_t *aqkv, *ao, *aug, *adn; /* LoRA A matrices (NULL: no LoRA) */
} hxo_moss_w;
typedef struct {
  uint16_t *h, *q, *k, *v, *o, *t; /* [T][D] */
  uint16_t *up, *gate, *mid;       /* [T][F] */
  uint16_t *lqkv, *lo, *lu, *ld;   /* LoRA L buffers [T][3r], [T][r] x 3 (NULL / unused without LoRA) */
} hxo_moss_buf;
int hxo_moss_block(const hxo_moss_cfg *cfg, const hxo_moss_w *w, float *x, const float *mod6, const float *cosT,
                   const float *sinT, hxo_moss_buf *b);

/* ---- caller-side glue (phone/animad.cpp) ---- */
void hxo_sinusoid(float t, int dim, float *out); /* animad.cpp:425: [cos(t w_i) | sin(t w_i)], w_i = 10000^(-i/(dim/2)) */
void hxo_patchify(const float *lat, int C, int H, int W, float *tok);      /* animad.cpp:447-450: [T][C*4], (c, ph, pw) */
void hxo_unpatchify(const float *y, int C, int H, int W, float *lat);      /* animad.cpp:490-491: y [T][4C], (ph, pw, c) */
void hxo_final_norm(float *x, int T, int D, const float *shift, const float *scale); /* animad.cpp:478-488 */

#ifdef __cplusplus
}
#endif
