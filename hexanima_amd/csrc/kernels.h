// Internal launch interface of the HIP kernels (device pointers; not part of the public C-ABI).
#pragma once
#include "hxa_common.h"

struct HxaGemm {
  const hxa_h *A;     // [M][lda] fp16
  long lda;
  int M;
  const HxaWeight *w; // W[N][K] in one of the HXA_W_* formats
  int ksplit;         // split-K slices (HXA_EPI_PARTIAL only)
  int epi;            // HXA_EPI_*
  hxa_h *out;         // STORE / GELU / PARTIAL / SITU: [M][ldo]; STORE_T: [N][ldo]; QKV: q/k part
  long ldo, out_zstride;
  float *x;           // RESADD: x[M][ldx] fp32
  long ldx;
  const float *gate;  // RESADD: gate[N]
  // [pf, pf + pf_bytes): memory the next kernel reads (its weights), touched once per 128-byte line after this
  // GEMM's main loop so that it streams in from HBM under the epilogue; 0 bytes: none.
  // Not with RESADD / RESADD_SPLIT2 or a head norm (their epilogues load, and would wait for the prefetch).
  const void *pf;
  long pf_bytes;
  hxa_h *out_t;       // QKV/KV split: columns >= split_col are written transposed to out_t[n - split_col][m]
  long ldo_t;
  int split_col;
  int force_bm, force_bn;  // 0 = automatic tile choice
  int force_nw;            // waves per workgroup with a forced tile: 0 / 4, 8, or 9 (the ping-pong kernel)
  // STORE with head norm: columns [0, hn_cols) (multiple of 128) get per-head RMSNorm * gain (gain hn_g0 for columns
  // < hn_gsplit, hn_g1 above) and, with hn_cos / hn_sin [hn_ttab][64], RoPE at token m % hn_ttab (kern.c:163-197)
  int hn_cols, hn_gsplit, hn_ttab;
  const float *hn_g0, *hn_g1, *hn_cos, *hn_sin;
  // a GEMV to run with this GEMM: in workgroups appended to a one-slice ping-pong grid whose last round leaves at
  // least 16 CUs idle, else as its own launch after the GEMM (nullptr: none)
  const HxaSideGemv *side;
};
int hxa_gemm_launch(const HxaGemm &g, hipStream_t st);
// the tile hxa_gemm_launch would run g on (bm x bn, nw waves per workgroup, 9 = the ping-pong kernel) and the
// rounds of workgroups over the CUs it would take (tile grid x ksplit / CUs, rounded up); HXA_OK, or the error
// hxa_gemm_launch would return
int hxa_gemm_plan(const HxaGemm &g, int *bm, int *bn, int *nw, int *rounds);
// two independent GEMMs in one launch (the second takes the first one's tile; same weight format, no split-K);
// falls back to two launches when the tile has no paired kernel
int hxa_gemm_pair_launch(const HxaGemm &g0, const HxaGemm &g1, hipStream_t st);
// The cross-attention site's q projection fused with its attention (blk.c:163-169): g is the cross-q GEMM (fp16
// weights, HXA_EPI_STORE, a head norm on every column, no RoPE); each 128 x 128 tile's queries (one head) attend to
// their image's keys. Returns HXA_E_ARG when the shapes do not fit the fused kernel (T % 128, N % 128, weight format,
// strides); the caller then runs the projection and hxa_attn_launch.
struct HxaXAttn {
  const hxa_h *k, *vt;  // k [NKV][ldk] (head h at column 128 h), vt [D][ldvt] (keys contiguous)
  hxa_h *o;             // [M][ldo]
  long ldk, ldvt, ldo;
  long kb, vb;          // per-image offsets: k elements, vt columns
  int NKV, nvalid, T;   // keys, valid keys, query rows per image
};
int hxa_gemm_xattn_launch(const HxaGemm &g, const HxaXAttn &a, hipStream_t st);
// whether the fused kernel's 128 x 128 tiles of an M x N projection fit in one round over the CUs (beyond one round
// the projection's own tile pick plus the attention kernel is faster)
bool hxa_gemm_xattn_fits(int M, int N);
// whether hxa_gemm_pair_launch(g0, g1) would be one launch that takes no more rounds of workgroups over the CUs than
// g0 alone (g1 only fills CUs g0 leaves idle)
bool hxa_gemm_pair_fits(const HxaGemm &g0, const HxaGemm &g1);
// G GEMMs of one shape and weight format (ksplit 1, no prefetch) in one launch on the ping-pong 192x256 tile, each
// with its own operands and epilogue. prepare fills params_host (hxa_gemm_group_param_bytes(G) bytes, to be copied
// to device memory as they are) and returns the tiles per GEMM and the launch format; the device copy stays valid
// while the GEMMs' operands stay where they are.
long hxa_gemm_group_param_bytes(int G);
int hxa_gemm_group_prepare(const HxaGemm *g, int G, void *params_host, int *tiles, int *fmt);
int hxa_gemm_group_launch(const void *params_dev, int G, int tiles, int fmt, hipStream_t st);
// int8 / int4 weight -> fp16 k-tiled [K/32][N][32] at out (2 N K bytes): the same values the GEMM main loops use
int hxa_dequant_launch(const HxaWeight &w, hxa_h *out, hipStream_t st);
// out[m][n] = f16(sum of the S fp32 slices p[z*zstride + m*ldp + n], added in order z = 0 .. S-1)
int hxa_sum_partials_launch(const float *p, int S, long zstride, long ldp, int M, int N, hxa_h *out, long ldo,
                            hipStream_t st);
// the K slices hxa_linear runs M x N x K in (1: one launch)
int hxa_linear_split(int M, int N, int K, int fmt);

struct HxaAttn {
  const hxa_h *q, *k, *vt;  // q [T][ldq], k [NKV][ldk] (head h at column h*128); vt [H*128][ldvt] (keys contiguous)
  long ldq, ldk, ldvt;
  hxa_h *o;                 // [T][ldo]
  long ldo;
  int T, NKV, nvalid, H, batch;
  long q_bstride, k_bstride, vt_bstride, o_bstride;  // per-image offsets (elements)
  HxaClk clk;  // shader-clock record: set by hxa_attn_launch from the current one (callers leave it empty)
  // [pf, pf + pf_bytes): memory the kernels after this one read (the next projections' weights), touched once per
  // 128-byte line while the key tiles run, so that it is in L2 / MALL when they start (attn_kernel only; pf_bytes a
  // multiple of 128)
  const uint8_t *pf = nullptr;
  long pf_bytes = 0;
  // side_wgs > 0 (batch 1): side runs in side_wgs workgroups past the attention tiles. Where the chosen kernel cannot
  // host it (at most 256 keys: the two-pass kernel), it runs as its own hxa_modgemv_launch after the attention.
  HxaSideGemv side{};
  int side_wgs = 0;
};
int hxa_attn_launch(const HxaAttn &p, hipStream_t st);
// workgroups an attention launch of T queries x H heads (batch 1) leaves idle on this GPU: what side_wgs may use
// (0 when the tiles leave fewer than a quarter of the CUs idle in their last round: too few to stream a GEMV in
// the attention's time)
int hxa_attn_idle_wgs(int T, int H, int batch);

// h[t][:] = f16(norm(x[t][:]) * mul + add); LN: (x-mu)*rsqrt(E[x^2]-mu^2+eps), RMS (w != NULL): x*rsqrt(E[x^2]+eps)
// with mul = (1 + scale) (LN) or (1 + scale) * w (RMS), add = shift.
// the same with the previous site's gated residual applied first: x += gate * t (fp16 t [T][ldt]), x written back
int hxa_resid_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, long ldt, const float *gate,
                              const float *shift, const float *scale, const float *w, float eps, hxa_h *h, long ldh,
                              hipStream_t st);
// the same with two pending fp16 terms: x += gate * (t + t2) (t2 NULL: the single-term form)
int hxa_resid2_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, const hxa_h *t2, long ldt,
                               const float *gate, const float *shift, const float *scale, const float *w, float eps,
                               hxa_h *h, long ldh, hipStream_t st);
// the same with np (0, 1, 2 or 4) pending fp16 terms, term j at t + j tz: x += gate * ((t0 + t1) + (t2 + t3))
int hxa_residn_norm_mod_launch(float *x, long ldx, int T, int D, const hxa_h *t, int np, long tz, long ldt,
                               const float *gate, const float *shift, const float *scale, const float *w, float eps,
                               hxa_h *h, long ldh, hipStream_t st);
int hxa_norm_mod_launch(const float *x, long ldx, int T, int D, const float *shift, const float *scale, const float *w,
                        float eps, hxa_h *h, long ldh, hipStream_t st);
// per-head RMSNorm * gain (+ RoPE on pairs (d, d+64)) in place for ntens tensors sharing a layout
int hxa_rmsrope_launch(hxa_h *q0, hxa_h *q1, const float *g0, const float *g1, long ldq, int T, int H, const float *cosT,
                       const float *sinT, int ttab, hipStream_t st);
// x[t][c] += gate[c] * (t1 + t2)
int hxa_resadd2_launch(float *x, long ldx, const hxa_h *t1, const hxa_h *t2, long ldt, int T, int D, const float *gate,
                       hipStream_t st);
// x[t][c] += gate[c] * (sum of np = 2 or 4 fp16 terms, term j at t + j tz, summed ((t0 + t1) + (t2 + t3)))
int hxa_resaddn_launch(float *x, long ldx, const hxa_h *t, int np, long tz, long ldt, int T, int D, const float *gate,
                       hipStream_t st);

// layout conversions between the reference's crouton tiles and row-major device buffers
int hxa_x32_to_rows_launch(const float *tiles, float *x, int R, int C, hipStream_t st);
int hxa_rows_to_x32_launch(const float *x, float *tiles, int R, int C, hipStream_t st);
int hxa_h16_to_rows_launch(const hxa_h *tiles, hxa_h *a, long lda, int R, int C, hipStream_t st);
int hxa_rows_to_h16_launch(const hxa_h *a, long lda, hxa_h *tiles, int R, int C, int transposed, hipStream_t st);
int hxa_cs_to_rows_launch(const float *tiles, float *rows, int T, hipStream_t st);  // [slab][2][32][32] -> [T][64]

// synthetic data (counter-based hash RNG; deterministic for a seed)
int hxa_fill_normal_launch(void *dst, int dtype, size_t n, uint64_t seed, float mean, float std, hipStream_t st);
int hxa_fill_uniform_int_launch(void *dst, int bits, size_t n, uint64_t seed, int lo, int hi, hipStream_t st);
int hxa_fill_const_launch(void *dst, int dtype, size_t n, float v, hipStream_t st);

// caller-side glue (phone/animad.cpp)
// sig[0..3] = {s0, s1, s1 - s0, 0} on the stream (the DiT step's sigma values)
int hxa_set_sigma_launch(float *sig, float s0, float s1, hipStream_t st);
int hxa_copy_f32_launch(const float *src, float *dst, int n, hipStream_t st);
int hxa_patchify_launch(const float *lat, int B, int Cc, int H, int W, float *tok, hipStream_t st);
// patch embed straight from the latent: x + (b * xrows + tk) * N <- the patchified token tk of image b times Wemb^T
// (Wemb [N][4 Cc] fp16), all B images in one launch
// side (optional): a GEMV run in workgroups appended to the embedding's grid (the DiT step's block-0 modulation)
int hxa_patch_embed_launch(const float *lat, int B, int Cc, int H, int W, const hxa_h *Wemb, int N, float *x, int xrows,
                           hipStream_t st, const HxaSideGemv *side = nullptr);
// stacked GEMV: y[(n / per) * ostride + r + (r >= split ? gap : 0)] = sum_k act(x[k]) W[n][k], r = n % per;
// K % 256 == 0, K <= 4096; act 1 = SiLU on the input
int hxa_modgemv_launch(const float *x, int K, const hxa_h *W, long N, float *y, int per, long ostride, int split, int gap,
                       int act, hipStream_t st);
// GEMV of M <= 8 rows (one wave per output; output index n -> n + gap for n >= split); act 0 none, 1 SiLU on the
// input, 2 the input row is the timestep sinusoid of t = x[0] at width K (M 1); more rows: HXA_E_ARG
int hxa_linear_f32_launch(const float *x, long ldx, int M, int K, const hxa_h *W, int N, float *y, long ldy, int act,
                          const float *bias, int split, int gap, hipStream_t st);
// the same with fp32 weights W [N][K] (8-byte aligned)
int hxa_linear_w32_launch(const float *x, long ldx, int M, int K, const float *W, int N, float *y, long ldy, int act,
                          const float *bias, int split, int gap, hipStream_t st);
// final layer over B images of T image tokens (image b's rows start at b*xrows); dtp == NULL: lat = v,
// else lat += (*dtp) * v (Euler step). Wf4: the [4 Cc][D] weights k-tiled by 4, [D/4][4 Cc][4] (hxa_ktile4_launch).
// normw != NULL: RMSNorm * normw instead of LN (the MOSS head); x0rows / zrows != NULL: write the token rows
// x0rows[t][o] = zrows[t][o] - v (rapid-moss) instead of the latent. w32: Wf4 holds fp32 weights
int hxa_final_launch(const float *x, int B, int T, int xrows, int D, const float *shift, const float *scale,
                     const void *Wf4, int Cc, int H, int W, float *lat, const float *dtp, hipStream_t st,
                     const float *normw = nullptr, float *x0rows = nullptr, const float *zrows = nullptr, int w32 = 0);
// W [N][K] fp16 (fp32) -> Wk [K/4][N][4]
int hxa_ktile4_launch(const hxa_h *W, int N, int K, hxa_h *Wk, hipStream_t st);
int hxa_ktile4_f32_launch(const float *W, int N, int K, float *Wk, hipStream_t st);
// the reference's own DiT glue: vector RMSNorm * w (fp16 w), G GEMVs with their own inputs, the rapid-moss latent mix +
// video embedding, and BN denorm + unpatchify of the x0 token rows
int hxa_rmsvec_launch(const float *x, int n, const hxa_h *w, float eps, float *y, hipStream_t st);
// group g of G: y + g*y_gs = act(x + g*x_gs) . (Wp[g / gpp] + w_off + (g % gpp)*w_gs)^T (+ bias); act 1 = SiLU
int hxa_ptr_gemv_launch(const float *x, long x_gs, int act, const hxa_h *const *Wp, int G, int gpp, long w_off, long w_gs,
                        int N, int K, const float *bias, float *y, long y_gs, hipStream_t st);
int hxa_grouped_gemv_launch(const float *x, long ldx, const hxa_h *W, int G, int N, int K, const float *bias, float *y,
                            long ldy, hipStream_t st);
// Wv [D][C4]: fp32 when w32, else fp16
int hxa_moss_embed_launch(const float *z, const float *x0, const float *Q, const void *Wv, int w32, const float *bv,
                          float *x, int B, int T, int xrows, int D, int C4, hipStream_t st);
int hxa_bn_unpatchify_launch(const float *x0, const float *mean, const float *var, int B, int Cc, int H, int W, float *lat,
                             hipStream_t st);
int hxa_quantize_launch(const float *W, int N, int K, int fmt, void *q, hxa_h *s, hipStream_t st);
int hxa_sinusoid_launch(const float *t, int n, int dim, float *out, hipStream_t st);
// low-res first steps (phone/animad.cpp:392-503, moss/mossrun/mossrun.cpp:278-313); sig: t, tn, tn - t on the device.
// x_low [BC][H/f][W/f] from the full-res noise and clean estimate [BC][H][W]
int hxa_lowres_pool_launch(const float *nfull, const float *dhat, long BC, int H, int W, int f, const float *sig,
                           float *xlow, hipStream_t st);
// the low-res velocity -> dhat (upsampled clean estimate) and the Euler step lat += (tn - t) v of the velocity that lands
// it on (1 - tn) dhat + tn noise
int hxa_lowres_velocity_launch(const float *xlow, const float *vlow, float *lat, const float *nfull, float *dhat, long BC,
                               int H, int W, int f, const float *sig, hipStream_t st);
// MOSS: token rows [B][H*W][C4] -> 2 x 2x2 mean [B][(H/2)*(W/2)][C4]; bilinear 2x of token rows [B][h*w][C4]
int hxa_moss_pool2_launch(const float *z, int B, int H, int W, int C4, float *zl, hipStream_t st);
int hxa_upsample2_rows_launch(const float *src, int B, int h, int w, int C4, float *dst, hipStream_t st);

// weight-file import (device memory in and out): fp16 crouton tiles of a [K][N] matrix (export_all.py:7-8), or q8
// records (export_all.py:10-18; record k-blocks >= nkb_main to k group lora_g + ...), -> rows row0.. of a k-tiled
// [K/32][ldn][32] pack matrix (+ the q8 scales [K/32][ldn])
int hxa_crouton_to_ktiled_launch(const void *src, int N, int K, void *dst, int row0, int ldn, hipStream_t st);
int hxa_q8rec_to_ktiled_launch(const void *rec, int N, int nkb, int kbt, void *q, void *s, int row0, int ldn, int nkb_main,
                               int lora_g, hipStream_t st);
// an Anima blkNN.bin in device memory -> a kind-0 GPU pack (D 2048, F 8192, DC 1024): woff[0..9] the byte offsets of
// sq sk sv so cq ck cv co m1 m2 (blk_wlayout.h order), woff[10] the gains; q8: q8 records, else fp16 crouton tiles
int hxa_anima_file_to_pack(const uint8_t *src, const long *woff, int q8, void *pack, hipStream_t st);
size_t hxa_anima_file_mat_bytes(int i, int q8);
// a MOSS blkNN.bin (moss/export_moss.py, HXA_MOSS_FILE_BYTES) in device memory -> a zeroed kind-2 pack (D 3072, F 8192,
// int8, the rapid-moss LoRA), queued on st
constexpr size_t HXA_MOSS_FILE_BYTES = 135397376;
int hxa_moss_file_to_pack(const uint8_t *src, void *pack, hipStream_t st);
// matrix shapes of a GPU block pack (see hxa_pack_layout); returns the matrix count
int hxa_pack_mats(int kind, int D, int F, int DC, int fa, int fm, int *N, int *K, int *fmt);

// the library's error record (hxa_last_error): sets it and returns code
int hxa_set_error(int code, const char *fmt, ...);
// device address of hxa_block_run_noalloc's static workspace on the current device (resolved once per device)
int hxa_noalloc_setup(void **out);

// hxa_block_run for a chain of blocks: pend_gate != NULL applies the previous block's pending MLP residual
// (x += pend_gate * (t1 + t2) from the workspace) in the first norm; defer != 0 leaves this block's MLP residual
// pending in t1 / t2
// fp16 partials of the MLP-down that a chained block leaves pending (t1 .. t1 + (n-1) BT D in its workspace)
int hxa_block_down_parts(const hxa_block_dims *d);
// ck_pre / cvt_pre (Anima blocks, no stage stop): the block's text k / v, computed before the chain
// (hxa_block_textkv_plan); the block then skips that projection. side: GEMVs (a later block's modulation) run with
// this block's kernels:
struct HxaBlockSide {
  HxaSideGemv attn;  // in attn_wgs workgroups appended to the self-attention launch (HxaAttn::side; batch 1)
  int attn_wgs = 0;
  HxaSideGemv qkv, up;  // with the qkv / MLP-up projection (HxaGemm::side; N == 0: none)
};
int hxa_block_run_chained(const hxa_block_dims *d, const void *pack, float *x, const void *ctx, const float *mod,
                          const float *cosT, const float *sinT, void *ws, int stop, int *stage_us, int nstage,
                          void *stream, const float *pend_gate, int defer, const hxa_h *ck_pre = nullptr,
                          const hxa_h *cvt_pre = nullptr, const struct HxaBlockSide *side = nullptr);
int hxa_block_textkv_plan(const hxa_block_dims *d, const void *pack, const void *ctx, hxa_h *ck, hxa_h *cvt,
                          HxaGemm *g, HxaWeight *w);
