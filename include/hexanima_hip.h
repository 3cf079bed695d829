/* hexanima_hip.h -- C-ABI of the MI355X (gfx950) DiT block runner, libhexanima_hip.so.
 *
 * The first section is the drop-in boundary: the same three symbols and C signatures as the reference's FastRPC
 * block interface, so a megarun/mossrun-style caller links against this library instead of the DSP stub.
 * Everything else is the device-level interface used by the runner, the benchmark and the parity tests
 * (plain device pointers and sizes; no framework types).
 *
 * All functions return 0 on success or a negative status (see HXA_E_*); hxa_last_error() describes the last one.
 * A handle / stream is not thread-safe: calls on one handle must be serialised by the caller, as the reference's
 * single caller thread does (megarun.cpp:176-184).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint64_t remote_handle64; /* the reference's remote handle type (remote.idl) */

/* status codes; -1/-2/-5/-6/-7 keep the reference's *rc meanings (blk.c:110-127, :188) */
#define HXA_OK 0
#define HXA_E_RESOURCE (-1) /* device resources could not be acquired (VTCM/HMX acquire in the reference) */
#define HXA_E_LOCK (-2)
#define HXA_E_WEIGHTS (-5)  /* weight buffer not registered / unreadable (HAP_mmap_get(wfd) failure) */
#define HXA_E_NOBLOB (-6)
#define HXA_E_BLOB (-7)     /* blob not registered (HAP_mmap_get(bfd) failure) */
#define HXA_E_META (-10)    /* bad meta[]: ntok % 32 != 0, ntok > TMAX, offsets outside the registered buffers */
#define HXA_E_MODE (-11)    /* unsupported mode / format */
#define HXA_E_ARG (-12)     /* invalid argument (shape, alignment, null pointer) */
#define HXA_E_HIP (-13)     /* HIP runtime error */

/* ============================================================================================================
 * 1. Reference block-execution ABI
 * ============================================================================================================ */

/* replaces mega_open (hexagon/mega/mega_imp.c:16): creates a context on the current HIP device. uri is ignored. */
int mega_open(const char *uri, remote_handle64 *h);
/* replaces mega_close (mega_imp.c:18): releases every device buffer of the handle. */
int mega_close(remote_handle64 h);
/* replaces mega_block (hexagon/mega/blk.c:186, IDL mega.idl:10): runs one Anima DiT block.
 *   meta[]   : the reference enum of blk_meta.h:3-4 (byte offsets into the blob / weight buffer + params)
 *   wfd, bfd : keys of buffers registered with hxa_register (the reference's rpcmem fds)
 *   mod      : 9 x 2048 fp32 (shift, scale, gate per site), modlen = 73728
 *   times    : per-stage microseconds (TICK order of blk.c:136), times[24] = entry overhead; times[17..22], the
 *              reference's attention sub-phases (K^T / V setup, QK, PV, row scale, softmax wait, flush: g_acc of
 *              blk.c:178), are 0: attention is one fused kernel here, timed whole in its stage slot
 *   *rc      : 0 or a status code; the return value is 0 as in the reference.
 * meta[M_FIRST] uploads x / ctx / cos / sin from the blob to device-resident copies; meta[M_REL] writes x back
 * to the blob (x32 tiles). Weights are converted to the GPU layout and uploaded on first use, then stay resident.
 * meta[M_STOP] = n stops after n stages and writes the stage buffers (h,q,k,v,o,t,mid,ck,cv) back to the blob.
 * A call with times == NULL (or ntimes <= 0) that neither stops nor releases returns once its block is queued on the
 * handle's stream (mod has been copied by then); the next call's block follows it, and the releasing call waits for
 * the whole chain. An execution error of a queued block is reported by the next call that waits. Calls on one handle
 * must not overlap. */
int mega_block(remote_handle64 h, const int *meta, int nmeta, int wfd, int bfd, const uint8_t *mod, int modlen, int *times,
               int ntimes, int *rc);
/* the MOSS build of the same entry (moss/hexagon/mega/blk.c:269-281) with the MOSS meta enum
 * (moss/hexagon/mega/blk_meta.h:3-4): MODE 0, the DiT block with its rapid-moss LoRA (blk.c:234-259); the text side's
 * modes (1, 2, 10, 11, 20, 21, 30) return *rc = HXA_E_MODE. mod = 6 x 3072 fp32. libhexanima_moss.so exports it under
 * the reference's own name, mega_block (include/hexanima_moss.h). */
int mega_moss_block(remote_handle64 h, const int *meta, int nmeta, int wfd, int bfd, const uint8_t *mod, int modlen,
                    int *times, int ntimes, int *rc);

/* buffer registration: replaces rpcmem_alloc + fastrpc_mmap of the caller (megarun.cpp:100-119, :141-148).
 * kind: HXA_KIND_* below. The host memory must stay valid until hxa_unregister / mega_close. */
#define HXA_KIND_WEIGHTS_ANIMA 0 /* blkNN.bin of hexagon/mega/export_all.py (fp16 crouton or q8 records) */
#define HXA_KIND_BLOB 1          /* activation blob (offsets in meta[]) */
#define HXA_KIND_WEIGHTS_MOSS 2  /* blkNN.bin of moss/export_moss.py (q8 records, LoRA-B rows appended, LoRA-A
                                    matrices): converted to a kind-2 pack */
int hxa_register(remote_handle64 h, int fd, void *host_ptr, size_t bytes, int kind);
int hxa_unregister(remote_handle64 h, int fd);
/* replaces megarun's modulation thread (megarun.cpp:156-171) with GPU GEMVs: for the Anima weight buffers registered
 * under wfds[0..count), s = silu(emb) and per site (self-attn, cross-attn, MLP) mod[k][3 site .. 3 site + 2] =
 * lora + B_site (A_site s), from the modulation weights of each blkNN.bin (A [256][2048], B [6144][256] fp16 per site
 * at W_MODW, or WQ_MODW for a q8 file, told apart by the file size as megarun.cpp:97 does; blk_wlayout.h:14-20),
 * uploaded on first use and then resident. emb [2048], lora [6144] fp32 host; mod [count][9][2048] fp32 host, ready
 * to pass to mega_block block by block. */
int hxa_anima_modulation(remote_handle64 h, const int *wfds, int count, const float *emb, const float *lora, float *mod);

/* ============================================================================================================
 * 2. Device runtime
 * ============================================================================================================ */
const char *hxa_last_error(void);
const char *hxa_version(void);
int hxa_init(int device);
int hxa_malloc(void **p, size_t bytes);
int hxa_free(void *p);
int hxa_h2d(void *dst, const void *src, size_t bytes);
int hxa_d2h(void *dst, const void *src, size_t bytes);
int hxa_d2d(void *dst, const void *src, size_t bytes);
int hxa_memset(void *p, int value, size_t bytes);
int hxa_sync(void);
int hxa_stream_create(void **stream);
int hxa_stream_destroy(void *stream);
int hxa_stream_sync(void *stream);
int hxa_event_create(void **ev);
int hxa_event_destroy(void *ev);
int hxa_event_record(void *ev, void *stream);
int hxa_stream_wait_event(void *stream, void *ev); /* later work on stream waits for ev */
int hxa_event_elapsed_ms(void *start, void *stop, float *ms);
int hxa_device_info(int *num_cu, int *clock_khz, size_t *mem_bytes, char *name, int name_len);
/* HIP graph capture of a stream, for callers that replay launch sequences (and the tests of the capture-safe entry
 * points); no counterpart in the reference. mode 0 global, 1 thread-local, 2 relaxed (hipStreamCaptureMode);
 * end_capture instantiates the captured graph into *exec, launched with hxa_graph_launch. */
int hxa_stream_begin_capture(void *stream, int mode);
int hxa_stream_end_capture(void *stream, void **exec);
int hxa_graph_launch(void *exec, void *stream);
int hxa_graph_exec_destroy(void *exec);
/* Shader-clock record, for measurement; no counterpart in the reference. kind 0: every GEMM launched after this call
 * (hxa_gemm*, the block runner's and DiT's projections, graphs captured after it) writes, per workgroup w < nrec,
 * four uint64 at rec[4w .. 4w+3] (device memory): s_memtime and s_memrealtime when the workgroup starts, both again
 * when its main loop ends; kind 1: the same for attention launches. s_memtime counts shader-clock cycles and
 * s_memrealtime a constant 100 MHz clock, so (c1-c0)/(r1-r0) x 100 MHz is the clock the workgroup ran at. Each launch
 * overwrites the records of its workgroup ids (the launch's flat workgroup index). rec NULL: off (the default). */
int hxa_clock_record(int kind, void *rec, long nrec);

/* ============================================================================================================
 * 3. Kernels (device pointers; stream NULL = the null stream)
 * ============================================================================================================ */
#define HXA_W_F16 0 /* w [N][K] fp16 */
#define HXA_W_Q8 1  /* q [N][K] int8, s [K/32][N] fp16; value f16(q*s) */
#define HXA_W_KTILED 16 /* OR'ed into a format: weights stored k-tiled, [K/32][N][32 values] (q4: 16 bytes per row and
                           tile); each 32-deep k step of the whole matrix is contiguous in memory (scales unchanged) */
#define HXA_W_Q4 2  /* q [N][K/2] (k0+2j at bits 4j, k0+2j+1 at bits 16+4j of each 32-bit word; nibble = q+8),
                       s [K/32][N] fp16, optional z [K/32][N]: value f16(nibble*s + z), z NULL: f16((nibble-8)*s) */
#define HXA_EPI_STORE 0
#define HXA_EPI_GELU_TANH 1
#define HXA_EPI_GELU_ERF 2
#define HXA_EPI_RESADD 3
#define HXA_EPI_STORE_T 4
#define HXA_EPI_SITU 5
#define HXA_EPI_PARTIAL 6
#define HXA_EPI_RESADD_SPLIT2 7
#define HXA_EPI_PARTIAL_F32 8

/* out = epi(A[M][K] . W[N][K]^T); replaces gemm_run_ex / gemm_run_geo (hexagon/mega/gemm2.c:96-141).
 * STORE: out[m][n] (ldo); with out_t != NULL the columns n >= split_col go to out_t[n - split_col][m] (ldo_t).
 * STORE_T: out[n][m]. GELU_*: out = f16(gelu(f16(acc))). RESADD: x[m][n] += gate[n] f16(acc) (x fp32, ldx).
 * GELU_ERF looks up a per-device table of f16(a * 0.5 * erfc(a / sqrt 2)), built by the first such launch on a
 * device, which waits for its stream once (a launch under stream capture before then evaluates erfc instead).
 * SITU: W rows interleaved per 32 (up_j, gate_j), out[m][j*32+c] (moss gemm2.c mode 5).
 * PARTIAL: ksplit slices, out[z*out_zstride + m*ldo + n] = f16(partial z) (blk.c:172-174).
 * PARTIAL_F32: the same slices unrounded, ((float *)out)[z*out_zstride + m*ldo + n] (out 16-byte aligned, ldo % 4 == 0);
 * hxa_sum_partials adds them (hxa_linear's split-K form).
 * RESADD_SPLIT2 (ksplit 1, K % 128 == 0): x[m][n] += gate[n] (f16(first K/2) + f16(second K/2)), the split-K
 * down projection and its residual (blk.c:172-174, kern.c:330-339) in one launch. */
int hxa_gemm(const void *A, long lda, int M, int fmt, const void *w, const void *s, const void *z, int N, int K,
             int ksplit, int epi, void *out, long ldo, long out_zstride, float *x, long ldx, const float *gate,
             void *out_t, long ldo_t, int split_col, void *stream);
/* same, with an explicit tile shape (tests / tuning). waves per workgroup 4 (0 = 4): bm x bn in {192x256, 192x192,
 * 192x128, 256x128, 128x256, 128x128, 64x128, 128x64}; 8: {192x256, 192x128, 128x256, 128x128}; 9, the ping-pong
 * kernel: {256x256, 192x256, 128x256, 128x128 (not int4)}. int4 weights need bn >= 128, SiTU bn % 128 == 0. */
int hxa_gemm_tile(const void *A, long lda, int M, int fmt, const void *w, const void *s, const void *z, int N, int K,
                  int ksplit, int epi, void *out, long ldo, long out_zstride, float *x, long ldx, const float *gate,
                  int bm, int bn, int waves, void *stream);
/* The plain linear out = f16(A[M][K] . W[N][K]^T) [M][ldo] (gemm_run_ex with STORE, hexagon/mega/gemm2.c:96-141;
 * with int8 / int4 weights the W8A16 / W4A16 linear): one hxa_gemm launch, or, where the tile model favours it (long K,
 * few output tiles: hxa_linear_split_k > 1), that many K slices as fp32 partials in ws (PARTIAL_F32) followed by
 * hxa_sum_partials. The output is rounded to fp16 once either way; only the fp32 summation order differs. ws:
 * hxa_linear_ws_bytes(M, N, K, fmt) bytes, 16-byte aligned (NULL or fewer bytes: the one-launch form). Calls that
 * share ws must not overlap. */
int hxa_linear(const void *A, long lda, int M, int fmt, const void *w, const void *s, const void *z, int N, int K,
               void *out, long ldo, void *ws, long ws_bytes, void *stream);
int hxa_linear_split_k(int M, int N, int K, int fmt); /* 1, 2 or 4 */
long hxa_linear_ws_bytes(int M, int N, int K, int fmt);
/* out[m][n] = f16(p[m*ldp + n] + p[zstride + m*ldp + n] + ... ) over nslice fp32 slices, added in slice order
 * (N % 8 == 0, ldp % 4 == 0, ldo % 8 == 0, p and out 16-byte aligned). Second step of hxa_linear's split form; the
 * reference's linears run unsplit, so it has no counterpart there. */
int hxa_sum_partials(const float *p, int nslice, long zstride, long ldp, int M, int N, void *out, long ldo,
                     void *stream);
/* The tile hxa_gemm chooses for these sizes, weight format (HXA_W_*, KTILED ignored), split and epilogue
 * (norm_cols > 0: hxa_gemm_headnorm's head-normed columns): *bm x *bn with *waves per workgroup (9: the ping-pong
 * kernel) and *rounds of workgroups over the GPU's CUs. Returns 0, or the error hxa_gemm would return for these
 * sizes. No counterpart in the reference (its GEMM has one tile); for tuning and benchmarks. */
int hxa_gemm_pick(int M, int N, int K, int fmt, int ksplit, int epi, int norm_cols, int *bm, int *bn, int *waves,
                  int *rounds);
/* out = f16(A[M][K] . W[N][K]^T) with the per-head norm fused into the store (blk.c:158-160, :164-167,
 * kern.c:163-197): columns [0, norm_cols) (whole heads of 128) become f16(RMSNorm(f16 value) * gain), gain0 for
 * columns < gain_split, gain1 above; with cosT / sinT [ttab][64] also RoPE on pairs (d, d+64) at token m % ttab.
 * Columns >= split_col go transposed to out_t[n - split_col][m] (out_t NULL: none). N, norm_cols, split_col: multiples
 * of 128. Same values as hxa_gemm + hxa_rmsrope. */
int hxa_gemm_headnorm(const void *A, long lda, int M, int fmt, const void *w, const void *s, const void *z, int N, int K,
                      void *out, long ldo, void *out_t, long ldo_t, int split_col, int norm_cols, const float *gain0,
                      const float *gain1, int gain_split, const float *cosT, const float *sinT, int ttab, void *stream);
/* attention over heads of 128 (blk.c:54-91): q [T][ldq], k [NKV][ldk], vt [H*128][ldvt] (V transposed),
 * o [T][ldo]; keys >= nvalid masked; batch images at element strides qb/kb/vb/ob; ldk < 2^24, ldvt < 2^23. */
int hxa_attention(const void *q, long ldq, const void *k, long ldk, const void *vt, long ldvt, void *o, long ldo, int T,
                  int NKV, int nvalid, int H, int batch, long qb, long kb, long vb, long ob, void *stream);
/* The cross-attention site's q projection fused with its attention (blk.c:163-169): q = f16(RMSNorm(f16(h W^T)) * gain)
 * per head of 128 (gain [128] fp32 with 1/sqrt(128) folded in, no RoPE; kern.c:163-197), then per head
 * o = attention(q, k, v) over the nvalid of NKV keys of the query row's image (rows [b T, (b+1) T) are image b):
 * k [NKV][ldk] at element offset b*kb, vt [N][ldvt] (V transposed) at column offset b*vb, o [M][ldo]. fp16 weights
 * (fmt HXA_W_F16, optionally | HXA_W_KTILED); T % 128 == 0, N % 128 == 0. The same values as hxa_gemm_headnorm
 * followed by hxa_attention, up to the softmax's summation order. The reference runs it as two stages. */
int hxa_cross_attention_fused(const void *h, long ldh, int M, int T, int fmt, const void *w, int N, int K,
                              const float *gain, const void *k, long ldk, const void *vt, long ldvt, int NKV, int nvalid,
                              long kb, long vb, void *o, long ldo, void *stream);
/* h = f16(norm(x) * (1 + scale) [* w] + shift); LN when w == NULL (kern.c:38-65), RMS otherwise (moss kern.c:353) */
int hxa_norm_mod(const float *x, long ldx, int T, int D, const float *shift, const float *scale, const float *w,
                 float eps, void *h, long ldh, void *stream);
/* the same after applying the previous site's gated residual, x += gate * t (kern.c:320-328; t fp16 [T][ldt]),
 * with x written back: one pass over x for the residual and the next site's norm */
int hxa_resadd_norm_mod(float *x, long ldx, int T, int D, const void *t, long ldt, const float *gate, const float *shift,
                        const float *scale, const float *w, float eps, void *h, long ldh, void *stream);
/* per-head RMSNorm * gain (+ RoPE when cosT != NULL) in place on q0 (and q1 when not NULL) (kern.c:163-197);
 * cos/sin [ttab][64], row t % ttab */
int hxa_rmsrope(void *q0, void *q1, const float *g0, const float *g1, long ldq, int T, int H, const float *cosT,
                const float *sinT, int ttab, void *stream);
/* x += gate * (t1 + t2) (kern.c:330-339) */
int hxa_resadd2(float *x, long ldx, const void *t1, const void *t2, long ldt, int T, int D, const float *gate,
                void *stream);
/* int8 / int4 weight w [N][K] (scales s [K/32][N], q4 mins z or NULL) -> fp16 k-tiled out [K/32][N][32]: the values
 * f16(q*s) (q4: f16(nibble*s + z), or f16((nibble-8)*s) without z) that hxa_gemm's main loops feed their MFMAs,
 * written once to memory (the block runner's dequantisation pass; gemm2.c:19-35 dq_tile, moss gemm2.c:39-56
 * dq4_tile). fmt may carry HXA_W_KTILED for a k-tiled source. out: 2 N K bytes, 16-byte aligned. */
int hxa_dequant(int fmt, const void *w, const void *s, const void *z, int N, int K, void *out, void *stream);
/* synthetic data: dtype 0 fp32, 1 fp16 */
int hxa_fill_normal(void *dst, int dtype, size_t n, uint64_t seed, float mean, float std, void *stream);
int hxa_fill_uniform_int(void *dst, int bits, size_t n, uint64_t seed, int lo, int hi, void *stream);
int hxa_fill_const(void *dst, int dtype, size_t n, float v, void *stream);
/* q8 / q4 quantisation of fp32 W[N][K] (export_all.py:10-18 semantics, group 32, fp16 scales); fmt may carry
 * HXA_W_KTILED to write q k-tiled */
int hxa_quantize(const float *W, int N, int K, int fmt, void *q, void *s, void *stream);
/* crouton <-> row-major conversions (kern.h:5-8) */
int hxa_x32_to_rows(const float *tiles, float *x, int R, int C, void *stream);
int hxa_rows_to_x32(const float *x, float *tiles, int R, int C, void *stream);

/* ============================================================================================================
 * 4. GPU block packs and the device-level block (weights resident in HBM)
 * ============================================================================================================ */
/* A pack is one device allocation holding every weight of one block in the GPU layouts above, at offsets
 * given by hxa_pack_layout (each matrix: w, then s, then z, 256-byte aligned). Every matrix w of a pack is stored
 * k-tiled (HXA_W_KTILED): [K/32][N][32 values] (q4: [K/32][N][16 bytes]).
 * kind 0 (Anima structure): matrices qkv [3D][D], o [D][D], cq [D][D], ckv [2D][DC], co [D][D], w1 [F][D],
 *   w2 [D][F], then gain fp32 [4][128] (q/sqrt(128), k, cross q/sqrt(128), cross k).
 * kind 1 (MOSS structure): qkv [3D][D], o [D][D], ug [2F][D] (rows interleaved per 32: up_j, gate_j),
 *   down [D][F], then fp32 gq[128], gk[128], n1[D], n2[D].
 * kind 2 (MOSS + LoRA, moss/export_moss.py:34-58): as kind 1 with each projection's 128 scaled LoRA-B columns after
 *   K -- qkv [3D][D + 384] (q rows use columns [D, D+128), k rows [D+128, D+256), v rows [D+256, D+384), zero
 *   elsewhere), o [D][D + 128], ug [2F][D + 128], down [D][F + 128] -- then the LoRA-A matrices A_qkv [384][D],
 *   A_o [128][D] (fmt_attn), A_ug [128][D], A_dn [128][F] (fmt_mlp); the same vectors as kind 1.
 * fmt_attn applies to the attention matrices, fmt_mlp to the MLP ones (asym q4 not used in packs).
 * offs receives 3 offsets (w, s, z; -1 when absent) per matrix followed by the vector offset; returns bytes. */
long hxa_pack_layout(int kind, int D, int F, int DC, int fmt_attn, int fmt_mlp, long *offs, int noffs);

typedef struct {
  int kind;      /* 0 Anima, 1 MOSS, 2 MOSS with the rapid-moss LoRA (rank 128, moss/hexagon/mega/blk.c:238-259) */
  int D, H, F;   /* width, heads (x128), MLP width (MOSS: up and gate each F) */
  int C, DC;     /* context tokens per image and context width (Anima) */
  int T, batch;  /* tokens per image (padded to 32), images */
  int nvalid;    /* MOSS: valid tokens per image (joint attention key mask) */
  int fmt_attn, fmt_mlp;
  int gelu;      /* Anima MLP activation: 0 erf (reference block), 1 tanh */
  int round_ref; /* 1: the reference's rounding points for the gated projections, o and cross-o rounded to fp16 once,
                    the MLP-down in two K halves (blk.c:161-162, :168-169, :172-174). 0: the runner may split the
                    o / cross-o projections into two fp16 K-half partials and, with int8 / int4 weights at
                    1024 .. 4095 rows, the o / cross-o / MLP-down into four K-quarter partials (faster; each partial
                    is rounded to fp16). mega_block / mega_moss_block always run with 1; a stage stop implies it */
} hxa_block_dims;
/* bytes of the activation workspace of hxa_block_run. With int8 / int4 weights it includes the dequantisation slot:
 * one fp16 copy of the largest quantised projection that runs from fp16 -- at 1024 .. 4095 rows (batch*T) the cross
 * q, from 4096 rows all of them -- and for Anima blocks a second slot for the text k / v weight; at 1024 .. 4095 rows
 * the int8 / int4 attention-output and MLP-down projections run fused into four fp16 split-K partials instead. */
long hxa_block_ws_bytes(const hxa_block_dims *d);
/* One block, everything on the device:
 *   x    [batch*T][D] fp32 residual stream, updated in place
 *   ctx  [batch*C][DC] fp16 (Anima; NULL for MOSS)
 *   mod  Anima: 9 x D fp32 (site s: shift 3s, scale 3s+1, gate 3s+2); MOSS: 6 x D (shift_a, scale_a, gate_a,
 *        shift_f, scale_f, gate_f)
 *   cos, sin [T][64] fp32 (NULL: no RoPE)
 *   stop: stop after this many stages (0 = all); stage_us: per-stage microseconds (NULL: not timed). */
int hxa_block_run(const hxa_block_dims *d, const void *pack, float *x, const void *ctx, const float *mod, const float *cosT,
                  const float *sinT, void *ws, int stop, int *stage_us, int nstage, void *stream);
/* hxa_block_run without a workspace argument and without any allocation: the workspace is a static device array of
 * HXA_NOALLOC_WS_MAX bytes held by each GPU the library runs on until the process ends (one 1536-token image of the
 * 2B fp16 / q8 and 2.9B-class q8 blocks fits; hxa_block_ws_bytes larger than that is HXA_E_ARG, nothing launched).
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). All calls on one GPU share the array, so calls that overlap on
 * one GPU race; no stage timing. Otherwise as hxa_block_run (same kernels, same results). */
#define HXA_NOALLOC_WS_MAX (160L << 20)
int hxa_block_run_noalloc(const hxa_block_dims *d, const void *pack, float *x, const void *ctx, const float *mod,
                          const float *cosT, const float *sinT, int stop, void *stream);
/* stage buffers of the workspace: which 0 h, 1 q, 2 k, 3 vT ([D][batch*T]), 4 o, 5 t1, 6 mid, 7 ck, 8 cvT, 9 t2,
 * 10 the dequantisation slot (k-tiled [K/32][N][32] fp16 copies; *ld = 0: no row stride);
 * returns the device pointer and its row stride in elements (kind 2: h, o and mid rows carry the LoRA L columns
 * after their D / D / F activations, so their strides are D + 384, D + 128, F + 128) */
void *hxa_block_ws_buf(const hxa_block_dims *d, void *ws, int which, long *ld);

/* ============================================================================================================
 * 5. DiT runner (the process above the boundary: patch embed, timestep modulation, blocks, final layer, Euler)
 * ============================================================================================================ */
typedef struct {
  hxa_block_dims blk;   /* per-block shape (T = gh*gw tokens per image); kind 0 Anima, 1 MOSS (synthetic seeded
                           weights), 2 MOSS with the rapid-moss LoRA (form 1 only; zero weights until
                           hxa_dit_load_moss_block) */
  int nblocks;
  int lat_c, lat_h, lat_w; /* latent [C][H][W]; patch 2 */
  int temb;             /* sinusoid width of the timestep embedding (form 0: 256; form 1: D for Anima, 256 for MOSS) */
  int ntxt_in;          /* MOSS: text width before projection (0 = none) */
  int form;             /* glue around the blocks. 0: the benchmark configurations' (Linear . SiLU . Linear of the
                           sinusoid to dense per-block [6D][D] modulation, LN final layer, Euler steps).
                           1: the reference's own. Anima (phone/animad.cpp:424-492, megarun.cpp:156-171): emb =
                           RMSNorm(sinusoid_D(t)) * w, lora = L2 silu(L1 sinusoid_D(t)) [3D], per block and site
                           mod = lora + B (A silu(emb)) with A [256][D], B [3D][256], final (shift, scale) =
                           F2 (F1 silu(emb)) + lora[0 : 2D]. MOSS, the rapid-moss sampler (mossrun.cpp:255-343):
                           time MLP with biases, shared block modulation and head modulation, per step x_in = z + Q x0
                           per token, video embedding with bias, the blocks, RMS head, x0 = z - v
                           (hxa_dit_moss_step); hxa_dit_get_latent returns the BN-denormalised x0. */
} hxa_dit_cfg;
int hxa_dit_create(const hxa_dit_cfg *cfg, uint64_t seed, void **dit);
int hxa_dit_destroy(void *dit);
/* set latents [batch][C][H][W] fp32 and the context [batch][C][DC] fp32 (host pointers) */
int hxa_dit_set_inputs(void *dit, const float *lat, const float *ctx);
int hxa_dit_get_latent(void *dit, float *lat);
/* one Euler step x <- x + (sigma_next - sigma) v(x, sigma); use_graph 1 replays a captured HIP graph */
int hxa_dit_step(void *dit, float sigma, float sigma_next, int use_graph);
/* the velocity v(x, sigma) of the current latent into v [batch][C][H][W] (host), without updating x */
int hxa_dit_velocity(void *dit, float sigma, float *v);
/* one step of the rapid-moss sampler (moss/mossrun/mossrun.cpp:307-334) for a MOSS DiT in form 1, with the step's
 * time code: x_in = z + Q x0, v = head(blocks(embed(x_in), text)), x0 = z - v; the latent set by hxa_dit_set_inputs
 * is the noise z, and x0 starts at 0 */
int hxa_dit_moss_step(void *dit, float code, int use_graph);
/* Low-res first steps (phone/animad.cpp:392-503). One Euler step from sigma to sigma_next whose velocity comes from the
 * DiT run on a latent downsampled by `factor` (a quarter of the tokens at 2): with the latent of the first low-res step
 * after hxa_dit_set_inputs taken as the noise n and dhat the last clean estimate (0 at first),
 * x_low = (1 - sigma) mean_fxf(dhat) + sigma sum_fxf(n) / factor; v_low = DiT(x_low, sigma);
 * dhat = bilinear_up(x_low - sigma v_low) (half-pixel centres); the latent becomes x + (sigma_next - sigma) v with
 * v = (x - ((1 - sigma_next) dhat + sigma_next n)) / (sigma - sigma_next), i.e. (1 - sigma_next) dhat + sigma_next n.
 * Low-res steps come first. A factor the latent does not divide into 2x2 patches, or whose token count is not a
 * multiple of 32, runs a full-resolution step instead, as the reference does. Anima-structure DiTs (either form). */
int hxa_dit_step_lowres(void *dit, float sigma, float sigma_next, int factor, int use_graph);
/* MOSS low-res first steps (moss/mossrun/mossrun.cpp:288-313): a rapid-moss step on the half-size token grid, from the
 * noise pooled 2x2 (2 x the mean) and its own clean estimate (0 at first), image RoPE positions times rope_scale
 * (MOSS_LOWSCALE, 2 in the reference); the first hxa_dit_moss_step after them starts from that clean estimate
 * upsampled 2x (bilinear, half-pixel centres). An odd token grid runs a full-resolution step instead. */
int hxa_dit_moss_step_lowres(void *dit, float code, float rope_scale, int use_graph);
/* copies of the device weights for checking (host may be NULL to query the size; returns bytes):
 *   which in [0, nblocks): block pack `which`
 *   which in [nblocks, 2 nblocks): modulation weights of block which-nblocks, fp16 [6D][D]
 *     (form 1 Anima: A [3 x 256][D] then B [3][3D][256]; MOSS: one shared [6D][D] matrix, which == nblocks)
 *   which == 2 nblocks: glue, fp16, concatenated: x_embed [D][4C], t_embed [D][temb], final_mod [2D][D],
 *     final_linear [4C][D], then (MOSS only) text_proj [D][ntxt_in].
 *     Form 1 Anima: x_embed [D][4C], t_l1 [D][D], t_l2 [3D][D], f1 [256][D], f2 [2D][256], final_linear [4C][D],
 *     t_norm [D]; form 1 MOSS: head_mod [2D][D], text_proj [D][ntxt_in]
 *   which == 2 nblocks + 1 (form 1 MOSS): fp32 b_video [D], b_t0 [D], b_t2 [D], b_smod [6D], b_hmod [2D],
 *     final_norm [D], latent_mix Q [4C][4C], bn_mean [4C], bn_var [4C], video_embed [D][4C], t0 [D][256], t2 [D][D],
 *     final_linear [4C][D] (the matrices the reference keeps fp32, moss/export_glue.py:7-12) */
long hxa_dit_export(void *dit, int which, void *host, size_t bytes);
/* the inverse of hxa_dit_export: overwrite section `which` with host bytes of the same layout and size (bytes must be
 * the size hxa_dit_export reports). Complete when the call returns; later steps (captured graphs included) use it. */
int hxa_dit_import(void *dit, int which, const void *host, size_t bytes);
/* Real weights into the reference form (form 1) of the DiT runner; each upload is complete when the call returns and
 * later steps (captured graphs included) use it. Errors: HXA_E_MODE (another form or kind), HXA_E_WEIGHTS (a file that
 * does not parse, or whose shapes are not the DiT's).
 * hxa_dit_load_block: block k from the bytes of an Anima blkNN.bin -- the buffer megarun registers with fastrpc_mmap
 *   (megarun.cpp:100-119) and this library's mega_block takes through hxa_register -- fp16 or q8 (told apart by size,
 *   blk_wlayout.h:3-20; the DiT's fmt_attn / fmt_mlp must match), its adaLN modulation weights included. Needs the
 *   Anima shape: D 2048, 16 heads, MLP 8192, context width 1024.
 * hxa_dit_load_anima_glue: the caller-side glue of animad (animad.cpp:424-492) from small.bin (phone/extract_small.py:
 *   u32 count; per tensor u32 name length, name, u32 ndim, i64 dims, fp16 data): t_embedder.1.linear_1 / _2,
 *   t_embedding_norm, x_embedder.proj.1 (its 4 mask-channel columns dropped: they multiply zeros, animad.cpp:446),
 *   final_layer.adaln_modulation.1 / .2 and final_layer.linear; other tensors are ignored.
 * hxa_dit_load_moss_glue: the MOSS DiT glue from glue.bin (MGL1, moss/export_glue.py:1-22), in the file's storage types
 *   (fp32 time MLP, video embedding, head linear and vectors; fp16 modulation matrices); rope.bands rebuilds the RoPE
 *   tables; step_codes stays with the caller (the code argument of hxa_dit_moss_step). */
int hxa_dit_load_block(void *dit, int k, const void *blk, size_t bytes);
/* block k of a MOSS DiT of LoRA blocks (blk.kind 2, form 1, D 3072, 24 heads, MLP 8192, int8) from the bytes of a MOSS
 * blkNN.bin (moss/export_moss.py; the buffer mossrun registers, 135397376 bytes), through the same conversion as
 * mega_moss_block's registered weights. Such a DiT starts with zero weights in every block. */
int hxa_dit_load_moss_block(void *dit, int k, const void *blk, size_t bytes);
int hxa_dit_load_anima_glue(void *dit, const void *small_bin, size_t bytes);
int hxa_dit_load_moss_glue(void *dit, const void *glue_bin, size_t bytes);
void *hxa_dit_stream(void *dit);

#ifdef __cplusplus
}
#endif
