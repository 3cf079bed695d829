// DiT runner: the layer directly above the block boundary. It owns every weight of a synthetic DiT in HBM
// (GPU block packs + glue), and runs one flow-matching Euler step entirely on the device:
//   timestep sinusoid -> t-embedding -> per-block adaLN modulation (megarun.cpp:156-171 role; animad.cpp:424-431)
//   patch embed (animad.cpp:447-452: patchify read straight from the latent by the x_embedder) [MOSS: + text
//   projection, joint token layout]
//   blocks 0..n-1 (hxa_block_run)
//   final adaLN + linear + unpatchify (animad.cpp:474-492) fused with the Euler update x += (s' - s) v
// A step is captured once into a HIP graph and replayed; sigma values are read from device memory so one graph
// serves every step.
// Two forms of the glue around the blocks (hxa_dit_cfg.form): 0, the benchmark configurations' (a 256-wide sinusoid,
// Linear . SiLU . Linear to dense per-block modulation, LN final layer); 1, the reference's own -- Anima: the
// RMSNorm'd 2048-wide sinusoid and its LoRA MLP (animad.cpp:424-431), low-rank per-block modulation
// (megarun.cpp:156-171) and final adaLN (animad.cpp:475-479); MOSS: the time MLP with biases, shared block and head
// modulation (mossrun.cpp:255-264), the rapid-moss sampler's latent mix and video embedding, the RMS head and
// x0 = z - v (mossrun.cpp:307-334), BN denorm + unpatchify of the result (mossrun.cpp:339-343). The reference form
// keeps each glue tensor in the reference's storage type: fp16 for Anima (phone/extract_small.py) and for the MOSS
// modulation matrices, fp32 for the MOSS time MLP, video embedding and head (moss/export_glue.py:7-12).
// Real weights come in through hxa_dit_load_block (Anima blkNN.bin), hxa_dit_load_anima_glue (small.bin) and
// hxa_dit_load_moss_glue (glue.bin, MGL1).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <map>
#include <string>
#include <vector>

#include "../../include/hexanima_hip.h"

#include "hxa_common.h"
#include "kernels.h"

namespace {

struct Dit {
  hxa_dit_cfg cfg{};
  hxa_block_dims bd{};
  int Timg = 0, Ttot = 0, ntxt = 0;
  hipStream_t st = nullptr;
  std::vector<void *> packs;
  // Anima blocks whose text k / v the chain computes up front (hxa_block_textkv_plan): block k's ck [B C][D] at
  // tkv + 2 B C D k, its cvt [D][B C] right after; the grouped launch's parameters on the device
  hxa_h *tkv = nullptr;
  void *tkv_par = nullptr;
  int tkv_tiles = 0, tkv_fmt = 0;
  long pack_bytes = 0;
  hxa_h *modw_all = nullptr;  // one allocation: every block's modulation weights, stacked
  std::vector<hxa_h *> modw;  // Anima: per block [6D][D]; MOSS: one shared [6D][D]
  hxa_h *glue = nullptr;      // fp16 glue matrices (layout per form below)
  long glue_elems = 0;
  hxa_h *Wemb = nullptr, *L1 = nullptr, *Lf = nullptr, *Wfin = nullptr, *Wtxt = nullptr;
  hxa_h *Wfin4 = nullptr;  // Wfin k-tiled by 4 ([D/4][4C][4]), what the final layer's kernel reads
  float *lat = nullptr, *vel = nullptr, *x = nullptr, *sinus = nullptr, *cvec = nullptr;
  float *mods = nullptr, *fmod = nullptr, *sig = nullptr, *cosT = nullptr, *sinT = nullptr, *ones = nullptr;
  hxa_h *ctx16 = nullptr;  // Anima: [B*C][DC]; MOSS: text [B*ntxt][ntxt_in]
  void *ws = nullptr;
  long ws_bytes = 0;  // the block workspace, sized for the full-resolution pass
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  // form 1 (the reference's glue): fp16 matrices inside `glue`, fp32 vectors in `vec`, per-step vectors below
  int form = 0;
  hxa_h *Wl2 = nullptr, *F1 = nullptr, *F2 = nullptr, *tnorm = nullptr, *T2 = nullptr, *Wh = nullptr;
  // MOSS: b_video [D] | b_t0 [D] | b_t2 [D] | b_smod [6D] | b_hmod [2D] | final_norm [D] | Q [4C][4C] | bn mean,
  // var [4C] | video_embed [D][4C] | t0 [D][256] | t2 [D][D] | final_lin [4C][D], all fp32
  float *vec = nullptr;
  long vec_elems = 0;
  float *bve = nullptr, *b0 = nullptr, *b2 = nullptr, *bm = nullptr, *bh = nullptr, *nfin = nullptr, *Q = nullptr;
  float *bnm = nullptr, *bnv = nullptr;
  float *Wv32 = nullptr, *T0f = nullptr, *T2f = nullptr, *Wfin32 = nullptr;  // the fp32 matrices inside vec
  float *Wfin4f = nullptr;                                                    // Wfin32 k-tiled by 4
  float bands[16];  // MOSS RoPE bands (rope.bands of glue.bin); synthetic 10000^(-i/16) until one is loaded
  float *emb = nullptr, *a1 = nullptr, *lora = nullptr, *h1 = nullptr;  // t-embedding work vectors
  float *zrows = nullptr, *x0rows = nullptr;  // rapid-moss state: noise z and clean estimate x0, token rows [B*T][4C]
  long modw_block = 0;                        // elements of one block's modulation weights
  // low-res first steps (animad.cpp:392-503; mossrun.cpp:288-313), allocated at the first such step.
  // Anima: the noise of the first step and the last clean estimate [B][C][H][W], the low-res latent and velocity
  // [B][C][H/f][W/f]; MOSS: the low-res noise and clean estimate, token rows [B][(gh/2)*(gw/2)][4C].
  float *nfull = nullptr, *dhat = nullptr, *xlow = nullptr, *vlow = nullptr, *zl = nullptr, *x0l = nullptr;
  bool low_init = false;      // the low-res state holds this input's noise (reset by hxa_dit_set_inputs)
  bool moss_low_live = false; // MOSS: the last step was low-res, so a full step first upsamples its clean estimate
  static constexpr int MAXF = 8;
  float *cosL[MAXF + 1] = {}, *sinL[MAXF + 1] = {};  // RoPE tables of the 1/f grid
  double ropeL_scale = 0.0;                          // MOSS: the position scale cosL[2] / sinL[2] were built with
  hipGraphExec_t execL[MAXF + 1] = {};
  hipGraph_t graphL[MAXF + 1] = {};
};

thread_local char g_derr[256];
int dfail(int code, const char *m) {
  snprintf(g_derr, sizeof g_derr, "%s", m);
  return code;
}
#define DHIP(x)                                  \
  do {                                           \
    if ((x) != hipSuccess) return dfail(HXA_E_HIP, #x); \
  } while (0)
#define DTRY(x)                     \
  do {                              \
    int r__ = (x);                  \
    if (r__ != HXA_OK) return r__;  \
  } while (0)

// megarun.cpp:77-90: 3-axis split-half table over hd = 128 (22 zero t-angles, 21 h, 21 w; theta 10000)
void rope_anima(int gh, int gw, std::vector<float> &c, std::vector<float> &s) {
  const int dim_h = 128 / 6 * 2, dim_t = 128 - 2 * dim_h, nt = dim_t / 2, nh = dim_h / 2;
  std::vector<double> fh(nh);
  for (int i = 0; i < nh; i++) fh[i] = 1.0 / pow(10000.0, (2.0 * i) / dim_h);
  c.assign((size_t)gh * gw * 64, 0.0f);
  s.assign((size_t)gh * gw * 64, 0.0f);
  for (int tk = 0; tk < gh * gw; tk++) {
    const int hh = tk / gw, ww = tk % gw;
    for (int d = 0; d < 64; d++) {
      const double ang = d < nt ? 0.0 : d < nt + nh ? hh * fh[d - nt] : ww * fh[d - nt - nh];
      c[(size_t)tk * 64 + d] = (float)cos(ang);
      s[(size_t)tk * 64 + d] = (float)sin(ang);
    }
  }
}
// moss_ref.py:27-35: 4 axes x 16 bands; image (0, ntxt, h-(H-1)/2, w-(W-1)/2), text (0, i, 0, 0);
// padding rows get the identity rotation
// image positions times `scale`: 1 on the full grid, MOSS_LOWSCALE (2) on the low-res steps' (mossrun.cpp:190-201, :313)
void rope_moss(int H, int W, int ntxt, int Ttot, const float *bands, std::vector<float> &c, std::vector<float> &s,
               double scale = 1.0) {
  c.assign((size_t)Ttot * 64, 1.0f);
  s.assign((size_t)Ttot * 64, 0.0f);
  const int nimg = H * W;
  for (int tk = 0; tk < nimg + ntxt; tk++) {
    double pos[4];
    if (tk < nimg) {
      pos[0] = 0;
      pos[1] = ntxt;
      pos[2] = ((tk / W) - (H - 1) / 2.0) * scale;
      pos[3] = ((tk % W) - (W - 1) / 2.0) * scale;
    } else {
      pos[0] = 0;
      pos[1] = tk - nimg;
      pos[2] = pos[3] = 0;
    }
    for (int d = 0; d < 64; d++) {
      const double band = (double)bands[d % 16];
      const double ph = pos[d / 16] * band;
      c[(size_t)tk * 64 + d] = (float)cos(ph);
      s[(size_t)tk * 64 + d] = (float)sin(ph);
    }
  }
}


uint16_t f2h_host(float f) {
  // round-to-nearest-even fp32 -> fp16 (inputs are finite and in range)
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sgn = (x >> 16) & 0x8000u;
  x &= 0x7fffffffu;
  if (x >= 0x477ff000u) return (uint16_t)(sgn | 0x7c00u);
  if (x >= 0x38800000u) {
    uint32_t h = (((x >> 23) - 112u) << 10) | ((x & 0x7fffffu) >> 13);
    const uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sgn | h);
  }
  const float a = fabsf(f) * 16777216.0f;  // subnormal: units of 2^-24
  return (uint16_t)(sgn | (uint32_t)nearbyintf(a));
}

int init_pack(Dit &d, void *pack, uint64_t seed, float *tmp32) {
  const hxa_block_dims &b = d.bd;
  int N[8], K[8], fmt[8];
  const int n = hxa_pack_mats(b.kind, b.D, b.F, b.DC, b.fmt_attn, b.fmt_mlp, N, K, fmt);
  long offs[32];
  hxa_pack_layout(b.kind, b.D, b.F, b.DC, b.fmt_attn, b.fmt_mlp, offs, 32);
  char *base = (char *)pack;
  for (int i = 0; i < n; i++) {
    const size_t elems = (size_t)N[i] * K[i];
    if (fmt[i] == HXA_W_F16) {
      DTRY(hxa_fill_normal_launch(base + offs[3 * i], 1, elems, seed * 131 + i, 0.0f, 0.02f, d.st));
    } else {
      DTRY(hxa_fill_normal_launch(tmp32, 0, elems, seed * 131 + i, 0.0f, 0.02f, d.st));
      // packs hold k-tiled matrices; the i.i.d. fp16 fill above needs no layout
      DTRY(hxa_quantize_launch(tmp32, N[i], K[i], fmt[i] | HXA_W_KTILED, base + offs[3 * i],
                               (hxa_h *)(base + offs[3 * i + 1]), d.st));
    }
  }
  float *vec = (float *)(base + offs[3 * n]);
  const float qg = 1.0f / sqrtf(128.0f);
  if (b.kind == 0) {  // q/k norm gains 1; the q gains carry 1/sqrt(128) (export_all.py:31-32)
    DTRY(hxa_fill_const_launch(vec, 0, 128, qg, d.st));
    DTRY(hxa_fill_const_launch(vec + 128, 0, 128, 1.0f, d.st));
    DTRY(hxa_fill_const_launch(vec + 256, 0, 128, qg, d.st));
    DTRY(hxa_fill_const_launch(vec + 384, 0, 128, 1.0f, d.st));
  } else {
    DTRY(hxa_fill_const_launch(vec, 0, 128, qg, d.st));
    DTRY(hxa_fill_const_launch(vec + 128, 0, 128 + 2 * b.D, 1.0f, d.st));
  }
  return HXA_OK;
}

enum { MODE_EULER = 0, MODE_VELOCITY = 1 };

// form 1, Anima (animad.cpp:424-431, megarun.cpp:156-171, animad.cpp:475-479): tp = sinusoid_D(t), emb = RMSNorm(tp)
// * w, lora = L2 silu(L1 tp); per block and site mod = lora + B (A silu(emb)); final (shift, scale) =
// F2 (F1 silu(emb)) + lora[0 : 2D]
int record_prelude_anima_ref(Dit &d) {
  const int D = d.bd.D, nb = d.cfg.nblocks;
  hipStream_t st = d.st;
  DTRY(hxa_sinusoid_launch(d.sig, 1, D, d.sinus, st));
  DTRY(hxa_rmsvec_launch(d.sinus, D, d.tnorm, 1e-6f, d.emb, st));
  DTRY(hxa_linear_f32_launch(d.sinus, D, 1, D, d.L1, D, d.a1, D, 0, nullptr, 0, 0, st));
  DTRY(hxa_linear_f32_launch(d.a1, D, 1, D, d.Wl2, 3 * D, d.lora, 3 * D, 1, nullptr, 0, 0, st));
  // all blocks' A (s = silu(emb)) in one launch, then all blocks' and sites' B with their own h1 in one launch
  DTRY(hxa_linear_f32_launch(d.emb, D, 1, D, d.modw_all, nb * 768, d.h1, nb * 768, 1, nullptr, 0, 0, st));
  DTRY(hxa_grouped_gemv_launch(d.h1, 256, d.modw_all + (long)nb * 768 * D, nb * 3, 3 * D, 256, d.lora, d.mods, 3L * D, st));
  DTRY(hxa_linear_f32_launch(d.emb, D, 1, D, d.F1, 256, d.h1 + (long)nb * 768, 256, 1, nullptr, 0, 0, st));
  DTRY(hxa_linear_f32_launch(d.h1 + (long)nb * 768, 256, 1, 256, d.F2, 2 * D, d.fmod, 2 * D, 0, d.lora, 0, 0, st));
  return HXA_OK;
}
// form 1, MOSS (mossrun.cpp:255-264): e = sinusoid_256(code), a = T0 e + b0, b = T2 silu(a) + b2; shared block
// modulation Wm b + bm [6D], head modulation Wh b + bh [2D]
int record_prelude_moss_ref(Dit &d) {
  const int D = d.bd.D, temb = d.cfg.temb;
  hipStream_t st = d.st;
  DTRY(hxa_linear_w32_launch(d.sig, temb, 1, temb, d.T0f, D, d.a1, D, 2, d.b0, 0, 0, st));  // sinusoid in the GEMV
  DTRY(hxa_linear_w32_launch(d.a1, D, 1, D, d.T2f, D, d.emb, D, 1, d.b2, 0, 0, st));
  DTRY(hxa_linear_f32_launch(d.emb, D, 1, D, d.modw_all, 6 * D, d.mods, 6 * D, 0, d.bm, 0, 0, st));
  DTRY(hxa_linear_f32_launch(d.emb, D, 1, D, d.Wh, 2 * D, d.fmod, 2 * D, 0, d.bh, 0, 0, st));
  return HXA_OK;
}

// One pass of the blocks over a latent grid: the full one, or a low-res step's 1/f grid.
struct Pass {
  int lat_h = 0, lat_w = 0;        // latent height and width of this pass
  int Timg = 0, Ttot = 0;          // image tokens; rows per image in x (MOSS: image + text, padded to 32)
  hxa_block_dims bd{};             // the blocks' shape (T = Ttot)
  const float *cosT = nullptr, *sinT = nullptr;
  const float *lat_in = nullptr;   // the latent the patch embedding reads
  float *lat_out = nullptr;        // the final layer's output: the Euler-updated latent (dtp) or the velocity
  const float *dtp = nullptr;      // device pointer to tn - t for the Euler update; nullptr: lat_out = v
  float *zrows = nullptr, *x0rows = nullptr;  // rapid-moss: noise and clean estimate of this grid (token rows)
};

Pass full_pass(Dit &d, int mode) {
  Pass q;
  q.lat_h = d.cfg.lat_h;
  q.lat_w = d.cfg.lat_w;
  q.Timg = d.Timg;
  q.Ttot = d.Ttot;
  q.bd = d.bd;
  q.cosT = d.cosT;
  q.sinT = d.sinT;
  q.lat_in = d.lat;
  q.lat_out = mode == MODE_EULER ? d.lat : d.vel;
  q.dtp = mode == MODE_EULER ? d.sig + 2 : nullptr;
  q.zrows = d.zrows;
  q.x0rows = d.x0rows;
  return q;
}

int record_step(Dit &d, const Pass &ps) {
  const hxa_block_dims &b = ps.bd;
  const int B = b.batch, D = b.D, C4 = 4 * d.cfg.lat_c, temb = d.cfg.temb, nb = d.cfg.nblocks;
  hipStream_t st = d.st;
  const bool moss_ref = d.form == 1 && b.kind != 0;
  if (hxa_block_ws_bytes(&b) > d.ws_bytes) return HXA_E_ARG;  // a low-res pass needs no more than the full one
  if (d.form == 1) DTRY(b.kind == 0 ? record_prelude_anima_ref(d) : record_prelude_moss_ref(d));
  // Anima blocks at batch 1: block k+1's modulation, and in the last block the final layer's, runs with block k's
  // kernels in CUs their grids leave idle (the same rows, the same bits); block 0's runs in the patch embed launch.
  // Where the self attention leaves a quarter of the CUs idle (2B: 192 workgroups on 256 CUs) it takes all of it;
  // else (2.9B-class: every launch 240 workgroups) the qkv projection takes rows 0 .. 3D and the MLP up the rest
  // (HxaBlockSide). HXA_DIT_SIDE=0 when a step is recorded: every modulation in its own launches, for comparison.
  const char *side_env = getenv("HXA_DIT_SIDE");
  const bool side_on = d.form == 0 && b.kind == 0 && b.batch == 1 && hxa_side_k_ok(D) && !(side_env && atoi(side_env) == 0);
  const int side_wgs = side_on ? hxa_attn_idle_wgs(b.T, b.H, b.batch) : 0;
  const bool side_gemm = side_on && side_wgs == 0;
  if (d.form == 0) {
  // timestep embedding and modulation
  DTRY(hxa_linear_f32_launch(d.sig, temb, 1, temb, d.L1, D, d.cvec, D, 2, nullptr, 0, 0, st));  // sinusoid in the GEMV
  // every block's modulation in one launch over the stacked [nb][6D][D] weights: rows 0-2 -> site 0, rows 3-5 ->
  // site 2 of that block's [9][D] (site 1 keeps the identity modulation); MOSS: one shared [6D][D]
  if (b.kind == 0 && !side_on)
    DTRY(hxa_modgemv_launch(d.cvec, D, d.modw_all, (long)nb * 6 * D, d.mods, 6 * D, 9L * D, 3 * D, 3 * D, 1, st));
  else if (b.kind != 0)
    DTRY(hxa_modgemv_launch(d.cvec, D, d.modw_all, 6L * D, d.mods, 6 * D, 0, 6 * D, 0, 1, st));
  if (!side_on) DTRY(hxa_modgemv_launch(d.cvec, D, d.Lf, 2L * D, d.fmod, 2 * D, 0, 2 * D, 0, 1, st));
  }
  // patch embed (rapid-moss: latent mix + video embedding of the token rows) (+ MOSS text tokens)
  if (moss_ref)
    DTRY(hxa_moss_embed_launch(ps.zrows, ps.x0rows, d.Q, d.Wv32, 1, d.bve, d.x, B, ps.Timg, ps.Ttot, D, C4, st));
  else {  // (with side_on, block 0's modulation runs in workgroups appended to the patch embed)
    const HxaSideGemv m0{d.cvec, d.modw_all, 6L * D, d.mods, 6 * D, 9L * D, 3 * D, 3 * D, 1, D};
    DTRY(hxa_patch_embed_launch(ps.lat_in, B, d.cfg.lat_c, ps.lat_h, ps.lat_w, d.Wemb, D, d.x, ps.Ttot, st,
                                side_on ? &m0 : nullptr));
  }
  for (int i = 0; i < B; i++) {
    if (b.kind != 0) {
      float *xt = d.x + ((long)i * ps.Ttot + ps.Timg) * D;
      DTRY(hxa_fill_const_launch(xt, 0, (size_t)(ps.Ttot - ps.Timg) * D, 0.0f, st));
      HxaWeight wt{HXA_W_F16, D, d.cfg.ntxt_in, d.Wtxt, nullptr, nullptr};
      HxaGemm g{};
      g.A = d.ctx16 + (long)i * d.ntxt * d.cfg.ntxt_in;
      g.lda = d.cfg.ntxt_in;
      g.M = d.ntxt;
      g.w = &wt;
      g.ksplit = 1;
      g.epi = HXA_EPI_RESADD;  // text projection x += 1 * f16(text W^T) (moss blk.c MODE 2)
      g.x = xt;
      g.ldx = D;
      g.gate = d.ones;
      DTRY(hxa_gemm_launch(g, st));
    }
  }
  // blocks, chained: each block's MLP residual (x += gate * (sum of its split-K partials), blk.c:172-174) is applied
  // by the next block's first norm, which reads x anyway; the last one is applied here
  auto mlp_gate = [&](int k) { return b.kind == 0 ? d.mods + (long)k * 9 * D + 8L * D : d.mods + 5L * D; };
  if (d.tkv_par) DTRY(hxa_gemm_group_launch(d.tkv_par, nb, d.tkv_tiles, d.tkv_fmt, st));  // every block's text k / v
  const long tkv_per = 2L * B * b.C * D;
  for (int k = 0; k < nb; k++) {
    const float *mod = b.kind == 0 ? d.mods + (long)k * 9 * D : d.mods;
    const hxa_h *ck = d.tkv ? d.tkv + tkv_per * k : nullptr, *cvt = d.tkv ? d.tkv + tkv_per * k + tkv_per / 2 : nullptr;
    // block k+1's [6D][D] modulation rows: 0 .. 3D -> site 0 of its [9][D], 3D .. 6D -> site 2 (row 6D on)
    HxaBlockSide sd{};
    const HxaSideGemv fin{d.cvec, d.Lf, 2L * D, d.fmod, 2 * D, 0, 2 * D, 0, 1, D};
    const hxa_h *wn = d.modw_all + (long)(k + 1) * 6 * D * D;
    float *yn = d.mods + (long)(k + 1) * 9 * D;
    if (side_wgs) {
      sd.attn = k + 1 < nb ? HxaSideGemv{d.cvec, wn, 6L * D, yn, 6 * D, 9L * D, 3 * D, 3 * D, 1, D} : fin;
      sd.attn_wgs = side_wgs;
    } else if (side_gemm && k + 1 < nb) {
      sd.qkv = HxaSideGemv{d.cvec, wn, 3L * D, yn, 3 * D, 0, 3 * D, 0, 1, D};
      sd.up = HxaSideGemv{d.cvec, wn + 3L * D * D, 3L * D, yn + 6L * D, 3 * D, 0, 3 * D, 0, 1, D};
    } else if (side_gemm) {
      sd.qkv = fin;
    }
    DTRY(hxa_block_run_chained(&b, d.packs[k], d.x, b.kind == 0 ? d.ctx16 : nullptr, mod, ps.cosT, ps.sinT, d.ws, 0,
                               nullptr, 0, st, k > 0 ? mlp_gate(k - 1) : nullptr, 1, ck, cvt, side_on ? &sd : nullptr));
  }
  {
    long ld = 0;
    const hxa_h *t1 = (const hxa_h *)hxa_block_ws_buf(&b, d.ws, 5, &ld);
    DTRY(hxa_resaddn_launch(d.x, D, t1, hxa_block_down_parts(&b), (long)B * ps.Ttot * D, ld, B * ps.Ttot, D,
                            mlp_gate(nb - 1), st));
  }
  // final layer (+ Euler update); rapid-moss: RMS head and x0 = z - v
  if (moss_ref)
    DTRY(hxa_final_launch(d.x, B, ps.Timg, ps.Ttot, D, d.fmod, d.fmod + D, d.Wfin4f, d.cfg.lat_c, ps.lat_h, ps.lat_w,
                          d.vel, nullptr, st, d.nfin, ps.x0rows, ps.zrows, 1));
  else
    DTRY(hxa_final_launch(d.x, B, ps.Timg, ps.Ttot, D, d.fmod, d.fmod + D, d.Wfin4, d.cfg.lat_c, ps.lat_h, ps.lat_w,
                          ps.lat_out, ps.dtp, st));
  return HXA_OK;
}

// sigma, sigma_next and their difference into device memory, where the (captured) step reads them: a one-workgroup
// kernel with the values as its arguments, ahead of the step on its stream (no host buffer to keep alive and no wait
// on an earlier upload, as a copy from pinned memory would need; the step time is the same either way)
int set_sigma(Dit &d, float s0, float s1) {
  return hxa_set_sigma_launch(d.sig, s0, s1, d.st);
}

}  // namespace

extern "C" int hxa_dit_create(const hxa_dit_cfg *cfg, uint64_t seed, void **out) {
  if (!cfg || !out) return dfail(HXA_E_ARG, "null");
  *out = nullptr;
  Dit *dp = new Dit();
  Dit &d = *dp;
  d.cfg = *cfg;
  d.bd = cfg->blk;
  hxa_block_dims &b = d.bd;
  const int D = b.D, B = b.batch, C4 = 4 * cfg->lat_c;
  // kind 2, MOSS blocks with the rapid-moss LoRA: the reference form only, weights loaded from MOSS block files
  // (hxa_dit_load_moss_block; the packs start at zero), the file's shape
  if (b.kind != 0 && b.kind != 1 && b.kind != 2) {
    delete dp;
    return dfail(HXA_E_MODE, "dit: block kind");
  }
  if (b.kind == 2 && (cfg->form != 1 || b.D != 3072 || b.H != 24 || b.F != 8192 || b.fmt_attn != HXA_W_Q8 ||
                      b.fmt_mlp != HXA_W_Q8)) {
    delete dp;
    return dfail(HXA_E_MODE, "dit: LoRA blocks run in the reference form at the MOSS block files' shape (D 3072, "
                             "24 heads, MLP 8192, int8)");
  }
  if (cfg->lat_h % 2 || cfg->lat_w % 2 || C4 > 256 || 256 % C4 || cfg->temb % 2 || cfg->nblocks < 1) {
    delete dp;
    return dfail(HXA_E_ARG, "dit: latent / embedding shape");
  }
  d.form = cfg->form;
  if (d.form != 0 && d.form != 1) {
    delete dp;
    return dfail(HXA_E_MODE, "dit: form");
  }
  // the reference's Anima t-embedding is a D-wide sinusoid (animad.cpp:425), the MOSS one 256-wide (mossrun.cpp:256)
  if (d.form == 1 && (b.kind == 0 ? cfg->temb != D : cfg->temb != 256)) {
    delete dp;
    return dfail(HXA_E_ARG, "dit: the reference form's sinusoid width");
  }
  d.Timg = (cfg->lat_h / 2) * (cfg->lat_w / 2);
  if (b.kind == 0) {
    b.T = d.Ttot = d.Timg;
    b.nvalid = b.T;
  } else {
    d.ntxt = b.C;
    d.Ttot = (d.Timg + d.ntxt + 31) / 32 * 32;
    b.T = d.Ttot;
    b.nvalid = d.Timg + d.ntxt;
    b.C = 0;
    b.DC = 0;
    if (cfg->ntxt_in <= 0 || cfg->ntxt_in % 64) {
      delete dp;
      return dfail(HXA_E_ARG, "dit: MOSS text width");
    }
  }
  if (b.kind == 0 && d.Timg % 32) {
    delete dp;
    return dfail(HXA_E_ARG, "dit: token count must be a multiple of 32");
  }
  int rc = HXA_OK;
  auto M = [&](void **p, size_t bytes) {
    if (rc == HXA_OK && hipMalloc(p, bytes) != hipSuccess) rc = dfail(HXA_E_RESOURCE, "dit: out of device memory");
  };
  if (hipStreamCreateWithFlags(&d.st, hipStreamNonBlocking) != hipSuccess) {
    delete dp;
    return dfail(HXA_E_RESOURCE, "dit: stream");
  }
  d.pack_bytes = hxa_pack_layout(b.kind, D, b.F, b.DC, b.fmt_attn, b.fmt_mlp, nullptr, 0);
  d.packs.assign(cfg->nblocks, nullptr);
  for (auto &p : d.packs) M(&p, d.pack_bytes);
  // modulation weights: per block [6D][D] (config form), per block A [3 x 256][D] + B [3][3D][256] (reference form;
  // stored all blocks' A first, then all B), or one shared [6D][D] (MOSS)
  const bool anima_ref = d.form == 1 && b.kind == 0;
  d.modw.assign(b.kind == 0 ? cfg->nblocks : 1, nullptr);
  d.modw_block = anima_ref ? 768L * D + 3L * 3 * D * 256 : 6L * D * D;
  M((void **)&d.modw_all, 2L * d.modw_block * (long)d.modw.size());
  for (size_t k = 0; k < d.modw.size() && d.modw_all; k++) d.modw[k] = d.modw_all + (anima_ref ? 768L * D : d.modw_block) * (long)k;
  // fp16 glue. config form: x_embed [D][4C] | t_embed [D][temb] | final_mod [2D][D] | final_lin [4C][D] | MOSS
  // text_proj [D][ntxt_in]. Reference form, Anima: x_embed | t_l1 [D][D] | t_l2 [3D][D] | f1 [256][D] | f2 [2D][256]
  // | final_lin | t_norm [D]; MOSS: head_mod [2D][D] | text_proj (its other matrices are fp32, in vec)
  const bool moss_ref = d.form == 1 && b.kind != 0;
  if (d.form == 0)
    d.glue_elems = (long)D * C4 + (long)D * cfg->temb + 2L * D * D + (long)C4 * D + (b.kind != 0 ? (long)D * cfg->ntxt_in : 0);
  else if (b.kind == 0)
    d.glue_elems = (long)D * C4 + (long)D * D + 3L * D * D + 256L * D + 2L * D * 256 + (long)C4 * D + D;
  else
    d.glue_elems = 2L * D * D + (long)D * cfg->ntxt_in;
  M((void **)&d.glue, 2 * d.glue_elems);
  if (moss_ref) M((void **)&d.Wfin4f, 4L * C4 * D);
  else M((void **)&d.Wfin4, 2L * C4 * D);
  for (int i = 0; i < 16; i++) d.bands[i] = (float)(1.0 / pow(10000.0, i / 16.0));
  if (d.form == 1) {
    d.vec_elems = b.kind == 0 ? 0 : 3L * D + 6L * D + 2L * D + D + (long)C4 * C4 + 2L * C4 + (long)D * C4 + 256L * D +
                                        (long)D * D + (long)C4 * D;
    if (d.vec_elems) M((void **)&d.vec, 4 * d.vec_elems);
    M((void **)&d.emb, 4L * D);
    M((void **)&d.a1, 4L * D);
    M((void **)&d.lora, 4L * 3 * D);
    M((void **)&d.h1, 4L * ((long)cfg->nblocks * 768 + 256));
    if (b.kind != 0) {
      M((void **)&d.zrows, 4L * B * d.Timg * C4);
      M((void **)&d.x0rows, 4L * B * d.Timg * C4);
    }
  }
  const long latn = (long)B * cfg->lat_c * cfg->lat_h * cfg->lat_w;
  M((void **)&d.lat, 4 * latn);
  M((void **)&d.vel, 4 * latn);
  M((void **)&d.x, 4L * B * d.Ttot * D);
  M((void **)&d.sinus, 4L * cfg->temb);
  M((void **)&d.cvec, 4L * D);
  M((void **)&d.mods, 4L * (b.kind == 0 ? cfg->nblocks * 9L : 6L) * D);
  M((void **)&d.fmod, 4L * 2 * D);
  M((void **)&d.sig, 16);
  M((void **)&d.cosT, 4L * d.Ttot * 64);
  M((void **)&d.sinT, 4L * d.Ttot * 64);
  M((void **)&d.ones, 4L * D);
  M((void **)&d.ctx16, b.kind == 0 ? 2L * B * b.C * b.DC : 2L * B * d.ntxt * cfg->ntxt_in);
  d.ws_bytes = hxa_block_ws_bytes(&b);
  M(&d.ws, d.ws_bytes);
  if (rc != HXA_OK) {
    hxa_dit_destroy(dp);
    return rc;
  }
  // weights: N(0, 0.02), quantised after generation for q8 / q4 formats
  long maxmat = 0;
  {
    int N[8], K[8], f[8];
    const int n = hxa_pack_mats(b.kind, D, b.F, b.DC, b.fmt_attn, b.fmt_mlp, N, K, f);
    for (int i = 0; i < n; i++) maxmat = std::max(maxmat, (long)N[i] * K[i]);
  }
  float *tmp = nullptr;
  if (b.kind != 2 && (b.fmt_attn != HXA_W_F16 || b.fmt_mlp != HXA_W_F16)) M((void **)&tmp, 4 * maxmat);
  for (int k = 0; k < cfg->nblocks && rc == HXA_OK; k++)
    rc = b.kind == 2 ? (hipMemsetAsync(d.packs[k], 0, d.pack_bytes, d.st) == hipSuccess ? HXA_OK : HXA_E_HIP)
                     : init_pack(d, d.packs[k], seed * 1000003ull + k, tmp);
  if (rc == HXA_OK)
    rc = hxa_fill_normal_launch(d.modw_all, 1, d.modw_block * (long)d.modw.size(), seed * 7919ull + 100000, 0.0f, 0.02f, d.st);
  if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.glue, 1, d.glue_elems, seed * 7919ull + 99999, 0.0f, 0.02f, d.st);
  if (!moss_ref) {
    d.Wemb = d.glue;
    d.L1 = d.Wemb + (long)D * C4;
  }
  if (d.form == 0) {
    d.Lf = d.L1 + (long)D * cfg->temb;
    d.Wfin = d.Lf + 2L * D * D;
    d.Wtxt = b.kind != 0 ? d.Wfin + (long)C4 * D : nullptr;
  } else if (b.kind == 0) {
    d.Wl2 = d.L1 + (long)D * D;
    d.F1 = d.Wl2 + 3L * D * D;
    d.F2 = d.F1 + 256L * D;
    d.Wfin = d.F2 + 2L * D * 256;
    d.tnorm = d.Wfin + (long)C4 * D;  // RMSNorm weight of the t-embedding, fp16 like the reference's tensors
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.tnorm, 1, D, seed * 7919ull + 99998, 1.0f, 0.1f, d.st);
  } else {
    d.Wh = d.glue;
    d.Wtxt = d.Wh + 2L * D * D;
    d.bve = d.vec;
    d.b0 = d.bve + D;
    d.b2 = d.b0 + D;
    d.bm = d.b2 + D;
    d.bh = d.bm + 6L * D;
    d.nfin = d.bh + 2L * D;
    d.Q = d.nfin + D;
    d.bnm = d.Q + (long)C4 * C4;
    d.bnv = d.bnm + C4;
    d.Wv32 = d.bnv + C4;
    d.T0f = d.Wv32 + (long)D * C4;
    d.T2f = d.T0f + 256L * D;
    d.Wfin32 = d.T2f + (long)D * D;
    // biases and the latent mix N(0, 0.02); the head's RMSNorm weight and the BN variance around 1, the BN mean
    // around 0 (N(0, 0.1))
    const uint64_t vs = seed * 7919ull + 99997;
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.bve, 0, 11L * D, vs, 0.0f, 0.02f, d.st);  // bve, b0, b2, bm, bh
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.Q, 0, (long)C4 * C4, vs + 4, 0.0f, 0.02f, d.st);
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.nfin, 0, D, vs + 1, 1.0f, 0.1f, d.st);
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.bnm, 0, C4, vs + 2, 0.0f, 0.1f, d.st);
    if (rc == HXA_OK) rc = hxa_fill_normal_launch(d.bnv, 0, C4, vs + 3, 1.0f, 0.1f, d.st);
    // the fp32 matrices N(0, 0.02)
    if (rc == HXA_OK)
      rc = hxa_fill_normal_launch(d.Wv32, 0, (long)D * C4 + 256L * D + (long)D * D + (long)C4 * D, vs + 5, 0.0f, 0.02f, d.st);
  }
  if (rc == HXA_OK) rc = moss_ref ? hxa_ktile4_f32_launch(d.Wfin32, C4, D, d.Wfin4f, d.st) : hxa_ktile4_launch(d.Wfin, C4, D, d.Wfin4, d.st);
  if (rc == HXA_OK) rc = hxa_fill_const_launch(d.ones, 0, D, 1.0f, d.st);
  if (rc == HXA_OK && b.kind == 0) {  // site-1 rows of every block: shift 0, scale 0, gate 1
    for (int k = 0; k < cfg->nblocks && rc == HXA_OK; k++) {
      rc = hxa_fill_const_launch(d.mods + (long)k * 9 * D + 3L * D, 0, 2L * D, 0.0f, d.st);
      if (rc == HXA_OK) rc = hxa_fill_const_launch(d.mods + (long)k * 9 * D + 5L * D, 0, D, 1.0f, d.st);
    }
  }
  if (rc == HXA_OK && hipMemsetAsync(d.x, 0, 4L * B * d.Ttot * D, d.st) != hipSuccess) rc = dfail(HXA_E_HIP, "memset");
  std::vector<float> c, s;
  if (b.kind == 0) {
    // token (gy, gx) of a gh x gw grid, gh = H/2 rows (megarun's gh, gw arguments)
    rope_anima(cfg->lat_h / 2, cfg->lat_w / 2, c, s);
  } else {
    rope_moss(cfg->lat_h / 2, cfg->lat_w / 2, d.ntxt, d.Ttot, d.bands, c, s);
  }
  if (rc == HXA_OK && (hipMemcpyAsync(d.cosT, c.data(), 4 * c.size(), hipMemcpyHostToDevice, d.st) != hipSuccess ||
                       hipMemcpyAsync(d.sinT, s.data(), 4 * s.size(), hipMemcpyHostToDevice, d.st) != hipSuccess))
    rc = dfail(HXA_E_HIP, "rope upload");
  if (rc == HXA_OK && hipStreamSynchronize(d.st) != hipSuccess) rc = dfail(HXA_E_HIP, "init sync");
  if (tmp) (void)hipFree(tmp);
  // text k / v up front: when the blocks' qkv grids cannot carry their text k / v tiles, every block's text k / v
  // projection (ctx only) runs at the start of the step in one grouped launch, and each block fuses its cross q with
  // the attention
  if (rc == HXA_OK && b.kind == 0) {
    const int nb = cfg->nblocks;
    const long per = 2L * B * b.C * D;  // elements of one block's ck + cvt
    std::vector<HxaGemm> gs(nb);
    std::vector<HxaWeight> ws(nb);
    hxa_h *probe = nullptr;  // planning needs real, aligned ck / cvt addresses: one block's worth first
    M((void **)&probe, 2L * per);
    bool use = rc == HXA_OK;
    for (int k = 0; k < nb && use; k++)
      use = hxa_block_textkv_plan(&b, d.packs[k], d.ctx16, probe, probe + per / 2, &gs[k], &ws[k]) == 1;
    if (probe) (void)hipFree(probe);
    if (use) {
      M((void **)&d.tkv, 2L * per * nb);
      for (int k = 0; k < nb && rc == HXA_OK; k++) {
        if (hxa_block_textkv_plan(&b, d.packs[k], d.ctx16, d.tkv + per * k, d.tkv + per * k + per / 2, &gs[k], &ws[k]) != 1)
          rc = dfail(HXA_E_ARG, "dit: text k / v plan");
        gs[k].w = &ws[k];
      }
      const long pb = hxa_gemm_group_param_bytes(nb);
      std::vector<uint8_t> par(pb);
      if (rc == HXA_OK) {
        const int r = hxa_gemm_group_prepare(gs.data(), nb, par.data(), &d.tkv_tiles, &d.tkv_fmt);
        if (r != HXA_OK) rc = dfail(r, "dit: text k / v grouped launch");
      }
      M(&d.tkv_par, pb);
      if (rc == HXA_OK && hipMemcpy(d.tkv_par, par.data(), pb, hipMemcpyHostToDevice) != hipSuccess)
        rc = dfail(HXA_E_HIP, "dit: text k / v parameters");
    }
  }
  if (rc != HXA_OK) {
    hxa_dit_destroy(dp);
    return rc;
  }
  *out = dp;
  return HXA_OK;
}

extern "C" int hxa_dit_destroy(void *p) {
  Dit *d = (Dit *)p;
  if (!d) return HXA_OK;
  if (d->st) (void)hipStreamSynchronize(d->st);
  if (d->exec) (void)hipGraphExecDestroy(d->exec);
  if (d->graph) (void)hipGraphDestroy(d->graph);
  for (int f = 0; f <= Dit::MAXF; f++) {
    if (d->execL[f]) (void)hipGraphExecDestroy(d->execL[f]);
    if (d->graphL[f]) (void)hipGraphDestroy(d->graphL[f]);
    if (d->cosL[f]) (void)hipFree(d->cosL[f]);
    if (d->sinL[f]) (void)hipFree(d->sinL[f]);
  }
  for (float *q : {d->nfull, d->dhat, d->xlow, d->vlow, d->zl, d->x0l}) if (q) (void)hipFree(q);
  for (void *q : d->packs) if (q) (void)hipFree(q);
  if (d->modw_all) (void)hipFree(d->modw_all);
  void *bufs[] = {d->glue, d->lat, d->vel, d->x, d->sinus, d->cvec, d->mods, d->fmod, d->sig, d->cosT, d->sinT,
                  d->ones, d->ctx16, d->ws, d->vec, d->emb, d->a1, d->lora, d->h1, d->zrows, d->x0rows, d->tkv,
                  d->tkv_par, d->Wfin4, d->Wfin4f};
  for (void *q : bufs) if (q) (void)hipFree(q);
  if (d->st) (void)hipStreamDestroy(d->st);
  delete d;
  return HXA_OK;
}

extern "C" int hxa_dit_set_inputs(void *p, const float *lat, const float *ctx) {
  Dit &d = *(Dit *)p;
  const hxa_block_dims &b = d.bd;
  const long latn = (long)b.batch * d.cfg.lat_c * d.cfg.lat_h * d.cfg.lat_w;
  if (lat) DHIP(hipMemcpyAsync(d.lat, lat, 4 * latn, hipMemcpyHostToDevice, d.st));
  if (lat) {  // new noise: the low-res steps start over from it
    d.low_init = false;
    d.moss_low_live = false;
  }
  if (lat && d.zrows) {  // rapid-moss: the latent is the noise z (token rows), the clean estimate starts at 0
    DTRY(hxa_patchify_launch(d.lat, b.batch, d.cfg.lat_c, d.cfg.lat_h, d.cfg.lat_w, d.zrows, d.st));
    DTRY(hxa_fill_const_launch(d.x0rows, 0, (size_t)latn, 0.0f, d.st));
  }
  if (ctx) {
    const long n = b.kind == 0 ? (long)b.batch * b.C * b.DC : (long)b.batch * d.ntxt * d.cfg.ntxt_in;
    std::vector<uint16_t> h(n);
    for (long i = 0; i < n; i++) h[i] = f2h_host(ctx[i]);
    DHIP(hipMemcpyAsync(d.ctx16, h.data(), 2 * n, hipMemcpyHostToDevice, d.st));
  }
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

extern "C" int hxa_dit_get_latent(void *p, float *lat) {
  Dit &d = *(Dit *)p;
  const long latn = (long)d.bd.batch * d.cfg.lat_c * d.cfg.lat_h * d.cfg.lat_w;
  if (d.x0rows) {  // rapid-moss: the BN-denormalised, unpatchified clean estimate (mossrun.cpp:339-343)
    DTRY(hxa_bn_unpatchify_launch(d.x0rows, d.bnm, d.bnv, d.bd.batch, d.cfg.lat_c, d.cfg.lat_h, d.cfg.lat_w, d.vel, d.st));
    DHIP(hipMemcpyAsync(lat, d.vel, 4 * latn, hipMemcpyDeviceToHost, d.st));
    DHIP(hipStreamSynchronize(d.st));
    return HXA_OK;
  }
  DHIP(hipMemcpyAsync(lat, d.lat, 4 * latn, hipMemcpyDeviceToHost, d.st));
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

namespace {
// record (use_graph 0) or replay the graph in (graph, exec) of `rec`, capturing it on first use
template <class Rec>
int run_graph(Dit &d, int use_graph, hipGraph_t &graph, hipGraphExec_t &exec, Rec rec) {
  if (!use_graph) return rec();
  if (!exec) {
    DHIP(hipStreamBeginCapture(d.st, hipStreamCaptureModeRelaxed));
    const int r = rec();
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(d.st, &g);
    if (r != HXA_OK) {
      if (g) (void)hipGraphDestroy(g);
      return r;
    }
    if (e != hipSuccess) return dfail(HXA_E_HIP, "graph capture");
    graph = g;
    DHIP(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
  }
  DHIP(hipGraphLaunch(exec, d.st));
  return HXA_OK;
}
// a MOSS full step after low-res ones starts from their clean estimate, upsampled (mossrun.cpp:311)
int moss_leave_low(Dit &d) {
  if (!d.moss_low_live) return HXA_OK;
  const int gh = d.cfg.lat_h / 2, gw = d.cfg.lat_w / 2;
  DTRY(hxa_upsample2_rows_launch(d.x0l, d.bd.batch, gh / 2, gw / 2, 4 * d.cfg.lat_c, d.x0rows, d.st));
  d.moss_low_live = false;
  return HXA_OK;
}
int run_step(Dit &d, int use_graph) {
  if (d.x0rows) DTRY(moss_leave_low(d));
  const Pass ps = full_pass(d, MODE_EULER);
  return run_graph(d, use_graph, d.graph, d.exec, [&]() { return record_step(d, ps); });
}
}  // namespace

extern "C" int hxa_dit_step(void *p, float sigma, float sigma_next, int use_graph) {
  Dit &d = *(Dit *)p;
  if (d.x0rows) return dfail(HXA_E_MODE, "dit: the rapid-moss form steps with hxa_dit_moss_step");
  DTRY(set_sigma(d, sigma, sigma_next));
  return run_step(d, use_graph);
}

extern "C" int hxa_dit_moss_step(void *p, float code, int use_graph) {
  Dit &d = *(Dit *)p;
  if (!d.x0rows) return dfail(HXA_E_MODE, "dit: hxa_dit_moss_step needs the MOSS reference form");
  DTRY(set_sigma(d, code, code));
  return run_step(d, use_graph);
}

namespace {
// the RoPE tables of the 1/f grid (MOSS: image positions times `scale`), built on first use (and again when the MOSS
// scale changes); the upload completes before the call returns
int low_rope(Dit &d, int f, double scale) {
  const bool moss = d.bd.kind != 0;
  if (d.cosL[f] && (!moss || d.ropeL_scale == scale)) return HXA_OK;
  const int gh = d.cfg.lat_h / 2 / f, gw = d.cfg.lat_w / 2 / f;
  const int Ttot = moss ? (gh * gw + d.ntxt + 31) / 32 * 32 : gh * gw;
  std::vector<float> c, sn;
  if (moss) rope_moss(gh, gw, d.ntxt, Ttot, d.bands, c, sn, scale);
  else rope_anima(gh, gw, c, sn);
  if (!d.cosL[f]) {
    DHIP(hipMalloc((void **)&d.cosL[f], 4L * Ttot * 64));
    DHIP(hipMalloc((void **)&d.sinL[f], 4L * Ttot * 64));
  }
  DHIP(hipMemcpyAsync(d.cosL[f], c.data(), 4 * c.size(), hipMemcpyHostToDevice, d.st));
  DHIP(hipMemcpyAsync(d.sinL[f], sn.data(), 4 * sn.size(), hipMemcpyHostToDevice, d.st));
  DHIP(hipStreamSynchronize(d.st));
  d.ropeL_scale = scale;
  return HXA_OK;
}
int ensure(float *&p, long floats) {
  if (!p && hipMalloc((void **)&p, 4 * floats) != hipSuccess) return dfail(HXA_E_RESOURCE, "dit: out of device memory");
  return HXA_OK;
}
// the pass over the 1/f grid
Pass low_pass(Dit &d, int f) {
  Pass q;
  q.lat_h = d.cfg.lat_h / f;
  q.lat_w = d.cfg.lat_w / f;
  q.Timg = (q.lat_h / 2) * (q.lat_w / 2);
  q.Ttot = d.bd.kind != 0 ? (q.Timg + d.ntxt + 31) / 32 * 32 : q.Timg;
  q.bd = d.bd;
  q.bd.T = q.Ttot;
  q.bd.nvalid = d.bd.kind != 0 ? q.Timg + d.ntxt : q.Timg;
  q.cosT = d.cosL[f];
  q.sinT = d.sinL[f];
  return q;
}
}  // namespace

extern "C" int hxa_dit_step_lowres(void *p, float sigma, float sigma_next, int factor, int use_graph) {
  Dit &d = *(Dit *)p;
  if (d.x0rows) return dfail(HXA_E_MODE, "dit: the rapid-moss form steps with hxa_dit_moss_step_lowres");
  const int H = d.cfg.lat_h, W = d.cfg.lat_w;
  // animad.cpp:407: a factor the latent does not divide into whole patches, or whose token count is not a multiple
  // of 32, runs the step at full resolution
  if (factor < 2 || factor > Dit::MAXF || H % (2 * factor) || W % (2 * factor) || ((H / 2 / factor) * (W / 2 / factor)) % 32)
    return hxa_dit_step(p, sigma, sigma_next, use_graph);
  const long BC = (long)d.bd.batch * d.cfg.lat_c, full = BC * H * W;
  DTRY(ensure(d.nfull, full));
  DTRY(ensure(d.dhat, full));
  DTRY(ensure(d.xlow, full / 4));  // the largest low grid (factor 2)
  DTRY(ensure(d.vlow, full / 4));
  DTRY(low_rope(d, factor, 1.0));
  DTRY(set_sigma(d, sigma, sigma_next));
  if (!d.low_init) {  // the first low-res step: its latent is the noise, no clean estimate yet (animad.cpp:430)
    DHIP(hipMemcpyAsync(d.nfull, d.lat, 4 * full, hipMemcpyDeviceToDevice, d.st));
    DTRY(hxa_fill_const_launch(d.dhat, 0, (size_t)full, 0.0f, d.st));
    d.low_init = true;
  }
  Pass ps = low_pass(d, factor);
  ps.lat_in = d.xlow;
  ps.lat_out = d.vlow;
  return run_graph(d, use_graph, d.graphL[factor], d.execL[factor], [&]() {
    DTRY(hxa_lowres_pool_launch(d.nfull, d.dhat, BC, H, W, factor, d.sig, d.xlow, d.st));
    DTRY(record_step(d, ps));
    return hxa_lowres_velocity_launch(d.xlow, d.vlow, d.lat, d.nfull, d.dhat, BC, H, W, factor, d.sig, d.st);
  });
}

extern "C" int hxa_dit_moss_step_lowres(void *p, float code, float rope_scale, int use_graph) {
  Dit &d = *(Dit *)p;
  if (!d.x0rows) return dfail(HXA_E_MODE, "dit: hxa_dit_moss_step_lowres needs the MOSS reference form");
  const int gh = d.cfg.lat_h / 2, gw = d.cfg.lat_w / 2, C4 = 4 * d.cfg.lat_c, B = d.bd.batch;
  if (gh % 2 || gw % 2) return hxa_dit_moss_step(p, code, use_graph);  // mossrun.cpp:289: an even grid only
  const long low = (long)B * (gh / 2) * (gw / 2) * C4;
  DTRY(ensure(d.zl, low));
  DTRY(ensure(d.x0l, low));
  DTRY(low_rope(d, 2, rope_scale));
  DTRY(set_sigma(d, code, code));
  if (!d.low_init) {  // mossrun.cpp:290-291: the low-res noise, and a clean estimate of 0
    DTRY(hxa_moss_pool2_launch(d.zrows, B, gh, gw, C4, d.zl, d.st));
    DTRY(hxa_fill_const_launch(d.x0l, 0, (size_t)low, 0.0f, d.st));
    d.low_init = true;
  }
  d.moss_low_live = true;
  Pass ps = low_pass(d, 2);
  ps.zrows = d.zl;
  ps.x0rows = d.x0l;
  return run_graph(d, use_graph, d.graphL[2], d.execL[2], [&]() { return record_step(d, ps); });
}

extern "C" int hxa_dit_velocity(void *p, float sigma, float *v) {
  Dit &d = *(Dit *)p;
  if (d.x0rows) return dfail(HXA_E_MODE, "dit: the rapid-moss form has no velocity output");
  DTRY(set_sigma(d, sigma, sigma));
  DTRY(record_step(d, full_pass(d, MODE_VELOCITY)));
  const long latn = (long)d.bd.batch * d.cfg.lat_c * d.cfg.lat_h * d.cfg.lat_w;
  DHIP(hipMemcpyAsync(v, d.vel, 4 * latn, hipMemcpyDeviceToHost, d.st));
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

extern "C" long hxa_dit_export(void *p, int which, void *host, size_t bytes) {
  Dit &d = *(Dit *)p;
  const int nb = d.cfg.nblocks, D = d.bd.D;
  struct Part {
    const void *src;
    long n;
  } parts[2] = {{nullptr, 0}, {nullptr, 0}};
  if (which >= 0 && which < nb) {
    parts[0] = {d.packs[which], d.pack_bytes};
  } else if (which >= nb && which < nb + (int)d.modw.size()) {
    const int k = which - nb;
    if (d.form == 1 && d.bd.kind == 0) {  // this block's A rows, then its B
      parts[0] = {d.modw_all + 768L * D * k, 2 * 768L * D};
      parts[1] = {d.modw_all + 768L * D * nb + 3L * 3 * D * 256 * k, 2 * 3L * 3 * D * 256};
    } else {
      parts[0] = {d.modw[k], 2 * d.modw_block};
    }
  } else if (which == 2 * nb) {
    parts[0] = {d.glue, 2 * d.glue_elems};
  } else if (which == 2 * nb + 1 && d.vec) {
    parts[0] = {d.vec, 4 * d.vec_elems};
  } else {
    return dfail(HXA_E_ARG, "dit export index");
  }
  const long n = parts[0].n + parts[1].n;
  if (!host) return n;
  if ((long)bytes < n) return dfail(HXA_E_ARG, "dit export buffer too small");
  if (hipStreamSynchronize(d.st) != hipSuccess) return dfail(HXA_E_HIP, "dit export sync");
  char *out = (char *)host;
  for (const Part &q : parts) {
    if (q.n && hipMemcpy(out, q.src, q.n, hipMemcpyDeviceToHost) != hipSuccess) return dfail(HXA_E_HIP, "dit export copy");
    out += q.n;
  }
  return n;
}

// the inverse of hxa_dit_export: the same `which` sections, the same byte images (host bytes must equal the export's
// size); the device copy is complete when the call returns. The step graphs hold pointers, not values, so the next
// step (replayed or recorded) runs on the imported weights.
extern "C" int hxa_dit_import(void *p, int which, const void *host, size_t bytes) {
  if (!p || !host) return dfail(HXA_E_ARG, "dit import: null");
  Dit &d = *(Dit *)p;
  const int nb = d.cfg.nblocks, D = d.bd.D;
  struct Part {
    void *dst;
    long n;
  } parts[2] = {{nullptr, 0}, {nullptr, 0}};
  if (which >= 0 && which < nb) {
    parts[0] = {d.packs[which], d.pack_bytes};
  } else if (which >= nb && which < nb + (int)d.modw.size()) {
    const int k = which - nb;
    if (d.form == 1 && d.bd.kind == 0) {
      parts[0] = {d.modw_all + 768L * D * k, 2 * 768L * D};
      parts[1] = {d.modw_all + 768L * D * nb + 3L * 3 * D * 256 * k, 2 * 3L * 3 * D * 256};
    } else {
      parts[0] = {d.modw[k], 2 * d.modw_block};
    }
  } else if (which == 2 * nb) {
    parts[0] = {d.glue, 2 * d.glue_elems};
  } else if (which == 2 * nb + 1 && d.vec) {
    parts[0] = {d.vec, 4 * d.vec_elems};
  } else {
    return dfail(HXA_E_ARG, "dit import index");
  }
  if ((long)bytes != parts[0].n + parts[1].n) return dfail(HXA_E_ARG, "dit import: size differs from the section's");
  DHIP(hipStreamSynchronize(d.st));
  const char *in = (const char *)host;
  for (const Part &q : parts) {
    if (q.n) DHIP(hipMemcpy(q.dst, in, q.n, hipMemcpyHostToDevice));
    in += q.n;
  }
  // the final layer's kernel reads its weights k-tiled by 4
  if (which == 2 * nb && d.Wfin) DTRY(hxa_ktile4_launch(d.Wfin, 4 * d.cfg.lat_c, D, d.Wfin4, d.st));
  if (which == 2 * nb + 1 && d.Wfin32) DTRY(hxa_ktile4_f32_launch(d.Wfin32, 4 * d.cfg.lat_c, D, d.Wfin4f, d.st));
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

namespace {
// host bytes -> device, through one synchronous copy
int upload(void *dst, const void *src, size_t bytes) {
  if (bytes && hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) != hipSuccess) return dfail(HXA_E_HIP, "dit: weight upload");
  return HXA_OK;
}
// tensors of a glue file: name -> (dtype 0 fp32 / 1 fp16, dims, data)
struct GlueTensor {
  int dtype = 0;
  std::vector<long> dims;
  const uint8_t *data = nullptr;
  long elems() const {
    long n = 1;
    for (long v : dims) n *= v;
    return n;
  }
};
bool shape_is(const GlueTensor &t, std::initializer_list<long> want) {
  return t.dims.size() == want.size() && std::equal(want.begin(), want.end(), t.dims.begin());
}
}  // namespace

// blk_wlayout.h:3-20: matrix offsets of an Anima blkNN.bin (q8 files: WQ(x) = x / 2048 * 1152), the adaLN modulation
// weights at W_MODW / WQ_MODW: per site A [256][2048] then B [6144][256], fp16 (export_all.py:59-61)
extern "C" int hxa_dit_load_block(void *p, int k, const void *blk, size_t bytes) {
  if (!p || !blk) return dfail(HXA_E_ARG, "dit load block: null");
  Dit &d = *(Dit *)p;
  const hxa_block_dims &b = d.bd;
  const int nb = d.cfg.nblocks, D = b.D;
  if (k < 0 || k >= nb) return dfail(HXA_E_ARG, "dit load block: block index");
  if (b.kind != 0 || d.form != 1 || D != 2048 || b.H != 16 || b.F != 8192 || b.DC != 1024)
    return dfail(HXA_E_MODE, "dit load block: blkNN.bin files hold the Anima reference form's blocks (D 2048, 16 heads, "
                             "MLP 8192, context 1024)");
  const size_t W_GAIN = 125829120, W_MODW = 125833216, W_TOTAL = 138416128;
  const size_t WQ_GAIN = W_GAIN / 2048 * 1152, WQ_MODW = WQ_GAIN + 4096, WQ_TOTAL = WQ_MODW + (W_TOTAL - W_MODW);
  const bool q8 = bytes == WQ_TOTAL;
  if (bytes != W_TOTAL && !q8) return dfail(HXA_E_WEIGHTS, "dit load block: neither an fp16 nor a q8 blkNN.bin (size)");
  const int fmt = q8 ? HXA_W_Q8 : HXA_W_F16;
  if (b.fmt_attn != fmt || b.fmt_mlp != fmt) return dfail(HXA_E_WEIGHTS, "dit load block: the file's format is not the DiT's");
  const long wf16[11] = {0, 8388608, 16777216, 25165824, 33554432, 41943040, 46137344, 50331648, 58720256, 92274688,
                         (long)W_GAIN};
  long woff[11];
  for (int i = 0; i < 11; i++) woff[i] = q8 ? wf16[i] / 2048 * 1152 : wf16[i];
  uint8_t *stage = nullptr;
  DHIP(hipStreamSynchronize(d.st));
  DHIP(hipMalloc((void **)&stage, bytes));
  int rc = upload(stage, blk, bytes);
  if (rc == HXA_OK) rc = hxa_anima_file_to_pack(stage, woff, q8, d.packs[k], d.st);
  // modulation weights: this block's A rows (3 sites x 256) and its three B matrices, where the prelude reads them
  const long A = 256L * D, Bm = 3L * D * 256;
  const uint8_t *mw = stage + (q8 ? WQ_MODW : W_MODW);
  for (int site = 0; site < 3 && rc == HXA_OK; site++) {
    const uint8_t *a = mw + 2 * site * (A + Bm);
    if (hipMemcpyAsync(d.modw_all + 768L * D * k + site * A, a, 2 * A, hipMemcpyDeviceToDevice, d.st) != hipSuccess ||
        hipMemcpyAsync(d.modw_all + 768L * D * nb + (3L * k + site) * Bm, a + 2 * A, 2 * Bm, hipMemcpyDeviceToDevice,
                       d.st) != hipSuccess)
      rc = dfail(HXA_E_HIP, "dit load block: modulation weights");
  }
  if (rc == HXA_OK && hipStreamSynchronize(d.st) != hipSuccess) rc = dfail(HXA_E_HIP, "dit load block: conversion");
  (void)hipFree(stage);
  return rc;
}

// moss/export_moss.py pack_layer (offsets moss blk_meta.h:6-17): block k from the bytes of a MOSS blkNN.bin, the
// buffer mossrun registers (mossrun.cpp:100-119), through the same conversion as mega_block's registered MOSS weights
extern "C" int hxa_dit_load_moss_block(void *p, int k, const void *blk, size_t bytes) {
  if (!p || !blk) return dfail(HXA_E_ARG, "dit load block: null");
  Dit &d = *(Dit *)p;
  if (k < 0 || k >= d.cfg.nblocks) return dfail(HXA_E_ARG, "dit load block: block index");
  if (d.bd.kind != 2) return dfail(HXA_E_MODE, "dit load block: MOSS block files need a DiT of LoRA blocks (kind 2)");
  if (bytes != HXA_MOSS_FILE_BYTES) return dfail(HXA_E_WEIGHTS, "dit load block: not a MOSS blkNN.bin (size)");
  uint8_t *stage = nullptr;
  DHIP(hipStreamSynchronize(d.st));
  DHIP(hipMalloc((void **)&stage, bytes));
  int rc = upload(stage, blk, bytes);
  if (rc == HXA_OK && hipMemsetAsync(d.packs[k], 0, d.pack_bytes, d.st) != hipSuccess) rc = dfail(HXA_E_HIP, "dit load block: zero");
  if (rc == HXA_OK) rc = hxa_moss_file_to_pack(stage, d.packs[k], d.st);
  if (rc == HXA_OK && hipStreamSynchronize(d.st) != hipSuccess) rc = dfail(HXA_E_HIP, "dit load block: conversion");
  (void)hipFree(stage);
  return rc;
}

// phone/extract_small.py format (read by animad.cpp:43-70): u32 count; per tensor u32 name length, the name, u32 ndim,
// i64 dims[ndim], fp16 data. The tensors of the reference glue (animad.cpp:424-492) are taken; others (the LLM
// adapter's) are skipped.
extern "C" int hxa_dit_load_anima_glue(void *p, const void *file, size_t bytes) {
  if (!p || !file) return dfail(HXA_E_ARG, "dit load glue: null");
  Dit &d = *(Dit *)p;
  const int D = d.bd.D, C4 = 4 * d.cfg.lat_c;
  if (d.form != 1 || d.bd.kind != 0) return dfail(HXA_E_MODE, "dit load glue: small.bin is the Anima reference form's");
  const uint8_t *q = (const uint8_t *)file, *end = q + bytes;
  auto take = [&](void *dst, size_t n) {
    if ((size_t)(end - q) < n) return false;
    memcpy(dst, q, n);
    q += n;
    return true;
  };
  uint32_t cnt = 0;
  if (!take(&cnt, 4)) return dfail(HXA_E_WEIGHTS, "dit load glue: truncated");
  std::map<std::string, GlueTensor> tens;
  for (uint32_t i = 0; i < cnt; i++) {
    uint32_t nl = 0, nd = 0;
    if (!take(&nl, 4) || nl > 4096 || (size_t)(end - q) < nl) return dfail(HXA_E_WEIGHTS, "dit load glue: truncated");
    std::string name((const char *)q, nl);
    q += nl;
    if (!take(&nd, 4) || nd > 8) return dfail(HXA_E_WEIGHTS, "dit load glue: bad tensor header");
    GlueTensor t;
    t.dtype = 1;
    t.dims.resize(nd);
    for (uint32_t j = 0; j < nd; j++) {
      int64_t v = 0;
      if (!take(&v, 8) || v < 0 || v > (1L << 32)) return dfail(HXA_E_WEIGHTS, "dit load glue: bad tensor header");
      t.dims[j] = v;
    }
    const long n = t.elems();
    if ((size_t)(end - q) < 2 * (size_t)n) return dfail(HXA_E_WEIGHTS, "dit load glue: truncated tensor data");
    t.data = q;
    q += 2 * (size_t)n;
    tens[name] = t;
  }
  struct Want {
    const char *name;
    hxa_h *dst;
    long rows, cols;
  };
  // x_embedder.proj.1 has 4 more columns than 4C (the zero mask channel, animad.cpp:446); they are dropped
  const Want want[] = {{"t_embedder.1.linear_1.weight", d.L1, D, D},
                       {"t_embedder.1.linear_2.weight", d.Wl2, 3L * D, D},
                       {"final_layer.adaln_modulation.1.weight", d.F1, 256, D},
                       {"final_layer.adaln_modulation.2.weight", d.F2, 2L * D, 256},
                       {"final_layer.linear.weight", d.Wfin, C4, D}};
  for (const Want &w : want) {
    auto it = tens.find(w.name);
    if (it == tens.end() || !shape_is(it->second, {w.rows, w.cols}))
      return dfail(HXA_E_WEIGHTS, "dit load glue: a tensor is missing or not of the DiT's shape");
  }
  auto xe = tens.find("x_embedder.proj.1.weight");
  auto tn = tens.find("t_embedding_norm.weight");
  if (xe == tens.end() || xe->second.dims.size() != 2 || xe->second.dims[0] != D ||
      (xe->second.dims[1] != C4 && xe->second.dims[1] != C4 + 4))
    return dfail(HXA_E_WEIGHTS, "dit load glue: x_embedder.proj.1.weight missing or not [D][4C (+4)]");
  if (tn == tens.end() || !shape_is(tn->second, {D})) return dfail(HXA_E_WEIGHTS, "dit load glue: t_embedding_norm.weight");
  DHIP(hipStreamSynchronize(d.st));
  for (const Want &w : want) DTRY(upload(w.dst, tens[w.name].data, 2 * (size_t)w.rows * w.cols));
  DTRY(upload(d.tnorm, tn->second.data, 2L * D));
  const long kx = xe->second.dims[1];
  std::vector<uint16_t> xw((size_t)D * C4);
  for (long r = 0; r < D; r++) memcpy(&xw[(size_t)r * C4], xe->second.data + 2 * r * kx, 2L * C4);
  DTRY(upload(d.Wemb, xw.data(), 2 * xw.size()));
  DTRY(hxa_ktile4_launch(d.Wfin, C4, D, d.Wfin4, d.st));
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

// moss/export_glue.py:1-22 (read by mossrun.cpp:129-139): "MGL1", i32 n; n entries { char name[40]; i32 dtype (0 fp32,
// 1 fp16); i32 nd; i32 dims[3]; i64 offset (from the file start); i64 bytes }; data 128-byte aligned. Every tensor of
// the DiT glue is taken (step_codes stays with the caller, who passes the step's code to hxa_dit_moss_step); rope.bands
// rebuilds the RoPE tables.
extern "C" int hxa_dit_load_moss_glue(void *p, const void *file, size_t bytes) {
  if (!p || !file) return dfail(HXA_E_ARG, "dit load glue: null");
  Dit &d = *(Dit *)p;
  const int D = d.bd.D, C4 = 4 * d.cfg.lat_c;
  if (d.form != 1 || d.bd.kind == 0) return dfail(HXA_E_MODE, "dit load glue: glue.bin is the MOSS reference form's");
  const uint8_t *base = (const uint8_t *)file;
  if (bytes < 8 || memcmp(base, "MGL1", 4)) return dfail(HXA_E_WEIGHTS, "dit load glue: not an MGL1 file");
  int32_t n = 0;
  memcpy(&n, base + 4, 4);
  if (n < 0 || n > 4096 || 8 + 76L * n > (long)bytes) return dfail(HXA_E_WEIGHTS, "dit load glue: bad entry count");
  std::map<std::string, GlueTensor> tens;
  for (int i = 0; i < n; i++) {
    const uint8_t *e = base + 8 + 76L * i;
    char name[41] = {0};
    memcpy(name, e, 40);
    int32_t dt, nd, dims[3];
    int64_t off, nbytes;
    memcpy(&dt, e + 40, 4);
    memcpy(&nd, e + 44, 4);
    memcpy(dims, e + 48, 12);
    memcpy(&off, e + 60, 8);
    memcpy(&nbytes, e + 68, 8);
    if ((dt != 0 && dt != 1) || nd < 1 || nd > 3 || off < 0 || nbytes < 0 || (uint64_t)off + (uint64_t)nbytes > bytes)
      return dfail(HXA_E_WEIGHTS, "dit load glue: bad entry");
    GlueTensor t;
    t.dtype = dt;
    for (int j = 0; j < nd; j++) t.dims.push_back(dims[j]);
    if (t.elems() * (dt == 0 ? 4 : 2) != nbytes) return dfail(HXA_E_WEIGHTS, "dit load glue: entry size and shape differ");
    t.data = base + off;
    tens[name] = t;
  }
  struct Want {
    const char *name;
    int dtype;
    void *dst;
    long rows, cols;  // cols 0: a vector of `rows`
  };
  const Want want[] = {{"video_embedder.weight", 0, d.Wv32, D, C4},
                       {"video_embedder.bias", 0, d.bve, D, 0},
                       {"time_embedding.0.weight", 0, d.T0f, D, 256},
                       {"time_embedding.0.bias", 0, d.b0, D, 0},
                       {"time_embedding.2.weight", 0, d.T2f, D, D},
                       {"time_embedding.2.bias", 0, d.b2, D, 0},
                       {"shared_block_modulation.weight", 1, d.modw_all, 6L * D, D},
                       {"shared_block_modulation.bias", 0, d.bm, 6L * D, 0},
                       {"video_head_modulation.weight", 1, d.Wh, 2L * D, D},
                       {"video_head_modulation.bias", 0, d.bh, 2L * D, 0},
                       {"final_linear_video.weight", 0, d.Wfin32, C4, D},
                       {"final_norm_video.weight", 0, d.nfin, D, 0},
                       {"latent_mix.Q", 0, d.Q, C4, C4},
                       {"bn.mean", 0, d.bnm, C4, 0},
                       {"bn.var", 0, d.bnv, C4, 0},
                       {"rope.bands", 0, nullptr, 16, 0}};
  for (const Want &w : want) {
    auto it = tens.find(w.name);
    const bool ok = it != tens.end() && it->second.dtype == w.dtype &&
                    (w.cols ? shape_is(it->second, {w.rows, w.cols}) : shape_is(it->second, {w.rows}));
    if (!ok) return dfail(HXA_E_WEIGHTS, "dit load glue: a tensor is missing or not of the DiT's shape / type");
  }
  DHIP(hipStreamSynchronize(d.st));
  for (const Want &w : want) {
    const GlueTensor &t = tens[w.name];
    if (w.dst) DTRY(upload(w.dst, t.data, (size_t)t.elems() * (w.dtype == 0 ? 4 : 2)));
  }
  memcpy(d.bands, tens["rope.bands"].data, sizeof d.bands);
  DTRY(hxa_ktile4_f32_launch(d.Wfin32, C4, D, d.Wfin4f, d.st));
  std::vector<float> c, sn;
  rope_moss(d.cfg.lat_h / 2, d.cfg.lat_w / 2, d.ntxt, d.Ttot, d.bands, c, sn);
  DTRY(upload(d.cosT, c.data(), 4 * c.size()));
  DTRY(upload(d.sinT, sn.data(), 4 * sn.size()));
  d.ropeL_scale = -1.0;  // the low-res tables are rebuilt with these bands at their next use
  DHIP(hipStreamSynchronize(d.st));
  return HXA_OK;
}

extern "C" void *hxa_dit_stream(void *p) { return p ? (void *)((Dit *)p)->st : nullptr; }
