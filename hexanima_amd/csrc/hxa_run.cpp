// hxa_run: the megarun protocol (hexagon/mega/megarun.cpp) on libhexanima_hip.so -- the process that sits directly
// above the block ABI in the Anima pipeline. It holds COUNT blocks' weights (blkNN.bin, fp16 crouton or q8 records,
// told apart by size) registered with the library, where they are converted once and stay resident in HBM.
//
//   usage: hxa_run HMXDIR [FIRST COUNT]
//   stdin: "run X_IN EMB LORA CTX X_OUT [GH GW] [SKIPMASK]" -> stdout "done <ms>" (or "error"); "quit"
//     X_IN / X_OUT fp32 [2048][T] (T = GH * GW, default 48 x 32), or x32 tiles when the name ends in ".x32";
//     EMB fp32 [2048], LORA fp32 [6144], CTX fp32 [1024][512]; bit i of SKIPMASK skips block i (x passes through)
//
// Per run, as megarun does: the activation blob is (re)built for T tokens (RoPE tables, fp16 context tiles, x32
// tiles), the 9 x 2048 modulation of every block is computed -- here on the GPU (hxa_anima_modulation) -- and
// mega_block runs the blocks in order, FIRST on the first block run and REL on the last.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "hexanima_hip.h"

namespace {
constexpr int D = 2048, NCTX = 512, TMAX = 6144;
// blk_meta.h:3-4
enum { M_X = 0, M_CTX, M_MOD, M_GAIN, M_COS, M_SIN, M_WSQ, M_WSK, M_WSV, M_WSO, M_WCQ, M_WCK, M_WCV, M_WCO, M_WM1, M_WM2,
       M_H, M_Q, M_K, M_V, M_O, M_T, M_MID, M_CK, M_CV, M_NTOK, M_NCTX, M_STOP, M_NW, M_REL, M_FIRST, M_Q8, M_NMETA };
// weight offsets inside blkNN.bin (blk_wlayout.h:3-20): fp16 crouton files, q8 files scale them by 1152 / 2048
constexpr uint32_t W_OFF[11] = {0u, 8388608u, 16777216u, 25165824u, 33554432u, 41943040u, 46137344u, 50331648u,
                                58720256u, 92274688u, 125829120u};  // SQ SK SV SO CQ CK CV CO M1 M2 GAIN
constexpr size_t W_TOTAL = 138416128u, WQ_TOTAL = 125829120u / 2048u * 1152u + 4096u + (138416128u - 125833216u);

double now_s() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }
size_t up4k(size_t x) { return (x + 4095) & ~(size_t)4095; }

bool read_file(const std::string &path, std::vector<char> &buf) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f) return false;
  fseek(f, 0, SEEK_END);
  const long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  buf.resize(n > 0 ? (size_t)n : 0);
  const bool ok = n >= 0 && fread(buf.data(), 1, buf.size(), f) == buf.size();
  fclose(f);
  return ok;
}

uint16_t f32_to_f16(float f) {  // round to nearest even
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sgn = (x >> 16) & 0x8000u;
  x &= 0x7fffffffu;
  if (x > 0x7f800000u) return (uint16_t)(sgn | 0x7e00u);
  if (x >= 0x477ff000u) return (uint16_t)(sgn | 0x7c00u);
  if (x >= 0x38800000u) {
    uint32_t h = (((x >> 23) - 112u) << 10) | ((x & 0x7fffffu) >> 13);
    const uint32_t rem = x & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sgn | h);
  }
  return (uint16_t)(sgn | (uint32_t)nearbyintf(fabsf(f) * 16777216.0f));
}

// Blob layout for T tokens: x (x32 tiles), ctx (fp16 tiles), cos / sin ([slab][2][32][32] fp32), page aligned.
// The stage buffers exist only for M_STOP dumps, which this runner does not request.
struct Blob {
  std::vector<uint8_t> mem;
  int meta[M_NMETA];
  int T = 0;
};
void layout(Blob &b, int T, bool q8) {
  memset(b.meta, 0, sizeof b.meta);
  size_t off = 0;
  auto put = [&](int id, size_t bytes) {
    b.meta[id] = (int)off;
    off += up4k(bytes);
  };
  put(M_X, (size_t)T * D * 4);
  put(M_CTX, (size_t)NCTX * 1024 * 2);
  put(M_COS, (size_t)T / 32 * 2 * 1024 * 4);
  put(M_SIN, (size_t)T / 32 * 2 * 1024 * 4);
  for (int id : {M_H, M_Q, M_K, M_V, M_O, M_T, M_MID, M_CK, M_CV}) b.meta[id] = -1;
  for (int i = 0; i < 11; i++) b.meta[i == 10 ? M_GAIN : M_WSQ + i] = (int)(q8 ? W_OFF[i] / 2048u * 1152u : W_OFF[i]);
  b.meta[M_MOD] = -1;  // the modulation travels by value (megarun.cpp:181)
  b.meta[M_Q8] = q8;
  b.meta[M_NTOK] = T;
  b.meta[M_NCTX] = NCTX;
  b.meta[M_NW] = 3;
  if (b.mem.size() < off) b.mem.assign(off, 0);
  b.T = T;
}

// RoPE tables of a gh x gw grid (megarun.cpp:77-90): 64 angles per token, 22 zero (t axis), 21 h, 21 w frequencies
// of 10000^(-2i/42); stored as tiles [slab][j][32 rows][32 cols], angle d = 32 j + col
void rope_tiles(int gh, int gw, float *cs, float *sn) {
  const int dh = 128 / 6 * 2, nt = (128 - 2 * dh) / 2, nh = dh / 2;
  double freq[64];
  for (int i = 0; i < nh; i++) freq[i] = 1.0 / pow(10000.0, 2.0 * i / dh);
  for (int tk = 0; tk < gh * gw; tk++)
    for (int d = 0; d < 64; d++) {
      const int y = tk / gw, x = tk % gw;
      double a = 0.0;
      if (d >= nt + nh) a = x * freq[d - nt - nh];
      else if (d >= nt) a = y * freq[d - nt];
      const size_t i = ((size_t)(tk / 32) * 2 + d / 32) * 1024 + (tk % 32) * 32 + d % 32;
      cs[i] = (float)cos(a);
      sn[i] = (float)sin(a);
    }
}
// [D][T] fp32 <-> x32 tiles [T/32][D/32][32 tokens][32 channels]
void cols_to_x32(const float *src, float *tiles, int T) {
  for (int c = 0; c < D; c++)
    for (int t = 0; t < T; t++) tiles[((size_t)(t / 32) * (D / 32) + c / 32) * 1024 + (t % 32) * 32 + c % 32] = src[(size_t)c * T + t];
}
void x32_to_cols(const float *tiles, float *dst, int T) {
  for (int c = 0; c < D; c++)
    for (int t = 0; t < T; t++) dst[(size_t)c * T + t] = tiles[((size_t)(t / 32) * (D / 32) + c / 32) * 1024 + (t % 32) * 32 + c % 32];
}
// context fp32 [1024 channels][512 tokens] -> fp16 h16 tiles of the [512][1024] matrix (halfword (r/2)*64 + c*2 + r%2)
void ctx_to_h16(const float *ct, uint16_t *tiles) {
  for (int c = 0; c < 1024; c++)
    for (int i = 0; i < NCTX; i++)
      tiles[((size_t)(i / 32) * 32 + c / 32) * 1024 + ((i % 32) / 2) * 64 + (c % 32) * 2 + i % 2] = f32_to_f16(ct[(size_t)c * NCTX + i]);
}
}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: hxa_run HMXDIR [FIRST COUNT]\n");
    return 1;
  }
  const std::string dir = argv[1];
  const int first = argc > 2 ? atoi(argv[2]) : 0, count = argc > 3 ? atoi(argv[3]) : 28;
  if (count < 1 || first < 0) return fprintf(stderr, "bad block range\n"), 1;
  const double t0 = now_s();
  std::vector<std::vector<char>> wts(count);
  bool q8 = false;
  for (int i = 0; i < count; i++) {
    char p[1024];
    snprintf(p, sizeof p, "%s/blk%02d.bin", dir.c_str(), first + i);
    if (!read_file(p, wts[i])) return fprintf(stderr, "cannot load %s\n", p), 1;
    const bool this_q8 = wts[i].size() == WQ_TOTAL;
    if (!this_q8 && wts[i].size() != W_TOTAL) return fprintf(stderr, "%s: %zu bytes is not a block file\n", p, wts[i].size()), 1;
    if (i > 0 && this_q8 != q8) return fprintf(stderr, "%s: fp16 and q8 blocks mixed\n", p), 1;
    q8 = this_q8;
  }
  remote_handle64 h = 0;
  if (mega_open("", &h)) return fprintf(stderr, "mega_open: %s\n", hxa_last_error()), 1;
  std::vector<int> wfd(count);
  for (int i = 0; i < count; i++) {
    wfd[i] = 1000 + first + i;
    if (hxa_register(h, wfd[i], wts[i].data(), wts[i].size(), HXA_KIND_WEIGHTS_ANIMA))
      return fprintf(stderr, "register block %d: %s\n", first + i, hxa_last_error()), 1;
  }
  fprintf(stderr, "hxa_run: %d %s blocks loaded %.1fs\n", count, q8 ? "q8" : "fp16", now_s() - t0);
  printf("ready\n");
  fflush(stdout);

  const int BLOB_FD = 1;
  Blob blob;
  int cur_gh = -1, cur_gw = -1;
  std::vector<float> mod((size_t)count * 9 * D), xcols((size_t)D * TMAX);
  std::string line;
  while (std::getline(std::cin, line)) {
    std::istringstream ss(line);
    std::string cmd;
    ss >> cmd;
    if (cmd == "quit") break;
    if (cmd != "run") continue;
    std::string xi, em, lo, cx, xo;
    int gh = 48, gw = 32;
    unsigned skip = 0;
    ss >> xi >> em >> lo >> cx >> xo >> gh >> gw >> skip;
    const int T = gh * gw;
    std::vector<char> xb, eb, lb, cb;
    const bool rd = read_file(xi, xb) && read_file(em, eb) && read_file(lo, lb) && read_file(cx, cb);
    if (!rd || gh <= 0 || gw <= 0 || T % 32 || T > TMAX || xb.size() != (size_t)D * T * 4 || eb.size() != (size_t)D * 4 ||
        lb.size() != 6144 * 4 || cb.size() != (size_t)1024 * NCTX * 4) {
      fprintf(stderr, "bad input T=%d\n", T);
      printf("error\n");
      fflush(stdout);
      continue;
    }
    const double ts = now_s();
    if (T != blob.T) {
      const size_t had = blob.mem.size();
      layout(blob, T, q8);
      if (blob.mem.size() != had && hxa_register(h, BLOB_FD, blob.mem.data(), blob.mem.size(), HXA_KIND_BLOB)) {
        fprintf(stderr, "register blob: %s\n", hxa_last_error());
        printf("error\n");
        fflush(stdout);
        continue;
      }
      cur_gh = -1;
    }
    uint8_t *B = blob.mem.data();
    if (gh != cur_gh || gw != cur_gw) {
      rope_tiles(gh, gw, (float *)(B + blob.meta[M_COS]), (float *)(B + blob.meta[M_SIN]));
      cur_gh = gh;
      cur_gw = gw;
    }
    ctx_to_h16((const float *)cb.data(), (uint16_t *)(B + blob.meta[M_CTX]));
    const bool x_tiled = xi.size() > 4 && xi.compare(xi.size() - 4, 4, ".x32") == 0;
    if (x_tiled) memcpy(B + blob.meta[M_X], xb.data(), xb.size());
    else cols_to_x32((const float *)xb.data(), (float *)(B + blob.meta[M_X]), T);
    const double t_conv = now_s();
    bool ok = hxa_anima_modulation(h, wfd.data(), count, (const float *)eb.data(), (const float *)lb.data(), mod.data()) == 0;
    if (!ok) fprintf(stderr, "modulation: %s\n", hxa_last_error());
    int first_run = -1, last_run = -1;
    for (int k = 0; k < count; k++)
      if (!((skip >> (first + k)) & 1u)) {
        if (first_run < 0) first_run = k;
        last_run = k;
      }
    // stage times are asked for where they are read: block 5 under HXA_RUN_DBG, as megarun logs them under MEGA_DBG
    // (megarun.cpp:182); a call without times returns once its block is queued, so the chain runs back to back
    int times[32];
    const bool dbg = getenv("HXA_RUN_DBG") != nullptr;
    for (int k = 0; k < count && ok; k++) {
      if ((skip >> (first + k)) & 1u) continue;
      blob.meta[M_FIRST] = k == first_run;
      blob.meta[M_REL] = k == last_run;
      int rc = 0;
      const bool timed = dbg && k == 5;
      const double tm1 = now_s();
      const int r = mega_block(h, blob.meta, M_NMETA, wfd[k], BLOB_FD, (const uint8_t *)&mod[(size_t)k * 9 * D], 9 * D * 4,
                               timed ? times : nullptr, timed ? 32 : 0, &rc);
      if (r || rc) {
        fprintf(stderr, "block %d failed r=%d rc=%d: %s\n", first + k, r, rc, hxa_last_error());
        ok = false;
      } else if (timed) {
        fprintf(stderr, "blk5 stages(us):");
        for (int q = 0; q < 25; q++) fprintf(stderr, " %d", times[q]);
        fprintf(stderr, " | call %.1f ms\n", (now_s() - tm1) * 1e3);
      }
    }
    const double t_blocks = now_s();
    if (!ok) {
      printf("error\n");
      fflush(stdout);
      continue;
    }
    const bool out_tiled = xo.size() > 4 && xo.compare(xo.size() - 4, 4, ".x32") == 0;
    const float *xt = (const float *)(B + blob.meta[M_X]);
    if (!out_tiled) x32_to_cols(xt, xcols.data(), T);
    FILE *f = fopen(xo.c_str(), "wb");
    const bool wrote = f && fwrite(out_tiled ? (const void *)xt : (const void *)xcols.data(), 4, (size_t)D * T, f) == (size_t)D * T;
    if (f) fclose(f);
    if (!wrote) {
      printf("error\n");
      fflush(stdout);
      continue;
    }
    const double t_end = now_s();
    if (getenv("HXA_RUN_DBG"))
      fprintf(stderr, "run: in+conv %.1f ms, modulation+blocks %.1f ms, out %.1f ms\n", (t_conv - ts) * 1e3,
              (t_blocks - t_conv) * 1e3, (t_end - t_blocks) * 1e3);
    printf("done %.0f\n", (t_end - ts) * 1000);
    fflush(stdout);
  }
  mega_close(h);
  return 0;
}
