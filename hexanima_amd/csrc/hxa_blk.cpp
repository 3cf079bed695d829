// hxa_blk: the single-block harness of the reference (hexagon/mega/blk_main.c) on libhexanima_hip.so. It reads one
// block's test files -- what export_block.py writes: x32.bin (x as x32 tiles), ctx16.bin (512 context tokens as fp16
// tiles), mod.bin (9 x 2048 fp32), cos.bin / sin.bin (RoPE tiles), the ten fp16 crouton weight files w_*.bin and
// gain.bin -- runs mega_block REPS times on 1536 tokens (x restored before each), prints each call's wall time and
// per-stage microseconds, and writes the block's output x to DIR/out32.bin (x32 tiles).
//
//   usage: hxa_blk DIR [REPS] [STOP] [NW]      (STOP = meta[M_STOP]: stop after that many stages; NW is accepted)
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "hexanima_hip.h"

namespace {
// blk_meta.h:3-4
enum { M_X = 0, M_CTX, M_MOD, M_GAIN, M_COS, M_SIN, M_WSQ, M_WSK, M_WSV, M_WSO, M_WCQ, M_WCK, M_WCV, M_WCO, M_WM1, M_WM2,
       M_H, M_Q, M_K, M_V, M_O, M_T, M_MID, M_CK, M_CV, M_NTOK, M_NCTX, M_STOP, M_NW, M_REL, M_FIRST, M_Q8, M_NMETA };
constexpr int NTOK = 1536, NCTX = 512, D = 2048;
constexpr size_t W_TOTAL = 138416128u;

bool read_exact(const std::string &dir, const char *name, void *dst, size_t want) {
  const std::string p = dir + "/" + name;
  FILE *f = fopen(p.c_str(), "rb");
  if (!f) return printf("missing %s\n", p.c_str()), false;
  const size_t n = fread(dst, 1, want, f);
  fclose(f);
  if (n != want) return printf("%s: got %zu want %zu\n", name, n, want), false;
  return true;
}
}  // namespace

int main(int argc, char **argv) {
  if (argc < 2) {
    fprintf(stderr, "usage: hxa_blk DIR [REPS] [STOP] [NW]\n");
    return 1;
  }
  const std::string dir = argv[1];
  const int reps = argc > 2 ? atoi(argv[2]) : 1;
  setvbuf(stdout, nullptr, _IONBF, 0);
  int meta[M_NMETA];
  memset(meta, 0, sizeof meta);
  // activations: the blob in the order blk_main lays it out (page aligned); inputs read from files
  struct Act {
    int id;
    const char *file;
    size_t bytes;
  };
  const size_t TD2 = (size_t)NTOK * D * 2;
  const Act acts[] = {{M_X, "x32.bin", (size_t)NTOK * D * 4}, {M_CTX, "ctx16.bin", (size_t)NCTX * 1024 * 2},
                      {M_MOD, "mod.bin", 9 * D * 4},           {M_COS, "cos.bin", (size_t)NTOK / 32 * 8192},
                      {M_SIN, "sin.bin", (size_t)NTOK / 32 * 8192}, {M_H, nullptr, TD2}, {M_Q, nullptr, TD2},
                      {M_K, nullptr, TD2}, {M_V, nullptr, TD2}, {M_O, nullptr, TD2}, {M_T, nullptr, TD2},
                      {M_MID, nullptr, (size_t)NTOK * 8192 * 2}, {M_CK, nullptr, (size_t)NCTX * D * 2},
                      {M_CV, nullptr, (size_t)NCTX * D * 2}};
  size_t off = 0;
  for (const Act &a : acts) {
    meta[a.id] = (int)off;
    off += (a.bytes + 4095) & ~(size_t)4095;
  }
  // weights: the fp16 crouton matrices at their blkNN.bin offsets (blk_wlayout.h:3-13)
  struct Wt {
    int id;
    const char *file;
    uint32_t off;
    size_t bytes;
  };
  const Wt wts[] = {{M_WSQ, "w_sq.bin", 0u, 8388608},        {M_WSK, "w_sk.bin", 8388608u, 8388608},
                    {M_WSV, "w_sv.bin", 16777216u, 8388608}, {M_WSO, "w_so.bin", 25165824u, 8388608},
                    {M_WCQ, "w_cq.bin", 33554432u, 8388608}, {M_WCK, "w_ck.bin", 41943040u, 4194304},
                    {M_WCV, "w_cv.bin", 46137344u, 4194304}, {M_WCO, "w_co.bin", 50331648u, 8388608},
                    {M_WM1, "w_m1.bin", 58720256u, 33554432}, {M_WM2, "w_m2.bin", 92274688u, 33554432},
                    {M_GAIN, "gain.bin", 125829120u, 2048}};
  meta[M_NTOK] = NTOK;
  meta[M_NCTX] = NCTX;
  meta[M_STOP] = argc > 3 ? atoi(argv[3]) : 0;
  meta[M_NW] = argc > 4 ? atoi(argv[4]) : 3;
  meta[M_FIRST] = 1;
  meta[M_REL] = 1;
  std::vector<uint8_t> w(W_TOTAL, 0), blob(off, 0);
  for (const Wt &t : wts) {
    meta[t.id] = (int)t.off;
    if (!read_exact(dir, t.file, w.data() + t.off, t.bytes)) return 1;
  }
  for (const Act &a : acts)
    if (a.file && !read_exact(dir, a.file, blob.data() + meta[a.id], a.bytes)) return 1;
  printf("files read\n");
  const std::vector<uint8_t> x0(blob.begin() + meta[M_X], blob.begin() + meta[M_X] + (size_t)NTOK * D * 4);
  remote_handle64 h = 0;
  if (mega_open("", &h)) return printf("open: %s\n", hxa_last_error()), 1;
  if (hxa_register(h, 1, w.data(), w.size(), HXA_KIND_WEIGHTS_ANIMA) || hxa_register(h, 2, blob.data(), blob.size(), HXA_KIND_BLOB))
    return printf("register: %s\n", hxa_last_error()), 1;
  int status = 0;
  for (int rep = 0; rep < reps; rep++) {
    memcpy(blob.data() + meta[M_X], x0.data(), x0.size());
    int times[32] = {0}, rc = 0;
    const auto a = std::chrono::steady_clock::now();
    const int r = mega_block(h, meta, M_NMETA, 1, 2, blob.data() + meta[M_MOD], 9 * D * 4, times, 32, &rc);
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - a).count();
    printf("rep %d r=0x%x rc=%d total %.2f ms | stages(us):", rep, r, rc, ms);
    for (int i = 0; i < 24; i++) printf(" %d", times[i]);
    printf("\n");
    if (r || rc) {
      printf("error: %s\n", hxa_last_error());
      status = 1;
      break;
    }
  }
  if (status == 0) {
    const std::string p = dir + "/out32.bin";
    FILE *f = fopen(p.c_str(), "wb");
    if (!f || fwrite(blob.data() + meta[M_X], 1, x0.size(), f) != x0.size()) status = 1;
    if (f) fclose(f);
  }
  mega_close(h);
  return status;
}
