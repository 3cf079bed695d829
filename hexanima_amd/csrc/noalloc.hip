// hxa_block_run_noalloc: hxa_block_run for callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc). The block workspace -- the only device memory the block needs
// beyond its inputs and outputs -- is a file-scope device array of HXA_NOALLOC_WS_MAX bytes instead of a caller
// buffer, and the call path allocates nothing (no hipMalloc / hipFree / events, no host containers).
//
// Every GPU the library runs on holds its own copy of the array until the process ends. All calls on one GPU share
// it and it keeps the last call's contents: calls that overlap on one GPU (two streams, two threads) race on it and
// must be serialised by the caller. Every workspace buffer the block reads is written earlier in the same call, so
// nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/hexanima_hip.h"
#include "hxa_common.h"
#include "kernels.h"

namespace {
static __device__ __align__(256) uint8_t scratch[HXA_NOALLOC_WS_MAX];

void *g_scratch[HXA_MAX_DEVICES];  // device address of `scratch` on each device (the host name is only a stand-in)
std::mutex g_scratch_mu;
}  // namespace

// Resolves the device address of `scratch` on the current device, once per device.
int hxa_noalloc_setup(void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= HXA_MAX_DEVICES)
    return hxa_set_error(HXA_E_RESOURCE, "noalloc: no current HIP device");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return hxa_set_error(HXA_E_HIP, "noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  if (out) *out = g_scratch[dev];
  return HXA_OK;
}

extern "C" int hxa_block_run_noalloc(const hxa_block_dims *d, const void *pack, float *x, const void *ctx,
                                     const float *mod, const float *cosT, const float *sinT, int stop, void *stream) {
  if (!d) return hxa_set_error(HXA_E_ARG, "block_run_noalloc: null dims");
  const long need = hxa_block_ws_bytes(d);
  if (need <= 0 || need > (long)HXA_NOALLOC_WS_MAX)
    return hxa_set_error(HXA_E_ARG, "block_run_noalloc: the block needs %ld bytes of workspace, the static scratch holds %ld",
                         need, (long)HXA_NOALLOC_WS_MAX);
  void *ws = nullptr;
  const int r = hxa_noalloc_setup(&ws);
  if (r != HXA_OK) return r;
  return hxa_block_run_chained(d, pack, x, ctx, mod, cosT, sinT, ws, stop, nullptr, 0, stream, nullptr, 0);
}
