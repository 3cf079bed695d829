// Shared definitions for the MI355X (gfx950) kernels of the DiT block runner.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 hxa_h;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

#define HXA_DEV __device__ __forceinline__

// status codes, weight formats (HXA_W_*) and GEMM epilogues (HXA_EPI_*) are those of the public C-ABI
#include "../../include/hexanima_hip.h"

struct HxaWeight {
  int fmt;            // HXA_W_*
  int N, K;
  const void *w;      // fp16 [N][K] | int8 [N][K] | packed int4 [N][K/2]
  const hxa_h *s;     // [K/32][N] scales (q8, q4)
  const hxa_h *z;     // [K/32][N] q4 offsets (optional)
};

// ---- direct-to-LDS loads and VMEM waits (gfx950) ----
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gmem_void_t;

// s_waitcnt vmcnt(N) only (expcnt / lgkmcnt left at their maxima); encoding of gfx9: vmcnt[3:0] | vmcnt_hi[15:14]
template <int N>
HXA_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// 16 bytes per lane from global memory straight into LDS: lane l writes lds_base + 16 l
HXA_DEV void g2l16(const void *g, void *lds_base) {
  __builtin_amdgcn_global_load_lds((gmem_void_t *)g, (lds_void_t *)lds_base, 16, 0, 0);
}

// global_load_lds_dwordx4 issued from inline asm: lane l's 16 bytes land at LDS byte address lds_addr + 16 l (M0).
// The compiler does not see this as an LDS write, so it keeps exact lgkmcnt waits for the fragment reads around it
// (it falls back to lgkmcnt(0) while a visible LDS DMA is in flight). Completion is awaited explicitly (vmcnt(0) and
// a barrier) before any wave reads the tile; LDS reads complete in order, so these loads can only lengthen an
// lgkmcnt wait, never satisfy one early.
HXA_DEV void g2l16_opaque(const void *g, const void *lds_ptr) {
  const uint32_t la = (uint32_t)(uintptr_t)(lds_void_t *)lds_ptr;
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(la) : "memory", "m0");
}

#define HXA_CHECK(x)                                  \
  do {                                                \
    hipError_t e_ = (x);                              \
    if (e_ != hipSuccess) return HXA_E_HIP;           \
  } while (0)
