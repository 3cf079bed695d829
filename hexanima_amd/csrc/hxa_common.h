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

#define HXA_CHECK(x)                                  \
  do {                                                \
    hipError_t e_ = (x);                              \
    if (e_ != hipSuccess) return HXA_E_HIP;           \
  } while (0)
