// Shared helpers for the lgml_hip kernels and host glue (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/lgml_hip.h"

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

namespace lgmlh {

// Thread-local error text behind lgmlh_last_error().
void set_error(const char *fmt, ...);

// Record a HIP failure; returns LGMLH_EHIP when e != hipSuccess.
int hip_check(hipError_t e, const char *what);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Cells per KV block; the pool layout and the attention tiles assume it.
constexpr int KV_BLOCK = 64;

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (f16)f);  // round to nearest even
}

// Wave64 reductions within groups of 16 lanes (lanes l, l^1, l^2, ...).
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  return v;
}
__device__ __forceinline__ float sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}

}  // namespace lgmlh

#define LGMLH_TRY(x)              \
  do {                            \
    int rc__ = (x);               \
    if (rc__ != LGMLH_OK) return rc__; \
  } while (0)
