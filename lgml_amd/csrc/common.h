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

// Split-K partial sums of a product not yet reduced: part[z][n][m] for
// z < splits, n < rows, m < cols (cols = the product's M). The consumer
// adds them in the canonical order: runs of `group` consecutive partials
// first (a run's sum starts from its first partial), then the runs in
// order from 0, then the residual, if any. (group 2: one partial per K
// split, the splits pair up; group 1: one per pair, already added.)
// With wts set, the terms are the expert outputs of a token's picks
// instead: part[n][z][m] times wts[n][z] for the splits = n_used picks.
// With post set (gemma post norms), the consumer adds rms_norm(sum) * post
// rather than the sum; then, with scale != 0, multiplies the new residual
// by scale (the layer output scale).
struct Pending {
  const float *part = nullptr;
  int splits = 0;
  int64_t rows = 0, cols = 0;
  const float *wts = nullptr;
  const float *post = nullptr;
  float scale = 0.0f;
  int group = 1;
  __device__ __forceinline__ float sum(int64_t n, int64_t m) const {
    float v = 0.0f;
    if (wts) {
      for (int z = 0; z < splits; z++)
        v += part[((int64_t)n * splits + z) * cols + m] * wts[(int64_t)n * splits + z];
      return v;
    }
    const int64_t zs = rows * cols;
    const float *p = part + n * cols + m;
    for (int z = 0; z < splits; z += group) {
      float g = p[z * zs];
      for (int i = 1; i < group && z + i < splits; i++) g += p[(z + i) * zs];
      v += g;
    }
    return v;
  }
  // The sums at (n, m0 .. m0 + 7), m0 % 4 == 0 and cols % 4 == 0: 16-byte
  // loads, up to four partials in flight, added in the canonical order.
  __device__ __forceinline__ void sum8(int64_t n, int64_t m0, float (&v)[8]) const {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (wts) {
      const float *p = part + (int64_t)n * splits * cols + m0;
      const float *wp = wts + (int64_t)n * splits;
      for (int z = 0; z < splits; z++, p += cols) {
        const float wz = wp[z];
        const f4 a0 = *(const f4 *)p, b0 = *(const f4 *)(p + 4);
        a += a0 * wz;
        b += b0 * wz;
      }
    } else {
      const float *p = part + n * cols + m0;
      const int64_t zs = rows * cols;
      int z = 0;
      // eight partials in flight at once (all loads before the adds)
      for (; z + 8 <= splits; z += 8, p += 8 * zs) {
        f4 ai[8], bi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          ai[i] = *(const f4 *)(p + i * zs);
          bi[i] = *(const f4 *)(p + i * zs + 4);
        }
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          if (group == 2) {
            a += ai[i] + ai[i + 1];
            b += bi[i] + bi[i + 1];
          } else {
            a += ai[i];
            b += bi[i];
            a += ai[i + 1];
            b += bi[i + 1];
          }
        }
      }
      if (group == 2) {
        for (; z + 4 <= splits; z += 4, p += 4 * zs) {
          const f4 a0 = *(const f4 *)p, b0 = *(const f4 *)(p + 4);
          const f4 a1 = *(const f4 *)(p + zs), b1 = *(const f4 *)(p + zs + 4);
          const f4 a2 = *(const f4 *)(p + 2 * zs), b2 = *(const f4 *)(p + 2 * zs + 4);
          const f4 a3 = *(const f4 *)(p + 3 * zs), b3 = *(const f4 *)(p + 3 * zs + 4);
          a += a0 + a1;
          b += b0 + b1;
          a += a2 + a3;
          b += b2 + b3;
        }
        for (; z + 2 <= splits; z += 2, p += 2 * zs) {
          const f4 a0 = *(const f4 *)p, b0 = *(const f4 *)(p + 4);
          const f4 a1 = *(const f4 *)(p + zs), b1 = *(const f4 *)(p + zs + 4);
          a += a0 + a1;
          b += b0 + b1;
        }
      } else {
        for (; z + 4 <= splits; z += 4, p += 4 * zs) {
          const f4 a0 = *(const f4 *)p, b0 = *(const f4 *)(p + 4);
          const f4 a1 = *(const f4 *)(p + zs), b1 = *(const f4 *)(p + zs + 4);
          const f4 a2 = *(const f4 *)(p + 2 * zs), b2 = *(const f4 *)(p + 2 * zs + 4);
          const f4 a3 = *(const f4 *)(p + 3 * zs), b3 = *(const f4 *)(p + 3 * zs + 4);
          a += a0;
          b += b0;
          a += a1;
          b += b1;
          a += a2;
          b += b2;
          a += a3;
          b += b3;
        }
      }
      for (; z < splits; z++, p += zs) {  // a last run of one
        a += *(const f4 *)p;
        b += *(const f4 *)(p + 4);
      }
    }
    for (int e = 0; e < 4; e++) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  }
  // The same at (n, m0 .. m0 + 3): the values of sum8's halves, for callers
  // that spread a row over more lanes.
  __device__ __forceinline__ void sum4(int64_t n, int64_t m0, float (&v)[4]) const {
    typedef float f4 __attribute__((ext_vector_type(4)));
    f4 a = {0.0f, 0.0f, 0.0f, 0.0f};
    if (wts) {
      const float *p = part + (int64_t)n * splits * cols + m0;
      const float *wp = wts + (int64_t)n * splits;
      for (int z = 0; z < splits; z++, p += cols) a += *(const f4 *)p * wp[z];
    } else {
      const float *p = part + n * cols + m0;
      const int64_t zs = rows * cols;
      int z = 0;
      // eight partials in flight at once (all loads before the adds)
      for (; z + 8 <= splits; z += 8, p += 8 * zs) {
        f4 ai[8];
#pragma unroll
        for (int i = 0; i < 8; i++) ai[i] = *(const f4 *)(p + i * zs);
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          if (group == 2) {
            a += ai[i] + ai[i + 1];
          } else {
            a += ai[i];
            a += ai[i + 1];
          }
        }
      }
      if (group == 2) {
        for (; z + 2 <= splits; z += 2, p += 2 * zs) {
          const f4 a0 = *(const f4 *)p, a1 = *(const f4 *)(p + zs);
          a += a0 + a1;
        }
      } else {
        for (; z + 4 <= splits; z += 4, p += 4 * zs) {
          const f4 a0 = *(const f4 *)p, a1 = *(const f4 *)(p + zs);
          const f4 a2 = *(const f4 *)(p + 2 * zs), a3 = *(const f4 *)(p + 3 * zs);
          a += a0;
          a += a1;
          a += a2;
          a += a3;
        }
      }
      for (; z < splits; z++, p += zs) a += *(const f4 *)p;
    }
    for (int e = 0; e < 4; e++) v[e] = a[e];
  }
};

// Cells per KV block; the pool layout and the attention tiles assume it.
constexpr int KV_BLOCK = 64;
// Query groups per shared attention run (lgmlh_plan's sets; the waves of
// the shared attention kernel).
constexpr int ATTN_SHARED = 8;

__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (f16)f);  // round to nearest even
}

// A lane reads another lane's value of its row of 16 by a DPP modifier on a
// VALU move (no trip through the LDS unit, as a shuffle takes). gfx9
// encodings: quad_perm [1,0,3,2] = lane ^ 1, [2,3,0,1] = lane ^ 2 (the
// same lanes as those shuffles, so sums keep their order and bits);
// row_half_mirror (lane 7 - i of its 8) and row_mirror (15 - i of its 16)
// pair other lanes, for reductions whose result does not depend on the
// order (max, exact integer sums).
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The largest v over aligned groups of W lanes (W = 2 .. 64, a power of
// two): after the quad steps every lane holds its quad's max, the mirrors
// pair the quads of 8 and the halves of 16, shuffles the rest.
template <int W>
__device__ __forceinline__ float group_max(float v) {
  static_assert(W >= 2 && W <= 64 && (W & (W - 1)) == 0, "group width");
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  if constexpr (W > 2) v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  if constexpr (W > 4) v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  if constexpr (W > 8) v = fmaxf(v, dpp_f<DPP_MIRROR>(v));
  if constexpr (W > 16) v = fmaxf(v, __shfl_xor(v, 16));
  if constexpr (W > 32) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// The signed value of the first element, in order of (lane, index), of an
// aligned group of W lanes holding E values each whose |value| is amax (the
// group's largest |value|, > 0; with amax = 0 the result is 0 or a zero of
// either sign). Every lane of the group gets it.
template <int W, int E>
__device__ __forceinline__ float group_first_abs(const float (&v)[E], float amax) {
  float mine = 0.0f;
  bool has = false;
#pragma unroll
  for (int e = E - 1; e >= 0; e--)
    if (fabsf(v[e]) == amax) {
      mine = v[e];
      has = true;
    }
  const int lane = __lane_id();
  const int base = lane & ~(W - 1);
  const unsigned long long bal = __ballot(has);
  const unsigned long long grp = W == 64 ? bal : (bal >> base) & ((1ull << W) - 1);
  const int src = base + (grp ? __builtin_ctzll(grp) : 0);
  return __shfl(mine, src);
}

}  // namespace lgmlh

#define LGMLH_TRY(x)              \
  do {                            \
    int rc__ = (x);               \
    if (rc__ != LGMLH_OK) return rc__; \
  } while (0)
