// Split activations: the B operand of the quantized GEMM.
//
// A GEMM input X (N rows of K f32 values) is handed over as four planes in
// one buffer, rows padded to Npad = N rounded up to 64:
//   hi [Npad][K]      f16(x)
//   lo [Npad][K]      f16(x - hi)            (x = hi + lo to ~22 bits)
//   gh [Npad][K / 32] f16(S), S = f32 sum of the 32-value group of x
//   gl [Npad][K / 32] f16(S - gh)
// The MFMA products run on hi and lo with exact integer weights, so a
// product is f32-accurate; the group sums feed the Q4_K min term. Rows
// N..Npad-1 are never written: each output column of an MFMA depends on
// its own B column only, and those columns are not stored.
// Values must lie within the f16 range (|x| < 65504).
#pragma once
#include "common.h"

namespace lgmlh {

__host__ __device__ inline int64_t split_npad(int64_t N) { return (N + 63) & ~int64_t(63); }

__host__ __device__ inline size_t split_bytes(int64_t N, int64_t K) {
  const int64_t P = split_npad(N);
  return (size_t)P * K * 2 * 2 + (size_t)P * (K / 32) * 2 * 2;
}

// Stores the 8 values v of row n at columns k0..k0+7 (k0 % 8 == 0). Called
// by the four lanes 4q..4q+3 of a wave that hold one 32-value group, in
// order of k0 (the group sum is taken across them).
__device__ __forceinline__ void split_store8(f16 *__restrict__ planes, int64_t Npad, int64_t K,
                                             int64_t n, int64_t k0, const float (&v)[8]) {
  f16x8 h, l;
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) {
    h[e] = (f16)v[e];
    l[e] = (f16)(v[e] - (float)h[e]);
    s += v[e];
  }
  f16 *hp = planes + n * K + k0;
  *(f16x8 *)hp = h;
  *(f16x8 *)(hp + Npad * K) = l;
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  if (((k0 >> 3) & 3) == 0) {
    f16 *g = planes + 2 * Npad * K + n * (K / 32) + (k0 >> 5);
    f16 sh = (f16)s;
    g[0] = sh;
    g[Npad * (K / 32)] = (f16)(s - (float)sh);
  }
}

// Stores 4 values of row n at columns k0..k0+3 (k0 % 4 == 0), hi and lo;
// the group sum goes separately (split_store_gsum).
__device__ __forceinline__ void split_store4(f16 *__restrict__ planes, int64_t Npad, int64_t K,
                                             int64_t n, int64_t k0, const float (&v)[4]) {
  f16x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    h[e] = (f16)v[e];
    l[e] = (f16)(v[e] - (float)h[e]);
  }
  f16 *hp = planes + n * K + k0;
  *(f16x4 *)hp = h;
  *(f16x4 *)(hp + Npad * K) = l;
}

// Stores the sum s of group g (columns 32 g .. 32 g + 31) of row n.
__device__ __forceinline__ void split_store_gsum(f16 *__restrict__ planes, int64_t Npad,
                                                 int64_t K, int64_t n, int64_t g, float s) {
  f16 *gp = planes + 2 * Npad * K + n * (K / 32) + g;
  const f16 sh = (f16)s;
  gp[0] = sh;
  gp[Npad * (K / 32)] = (f16)(s - (float)sh);
}

}  // namespace lgmlh
