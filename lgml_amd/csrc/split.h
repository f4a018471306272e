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

// ---- quantized activations ---------------------------------------------------
// ggml's CPU backend quantizes X to the weight type's vec_dot_type before a
// quantized product (Q8_K for Q4_K / Q6_K, Q8_0 for Q8_0) and takes integer
// dots per block. In that mode (lgmlh_model.act = LGMLH_ACT_GGML) a product
// takes its X as these planes, rows padded to Npad:
//   q  [Npad][K]       f16 of the int8 q (exact)
//   bs [Npad][K / 16]  f16 of the Q8_K sums of 16 q (|s| <= 2032, exact)
//   d  [Npad][K / QB]  f32 block scales: Q8_K d (QB = 256); Q8_0 the f16 d
//                      widened to f32 (QB = 32)
// They fit in split_bytes(N, K).
enum { XF_SPLIT = 0, XF_Q8K = 1, XF_Q80 = 2 };

__host__ __device__ inline int64_t q8_bs_off(int64_t Npad, int64_t K) { return Npad * K; }
__host__ __device__ inline size_t q8_d_off(int64_t Npad, int64_t K) {  // bytes
  return (size_t)Npad * K * 2 + (size_t)Npad * (K / 16) * 2;
}

// One step of a Q8_K block's maximum across lanes (quantize_row_q8_K: the
// value of largest |x|, ties to its first occurrence in the block): amax,
// the signed value and its index in the block, merged with lane ^ o.
__device__ __forceinline__ void q8k_amax_step(float &amax, float &mx, int &at, int o) {
  const float a2 = __shfl_xor(amax, o), m2 = __shfl_xor(mx, o);
  const int i2 = __shfl_xor(at, o);
  if (a2 > amax || (a2 == amax && i2 < at)) {
    amax = a2;
    mx = m2;
    at = i2;
  }
}

// quantize_row_q8_K of one 256-value block held by 32 aligned lanes (lane j
// of the group: values 8j .. 8j + 7). amax = the largest |x|, its first
// occurrence gives the signed max; iscale = -127 / max; q = min(127,
// nearest-even(iscale x)); d = 1 / iscale; an all-zero block has q = 0, d =
// 0. bs: the sum of the 16 q of the lane pair (j & ~1, j | 1).
__device__ __forceinline__ void q8k_block8(const float (&v)[8], float (&q)[8], float &d,
                                           float &bs) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));  // NaN never counts
  amax = group_max<32>(amax);
  const float mx = group_first_abs<32, 8>(v, amax);
  float s = 0.0f;
  if (amax == 0.0f) {
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = 0.0f;
    d = 0.0f;
  } else {
    const float iscale = -127.0f / mx;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      q[e] = fminf(127.0f, __builtin_rintf(iscale * v[e]));
      s += q[e];
    }
    d = 1.0f / iscale;
  }
  bs = s + dpp_f<DPP_XOR1>(s);
}

// quantize_row_q8_0 of one 32-value block held by 4 lanes (lane j: values
// 8j .. 8j + 7): d = amax / 127, id = d ? 1 / d : 0, q = roundf(x id)
// (ties away from zero); d is kept as f16 (dh, its bits) and f32(dh).
__device__ __forceinline__ void q80_block8(const float (&v)[8], float (&q)[8], float &d,
                                           uint16_t &dh) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
  amax = group_max<4>(amax);
  const float dd = amax / 127.0f;
  const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
#pragma unroll
  for (int e = 0; e < 8; e++) q[e] = __builtin_roundf(v[e] * id);
  const f16 h = (f16)dd;
  dh = __builtin_bit_cast(uint16_t, h);
  d = (float)h;
}

// Stores the 8 values v of row n at columns k0..k0+7 in the form xf. The
// lanes of a block call it together, in order of k0: 4 for XF_SPLIT and
// XF_Q80, 32 for XF_Q8K (all of them active).
__device__ __forceinline__ void act_store8(int xf, f16 *__restrict__ planes, int64_t Npad,
                                           int64_t K, int64_t n, int64_t k0, const float (&v)[8]) {
  if (xf == XF_SPLIT) {
    split_store8(planes, Npad, K, n, k0, v);
    return;
  }
  float q[8], d;
  f16x8 h;
  float *dp = (float *)((char *)planes + q8_d_off(Npad, K));
  if (xf == XF_Q8K) {
    float bs;
    q8k_block8(v, q, d, bs);
    if ((k0 & 15) == 0) planes[q8_bs_off(Npad, K) + n * (K / 16) + (k0 >> 4)] = (f16)bs;
    if ((k0 & 255) == 0) dp[n * (K / 256) + (k0 >> 8)] = d;
  } else {
    uint16_t dh;
    q80_block8(v, q, d, dh);
    if ((k0 & 31) == 0) dp[n * (K / 32) + (k0 >> 5)] = d;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) h[e] = (f16)q[e];
  *(f16x8 *)(planes + n * K + k0) = h;
}

// Host side (gemm.hip): the X form of a weight type under an act mode;
// products on planes; planes from f32 / f16 rows.
int xf_for(int type, int act);
int mul_mat_split(int type, const void *w, int64_t M, int64_t K, const f16 *xs, int64_t N,
                  float *y, int64_t ldy, const float *residual, float *part, size_t part_bytes,
                  hipStream_t st, Pending *deferred, int xf);
int mul_mat_grouped(int type, const void *w, int64_t expert_bytes, int64_t M, int64_t K,
                    const f16 *xs, int64_t Npad, int n_used, int U, const int32_t *sorted,
                    const int4 *tiles, const int32_t *n_tiles, int max_tiles, int tile_cols,
                    float *y, hipStream_t st, int xf);
int split_x(const void *x, int xtype, int64_t N, int64_t K, f16 *xs, hipStream_t st, int xf);

}  // namespace lgmlh
