// Quantized block formats on the device (the public ggml layouts):
//   Q4_K: 256 values, 144 B {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}
//   Q6_K: 256 values, 210 B {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}
//   Q8_0:  32 values,  34 B {f16 d; i8 qs[32]}
// The closed forms below are bit-exact with the CPU reference with or
// without FMA contraction: d*sc*q is exact in f32 for Q4_K, and the Q6_K
// and Q8_0 forms have no add.
#pragma once
#include "common.h"

namespace lgmlh {

constexpr int QK_K = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8_0_BYTES = 34;

__host__ __device__ inline int64_t row_bytes(int type, int64_t n) {
  switch (type) {
    case LGMLH_F32: return n * 4;
    case LGMLH_F16: return n * 2;
    case LGMLH_Q8_0: return n % 32 ? -1 : n / 32 * Q8_0_BYTES;
    case LGMLH_Q4_K: return n % QK_K ? -1 : n / QK_K * Q4K_BYTES;
    case LGMLH_Q6_K: return n % QK_K ? -1 : n / QK_K * Q6K_BYTES;
  }
  return -1;
}

__device__ __forceinline__ uint16_t ld16(const uint8_t *p) {
  return (uint16_t)(p[0] | (p[1] << 8));
}

// Scale and min of 32-group j (0..7) from the 12 packed scale bytes.
__device__ __forceinline__ void q4k_scale_min(int j, const uint8_t *s, int &sc, int &m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// Value v (0..255) of a Q4_K super-block.
__device__ __forceinline__ float q4k_value(const uint8_t *b, int v) {
  float d = h2f(ld16(b)), dmin = h2f(ld16(b + 2));
  int sc, m;
  q4k_scale_min(v >> 5, b + 4, sc, m);
  int byte = b[16 + 32 * (v >> 6) + (v & 31)];
  int q = (v & 32) ? (byte >> 4) : (byte & 15);
  float d1 = d * (float)sc, m1 = dmin * (float)m;
  return d1 * (float)q - m1;
}

// Value v (0..255) of a Q6_K super-block.
__device__ __forceinline__ float q6k_value(const uint8_t *b, int v) {
  int h = v >> 7, r = v & 127, t = r >> 5, l = r & 31;
  int lo = b[64 * h + l + 32 * (t & 1)];
  lo = t < 2 ? (lo & 15) : (lo >> 4);
  int hb = (b[128 + 32 * h + l] >> (2 * t)) & 3;
  int q = (lo | (hb << 4)) - 32;
  float d = h2f(ld16(b + 208));
  float sc = (float)(int8_t)b[192 + (v >> 4)];
  return d * sc * (float)q;
}

// Value v (0..31) of a Q8_0 block.
__device__ __forceinline__ float q8_0_value(const uint8_t *b, int v) {
  return h2f(ld16(b)) * (float)(int8_t)b[2 + v];
}

// Element k of a row in `type` (ggml layout).
__device__ __forceinline__ float row_value(int type, const uint8_t *row, int64_t k) {
  switch (type) {
    case LGMLH_F32: return ((const float *)row)[k];
    case LGMLH_F16: return h2f(((const uint16_t *)row)[k]);
    case LGMLH_Q4_K: return q4k_value(row + (k / QK_K) * Q4K_BYTES, (int)(k % QK_K));
    case LGMLH_Q6_K: return q6k_value(row + (k / QK_K) * Q6K_BYTES, (int)(k % QK_K));
    case LGMLH_Q8_0: return q8_0_value(row + (k / 32) * Q8_0_BYTES, (int)(k % 32));
  }
  return 0.0f;
}

}  // namespace lgmlh
