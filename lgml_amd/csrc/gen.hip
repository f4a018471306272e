// Seeded random-init weights on the device, in the ggml block layouts: the
// "normal" fill of tensor:fill (src/lgml.c:3064-3079,3130-3136: splitmix64
// pairs through Box-Muller) followed by a quantizer (lgml.quantize,
// src/quant.c:107). splitmix64's state after j draws is seed + j * gamma,
// so value i (draws 2i+1 and 2i+2) needs no sequential pass and each
// thread makes one block. The quantizers are this library's own: per
// 32-value groups an affine (Q4_K) or symmetric (Q6_K, Q8_0) range with
// scales relative to the super-block maximum.
#include <math.h>

#include "common.h"
#include "quant.h"

namespace lgmlh {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
  return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t seed, int64_t i, double mean, double sd) {
  const uint64_t g = 0x9e3779b97f4a7c15ULL;
  uint64_t a = seed + (uint64_t)(2 * i + 1) * g, b = seed + (uint64_t)(2 * i + 2) * g;
  double u1 = (double)(mix64(a) >> 11) * (1.0 / 9007199254740992.0);
  double u2 = (double)(mix64(b) >> 11) * (1.0 / 9007199254740992.0);
  return (float)(mean + sd * sqrt(-2.0 * log(u1 > 0 ? u1 : 1e-300)) *
                            cos(6.283185307179586 * u2));
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }
__device__ __forceinline__ void st16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)v;
  p[1] = (uint8_t)(v >> 8);
}

__device__ void quant_q4k(const float *x, uint8_t *b) {
  float scale[8], mins[8], ms = 0, mm = 0;
  for (int g = 0; g < 8; g++) {
    float lo = x[32 * g], hi = x[32 * g];
    for (int l = 1; l < 32; l++) {
      lo = fminf(lo, x[32 * g + l]);
      hi = fmaxf(hi, x[32 * g + l]);
    }
    if (lo > 0) lo = 0;
    scale[g] = (hi - lo) / 15.0f;
    mins[g] = -lo;
    ms = fmaxf(ms, scale[g]);
    mm = fmaxf(mm, mins[g]);
  }
  uint16_t hd = f2h(ms / 63.0f), hm = f2h(mm / 63.0f);
  float d = h2f(hd), dmin = h2f(hm);
  int sc[8], mn[8];
  for (int g = 0; g < 8; g++) {
    sc[g] = d > 0 ? clampi((int)rintf(scale[g] / d), 0, 63) : 0;
    mn[g] = dmin > 0 ? clampi((int)rintf(mins[g] / dmin), 0, 63) : 0;
  }
  for (int i = 0; i < Q4K_BYTES; i++) b[i] = 0;
  st16(b, hd);
  st16(b + 2, hm);
  uint8_t *s = b + 4, *qs = b + 16;
  for (int j = 0; j < 8; j++) {
    if (j < 4) {
      s[j] |= (uint8_t)sc[j];
      s[j + 4] |= (uint8_t)mn[j];
    } else {
      s[j + 4] = (uint8_t)((sc[j] & 0xF) | ((mn[j] & 0xF) << 4));
      s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
      s[j] |= (uint8_t)((mn[j] >> 4) << 6);
    }
  }
  for (int g = 0; g < 8; g++) {
    float d1 = d * (float)sc[g], m1 = dmin * (float)mn[g];
    for (int l = 0; l < 32; l++) {
      int q = d1 > 0 ? clampi((int)rintf((x[32 * g + l] + m1) / d1), 0, 15) : 0;
      qs[32 * (g / 2) + l] |= (uint8_t)(g & 1 ? q << 4 : q);
    }
  }
}

__device__ void quant_q6k(const float *x, uint8_t *b) {
  float gs[16], ms = 0;
  for (int g = 0; g < 16; g++) {
    float a = 0;
    for (int l = 0; l < 16; l++) a = fmaxf(a, fabsf(x[16 * g + l]));
    gs[g] = a / 31.0f;
    ms = fmaxf(ms, gs[g]);
  }
  uint16_t hd = f2h(ms / 127.0f);
  float d = h2f(hd);
  for (int i = 0; i < Q6K_BYTES; i++) b[i] = 0;
  int8_t *sc = (int8_t *)(b + 192);
  for (int g = 0; g < 16; g++) sc[g] = (int8_t)(d > 0 ? clampi((int)rintf(gs[g] / d), -128, 127) : 0);
  uint8_t *ql = b, *qh = b + 128;
  for (int v = 0; v < QK_K; v++) {
    float s = d * (float)sc[v / 16];
    int q = s > 0 ? clampi((int)rintf(x[v] / s), -32, 31) : 0;
    int u = q + 32;
    int h = v / 128, r = v % 128, t = r / 32, l = r % 32;
    ql[64 * h + l + 32 * (t & 1)] |= (uint8_t)(t < 2 ? (u & 0xF) : ((u & 0xF) << 4));
    qh[32 * h + l] |= (uint8_t)(((u >> 4) & 3) << (2 * t));
  }
  st16(b + 208, hd);
}

__device__ void quant_q8_0(const float *x, uint8_t *b) {
  float a = 0;
  for (int l = 0; l < 32; l++) a = fmaxf(a, fabsf(x[l]));
  float d = a / 127.0f;
  st16(b, f2h(d));
  float id = d > 0 ? 1.0f / d : 0.0f;
  for (int l = 0; l < 32; l++) ((int8_t *)(b + 2))[l] = (int8_t)clampi((int)rintf(x[l] * id), -127, 127);
}

// One thread per block of the output: a 256-value super-block (Q4_K,
// Q6_K), a 32-value block (Q8_0) or 32 values (f32).
__global__ void gen_kernel(uint64_t seed, int type, int64_t rows, int64_t cols, double mean,
                           double sd, uint8_t *__restrict__ out) {
  const int bv = (type == LGMLH_Q4_K || type == LGMLH_Q6_K) ? QK_K : 32;
  const int64_t per_row = cols / bv;
  int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= rows * per_row) return;
  int64_t r = t / per_row, blk = t % per_row;
  float x[QK_K];
  for (int i = 0; i < bv; i++) x[i] = normal_at(seed, r * cols + blk * bv + i, mean, sd);
  const int64_t rb = row_bytes(type, cols);
  uint8_t *row = out + r * rb;
  switch (type) {
    case LGMLH_Q4_K: quant_q4k(x, row + blk * Q4K_BYTES); break;
    case LGMLH_Q6_K: quant_q6k(x, row + blk * Q6K_BYTES); break;
    case LGMLH_Q8_0: quant_q8_0(x, row + blk * Q8_0_BYTES); break;
    default:
      for (int i = 0; i < 32; i++) ((float *)row)[blk * 32 + i] = x[i];
  }
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" int lgmlh_gen_normal(uint64_t seed, int type, int64_t rows, int64_t cols, double mean,
                                double sd, void *out, void *stream) {
  int64_t rb = row_bytes(type, cols);
  if (!out || rows < 0 || rb <= 0 || type == LGMLH_F16 || (type == LGMLH_F32 && cols % 32)) {
    set_error("gen_normal: bad arguments (type %d, cols %lld)", type, (long long)cols);
    return LGMLH_EINVAL;
  }
  const int bv = (type == LGMLH_Q4_K || type == LGMLH_Q6_K) ? QK_K : 32;
  int64_t n = rows * (cols / bv);
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(gen_kernel, dim3((unsigned)((n + 127) / 128)), dim3(128), 0,
                     as_stream(stream), seed, type, rows, cols, mean, sd, (uint8_t *)out);
  return hip_check(hipGetLastError(), "gen_normal");
}
