// Error state and the dense-layer ops around the hot path (gfx950).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "quant.h"

namespace lgmlh {

static thread_local char g_err[512] = "no error";

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

int hip_check(hipError_t e, const char *what) {
  if (e == hipSuccess) return LGMLH_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return LGMLH_EHIP;
}

// ---- get_rows (graph:get_rows, src/lgml.c:1913-1935) ----------------------
__global__ void get_rows_kernel(int type, const uint8_t *__restrict__ table, int64_t rb,
                                int64_t n_cols, const int32_t *__restrict__ ids,
                                float *__restrict__ out) {
  int64_t j = blockIdx.x;
  const uint8_t *row = table + (int64_t)ids[j] * rb;
  for (int64_t k = threadIdx.x; k < n_cols; k += blockDim.x)
    out[j * n_cols + k] = row_value(type, row, k);
}

__global__ void dequant_kernel(int type, const uint8_t *__restrict__ w, int64_t rb, int64_t K,
                               float *__restrict__ out) {
  int64_t m = blockIdx.x;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    out[m * K + k] = row_value(type, w + m * rb, k);
}

// ---- rms_norm * w ----------------------------------------------------------
// Sum of squares in f64 (as the CPU reference's ggml_float), mean rounded
// to f32, scale = 1 / sqrtf(mean + eps), y = (x * scale) * w.
template <typename OutT>
__global__ void rms_norm_kernel(const float *__restrict__ x, int64_t n, float eps,
                                const float *__restrict__ w, OutT *__restrict__ out) {
  __shared__ double part[256];
  int64_t r = blockIdx.x;
  const float *xr = x + r * n;
  double s = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += (double)xr[i] * (double)xr[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  float mean = (float)(part[0] / (double)n);
  float scale = 1.0f / sqrtf(mean + eps);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = xr[i] * scale;
    if (w) v = v * w[i];
    out[r * n + i] = (OutT)v;
  }
}

// ---- q/k norm, rope and KV store -------------------------------------------
// One workgroup per token. The row [q | k | v] is staged in LDS.
__device__ void head_rms_norm(float *v, int D, float eps, const float *w) {
  double s = 0;
  for (int i = 0; i < D; i++) s += (double)v[i] * (double)v[i];
  float mean = (float)(s / (double)D);
  float scale = 1.0f / sqrtf(mean + eps);
  for (int i = 0; i < D; i++) v[i] = (v[i] * scale) * w[i];
}

__global__ void qkv_rope_store_kernel(const float *__restrict__ qkv, int H, int Hkv, int D,
                                      int n_rot, int neox, float theta_scale,
                                      const float *__restrict__ ff,
                                      const float *__restrict__ q_norm,
                                      const float *__restrict__ k_norm, float eps,
                                      const int32_t *__restrict__ pos,
                                      uint16_t *__restrict__ kp, uint16_t *__restrict__ vp,
                                      const int64_t *__restrict__ cells,
                                      float *__restrict__ q_out) {
  extern __shared__ float row[];
  int64_t t = blockIdx.x;
  int W = (H + 2 * Hkv) * D;
  const float *src = qkv + t * W;
  for (int e = threadIdx.x; e < W; e += blockDim.x) row[e] = src[e];
  __syncthreads();
  if (q_norm || k_norm) {
    for (int h = threadIdx.x; h < H + Hkv; h += blockDim.x) {
      if (h < H && q_norm) head_rms_norm(row + h * D, D, eps, q_norm);
      if (h >= H && k_norm) head_rms_norm(row + h * D, D, eps, k_norm);
    }
    __syncthreads();
  }
  int p = pos[t];
  int half = n_rot / 2;
  for (int e = threadIdx.x; e < (H + Hkv) * half; e += blockDim.x) {
    int h = e / half, i = e % half;
    // theta_0 = pos, theta_{i+1} = theta_i * base^(-2/n_rot), in f32.
    float theta = (float)p;
    for (int j = 0; j < i; j++) theta *= theta_scale;
    float tt = theta / (ff ? ff[i] : 1.0f);
    double cs = (double)cosf(tt), sn = (double)sinf(tt);
    float *v = row + h * D;
    int a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
    double x0 = v[a], x1 = v[b];
    v[a] = (float)(x0 * cs - x1 * sn);
    v[b] = (float)(x0 * sn + x1 * cs);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < H * D; e += blockDim.x) q_out[t * H * D + e] = row[e];
  int64_t cell = cells[t];
  int64_t b = cell / KV_BLOCK, o = cell % KV_BLOCK;
  for (int e = threadIdx.x; e < Hkv * D; e += blockDim.x) {
    int h = e / D, d = e % D;
    kp[((b * Hkv + h) * KV_BLOCK + o) * D + d] = f2h(row[H * D + e]);
    vp[((b * Hkv + h) * (int64_t)D + d) * KV_BLOCK + o] = f2h(row[(H + Hkv) * D + e]);
  }
}

// ---- swiglu: silu(g) * u, in f64 --------------------------------------------
template <typename OutT>
__global__ void swiglu_kernel(const float *__restrict__ gu, int64_t n, int64_t F,
                              OutT *__restrict__ out) {
  int64_t total = n * F;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e / F, c = e % F;
    double g = gu[r * 2 * F + c], u = gu[r * 2 * F + F + c];
    out[e] = (OutT)(float)(g / (1.0 + exp(-g)) * u);
  }
}

// ---- argmax: first index of the maximum --------------------------------------
__global__ void argmax_kernel(const float *__restrict__ x, int64_t n, int32_t *__restrict__ out) {
  __shared__ float bv[256];
  __shared__ int64_t bi[256];
  int64_t r = blockIdx.x;
  const float *xr = x + r * n;
  float best = -INFINITY;
  int64_t idx = -1;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = xr[i];
    if (idx < 0 || v > best) {
      best = v;
      idx = i;
    }
  }
  bv[threadIdx.x] = best;
  bi[threadIdx.x] = idx;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      float v2 = bv[threadIdx.x + o];
      int64_t i2 = bi[threadIdx.x + o];
      if (i2 >= 0 && (bi[threadIdx.x] < 0 || v2 > bv[threadIdx.x] ||
                      (v2 == bv[threadIdx.x] && i2 < bi[threadIdx.x]))) {
        bv[threadIdx.x] = v2;
        bi[threadIdx.x] = i2;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[r] = (int32_t)bi[0];
}

int get_rows_dev(int type, const void *table, int64_t n_cols, const int32_t *ids, int64_t n,
                 float *out, hipStream_t st) {
  int64_t rb = row_bytes(type, n_cols);
  if (rb <= 0) {
    set_error("get_rows: bad type %d for %lld columns", type, (long long)n_cols);
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(get_rows_kernel, dim3((unsigned)n), dim3(256), 0, st, type,
                     (const uint8_t *)table, rb, n_cols, ids, out);
  return hip_check(hipGetLastError(), "get_rows");
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" const char *lgmlh_last_error(void) { return g_err; }
extern "C" int lgmlh_abi_version(void) { return LGMLH_ABI_VERSION; }
extern "C" int64_t lgmlh_row_size(int type, int64_t n) { return row_bytes(type, n); }

extern "C" int lgmlh_get_rows(int type, const void *table, int64_t n_rows, int64_t n_cols,
                              const int32_t *ids, const int32_t *h_ids, int64_t n, float *out,
                              void *stream) {
  int64_t rb = row_bytes(type, n_cols);
  if (!table || !ids || !out || rb <= 0 || n < 0) {
    set_error("get_rows: bad arguments");
    return LGMLH_EINVAL;
  }
  if (!h_ids) {
    set_error("get_rows: the host copy of the ids is required for the range check");
    return LGMLH_EINVAL;
  }
  for (int64_t j = 0; j < n; j++)
    if (h_ids[j] < 0 || h_ids[j] >= n_rows) {
      set_error("get_rows: id %d out of range [0, %lld)", h_ids[j], (long long)n_rows);
      return LGMLH_ERANGE;
    }
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(get_rows_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream), type,
                     (const uint8_t *)table, rb, n_cols, ids, out);
  return hip_check(hipGetLastError(), "get_rows");
}

extern "C" int lgmlh_dequantize(int type, const void *src, int64_t M, int64_t K, float *out,
                                void *stream) {
  int64_t rb = row_bytes(type, K);
  if (!src || !out || rb <= 0 || M < 0) {
    set_error("dequantize: bad arguments");
    return LGMLH_EINVAL;
  }
  if (M == 0) return LGMLH_OK;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)M), dim3(256), 0, as_stream(stream), type,
                     (const uint8_t *)src, rb, K, out);
  return hip_check(hipGetLastError(), "dequantize");
}

extern "C" int lgmlh_rms_norm(const float *x, int64_t n_rows, int64_t n, float eps,
                              const float *w, void *out, int out_type, void *stream) {
  if (!x || !out || n <= 0 || n_rows < 0 || (out_type != LGMLH_F32 && out_type != LGMLH_F16)) {
    set_error("rms_norm: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n_rows == 0) return LGMLH_OK;
  if (out_type == LGMLH_F32)
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)n_rows), dim3(256), 0,
                       as_stream(stream), x, n, eps, w, (float *)out);
  else
    hipLaunchKernelGGL(rms_norm_kernel<f16>, dim3((unsigned)n_rows), dim3(256), 0,
                       as_stream(stream), x, n, eps, w, (f16 *)out);
  return hip_check(hipGetLastError(), "rms_norm");
}

extern "C" int lgmlh_qkv_rope_store(float *qkv, int64_t n, int n_head, int n_head_kv,
                                    int head_dim, int n_rot, int neox, float freq_base,
                                    const float *freq_factors, const float *q_norm,
                                    const float *k_norm, float eps, const int32_t *pos,
                                    void *kpool, void *vpool, int64_t n_cells,
                                    const int64_t *cells, float *q_out, void *stream) {
  if (!qkv || !pos || !kpool || !vpool || !cells || !q_out || n < 0 || n_head <= 0 ||
      n_head_kv <= 0 || head_dim <= 0 || n_rot <= 0 || n_rot > head_dim || n_rot % 2 ||
      n_cells % KV_BLOCK) {
    set_error("qkv_rope_store: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  // base^(-2/n_rot) rounded to f32 on the host, as the CPU reference does.
  float theta_scale = powf(freq_base, -2.0f / (float)n_rot);
  size_t lds = (size_t)(n_head + 2 * n_head_kv) * head_dim * sizeof(float);
  if (lds > 160 * 1024) {
    set_error("qkv_rope_store: row too wide");
    return LGMLH_EINVAL;
  }
  hipLaunchKernelGGL(qkv_rope_store_kernel, dim3((unsigned)n), dim3(256), lds,
                     as_stream(stream), qkv, n_head, n_head_kv, head_dim, n_rot, neox,
                     theta_scale, freq_factors, q_norm, k_norm, eps, pos, (uint16_t *)kpool,
                     (uint16_t *)vpool, cells, q_out);
  return hip_check(hipGetLastError(), "qkv_rope_store");
}

extern "C" int lgmlh_swiglu(const float *gu, int64_t n, int64_t F, void *out, int out_type,
                            void *stream) {
  if (!gu || !out || n < 0 || F <= 0 || (out_type != LGMLH_F32 && out_type != LGMLH_F16)) {
    set_error("swiglu: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  int64_t total = n * F;
  unsigned blocks = (unsigned)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  if (out_type == LGMLH_F32)
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3(blocks), dim3(256), 0, as_stream(stream), gu,
                       n, F, (float *)out);
  else
    hipLaunchKernelGGL(swiglu_kernel<f16>, dim3(blocks), dim3(256), 0, as_stream(stream), gu, n,
                       F, (f16 *)out);
  return hip_check(hipGetLastError(), "swiglu");
}

extern "C" int lgmlh_argmax(const float *x, int64_t n_rows, int64_t n_cols, int32_t *out,
                            void *stream) {
  if (!x || !out || n_rows < 0 || n_cols <= 0) {
    set_error("argmax: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n_rows == 0) return LGMLH_OK;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)n_rows), dim3(256), 0, as_stream(stream), x,
                     n_cols, out);
  return hip_check(hipGetLastError(), "argmax");
}
