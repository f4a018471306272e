// Error state and the dense-layer ops around the hot path (gfx950).
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "quant.h"
#include "split.h"

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
// With scale != 0 the rows are multiplied by it (the gemma embedding scale,
// transformer.lua:2304-2306).
__global__ void get_rows_kernel(int type, const uint8_t *__restrict__ table, int64_t rb,
                                int64_t n_cols, const int32_t *__restrict__ ids,
                                float *__restrict__ out, float scale) {
  int64_t j = blockIdx.x;
  const uint8_t *row = table + (int64_t)ids[j] * rb;
  for (int64_t k = threadIdx.x; k < n_cols; k += blockDim.x) {
    const float v = row_value(type, row, k);
    out[j * n_cols + k] = scale != 0.0f ? v * scale : v;
  }
}

__global__ void dequant_kernel(int type, const uint8_t *__restrict__ w, int64_t rb, int64_t K,
                               float *__restrict__ out) {
  int64_t m = blockIdx.x;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    out[m * K + k] = row_value(type, w + m * rb, k);
}

// One workgroup per row, one 8-value piece per thread (rows of up to 8192
// values): the many loads of a row's pending split sums go out at once.
constexpr int RMS_THREADS = 1024, RMS_PIECES = 1;
// Past 512 rows (one round of two workgroups per CU) a launch takes n / 8
// threads rounded up to whole waves instead, so that all rows run at once:
// the waves a row leaves without a piece would add only zeros to its sum,
// so the sums are the same. (C2's prefill rows: 22.8 -> 19.3 us per launch;
// at 64 rows the 1024-thread shape is faster, 6.2 against 6.9 us.)
static unsigned rms_threads(int64_t n, int64_t n_rows) {
  return n_rows > 512 ? (unsigned)((n / 8 + 63) / 64 * 64) : (unsigned)RMS_THREADS;
}

// ---- rms_norm * w ----------------------------------------------------------
// Sum of squares in f64 (as the CPU reference's ggml_float), mean rounded
// to f32, scale = 1 / sqrtf(mean + eps), y = (x * scale) * w. Row
// blockIdx.x of the output is input row rows[blockIdx.x] (all rows when
// rows is null); the result goes to out (f32 / f16) and / or to split
// planes for a quantized product (n % 256 == 0).
template <typename OutT>
__global__ void rms_norm_kernel(float *__restrict__ x, const int32_t *__restrict__ rows,
                                int64_t n, float eps, const float *__restrict__ w,
                                OutT *__restrict__ out, f16 *__restrict__ planes, int64_t npad,
                                Pending pend, bool writeback, int xf) {
  __shared__ double part[2][RMS_THREADS / 64];
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int64_t rr = rows ? (int64_t)rows[r] : r;
  float *xr = x + rr * n;
  // sum of squares over the row (f64, fixed order) into slot k
  auto row_sumsq = [&](double s, int k) -> double {
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((tid & 63) == 0) part[k][tid >> 6] = s;
    __syncthreads();
    double tot = 0;
    const int nw = (int)(blockDim.x >> 6);
#pragma unroll
    for (int i = 0; i < RMS_THREADS / 64; i++)
      if (i < nw) tot += part[k][i];
    return tot;
  };
  // The row stays in registers: thread tid holds pieces tid + RMS_THREADS j
  // of 8 values (n % 8 == 0 and n <= 8 * RMS_THREADS * RMS_PIECES).
  // The weight's pieces are loaded with the row's, not after the sum.
  f32x4 v[RMS_PIECES][2], t[RMS_PIECES][2], wv[RMS_PIECES][2], pw[RMS_PIECES][2];
  double st = 0;
#pragma unroll
  for (int j = 0; j < RMS_PIECES; j++) {
    const int64_t pc = tid + (int64_t)RMS_THREADS * j;
    if (pc < n / 8) {
      const f32x4 *src = (const f32x4 *)(xr + 8 * pc);
      v[j][0] = src[0];
      v[j][1] = src[1];
      if (w) {
#pragma unroll
        for (int e = 0; e < 8; e++) wv[j][e >> 2][e & 3] = w[8 * pc + e];
      }
      if (pend.splits && pend.post) {
#pragma unroll
        for (int e = 0; e < 8; e++) pw[j][e >> 2][e & 3] = pend.post[8 * pc + e];
      }
      if (pend.splits) {
        // the pending product: its split sums in order
        float ps[8];
        pend.sum8(rr, 8 * pc, ps);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          if (pend.post) {
            t[j][e >> 2][e & 3] = ps[e];
            st += (double)ps[e] * (double)ps[e];
          } else {
            v[j][e >> 2][e & 3] = ps[e] + v[j][e >> 2][e & 3];  // then the residual
          }
        }
      }
    }
  }
  if (pend.splits && pend.post) {
    // x += rms_norm(product) * post (the gemma post norm, then the residual)
    const float mean_t = (float)(row_sumsq(st, 1) / (double)n);
    const float sc_t = 1.0f / sqrtf(mean_t + eps);
#pragma unroll
    for (int j = 0; j < RMS_PIECES; j++) {
      const int64_t pc = tid + (int64_t)RMS_THREADS * j;
      if (pc < n / 8)
#pragma unroll
        for (int e = 0; e < 8; e++)
          v[j][e >> 2][e & 3] = t[j][e >> 2][e & 3] * sc_t * pw[j][e >> 2][e & 3] + v[j][e >> 2][e & 3];
    }
  }
  double s = 0;
#pragma unroll
  for (int j = 0; j < RMS_PIECES; j++) {
    const int64_t pc = tid + (int64_t)RMS_THREADS * j;
    if (pc < n / 8) {
      if (pend.splits && pend.scale != 0.0f) {
        v[j][0] *= pend.scale;  // the layer output scale
        v[j][1] *= pend.scale;
      }
      if (pend.splits && writeback) {
        f32x4 *dst = (f32x4 *)(xr + 8 * pc);
        dst[0] = v[j][0];
        dst[1] = v[j][1];
      }
#pragma unroll
      for (int e = 0; e < 4; e++)
        s += (double)v[j][0][e] * (double)v[j][0][e] + (double)v[j][1][e] * (double)v[j][1][e];
    }
  }
  const double tot = row_sumsq(s, 0);
  const float mean = (float)(tot / (double)n);
  const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
  for (int j = 0; j < RMS_PIECES; j++) {
    const int64_t pc = tid + (int64_t)RMS_THREADS * j;
    if (pc < n / 8) {  // n / 8 is a multiple of 4 when planes are written
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        y[e] = v[j][e >> 2][e & 3] * scale;
        if (w) y[e] = y[e] * wv[j][e >> 2][e & 3];
      }
      if (out)
#pragma unroll
        for (int e = 0; e < 8; e++) out[r * n + 8 * pc + e] = (OutT)y[e];
      if (planes) act_store8(xf, planes, npad, n, r, 8 * pc, y);
    }
  }
}

// ---- q/k norm, rope and KV store -------------------------------------------
constexpr int QKV_V_FROM_K = 1, QKV_V_NORM = 2;
// rms_norm of one head by one wave: f64 sum of squares, mean rounded to
// f32, scale = 1 / sqrtf(mean + eps), v = (v * scale) * w.
__device__ void head_rms_norm(float *v, int D, float eps, const float *w) {
  const int lane = threadIdx.x & 63;
  double s = 0;
  for (int i = lane; i < D; i += 64) s += (double)v[i] * (double)v[i];
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const float mean = (float)(s / (double)D);
  const float scale = 1.0f / sqrtf(mean + eps);
  for (int i = lane; i < D; i += 64) v[i] = w ? (v[i] * scale) * w[i] : v[i] * scale;
}

// The rotation of pair i at position p: theta_0 = p, theta_{i+1} = theta_i
// * base^(-2/n_rot) (a running f32 product, as the CPU reference's rope
// cache), divided by the frequency factor; its cos and sin.
__device__ __forceinline__ void rope_angle(int p, int i, float theta_scale,
                                           const float *__restrict__ ff, float &c, float &s) {
  float theta = (float)p;
  for (int j = 0; j < i; j++) theta *= theta_scale;
  const float tt = theta / (ff ? ff[i] : 1.0f);
  c = cosf(tt);
  s = sinf(tt);
}

// The angle table of a pass for one rope setting: row t (n_rot floats) holds
// the cos of pairs 0 .. n_rot / 2 - 1 at position pos[t], then their sin.
// Every layer with that setting reads it instead of making its own.
__global__ void rope_table_kernel(const int32_t *__restrict__ pos, int n_rot, float theta_scale,
                                  const float *__restrict__ ff, float *__restrict__ table) {
  const int64_t t = blockIdx.x;
  const int half = n_rot / 2, p = pos[t];
  for (int i = threadIdx.x; i < half; i += blockDim.x)
    rope_angle(p, i, theta_scale, ff, table[t * n_rot + i], table[t * n_rot + half + i]);
}

// One workgroup per (token, 8 heads) and one wave per head of [q | k | v]:
// the head's values (with the pending split sums) go to LDS, then its norm
// (q_norm / k_norm; on gemma the V norm without a weight, :1782-1784),
// rope for q and k heads, and the store: q to q_out, k and v to their pool
// cell. With QKV_V_FROM_K a V head is the raw K head (transformer.lua:1779).
constexpr int QKV_HEADS = 8;
__global__ void __launch_bounds__(64 * QKV_HEADS)
qkv_rope_store_kernel(const float *__restrict__ qkv, int H, int Hkv, int D, int n_rot, int neox,
                      float theta_scale, const float *__restrict__ ff,
                      const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                      float eps, const int32_t *__restrict__ pos, uint16_t *__restrict__ kp,
                      uint16_t *__restrict__ vp, const int64_t *__restrict__ cells,
                      int64_t n_cells, float *__restrict__ q_out, Pending pa, Pending pb,
                      int vmode, const float *__restrict__ table) {
  extern __shared__ float lds[];
  const int64_t t = blockIdx.x;
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int NH = H + 2 * Hkv, W = NH * D;
  const int h = blockIdx.y * QKV_HEADS + wv;  // this wave's head
  const int half = n_rot / 2;
  float *cs_ = lds, *sn_ = lds + half, *v = lds + n_rot + wv * D;
  const bool has = h < NH;  // wave-uniform
  const bool is_q = h < H, is_k = !is_q && h < H + Hkv, is_v = h >= H + Hkv;
  // One angle per rotated pair i, shared by every head (rope_angle), from
  // the pass's table when one is given.
  // Columns of the head: [0, pa.cols) may come from pending partials pa,
  // the rest from pb; pieces of 4 (W, pa.cols, pb.cols multiples of 8).
  // A lane's first piece is loaded before the angles are made, so that the
  // loads are in flight meanwhile.
  const int sh = is_v && (vmode & QKV_V_FROM_K) ? h - Hkv : h;
  const float *src = qkv + t * W;
  auto piece = [&](int pc, float (&x)[4]) {
    const int e = sh * D + 4 * pc;
    if (pa.splits && e < pa.cols)
      pa.sum4(t, e, x);
    else if (pb.splits && e >= W - pb.cols)
      pb.sum4(t, e - (W - pb.cols), x);
    else
#pragma unroll
      for (int i = 0; i < 4; i++) x[i] = src[e + i];
  };
  float x0[4];
  const bool first = has && lane < D / 4;
  if (first) piece(lane, x0);
  if (table) {  // the pass's angle table (rope_table_kernel): cos, then sin
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      cs_[i] = table[t * n_rot + i];
      sn_[i] = table[t * n_rot + half + i];
    }
  } else {
    const int p = pos[t];
    for (int i = threadIdx.x; i < half; i += blockDim.x) rope_angle(p, i, theta_scale, ff, cs_[i], sn_[i]);
  }
  if (first)
#pragma unroll
    for (int i = 0; i < 4; i++) v[4 * lane + i] = x0[i];
  if (has)
    for (int pc = lane + 64; pc < D / 4; pc += 64) {  // heads of more than 256
      float x[4];
      piece(pc, x);
#pragma unroll
      for (int i = 0; i < 4; i++) v[4 * pc + i] = x[i];
    }
  __syncthreads();  // the angles and each wave's head
  if (!has) return;
  if (is_q ? q_norm != nullptr : is_k ? k_norm != nullptr : (vmode & QKV_V_NORM) != 0) {
    head_rms_norm(v, D, eps, is_q ? q_norm : is_k ? k_norm : nullptr);
    __builtin_amdgcn_wave_barrier();
  }
  if (!is_v) {
    for (int i = lane; i < half; i += 64) {
      const double cs = (double)cs_[i], sn = (double)sn_[i];
      const int a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
      const double x0 = v[a], x1 = v[b];
      v[a] = (float)(x0 * cs - x1 * sn);
      v[b] = (float)(x0 * sn + x1 * cs);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (is_q) {
    for (int d = lane; d < D; d += 64) q_out[(t * H + h) * D + d] = v[d];
    return;
  }
  const int64_t cell = cells[t];
  if (cell < 0 || cell >= n_cells) return;  // a cell outside the pool is never written
  const int64_t b = cell / KV_BLOCK, o = cell % KV_BLOCK;
  if (is_k) {
    const int hk = h - H;
    for (int d = lane; d < D; d += 64) kp[((b * Hkv + hk) * KV_BLOCK + o) * D + d] = f2h(v[d]);
  } else {
    const int hv = h - H - Hkv;
    for (int d = lane; d < D; d += 64)
      vp[((b * Hkv + hv) * (int64_t)D + d) * KV_BLOCK + o] = f2h(v[d]);
  }
}

// ---- gated units: silu(g) * u (swiglu) or gelu(g) * u (geglu), in f64 ------
// gelu is ggml's tanh form, 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))
// (geglu_split, src/ops_nn.c:165-172).
__device__ __forceinline__ double glu_act(double g, int gelu) {
  return gelu ? 0.5 * g * (1.0 + tanh(0.7978845608028654 * (g + 0.044715 * g * g * g)))
              : g / (1.0 + exp(-g));
}

template <typename OutT>
__global__ void swiglu_kernel(const float *__restrict__ gu, int64_t n, int64_t F,
                              OutT *__restrict__ out, Pending pend, int gelu) {
  int64_t total = n * F;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = e / F, c = e % F;
    double g = pend.splits ? pend.sum(r, c) : gu[r * 2 * F + c];
    double u = pend.splits ? pend.sum(r, F + c) : gu[r * 2 * F + F + c];
    float v = (float)(glu_act(g, gelu) * u);
    // An f16 output is f16 of this f32 value. Left free, the compiler folds
    // the two conversions into one f64 -> f16 rounding, which differs at
    // f16 ties (rounding an arbitrary f64 value twice is not innocuous).
    asm volatile("" : "+v"(v));
    out[e] = (OutT)v;
  }
}

// The same values into split planes (F % 256 == 0); one thread per 8.
__global__ void swiglu_split_kernel(const float *__restrict__ gu, int64_t n, int64_t F,
                                    f16 *__restrict__ planes, int64_t npad, Pending pend,
                                    int gelu, int xf) {
  const int64_t per_row = F / 8;
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= n * per_row) return;  // whole 4-lane groups leave together
  const int64_t r = t / per_row, c0 = (t % per_row) * 8;
  float g8[8], u8[8], v[8];
  if (pend.splits) {
    pend.sum8(r, c0, g8);
    pend.sum8(r, F + c0, u8);
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      g8[e] = gu[r * 2 * F + c0 + e];
      u8[e] = gu[r * 2 * F + F + c0 + e];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = (float)(glu_act(g8[e], gelu) * (double)u8[e]);
  act_store8(xf, planes, npad, F, r, c0, v);
}

// ---- logit softcap: cap * tanh(x * (1 / cap)) (transformer.lua:2097-2099) ----
__global__ void softcap_kernel(float *__restrict__ x, int64_t n, float cap) {
  const float inv = 1.0f / cap;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    x[i] = tanhf(x[i] * inv) * cap;
}

// ---- argmax: first index of the maximum --------------------------------------
// src/sample.c:914-925: m = x[0], then x[i] replaces it only when x[i] > m.
// So a NaN at index 0 gives 0 (nothing compares greater than it), a NaN
// elsewhere is never taken, and ties keep the first index. Here: each
// thread scans its strided slice for the first maximum of its non-NaN
// values (float4 loads when rows are 16-byte aligned), the candidates meet
// in a fixed-order tree that keeps the smaller index on ties, and a NaN at
// index 0 decides the row alone.
constexpr int ARGMAX_THREADS = 1024;
__device__ __forceinline__ void amax_take(float &bv, int64_t &bi, float v, int64_t i) {
  if (i >= 0 && (bi < 0 || v > bv || (v == bv && i < bi))) {
    bv = v;
    bi = i;
  }
}
__global__ void __launch_bounds__(ARGMAX_THREADS)
argmax_kernel(const float *__restrict__ x, int64_t n, int32_t *__restrict__ out) {
  __shared__ float sv[ARGMAX_THREADS / 64];
  __shared__ int64_t si[ARGMAX_THREADS / 64];
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const float *xr = x + r * n;
  float best = 0.0f;
  int64_t idx = -1;  // no candidate yet (NaN values never become one)
  if ((n & 3) == 0 && (((uintptr_t)x) & 15) == 0) {
    for (int64_t q = tid; q < n / 4; q += ARGMAX_THREADS) {
      const f32x4 v = ((const f32x4 *)xr)[q];
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (v[e] == v[e] && (idx < 0 || v[e] > best)) {
          best = v[e];
          idx = 4 * q + e;
        }
    }
  } else {
    for (int64_t i = tid; i < n; i += ARGMAX_THREADS) {
      const float v = xr[i];
      if (v == v && (idx < 0 || v > best)) {
        best = v;
        idx = i;
      }
    }
  }
  for (int o = 1; o < 64; o <<= 1) {
    const float v2 = __shfl_xor(best, o);
    const int64_t i2 = __shfl_xor(idx, o);
    amax_take(best, idx, v2, i2);
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = best;
    si[tid >> 6] = idx;
  }
  __syncthreads();
  if (tid == 0) {
    float b = sv[0];
    int64_t bi = si[0];
    for (int k = 1; k < ARGMAX_THREADS / 64; k++) amax_take(b, bi, sv[k], si[k]);
    const float x0 = n > 0 ? xr[0] : 0.0f;
    out[r] = x0 != x0 || bi < 0 ? 0 : (int32_t)bi;
  }
}

int get_rows_dev(int type, const void *table, int64_t n_cols, const int32_t *ids, int64_t n,
                 float *out, hipStream_t st, float scale) {
  int64_t rb = row_bytes(type, n_cols);
  if (rb <= 0) {
    set_error("get_rows: bad type %d for %lld columns", type, (long long)n_cols);
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(get_rows_kernel, dim3((unsigned)n), dim3(256), 0, st, type,
                     (const uint8_t *)table, rb, n_cols, ids, out, scale);
  return hip_check(hipGetLastError(), "get_rows");
}


// rms_norm of n_rows rows (input rows[j] when rows is given) into f32 out
// and / or X planes of the form xf (planes sized for n_rows rows).
// pend: a pending product added to x first (written back to x when
// writeback; never with rows, which may repeat).
int rms_norm_dev(float *x, const int32_t *rows, int64_t n_rows, int64_t n, float eps,
                 const float *w, float *out, f16 *planes, hipStream_t st, Pending pend,
                 bool writeback, int xf) {
  if (n_rows == 0) return LGMLH_OK;
  if ((planes && n % 256) || n % 8 || n > 8 * RMS_THREADS * RMS_PIECES) {
    set_error("rms_norm: bad row length %lld", (long long)n);
    return LGMLH_EINVAL;
  }
  hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)n_rows), dim3(rms_threads(n, n_rows)), 0, st, x, rows,
                     n, eps, w, out, planes, split_npad(n_rows), pend, writeback && !rows, xf);
  return hip_check(hipGetLastError(), "rms_norm");
}

// silu(g) * u (gelu(g) * u with gelu set) into f32 out and / or X planes of
// the form xf.
int swiglu_dev(const float *gu, int64_t n, int64_t F, float *out, f16 *planes, hipStream_t st,
               Pending pend, int gelu, int xf) {
  if (n == 0) return LGMLH_OK;
  if (out) {
    int64_t total = n * F;
    unsigned blocks = (unsigned)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3(blocks), dim3(256), 0, st, gu, n, F, out, pend,
                       gelu);
  }
  if (planes) {
    if (F % 256) {
      set_error("swiglu: split output needs F %% 256 == 0 (F = %lld)", (long long)F);
      return LGMLH_EINVAL;
    }
    int64_t total = n * (F / 8);
    hipLaunchKernelGGL(swiglu_split_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       st, gu, n, F, planes, split_npad(n), pend, gelu, xf);
  }
  return hip_check(hipGetLastError(), "swiglu");
}

int softcap_dev(float *x, int64_t n, float cap, hipStream_t st) {
  if (n == 0 || cap <= 0.0f) return LGMLH_OK;
  unsigned blocks = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(softcap_kernel, dim3(blocks), dim3(256), 0, st, x, n, cap);
  return hip_check(hipGetLastError(), "softcap");
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
                     (const uint8_t *)table, rb, n_cols, ids, out, 0.0f);
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
  if (!x || !out || n <= 0 || n_rows < 0 || n % 8 || n > 8 * RMS_THREADS * RMS_PIECES ||
      (out_type != LGMLH_F32 && out_type != LGMLH_F16)) {
    set_error("rms_norm: bad arguments (n must be a multiple of 8, at most %d)",
              8 * RMS_THREADS * RMS_PIECES);
    return LGMLH_EINVAL;
  }
  if (n_rows == 0) return LGMLH_OK;
  if (out_type == LGMLH_F32)
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)n_rows), dim3(rms_threads(n, n_rows)), 0,
                       as_stream(stream), (float *)x, nullptr, n, eps, w, (float *)out, nullptr, 0,
                       Pending{}, false, (int)XF_SPLIT);
  else
    hipLaunchKernelGGL(rms_norm_kernel<f16>, dim3((unsigned)n_rows), dim3(rms_threads(n, n_rows)), 0,
                       as_stream(stream), (float *)x, nullptr, n, eps, w, (f16 *)out, nullptr, 0,
                       Pending{}, false, (int)XF_SPLIT);
  return hip_check(hipGetLastError(), "rms_norm");
}

namespace lgmlh {
// base^(-2/n_rot) rounded to f32 on the host, as the CPU reference does.
static float rope_theta_scale(float freq_base, int n_rot) {
  return powf(freq_base, -2.0f / (float)n_rot);
}

int qkv_rope_store_dev(float *qkv, int64_t n, int n_head, int n_head_kv,
                                    int head_dim, int n_rot, int neox, float freq_base,
                                    const float *freq_factors, const float *q_norm,
                                    const float *k_norm, float eps, const int32_t *pos,
                                    void *kpool, void *vpool, int64_t n_cells,
                                    const int64_t *cells, float *q_out, void *stream, Pending pa,
                       Pending pb, int vmode, const float *table) {
  if (!qkv || !pos || !kpool || !vpool || !cells || !q_out || n < 0 || n_head <= 0 ||
      n_head_kv <= 0 || head_dim <= 0 || head_dim % 8 || head_dim > 1024 || n_rot <= 0 ||
      n_rot > head_dim ||
      n_rot % 2 || n_cells % KV_BLOCK || pa.cols % 8 || pb.cols % 8) {
    set_error("qkv_rope_store: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  const float theta_scale = rope_theta_scale(freq_base, n_rot);
  const size_t lds = ((size_t)QKV_HEADS * head_dim + n_rot) * sizeof(float);
  const int groups = (n_head + 2 * n_head_kv + QKV_HEADS - 1) / QKV_HEADS;
  hipLaunchKernelGGL(qkv_rope_store_kernel, dim3((unsigned)n, (unsigned)groups),
                     dim3(64 * QKV_HEADS), lds,
                     as_stream(stream), qkv, n_head, n_head_kv, head_dim, n_rot, neox,
                     theta_scale, freq_factors, q_norm, k_norm, eps, pos, (uint16_t *)kpool,
                     (uint16_t *)vpool, cells, n_cells, q_out, pa, pb, vmode, table);
  return hip_check(hipGetLastError(), "qkv_rope_store");
}

int rope_table_dev(const int32_t *pos, int64_t n, int n_rot, float freq_base,
                   const float *freq_factors, float *table, hipStream_t st) {
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)n), dim3(64), 0, st, pos, n_rot,
                     rope_theta_scale(freq_base, n_rot), freq_factors, table);
  return hip_check(hipGetLastError(), "rope_table");
}
}  // namespace lgmlh

extern "C" int lgmlh_qkv_rope_store(float *qkv, int64_t n, int n_head, int n_head_kv,
                                    int head_dim, int n_rot, int neox, float freq_base,
                                    const float *freq_factors, const float *q_norm,
                                    const float *k_norm, float eps, const int32_t *pos,
                                    void *kpool, void *vpool, int64_t n_cells,
                                    const int64_t *cells, float *q_out, void *stream) {
  return qkv_rope_store_dev(qkv, n, n_head, n_head_kv, head_dim, n_rot, neox, freq_base,
                            freq_factors, q_norm, k_norm, eps, pos, kpool, vpool, n_cells, cells,
                            q_out, stream, Pending{}, Pending{}, 0, nullptr);
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
                       n, F, (float *)out, Pending{}, 0);
  else
    hipLaunchKernelGGL(swiglu_kernel<f16>, dim3(blocks), dim3(256), 0, as_stream(stream), gu, n,
                       F, (f16 *)out, Pending{}, 0);
  return hip_check(hipGetLastError(), "swiglu");
}

extern "C" int lgmlh_geglu(const float *gu, int64_t n, int64_t F, void *out, int out_type,
                           void *stream) {
  if (!gu || !out || n < 0 || F <= 0 || (out_type != LGMLH_F32 && out_type != LGMLH_F16)) {
    set_error("geglu: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  int64_t total = n * F;
  unsigned blocks = (unsigned)((total + 255) / 256 < 8192 ? (total + 255) / 256 : 8192);
  if (out_type == LGMLH_F32)
    hipLaunchKernelGGL(swiglu_kernel<float>, dim3(blocks), dim3(256), 0, as_stream(stream), gu,
                       n, F, (float *)out, Pending{}, 1);
  else
    hipLaunchKernelGGL(swiglu_kernel<f16>, dim3(blocks), dim3(256), 0, as_stream(stream), gu, n,
                       F, (f16 *)out, Pending{}, 1);
  return hip_check(hipGetLastError(), "geglu");
}

extern "C" int lgmlh_softcap(float *x, int64_t n, float cap, void *stream) {
  if (!x || n < 0 || !(cap > 0.0f)) {
    set_error("softcap: bad arguments");
    return LGMLH_EINVAL;
  }
  return softcap_dev(x, n, cap, as_stream(stream));
}

extern "C" int lgmlh_argmax(const float *x, int64_t n_rows, int64_t n_cols, int32_t *out,
                            void *stream) {
  if (!x || !out || n_rows < 0 || n_cols <= 0) {
    set_error("argmax: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n_rows == 0) return LGMLH_OK;
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)n_rows), dim3(ARGMAX_THREADS), 0, as_stream(stream), x,
                     n_cols, out);
  return hip_check(hipGetLastError(), "argmax");
}
