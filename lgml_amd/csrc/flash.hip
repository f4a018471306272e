// Attention over strided K / V views with an explicit additive mask: the
// semantics of graph:flash_attn (src/lgml.c:2121-2170), i.e.
// ggml_flash_attn_ext's softmax(scale q k^T [softcap] + slope * mask) v.
// It serves callers whose K / V are plain (n_kv, Hkv * D) rows rather than
// this library's block pool (the paged path is attn.hip).
//
// One wave64 per (query row, head). Per tile of 64 columns each lane
// scores one column (q from LDS against its own K row, 16-byte loads), the
// wave takes the tile max and sum with shuffles (online softmax in f32),
// and each lane accumulates D / 64 output values from coalesced V rows.
#include <math.h>

#include "common.h"

namespace lgmlh {

constexpr int FA_MAX_D = 256;

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ALiBi slope of head h (1 without max_bias): with n the largest power of
// two <= H, heads below n take (2^(-max_bias / n))^(h + 1), the others
// (2^(-max_bias / 2 / n))^(2 (h - n) + 1).
__device__ __forceinline__ float alibi(int h, int H, float max_bias) {
  if (max_bias <= 0.0f) return 1.0f;
  int n = 1;
  while (n * 2 <= H) n *= 2;
  const float m0 = powf(2.0f, -max_bias / (float)n);
  const float m1 = powf(2.0f, -(max_bias / 2.0f) / (float)n);
  return h < n ? powf(m0, (float)(h + 1)) : powf(m1, (float)(2 * (h - n) + 1));
}

__global__ void __launch_bounds__(64)
flash_attn_kernel(const float *__restrict__ q, int H, int T, int D,
                  const uint16_t *__restrict__ k, const uint16_t *__restrict__ v, int G, int n_kv,
                  int64_t k_rs, int64_t k_hs, int64_t v_rs, int64_t v_hs,
                  const uint16_t *__restrict__ mask, int mask_heads, int mask_rows, float scale,
                  float max_bias, float softcap, float *__restrict__ out) {
  __shared__ float qs[FA_MAX_D];
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int kh = h / G;
  const float *qr = q + ((int64_t)h * T + t) * D;
  for (int i = lane; i < D; i += 64) qs[i] = qr[i];
  __syncthreads();
  const uint16_t *mr = mask ? mask + ((int64_t)(h % mask_heads) * mask_rows + t) * n_kv : nullptr;
  const float slope = alibi(h, H, max_bias);
  // with a softcap the scale goes inside the tanh: softcap tanh(s (scale / softcap))
  const float sc = softcap > 0.0f ? scale / softcap : scale;
  const uint16_t *kb = k + (int64_t)kh * k_hs, *vb = v + (int64_t)kh * v_hs;
  float m = -INFINITY, l = 0.0f, o[FA_MAX_D / 64];
#pragma unroll
  for (int i = 0; i < FA_MAX_D / 64; i++) o[i] = 0.0f;
  for (int j0 = 0; j0 < n_kv; j0 += 64) {
    const int j = j0 + lane;
    float s = -INFINITY;
    if (j < n_kv) {
      const float mv = mr ? h2f(mr[j]) : 0.0f;
      if (mv != -INFINITY) {
        const uint16_t *kr = kb + (int64_t)j * k_rs;
        float a = 0.0f;
        for (int d = 0; d < D; d += 8) {
          const u32x4 w = *(const u32x4 *)(kr + d);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            a = fmaf(qs[d + 2 * e], h2f((uint16_t)(w[e] & 0xffffu)), a);
            a = fmaf(qs[d + 2 * e + 1], h2f((uint16_t)(w[e] >> 16)), a);
          }
        }
        a *= sc;
        if (softcap > 0.0f) a = softcap * tanhf(a);
        s = a + slope * mv;
      }
    }
    const float mt = wave_max(s);
    if (mt == -INFINITY) continue;  // every column of the tile is masked
    const float mn = fmaxf(m, mt);
    const float corr = expf(m - mn);  // 0 while m is -inf
    const float p = s == -INFINITY ? 0.0f : expf(s - mn);
    l = l * corr + wave_sum(p);
#pragma unroll
    for (int i = 0; i < FA_MAX_D / 64; i++) o[i] *= corr;
    const int nj = n_kv - j0 < 64 ? n_kv - j0 : 64;
    for (int jj = 0; jj < nj; jj++) {
      const float pj = __shfl(p, jj);
      if (pj == 0.0f) continue;  // wave-uniform
      const uint16_t *vr = vb + (int64_t)(j0 + jj) * v_rs;
#pragma unroll
      for (int i = 0; i < FA_MAX_D / 64; i++)
        if (lane + 64 * i < D) o[i] = fmaf(pj, h2f(vr[lane + 64 * i]), o[i]);
    }
    m = mn;
  }
  float *orow = out + ((int64_t)t * H + h) * D;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int i = 0; i < FA_MAX_D / 64; i++)
    if (lane + 64 * i < D) orow[lane + 64 * i] = o[i] * inv;
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" int lgmlh_flash_attn(const float *q, int n_head, int n_tokens, int head_dim,
                                const uint16_t *k, const uint16_t *v, int n_head_kv, int n_kv,
                                int64_t k_row_stride, int64_t k_head_stride,
                                int64_t v_row_stride, int64_t v_head_stride,
                                const uint16_t *mask, int mask_heads, int mask_rows, float scale,
                                float max_bias, float softcap, float *out, void *stream) {
  if (!q || !k || !v || !out || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv ||
      n_tokens < 0 || n_kv < 0 || head_dim <= 0 || head_dim > FA_MAX_D || head_dim % 8 ||
      k_row_stride % 8 || k_head_stride % 8 || v_row_stride < 0 || v_head_stride < 0 ||
      k_row_stride < 0 || k_head_stride < 0 || ((uintptr_t)k & 15) || softcap < 0.0f) {
    set_error("flash_attn: bad arguments (head size %d: a multiple of 8 up to %d; K rows "
              "16-byte aligned)", head_dim, FA_MAX_D);
    return LGMLH_EINVAL;
  }
  if (mask && (mask_heads <= 0 || n_head % mask_heads || mask_rows < n_tokens)) {
    set_error("flash_attn: mask shape mismatch");
    return LGMLH_EINVAL;
  }
  if (!mask && max_bias > 0.0f) {
    set_error("max_bias needs a mask");
    return LGMLH_EINVAL;
  }
  if (n_tokens == 0) return LGMLH_OK;
  hipLaunchKernelGGL(flash_attn_kernel, dim3((unsigned)n_tokens, (unsigned)n_head), dim3(64), 0,
                     as_stream(stream), q, n_head, n_tokens, head_dim, k, v, n_head / n_head_kv,
                     n_kv, k_row_stride, k_head_stride, v_row_stride, v_head_stride, mask,
                     mask_heads, mask_rows, scale, max_bias, softcap, out);
  return hip_check(hipGetLastError(), "flash_attn");
}
