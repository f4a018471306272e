// Paged GQA attention over 64-cell KV blocks (gfx950, wave64, MFMA).
//
// One wavefront per work item: (sequence, KV head, group of query tokens,
// split of KV blocks). The 16 MFMA rows are (token, query head) pairs of
// the group: row r = token (r / G) and head (r % G) of the KV head's G
// query heads, so decode (one token) uses G rows and a prefill chunk packs
// 16 / G tokens per wave.
//
// Per 64-cell block the wave computes S^T = K Q^T with 16x16x32 f16 MFMAs
// (K rows straight from the [cell][D] tile), an online softmax per row in
// f32 (each lane owns one row; reductions over 4 lanes with shuffles), and
// O^T += V^T P^T (V columns straight from the transposed [D][cell] tile, P
// through 4.6 KB of LDS). K and V are exact f16; Q and P enter the MFMAs as
// f16 hi + lo pairs, so every product is f32-accurate. Splits of one token group are merged in a fixed
// order by lgmlh_merge_kernel, so results are deterministic and the same
// for a sequence alone or in any batch.
#include <math.h>

#include "common.h"

namespace lgmlh {

constexpr int ROWS = 16;      // MFMA rows per wave
constexpr int P_STRIDE = 72;  // f16 per LDS row of P (64 cells + pad)
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 load_f16x8(const uint16_t *p) {
  return __builtin_bit_cast(f16x8, *(const u32x4 *)p);
}

// Partial state of one (item, kv head): O^T rows then m, l per row.
template <int D>
struct Partial {
  static constexpr int floats = ROWS * D + 2 * ROWS;
};

template <int D>
__global__ void __launch_bounds__(64)
paged_attn_kernel(const float *__restrict__ q, int H, int Hkv, float scale_log2,
                  const uint16_t *__restrict__ kpool, const uint16_t *__restrict__ vpool,
                  const int32_t *__restrict__ items, const int32_t *__restrict__ seq_off,
                  const int32_t *__restrict__ seq_npast, const int32_t *__restrict__ block_tab,
                  int max_blocks, float *__restrict__ out, float *__restrict__ part) {
  constexpr int KS = D / 32;   // MFMA k-steps over D
  constexpr int DT = D / 16;   // d tiles of the output
  __shared__ __align__(16) uint16_t plh[ROWS * P_STRIDE];  // P as f16 hi
  __shared__ __align__(16) uint16_t pll[ROWS * P_STRIDE];  // and lo

  const int lane = threadIdx.x;
  const int item = blockIdx.x;
  const int kvh = blockIdx.y;
  const int G = H / Hkv;
  const int s = items[4 * item + 0];
  const int tok0 = items[4 * item + 1];
  const int ntok = items[4 * item + 2] & 0xffff;
  const bool direct = (items[4 * item + 2] >> 16) & 1;
  const int blo = items[4 * item + 3] & 0xffff;
  const int bhi = (items[4 * item + 3] >> 16) & 0xffff;

  const int row = lane & 15;       // the row this lane owns in S^T / O^T
  const int quad = lane >> 4;      // 0..3
  const int rtok = row / G;        // token of the row within the group
  const int rhead = kvh * G + row % G;
  const bool rvalid = rtok < ntok;
  const int p_first = seq_npast[s] + (tok0 - seq_off[s]);
  const int p_row = p_first + rtok;  // last visible position of the row

  // Q fragments (B operand): Q[row][ks*32 + quad*8 .. +7] as f16 hi + lo
  // (q = hi + lo to 22 bits; K is exact f16, so S^T is f32-accurate).
  f16x8 qh[KS], ql[KS];
  {
    const float *qr = q + ((int64_t)(tok0 + rtok) * H + rhead) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      f16x8 h = f16x8{0, 0, 0, 0, 0, 0, 0, 0}, lo = h;
      if (rvalid) {
        const f32x4 *p4 = (const f32x4 *)(qr + ks * 32 + quad * 8);
        f32x4 a = p4[0], b = p4[1];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          h[e] = (f16)a[e];
          lo[e] = (f16)(a[e] - (float)h[e]);
          h[4 + e] = (f16)b[e];
          lo[4 + e] = (f16)(b[e] - (float)h[4 + e]);
        }
      }
      qh[ks] = h;
      ql[ks] = lo;
    }
  }

  f32x4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; i++) o[i] = f32x4{0, 0, 0, 0};
  float m = -INFINITY, l = 0.0f;

  const int32_t *bt = block_tab + (int64_t)s * max_blocks;
  for (int blk = blo; blk < bhi; blk++) {
    const int64_t bid = bt[blk];
    const uint16_t *kt = kpool + (bid * Hkv + kvh) * (int64_t)(64 * D);
    const uint16_t *vt = vpool + (bid * Hkv + kvh) * (int64_t)(64 * D);

    // V^T fragments (A operand of O^T += V^T P^T), issued early.
    f16x8 vf[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int kc = 0; kc < 2; kc++)
        vf[dt][kc] = load_f16x8(vt + (dt * 16 + row) * 64 + kc * 32 + quad * 8);

    // S^T[cell][row] for 4 tiles of 16 cells.
    f32x4 st[4];
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        f16x8 kf = load_f16x8(kt + (ct * 16 + row) * D + ks * 32 + quad * 8);
        acc = mfma16(kf, qh[ks], acc);
        acc = mfma16(kf, ql[ks], acc);
      }
      st[ct] = acc;
    }

    // Mask and row max: lane holds cells ct*16 + quad*4 + i of its row.
    const int cbase = blk * 64;
    float mx = -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int p = cbase + ct * 16 + quad * 4 + i;
        float v = (rvalid && p <= p_row) ? st[ct][i] * scale_log2 : -INFINITY;
        st[ct][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = exp2f(m - m_use);  // 0 when m is -inf
    float rs = 0.0f;
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      uint16_t ph[4], pq[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float pv = exp2f(st[ct][i] - m_use);
        rs += pv;
        f16 hv = (f16)pv;
        ph[i] = __builtin_bit_cast(uint16_t, hv);
        pq[i] = f2h(pv - (float)hv);
      }
      u32x2 wh = u32x2{(uint32_t)ph[0] | ((uint32_t)ph[1] << 16),
                       (uint32_t)ph[2] | ((uint32_t)ph[3] << 16)};
      u32x2 wl = u32x2{(uint32_t)pq[0] | ((uint32_t)pq[1] << 16),
                       (uint32_t)pq[2] | ((uint32_t)pq[3] << 16)};
      *(u32x2 *)(plh + row * P_STRIDE + ct * 16 + quad * 4) = wh;
      *(u32x2 *)(pll + row * P_STRIDE + ct * 16 + quad * 4) = wl;
    }
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) o[dt] *= alpha;
    __syncthreads();  // one wave per workgroup: orders the P writes before the reads
    f16x8 pfh[2], pfl[2];
#pragma unroll
    for (int kc = 0; kc < 2; kc++) {
      pfh[kc] = load_f16x8(plh + row * P_STRIDE + kc * 32 + quad * 8);
      pfl[kc] = load_f16x8(pll + row * P_STRIDE + kc * 32 + quad * 8);
    }
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int kc = 0; kc < 2; kc++) {
        o[dt] = mfma16(vf[dt][kc], pfh[kc], o[dt]);
        o[dt] = mfma16(vf[dt][kc], pfl[kc], o[dt]);
      }
    __syncthreads();  // P reads done before the next block's writes
  }

  // Lane holds O^T[d = dt*16 + quad*4 + i][row].
  if (direct) {
    if (rvalid) {
      const float inv = 1.0f / l;
      float *orow = out + ((int64_t)(tok0 + rtok) * H + rhead) * D;
#pragma unroll
      for (int dt = 0; dt < DT; dt++) *(f32x4 *)(orow + dt * 16 + quad * 4) = o[dt] * inv;
    }
  } else {
    float *pp = part + ((int64_t)item * Hkv + kvh) * Partial<D>::floats;
#pragma unroll
    for (int dt = 0; dt < DT; dt++) *(f32x4 *)(pp + row * D + dt * 16 + quad * 4) = o[dt];
    if (quad == 0) {
      pp[ROWS * D + row] = m;
      pp[ROWS * D + ROWS + row] = l;
    }
  }
}

// Fixed-order merge of the splits of one token group (merge item:
// first item, split count, first token, token count).
template <int D>
__global__ void __launch_bounds__(256)
merge_kernel(const int32_t *__restrict__ merge, int H, int Hkv, const float *__restrict__ part,
             float *__restrict__ out) {
  const int mi = blockIdx.x, kvh = blockIdx.y;
  const int first = merge[4 * mi + 0], ns = merge[4 * mi + 1];
  const int tok0 = merge[4 * mi + 2], ntok = merge[4 * mi + 3];
  const int G = H / Hkv;
  for (int e = threadIdx.x; e < ROWS * D; e += blockDim.x) {
    int row = e / D, d = e % D;
    int rtok = row / G;
    if (rtok >= ntok) continue;
    float M = -INFINITY;
    for (int sp = 0; sp < ns; sp++) {
      const float *pp = part + ((int64_t)(first + sp) * Hkv + kvh) * Partial<D>::floats;
      M = fmaxf(M, pp[ROWS * D + row]);
    }
    float L = 0.0f, acc = 0.0f;
    for (int sp = 0; sp < ns; sp++) {
      const float *pp = part + ((int64_t)(first + sp) * Hkv + kvh) * Partial<D>::floats;
      float w = exp2f(pp[ROWS * D + row] - M);  // 0 for a split that saw no cell
      L += pp[ROWS * D + ROWS + row] * w;
      acc += pp[row * D + d] * w;
    }
    out[((int64_t)(tok0 + rtok) * H + kvh * G + row % G) * D + d] = acc / L;
  }
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" size_t lgmlh_attention_workspace(const lgmlh_plan_info *info, int head_dim) {
  if (!info) return 0;
  return (size_t)info->n_items * info->n_head_kv * (ROWS * head_dim + 2 * ROWS) * sizeof(float);
}

template <int D>
static void launch_attn(const float *q, int H, int Hkv, float scale_log2, const void *kp,
                        const void *vp, const lgmlh_ubatch *ub, float *out, float *part,
                        hipStream_t st) {
  hipLaunchKernelGGL(paged_attn_kernel<D>, dim3(ub->n_items, Hkv), dim3(64), 0, st, q, H, Hkv,
                     scale_log2, (const uint16_t *)kp, (const uint16_t *)vp, ub->items,
                     ub->seq_off, ub->seq_npast, ub->block_tab, ub->max_blocks, out, part);
  if (ub->n_merge > 0)
    hipLaunchKernelGGL(merge_kernel<D>, dim3(ub->n_merge, Hkv), dim3(256), 0, st, ub->merge, H,
                       Hkv, part, out);
}

extern "C" int lgmlh_paged_attention(const float *q, int n_head, int n_head_kv, int head_dim,
                                     float scale, const void *kpool, const void *vpool,
                                     const lgmlh_ubatch *ub, float *out, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  if (!q || !kpool || !vpool || !ub || !out || n_head_kv <= 0 || n_head % n_head_kv) {
    set_error("paged_attention: bad arguments");
    return LGMLH_EINVAL;
  }
  int G = n_head / n_head_kv;
  if (G > ROWS || ROWS % G || ub->rows != ROWS || ub->n_head_kv != n_head_kv) {
    set_error("paged_attention: %d query heads per KV head does not match the plan", G);
    return LGMLH_EINVAL;
  }
  size_t need = (size_t)ub->n_items * n_head_kv * (ROWS * head_dim + 2 * ROWS) * sizeof(float);
  if (ub->n_merge > 0 && (!workspace || workspace_bytes < need)) {
    set_error("paged_attention: workspace of %zu bytes, need %zu", workspace_bytes, need);
    return LGMLH_ENOMEM;
  }
  if (ub->n_items == 0) return LGMLH_OK;
  float sl = scale * LOG2E;
  hipStream_t st = as_stream(stream);
  switch (head_dim) {
    case 64: launch_attn<64>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, (float *)workspace, st); break;
    case 128: launch_attn<128>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, (float *)workspace, st); break;
    case 256: launch_attn<256>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, (float *)workspace, st); break;
    default:
      set_error("paged_attention: head_dim %d not supported (64, 128, 256)", head_dim);
      return LGMLH_EINVAL;
  }
  return hip_check(hipGetLastError(), "paged_attention");
}
