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
// f16 hi + lo pairs, so every product is f32-accurate. The loads of block
// b + 1 are issued as soon as block b's registers are consumed (K after
// S, V after O), so they overlap block b's softmax and products.
// Items start longest run first (the plan's order): all of a launch's
// waves are resident at once, and the ones that share a SIMD with an older
// wave advance slowly until it ends, so those should be the shortest.
//
// The splits of a token group are merged by merge_kernel in a fixed order,
// so results are deterministic and, since the split points depend only on
// the sequence's own length, the same for a sequence alone or in any batch.
// (Merging inside the attention kernel by the last split to arrive needs a
// device-scope release per split, an L2 write-back on this multi-XCD part,
// which costs more than the second launch.)
#include <math.h>

#include <type_traits>

#include "common.h"
#include "split.h"

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

// The Q8_K blocks of the output product's X (ggml's arithmetic) from the
// rows of an item in one run: a block (256 values) is 256 / D heads of one
// token, rows row .. of one row group and all four quads: value
// (row % HB) D + 16 dt + 4 quad + i of the block. The same steps as
// q8k_block8 (largest |x| and its first occurrence, iscale = -127 / max,
// q = min(127, nearest-even(iscale x)), d = 1 / iscale, the 16 sums of 16
// q); every lane takes part in the reductions, lanes of rows past the
// item's store nothing.
template <int D>
__device__ __forceinline__ void finish_q8k(const f32x4 (&o)[D / 16], float l, bool rvalid,
                                           int64_t n, int rhead, int H, int row, int quad,
                                           f16 *__restrict__ planes, int64_t npad) {
  constexpr int DT = D / 16, HB = 256 / D;
  const int64_t K = (int64_t)H * D;
  f32x4 y[DT];
  float amax = 0.0f, mx = 0.0f;
  int at = 1 << 30;
  const int kb = (row % HB) * D + quad * 4;
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
    y[dt] = o[dt] / l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float a = fabsf(y[dt][i]);
      if (a > amax) {
        amax = a;
        mx = y[dt][i];
        at = kb + dt * 16 + i;
      }
    }
  }
#pragma unroll
  for (int s = 1; s < HB; s <<= 1) q8k_amax_step(amax, mx, at, s);
  q8k_amax_step(amax, mx, at, 16);
  q8k_amax_step(amax, mx, at, 32);
  const float iscale = amax == 0.0f ? 0.0f : -127.0f / mx;
  const int64_t col = (int64_t)rhead * D + quad * 4;
  f16 *qrow = planes + n * K;
  f16 *bsrow = planes + q8_bs_off(npad, K) + n * (K / 16);
#pragma unroll
  for (int dt = 0; dt < DT; dt++) {
    float qv[4], s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      qv[i] = amax == 0.0f ? 0.0f : fminf(127.0f, __builtin_rintf(iscale * y[dt][i]));
      s += qv[i];
    }
    s += __shfl_xor(s, 16);
    s += __shfl_xor(s, 32);
    if (rvalid) {
      *(f16x4 *)(qrow + col + dt * 16) = f16x4{(f16)qv[0], (f16)qv[1], (f16)qv[2], (f16)qv[3]};
      if (quad == 0) bsrow[(col + dt * 16) >> 4] = (f16)s;
    }
  }
  if (rvalid && quad == 0 && row % HB == 0) {
    float *dp = (float *)((char *)planes + q8_d_off(npad, K));
    dp[n * (K / 256) + (int64_t)rhead * D / 256] = amax == 0.0f ? 0.0f : 1.0f / iscale;
  }
}

// The Q8_0 blocks of the output product's X (ggml's arithmetic, a Q8_0
// output matrix) from the rows of an item in one run: block g of a head is
// its d tiles 2g and 2g + 1, held by the row's four quads; the steps of
// q80_block8 (d = amax / 127, q = roundf(x / d), d kept as f16).
template <int D>
__device__ __forceinline__ void finish_q80(const f32x4 (&o)[D / 16], float l, bool rvalid,
                                           int64_t n, int rhead, int H, int quad,
                                           f16 *__restrict__ planes, int64_t npad) {
  constexpr int DT = D / 16;
  const int64_t K = (int64_t)H * D;
  float *dp = (float *)((char *)planes + q8_d_off(npad, K));
#pragma unroll
  for (int g = 0; g < DT / 2; g++) {
    const f32x4 y0 = o[2 * g] / l, y1 = o[2 * g + 1] / l;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fmaxf(fabsf(y0[i]), fabsf(y1[i])));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    if (rvalid) {
      const int64_t col = (int64_t)rhead * D + 32 * g + quad * 4;
      f16x4 h0, h1;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        h0[i] = (f16)__builtin_roundf(y0[i] * id);
        h1[i] = (f16)__builtin_roundf(y1[i] * id);
      }
      *(f16x4 *)(planes + n * K + col) = h0;
      *(f16x4 *)(planes + n * K + col + 16) = h1;
      if (quad == 0) dp[n * (K / 32) + (col >> 5)] = (float)(f16)dd;
    }
  }
}

// The end of a work item: lane holds O^T[d = dt*16 + quad*4 + i][row].
// A group in one run writes o / l (as the merge divides: a token's output
// does not depend on whether its group was split) to out or, with planes,
// to the output product's X in the form xf (split planes, or Q8_K blocks);
// a run of a split group writes its partial state (rows in use only) for
// the merge.
template <int D>
__device__ __forceinline__ void finish_item(const f32x4 (&o)[D / 16], float m, float l, int mg,
                                            bool rvalid, int tok0, int rtok, int rhead, int ntok,
                                            int G, int row, int quad, int item, int kvh, int Hkv,
                                            int H, float *__restrict__ out,
                                            f16 *__restrict__ planes, int64_t npad, int xf,
                                            float *__restrict__ part) {
  constexpr int DT = D / 16;
  if (mg < 0) {
    if constexpr (D >= 64) {
      if (planes && xf == XF_Q8K) {  // wave-uniform
        finish_q8k<D>(o, l, rvalid, tok0 + rtok, rhead, H, row, quad, planes, npad);
        return;
      }
    }
    if constexpr (D >= 32) {
      if (planes && xf == XF_Q80) {
        finish_q80<D>(o, l, rvalid, tok0 + rtok, rhead, H, quad, planes, npad);
        return;
      }
    }
    if (rvalid) {
      const int64_t n = tok0 + rtok;
      if (planes) {
        // split planes of the output product's X: the lanes of a row hold
        // 8 values of each 32-value group (d tiles 2g and 2g + 1)
        const int64_t K = (int64_t)H * D, k0 = (int64_t)rhead * D;
#pragma unroll
        for (int g = 0; g < DT / 2; g++) {
          float s = 0.0f;
#pragma unroll
          for (int h2 = 0; h2 < 2; h2++) {
            const f32x4 y = o[2 * g + h2] / l;
            const float v[4] = {y[0], y[1], y[2], y[3]};
            split_store4(planes, npad, K, n, k0 + (2 * g + h2) * 16 + quad * 4, v);
            s += v[0] + v[1] + v[2] + v[3];
          }
          s += __shfl_xor(s, 16);
          s += __shfl_xor(s, 32);
          if (quad == 0) split_store_gsum(planes, npad, K, n, (k0 >> 5) + g, s);
        }
      } else {
        float *orow = out + (n * H + rhead) * D;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) *(f32x4 *)(orow + dt * 16 + quad * 4) = o[dt] / l;
      }
    }
    return;
  }
  const int nrows = ntok * G;
  float *pp = part + ((int64_t)item * Hkv + kvh) * Partial<D>::floats;
  if (row < nrows) {
#pragma unroll
    for (int dt = 0; dt < DT; dt++) *(f32x4 *)(pp + row * D + dt * 16 + quad * 4) = o[dt];
    if (quad == 0) {
      pp[ROWS * D + row] = m;
      pp[ROWS * D + ROWS + row] = l;
    }
  }
}

// RING: a sliding-window plan. Items hold logical block ranges; logical
// block b of sequence s is ring entry b % ring, and row position p sees
// positions p - window + 1 .. p only.
template <int D, bool RING>
__global__ void __launch_bounds__(64, D <= 128 ? 2 : 1)
paged_attn_kernel(const float *__restrict__ q, int H, int Hkv, float scale_log2,
                  const uint16_t *__restrict__ kpool, const uint16_t *__restrict__ vpool,
                  const int32_t *__restrict__ items, const int32_t *__restrict__ seq_off,
                  const int32_t *__restrict__ seq_npast, const int32_t *__restrict__ block_tab,
                  int max_blocks, int ring, int window, float *__restrict__ out,
                  f16 *__restrict__ planes, int64_t npad, int xf, float *__restrict__ part,
                  const int32_t *__restrict__ order, int n_order) {
  // MFMA k-steps over D; a head of 16 takes one step of 32 whose upper
  // half is zero in K and Q (the lanes of quads 2 and 3 load nothing)
  constexpr int KS = D >= 32 ? D / 32 : 1;
  constexpr int DT = D / 16;   // d tiles of the output
  __shared__ __align__(16) uint16_t plh[ROWS * P_STRIDE];  // P as f16 hi
  __shared__ __align__(16) uint16_t pll[ROWS * P_STRIDE];  // and lo
  __shared__ __align__(16) f16x8 qsh[KS * 64], qsl[KS * 64];  // Q fragments, hi and lo

  const int lane = threadIdx.x;
  // a flat grid, KV heads fastest: workgroup w runs KV head w % Hkv of
  // slot w / Hkv, which is item order[slot] (slots past the order: item
  // slot)
  const int slot = (int)(blockIdx.x / (uint32_t)Hkv);
  const int kvh = (int)(blockIdx.x % (uint32_t)Hkv);
  const int item = order && slot < n_order ? order[slot] : slot;
  const int G = H / Hkv;
  const int s = items[4 * item + 0];
  const int tok0 = items[4 * item + 1];
  const int ntok = items[4 * item + 2] & 31;
  const int mg = (items[4 * item + 2] >> 5) - 1;  // merge group, -1: one split
  const int blo = items[4 * item + 3] & 0xffff;
  const int bhi = (items[4 * item + 3] >> 16) & 0xffff;

  const int row = lane & 15;       // the row this lane owns in S^T / O^T
  const int quad = lane >> 4;      // 0..3
  const int rtok = row / G;        // token of the row within the group
  const int rhead = kvh * G + row % G;
  const bool rvalid = rtok < ntok;
  const int p_first = seq_npast[s] + (tok0 - seq_off[s]);
  const int p_row = p_first + rtok;  // last visible position of the row

  const int32_t *bt = block_tab + (int64_t)s * max_blocks;
  auto phys = [&](int blk) -> int64_t { return RING ? bt[blk % ring] : bt[blk]; };
  auto ktile = [&](int blk) { return kpool + (phys(blk) * Hkv + kvh) * (int64_t)(64 * D); };
  auto vtile = [&](int blk) { return vpool + (phys(blk) * Hkv + kvh) * (int64_t)(64 * D); };
  // K rows (A operand of S^T = K Q^T) and V^T columns (A operand of
  // O^T += V^T P^T) of one block, straight from the pool tiles.
  f16x8 kf[4][KS], vf[DT][2];
  const bool kpart = D >= 32 || quad < 2;  // this lane's k range lies in the head
  auto load_k = [&](const uint16_t *kt) {
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
      for (int ks = 0; ks < KS; ks++)
        kf[ct][ks] = kpart ? load_f16x8(kt + (ct * 16 + row) * D + ks * 32 + quad * 8)
                           : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  };
  auto load_v = [&](const uint16_t *vt) {
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int kc = 0; kc < 2; kc++) vf[dt][kc] = load_f16x8(vt + (dt * 16 + row) * 64 + kc * 32 + quad * 8);
  };
  // Q fragments (B operand): Q[row][ks*32 + quad*8 .. +7] as f16 hi + lo
  // (q = hi + lo to 22 bits; K is exact f16, so S^T is f32-accurate). Kept
  // in LDS to leave registers for the next block's tiles. Every lane
  // addresses a valid row (rows past the group read its last token and are
  // zeroed), so all pieces load together.
  {
    const int qt = rvalid ? rtok : ntok - 1;
    const float *qr = q + ((int64_t)(tok0 + qt) * H + rhead) * D;
    f32x4 qa[2 * KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      qa[2 * ks] = kpart ? *(const f32x4 *)(qr + ks * 32 + quad * 8) : f32x4{0, 0, 0, 0};
      qa[2 * ks + 1] = kpart ? *(const f32x4 *)(qr + ks * 32 + quad * 8 + 4) : f32x4{0, 0, 0, 0};
    }
    // The first block's tiles go out before the Q pieces are converted,
    // so the two loads overlap. Unconditional, so that the conversion waits
    // for the Q pieces only (a run always has a block; block 0 of every
    // planned sequence is a valid pool block).
    const int b_first = blo < bhi ? blo : 0;
    load_k(ktile(b_first));
    load_v(vtile(b_first));
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      f16x8 h, lo;
      const f32x4 a = rvalid ? qa[2 * ks] : f32x4{0, 0, 0, 0};
      const f32x4 b = rvalid ? qa[2 * ks + 1] : f32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        h[e] = (f16)a[e];
        lo[e] = (f16)(a[e] - (float)h[e]);
        h[4 + e] = (f16)b[e];
        lo[4 + e] = (f16)(b[e] - (float)h[4 + e]);
      }
      qsh[ks * 64 + lane] = h;
      qsl[ks * 64 + lane] = lo;
    }
  }

  f32x4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; i++) o[i] = f32x4{0, 0, 0, 0};
  float m = -INFINITY, l = 0.0f;

  // One block; NEXT: the next block's tiles are loaded meanwhile
  // (straight-line code keeps the load counter waits exact, so the O
  // products do not wait for the next K). Heads of up to 128 run the last
  // block without NEXT, so no tile is loaded twice; heads of 256 (whose
  // registers are full) load the last block's tiles again, from L2.
  constexpr bool PEEL = D <= 128;
  auto block = [&](int blk, auto next) __attribute__((always_inline)) {
    constexpr bool NEXT = decltype(next)::value;
    const int nxt = blk + 1 < bhi ? blk + 1 : blk;
    // S^T[cell][row] for 4 tiles of 16 cells.
    f32x4 st[4];
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < KS; ks++) {
        acc = mfma16(kf[ct][ks], qsh[ks * 64 + lane], acc);
        acc = mfma16(kf[ct][ks], qsl[ks * 64 + lane], acc);
      }
      st[ct] = acc;
    }
    if constexpr (NEXT) load_k(ktile(nxt));

    // Mask and row max: lane holds cells ct*16 + quad*4 + i of its row. A
    // block that ends at or before the group's first position (and, with a
    // window, starts inside the window of its last) is visible to every
    // valid row.
    const int cbase = blk * 64;
    const bool full = cbase + 63 <= p_first &&
                      (!RING || cbase > p_first + ntok - 1 - window);
    float mx = -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 4; ct++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int p = cbase + ct * 16 + quad * 4 + i;
        const bool vis = full || (p <= p_row && (!RING || p > p_row - window));
        const float v = (rvalid && vis) ? st[ct][i] * scale_log2 : -INFINITY;
        st[ct][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    float rs = 0.0f;
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      uint16_t ph[4], pq[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float pv = __builtin_amdgcn_exp2f(st[ct][i] - m_use);  // exp2(-inf) = 0
        rs += pv;
        const f16 hv = (f16)pv;
        ph[i] = __builtin_bit_cast(uint16_t, hv);
        pq[i] = f2h(pv - (float)hv);
      }
      const u32x2 wh = u32x2{(uint32_t)ph[0] | ((uint32_t)ph[1] << 16),
                             (uint32_t)ph[2] | ((uint32_t)ph[3] << 16)};
      const u32x2 wl = u32x2{(uint32_t)pq[0] | ((uint32_t)pq[1] << 16),
                             (uint32_t)pq[2] | ((uint32_t)pq[3] << 16)};
      *(u32x2 *)(plh + row * P_STRIDE + ct * 16 + quad * 4) = wh;
      *(u32x2 *)(pll + row * P_STRIDE + ct * 16 + quad * 4) = wl;
    }
    rs += __shfl_xor(rs, 16);
    rs += __shfl_xor(rs, 32);
    // rescale only when some row's maximum moved
    if (__builtin_amdgcn_ballot_w64(m_new != m)) {
      const float alpha = __builtin_amdgcn_exp2f(m - m_use);  // 0 when m is -inf
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; dt++) o[dt] *= alpha;
    }
    l += rs;
    m = m_new;
    // The workgroup is one wave and a wave's LDS operations complete in
    // order: a compiler barrier orders the P writes before the reads (an
    // s_barrier would also wait for the next block's loads).
    __asm__ volatile("" ::: "memory");
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
    if constexpr (NEXT) load_v(vtile(nxt));
    __asm__ volatile("" ::: "memory");  // the P reads before the next block's writes
  };
  for (int blk = blo; blk + (PEEL ? 1 : 0) < bhi; blk++) block(blk, std::true_type{});
  if constexpr (PEEL)
    if (blo < bhi) block(bhi - 1, std::false_type{});

  finish_item<D>(o, m, l, mg, rvalid, tok0, rtok, rhead, ntok, G, row, quad, item, kvh, Hkv, H,
                 out, planes, npad, xf, part);
}

// Shared runs (a prompt chunk's query groups in sets, lgmlh_plan): one
// workgroup of SHARED_WAVES waves per (run, KV head), wave w on item
// first + w (w < n). Each K / V block of the run is loaded once into LDS
// (global-to-LDS, the next block's loads in flight while this one is
// used) and every wave reads its MFMA fragments from there: the context
// of a chunk is read once per set instead of once per group. The
// arithmetic of a wave is the per-item kernel's (same fragments, same
// order), so an item gives the same bits in either kernel. A block past a
// wave's last position is skipped (it would add nothing).
// LDS slots of 16 B: K slot (r, c) = row r (cell), chunk c of D / 8 holds
// the pool's chunk c ^ swk(r); V slot (r, c) = row r (d), chunk c of 8
// (cells) holds chunk c ^ swv(r): a 16-row fragment read touches every
// bank once.
constexpr int SHARED_WAVES = ATTN_SHARED;

template <int D>
__device__ __forceinline__ int swk(int r) {
  return D / 8 >= 16 ? (r & 15) : ((r >> 1) & 7);
}
__device__ __forceinline__ int swv(int r) { return (r >> 1) & 7; }

template <int D>
__global__ void __launch_bounds__(64 * SHARED_WAVES)
paged_attn_shared_kernel(const float *__restrict__ q, int H, int Hkv, float scale_log2,
                         const uint16_t *__restrict__ kpool, const uint16_t *__restrict__ vpool,
                         const int32_t *__restrict__ items, const int32_t *__restrict__ shared,
                         const int32_t *__restrict__ seq_off, const int32_t *__restrict__ seq_npast,
                         const int32_t *__restrict__ block_tab, int max_blocks,
                         float *__restrict__ out, f16 *__restrict__ planes, int64_t npad,
                         int xf, float *__restrict__ part) {
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int TILE = 64 * D;             // f16 of one K (or V) tile
  constexpr int KC = D / 8;                // 16-byte chunks per K row
  constexpr int LOADS = TILE / 8 / (64 * SHARED_WAVES);  // per lane and tile
  __shared__ __align__(16) uint16_t kb0[TILE], kb1[TILE], vb0[TILE], vb1[TILE];
  __shared__ __align__(16) uint16_t plh_[SHARED_WAVES][ROWS * P_STRIDE];
  __shared__ __align__(16) uint16_t pll_[SHARED_WAVES][ROWS * P_STRIDE];
  typedef __attribute__((address_space(3))) void lds_t;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int first = shared[2 * blockIdx.x], n = shared[2 * blockIdx.x + 1];
  const int kvh = blockIdx.y;
  const int G = H / Hkv;
  const bool active = wave < n;
  const int item = first + (active ? wave : 0);
  const int s = items[4 * first + 0];
  const int blo = items[4 * first + 3] & 0xffff;
  const int bhi = (items[4 * first + 3] >> 16) & 0xffff;
  const int tok0 = items[4 * item + 1];
  const int ntok = items[4 * item + 2] & 31;
  const int mg = (items[4 * item + 2] >> 5) - 1;
  uint16_t *plh = plh_[wave], *pll = pll_[wave];

  const int row = lane & 15, quad = lane >> 4;
  const int rtok = row / G;
  const int rhead = kvh * G + row % G;
  const bool rvalid = rtok < ntok;
  const int p_first = seq_npast[s] + (tok0 - seq_off[s]);
  const int p_row = p_first + rtok;
  const int p_last = p_first + ntok - 1;  // the wave's last position

  // Q fragments in registers: Q[row][ks*32 + quad*8 .. +7] as f16 hi + lo
  f16x8 qh[KS], ql[KS];
  {
    const int qt = rvalid ? rtok : ntok - 1;
    const float *qr = q + ((int64_t)(tok0 + qt) * H + rhead) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      const f32x4 a = rvalid ? *(const f32x4 *)(qr + ks * 32 + quad * 8) : f32x4{0, 0, 0, 0};
      const f32x4 b = rvalid ? *(const f32x4 *)(qr + ks * 32 + quad * 8 + 4) : f32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        qh[ks][e] = (f16)a[e];
        ql[ks][e] = (f16)(a[e] - (float)qh[ks][e]);
        qh[ks][4 + e] = (f16)b[e];
        ql[ks][4 + e] = (f16)(b[e] - (float)qh[ks][4 + e]);
      }
    }
  }

  f32x4 o[DT];
#pragma unroll
  for (int i = 0; i < DT; i++) o[i] = f32x4{0, 0, 0, 0};
  float m = -INFINITY, l = 0.0f;

  const int32_t *bt = block_tab + (int64_t)s * max_blocks;
  // Global-to-LDS loads of block blk into buffer buf: load j of this lane
  // fills slot (j * SHARED_WAVES + wave) * 64 + lane of each tile.
  auto load = [&](int blk, int buf) {
    const int64_t base = ((int64_t)bt[blk] * Hkv + kvh) * TILE;
    uint16_t *kd = buf ? kb1 : kb0, *vd = buf ? vb1 : vb0;
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
      const int slot0 = (j * SHARED_WAVES + wave) * 64, sl = slot0 + lane;
      const int kr = sl / KC, kc = (sl % KC) ^ swk<D>(sl / KC);
      const int vr = sl / 8, vc = (sl % 8) ^ swv(sl / 8);
      __builtin_amdgcn_global_load_lds((const void *)(kpool + base + kr * D + kc * 8),
                                       (lds_t *)(kd + slot0 * 8), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void *)(vpool + base + vr * 64 + vc * 8),
                                       (lds_t *)(vd + slot0 * 8), 16, 0, 0);
    }
  };
  if (blo < bhi) {
    load(blo, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (int blk = blo; blk < bhi; blk++) {
    const int buf = (blk - blo) & 1;
    if (blk + 1 < bhi) load(blk + 1, buf ^ 1);  // into the buffer freed by the last barrier
    const int cbase = blk * 64;
    if (active && cbase <= p_last) {
      const uint16_t *kt = buf ? kb1 : kb0, *vt = buf ? vb1 : vb0;
      // S^T[cell][row] for 4 tiles of 16 cells, K fragments from LDS
      f32x4 st[4];
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        const int r = ct * 16 + row;
        f16x8 kf[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
          kf[ks] = load_f16x8(kt + (r * KC + ((ks * 4 + quad) ^ swk<D>(r))) * 8);
        f32x4 acc = f32x4{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
          acc = mfma16(kf[ks], qh[ks], acc);
          acc = mfma16(kf[ks], ql[ks], acc);
        }
        st[ct] = acc;
      }
      const bool full = cbase + 63 <= p_first;
      float mx = -INFINITY;
#pragma unroll
      for (int ct = 0; ct < 4; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int p = cbase + ct * 16 + quad * 4 + i;
          const bool vis = full || p <= p_row;
          const float v = (rvalid && vis) ? st[ct][i] * scale_log2 : -INFINITY;
          st[ct][i] = v;
          mx = fmaxf(mx, v);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      float rs = 0.0f;
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        uint16_t ph[4], pq[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float pv = __builtin_amdgcn_exp2f(st[ct][i] - m_use);  // exp2(-inf) = 0
          rs += pv;
          const f16 hv = (f16)pv;
          ph[i] = __builtin_bit_cast(uint16_t, hv);
          pq[i] = f2h(pv - (float)hv);
        }
        const u32x2 wh = u32x2{(uint32_t)ph[0] | ((uint32_t)ph[1] << 16),
                               (uint32_t)ph[2] | ((uint32_t)ph[3] << 16)};
        const u32x2 wl = u32x2{(uint32_t)pq[0] | ((uint32_t)pq[1] << 16),
                               (uint32_t)pq[2] | ((uint32_t)pq[3] << 16)};
        *(u32x2 *)(plh + row * P_STRIDE + ct * 16 + quad * 4) = wh;
        *(u32x2 *)(pll + row * P_STRIDE + ct * 16 + quad * 4) = wl;
      }
      rs += __shfl_xor(rs, 16);
      rs += __shfl_xor(rs, 32);
      if (__builtin_amdgcn_ballot_w64(m_new != m)) {
        const float alpha = __builtin_amdgcn_exp2f(m - m_use);  // 0 when m is -inf
        l *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; dt++) o[dt] *= alpha;
      }
      l += rs;
      m = m_new;
      // a wave's LDS operations complete in order: the P writes before the reads
      __asm__ volatile("" ::: "memory");
      f16x8 pfh[2], pfl[2];
#pragma unroll
      for (int kc = 0; kc < 2; kc++) {
        pfh[kc] = load_f16x8(plh + row * P_STRIDE + kc * 32 + quad * 8);
        pfl[kc] = load_f16x8(pll + row * P_STRIDE + kc * 32 + quad * 8);
      }
#pragma unroll
      for (int dt = 0; dt < DT; dt++) {
        const int r = dt * 16 + row;
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
          const f16x8 vf = load_f16x8(vt + (r * 8 + ((kc * 4 + quad) ^ swv(r))) * 8);
          o[dt] = mfma16(vf, pfh[kc], o[dt]);
          o[dt] = mfma16(vf, pfl[kc], o[dt]);
        }
      }
      __asm__ volatile("" ::: "memory");  // the P reads before the next block's writes
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of blk + 1 have landed
    __syncthreads();                // ... and everyone's; buffer buf is free again
  }
  if (!active) return;
  finish_item<D>(o, m, l, mg, rvalid, tok0, rtok, rhead, ntok, G, row, quad, item, kvh, Hkv, H,
                 out, planes, npad, xf, part);
}

// Fixed-order merge of the splits of one token group (merge group: first
// item, splits, first token, tokens), one workgroup of MERGE_THREADS per
// (group, KV head). Each thread holds a position of 4 output columns (up to
// 4 per round); for each it loads, in one go per SC splits, the split
// outputs with the m and l of the position's row, and finds the row's max
// M, the split weights w = exp2(m - M) and L = sum l w itself (the threads
// of a row agree), adding the outputs weighted, in split order. A merge of
// up to SC splits is one round trip.
constexpr int MERGE_THREADS = 256;
template <int D>
__global__ void __launch_bounds__(MERGE_THREADS)
merge_kernel(const int32_t *__restrict__ merge, int H, int Hkv, const float *__restrict__ part,
             float *__restrict__ out, f16 *__restrict__ planes, int64_t npad, int xf) {
  constexpr int SC = 16, MT = MERGE_THREADS;  // splits per load round
  const int tid = threadIdx.x, lane = tid & 63, mg = blockIdx.x, kvh = blockIdx.y;
  const int first = merge[4 * mg + 0], ns = merge[4 * mg + 1];
  const int tok0 = merge[4 * mg + 2], ntok = merge[4 * mg + 3] & 0xff;
  const int stride = merge[4 * mg + 3] >> 8;  // items from one split to the next
  const int G = H / Hkv, nrows = ntok * G;
  const float *p0 = part + ((int64_t)first * Hkv + kvh) * Partial<D>::floats;
  const int64_t pstride = (int64_t)stride * Hkv * Partial<D>::floats;
  const float *ml = p0 + ROWS * D;  // m of row r at ml[r], l at ml[ROWS + r]
  const int n4 = nrows * (D / 4);
  for (int base = 0; base < n4; base += 4 * MT) {
    const int nj = min(4, (n4 - base + MT - 1) / MT);  // workgroup-uniform
    int rr[4], dd[4];
    f32x4 acc[4];
    float M[4], L[4];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      const int e4 = min(base + tid + MT * jj, n4 - 1);
      rr[jj] = e4 / (D / 4);
      dd[jj] = 4 * (e4 % (D / 4));
      acc[jj] = f32x4{0, 0, 0, 0};
      M[jj] = -INFINITY;
      L[jj] = 0.0f;
    }
    // More than SC splits: the maxima first, over every split's m.
    if (ns > SC)
      for (int s0 = 0; s0 < ns; s0 += SC) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
          if (jj < nj) {
            float mv[SC];
#pragma unroll
            for (int i = 0; i < SC; i++) mv[i] = ml[(int64_t)min(s0 + i, ns - 1) * pstride + rr[jj]];
#pragma unroll
            for (int i = 0; i < SC; i++) M[jj] = fmaxf(M[jj], mv[i]);  // repeats: same max
          }
      }
    for (int s0 = 0; s0 < ns; s0 += SC) {
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
        if (jj < nj) {
          f32x4 a[SC];
          float mv[SC], lv[SC];
#pragma unroll
          for (int i = 0; i < SC; i++) {
            const int64_t o = (int64_t)min(s0 + i, ns - 1) * pstride;
            a[i] = *(const f32x4 *)(p0 + o + rr[jj] * D + dd[jj]);
            mv[i] = ml[o + rr[jj]];
            lv[i] = ml[o + ROWS + rr[jj]];
          }
          if (ns <= SC)
#pragma unroll
            for (int i = 0; i < SC; i++) M[jj] = fmaxf(M[jj], mv[i]);
#pragma unroll
          for (int i = 0; i < SC; i++)
            if (s0 + i < ns) {
              const float w = exp2f(mv[i] - M[jj]);  // 0 for a split that saw no cell
              L[jj] += lv[i] * w;
              acc[jj] += a[i] * w;
            }
        }
    }
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
      const int e4 = base + tid + MT * jj;
      // groups of 8 lanes (D / 4 is a multiple of 8) leave together, and
      // whole waves where a wave holds a Q8_K block (n4 a multiple of 64)
      if (jj >= nj || e4 >= n4) continue;
      const int r = rr[jj], d0 = dd[jj];
      const f32x4 y = acc[jj] / L[jj];
      const int64_t n = tok0 + r / G, k = (int64_t)(kvh * G + r % G) * D + d0;
      if (planes && xf == XF_Q8K) {
        // the 64 lanes hold one Q8_K block (whole chunks: G D % 256 == 0),
        // value 4 lane + i of the block; the steps of finish_q8k
        const int64_t K = (int64_t)H * D;
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(y[i]));
        amax = group_max<64>(amax);
        const float yv[4] = {y[0], y[1], y[2], y[3]};
        const float mx = group_first_abs<64, 4>(yv, amax);
        const float iscale = amax == 0.0f ? 0.0f : -127.0f / mx;
        float qv[4], s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          qv[i] = amax == 0.0f ? 0.0f : fminf(127.0f, __builtin_rintf(iscale * y[i]));
          s += qv[i];
        }
        s += dpp_f<DPP_XOR1>(s);
        s += dpp_f<DPP_XOR2>(s);
        *(f16x4 *)(planes + n * K + k) = f16x4{(f16)qv[0], (f16)qv[1], (f16)qv[2], (f16)qv[3]};
        if ((lane & 3) == 0) planes[q8_bs_off(npad, K) + n * (K / 16) + (k >> 4)] = (f16)s;
        if (lane == 0) {
          float *dp = (float *)((char *)planes + q8_d_off(npad, K));
          dp[n * (K / 256) + (k >> 8)] = amax == 0.0f ? 0.0f : 1.0f / iscale;
        }
      } else if (planes && xf == XF_Q80) {
        // 8 lanes hold a Q8_0 block (32 values); the steps of q80_block8
        const int64_t K = (int64_t)H * D;
        float amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
        amax = group_max<8>(amax);
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        *(f16x4 *)(planes + n * K + k) =
            f16x4{(f16)__builtin_roundf(y[0] * id), (f16)__builtin_roundf(y[1] * id),
                  (f16)__builtin_roundf(y[2] * id), (f16)__builtin_roundf(y[3] * id)};
        if ((e4 & 7) == 0) {
          float *dp = (float *)((char *)planes + q8_d_off(npad, K));
          dp[n * (K / 32) + (k >> 5)] = (float)(f16)dd;
        }
      } else if (planes) {
        // 8 lanes hold a 32-value group
        const int64_t K = (int64_t)H * D;
        const float v[4] = {y[0], y[1], y[2], y[3]};
        split_store4(planes, npad, K, n, k, v);
        float s = v[0] + v[1] + v[2] + v[3];
        s += dpp_f<DPP_XOR1>(s);
        s += dpp_f<DPP_XOR2>(s);
        s += __shfl_xor(s, 4);
        if ((e4 & 7) == 0) split_store_gsum(planes, npad, K, n, k >> 5, s);
      } else {
        *(f32x4 *)(out + n * H * D + k) = y;
      }
    }
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
                        const void *vp, const lgmlh_ubatch *ub, float *out, f16 *planes,
                        int64_t npad, int xf, float *part, hipStream_t st) {
  // one workgroup per (item, KV head), the items on their own in the
  // plan's order
  if (ub->ring > 0)
    hipLaunchKernelGGL((paged_attn_kernel<D, true>), dim3((uint32_t)ub->n_single * Hkv),
                       dim3(64), 0, st, q, H, Hkv, scale_log2, (const uint16_t *)kp,
                       (const uint16_t *)vp, ub->items, ub->seq_off, ub->seq_npast, ub->block_tab,
                       ub->max_blocks, ub->ring, ub->window, out, planes, npad, xf, part,
                       ub->order, ub->n_single);
  // heads of 256, and of 32 or less, run the shared runs' items with the
  // per-item kernel too
  else if (const int n1 = D <= 128 && D >= 64 ? ub->n_single : ub->n_items; n1 > 0)
    hipLaunchKernelGGL((paged_attn_kernel<D, false>), dim3((uint32_t)n1 * Hkv), dim3(64), 0, st,
                       q, H, Hkv, scale_log2, (const uint16_t *)kp, (const uint16_t *)vp,
                       ub->items, ub->seq_off, ub->seq_npast, ub->block_tab, ub->max_blocks, 0,
                       0, out, planes, npad, xf, part, ub->order, ub->n_single);
  if (ub->ring == 0 && ub->n_shared > 0) {
    if constexpr (D <= 128 && D >= 64)
      hipLaunchKernelGGL(paged_attn_shared_kernel<D>, dim3(ub->n_shared, Hkv),
                         dim3(64 * SHARED_WAVES), 0, st, q, H, Hkv, scale_log2,
                         (const uint16_t *)kp, (const uint16_t *)vp, ub->items, ub->shared,
                         ub->seq_off, ub->seq_npast, ub->block_tab, ub->max_blocks, out, planes,
                         npad, xf, part);
  }
  if (ub->n_merge > 0)
    hipLaunchKernelGGL(merge_kernel<D>, dim3(ub->n_merge, Hkv), dim3(MERGE_THREADS), 0, st, ub->merge, H,
                       Hkv, part, out, planes, npad, xf);
}

namespace lgmlh {
// The attention output as f32 rows (out) or, with planes set, as the
// output product's X in the form xf (rows padded to npad): XF_SPLIT split
// planes or XF_Q80 blocks (heads of 32 or more), or XF_Q8K blocks when a
// block's 256 / D heads are of one KV head's group (heads of 64 or more,
// G % (256 / D) == 0: attn_q8k_fits).
bool attn_q8k_fits(int head_dim, int G) {
  return head_dim >= 64 && head_dim <= 256 && G % (256 / head_dim) == 0;
}

int paged_attention_dev(const float *q, int n_head, int n_head_kv, int head_dim, float scale,
                        const void *kpool, const void *vpool, const lgmlh_ubatch *ub, float *out,
                        f16 *planes, int64_t npad, void *workspace, size_t workspace_bytes,
                        hipStream_t st, int xf) {
  if (!q || !kpool || !vpool || !ub || !(out || planes) || n_head_kv <= 0 ||
      n_head % n_head_kv) {
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
  if ((int64_t)ub->n_items * n_head_kv > (int64_t)1 << 25) {  // the per-item grid's threads
    set_error("paged_attention: %d items x %d KV heads in one launch", ub->n_items, n_head_kv);
    return LGMLH_EINVAL;
  }
  if (planes && (xf == XF_Q8K ? !attn_q8k_fits(head_dim, G) : head_dim < 32)) {
    set_error("paged_attention: heads of %d (%d per KV head) cannot write X form %d", head_dim,
              G, xf);
    return LGMLH_EINVAL;
  }
  float sl = scale * LOG2E;
  float *part = (float *)workspace;
  switch (head_dim) {
    case 16: launch_attn<16>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, planes, npad, xf, part, st); break;
    case 32: launch_attn<32>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, planes, npad, xf, part, st); break;
    case 64: launch_attn<64>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, planes, npad, xf, part, st); break;
    case 128: launch_attn<128>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, planes, npad, xf, part, st); break;
    case 256: launch_attn<256>(q, n_head, n_head_kv, sl, kpool, vpool, ub, out, planes, npad, xf, part, st); break;
    default:
      set_error("paged_attention: head_dim %d not supported (16, 32, 64, 128, 256)", head_dim);
      return LGMLH_EINVAL;
  }
  return hip_check(hipGetLastError(), "paged_attention");
}
}  // namespace lgmlh

extern "C" int lgmlh_paged_attention(const float *q, int n_head, int n_head_kv, int head_dim,
                                     float scale, const void *kpool, const void *vpool,
                                     const lgmlh_ubatch *ub, float *out, void *workspace,
                                     size_t workspace_bytes, void *stream) {
  if (!out) {
    set_error("paged_attention: bad arguments");
    return LGMLH_EINVAL;
  }
  return paged_attention_dev(q, n_head, n_head_kv, head_dim, scale, kpool, vpool, ub, out,
                             nullptr, 0, workspace, workspace_bytes, as_stream(stream), XF_SPLIT);
}
