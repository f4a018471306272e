// Routed experts (mixture of experts) of qwen3moe-style layers: the router
// of M.moe (transformer.lua:1989-2027) and graph:mul_mat_id
// (src/ops_nn.c:322-362) with the weighted sum of the picks (experts and
// sum_picks, transformer.lua:1875-1910).
//
// A pass of T tokens with n_used picks each has P = T n_used picks. The
// router logits come from a split-K f32 product; one workgroup then turns
// them into the picks and weights and groups the picks by expert: sorted
// holds the picks of expert 0, then of expert 1, ... (each in pick order),
// and a tile list cuts every expert's picks into column tiles of 16 (or
// 64) for the grouped quantized product (gemm.hip, Gather). Experts nobody
// picked cost nothing; an expert's weights are read once per tile.
#include <math.h>

#include "common.h"
#include "moe.h"
#include "quant.h"
#include "split.h"

namespace lgmlh {


constexpr int ROUTE_THREADS = 1024;
constexpr int ROUTE_WAVES = ROUTE_THREADS / 64;
constexpr int MOE_MAX_EXPERTS = 512;  // 8 logits per lane
constexpr int MOE_MAX_USED = 16;
constexpr int MOE_MAX_PICKS = 8192;   // picks of one pass (LDS)

// ---- router logits: split-K f32 product -------------------------------------
// part[z][n][e] = sum over k in [256 z, 256 z + 256) of W[e][k] x[n][k], in
// k order (fmaf). A workgroup takes 16 experts x TOK tokens of one K chunk;
// thread t owns expert t % 16 for tokens t / 16 + 16 j (j < TOK / 16).
// TOK is 64, or 16 for a batch of at most 64 tokens (four times the
// workgroups; each sum is the same fmaf chain either way).
constexpr int ROUTER_KC = 256;
constexpr int ROUTER_LD = ROUTER_KC + 4;  // row pitch (floats): 16-byte rows, no bank conflicts
template <int TOK>
__global__ void __launch_bounds__(256)
router_part_kernel(const float *__restrict__ w, int NE, int64_t K, const float *__restrict__ x,
                   int64_t N, float *__restrict__ part) {
  constexpr int TJ = TOK / 16;  // tokens per thread
  __shared__ __align__(16) float ws_[16 * ROUTER_LD];
  __shared__ __align__(16) float xs_[TOK * ROUTER_LD];
  const int t = threadIdx.x, e = t & 15, tq = t >> 4;
  const int64_t e0 = (int64_t)blockIdx.x * 16, n0 = (int64_t)blockIdx.z * TOK;
  const int64_t k0 = (int64_t)blockIdx.y * ROUTER_KC;
  // 16-byte loads, all issued before the first LDS store: float4 i of a
  // row of ROUTER_KC / 4 (K % 4 == 0)
  constexpr int Q = ROUTER_KC / 4;
  constexpr int WJ = 16 * Q / 256, XJ = TOK * Q / 256;
  f32x4 wv_[WJ], xv_[XJ];
#pragma unroll
  for (int j = 0; j < WJ; j++) {
    const int i = t + 256 * j, r = i / Q, c4 = 4 * (i % Q);
    wv_[j] = f32x4{0, 0, 0, 0};
    if (e0 + r < NE && k0 + c4 < K) wv_[j] = *(const f32x4 *)(w + (e0 + r) * K + k0 + c4);
  }
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int i = t + 256 * j, r = i / Q, c4 = 4 * (i % Q);
    xv_[j] = f32x4{0, 0, 0, 0};
    if (n0 + r < N && k0 + c4 < K) xv_[j] = *(const f32x4 *)(x + (n0 + r) * K + k0 + c4);
  }
#pragma unroll
  for (int j = 0; j < WJ; j++) {
    const int i = t + 256 * j;
    *(f32x4 *)&ws_[(i / Q) * ROUTER_LD + 4 * (i % Q)] = wv_[j];
  }
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int i = t + 256 * j;
    *(f32x4 *)&xs_[(i / Q) * ROUTER_LD + 4 * (i % Q)] = xv_[j];
  }
  __syncthreads();
  float acc[TJ];
#pragma unroll
  for (int j = 0; j < TJ; j++) acc[j] = 0.0f;
  const float *wr = ws_ + e * ROUTER_LD;
#pragma unroll 4
  for (int c = 0; c < ROUTER_KC; c += 4) {
    const f32x4 wv = *(const f32x4 *)(wr + c);
#pragma unroll
    for (int j = 0; j < TJ; j++) {
      const f32x4 xv = *(const f32x4 *)(xs_ + (tq + 16 * j) * ROUTER_LD + c);
      acc[j] = fmaf(wv[0], xv[0], acc[j]);
      acc[j] = fmaf(wv[1], xv[1], acc[j]);
      acc[j] = fmaf(wv[2], xv[2], acc[j]);
      acc[j] = fmaf(wv[3], xv[3], acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int64_t n = n0 + tq + 16 * j;
    if (e0 + e < NE && n < N) part[((int64_t)blockIdx.y * N + n) * NE + e0 + e] = acc[j];
  }
}

// The same partials for a prefill-sized batch: a workgroup takes 64
// experts x ROUTER_TT tokens of one K chunk, thread t experts t % 16 + 16 i
// (i < 4) and tokens t / 16 + 16 j (j < ROUTER_TT / 16), so each K fragment
// read from LDS feeds several products. Each sum is the same fmaf chain in
// k order.
constexpr int ROUTER_TT = 64;
__global__ void __launch_bounds__(256)
router_tile_kernel(const float *__restrict__ w, int NE, int64_t K, const float *__restrict__ x,
                   int64_t N, float *__restrict__ part) {
  constexpr int TE = 64, TT = ROUTER_TT, TJ = TT / 16, Q = ROUTER_KC / 4;
  __shared__ __align__(16) float ws_[TE * ROUTER_LD];
  __shared__ __align__(16) float xs_[TT * ROUTER_LD];
  const int t = threadIdx.x, ei = t & 15, ti = t >> 4;
  const int64_t e0 = (int64_t)blockIdx.x * TE, n0 = (int64_t)blockIdx.z * TT;
  const int64_t k0 = (int64_t)blockIdx.y * ROUTER_KC;
  // 16-byte loads, all issued before the first LDS store
  constexpr int WJ = TE * Q / 256, XJ = TT * Q / 256;
  f32x4 wv_[WJ], xv_[XJ];
#pragma unroll
  for (int j = 0; j < WJ; j++) {
    const int i = t + 256 * j, r = i / Q, c4 = 4 * (i % Q);
    wv_[j] = f32x4{0, 0, 0, 0};
    if (e0 + r < NE && k0 + c4 < K) wv_[j] = *(const f32x4 *)(w + (e0 + r) * K + k0 + c4);
  }
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int i = t + 256 * j, r = i / Q, c4 = 4 * (i % Q);
    xv_[j] = f32x4{0, 0, 0, 0};
    if (n0 + r < N && k0 + c4 < K) xv_[j] = *(const f32x4 *)(x + (n0 + r) * K + k0 + c4);
  }
#pragma unroll
  for (int j = 0; j < WJ; j++) {
    const int i = t + 256 * j;
    *(f32x4 *)&ws_[(i / Q) * ROUTER_LD + 4 * (i % Q)] = wv_[j];
  }
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int i = t + 256 * j;
    *(f32x4 *)&xs_[(i / Q) * ROUTER_LD + 4 * (i % Q)] = xv_[j];
  }
  __syncthreads();
  float acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = 0.0f;
#pragma unroll 2
  for (int c = 0; c < ROUTER_KC; c += 4) {
    f32x4 wv[4], xv[TJ];
#pragma unroll
    for (int i = 0; i < 4; i++) wv[i] = *(const f32x4 *)(ws_ + (ei + 16 * i) * ROUTER_LD + c);
#pragma unroll
    for (int j = 0; j < TJ; j++) xv[j] = *(const f32x4 *)(xs_ + (ti + 16 * j) * ROUTER_LD + c);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < TJ; j++) {
        acc[i][j] = fmaf(wv[i][0], xv[j][0], acc[i][j]);
        acc[i][j] = fmaf(wv[i][1], xv[j][1], acc[i][j]);
        acc[i][j] = fmaf(wv[i][2], xv[j][2], acc[i][j]);
        acc[i][j] = fmaf(wv[i][3], xv[j][3], acc[i][j]);
      }
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) {
      const int64_t e = e0 + ei + 16 * i, n = n0 + ti + 16 * j;
      if (e < NE && n < N) part[((int64_t)blockIdx.y * N + n) * NE + e] = acc[i][j];
    }
}

// ---- picks and weights ---------------------------------------------------------
// (value, index) order of the top-k: larger value first, then smaller index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  return a > b || (a == b && ia < ib);
}

// Reductions over the 16 lanes of a lane group (one DPP row) by a butterfly
// of row permutes (dpp_f, common.h): lane ^ 1, lane ^ 2 (quad permutes),
// then the mirrors within 8 and within 16 lanes. Every lane ends with the
// same result.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, dpp_f<DPP_XOR1>(v));
  v = fmaxf(v, dpp_f<DPP_XOR2>(v));
  v = fmaxf(v, dpp_f<DPP_HALF_MIRROR>(v));
  return fmaxf(v, dpp_f<DPP_MIRROR>(v));
}
// Partner sums: a + b at one lane, b + a at its partner (equal), so every
// lane holds the same sum.
__device__ __forceinline__ float row_sum(float v) {
  v += dpp_f<DPP_XOR1>(v);
  v += dpp_f<DPP_XOR2>(v);
  v += dpp_f<DPP_HALF_MIRROR>(v);
  return v + dpp_f<DPP_MIRROR>(v);
}
// The best (value, index) of the row. NaN values never win (better() is
// false both ways), so the order is total over the candidates and every
// pairing gives the same winner.
template <int CTRL>
__device__ __forceinline__ void best_step(float &bv, int &bi) {
  const float ov = dpp_f<CTRL>(bv);
  const int oi = dpp_i<CTRL>(bi);
  if (better(ov, oi, bv, bi)) {
    bv = ov;
    bi = oi;
  }
}
__device__ __forceinline__ void row_best(float &bv, int &bi) {
  best_step<DPP_XOR1>(bv, bi);
  best_step<DPP_XOR2>(bv, bi);
  best_step<DPP_HALF_MIRROR>(bv, bi);
  best_step<DPP_MIRROR>(bv, bi);
}

// Routing of token t by the 16 lanes sub = 0..15 of a lane group (lane
// holds experts sub + 16 i, i < PER): logits l = sum of the nz partial
// rows (in order); probs = soft_max (f32: max, exp, sum over the group in a
// fixed tree) or sigmoid; the n_used largest logits (the gating is
// monotone) as ids, largest first, ties to the smaller index
// (argsort_top_k); weights = probs of the ids, / max(sum, 6.103515625e-5)
// when norm_topk (transformer.lua:2003-2005), times scale (:2006-2008).
// Tokens t >= T run along (their lanes take part in the row permutes) and
// write nothing.
template <int PER>
__device__ void route_token(const float *__restrict__ part, int nz, int64_t T, int64_t t, int NE,
                            int n_used, int gating, int norm_topk, float scale, int sub,
                            int32_t *__restrict__ ids, float *__restrict__ wts,
                            int32_t *ids_lds) {
  const bool live = t < T;
  const int64_t tt = live ? t : 0;
  float l[PER], p[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) l[i] = 0.0f;
  // Split sums in split order. Every lane loads an in-range address
  // (experts past NE read expert 0 and are dropped below), ZB splits at a
  // time, so the loads of a batch are in flight together.
  constexpr int ZB = PER <= 8 ? 4 : PER <= 16 ? 2 : 1;
  // (32-bit element offsets: the partials of a pass stay far below 2^30
  // floats, and the loads then share one 64-bit base)
  auto load = [&](int z, float (&v)[PER]) {
    const uint32_t row = (uint32_t)(((int64_t)z * T + tt) * NE);
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = sub + 16 * i;
      v[i] = part[row + (uint32_t)(e < NE ? e : 0)];
    }
  };
  int z = 0;
  for (; z + ZB <= nz; z += ZB) {
    float v[ZB][PER];
#pragma unroll
    for (int zz = 0; zz < ZB; zz++) load(z + zz, v[zz]);
#pragma unroll
    for (int zz = 0; zz < ZB; zz++)
#pragma unroll
      for (int i = 0; i < PER; i++) l[i] += v[zz][i];
  }
  for (; z < nz; z++) {
    float v[PER];
    load(z, v);
#pragma unroll
    for (int i = 0; i < PER; i++) l[i] += v[i];
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    if (sub + 16 * i >= NE) l[i] = -INFINITY;
    mx = fmaxf(mx, l[i]);
  }
  mx = row_max(mx);
  if (gating == LGMLH_GATING_SOFTMAX) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      p[i] = sub + 16 * i < NE ? expf(l[i] - mx) : 0.0f;
      s += p[i];
    }
    s = row_sum(s);
#pragma unroll
    for (int i = 0; i < PER; i++) p[i] = p[i] / s;
  } else {
#pragma unroll
    for (int i = 0; i < PER; i++) p[i] = 1.0f / (1.0f + expf(-l[i]));
  }
  // Round j picks the j-th id; lane sub == j keeps it. Every lane adds the
  // weights in pick order (the norm_topk sum).
  uint32_t taken = 0;
  int my_sel = 0;
  float my_w = 0.0f, wsum = 0.0f;
  for (int j = 0; j < n_used; j++) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = sub + 16 * i;
      if (e < NE && !(taken >> i & 1u) && better(l[i], e, bv, bi)) {
        bv = l[i];
        bi = e;
      }
    }
    row_best(bv, bi);
    // every lane of the group holds the winner now (none when the logits
    // are NaN: expert 0 then, so ids stay in range); its owner marks it
    // and sends its prob
    if (bi >= NE) bi = 0;
    float pw = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; i++)
      if (bi == sub + 16 * i) {
        taken |= 1u << i;
        pw = p[i];
      }
    // from lane (bi % 16) of this group
    const float w = __shfl(pw, (int)(__lane_id() & ~15u) + (bi & 15));
    wsum += w;
    if (sub == j) {
      my_sel = bi;
      my_w = w;
    }
  }
  if (norm_topk) my_w = my_w / fmaxf(wsum, 6.103515625e-5f);
  if (scale != 1.0f) my_w = my_w * scale;
  if (live && sub < n_used) {
    ids[t * n_used + sub] = my_sel;
    wts[t * n_used + sub] = my_w;
    if (ids_lds) ids_lds[t * n_used + sub] = my_sel;
  }
}

// ---- grouping of the picks by expert ------------------------------------------

struct GroupLds {
  int32_t ids[MOE_MAX_PICKS];
  int32_t base[ROUTE_WAVES][MOE_MAX_EXPERTS];  // per wave chunk: counts, then bases
  int32_t off[MOE_MAX_EXPERTS + 1];
  int32_t toff[MOE_MAX_EXPERTS + 1];
};

// Counting sort of the picks (ids in lds.ids; negative = no expert) by
// expert, stable: wave w ranks the picks of its chunk. Called by all
// ROUTE_THREADS threads.
__device__ void group_picks(GroupLds &lds, int P, int NE, const GroupOut &go) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < ROUTE_WAVES * MOE_MAX_EXPERTS; i += ROUTE_THREADS)
    (&lds.base[0][0])[i] = 0;
  __syncthreads();
  const int chunk = ((P + ROUTE_WAVES - 1) / ROUTE_WAVES + 63) & ~63;
  const int lo = wave * chunk, hi = lo + chunk < P ? lo + chunk : P;
  for (int p = lo + lane; p < hi; p += 64) {
    int e = lds.ids[p];
    if ((unsigned)e >= (unsigned)NE) lds.ids[p] = e = -1;  // no expert
    if (e >= 0) atomicAdd(&lds.base[wave][e], 1);  // counts: order-free
  }
  __syncthreads();
  // per expert (one thread each): its total, its tiles, and the bases of
  // the wave chunks relative to the expert's first pick
  int cnt = 0, nt = 0;
  if (tid < NE) {
    int c[ROUTE_WAVES];
#pragma unroll
    for (int ww = 0; ww < ROUTE_WAVES; ww++) c[ww] = lds.base[ww][tid];
#pragma unroll
    for (int ww = 0; ww < ROUTE_WAVES; ww++) {
      lds.base[ww][tid] = cnt;
      cnt += c[ww];
    }
    nt = (cnt + go.tile_cols - 1) / go.tile_cols;
  }
  // exclusive scans of cnt and nt over the experts: within each wave, then
  // over the waves (NE <= 512: 8 waves)
  int ci = cnt, ti = nt;
  for (int o = 1; o < 64; o <<= 1) {
    const int a = __shfl_up(ci, o), b = __shfl_up(ti, o);
    if (lane >= o) {
      ci += a;
      ti += b;
    }
  }
  if (lane == 63 && wave < MOE_MAX_EXPERTS / 64) {
    lds.off[wave] = ci;   // wave totals (off / toff are rewritten below)
    lds.toff[wave] = ti;
  }
  __syncthreads();
  int cw = 0, tw = 0;
  for (int ww = 0; ww < wave && ww < MOE_MAX_EXPERTS / 64; ww++) {
    cw += lds.off[ww];
    tw += lds.toff[ww];
  }
  __syncthreads();
  if (tid < NE) {
    const int c0 = cw + ci - cnt, t0 = tw + ti - nt;
    lds.off[tid] = c0;
    lds.toff[tid] = t0;
#pragma unroll
    for (int ww = 0; ww < ROUTE_WAVES; ww++) lds.base[ww][tid] += c0;
    if (tid == NE - 1) {
      lds.off[NE] = c0 + cnt;
      lds.toff[NE] = t0 + nt;
      *go.n_tiles = t0 + nt;
    }
  }
  __syncthreads();
  // stable placement: rounds of 64 picks; a pick's rank among the round's
  // picks of the same expert comes from the lanes before it
  for (int r0 = lo; r0 < hi; r0 += 64) {
    const int p = r0 + lane;
    const int e = p < hi ? lds.ids[p] : -1;
    int rank = 0, tot = 0;
    for (int l2 = 0; l2 < 64; l2++) {
      const int e2 = __builtin_amdgcn_readlane(e, l2);  // lane l2's expert, to every lane
      const int same = e2 == e ? 1 : 0;
      tot += same;
      rank += l2 < lane ? same : 0;
    }
    const int b = e >= 0 ? lds.base[wave][e] : 0;
    if (e >= 0) go.sorted[b + rank] = p;
    __builtin_amdgcn_wave_barrier();  // all lanes read base before it moves
    if (e >= 0 && rank == 0) lds.base[wave][e] = b + tot;
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // the tile list, expert by expert
  for (int e = tid; e < NE; e += ROUTE_THREADS) {
    const int c = lds.off[e + 1] - lds.off[e];
    for (int i = 0, t = lds.toff[e]; i * go.tile_cols < c; i++, t++) {
      const int first = lds.off[e] + i * go.tile_cols;
      const int n = c - i * go.tile_cols < go.tile_cols ? c - i * go.tile_cols : go.tile_cols;
      go.tiles[t] = int4{e, first, n, 0};
    }
  }
}

// Routing of T tokens (one workgroup, 16 lanes per token); with group
// set, also the grouping. PER = experts per lane (NE <= 16 PER).
template <int PER>
__global__ void __launch_bounds__(ROUTE_THREADS)
route_kernel(const float *__restrict__ part, int nz, int64_t T, int NE, int n_used, int gating,
             int norm_topk, float scale, int32_t *__restrict__ ids, float *__restrict__ wts,
             int group, GroupOut go) {
  __shared__ GroupLds lds;
  const int tid = threadIdx.x;
  for (int64_t t0 = 0; t0 < T; t0 += ROUTE_THREADS / 16)
    route_token<PER>(part, nz, T, t0 + tid / 16, NE, n_used, gating, norm_topk, scale, tid & 15,
                     ids, wts, group ? lds.ids : nullptr);
  if (!group) return;
  __syncthreads();
  group_picks(lds, (int)(T * n_used), NE, go);
}

// Routing alone over many workgroups: 16 tokens per workgroup of 256
// threads (no LDS), so the tokens spread over the CUs.
template <int PER>
__global__ void __launch_bounds__(256)
route_many_kernel(const float *__restrict__ part, int nz, int64_t T, int NE, int n_used,
                  int gating, int norm_topk, float scale, int32_t *__restrict__ ids,
                  float *__restrict__ wts) {
  const int64_t t = (int64_t)blockIdx.x * 16 + threadIdx.x / 16;
  route_token<PER>(part, nz, T, t, NE, n_used, gating, norm_topk, scale, threadIdx.x & 15, ids,
                   wts, nullptr);
}

// Grouping of given ids (graph:mul_mat_id's ids). Picks whose id is outside
// [0, NE) join no expert; their Y rows (M values) are written as zeros.
__global__ void __launch_bounds__(ROUTE_THREADS)
group_kernel(const int32_t *__restrict__ ids, int P, int NE, GroupOut go, float *__restrict__ y,
             int64_t M) {
  __shared__ GroupLds lds;
  for (int p = threadIdx.x; p < P; p += ROUTE_THREADS) {
    const int e = ids[p];
    const bool ok = e >= 0 && e < NE;
    lds.ids[p] = ok ? e : -1;
    if (!ok)
      for (int64_t m = 0; m < M; m++) y[(int64_t)p * M + m] = 0.0f;
  }
  __syncthreads();
  group_picks(lds, P, NE, go);
}

// Grouping over many workgroups, for thousands of picks: chunks of
// GROUP_CHUNK picks. group_count_kernel ranks each pick among the picks of
// its chunk with the same expert (stable) and counts the chunk's picks per
// expert; group_place_kernel adds the counts of the chunks before its own
// and the experts before each expert, and places its picks. The result is
// the one-workgroup grouping's: expert-major, pick order within an expert.
constexpr int GROUP_CHUNK = 256;
constexpr int GROUP_ONE = 1024;  // picks grouped by one workgroup

__global__ void __launch_bounds__(GROUP_CHUNK)
group_count_kernel(const int32_t *__restrict__ ids, int P, int NE, GroupOut go,
                   float *__restrict__ y, int64_t M) {
  __shared__ int32_t cnt[GROUP_CHUNK / 64][MOE_MAX_EXPERTS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < (GROUP_CHUNK / 64) * MOE_MAX_EXPERTS; i += GROUP_CHUNK)
    (&cnt[0][0])[i] = 0;
  const int p = blockIdx.x * GROUP_CHUNK + tid;
  int e = p < P ? ids[p] : -1;
  if (p < P && (e < 0 || e >= NE)) {
    e = -1;  // no expert: its Y row is zeros
    if (y)
      for (int64_t m = 0; m < M; m++) y[(int64_t)p * M + m] = 0.0f;
  }
  // rank among the wave's earlier lanes with the same expert
  int rank = 0;
  for (int l2 = 0; l2 < 64; l2++) {
    const int e2 = __builtin_amdgcn_readlane(e, l2);
    rank += (l2 < lane && e2 == e) ? 1 : 0;
  }
  __syncthreads();
  if (e >= 0) atomicAdd(&cnt[wave][e], 1);  // counts: order-free
  __syncthreads();
  if (p < P) {
    // the pick's expert and rank in its chunk (-1: no expert)
    for (int w2 = 0; w2 < wave && e >= 0; w2++) rank += cnt[w2][e];
    go.rank[p] = e >= 0 ? (e << 16) | rank : -1;
  }
  for (int ee = tid; ee < NE; ee += GROUP_CHUNK) {
    int c = 0;
#pragma unroll
    for (int w2 = 0; w2 < GROUP_CHUNK / 64; w2++) c += cnt[w2][ee];
    go.counts[(int64_t)blockIdx.x * NE + ee] = c;
  }
}

__global__ void __launch_bounds__(GROUP_CHUNK)
group_place_kernel(int P, int NE, GroupOut go) {
  __shared__ int32_t base[MOE_MAX_EXPERTS];
  __shared__ int32_t off[MOE_MAX_EXPERTS + 1], toff[MOE_MAX_EXPERTS + 1];
  __shared__ int32_t wsum[2][GROUP_CHUNK / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = (P + GROUP_CHUNK - 1) / GROUP_CHUNK, c0 = blockIdx.x;
  // experts tid, tid + GROUP_CHUNK (NE <= 512): their totals and the picks
  // of the chunks before this one
  constexpr int EPT = MOE_MAX_EXPERTS / GROUP_CHUNK;
  int tot[EPT], pre[EPT];
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int e = tid + j * GROUP_CHUNK;
    tot[j] = pre[j] = 0;
    if (e < NE)
      for (int c = 0; c < C; c++) {
        const int v = go.counts[(int64_t)c * NE + e];
        tot[j] += v;
        pre[j] += c < c0 ? v : 0;
      }
  }
  // exclusive scans over the experts of the totals and of the tile counts:
  // expert e = tid + j GROUP_CHUNK, scanned in e order
  int run_c = 0, run_t = 0;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int e = tid + j * GROUP_CHUNK;
    const int nt = (tot[j] + go.tile_cols - 1) / go.tile_cols;
    int ci = tot[j], ti = nt;
    for (int o = 1; o < 64; o <<= 1) {
      const int a = __shfl_up(ci, o), b = __shfl_up(ti, o);
      if (lane >= o) {
        ci += a;
        ti += b;
      }
    }
    if (lane == 63) {
      wsum[0][wave] = ci;
      wsum[1][wave] = ti;
    }
    __syncthreads();
    int cw = run_c, tw = run_t;
    for (int w2 = 0; w2 < wave; w2++) {
      cw += wsum[0][w2];
      tw += wsum[1][w2];
    }
    for (int w2 = 0; w2 < GROUP_CHUNK / 64; w2++) {
      run_c += wsum[0][w2];
      run_t += wsum[1][w2];
    }
    if (e < NE) {
      off[e] = cw + ci - tot[j];
      toff[e] = tw + ti - nt;
      base[e] = off[e] + pre[j];
    }
    __syncthreads();
  }
  if (tid == 0) {
    off[NE] = run_c;
    toff[NE] = run_t;
    if (c0 == 0) *go.n_tiles = run_t;
  }
  __syncthreads();
  const int p = c0 * GROUP_CHUNK + tid;
  if (p < P) {
    const int v = go.rank[p];
    if (v >= 0) go.sorted[base[v >> 16] + (v & 0xffff)] = p;
  }
  if (c0 != 0) return;
  // the tile list, expert by expert
  for (int e = tid; e < NE; e += GROUP_CHUNK) {
    const int c = off[e + 1] - off[e];
    for (int i = 0, t = toff[e]; i * go.tile_cols < c; i++, t++) {
      const int first = off[e] + i * go.tile_cols;
      const int n = c - i * go.tile_cols < go.tile_cols ? c - i * go.tile_cols : go.tile_cols;
      go.tiles[t] = int4{e, first, n, 0};
    }
  }
}

// ---- f32 experts: one workgroup per (pick, 256 rows), k in order ---------------
__global__ void __launch_bounds__(256)
f32_id_kernel(const float *__restrict__ w, int NE, int64_t M, int64_t K,
              const float *__restrict__ x, int U, const int32_t *__restrict__ ids, int n_used,
              float *__restrict__ y) {
  const int64_t p = blockIdx.x;
  const int64_t m = (int64_t)blockIdx.y * 256 + threadIdx.x;
  const int e = ids[p];
  if (m >= M) return;
  if (e < 0 || e >= NE) {
    y[p * M + m] = 0.0f;
    return;
  }
  const float *xr = x + ((p / n_used) * U + (p % n_used) % U) * K;
  const float *wr = w + ((int64_t)e * M + m) * K;
  float acc = 0.0f;
  for (int64_t k = 0; k < K; k++) acc = fmaf(wr[k], xr[k], acc);
  y[p * M + m] = acc;
}

// ---- weighted sum of the picks ------------------------------------------------------
// out[t][m] = (y[t][0][m] w[t][0] + y[t][1][m] w[t][1] + ...) (+ residual),
// products and sums in pick order (g:mul then sum_picks).
__global__ void moe_sum_kernel(const float *__restrict__ y, const float *__restrict__ wts,
                               int64_t T, int n_used, int64_t M,
                               const float *__restrict__ residual, float *__restrict__ out) {
  const int64_t total = T * M;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / M, m = i % M;
    float s = 0.0f;
    for (int j = 0; j < n_used; j++) s += y[(t * n_used + j) * M + m] * wts[t * n_used + j];
    if (residual) s += residual[i];
    out[i] = s;
  }
}

// ---- host side --------------------------------------------------------------------
static size_t a256(size_t b) { return (b + 255) & ~size_t(255); }

// Column tile width for P picks over NE experts: 64 once an expert averages
// 128 picks, else 16. (A 512-token prefill pass of C5 gives an expert about
// 36 picks: in 64-column tiles those are half empty, and 16-column ones,
// two workgroups per CU, made C5's mixed phase 9% faster.)
int moe_tile_cols(int64_t P, int NE) { return P >= 128 * (int64_t)NE ? 64 : 16; }

// An upper bound of the tiles of a grouping: sum over experts of
// ceil(c_e / tc) <= (P + (tc - 1) * min(NE, P)) / tc, and <= P.
int moe_max_tiles(int64_t P, int NE, int tc) {
  const int64_t nz = P < NE ? P : NE;
  int64_t b = (P + (int64_t)(tc - 1) * nz) / tc;
  return (int)(b < P ? b : P);
}

int router_splits(int64_t K) { return (int)((K + ROUTER_KC - 1) / ROUTER_KC); }

// Router partials (router_splits(K) x T x NE floats) of rows x (T, K).
int router_logits(const float *w, int NE, int64_t K, const float *x, int64_t T, float *part,
                  hipStream_t st) {
  if (T == 0) return LGMLH_OK;
  if (K % 4) {
    set_error("moe router: K %lld is not a multiple of 4", (long long)K);
    return LGMLH_EINVAL;
  }
  if (T > 64 && NE >= 64) {  // prefill-sized: 64 x 64 tiles
    dim3 grid((unsigned)((NE + 63) / 64), (unsigned)router_splits(K),
              (unsigned)((T + ROUTER_TT - 1) / ROUTER_TT));
    hipLaunchKernelGGL(router_tile_kernel, grid, dim3(256), 0, st, w, NE, K, x, T, part);
    return hip_check(hipGetLastError(), "moe router");
  }
  const int tok = T <= 64 ? 16 : 64;
  dim3 grid((unsigned)((NE + 15) / 16), (unsigned)router_splits(K), (unsigned)((T + tok - 1) / tok));
  if (tok == 16)
    hipLaunchKernelGGL(router_part_kernel<16>, grid, dim3(256), 0, st, w, NE, K, x, T, part);
  else
    hipLaunchKernelGGL(router_part_kernel<64>, grid, dim3(256), 0, st, w, NE, K, x, T, part);
  return hip_check(hipGetLastError(), "moe router");
}

static int check_route(int64_t T, int NE, int n_used, int gating) {
  if (NE < 1 || NE > MOE_MAX_EXPERTS || n_used < 1 || n_used > MOE_MAX_USED || n_used > NE ||
      T < 0 || (gating != LGMLH_GATING_SOFTMAX && gating != LGMLH_GATING_SIGMOID)) {
    set_error("moe: bad routing arguments (experts %d, used %d, gating %d)", NE, n_used, gating);
    return LGMLH_EINVAL;
  }
  if (T * n_used > MOE_MAX_PICKS) {
    set_error("moe: %lld picks in one pass (at most %d)", (long long)(T * n_used), MOE_MAX_PICKS);
    return LGMLH_EINVAL;
  }
  return LGMLH_OK;
}

static void launch_group(const int32_t *ids, int P, int NE, const GroupOut &g, float *y,
                         int64_t M, hipStream_t st);

// Picks, weights and (with go) the grouping, from nz router partials.
int moe_route_dev(const float *part, int nz, int64_t T, int NE, int n_used, int gating,
                  int norm_topk, float scale, int32_t *ids, float *wts, const GroupOut *go,
                  hipStream_t st) {
  LGMLH_TRY(check_route(T, NE, n_used, gating));
  if (T == 0) return LGMLH_OK;
  GroupOut g = go ? *go : GroupOut{nullptr, nullptr, nullptr, 16, nullptr, nullptr};
  const int grp = go ? 1 : 0;
  // Up to 16 tokens: routing and grouping in one workgroup (one launch).
  // More: the routing spreads over workgroups of 16 tokens (one per CU
  // instead of 16 waves sharing one), then one workgroup groups the picks
  // (two launches; the same ids and order).
  if (T <= 16) {
    if (NE <= 128)
      hipLaunchKernelGGL(route_kernel<8>, dim3(1), dim3(ROUTE_THREADS), 0, st, part, nz, T, NE,
                         n_used, gating, norm_topk, scale, ids, wts, grp, g);
    else if (NE <= 256)
      hipLaunchKernelGGL(route_kernel<16>, dim3(1), dim3(ROUTE_THREADS), 0, st, part, nz, T, NE,
                         n_used, gating, norm_topk, scale, ids, wts, grp, g);
    else
      hipLaunchKernelGGL(route_kernel<32>, dim3(1), dim3(ROUTE_THREADS), 0, st, part, nz, T, NE,
                         n_used, gating, norm_topk, scale, ids, wts, grp, g);
    return hip_check(hipGetLastError(), "moe route");
  }
  const dim3 grid((unsigned)((T + 15) / 16));
  if (NE <= 128)
    hipLaunchKernelGGL(route_many_kernel<8>, grid, dim3(256), 0, st, part, nz, T, NE, n_used,
                       gating, norm_topk, scale, ids, wts);
  else if (NE <= 256)
    hipLaunchKernelGGL(route_many_kernel<16>, grid, dim3(256), 0, st, part, nz, T, NE, n_used,
                       gating, norm_topk, scale, ids, wts);
  else
    hipLaunchKernelGGL(route_many_kernel<32>, grid, dim3(256), 0, st, part, nz, T, NE, n_used,
                       gating, norm_topk, scale, ids, wts);
  if (grp) launch_group(ids, (int)(T * n_used), NE, g, nullptr, 0, st);
  return hip_check(hipGetLastError(), "moe route");
}

// Workspace of a grouping of P picks: sorted, tiles, count, and the
// many-workgroup grouping's ranks and chunk counts.
static int64_t group_chunks(int64_t P) { return (P + GROUP_CHUNK - 1) / GROUP_CHUNK; }

size_t group_bytes(int64_t P, int NE, int tc) {
  return a256((size_t)P * 4) + a256((size_t)moe_max_tiles(P, NE, tc) * 16) + 256 +
         a256((size_t)P * 4) + a256((size_t)group_chunks(P) * NE * 4);
}

GroupOut group_carve(void *ws, int64_t P, int NE, int tc) {
  char *b = (char *)ws;
  GroupOut g;
  g.sorted = (int32_t *)b;
  b += a256((size_t)P * 4);
  g.tiles = (int4 *)b;
  b += a256((size_t)moe_max_tiles(P, NE, tc) * 16);
  g.n_tiles = (int32_t *)b;
  b += 256;
  g.rank = (int32_t *)b;
  b += a256((size_t)P * 4);
  g.counts = (int32_t *)b;
  g.tile_cols = tc;
  return g;
}

// The grouping of P picks: one workgroup for a few (decode), chunked over
// many workgroups for a prefill pass's thousands (the same sorted order
// and tiles either way).
static void launch_group(const int32_t *ids, int P, int NE, const GroupOut &g, float *y, int64_t M,
                         hipStream_t st) {
  if (P <= GROUP_ONE) {
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(ROUTE_THREADS), 0, st, ids, P, NE, g, y, M);
    return;
  }
  const unsigned C = (unsigned)group_chunks(P);
  hipLaunchKernelGGL(group_count_kernel, dim3(C), dim3(GROUP_CHUNK), 0, st, ids, P, NE, g, y, M);
  hipLaunchKernelGGL(group_place_kernel, dim3(C), dim3(GROUP_CHUNK), 0, st, P, NE, g);
}

// Y (P, M) of the experts of the picks; x is f32 (T * U rows, f32
// experts) or split planes (quantized experts, xnpad rows).
int experts_dev(int type, const void *w, int NE, int64_t M, int64_t K, const float *xf,
                const f16 *xs, int64_t xnpad, int U, const int32_t *ids, int64_t T, int n_used,
                const GroupOut &go, float *y, hipStream_t st, int xform) {
  const int64_t P = T * n_used;
  if (P == 0) return LGMLH_OK;
  if (type == LGMLH_F32) {
    dim3 grid((unsigned)P, (unsigned)((M + 255) / 256));
    hipLaunchKernelGGL(f32_id_kernel, grid, dim3(256), 0, st, (const float *)w, NE, M, K, xf, U,
                       ids, n_used, y);
    return hip_check(hipGetLastError(), "mul_mat_id");
  }
  const int64_t eb = lgmlh_repacked_bytes(type, M, K);
  if (eb < 0) {
    set_error("mul_mat_id: type %d with K %lld", type, (long long)K);
    return LGMLH_EINVAL;
  }
  return mul_mat_grouped(type, w, eb, M, K, xs, xnpad, n_used, U, go.sorted, go.tiles, go.n_tiles,
                         moe_max_tiles(P, NE, go.tile_cols), go.tile_cols, y, st, xform);
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" int lgmlh_moe_route(const float *logits, int64_t n, int n_expert, int n_used,
                               int gating, int norm_topk, float scale, int32_t *ids,
                               float *weights, void *stream) {
  if (!logits || !ids || !weights) {
    set_error("moe_route: null argument");
    return LGMLH_EINVAL;
  }
  return moe_route_dev(logits, 1, n, n_expert, n_used, gating, norm_topk, scale, ids, weights,
                       nullptr, as_stream(stream));
}

extern "C" size_t lgmlh_mul_mat_id_workspace(int type, int64_t n_expert, int64_t M, int64_t K,
                                             int64_t T, int64_t U, int n_used) {
  (void)M;
  const int64_t P = T * n_used;
  const int tc = moe_tile_cols(P, (int)n_expert);
  size_t b = group_bytes(P, (int)n_expert, tc);
  if (type != LGMLH_F32) b += a256(split_bytes(T * U, K));
  return b;
}

static int mul_mat_id_entry(int act, int type, const void *w, int64_t n_expert, int64_t M,
                            int64_t K, const void *x, int xtype, int64_t U, const int32_t *ids,
                            int64_t T, int n_used, float *y, void *workspace, size_t ws_bytes,
                            void *stream) {
  if (!w || !x || !ids || !y || M <= 0 || K <= 0 || T < 0 || U < 1 || n_used < 1 ||
      n_used % U || n_expert < 1 || n_expert > MOE_MAX_EXPERTS) {
    set_error("mul_mat_id: bad arguments (experts %lld, M %lld, K %lld, U %lld, used %d)",
              (long long)n_expert, (long long)M, (long long)K, (long long)U, n_used);
    return LGMLH_EINVAL;
  }
  if (T * n_used > MOE_MAX_PICKS) {
    set_error("mul_mat_id: %lld picks (at most %d)", (long long)(T * n_used), MOE_MAX_PICKS);
    return LGMLH_EINVAL;
  }
  if (type == LGMLH_F32 ? xtype != LGMLH_F32 : (xtype != LGMLH_F32 && xtype != LGMLH_F16)) {
    set_error("mul_mat_id: bad x type %d for weights of type %d", xtype, type);
    return LGMLH_EINVAL;
  }
  if (type != LGMLH_F32 && K % QK_K) {
    set_error("mul_mat_id: K %lld is not a multiple of 256", (long long)K);
    return LGMLH_EINVAL;
  }
  const size_t need = lgmlh_mul_mat_id_workspace(type, n_expert, M, K, T, U, n_used);
  if (!workspace || ws_bytes < need) {
    set_error("mul_mat_id: workspace of %zu bytes, need %zu", ws_bytes, need);
    return LGMLH_ENOMEM;
  }
  const int64_t P = T * n_used;
  if (P == 0) return LGMLH_OK;
  hipStream_t st = as_stream(stream);
  const int NE = (int)n_expert;
  const int tc = moe_tile_cols(P, NE);
  GroupOut go = group_carve(workspace, P, NE, tc);
  launch_group(ids, (int)P, NE, go, y, M, st);
  LGMLH_TRY(hip_check(hipGetLastError(), "mul_mat_id group"));
  f16 *xs = nullptr;
  const int xform = xf_for(type, act);
  if (type != LGMLH_F32) {
    xs = (f16 *)((char *)workspace + group_bytes(P, NE, tc));
    LGMLH_TRY(split_x(x, xtype, T * U, K, xs, st, xform));
  }
  return experts_dev(type, w, NE, M, K, (const float *)x, xs, split_npad(T * U), (int)U, ids, T,
                     n_used, go, y, st, xform);
}

extern "C" int lgmlh_mul_mat_id(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
                                const void *x, int xtype, int64_t U, const int32_t *ids,
                                int64_t T, int n_used, float *y, void *workspace,
                                size_t ws_bytes, void *stream) {
  return mul_mat_id_entry(LGMLH_ACT_EXACT, type, w, n_expert, M, K, x, xtype, U, ids, T, n_used,
                          y, workspace, ws_bytes, stream);
}

extern "C" int lgmlh_mul_mat_id_ggml(int type, const void *w, int64_t n_expert, int64_t M,
                                     int64_t K, const void *x, int xtype, int64_t U,
                                     const int32_t *ids, int64_t T, int n_used, float *y,
                                     void *workspace, size_t ws_bytes, void *stream) {
  return mul_mat_id_entry(LGMLH_ACT_GGML, type, w, n_expert, M, K, x, xtype, U, ids, T, n_used,
                          y, workspace, ws_bytes, stream);
}

extern "C" int lgmlh_moe_sum(const float *y, const float *weights, int64_t T, int n_used,
                             int64_t M, const float *residual, float *out, void *stream) {
  if (!y || !weights || !out || T < 0 || n_used < 1 || M <= 0) {
    set_error("moe_sum: bad arguments");
    return LGMLH_EINVAL;
  }
  const int64_t total = T * M;
  if (total == 0) return LGMLH_OK;
  unsigned blocks = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
  hipLaunchKernelGGL(moe_sum_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), y, weights,
                     T, n_used, M, residual, out);
  return hip_check(hipGetLastError(), "moe_sum");
}
