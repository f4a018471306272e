// Ubatch packing and the attention work list (host side).
//
// Packs what fill_batch / batch_inputs (lua/lgml/transformer.lua:2433-2551)
// put in the graph leaves -- ids, positions n_past + j, the pool cell of
// every token (seq_cells, :1126-1133), the block tables, the logit rows
// off + n - 1 -- into one buffer for a single host-to-device copy, and adds
// the work list of the paged attention kernel: for every sequence, groups
// of 16 / G query tokens, each split into the fewest runs of at most
// blocks_per_split KV blocks (balanced lengths), plus one merge item per
// group with more than one split. A ring plan (sliding-window layers) maps
// positions into each sequence's ring of blocks and starts each group's
// runs at its window.
//
// A sequence with more than one query group in the pass (a prompt chunk)
// has its groups in shared sets of up to SHARED consecutive groups that
// take the same runs (those of the set's last token; blocks past a
// group's own last position are masked for it and change nothing): the
// shared attention kernel reads each K / V block once per set into LDS
// for all its groups. Items are ordered so that items [0, n_single) are
// groups on their own (decode tokens, ring plans) and every shared run is
// n consecutive items, listed in `shared` as {first item, n}. The items on
// their own are started longest run first (`order`): every item runs as
// one wave, all at once, so the waves that share a SIMD once the SIMDs
// are full are the shortest ones, and they end early.
#include <string.h>

#include <utility>

#include "common.h"

namespace lgmlh {
static int64_t align16(int64_t x) { return (x + 15) & ~int64_t(15); }
constexpr int SHARED = ATTN_SHARED;  // query groups per shared set
}  // namespace lgmlh

using namespace lgmlh;

// The plan of a pass; ring > 0 makes the sliding-window plan of
// lgmlh_plan_ring (block_tab = the ring tables, max_blocks = ring).
static int plan_impl(int n_seq, const int32_t *seq_n, const int32_t *seq_npast,
                     const int32_t *block_tab, int max_blocks, int64_t pool_blocks,
                     const int32_t *ids, int n_head, int n_head_kv, int blocks_per_split,
                     int window, int ring, void *buf, size_t buf_bytes, lgmlh_plan_info *info) {
  if (n_seq < 0 || !seq_n || !seq_npast || !block_tab || max_blocks <= 0 || !info ||
      n_head_kv <= 0 || n_head % n_head_kv || n_head / n_head_kv > 16 ||
      16 % (n_head / n_head_kv) || blocks_per_split < 0 || (ring > 0 && window < 1)) {
    set_error("plan: bad arguments");
    return LGMLH_EINVAL;
  }
  const int G = n_head / n_head_kv, T = 16 / G, B = KV_BLOCK;
  int64_t N = 0;
  for (int s = 0; s < n_seq; s++) {
    if (seq_n[s] < 0 || seq_npast[s] < 0) {
      set_error("plan: negative count");
      return LGMLH_EINVAL;
    }
    int64_t n_kv = (int64_t)seq_npast[s] + seq_n[s];
    int64_t nb = (n_kv + B - 1) / B;
    if (nb > 0xffff || (!ring && nb > max_blocks)) {
      set_error("plan: sequence %d needs %lld blocks (table has %d)", s, (long long)nb,
                max_blocks);
      return LGMLH_ERANGE;
    }
    if (ring) {
      // every query's window must still be in the ring after the pass writes
      if ((int64_t)ring * B < (int64_t)window - 1 + seq_n[s]) {
        set_error("plan: %d tokens in one pass; the ring of %d cells takes %lld", seq_n[s],
                  ring * B, (long long)ring * B - window + 1);
        return LGMLH_ERANGE;
      }
      nb = nb < ring ? nb : ring;  // the ring entries in use
    }
    for (int64_t i = 0; i < nb; i++) {
      int32_t b = block_tab[(int64_t)s * max_blocks + i];
      if (b < 0 || b >= pool_blocks) {
        set_error("plan: position %lld of sequence %d is in no block (block %d, pool of %lld)",
                  (long long)(i * B), s, b, (long long)pool_blocks);
        return LGMLH_ERANGE;
      }
    }
    N += seq_n[s];
  }
  if (N > INT32_MAX / 2) {
    set_error("plan: too many tokens");
    return LGMLH_EINVAL;
  }
  // A fixed default: the split points of a sequence must not depend on the
  // rest of the batch (a sequence gives the same bits alone or batched).
  const int bps = blocks_per_split ? blocks_per_split : 16;
  // The work list is walked twice with no allocation: once to count the
  // items, merges and shared runs (the buffer layout), once to write them
  // into buf. emit(item index, item[4], merge[4] or NULL, merge index,
  // shared[2] or NULL, shared index) gets each item; the first item of a
  // group with more than one run passes the group's merge (its runs are
  // `stride` items apart: the set's size), the first item of a shared run
  // passes the run's entry.
  struct Counts {
    int64_t items = 0, merges = 0, single = 0, shared = 0;
  };
  auto walk = [&](auto &&emit) {
    Counts n;
    for (int phase = 0; phase < 2; phase++) {  // 0: groups on their own, 1: shared sets
      for (int s = 0, off = 0; s < n_seq; off += seq_n[s], s++) {
        const int ng = (seq_n[s] + T - 1) / T;  // query groups of s
        const int W = ring || ng < 2 ? 1 : SHARED;
        if ((W > 1) != (phase == 1)) continue;
        for (int sg = 0; sg < ng; sg += W) {
          const int nm = ng - sg < W ? ng - sg : W;  // groups in the set
          const int g0 = sg * T, ge = (sg + nm) * T < seq_n[s] ? (sg + nm) * T : seq_n[s];
          // logical blocks [b0, nbg): from the window of the set's first
          // token (ring plans) or from 0, to the set's last position
          const int64_t pf = (int64_t)seq_npast[s] + g0, pl = (int64_t)seq_npast[s] + ge - 1;
          const int b0 = ring ? (int)((pf - window + 1 > 0 ? pf - window + 1 : 0) / B) : 0;
          const int nbg = (int)(pl / B + 1);
          // the fewest runs of at most bps blocks, of lengths that differ
          // by at most one (the longest run bounds the kernel's time)
          const int len = nbg - b0, ns = (len + bps - 1) / bps;
          const int64_t first = n.items;
          for (int j = 0; j < ns; j++) {
            const uint32_t lo = (uint32_t)(b0 + (int)((int64_t)j * len / ns));
            const uint32_t hi = (uint32_t)(b0 + (int)((int64_t)(j + 1) * len / ns));
            const int32_t sh[2] = {(int32_t)n.items, nm};
            for (int m = 0; m < nm; m++) {
              const int t0 = g0 + m * T, te = t0 + T < seq_n[s] ? t0 + T : seq_n[s];
              const uint32_t mg = ns > 1 ? (uint32_t)(n.merges + m) + 1 : 0;
              const int32_t item[4] = {s, off + t0, (int32_t)((uint32_t)(te - t0) | (mg << 5)),
                                       (int32_t)(lo | (hi << 16))};
              const int32_t mrg[4] = {(int32_t)(first + m), ns, off + t0,
                                      (int32_t)((uint32_t)(te - t0) | ((uint32_t)nm << 8))};
              emit(n.items, item, j == 0 && ns > 1 ? mrg : nullptr, n.merges + m,
                   W > 1 && m == 0 ? sh : nullptr, n.shared);
              n.items++;
            }
            if (W > 1) n.shared++;
          }
          if (ns > 1) n.merges += nm;
        }
      }
      if (phase == 0) n.single = n.items;
    }
    return n;
  };
  const Counts counts = walk([](int64_t, const int32_t *, const int32_t *, int64_t,
                                const int32_t *, int64_t) {});
  if (counts.items > INT32_MAX / 8 || counts.merges > INT32_MAX / 8) {
    set_error("plan: too many work items");
    return LGMLH_EINVAL;
  }
  lgmlh_plan_info in;
  memset(&in, 0, sizeof in);
  in.n_seq = n_seq;
  in.n_tokens = (int32_t)N;
  in.max_blocks = max_blocks;
  in.block = B;
  in.n_items = (int32_t)counts.items;
  in.n_merge = (int32_t)counts.merges;
  in.n_single = (int32_t)counts.single;
  in.n_shared = (int32_t)counts.shared;
  in.rows = 16;
  in.n_head_kv = n_head_kv;
  in.window = ring ? window : 0;
  in.ring = ring;
  int64_t o = 0;
  in.off_ids = o;          o = align16(o + 4 * N);
  in.off_pos = o;          o = align16(o + 4 * N);
  in.off_cells = o;        o = align16(o + 8 * N);
  in.off_seq_off = o;      o = align16(o + 4 * ((int64_t)n_seq + 1));
  in.off_npast = o;        o = align16(o + 4 * (int64_t)n_seq);
  in.off_block_tab = o;    o = align16(o + 4 * (int64_t)n_seq * max_blocks);
  in.off_logit_rows = o;   o = align16(o + 4 * (int64_t)n_seq);
  in.off_items = o;        o = align16(o + 16 * (int64_t)in.n_items);
  in.off_merge = o;        o = align16(o + 16 * (int64_t)in.n_merge);
  in.off_shared = o;       o = align16(o + 8 * (int64_t)in.n_shared);
  in.off_order = o;        o = align16(o + 4 * (int64_t)in.n_single);
  in.bytes = o;
  *info = in;
  if (!buf) return LGMLH_OK;
  if (buf_bytes < (size_t)in.bytes) {
    set_error("plan: buffer of %zu bytes, need %lld", buf_bytes, (long long)in.bytes);
    return LGMLH_ENOMEM;
  }
  char *b = (char *)buf;
  memset(b, 0, (size_t)in.bytes);
  int32_t *pid = (int32_t *)(b + in.off_ids), *ppos = (int32_t *)(b + in.off_pos);
  int64_t *pcell = (int64_t *)(b + in.off_cells);
  int32_t *psoff = (int32_t *)(b + in.off_seq_off), *pnp = (int32_t *)(b + in.off_npast);
  int32_t *plr = (int32_t *)(b + in.off_logit_rows);
  int64_t t = 0;
  for (int s = 0; s < n_seq; s++) {
    psoff[s] = (int32_t)t;
    pnp[s] = seq_npast[s];
    for (int j = 0; j < seq_n[s]; j++, t++) {
      int p = seq_npast[s] + j;
      if (ids) pid[t] = ids[t];
      ppos[t] = p;
      const int bi = ring ? (p / B) % ring : p / B;
      pcell[t] = (int64_t)block_tab[(int64_t)s * max_blocks + bi] * B + p % B;
    }
    plr[s] = (int32_t)t - 1;
  }
  psoff[n_seq] = (int32_t)t;
  memcpy(b + in.off_block_tab, block_tab, 4 * (size_t)n_seq * max_blocks);
  int32_t *pit = (int32_t *)(b + in.off_items), *pmg = (int32_t *)(b + in.off_merge);
  int32_t *psh = (int32_t *)(b + in.off_shared);
  walk([&](int64_t i, const int32_t *item, const int32_t *mrg, int64_t m, const int32_t *sh,
           int64_t k) {
    memcpy(pit + 4 * i, item, 16);
    if (mrg) memcpy(pmg + 4 * m, mrg, 16);
    if (sh) memcpy(psh + 2 * k, sh, 8);
  });
  // order: the items on their own by run length, longest first, then by
  // index (a counting sort; runs longer than 256 blocks share a key)
  int32_t *pord = (int32_t *)(b + in.off_order);
  int64_t start[258];
  memset(start, 0, sizeof start);
  auto key = [&](int64_t i) {
    const uint32_t r = (uint32_t)pit[4 * i + 3];
    const int len = (int)(r >> 16) - (int)(r & 0xffff);
    return 256 - (len < 0 ? 0 : len > 256 ? 256 : len);  // ascending key, descending length
  };
  for (int64_t i = 0; i < in.n_single; i++) start[key(i) + 1]++;
  for (int k = 0; k < 257; k++) start[k + 1] += start[k];
  for (int64_t i = 0; i < in.n_single; i++) pord[start[key(i)]++] = (int32_t)i;
  return LGMLH_OK;
}

extern "C" int lgmlh_plan(int n_seq, const int32_t *seq_n, const int32_t *seq_npast,
                          const int32_t *block_tab, int max_blocks, int64_t pool_blocks,
                          const int32_t *ids, int n_head, int n_head_kv, int blocks_per_split,
                          void *buf, size_t buf_bytes, lgmlh_plan_info *info) {
  return plan_impl(n_seq, seq_n, seq_npast, block_tab, max_blocks, pool_blocks, ids, n_head,
                   n_head_kv, blocks_per_split, 0, 0, buf, buf_bytes, info);
}

extern "C" int lgmlh_plan_ring(int n_seq, const int32_t *seq_n, const int32_t *seq_npast,
                               const int32_t *ring_tab, int ring_blocks, int64_t pool_blocks,
                               int window, const int32_t *ids, int n_head, int n_head_kv,
                               int blocks_per_split, void *buf, size_t buf_bytes,
                               lgmlh_plan_info *info) {
  if (ring_blocks < 1 || window < 1) {
    set_error("plan_ring: ring of %d blocks, window %d", ring_blocks, window);
    return LGMLH_EINVAL;
  }
  return plan_impl(n_seq, seq_n, seq_npast, ring_tab, ring_blocks, pool_blocks, ids, n_head,
                   n_head_kv, blocks_per_split, window, ring_blocks, buf, buf_bytes, info);
}

extern "C" int lgmlh_plan_bind(const lgmlh_plan_info *info, const void *dev, lgmlh_ubatch *ub) {
  if (!info || !dev || !ub) {
    set_error("plan_bind: bad arguments");
    return LGMLH_EINVAL;
  }
  const char *b = (const char *)dev;
  ub->n_seq = info->n_seq;
  ub->n_tokens = info->n_tokens;
  ub->max_blocks = info->max_blocks;
  ub->block = info->block;
  ub->n_items = info->n_items;
  ub->n_merge = info->n_merge;
  ub->rows = info->rows;
  ub->n_head_kv = info->n_head_kv;
  ub->ids = (const int32_t *)(b + info->off_ids);
  ub->pos = (const int32_t *)(b + info->off_pos);
  ub->cells = (const int64_t *)(b + info->off_cells);
  ub->seq_off = (const int32_t *)(b + info->off_seq_off);
  ub->seq_npast = (const int32_t *)(b + info->off_npast);
  ub->block_tab = (const int32_t *)(b + info->off_block_tab);
  ub->logit_rows = (const int32_t *)(b + info->off_logit_rows);
  ub->items = (const int32_t *)(b + info->off_items);
  ub->merge = (const int32_t *)(b + info->off_merge);
  ub->n_single = info->n_single;
  ub->n_shared = info->n_shared;
  ub->shared = (const int32_t *)(b + info->off_shared);
  ub->order = (const int32_t *)(b + info->off_order);
  ub->window = info->window;
  ub->ring = info->ring;
  return LGMLH_OK;
}
