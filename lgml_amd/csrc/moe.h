// Internal interface of the routed-expert kernels (moe.hip) for the
// forward pass.
#pragma once
#include "common.h"

namespace lgmlh {

// A grouping of the picks of a pass by expert (device buffers).
struct GroupOut {
  int32_t *sorted;    // [P] picks, expert-major, pick order within an expert
  int4 *tiles;        // {expert, first, count, 0} per column tile
  int32_t *n_tiles;   // [1] tiles in use
  int tile_cols;      // 16 or 64
  int32_t *rank;      // [P] scratch of the many-workgroup grouping
  int32_t *counts;    // [chunks][NE] scratch of the many-workgroup grouping
};

int moe_tile_cols(int64_t P, int NE);
int moe_max_tiles(int64_t P, int NE, int tc);
int router_splits(int64_t K);
int router_logits(const float *w, int NE, int64_t K, const float *x, int64_t T, float *part,
                  hipStream_t st);
int moe_route_dev(const float *part, int nz, int64_t T, int NE, int n_used, int gating,
                  int norm_topk, float scale, int32_t *ids, float *wts, const GroupOut *go,
                  hipStream_t st);
size_t group_bytes(int64_t P, int NE, int tc);
GroupOut group_carve(void *ws, int64_t P, int NE, int tc);
int experts_dev(int type, const void *w, int NE, int64_t M, int64_t K, const float *xf,
                const f16 *xs, int64_t xnpad, int U, const int32_t *ids, int64_t T, int n_used,
                const GroupOut &go, float *y, hipStream_t st, int xform);

}  // namespace lgmlh
