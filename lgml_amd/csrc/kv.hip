// KV pool scatter / gather / block copy (gfx950).
//
// Pool layout, per layer (see include/lgml_hip.h):
//   K: [block][kv_head][cell % 64][D]   V: [block][kv_head][D][cell % 64]
// so one (block, head) tile is 64 * D * 2 contiguous bytes in both, and the
// attention kernels read K rows and V columns (cells contiguous) straight
// into MFMA operands.
#include "common.h"

namespace lgmlh {

__device__ __forceinline__ int64_t k_index(int64_t cell, int h, int d, int Hkv, int D) {
  int64_t b = cell / KV_BLOCK, o = cell % KV_BLOCK;
  return ((b * Hkv + h) * KV_BLOCK + o) * D + d;
}
__device__ __forceinline__ int64_t v_index(int64_t cell, int h, int d, int Hkv, int D) {
  int64_t b = cell / KV_BLOCK, o = cell % KV_BLOCK;
  return ((b * Hkv + h) * (int64_t)D + d) * KV_BLOCK + o;
}

// One workgroup per token; threads over Hkv * D.
__global__ void kv_store_kernel(uint16_t *__restrict__ kp, uint16_t *__restrict__ vp,
                                const float *__restrict__ ks, const float *__restrict__ vs,
                                int64_t src_stride, const int64_t *__restrict__ cells, int Hkv,
                                int D) {
  int64_t j = blockIdx.x;
  int64_t cell = cells[j];
  int row = Hkv * D;
  for (int e = threadIdx.x; e < row; e += blockDim.x) {
    int h = e / D, d = e % D;
    kp[k_index(cell, h, d, Hkv, D)] = f2h(ks[j * src_stride + e]);
    vp[v_index(cell, h, d, Hkv, D)] = f2h(vs[j * src_stride + e]);
  }
}

__global__ void kv_gather_kernel(const uint16_t *__restrict__ pool, int which,
                                 const int64_t *__restrict__ cells, int Hkv, int D,
                                 uint16_t *__restrict__ out) {
  int64_t j = blockIdx.x;
  int64_t cell = cells[j];
  int row = Hkv * D;
  for (int e = threadIdx.x; e < row; e += blockDim.x) {
    int h = e / D, d = e % D;
    out[j * row + e] = pool[which ? v_index(cell, h, d, Hkv, D) : k_index(cell, h, d, Hkv, D)];
  }
}

// Copy the first n cells of block src to block dst. K tiles copy rows
// [0, n) of each head; V tiles copy columns [0, n) of each (head, d) row.
__global__ void kv_copy_block_kernel(uint16_t *__restrict__ kp, uint16_t *__restrict__ vp,
                                     int32_t src, int32_t dst, int n, int Hkv, int D) {
  int64_t tile = (int64_t)KV_BLOCK * D;
  int64_t total = (int64_t)Hkv * tile;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t in_tile = e % tile;
    int k_cell = (int)(in_tile / D);          // K: row-major cells
    int v_cell = (int)(in_tile % KV_BLOCK);   // V: cells innermost
    if (k_cell < n) kp[(int64_t)dst * total + e] = kp[(int64_t)src * total + e];
    if (v_cell < n) vp[(int64_t)dst * total + e] = vp[(int64_t)src * total + e];
  }
}

__global__ void set_rows_f16_kernel(uint16_t *__restrict__ dst, int64_t row,
                                    const float *__restrict__ src,
                                    const int64_t *__restrict__ ids) {
  int64_t j = blockIdx.x;
  int64_t r = ids[j];
  for (int64_t e = threadIdx.x; e < row; e += blockDim.x) dst[r * row + e] = f2h(src[j * row + e]);
}

static int check_cells(const int64_t *h, int64_t n, int64_t limit, const char *what) {
  if (!h) {
    set_error("%s: the host copy of the ids is required for the range check", what);
    return LGMLH_EINVAL;
  }
  for (int64_t j = 0; j < n; j++)
    if (h[j] < 0 || h[j] >= limit) {
      set_error("%s: id %lld out of range [0, %lld)", what, (long long)h[j], (long long)limit);
      return LGMLH_ERANGE;
    }
  return LGMLH_OK;
}

int kv_store_strided(void *kpool, void *vpool, int64_t n_cells, int Hkv, int D, const float *k,
                     const float *v, int64_t src_stride, const int64_t *cells, int64_t n,
                     hipStream_t st) {
  if (n == 0) return LGMLH_OK;
  int threads = Hkv * D >= 256 ? 256 : 64;
  hipLaunchKernelGGL(kv_store_kernel, dim3((unsigned)n), dim3(threads), 0, st,
                     (uint16_t *)kpool, (uint16_t *)vpool, k, v, src_stride, cells, Hkv, D);
  return hip_check(hipGetLastError(), "kv_store");
}

// One block of every pool tensor to (out) or from host memory: pools[p]
// is a tensor of the block layout; block b's bytes (the same count in each
// tensor, K or V) go to host + p * block_bytes. 16 bytes per thread.
__global__ void kv_block_host_kernel(void *const *__restrict__ pools, int64_t block_bytes,
                                     int32_t b, uint8_t *__restrict__ host, int out) {
  const int p = blockIdx.y;
  uint8_t *dev = (uint8_t *)pools[p] + (int64_t)b * block_bytes;
  uint8_t *hst = host + (int64_t)p * block_bytes;
  for (int64_t o = 16 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x); o < block_bytes;
       o += 16 * (int64_t)gridDim.x * blockDim.x) {
    if (out)
      *(u32x4 *)(hst + o) = *(const u32x4 *)(dev + o);
    else
      *(u32x4 *)(dev + o) = *(const u32x4 *)(hst + o);
  }
}

__global__ void zero_kernel(u32x4 *__restrict__ p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0, 0, 0, 0};
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" int64_t lgmlh_kv_block_bytes(int n_head_kv, int head_dim) {
  if (n_head_kv <= 0 || head_dim <= 0) return -1;
  return (int64_t)KV_BLOCK * n_head_kv * head_dim * 2;
}

extern "C" int lgmlh_kv_block_host(void *const *pools, int n_pools, int64_t n_cells,
                                   int n_head_kv, int head_dim, int32_t block, void *host, int out,
                                   void *stream) {
  const int64_t bb = lgmlh_kv_block_bytes(n_head_kv, head_dim);
  if (!pools || !host || n_pools <= 0 || n_pools > 65535 || bb <= 0 || bb % 16 ||
      n_cells % KV_BLOCK || block < 0 || block >= n_cells / KV_BLOCK || ((uintptr_t)host & 15)) {
    set_error("kv_block_host: bad arguments");
    return LGMLH_EINVAL;
  }
  const int64_t chunks = bb / 16;
  const unsigned gx = (unsigned)((chunks + 255) / 256 < 64 ? (chunks + 255) / 256 : 64);
  hipLaunchKernelGGL(kv_block_host_kernel, dim3(gx, (unsigned)n_pools), dim3(256), 0,
                     as_stream(stream), pools, bb, block, (uint8_t *)host, out);
  return hip_check(hipGetLastError(), "kv_block_host");
}

extern "C" int lgmlh_kv_grow(const void *old_pool, int64_t old_cells, void *new_pool,
                             int64_t new_cells, int n_head_kv, int head_dim, void *stream) {
  const int64_t ob = lgmlh_kv_layer_bytes(old_cells, n_head_kv, head_dim);
  const int64_t nb = lgmlh_kv_layer_bytes(new_cells, n_head_kv, head_dim);
  if (!old_pool || !new_pool || ob <= 0 || nb < ob || old_pool == new_pool) {
    set_error("kv_grow: bad arguments (cells %lld -> %lld)", (long long)old_cells,
              (long long)new_cells);
    return LGMLH_EINVAL;
  }
  hipStream_t st = as_stream(stream);
  LGMLH_TRY(hip_check(hipMemcpyAsync(new_pool, old_pool, (size_t)ob, hipMemcpyDeviceToDevice, st),
                      "kv_grow"));
  const int64_t n16 = (nb - ob) / 16;  // the new cells start zeroed (a fill, not a memset)
  if (n16 > 0) {
    const unsigned g = (unsigned)((n16 + 255) / 256 < 4096 ? (n16 + 255) / 256 : 4096);
    hipLaunchKernelGGL(zero_kernel, dim3(g), dim3(256), 0, st, (u32x4 *)((uint8_t *)new_pool + ob),
                       n16);
  }
  return hip_check(hipGetLastError(), "kv_grow");
}

extern "C" int64_t lgmlh_kv_layer_bytes(int64_t n_cells, int n_head_kv, int head_dim) {
  if (n_cells <= 0 || n_cells % KV_BLOCK || n_head_kv <= 0 || head_dim <= 0) return -1;
  return n_cells * n_head_kv * head_dim * 2;
}

extern "C" int lgmlh_kv_store(void *kpool, void *vpool, int64_t n_cells, int n_head_kv,
                              int head_dim, const float *k_src, const float *v_src,
                              const int64_t *cells, const int64_t *h_cells, int64_t n,
                              void *stream) {
  if (!kpool || !vpool || !k_src || !v_src || !cells || n < 0 || n_cells % KV_BLOCK ||
      n_head_kv <= 0 || head_dim <= 0) {
    set_error("kv_store: bad arguments");
    return LGMLH_EINVAL;
  }
  LGMLH_TRY(check_cells(h_cells, n, n_cells, "kv_store"));
  return kv_store_strided(kpool, vpool, n_cells, n_head_kv, head_dim, k_src, v_src,
                          (int64_t)n_head_kv * head_dim, cells, n, as_stream(stream));
}

extern "C" int lgmlh_kv_gather(const void *pool, int which, int64_t n_cells, int n_head_kv,
                               int head_dim, const int64_t *cells, int64_t n, uint16_t *out,
                               void *stream) {
  if (!pool || !cells || !out || n < 0 || (which != 0 && which != 1) || n_cells % KV_BLOCK) {
    set_error("kv_gather: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream),
                     (const uint16_t *)pool, which, cells, n_head_kv, head_dim, out);
  return hip_check(hipGetLastError(), "kv_gather");
}

extern "C" int lgmlh_kv_copy_block(void *kpool, void *vpool, int64_t n_cells, int n_head_kv,
                                   int head_dim, int32_t src, int32_t dst, int n, void *stream) {
  int64_t nb = n_cells / KV_BLOCK;
  if (!kpool || !vpool || n_cells % KV_BLOCK || src < 0 || dst < 0 || src >= nb || dst >= nb ||
      n < 0 || n > KV_BLOCK) {
    set_error("kv_copy_block: bad arguments");
    return LGMLH_EINVAL;
  }
  if (n == 0 || src == dst) return LGMLH_OK;
  hipLaunchKernelGGL(kv_copy_block_kernel, dim3(64), dim3(256), 0, as_stream(stream),
                     (uint16_t *)kpool, (uint16_t *)vpool, src, dst, n, n_head_kv, head_dim);
  return hip_check(hipGetLastError(), "kv_copy_block");
}

extern "C" int lgmlh_set_rows_f16(uint16_t *dst, int64_t dst_rows, int64_t row,
                                  const float *src, const int64_t *ids, const int64_t *h_ids,
                                  int64_t n, void *stream) {
  if (!dst || !src || !ids || row <= 0 || n < 0) {
    set_error("set_rows: bad arguments");
    return LGMLH_EINVAL;
  }
  LGMLH_TRY(check_cells(h_ids, n, dst_rows, "set_rows"));
  if (n == 0) return LGMLH_OK;
  hipLaunchKernelGGL(set_rows_f16_kernel, dim3((unsigned)n), dim3(256), 0, as_stream(stream),
                     dst, row, src, ids);
  return hip_check(hipGetLastError(), "set_rows");
}
