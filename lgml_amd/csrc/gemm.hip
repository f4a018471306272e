// Weight products Y (N, M) = X (N, K) W^T for f32 / Q4_K / Q6_K / Q8_0 W
// (graph:mul_mat, src/lgml.c:1811-1839) on gfx950.
//
// Quantized W is repacked once into row tiles of 16 rows. For row tile rt
// and K step sb (256 values) one chunk holds the tile's block headers and
// then, for each of the 64 lanes of a wavefront (lane = r + 16 c: row r,
// 8-value k chunk c of every 32-value group), exactly the bytes that lane
// dequantizes into its MFMA A fragment. A wave streams its chunks with
// 16-byte loads, dequantizes in registers (closed forms of quant.h, one
// rounding to f16), and multiplies with 16x16x32 f16 MFMAs against X
// staged in LDS as f16. Every output element is the same f32 sum over K in
// the same order for any N, so a row gives the same bits alone or batched.
// K is split over workgroups when M alone gives too few; the splits are
// added in a fixed order by the last workgroup of each tile.
#include "common.h"
#include "quant.h"

namespace lgmlh {

constexpr int GEMM_WAVES = 8;      // waves per workgroup
constexpr int GEMM_THREADS = GEMM_WAVES * 64;
constexpr int RT_PER_WAVE = 2;     // 16-row tiles per wave
constexpr int WG_ROWS = GEMM_WAVES * RT_PER_WAVE * 16;  // 256
constexpr int WG_COLS = 64;        // N columns per workgroup (4 tiles)
constexpr int X_STRIDE = 264;      // f16 per LDS row of X (256 + pad)

// Bytes of one repacked chunk (16 rows x 256 values).
__host__ __device__ constexpr int chunk_bytes(int type) {
  return type == LGMLH_Q4_K ? 16 * Q4K_BYTES
       : type == LGMLH_Q6_K ? 16 * Q6K_BYTES
       : type == LGMLH_Q8_0 ? 16 * 8 * Q8_0_BYTES : 0;
}
// Bytes of the header part of a chunk.
__host__ __device__ constexpr int chunk_hdr(int type) {
  return type == LGMLH_Q4_K ? 256 : type == LGMLH_Q6_K ? 288 : type == LGMLH_Q8_0 ? 256 : 0;
}
// Bytes of one lane's data in a chunk.
__host__ __device__ constexpr int lane_bytes(int type) {
  return type == LGMLH_Q4_K ? 32 : type == LGMLH_Q6_K ? 48 : type == LGMLH_Q8_0 ? 64 : 0;
}

// ---- repack: ggml row blocks -> row-tile chunks ------------------------------
// One thread per (row tile, sb, lane): copies the lane's bytes and, for
// c == 0, the row's header.
template <int TYPE>
__global__ void repack_kernel(const uint8_t *__restrict__ src, int64_t M, int64_t NSB,
                              uint8_t *__restrict__ dst) {
  int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int64_t MT = (M + 15) / 16;
  if (gid >= MT * NSB * 64) return;
  int lane = (int)(gid % 64);
  int64_t sb = (gid / 64) % NSB, rt = gid / 64 / NSB;
  int r = lane % 16, c = lane / 16;
  int64_t m = rt * 16 + r;
  uint8_t *ch = dst + (rt * NSB + sb) * chunk_bytes(TYPE);
  uint8_t *ld = ch + chunk_hdr(TYPE) + lane * lane_bytes(TYPE);
  if (m >= M) {  // padding rows: zero bytes dequantize to 0
    for (int i = 0; i < lane_bytes(TYPE); i++) ld[i] = 0;
    if (c == 0)
      for (int i = 0; i < chunk_hdr(TYPE) / 16; i++) ch[r * (chunk_hdr(TYPE) / 16) + i] = 0;
    return;
  }
  if (TYPE == LGMLH_Q4_K) {
    const uint8_t *b = src + (m * NSB + sb) * Q4K_BYTES;
    if (c == 0)
      for (int i = 0; i < 16; i++) ch[r * 16 + i] = b[i];
    for (int j = 0; j < 4; j++)
      for (int e = 0; e < 8; e++) ld[8 * j + e] = b[16 + 32 * j + 8 * c + e];
  } else if (TYPE == LGMLH_Q6_K) {
    const uint8_t *b = src + (m * NSB + sb) * Q6K_BYTES;
    if (c == 0) {
      ch[r * 18 + 0] = b[208];
      ch[r * 18 + 1] = b[209];
      for (int i = 0; i < 16; i++) ch[r * 18 + 2 + i] = b[192 + i];
    }
    // ql pieces (h, tb): ql[64h + 32tb + 8c .. +7]; then qh pieces h: qh[32h + 8c .. +7]
    for (int h = 0; h < 2; h++)
      for (int tb = 0; tb < 2; tb++)
        for (int e = 0; e < 8; e++) ld[8 * (2 * h + tb) + e] = b[64 * h + 32 * tb + 8 * c + e];
    for (int h = 0; h < 2; h++)
      for (int e = 0; e < 8; e++) ld[32 + 8 * h + e] = b[128 + 32 * h + 8 * c + e];
  } else {  // Q8_0: 8 blocks of 32 per 256 values
    const uint8_t *b = src + (m * NSB * 8 + sb * 8) * Q8_0_BYTES;
    if (c == 0)
      for (int g = 0; g < 8; g++) {
        ch[r * 16 + 2 * g] = b[g * Q8_0_BYTES];
        ch[r * 16 + 2 * g + 1] = b[g * Q8_0_BYTES + 1];
      }
    for (int g = 0; g < 8; g++)
      for (int e = 0; e < 8; e++) ld[8 * g + e] = b[g * Q8_0_BYTES + 2 + 8 * c + e];
  }
}

// ---- per-lane weight data of one chunk --------------------------------------
// A fragments hold exact small integers in f16 -- the group scale times the
// quant (Q4_K: sc * q <= 945; Q6_K: sc * q split as 16 * s_hi * q + s_lo * q,
// both exact; Q8_0: q) -- so the MFMA sees the weights without rounding; the
// f16 super-block scales d (and dmin) are applied in f32 when a chunk is
// flushed into the accumulator.
template <int TYPE>
struct WFrag;

__device__ __forceinline__ f16x2 u16pair_to_f16(uint32_t lo16_hi16) {
  // two small non-negative integers (< 1024) in the 16-bit halves -> exact f16
  uint32_t m = lo16_hi16 | 0x64006400u;  // 1024 + v
  return __builtin_bit_cast(f16x2, m) - f16x2{(f16)1024.0f, (f16)1024.0f};
}

template <>
struct WFrag<LGMLH_Q4_K> {
  u32x4 hdr;       // d | dmin << 16, scales[0..3], scales[4..7], scales[8..11]
  u32x4 qs[2];     // 4 pieces of 8 bytes
  __device__ void load(const uint8_t *ch, int lane) {
    hdr = *(const u32x4 *)(ch + (lane & 15) * 16);
    const u32x4 *p = (const u32x4 *)(ch + 256 + lane * 32);
    qs[0] = p[0];
    qs[1] = p[1];
  }
  __device__ __forceinline__ uint32_t sbyte(int i) const {
    return (hdr[1 + (i >> 2)] >> (8 * (i & 3))) & 0xffu;
  }
  __device__ __forceinline__ void scale_min(int g, int &sc, int &m) const {
    if (g < 4) {
      sc = sbyte(g) & 63;
      m = sbyte(g + 4) & 63;
    } else {
      sc = (sbyte(g + 4) & 0xF) | ((sbyte(g - 4) >> 6) << 4);
      m = (sbyte(g + 4) >> 4) | ((sbyte(g) >> 6) << 4);
    }
  }
  // sc_g * q for k = 32g + 8c + e, e = 0..7.
  __device__ __forceinline__ f16x8 frag(int g) const {
    int sc, m;
    scale_min(g, sc, m);
    int j = g >> 1;
    uint32_t lo = qs[j >> 1][2 * (j & 1)], hi = qs[j >> 1][2 * (j & 1) + 1];
    int sh = (g & 1) * 4;
    uint32_t a = (lo >> sh) & 0x0F0F0F0Fu, b = (hi >> sh) & 0x0F0F0F0Fu;
    f16x2 s2 = f16x2{(f16)(float)sc, (f16)(float)sc};
    f16x2 p0 = u16pair_to_f16((a & 0xffu) | ((a & 0xff00u) << 8)) * s2;
    f16x2 p1 = u16pair_to_f16(((a >> 16) & 0xffu) | ((a >> 8) & 0xff0000u)) * s2;
    f16x2 p2 = u16pair_to_f16((b & 0xffu) | ((b & 0xff00u) << 8)) * s2;
    f16x2 p3 = u16pair_to_f16(((b >> 16) & 0xffu) | ((b >> 8) & 0xff0000u)) * s2;
    return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  }
  // The 16x16x16 A fragment of the mins: row lane%16, k = groups 4c..4c+3
  // (zero for c >= 2).
  __device__ __forceinline__ f16x4 mins(int c) const {
    f16x4 r = f16x4{0, 0, 0, 0};
    if (c < 2) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int sc, m;
        scale_min(4 * c + i, sc, m);
        r[i] = (f16)(float)m;
      }
    }
    return r;
  }
};

template <>
struct WFrag<LGMLH_Q6_K> {
  uint32_t hdr[5];  // d (16 bits) + 16 int8 scales, 18 bytes from row r's header
  u32x4 ql[2];      // pieces (h, tb) of 8 bytes: index 2h + tb
  u32x4 qh;         // pieces h of 8 bytes
  __device__ void load(const uint8_t *ch, int lane) {
    const uint16_t *h = (const uint16_t *)(ch + (lane & 15) * 18);
#pragma unroll
    for (int i = 0; i < 4; i++) hdr[i] = (uint32_t)h[2 * i] | ((uint32_t)h[2 * i + 1] << 16);
    hdr[4] = h[8];
    const u32x4 *p = (const u32x4 *)(ch + 288 + lane * 48);
    ql[0] = p[0];
    ql[1] = p[1];
    qh = p[2];
  }
  // Two fragments whose sum is sc * q (scale index (32g + 8c) / 16):
  // a1 = 16 * (sc >> 4) * q, a2 = (sc & 15) * q, both exact in f16.
  __device__ __forceinline__ void frag(int g, int c, f16x8 &a1, f16x8 &a2) const {
    int si = 2 + 2 * g + (c >> 1);
    int sc = (int)(int8_t)(hdr[si >> 2] >> (8 * (si & 3)));
    int s_hi = sc >> 4, s_lo = sc & 15;
    int h = g >> 2, t = g & 3;
    int piece = 2 * h + (t & 1);
    uint32_t lo = ql[piece >> 1][2 * (piece & 1)], hi = ql[piece >> 1][2 * (piece & 1) + 1];
    uint32_t hlo = qh[2 * h], hhi = qh[2 * h + 1];
    int nsh = t < 2 ? 0 : 4;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      int q0 = (int)(((lo >> (8 * e + nsh)) & 15) | (((hlo >> (8 * e + 2 * t)) & 3) << 4)) - 32;
      int q1 = (int)(((hi >> (8 * e + nsh)) & 15) | (((hhi >> (8 * e + 2 * t)) & 3) << 4)) - 32;
      a1[e] = (f16)(float)(16 * s_hi * q0);
      a1[4 + e] = (f16)(float)(16 * s_hi * q1);
      a2[e] = (f16)(float)(s_lo * q0);
      a2[4 + e] = (f16)(float)(s_lo * q1);
    }
  }
};

template <>
struct WFrag<LGMLH_Q8_0> {
  const uint8_t *qs;   // the lane's 8 blocks x 8 int8, read per group
  __device__ void load(const uint8_t *ch, int lane) { qs = ch + 256 + lane * 64; }
  __device__ __forceinline__ f16x8 frag(int g) const {
    u32x2 q = *(const u32x2 *)(qs + 8 * g);
    f16x8 r;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      r[e] = (f16)(float)(int8_t)(q[0] >> (8 * e));
      r[4 + e] = (f16)(float)(int8_t)(q[1] >> (8 * e));
    }
    return r;
  }
};

// ---- the quantized GEMM --------------------------------------------------------
// grid: (ceil(N / 64), ceil(M / WG_ROWS), splits); blockIdx.x (N tiles) varies
// fastest so the workgroups that share a weight tile run together.
//
// X is staged per K step as f16 hi and lo planes (x = hi + lo to 22 bits)
// plus the 32-value group sums (Q4_K min term); each product is the MFMA
// of the exact integer weights with hi, then with lo, summed in f32.
//
// Pipeline: the weight fragments and X pieces of K step sb + 1 load into
// registers while sb computes (two register sets, two LDS X buffers, one
// barrier per step). A split writes its partial sums; a second kernel adds
// the splits in order (no inter-workgroup sync).
template <int TYPE, bool XF32>
__global__ void __launch_bounds__(GEMM_THREADS)
qgemm_kernel(const uint8_t *__restrict__ w, int64_t M, int64_t K, const void *__restrict__ xv,
             int64_t N, float *__restrict__ y, int64_t ldy, const float *__restrict__ residual,
             int splits, int sb_per_split, float *__restrict__ part) {
  // Two X buffers: step sb computes from buffer sb & 1 while the pieces of
  // sb + 1 are staged into the other one (one barrier per step).
  __shared__ __align__(16) f16 xh_[2][WG_COLS * X_STRIDE];
  __shared__ __align__(16) f16 xl_[2][WG_COLS * X_STRIDE];
  __shared__ __align__(16) f16 gsh_[2][WG_COLS * 8];  // group sums, hi
  __shared__ __align__(16) f16 gsl_[2][WG_COLS * 8];  // group sums, lo
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t NSB = K / QK_K;
  const int64_t MT = (M + 15) / 16;
  const int64_t n0 = (int64_t)blockIdx.x * WG_COLS;
  const int64_t rt0 = (int64_t)blockIdx.y * (WG_ROWS / 16) + wave * RT_PER_WAVE;
  const int z = blockIdx.z;
  const int64_t sb_lo = (int64_t)z * sb_per_split;
  const int64_t sb_hi = sb_lo + sb_per_split < NSB ? sb_lo + sb_per_split : NSB;
  const int c = lane >> 4, r16 = lane & 15;

  f32x4 acc[RT_PER_WAVE][4];
#pragma unroll
  for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = f32x4{0, 0, 0, 0};

  // Thread tid stages pieces p = tid % 64 of X rows tid / 64 + 8 j: one
  // wave per row, so a 32-value group is 8 consecutive lanes.
  constexpr int XP = WG_COLS * 64 / GEMM_THREADS;  // pieces of 4 values per thread
  const int xp = tid & 63, xr0 = tid >> 6;
  f32x4 xreg[XP];
  auto load_x = [&](int64_t sbk) {
#pragma unroll
    for (int j = 0; j < XP; j++) {
      int64_t n = n0 + xr0 + 8 * j;
      f32x4 v = f32x4{0, 0, 0, 0};
      if (n < N) {
        if constexpr (XF32) {
          v = *(const f32x4 *)((const float *)xv + n * K + sbk * QK_K + xp * 4);
        } else {
          u32x2 hv = *(const u32x2 *)((const f16 *)xv + n * K + sbk * QK_K + xp * 4);
          f16x4 h = __builtin_bit_cast(f16x4, hv);
          v = f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        }
      }
      xreg[j] = v;
    }
  };
  auto stage_x = [&](int buf) {
    f16 *xh = xh_[buf], *xl = xl_[buf], *gsh = gsh_[buf], *gsl = gsl_[buf];
#pragma unroll
    for (int j = 0; j < XP; j++) {
      const int r = xr0 + 8 * j;
      f32x4 v = xreg[j];
      f16x4 h, l;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        h[e] = (f16)v[e];
        l[e] = (f16)(v[e] - (float)h[e]);
      }
      *(f16x4 *)(xh + r * X_STRIDE + xp * 4) = h;
      *(f16x4 *)(xl + r * X_STRIDE + xp * 4) = l;
      if constexpr (TYPE == LGMLH_Q4_K) {
        float gs = (v[0] + v[1]) + (v[2] + v[3]);
        gs += __shfl_xor(gs, 1);
        gs += __shfl_xor(gs, 2);
        gs += __shfl_xor(gs, 4);
        if ((xp & 7) == 0) {
          f16 gh = (f16)gs;
          gsh[r * 8 + (xp >> 3)] = gh;
          gsl[r * 8 + (xp >> 3)] = (f16)(gs - (float)gh);
        }
      }
    }
  };
  auto chunk_of = [&](int a, int64_t sbk) {
    int64_t rt = rt0 + a < MT ? rt0 + a : MT - 1;  // clamp: rows past M are never stored
    return w + (rt * NSB + sbk) * chunk_bytes(TYPE);
  };
  auto load_w = [&](WFrag<TYPE>(&dst)[RT_PER_WAVE], int64_t sbk) {
#pragma unroll
    for (int a = 0; a < RT_PER_WAVE; a++) dst[a].load(chunk_of(a, sbk), lane);
  };

  // One K step on the staged X with the weight fragments cur.
  auto compute = [&](int64_t sb, const WFrag<TYPE>(&cur)[RT_PER_WAVE], int buf) {
    const f16 *xh = xh_[buf], *xl = xl_[buf], *gsh = gsh_[buf], *gsl = gsl_[buf];
    f32x4 cm[RT_PER_WAVE][4];
#pragma unroll
    for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
      for (int b = 0; b < 4; b++) cm[a][b] = f32x4{0, 0, 0, 0};
#pragma unroll
    for (int g = 0; g < 8; g++) {
      f16x8 af[RT_PER_WAVE], af2[RT_PER_WAVE];
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        if constexpr (TYPE == LGMLH_Q6_K)
          cur[a].frag(g, c, af[a], af2[a]);
        else
          af[a] = cur[a].frag(g);
      }
#pragma unroll
      for (int ct = 0; ct < 4; ct++) {
        const int off = (ct * 16 + r16) * X_STRIDE + g * 32 + c * 8;
        f16x8 bh = *(const f16x8 *)(xh + off);
        f16x8 bl;
        if constexpr (XF32) bl = *(const f16x8 *)(xl + off);
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++) {
          cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bh, cm[a][ct], 0, 0, 0);
          if constexpr (TYPE == LGMLH_Q6_K)
            cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af2[a], bh, cm[a][ct], 0, 0, 0);
          if constexpr (XF32) {
            cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bl, cm[a][ct], 0, 0, 0);
            if constexpr (TYPE == LGMLH_Q6_K)
              cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af2[a], bl, cm[a][ct], 0, 0, 0);
          }
        }
      }
      if constexpr (TYPE == LGMLH_Q8_0) {
        // Q8_0: one scale per 32-value block: flush every group.
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++) {
          const uint8_t *hd = chunk_of(a, sb);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float d = h2f(*(const uint16_t *)(hd + (4 * c + i) * 16 + 2 * g));
#pragma unroll
            for (int ct = 0; ct < 4; ct++) {
              acc[a][ct][i] += d * cm[a][ct][i];
              cm[a][ct][i] = 0.0f;
            }
          }
        }
      }
    }
    if constexpr (TYPE == LGMLH_Q4_K) {
      // min term: sum_g m_g * S_g[n] as one 16x16x16 MFMA over the 8 groups.
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        f16x4 am = cur[a].mins(c);
        const uint8_t *hd = chunk_of(a, sb);
        float dd[4], dm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t h = *(const uint32_t *)(hd + (4 * c + i) * 16);
          dd[i] = h2f((uint16_t)h);
          dm[i] = h2f((uint16_t)(h >> 16));
        }
#pragma unroll
        for (int ct = 0; ct < 4; ct++) {
          f16x4 sh4 = f16x4{0, 0, 0, 0}, sl4 = sh4;
          if (c < 2) {
            sh4 = *(const f16x4 *)(gsh + (ct * 16 + r16) * 8 + 4 * c);
            sl4 = *(const f16x4 *)(gsl + (ct * 16 + r16) * 8 + 4 * c);
          }
          f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x16f16(am, sh4, f32x4{0, 0, 0, 0}, 0, 0, 0);
          mn = __builtin_amdgcn_mfma_f32_16x16x16f16(am, sl4, mn, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) acc[a][ct][i] += dd[i] * cm[a][ct][i] - dm[i] * mn[i];
        }
      }
    } else if constexpr (TYPE == LGMLH_Q6_K) {
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        const uint8_t *hd = chunk_of(a, sb);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float d = h2f(*(const uint16_t *)(hd + (4 * c + i) * 18));
#pragma unroll
          for (int ct = 0; ct < 4; ct++) acc[a][ct][i] += d * cm[a][ct][i];
        }
      }
    }
  };

  // Step sb: the loads of sb + 1 (weights into the other register set, X
  // pieces into xreg) go out first, compute runs on sb, then the X of sb + 1
  // is staged into the free LDS buffer and one barrier publishes it.
  WFrag<TYPE> w0[RT_PER_WAVE], w1[RT_PER_WAVE];
  auto step = [&](int64_t sb, const WFrag<TYPE>(&cur)[RT_PER_WAVE],
                  WFrag<TYPE>(&nxt)[RT_PER_WAVE]) {
    const bool more = sb + 1 < sb_hi;
    if (more) {
      load_w(nxt, sb + 1);
      load_x(sb + 1);
    }
    compute(sb, cur, (int)((sb - sb_lo) & 1));
    if (more) stage_x((int)((sb + 1 - sb_lo) & 1));
    __syncthreads();
  };
  if (sb_lo < sb_hi) {
    load_w(w0, sb_lo);
    load_x(sb_lo);
    stage_x(0);
    __syncthreads();
  }
  for (int64_t sb = sb_lo; sb < sb_hi; sb += 2) {
    step(sb, w0, w1);
    if (sb + 1 < sb_hi) step(sb + 1, w1, w0);
  }

  // acc[a][ct][i] = Y[n0 + ct*16 + lane%16][(rt0+a)*16 + 4*(lane/16) + i]
  float *dst = splits == 1 ? y : part + (int64_t)z * N * M;
  const int64_t ld = splits == 1 ? ldy : M;
#pragma unroll
  for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
    for (int ct = 0; ct < 4; ct++) {
      int64_t n = n0 + ct * 16 + r16;
      int64_t m = (rt0 + a) * 16 + 4 * c;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (m + i < M) {
          float v = acc[a][ct][i];
          if (splits == 1 && residual) v += residual[n * ldy + m + i];
          dst[n * ld + m + i] = v;
        }
    }
}

// The splits of a split-K product, added in order 0..splits-1.
__global__ void splitk_reduce_kernel(const float *__restrict__ part, int splits, int64_t N,
                                     int64_t M, float *__restrict__ y, int64_t ldy,
                                     const float *__restrict__ residual) {
  int64_t total = N * M;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t n = e / M, m = e % M;
    float v = 0.0f;
    for (int zz = 0; zz < splits; zz++) v += part[(int64_t)zz * total + e];
    if (residual) v += residual[n * ldy + m];
    y[n * ldy + m] = v;
  }
}

// ---- f32 weights: LDS-tiled VALU GEMM, sequential k order ----------------------
__global__ void __launch_bounds__(256)
f32gemm_kernel(const float *__restrict__ w, int64_t M, int64_t K, const float *__restrict__ x,
               int64_t N, float *__restrict__ y, int64_t ldy, const float *__restrict__ residual) {
  __shared__ float ws_[16][17], xs_[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t m = (int64_t)blockIdx.x * 16 + tx, n = (int64_t)blockIdx.y * 16 + ty;
  float acc = 0.0f;
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    int64_t wm = (int64_t)blockIdx.x * 16 + ty, xn = (int64_t)blockIdx.y * 16 + ty;
    ws_[ty][tx] = (wm < M && k0 + tx < K) ? w[wm * K + k0 + tx] : 0.0f;
    xs_[ty][tx] = (xn < N && k0 + tx < K) ? x[xn * K + k0 + tx] : 0.0f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; k++) acc = fmaf(xs_[ty][k], ws_[tx][k], acc);
    __syncthreads();
  }
  if (m < M && n < N) {
    float v = acc;
    if (residual) v += residual[n * ldy + m];
    y[n * ldy + m] = v;
  }
}

// K splits depend on M and K only, never on N: each output element is then
// the same sum in the same order for any batch size.
int splits_for(int64_t M, int64_t K, int64_t N) {
  (void)N;
  int64_t NSB = K / QK_K;
  int64_t tiles = (M + WG_ROWS - 1) / WG_ROWS;
  // About one workgroup per CU (256) at 64 columns, at least 2 K steps per
  // split so the pipeline has a step to overlap.
  int64_t want = (256 + tiles / 2) / tiles;
  int64_t maxs = NSB / 2 > 1 ? NSB / 2 : 1;
  if (want > maxs) want = maxs;
  if (want < 1) want = 1;
  return (int)want;
}

// Split-K partial sums of a call (0 when K is not split).
size_t partial_bytes(int type, int64_t M, int64_t K, int64_t N) {
  if (type == LGMLH_F32) return 0;
  int s = splits_for(M, K, N);
  return s == 1 ? 0 : (size_t)s * N * M * 4;
}

size_t workspace_for(int type, int64_t M, int64_t K, int64_t N) {
  return partial_bytes(type, M, K, N);
}

template <int TYPE>
static void launch_q(const void *w, int64_t M, int64_t K, const void *x, int xtype, int64_t N,
                     float *y, int64_t ldy, const float *res, int splits, float *part,
                     hipStream_t st) {
  int64_t NSB = K / QK_K;
  int spb = (int)((NSB + splits - 1) / splits);
  splits = (int)((NSB + spb - 1) / spb);
  dim3 grid((unsigned)((N + WG_COLS - 1) / WG_COLS), (unsigned)((M + WG_ROWS - 1) / WG_ROWS),
            (unsigned)splits);
  if (xtype == LGMLH_F32)
    hipLaunchKernelGGL((qgemm_kernel<TYPE, true>), grid, dim3(GEMM_THREADS), 0, st,
                       (const uint8_t *)w, M, K, x, N, y, ldy, res, splits, spb, part);
  else
    hipLaunchKernelGGL((qgemm_kernel<TYPE, false>), grid, dim3(GEMM_THREADS), 0, st,
                       (const uint8_t *)w, M, K, x, N, y, ldy, res, splits, spb, part);
  if (splits > 1) {
    int64_t total = N * M;
    unsigned blocks = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, part, splits, N, M,
                       y, ldy, res);
  }
}

// Internal entry with an output row stride (the executor writes [q|k|v]
// and [gate|up] rows from separate weights into one buffer) and a partial-
// sum region for split K.
int mul_mat_ldy(int type, const void *w, int64_t M, int64_t K, const void *x, int xtype,
                int64_t N, float *y, int64_t ldy, const float *residual, float *part,
                size_t part_bytes, hipStream_t st) {
  if (!w || !x || !y || M <= 0 || K <= 0 || N < 0 || ldy < M ||
      (xtype != LGMLH_F32 && xtype != LGMLH_F16)) {
    set_error("mul_mat: bad arguments");
    return LGMLH_EINVAL;
  }
  if (N == 0) return LGMLH_OK;
  if (type == LGMLH_F32) {
    if (xtype != LGMLH_F32) {
      set_error("mul_mat: f32 weights take f32 x");
      return LGMLH_EINVAL;
    }
    dim3 grid((unsigned)((M + 15) / 16), (unsigned)((N + 15) / 16));
    hipLaunchKernelGGL(f32gemm_kernel, grid, dim3(256), 0, st, (const float *)w, M, K,
                       (const float *)x, N, y, ldy, residual);
    return hip_check(hipGetLastError(), "mul_mat");
  }
  if (K % QK_K) {
    set_error("mul_mat: K = %lld is not a multiple of 256", (long long)K);
    return LGMLH_EINVAL;
  }
  int splits = splits_for(M, K, N);
  if (splits > 1 && (!part || part_bytes < partial_bytes(type, M, K, N))) {
    set_error("mul_mat: workspace too small for %d K splits", splits);
    return LGMLH_ENOMEM;
  }
  switch (type) {
    case LGMLH_Q4_K: launch_q<LGMLH_Q4_K>(w, M, K, x, xtype, N, y, ldy, residual, splits, part, st); break;
    case LGMLH_Q6_K: launch_q<LGMLH_Q6_K>(w, M, K, x, xtype, N, y, ldy, residual, splits, part, st); break;
    case LGMLH_Q8_0: launch_q<LGMLH_Q8_0>(w, M, K, x, xtype, N, y, ldy, residual, splits, part, st); break;
    default:
      set_error("mul_mat: type %d not supported", type);
      return LGMLH_EINVAL;
  }
  return hip_check(hipGetLastError(), "mul_mat");
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" int64_t lgmlh_repacked_bytes(int type, int64_t M, int64_t K) {
  if (M <= 0 || K <= 0) return -1;
  if (type == LGMLH_F32) return M * K * 4;
  if (chunk_bytes(type) == 0 || K % QK_K) return -1;
  return ((M + 15) / 16) * (K / QK_K) * chunk_bytes(type);
}

extern "C" int lgmlh_repack(int type, int64_t M, int64_t K, const void *src, void *dst,
                            void *stream) {
  if (!src || !dst || lgmlh_repacked_bytes(type, M, K) < 0) {
    set_error("repack: bad arguments (type %d, M %lld, K %lld)", type, (long long)M, (long long)K);
    return LGMLH_EINVAL;
  }
  hipStream_t st = as_stream(stream);
  if (type == LGMLH_F32)
    return hip_check(hipMemcpyAsync(dst, src, (size_t)(M * K * 4), hipMemcpyDeviceToDevice, st),
                     "repack");
  int64_t NSB = K / QK_K, total = ((M + 15) / 16) * NSB * 64;
  unsigned blocks = (unsigned)((total + 255) / 256);
  switch (type) {
    case LGMLH_Q4_K: hipLaunchKernelGGL(repack_kernel<LGMLH_Q4_K>, dim3(blocks), dim3(256), 0, st, (const uint8_t *)src, M, NSB, (uint8_t *)dst); break;
    case LGMLH_Q6_K: hipLaunchKernelGGL(repack_kernel<LGMLH_Q6_K>, dim3(blocks), dim3(256), 0, st, (const uint8_t *)src, M, NSB, (uint8_t *)dst); break;
    case LGMLH_Q8_0: hipLaunchKernelGGL(repack_kernel<LGMLH_Q8_0>, dim3(blocks), dim3(256), 0, st, (const uint8_t *)src, M, NSB, (uint8_t *)dst); break;
  }
  return hip_check(hipGetLastError(), "repack");
}

extern "C" size_t lgmlh_mul_mat_workspace(int type, int64_t M, int64_t K, int64_t N) {
  return workspace_for(type, M, K, N);
}

extern "C" int lgmlh_mul_mat(int type, const void *w, int64_t M, int64_t K, const void *x,
                             int xtype, int64_t N, float *y, int epi, const float *residual,
                             void *workspace, size_t ws_bytes, void *stream) {
  if (epi != LGMLH_EPI_NONE && epi != LGMLH_EPI_ADD) {
    set_error("mul_mat: bad epilogue");
    return LGMLH_EINVAL;
  }
  if (epi == LGMLH_EPI_ADD && !residual) {
    set_error("mul_mat: the add epilogue needs a residual");
    return LGMLH_EINVAL;
  }
  size_t need = workspace_for(type, M, K, N);
  if (need > 0 && (!workspace || ws_bytes < need)) {
    set_error("mul_mat: workspace of %zu bytes, need %zu", ws_bytes, need);
    return LGMLH_ENOMEM;
  }
  return mul_mat_ldy(type, w, M, K, x, xtype, N, y, M, epi == LGMLH_EPI_ADD ? residual : nullptr,
                     (float *)workspace, ws_bytes, as_stream(stream));
}
