// Weight products Y (N, M) = X (N, K) W^T for f32 / Q4_K / Q6_K / Q8_0 W
// (graph:mul_mat, src/lgml.c:1811-1839) on gfx950.
//
// Quantized W is repacked once into row tiles of 16 rows. For row tile rt
// and K step sb (256 values) one chunk holds the tile's block headers and
// then, for each of the 64 lanes of a wavefront (lane = r + 16 c: row r,
// 8-value k chunk c of every 32-value group), exactly the bytes that lane
// turns into its MFMA A fragment. The headers are laid out so that a lane
// finds the scales of its row, and the super-block scales of the four
// output rows it accumulates, in one load each.
//
// X arrives split (split.h): f16 hi and lo planes and the 32-value group
// sums. A wave streams its chunks with 16-byte loads and builds exact
// integer A fragments with byte permutes and one packed f16 FMA per pair
// (Q4_K: sc * q; Q6_K: sc * q / 4 as two exact parts; Q8_0: q); each
// 16x16x32 f16 MFMA takes A against hi and against lo, so a product is
// f32-accurate. Super-block scales (d, dmin) are applied in f32 per K step
// (Q8_0: per 32-value block).
//
// Every output element is the same f32 sum over K in the same order for any
// N, so a row gives the same bits alone or batched. K is split over
// workgroups when M alone gives too few (split count from M and K only);
// the splits are added in a fixed order by a second kernel.
#include <mutex>

#include "common.h"
#include "quant.h"
#include "split.h"

namespace lgmlh {

constexpr int GEMM_WAVES = 8;      // waves per workgroup (4 for Q4_K / Q6_K wide tiles: gemm_waves)
constexpr int RT_PER_WAVE = 2;     // 16-row tiles per wave
// Rows of an 8-wave workgroup: the unit in which the K-split count and the
// tiling rules count row tiles (fixed, so the splits do not depend on N).
constexpr int WG_ROWS = GEMM_WAVES * RT_PER_WAVE * 16;  // 256
constexpr int WG_COLS = 64;        // N columns per workgroup of a plain product (4 tiles)
// X in LDS: per plane NCT * 16 rows x 32 pieces of 8 f16 (16 B), piece kp
// of row n at slot n * 32 + (kp ^ (n & 15)) (no padding: global-to-LDS
// loads write 64 consecutive slots; the swizzle keeps a 16-row B read
// conflict-free).

// Grouped products (mul_mat_id): the columns of a workgroup are picks of
// one expert, gathered from the X planes. tiles[i] = {expert, first,
// count, 0}: columns 0..count-1 are picks sorted[first ..]; pick p reads
// X row (p / n_used) * U + (p % n_used) % U and writes Y row p.
struct Gather {
  const int32_t *sorted = nullptr;
  const int4 *tiles = nullptr;
  const int32_t *n_tiles = nullptr;  // tiles in use (device)
  int64_t expert_bytes = 0;          // one expert's repacked matrix
  int n_used = 1, U = 1;
  __device__ __forceinline__ int64_t xrow(int p) const {
    return (int64_t)(p / n_used) * U + (p % n_used) % U;
  }
};

// Bytes of one repacked chunk (16 rows x 256 values).
__host__ __device__ constexpr int chunk_bytes(int type) {
  return type == LGMLH_Q4_K ? 16 * Q4K_BYTES
       : type == LGMLH_Q6_K ? 16 * Q6K_BYTES
       : type == LGMLH_Q8_0 ? 16 * 8 * Q8_0_BYTES : 0;
}
// Bytes of the header part of a chunk:
//   Q4_K: [16 rows: u32 d | dmin << 16] [16 rows: 12 scale bytes]
//   Q6_K: [16 rows: f16 d] [16 rows: 16 int8 scales]
//   Q8_0: [4 c][8 blocks g][4 i] f16 d of row 4c + i, block g
__host__ __device__ constexpr int chunk_hdr(int type) {
  return type == LGMLH_Q4_K ? 256 : type == LGMLH_Q6_K ? 288 : type == LGMLH_Q8_0 ? 256 : 0;
}
// Bytes of one lane's data in a chunk.
__host__ __device__ constexpr int lane_bytes(int type) {
  return type == LGMLH_Q4_K ? 32 : type == LGMLH_Q6_K ? 48 : type == LGMLH_Q8_0 ? 64 : 0;
}

// ---- repack: ggml row blocks -> row-tile chunks ------------------------------
// One thread per (row tile, sb, lane): copies the lane's bytes and, for
// c == 0, the row's header fields.
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
  const bool pad = m >= M;  // padding rows: zero bytes give zero weights
  if (TYPE == LGMLH_Q4_K) {
    const uint8_t *b = src + (m * NSB + sb) * Q4K_BYTES;
    if (c == 0) {
      for (int i = 0; i < 4; i++) ch[4 * r + i] = pad ? 0 : b[i];
      for (int i = 0; i < 12; i++) ch[64 + 12 * r + i] = pad ? 0 : b[4 + i];
    }
    // piece j: qs[32j + 8c .. +7] (low nibbles group 2j, high nibbles 2j + 1)
    for (int j = 0; j < 4; j++)
      for (int e = 0; e < 8; e++) ld[8 * j + e] = pad ? 0 : b[16 + 32 * j + 8 * c + e];
  } else if (TYPE == LGMLH_Q6_K) {
    const uint8_t *b = src + (m * NSB + sb) * Q6K_BYTES;
    if (c == 0) {
      ch[2 * r] = pad ? 0 : b[208];
      ch[2 * r + 1] = pad ? 0 : b[209];
      for (int i = 0; i < 16; i++) ch[32 + 16 * r + i] = pad ? 0 : b[192 + i];
    }
    // ql pieces (h, tb): ql[64h + 32tb + 8c .. +7]; then qh pieces h: qh[32h + 8c .. +7]
    for (int h = 0; h < 2; h++)
      for (int tb = 0; tb < 2; tb++)
        for (int e = 0; e < 8; e++)
          ld[8 * (2 * h + tb) + e] = pad ? 0 : b[64 * h + 32 * tb + 8 * c + e];
    for (int h = 0; h < 2; h++)
      for (int e = 0; e < 8; e++) ld[32 + 8 * h + e] = pad ? 0 : b[128 + 32 * h + 8 * c + e];
  } else {  // Q8_0: 8 blocks of 32 per 256 values
    const uint8_t *b = src + (m * NSB * 8 + sb * 8) * Q8_0_BYTES;
    if (c == 0)
      for (int g = 0; g < 8; g++) {
        uint8_t *d = ch + 64 * (r >> 2) + 8 * g + 2 * (r & 3);
        d[0] = pad ? 0 : b[g * Q8_0_BYTES];
        d[1] = pad ? 0 : b[g * Q8_0_BYTES + 1];
      }
    for (int g = 0; g < 8; g++)
      for (int e = 0; e < 8; e++) ld[8 * g + e] = pad ? 0 : b[g * Q8_0_BYTES + 2 + 8 * c + e];
  }
}

// ---- A fragments -----------------------------------------------------------
// biased(bytes, SEL_*): two bytes b of `bytes` as the f16 pair 1024 + b
// (0x64 in the high byte, b in the mantissa); SEL_01 takes bytes 0, 1 and
// SEL_23 bytes 2, 3. An FMA with (s, -1024 s) then gives s * b exactly
// whenever the result fits 11 significant bits.
constexpr uint32_t SEL_01 = 0x04010400u, SEL_23 = 0x04030402u;
// hbiased(bytes, HSEL_*): the f16 pair whose high bytes are bytes 0, 1 (or
// 2, 3) and whose low bytes are zero.
constexpr uint32_t HSEL_01 = 0x050c040cu, HSEL_23 = 0x070c060cu;

__device__ __forceinline__ f16x2 biased(uint32_t bytes, uint32_t sel) {
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, bytes, sel));
}
__device__ __forceinline__ f16x2 hbiased(uint32_t bytes, uint32_t sel) {
  return __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(bytes, 0u, sel));
}
__device__ __forceinline__ f16x2 fma2(f16x2 a, f16 s, f16 c) {
  return __builtin_elementwise_fma(a, f16x2{s, s}, f16x2{c, c});
}
__device__ __forceinline__ f16x8 cat4(f16x2 a, f16x2 b, f16x2 c, f16x2 d) {
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

template <int TYPE>
struct WFrag;

template <>
struct WFrag<LGMLH_Q4_K> {
  u32x4 dm;               // d | dmin << 16 of rows 4c + i, i = 0..3
  uint32_t s0, s1, s2;    // the 12 scale bytes of row r
  u32x4 qs[2];            // 4 pieces of 8 bytes
  __device__ __forceinline__ void load(const uint8_t *ch, uint32_t lane) {
    dm = *(const u32x4 *)(ch + 16u * (lane >> 4));
    const uint32_t *sp = (const uint32_t *)(ch + 64u + 12u * (lane & 15));
    s0 = sp[0];
    s1 = sp[1];
    s2 = sp[2];
    const u32x4 *p = (const u32x4 *)(ch + 256u + lane * 32u);
    qs[0] = p[0];
    qs[1] = p[1];
  }
  // 6-bit scales (sc) and mins (m) of groups 0..3 / 4..7, one per byte
  // (get_scale_min_k4 of the block format).
  __device__ __forceinline__ uint32_t sc03() const { return s0 & 0x3F3F3F3Fu; }
  __device__ __forceinline__ uint32_t sc47() const {
    return (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
  }
  __device__ __forceinline__ uint32_t m03() const { return s1 & 0x3F3F3F3Fu; }
  __device__ __forceinline__ uint32_t m47() const {
    return ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
  }
  // The multipliers of groups 2j (low nibbles) and 2j + 1 (high nibbles):
  // s = {sc_2j, sc_2j+1 / 16}, cc = {-1024 sc_2j, -64 sc_2j+1} (all exact
  // in f16), from the scale bytes of g's half (sc03 or sc47) by one
  // permute and packed f16 arithmetic.
  __device__ __forceinline__ void pair(int j, uint32_t scb, f16x2 &s, f16x2 &cc) const {
    const f16x2 sc = biased(scb, (j & 1) ? SEL_23 : SEL_01) - f16x2{(f16)1024.0f, (f16)1024.0f};
    s = sc * f16x2{(f16)1.0f, (f16)0.0625f};
    cc = sc * f16x2{(f16)-1024.0f, (f16)-64.0f};
  }
  // sc_g * q for k = 32g + 8c + e, e = 0..7 (<= 945, exact), with s / cc
  // of g's pair. Low nibbles: (1024 + q) sc - 1024 sc; high nibbles kept
  // in place: (1024 + 16 q) sc / 16 - 64 sc.
  __device__ __forceinline__ f16x8 frag(int g, f16x2 sp, f16x2 cp) const {
    const int j = g >> 1;
    const uint32_t w0 = qs[j >> 1][2 * (j & 1)], w1 = qs[j >> 1][2 * (j & 1) + 1];
    uint32_t n0, n1;
    f16 s, cc;
    if (g & 1) {
      n0 = w0 & 0xF0F0F0F0u;
      n1 = w1 & 0xF0F0F0F0u;
      s = sp[1];
      cc = cp[1];
    } else {
      n0 = w0 & 0x0F0F0F0Fu;
      n1 = w1 & 0x0F0F0F0Fu;
      s = sp[0];
      cc = cp[0];
    }
    return cat4(fma2(biased(n0, SEL_01), s, cc), fma2(biased(n0, SEL_23), s, cc),
                fma2(biased(n1, SEL_01), s, cc), fma2(biased(n1, SEL_23), s, cc));
  }
  // The 16x16x16 A fragment of the mins against the 16 sums of 16 values
  // (Q8_K bsums): row r, k = 4c .. 4c + 3, sum k in group k / 2, so
  // {m_2c, m_2c, m_2c+1, m_2c+1}.
  __device__ __forceinline__ f16x4 mins16(int c) const {
    const uint32_t mb = c < 2 ? m03() : m47();
    const f16x2 k = f16x2{(f16)1024.0f, (f16)1024.0f};
    const f16x2 a = biased(mb, (c & 1) ? SEL_23 : SEL_01) - k;
    return f16x4{a[0], a[0], a[1], a[1]};
  }
  // The 16x16x16 A fragment of the mins: row r, k = groups 4c .. 4c + 3
  // (zero for c >= 2).
  __device__ __forceinline__ f16x4 mins(int c) const {
    const uint32_t mb = c == 0 ? m03() : m47();
    const f16x2 k = f16x2{(f16)1024.0f, (f16)1024.0f};
    const f16x2 a = biased(mb, SEL_01) - k, b = biased(mb, SEL_23) - k;
    return c < 2 ? f16x4{a[0], a[1], b[0], b[1]} : f16x4{0, 0, 0, 0};
  }
};

template <>
struct WFrag<LGMLH_Q6_K> {
  u32x2 d4;        // f16 d of rows 4c + i, i = 0..3
  u32x4 scl;       // the 16 int8 scales of row r
  u32x4 ql[2];     // ql pieces (h, tb), index 2h + tb
  u32x4 qh;        // qh pieces h
  __device__ __forceinline__ void load(const uint8_t *ch, uint32_t lane) {
    d4 = *(const u32x2 *)(ch + 8u * (lane >> 4));
    scl = *(const u32x4 *)(ch + 32u + 16u * (lane & 15));
    const u32x4 *p = (const u32x4 *)(ch + 288u + lane * 48u);
    ql[0] = p[0];
    ql[1] = p[1];
    qh = p[2];
  }
  // sc * q / 4 for k = 32g + 8c + e, with q = u - 32, u = u_lo + 16 u_hi:
  //   a1 = sc u_lo / 4       = (1024 + u_lo) (sc / 4) - 256 sc      exact
  //   a2 = 4 sc (u_hi - 2)   = (1 + u_hi / 4) (16 sc) - 24 sc        exact
  //   ar = f16(a1 + a2)      rounded, for the product with x lo.
  // sh = 8 * (c >> 1): the lane's scale (16-value block 2g + c / 2).
  __device__ __forceinline__ void frag(int g, uint32_t sh, f16x8 &a1, f16x8 &a2, f16x8 &ar) const {
    const int hh = g >> 2, t = g & 3, piece = 2 * hh + (t & 1);
    const uint32_t lq0 = ql[piece >> 1][2 * (piece & 1)], lq1 = ql[piece >> 1][2 * (piece & 1) + 1];
    const uint32_t hq0 = qh[2 * hh], hq1 = qh[2 * hh + 1];
    uint32_t n0, n1;
    if (t < 2) {
      n0 = lq0 & 0x0F0F0F0Fu;
      n1 = lq1 & 0x0F0F0F0Fu;
    } else {
      n0 = (lq0 >> 4) & 0x0F0F0F0Fu;
      n1 = (lq1 >> 4) & 0x0F0F0F0Fu;
    }
    const uint32_t b0 = ((hq0 >> (2 * t)) & 0x03030303u) | 0x3C3C3C3Cu;
    const uint32_t b1 = ((hq1 >> (2 * t)) & 0x03030303u) | 0x3C3C3C3Cu;
    const int sc = (int)(int8_t)(scl[g >> 1] >> (16 * (g & 1) + sh));
    const f16 scf = (f16)(float)sc;
    const f16 s1 = scf * (f16)0.25f, c1 = scf * (f16)-256.0f;
    const f16 s2 = scf * (f16)16.0f, c2 = scf * (f16)-24.0f;
    a1 = cat4(fma2(biased(n0, SEL_01), s1, c1), fma2(biased(n0, SEL_23), s1, c1),
              fma2(biased(n1, SEL_01), s1, c1), fma2(biased(n1, SEL_23), s1, c1));
    a2 = cat4(fma2(hbiased(b0, HSEL_01), s2, c2), fma2(hbiased(b0, HSEL_23), s2, c2),
              fma2(hbiased(b1, HSEL_01), s2, c2), fma2(hbiased(b1, HSEL_23), s2, c2));
    ar = a1 + a2;
  }
};

template <>
struct WFrag<LGMLH_Q8_0> {
  u32x4 qs[4];           // 8 blocks x 8 int8 (the header goes through LDS)
  __device__ __forceinline__ void load(const uint8_t *ch, uint32_t lane) {
    const u32x4 *p = (const u32x4 *)(ch + 256u + lane * 64u);
#pragma unroll
    for (int i = 0; i < 4; i++) qs[i] = p[i];
  }
  // q for k = 32g + 8c + e: (1024 + (q + 128)) - 1152, exact.
  __device__ __forceinline__ f16x8 frag(int g) const {
    const uint32_t w0 = qs[g >> 1][2 * (g & 1)] ^ 0x80808080u;
    const uint32_t w1 = qs[g >> 1][2 * (g & 1) + 1] ^ 0x80808080u;
    const f16x2 k = f16x2{(f16)1152.0f, (f16)1152.0f};
    return cat4(biased(w0, SEL_01) - k, biased(w0, SEL_23) - k, biased(w1, SEL_01) - k,
                biased(w1, SEL_23) - k);
  }
};

// ---- the quantized GEMM --------------------------------------------------------
// grid: (ceil(N / (16 NCT)), ceil(M / rows per workgroup), splits);
// blockIdx.x (N tiles) varies fastest so the workgroups that share a
// weight tile run together (the wide tiles renumber them per XCD).
//
// Pipeline: the weight fragments (into registers) and X pieces (global-to-
// LDS) of K step sb + 1 are issued at the start of step sb and load while
// it computes (two register sets, two LDS buffers, each buffer its own LDS
// object so that reads of one need not wait for loads into the other; one
// barrier per step; with one buffer, the X loads follow the step's
// products and a barrier). Q8_0 chunk headers (a d per row and 32-value block)
// travel with X, global-to-LDS, and each group's d are read from LDS one
// group ahead. A split writes its partial sums; a second kernel adds the
// splits in order (no inter-workgroup sync).
// One column tile of Q4_K / Q6_K (the grouped expert products; plain
// products of at most 16 columns): registers capped at 128 (4 waves per
// SIMD) so that two workgroups share a CU, twice the weight loads in
// flight (C5's expert products 5.18 -> 4.42 ms per step). Q8_0 would spill
// under the cap, and so does Q6_K on ggml's X (its two exact parts per
// group): capped at 256 it takes 149 and runs 3 waves per SIMD (the V
// product of C2's mix, 1024 x 4096 at 64 columns, 19.1 -> 17.5 us with its
// reduction; 4096 x 14336 at 16 columns 31.4 -> 26.1 us).
// Q4_K with 64-column tiles: workgroups of 4 waves (128 rows) with one X
// buffer (66 KB of LDS), so that two share a CU; one's waits for its next
// K step (the X loads, the barriers) are filled by the other's products
// (C2's Q4_K shapes at N = 576: 4-15% faster, gate|up at N = 64 6%; the
// mixed phase 3228 -> 3397 tok/s). Q6_K on ggml's X the same, with two X
// buffers (70 KB): C2's Q6_K down products at a 512-token prefill pass 4.21
// -> 3.27 ms. A tile's sums do not depend on the workgroup shape: each
// 16-row tile takes the same fragments in the same K steps.
__host__ __device__ constexpr int gemm_waves(int type, int nct, bool q8) {
  return nct == 4 && (type == LGMLH_Q4_K || (type == LGMLH_Q6_K && q8)) ? 4 : GEMM_WAVES;
}
//
// Q8: X as ggml's quantized activations (split.h: Q8_K for Q4_K / Q6_K,
// Q8_0 for Q8_0), the reference CPU path's arithmetic. The B fragments are
// the integer q (exact in f16), so one MFMA per group replaces the hi + lo
// pair (Q6_K: the two exact parts of sc q against q, no rounded third);
// every block sum is an exact integer in the f32 accumulator (below 2^24
// unless a block is extreme). Per K step the Q4_K min term is one 16x16x16
// MFMA of the mins against the 16 sums of 16 q, and the block scales go on
// in f32: Q4_K d_x (d_w I - dmin_w Mn), Q6_K (d_w d_x) I, Q8_0 per 32-value
// block (d_w d_x) I. X is half the bytes to stage (no lo plane), so the
// 4-wave Q4_K / Q6_K workgroups keep two X buffers.
template <int TYPE, int NCT, bool GATHER, bool Q8>
__global__ void __launch_bounds__(gemm_waves(TYPE, NCT, Q8) * 64,
                                  NCT == 1 && TYPE == LGMLH_Q6_K && Q8 ? 2
                                  : NCT == 1 && TYPE != LGMLH_Q8_0   ? 4
                                  : gemm_waves(TYPE, NCT, Q8) == 4 ? 2
                                                                   : 1)
qgemm_kernel(const uint8_t *__restrict__ w, int64_t M, int64_t K, const f16 *__restrict__ xs,
             int64_t Npad, int64_t N, float *__restrict__ y, int64_t ldy,
             const float *__restrict__ residual, int nz, int sb_per_split, int fold,
             float *__restrict__ part, Gather gt) {
  constexpr int WVS = gemm_waves(TYPE, NCT, Q8);  // waves per workgroup
  constexpr bool ONEBUF = WVS < GEMM_WAVES && !Q8;  // one X buffer
  constexpr int COLS = NCT * 16;            // N columns per workgroup
  constexpr int X_SLOTS = COLS * 32;
  constexpr int XL_SLOTS = Q8 ? 1 : X_SLOTS;
  // Q8: the X block scales of a K step: Q8_K one f32 per column (16
  // slots); Q8_0 8 per column, [half][column][4] (128 slots)
  constexpr int DX_SLOTS = !Q8 ? 1 : TYPE == LGMLH_Q8_0 ? 128 : 16;
  __shared__ __align__(16) u32x4 xh0_[X_SLOTS], xh1_[ONEBUF ? 1 : X_SLOTS];
  __shared__ __align__(16) u32x4 xl0_[XL_SLOTS], xl1_[ONEBUF ? 1 : XL_SLOTS];
  // Q4_K group sums, 8 f16 per row: hi at slots 0..63, lo at 64..127 (Q8:
  // the 16 sums of 16 q, 0..7 and 8..15), slot 128 zeros for lanes c >= 2.
  // One LDS object per buffer: the compiler then knows that reads of one
  // buffer need not wait for the loads in flight into the other.
  __shared__ __align__(16) u32x4 gs0_[129], gs1_[129];
  __shared__ __align__(16) u32x4 dx0_[DX_SLOTS], dx1_[DX_SLOTS];
  // Q8_0: the 256-byte headers of every wave's chunks (wave w, tile a at
  // slots 32 w + 16 a .. + 15)
  constexpr int HD_SLOTS = TYPE == LGMLH_Q8_0 ? WVS * RT_PER_WAVE * 16 : 1;
  __shared__ __align__(16) u32x4 hd0_[HD_SLOTS], hd1_[HD_SLOTS];
  auto XH = [&](int b) { return b && !ONEBUF ? xh1_ : xh0_; };
  auto XL = [&](int b) { return b && !ONEBUF ? xl1_ : xl0_; };
  auto GS = [&](int b) { return b && !ONEBUF ? gs1_ : gs0_; };
  auto HD = [&](int b) { return b ? hd1_ : hd0_; };
  auto DX = [&](int b) { return (const float *)(b ? dx1_ : dx0_); };
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  if (tid == 0) {  // read after the prologue's barrier
    gs0_[128] = u32x4{0, 0, 0, 0};
    gs1_[128] = u32x4{0, 0, 0, 0};
  }
  const int64_t NSB = K / QK_K;
  const int64_t MT = (M + 15) / 16;
  // Tile order for the wide tiles: the dispatcher deals workgroups round-
  // robin to the 8 XCDs, each with its own L2, so the tiles are renumbered
  // to give consecutive tiles to one XCD, and ordered in groups of 3
  // column tiles: the workgroups an XCD runs together share the weights
  // of a few row blocks and the X of 3 column tiles in its L2. Which
  // workgroup computes a tile changes, not how (prefill products 4%, then
  // 2% faster; no gain for 16-column tiles).
  uint32_t bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if constexpr (NCT == 4 && !GATHER) {
    const uint32_t gx = gridDim.x, gy = gridDim.y, total = gx * gy * gridDim.z;
    const uint32_t L = bx + gx * (by + gy * bz);
    const uint32_t xcd = L & 7u, per = total >> 3, rem = total & 7u;
    const uint32_t t = xcd * per + (xcd < rem ? xcd : rem) + (L >> 3);
    constexpr uint32_t CG = 3;  // column tiles per group
    bz = t / (gx * gy);
    const uint32_t r = t % (gx * gy), g = r / (CG * gy), rr = r - g * CG * gy;
    const uint32_t wg = gx - g * CG < CG ? gx - g * CG : CG;  // the last group may be narrower
    by = rr / wg;
    bx = g * CG + rr % wg;
  }
  int64_t n0 = (int64_t)bx * COLS;
  int first = 0, count = 0;
  if constexpr (GATHER) {
    // tiles past the ones in use leave at once (the whole workgroup)
    if ((int)blockIdx.x >= *gt.n_tiles) return;
    const int4 tl = gt.tiles[blockIdx.x];
    w += tl.x * gt.expert_bytes;
    first = tl.y;
    count = tl.z;
    n0 = 0;
  }
  const int64_t rt0 = (int64_t)by * (WVS * RT_PER_WAVE) + wave * RT_PER_WAVE;
  // K range: splits fold z .. fold z + fold - 1 of sb_per_split steps each
  const int z = (int)bz;
  const int64_t sb_lo = (int64_t)z * fold * sb_per_split;
  const int64_t sb_hi = sb_lo + fold * sb_per_split < NSB ? sb_lo + fold * sb_per_split : NSB;
  const int c = lane >> 4, r16 = lane & 15;
  // X row of column n (GATHER: of its pick; columns past count repeat the
  // first pick and are never stored)
  auto xrow = [&](int n) -> int64_t {
    if constexpr (GATHER) return gt.xrow(gt.sorted[first + (n < count ? n : 0)]);
    else return n;
  };

  f32x4 acc[RT_PER_WAVE][NCT];
#pragma unroll
  for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
    for (int b = 0; b < NCT; b++) acc[a][b] = f32x4{0, 0, 0, 0};

  // Staging: global-to-LDS loads (no registers). Per plane and step, wave
  // w fills slots [64 XJ w, 64 XJ (w + 1)) with XJ loads of 64 slots; lane
  // l of load j writes slot s = 64 (XJ w + j) + l, which holds piece
  // kp = (s % 32) ^ (row & 15) of row s / 32.
  typedef __attribute__((address_space(3))) void lds_t;
  constexpr int XJ = X_SLOTS / (WVS * 64);  // NCT
  const f16 *xhi = xs + n0 * K + sb_lo * QK_K, *xlo = xhi + Npad * K;
  const f16 *ghi = xs + 2 * Npad * K + n0 * (K / 32) + sb_lo * 8, *glo = ghi + Npad * (K / 32);
  // Q8: the 16-value sums and the block scales from the K range's start
  // (per column: xrow * K / 16, xrow * K / QB added per lane)
  constexpr int QB = TYPE == LGMLH_Q8_0 ? 32 : QK_K;
  const f16 *bsp = xs + q8_bs_off(Npad, K) + n0 * (K / 16) + sb_lo * 16;
  const float *dxp = (const float *)((const char *)xs + q8_d_off(Npad, K)) + n0 * (K / QB) +
                     sb_lo * (QK_K / QB);
  // byte offsets of a lane's pieces from the plane's K step (the planes
  // stay under 4 GiB: checked at launch)
  uint32_t xoff[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int sl = (wave * XJ + j) * 64 + lane, n = sl >> 5, kp = (sl & 31) ^ (n & 15);
    xoff[j] = (uint32_t)(xrow(n) * K + kp * 8) * 2u;
  }
  // group sums: lane = column (lanes past the workgroup's columns load a
  // valid row into slots that are never read)
  const int64_t xr_lane = xrow(lane < COLS ? lane : 0);
  const uint32_t goff = (uint32_t)(xr_lane * (Q8 ? K / 16 : K / 32));
  const uint32_t doff = (uint32_t)(xr_lane * (K / QB));
  // Chunk of tile a at K step sb_lo + kstep: a wave-uniform address (rows
  // past M clamp to the last tile; they are computed but never stored).
  const uint8_t *wt[RT_PER_WAVE];
#pragma unroll
  for (int a = 0; a < RT_PER_WAVE; a++) {
    const int64_t rt = rt0 + a < MT ? rt0 + a : MT - 1;
    wt[a] = w + (rt * NSB + sb_lo) * chunk_bytes(TYPE);
  }
  // Q8_0 header piece of lane < 32: tile lane / 16, bytes 16 (lane % 16)
  const uint8_t *hsrc = wt[(lane >> 4) & 1] + 16 * (lane & 15);
  auto load_x = [&](uint32_t kstep, int buf) {  // kstep = sb - sb_lo
#pragma unroll
    for (int j = 0; j < XJ; j++) {
      const int slot0 = (wave * XJ + j) * 64;
      // a wave-uniform base plus a 32-bit lane offset (no 64-bit adds per lane)
      const uint8_t *bh = (const uint8_t *)(xhi + kstep * QK_K);
      const uint8_t *bl = (const uint8_t *)(xlo + kstep * QK_K);
      __builtin_amdgcn_global_load_lds((const void *)(bh + xoff[j]), (lds_t *)&XH(buf)[slot0],
                                       16, 0, 0);
      if constexpr (!Q8)
        __builtin_amdgcn_global_load_lds((const void *)(bl + xoff[j]), (lds_t *)&XL(buf)[slot0],
                                         16, 0, 0);
    }
    if constexpr (TYPE == LGMLH_Q4_K && !Q8) {
      if (wave < 2)  // wave 0: hi sums, wave 1: lo sums
        __builtin_amdgcn_global_load_lds(
            (const void *)((wave == 0 ? ghi : glo) + goff + kstep * 8),
            (lds_t *)(GS(buf) + 64 * wave), 16, 0, 0);
    }
    if constexpr (TYPE == LGMLH_Q4_K && Q8) {
      if (wave < 2)  // wave 0: sums 0..7 of 16 q, wave 1: sums 8..15
        __builtin_amdgcn_global_load_lds((const void *)(bsp + goff + kstep * 16 + 8 * wave),
                                         (lds_t *)(GS(buf) + 64 * wave), 16, 0, 0);
    }
    if constexpr (Q8 && TYPE != LGMLH_Q8_0) {
      if (wave == 2)  // the d of each column (lane)
        __builtin_amdgcn_global_load_lds((const void *)(dxp + doff + kstep),
                                         (lds_t *)(buf ? dx1_ : dx0_), 4, 0, 0);
    }
    if constexpr (Q8 && TYPE == LGMLH_Q8_0) {
      if (wave < 2)  // the d of blocks 4 wave .. 4 wave + 3 of each column (lane)
        __builtin_amdgcn_global_load_lds((const void *)(dxp + doff + kstep * 8 + 4 * wave),
                                         (lds_t *)((buf ? dx1_ : dx0_) + 64 * wave), 16, 0, 0);
    }
    if constexpr (TYPE == LGMLH_Q8_0) {
      if (lane < 32)
        __builtin_amdgcn_global_load_lds(
            (const void *)(hsrc + kstep * (uint32_t)chunk_bytes(TYPE)),
            (lds_t *)&HD(buf)[wave * RT_PER_WAVE * 16], 16, 0, 0);
    }
  };
  auto load_w = [&](WFrag<TYPE>(&dst)[RT_PER_WAVE], uint32_t kstep) {
#pragma unroll
    for (int a = 0; a < RT_PER_WAVE; a++) dst[a].load(wt[a] + kstep * (uint32_t)chunk_bytes(TYPE), (uint32_t)lane);
  };
  const uint32_t sh6 = 8u * (uint32_t)(c >> 1);

  // One K step on the staged X with the weight fragments cur. The B
  // fragments of group g + 1 are read while group g multiplies; within a
  // group the products with hi go before those with lo, so no MFMA waits
  // for the one just issued.
  auto compute = [&](const WFrag<TYPE>(&cur)[RT_PER_WAVE], int buf) {
    const u32x4 *xh = XH(buf), *xl = XL(buf);
    f32x4 cm[RT_PER_WAVE][NCT];
    // The two buffers are separate LDS objects, so the compiler lets these
    // reads run while the next step's global-to-LDS loads into the other
    // buffer are in flight.
    f16x4 sh4[NCT], sl4[NCT];
    if constexpr (TYPE == LGMLH_Q4_K && !Q8) {
      // lanes c >= 2 (k past the 8 groups) read zeros: no branch per step
      const bool gs = c < 2;
      const f16 *gh = (const f16 *)GS(buf) + (gs ? r16 * 8 + 4 * c : 128 * 8);
      const f16 *gl = gh + (gs ? 64 * 8 : 0);
      const int cstride = gs ? 16 * 8 : 0;
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) {
        sh4[ct] = *(const f16x4 *)(gh + ct * cstride);
        sl4[ct] = *(const f16x4 *)(gl + ct * cstride);
      }
    }
    if constexpr (TYPE == LGMLH_Q4_K && Q8) {
      // the 16 sums of 16 q: lane c holds sums 4c .. 4c + 3 of its column
      const f16 *gs = (const f16 *)GS(buf) + (c < 2 ? 0 : 64 * 8) + r16 * 8 + 4 * (c & 1);
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) sh4[ct] = *(const f16x4 *)(gs + ct * 16 * 8);
    }
    uint32_t scb[RT_PER_WAVE][2];
    if constexpr (TYPE == LGMLH_Q4_K) {
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        scb[a][0] = cur[a].sc03();
        scb[a][1] = cur[a].sc47();
      }
    }
    // B fragments: a group's hi (lo) fragments are read right after the
    // previous group's products with hi (lo) are issued.
    f16x8 bh[NCT], bl[NCT];
    auto read_bh = [&](int g) {
      const int slot = r16 * 32 + ((4 * g + c) ^ r16);
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) bh[ct] = __builtin_bit_cast(f16x8, xh[ct * 16 * 32 + slot]);
    };
    auto read_bl = [&](int g) {
      if constexpr (!Q8) {
        const int slot = r16 * 32 + ((4 * g + c) ^ r16);
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) bl[ct] = __builtin_bit_cast(f16x8, xl[ct * 16 * 32 + slot]);
      }
    };
    // Q8_0: d of rows 4c .. 4c + 3 of tile a, block g
    u32x2 dv[RT_PER_WAVE];
    auto read_d = [&](int g) {
      if constexpr (TYPE == LGMLH_Q8_0) {
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++)
          dv[a] = *(const u32x2 *)((const uint8_t *)&HD(buf)[(wave * RT_PER_WAVE + a) * 16] +
                                   64 * c + 8 * g);
      }
    };
    read_bh(0);
    read_bl(0);
    read_d(0);
    f16x2 sp[RT_PER_WAVE], cp[RT_PER_WAVE];  // Q4_K: multipliers of g's pair
#pragma unroll
    for (int g = 0; g < 8; g++) {
      f16x8 af[RT_PER_WAVE], af2[RT_PER_WAVE], afr[RT_PER_WAVE];
      if constexpr (TYPE == LGMLH_Q4_K) {
        if ((g & 1) == 0) {
#pragma unroll
          for (int a = 0; a < RT_PER_WAVE; a++) cur[a].pair(g >> 1, scb[a][g >> 2], sp[a], cp[a]);
        }
      }
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        if constexpr (TYPE == LGMLH_Q4_K)
          af[a] = cur[a].frag(g, sp[a], cp[a]);
        else if constexpr (TYPE == LGMLH_Q6_K)
          cur[a].frag(g, sh6, af[a], af2[a], afr[a]);  // afr unused with Q8
        else
          af[a] = cur[a].frag(g);
      }
      // the first product of a K step (of a block for Q8_0) starts from 0
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
          const f32x4 c0 = (g == 0 || TYPE == LGMLH_Q8_0) ? f32x4{0, 0, 0, 0} : cm[a][ct];
          cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bh[ct], c0, 0, 0, 0);
        }
      if constexpr (TYPE == LGMLH_Q6_K) {
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
          for (int ct = 0; ct < NCT; ct++)
            cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af2[a], bh[ct], cm[a][ct], 0, 0, 0);
      }
      if (g < 7) read_bh(g + 1);
      if constexpr (!Q8) {
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
          for (int ct = 0; ct < NCT; ct++)
            cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                TYPE == LGMLH_Q6_K ? afr[a] : af[a], bl[ct], cm[a][ct], 0, 0, 0);
        if (g < 7) read_bl(g + 1);
      }
      u32x2 dg[RT_PER_WAVE];
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) dg[a] = dv[a];
      if (g < 7) read_d(g + 1);
      if constexpr (TYPE == LGMLH_Q8_0) {
        // one scale per 32-value block: flush every group (Q8: times the
        // column's d of the block, (d_w d_x) I as ggml's q8_0 dot)
        float dxg[NCT];
        if constexpr (Q8) {
#pragma unroll
          for (int ct = 0; ct < NCT; ct++)
            dxg[ct] = DX(buf)[(g >> 2) * 256 + (ct * 16 + r16) * 4 + (g & 3)];
        }
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float d = h2f((uint16_t)(dg[a][i >> 1] >> (16 * (i & 1))));
#pragma unroll
            for (int ct = 0; ct < NCT; ct++) {
              if constexpr (Q8)
                acc[a][ct][i] = fmaf(d * dxg[ct], cm[a][ct][i], acc[a][ct][i]);
              else
                acc[a][ct][i] += d * cm[a][ct][i];
            }
          }
        }
        // pin the flush here: left free, the compiler sinks every group's
        // flush to the end of the step, keeping 8 groups of products live
        // (spills)
#pragma unroll
        for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
          for (int ct = 0; ct < NCT; ct++) asm volatile("" : "+v"(acc[a][ct]));
      }
    }
    // Q8 (Q8_K): the column's d of this K step
    float dxs[NCT];
    if constexpr (Q8 && TYPE != LGMLH_Q8_0) {
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) dxs[ct] = DX(buf)[ct * 16 + r16];
    }
    if constexpr (TYPE == LGMLH_Q4_K) {
      // min term: sum_g m_g * S_g[n] as a 16x16x16 MFMA over the 8 groups
      // (Q8: over the 16 sums of 16 q)
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
        const f16x4 am = Q8 ? cur[a].mins16(c) : cur[a].mins(c);
        float dd[4], dm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          dd[i] = h2f((uint16_t)cur[a].dm[i]);
          dm[i] = h2f((uint16_t)(cur[a].dm[i] >> 16));
        }
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
          f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x16f16(am, sh4[ct], f32x4{0, 0, 0, 0}, 0, 0, 0);
          if constexpr (!Q8) {
            mn = __builtin_amdgcn_mfma_f32_16x16x16f16(am, sl4[ct], mn, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc[a][ct][i] = fmaf(-dm[i], mn[i], fmaf(dd[i], cm[a][ct][i], acc[a][ct][i]));
          } else {
            // d_x (d_w I - dmin_w Mn): I and Mn are exact integers
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc[a][ct][i] = fmaf(dxs[ct], fmaf(dd[i], cm[a][ct][i], -(dm[i] * mn[i])),
                                   acc[a][ct][i]);
          }
        }
      }
    } else if constexpr (TYPE == LGMLH_Q6_K) {
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          // the fragments carry sc * q / 4
          const float d4 = 4.0f * h2f((uint16_t)(cur[a].d4[i >> 1] >> (16 * (i & 1))));
#pragma unroll
          for (int ct = 0; ct < NCT; ct++) {
            if constexpr (Q8)
              acc[a][ct][i] = fmaf(d4 * dxs[ct], cm[a][ct][i], acc[a][ct][i]);
            else
              acc[a][ct][i] += d4 * cm[a][ct][i];
          }
        }
      }
    }
  };

  // Step sb: the loads of sb + 1 (weights into the other register set, X
  // straight into the other LDS buffer) go out first, compute runs on sb,
  // then one barrier publishes the new X.
  WFrag<TYPE> w0[RT_PER_WAVE], w1[RT_PER_WAVE];
  const uint32_t nsteps = (uint32_t)(sb_hi - sb_lo);
  // The next step's loads go out unconditionally (the last step reloads
  // its own chunk and X, still in L2): straight-line code keeps the load
  // counter waits exact, so compute never waits for the next step's data.
  auto step = [&](uint32_t k, const WFrag<TYPE>(&cur)[RT_PER_WAVE],
                  WFrag<TYPE>(&nxt)[RT_PER_WAVE], int buf) {
    const uint32_t kn = k + 1 < nsteps ? k + 1 : k;
    load_w(nxt, kn);
    if constexpr (ONEBUF) {
      // one buffer: the next step's X goes in once every wave has read it
      compute(cur, 0);
      __syncthreads();
      load_x(kn, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    } else {
      load_x(kn, buf ^ 1);
      compute(cur, buf);
      __builtin_amdgcn_s_waitcnt(0);  // this wave's X loads have landed in LDS
      __syncthreads();                // ... and everyone's; buffer buf is free again
    }
  };
  if (nsteps > 0) {
    load_w(w0, 0);
    load_x(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // acc[a][ct][i] = Y[n0 + ct*16 + lane%16][(rt0+a)*16 + 4*(lane/16) + i]
  // (GATHER: Y row = the pick of column ct*16 + lane%16)
  float *const out = nz == 1 ? y : part + (int64_t)z * N * M;
  const int64_t ld_out = nz == 1 ? ldy : M;
  // The first split of a folded pair waits in part (y may be the
  // residual). Compiled for the wide Q4_K / Q6_K tiles only: elsewhere the
  // registers it holds would spill.
  constexpr bool CAN_FOLD = NCT == 4 && !GATHER && TYPE != LGMLH_Q8_0;
  float *const pair = CAN_FOLD ? part + (int64_t)z * N * M : nullptr;
  // A lane's 4 values are consecutive rows of one output column: one
  // 16-byte store when the layout allows (4-byte stores spread over 16
  // columns cost the launch about 6 us more). add: the sum is the pair's
  // first split (each lane reads back only what it stored) + acc; res: the
  // residual goes on last.
  auto emit = [&](float *dst, int64_t ld, bool add, bool res) {
    const bool vec = (ld & 3) == 0 && ((uintptr_t)dst & 15) == 0 &&
                     (!add || ((M & 3) == 0 && ((uintptr_t)pair & 15) == 0)) &&
                     (!res || ((ldy & 3) == 0 && ((uintptr_t)residual & 15) == 0));
#pragma unroll
    for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) {
        int64_t n = n0 + ct * 16 + r16;
        int64_t m = (rt0 + a) * 16 + 4 * c;
        if constexpr (GATHER) {
          if (ct * 16 + r16 >= count) continue;
          n = gt.sorted[first + ct * 16 + r16];
        } else if (n >= N) {
          continue;
        }
        if (vec && m + 3 < M) {
          f32x4 v = acc[a][ct];
          if (add) v = *(volatile f32x4 *)(pair + n * M + m) + v;
          if (res) v += *(const f32x4 *)(residual + n * ldy + m);
          *(f32x4 *)(dst + n * ld + m) = v;
          continue;
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (m + i < M) {
            float v = acc[a][ct][i];
            if (add) v = *(volatile float *)(pair + n * M + m + i) + v;
            if (res) v += residual[n * ldy + m + i];
            dst[n * ld + m + i] = v;
          }
      }
  };
  // A folded pair: the first split's sum is stored at its last step and
  // the accumulators start again from 0, so each split is the same sum as
  // in a workgroup of its own.
  const uint32_t split_end =
      CAN_FOLD && fold > 1 && nsteps > (uint32_t)sb_per_split ? sb_per_split : 0;
  auto boundary = [&](uint32_t k) {
    if (CAN_FOLD && k + 1 == split_end) {
      emit(pair, M, false, false);
#pragma unroll
      for (int a = 0; a < RT_PER_WAVE; a++)
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) acc[a][ct] = f32x4{0, 0, 0, 0};
    }
  };
  for (uint32_t k = 0; k < nsteps; k += 2) {
    step(k, w0, w1, 0);
    boundary(k);
    if (k + 1 < nsteps) {
      step(k + 1, w1, w0, 1);
      boundary(k + 1);
    }
  }
  if (CAN_FOLD && split_end)
    emit(out, ld_out, true, nz == 1 && residual);
  else
    emit(out, ld_out, false, nz == 1 && residual);
}

// ---- decode-sized products: the weights stream through LDS ----------------------
// At N <= 64 columns in ggml arithmetic, qstream_kernel keeps two K steps of
// weights in flight per wave at all times: they travel by global-to-LDS
// loads (no registers held) into a ring of two LDS stages per wave; at each
// step boundary a wave reads the next step's weights from the ring into
// registers and sends the loads of the step after next into the stage it
// just read. X is double-buffered in LDS as in qgemm_kernel. A wave waits
// for its own loads of the next step only (s_waitcnt vmcnt leaving the
// younger loads of the step after in flight), then one barrier publishes
// the next step's X. (qgemm_kernel waits for every load in flight at each
// step, the next step's weights included.)
//
// One workgroup of 8 waves per CU, one 16-row tile per wave (LDS at 64
// columns: Q4_K 106.5 KB, Q6_K 117 KB, Q8_0 136 KB). Measured on the
// MI355X, the kernel is bound by issue, not by its bytes: a copy with its
// loads taken out runs as long, and the fragment builds and scale flushes
// (about 4.5 VALU instructions per MFMA) co-issue with the MFMAs only in
// part. Each 16-row tile takes the fragments, MFMAs, K steps, split ranges
// and scale flushes of qgemm_kernel's ggml mode in the same order, so a
// product gives the same bits through either kernel.
// Workgroup shape: WV waves of R row tiles each.
__host__ __device__ constexpr int qs_waves(int type) { return 8; }
__host__ __device__ constexpr int qs_rt(int type) { return 1; }
// One wave's stage: the chunk headers of its tiles (16-byte slots), then
// each tile's lane data as planes of 64 x 16 B (plane p holds bytes 16 p ..
// 16 p + 15 of every lane's record, so a lane's 16-byte read of a plane is
// conflict-free).
__host__ __device__ constexpr int qs_hslots(int type) { return chunk_hdr(type) / 16; }
__host__ __device__ constexpr int qs_planes(int type) { return lane_bytes(type) / 16; }
__host__ __device__ constexpr int qs_stage_slots(int type, int R) {
  return R * (qs_hslots(type) + 64 * qs_planes(type));
}

// s_waitcnt with only the vector-memory counter (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt and lgkmcnt at their maxima).
#define LGMLH_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// A workgroup barrier that waits for nothing itself: __syncthreads()'s
// fence would wait for every load in flight (vmcnt(0)), the younger
// weight loads included. The global-to-LDS loads a barrier publishes are
// waited for before it with LGMLH_WAIT_VMCNT; the empty asm statements
// keep the compiler from moving memory operations across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Global-to-LDS loads of 16 (4) bytes per lane into lds + 16 (4) * lane,
// issued as inline assembly. The compiler's wait insertion tells such
// loads' targets apart only for a few LDS objects with precise alias
// information; here, where it cannot, it would wait for every load in
// flight before each LDS read. qstream_kernel waits for its loads itself
// (LGMLH_WAIT_VMCNT, then a barrier), and the compiler's own waits for
// other memory operations stay correct: these loads only add to the
// counter it waits on.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void *g, const void *lds) {
  const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)lds;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(g), "s"(l) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void *g, const void *lds) {
  const uint32_t l = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)lds;
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(g), "s"(l) : "memory", "m0");
}
#pragma clang diagnostic pop

// A wave's weights of one K step for R row tiles (chunks at wt[a] + ko)
// into its stage region `mine`: the R * HS header slots (64 per load), then
// R * NP planes. stage_loads() global-to-LDS loads per wave.
template <int TYPE, int R>
__host__ __device__ constexpr int stage_loads() {
  return (R * qs_hslots(TYPE) + 63) / 64 + R * qs_planes(TYPE);
}
template <int TYPE, int R>
__device__ __forceinline__ void stage_w(const uint8_t *const (&wt)[R], uint32_t ko, u32x4 *mine,
                                        int lane) {
  constexpr int HS = qs_hslots(TYPE), NP = qs_planes(TYPE), NHI = (R * HS + 63) / 64;
#pragma unroll
  for (int h = 0; h < NHI; h++) {
    const int sl = 64 * h + lane;
    if (sl < R * HS) {
      const int a = R == 1 ? 0 : sl / HS;
      lds_dma16(wt[a] + ko + 16 * (sl - a * HS), mine + 64 * h);
    }
  }
#pragma unroll
  for (int a = 0; a < R; a++)
#pragma unroll
    for (int p = 0; p < NP; p++)
      lds_dma16(wt[a] + ko + chunk_hdr(TYPE) + lane * lane_bytes(TYPE) + 16 * p,
                mine + R * HS + (a * NP + p) * 64);
}
// The WFrag fields of R tiles from a stage region (Q8_0 also the d of the
// lane's rows, 8 blocks: bytes 64 c .. 64 c + 63 of the header, into q8d).
template <int TYPE, int R>
__device__ __forceinline__ void read_stage(const u32x4 *mine, int lane, WFrag<TYPE> (&cur)[R],
                                           u32x4 (&q8d)[R][4]) {
  constexpr int HS = qs_hslots(TYPE), NP = qs_planes(TYPE);
  const int c = lane >> 4, r16 = lane & 15;
#pragma unroll
  for (int a = 0; a < R; a++) {
    const u32x4 *hdr = mine + a * HS, *pl = mine + R * HS + a * NP * 64 + lane;
    if constexpr (TYPE == LGMLH_Q4_K) {
      cur[a].dm = hdr[c];
      const uint32_t *sp = (const uint32_t *)hdr + 16 + 3 * r16;
      cur[a].s0 = sp[0];
      cur[a].s1 = sp[1];
      cur[a].s2 = sp[2];
      cur[a].qs[0] = pl[0];
      cur[a].qs[1] = pl[64];
    } else if constexpr (TYPE == LGMLH_Q6_K) {
      cur[a].d4 = ((const u32x2 *)hdr)[c];
      cur[a].scl = hdr[2 + r16];
      cur[a].ql[0] = pl[0];
      cur[a].ql[1] = pl[64];
      cur[a].qh = pl[128];
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        cur[a].qs[i] = pl[64 * i];
        q8d[a][i] = hdr[4 * c + i];
      }
    }
  }
}

template <int TYPE, int NCT, int WV, int R>
__global__ void __launch_bounds__(WV * 64, 1)
qstream_kernel(const uint8_t *__restrict__ w, int64_t M, int64_t K, const f16 *__restrict__ xs,
               int64_t Npad, int64_t N, float *__restrict__ y, int64_t ldy,
               const float *__restrict__ residual, int nz, int sb_per_split,
               float *__restrict__ part) {
  constexpr int SS = qs_stage_slots(TYPE, R);  // slots of one wave's stage
  constexpr int COLS = NCT * 16, X_SLOTS = COLS * 32;
  constexpr int DX_SLOTS = TYPE == LGMLH_Q8_0 ? 128 : 16;
  constexpr int GS_SLOTS = TYPE == LGMLH_Q4_K ? 128 : 1;
  // Two weight stages and two X buffers, each of the latter holding the q
  // slots, then (Q4_K) the sums of 16 q, then the d.
  constexpr int XB_SLOTS = X_SLOTS + GS_SLOTS + DX_SLOTS;
  __shared__ __align__(16) u32x4 ws0_[WV * SS], ws1_[WV * SS];
  __shared__ __align__(16) u32x4 x0_[XB_SLOTS], x1_[XB_SLOTS];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane >> 4, r16 = lane & 15;
  const int64_t NSB = K / QK_K, MT = (M + 15) / 16;
  const int z = (int)blockIdx.y;
  const int64_t sb_lo = (int64_t)z * sb_per_split;
  const int64_t sb_hi = sb_lo + sb_per_split < NSB ? sb_lo + sb_per_split : NSB;
  const uint32_t nsteps = (uint32_t)(sb_hi - sb_lo);
  const int64_t rt0 = ((int64_t)blockIdx.x * WV + wave) * R;
  const uint8_t *wt[R];
#pragma unroll
  for (int a = 0; a < R; a++) {
    const int64_t rt = rt0 + a < MT ? rt0 + a : MT - 1;  // computed, never stored
    wt[a] = w + (rt * NSB + sb_lo) * chunk_bytes(TYPE);
  }
  // X: the plane slots as qgemm_kernel stages them (piece kp of column n at
  // slot n * 32 + (kp ^ (n & 15))), XJ loads of 64 slots per wave
  // (with fewer slots than lanes, the first X_SLOTS / 64 waves load one each)
  constexpr int XJ = X_SLOTS >= WV * 64 ? X_SLOTS / (WV * 64) : 1;
  static_assert(X_SLOTS >= WV * 64 ? XJ * WV * 64 == X_SLOTS : X_SLOTS % 64 == 0,
                "X slots per wave");
  const f16 *xq = xs + sb_lo * QK_K;
  constexpr int QB = TYPE == LGMLH_Q8_0 ? 32 : QK_K;
  const f16 *bsp = xs + q8_bs_off(Npad, K) + sb_lo * 16;
  const float *dxp =
      (const float *)((const char *)xs + q8_d_off(Npad, K)) + sb_lo * (QK_K / QB);
  uint32_t xoff[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const int sl = (wave * XJ + j) * 64 + lane, n = sl >> 5, kp = (sl & 31) ^ (n & 15);
    xoff[j] = (uint32_t)(n * K + kp * 8) * 2u;
  }
  const int64_t xr_lane = lane < COLS ? lane : 0;  // gs / d: lane = column
  const uint32_t goff = (uint32_t)(xr_lane * (K / 16)), doff = (uint32_t)(xr_lane * (K / QB));

  auto load_x = [&](uint32_t kstep, u32x4 *xb) __attribute__((always_inline)) {
    u32x4 *gb = xb + X_SLOTS, *db = xb + X_SLOTS + GS_SLOTS;
#pragma unroll
    for (int j = 0; j < XJ; j++)
      if (X_SLOTS >= WV * 64 || wave < X_SLOTS / 64)
        lds_dma16((const uint8_t *)(xq + kstep * QK_K) + xoff[j], &xb[(wave * XJ + j) * 64]);
    if constexpr (TYPE == LGMLH_Q4_K) {
      if (wave < 2)  // the 16 sums of 16 q: wave 0 sums 0..7, wave 1 8..15
        lds_dma16(bsp + goff + kstep * 16 + 8 * wave, gb + 64 * wave);
    }
    if constexpr (TYPE != LGMLH_Q8_0) {
      if (wave == 2)  // the Q8_K d of each column
        lds_dma4(dxp + doff + kstep, db);
    } else {
      if (wave < 2)  // the d of blocks 4 wave .. 4 wave + 3 of each column
        lds_dma16(dxp + doff + kstep * 8 + 4 * wave, db + 64 * wave);
    }
  };
  constexpr int NWI = stage_loads<TYPE, R>();  // weight loads per wave and step
  auto load_w = [&](uint32_t kstep, u32x4 *stage) __attribute__((always_inline)) {
    stage_w<TYPE, R>(wt, kstep * (uint32_t)chunk_bytes(TYPE), stage + wave * SS, lane);
  };
  // Registers of the step being computed.
  WFrag<TYPE> cur[R];
  u32x4 q8d[R][4];
  auto read_w = [&](const u32x4 *stage) __attribute__((always_inline)) {
    read_stage<TYPE, R>(stage + wave * SS, lane, cur, q8d);
  };

  f32x4 acc[R][NCT];
#pragma unroll
  for (int a = 0; a < R; a++)
#pragma unroll
    for (int b = 0; b < NCT; b++) acc[a][b] = f32x4{0, 0, 0, 0};
  const uint32_t sh6 = 8u * (uint32_t)(c >> 1);

  // One K step on registers cur and the X buffers (qgemm_kernel's ggml
  // mode: one MFMA per group and tile on the integer q; Q6_K the two exact
  // parts; Q8_0 a flush per block; Q4_K / Q6_K the scales per step).
  auto compute = [&](const u32x4 *xb) __attribute__((always_inline)) {
    const u32x4 *gb = xb + X_SLOTS, *db = xb + X_SLOTS + GS_SLOTS;
    const float *dxf = (const float *)db;
    f32x4 cm[R][NCT];
    f16x4 sh4[NCT];
    if constexpr (TYPE == LGMLH_Q4_K) {
      const f16 *gsr = (const f16 *)gb + (c < 2 ? 0 : 64 * 8) + r16 * 8 + 4 * (c & 1);
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) sh4[ct] = *(const f16x4 *)(gsr + ct * 16 * 8);
    }
    uint32_t scb[R][2];
    if constexpr (TYPE == LGMLH_Q4_K) {
#pragma unroll
      for (int a = 0; a < R; a++) {
        scb[a][0] = cur[a].sc03();
        scb[a][1] = cur[a].sc47();
      }
    }
    f16x8 bh[NCT];
    auto read_bh = [&](int g) __attribute__((always_inline)) {
      const int slot = r16 * 32 + ((4 * g + c) ^ r16);
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) bh[ct] = __builtin_bit_cast(f16x8, xb[ct * 16 * 32 + slot]);
    };
    read_bh(0);
    f16x2 sp[R], cp[R];
#pragma unroll
    for (int g = 0; g < 8; g++) {
      f16x8 af[R], af2[R], afr[R];
      if constexpr (TYPE == LGMLH_Q4_K) {
        if ((g & 1) == 0) {
#pragma unroll
          for (int a = 0; a < R; a++) cur[a].pair(g >> 1, scb[a][g >> 2], sp[a], cp[a]);
        }
      }
#pragma unroll
      for (int a = 0; a < R; a++) {
        if constexpr (TYPE == LGMLH_Q4_K)
          af[a] = cur[a].frag(g, sp[a], cp[a]);
        else if constexpr (TYPE == LGMLH_Q6_K)
          cur[a].frag(g, sh6, af[a], af2[a], afr[a]);  // afr unused
        else
          af[a] = cur[a].frag(g);
      }
#pragma unroll
      for (int a = 0; a < R; a++)
#pragma unroll
        for (int ct = 0; ct < NCT; ct++) {
          const f32x4 c0 = (g == 0 || TYPE == LGMLH_Q8_0) ? f32x4{0, 0, 0, 0} : cm[a][ct];
          cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bh[ct], c0, 0, 0, 0);
        }
      if constexpr (TYPE == LGMLH_Q6_K) {
#pragma unroll
        for (int a = 0; a < R; a++)
#pragma unroll
          for (int ct = 0; ct < NCT; ct++)
            cm[a][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af2[a], bh[ct], cm[a][ct], 0, 0, 0);
      }
      if (g < 7) read_bh(g + 1);
      if constexpr (TYPE == LGMLH_Q8_0) {
        float dxg[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ct++)
          dxg[ct] = dxf[(g >> 2) * 256 + (ct * 16 + r16) * 4 + (g & 3)];
#pragma unroll
        for (int a = 0; a < R; a++) {
          const uint32_t dlo = q8d[a][g >> 1][2 * (g & 1)], dhi = q8d[a][g >> 1][2 * (g & 1) + 1];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float d = h2f((uint16_t)((i < 2 ? dlo : dhi) >> (16 * (i & 1))));
#pragma unroll
            for (int ct = 0; ct < NCT; ct++)
              acc[a][ct][i] = fmaf(d * dxg[ct], cm[a][ct][i], acc[a][ct][i]);
          }
        }
#pragma unroll
        for (int a = 0; a < R; a++)
#pragma unroll
          for (int ct = 0; ct < NCT; ct++) asm volatile("" : "+v"(acc[a][ct]));
      }
    }
    if constexpr (TYPE != LGMLH_Q8_0) {
      float dxs[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ct++) dxs[ct] = dxf[ct * 16 + r16];
      if constexpr (TYPE == LGMLH_Q4_K) {
#pragma unroll
        for (int a = 0; a < R; a++) {
          const f16x4 am = cur[a].mins16(c);
          float dd[4], dm[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            dd[i] = h2f((uint16_t)cur[a].dm[i]);
            dm[i] = h2f((uint16_t)(cur[a].dm[i] >> 16));
          }
#pragma unroll
          for (int ct = 0; ct < NCT; ct++) {
            const f32x4 mn =
                __builtin_amdgcn_mfma_f32_16x16x16f16(am, sh4[ct], f32x4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
              acc[a][ct][i] = fmaf(dxs[ct], fmaf(dd[i], cm[a][ct][i], -(dm[i] * mn[i])),
                                   acc[a][ct][i]);
          }
        }
      } else {
#pragma unroll
        for (int a = 0; a < R; a++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float d4 = 4.0f * h2f((uint16_t)(cur[a].d4[i >> 1] >> (16 * (i & 1))));
#pragma unroll
            for (int ct = 0; ct < NCT; ct++)
              acc[a][ct][i] = fmaf(d4 * dxs[ct], cm[a][ct][i], acc[a][ct][i]);
          }
      }
    }
  };

  // Step k (buffers of parity P = k % 2): compute on cur; then wait for this
  // wave's loads of step k + 1 (the loads of k + 2 stay in flight), a
  // barrier (everyone's X of k + 1 has landed, everyone is done with the X
  // of k), read the weights of k + 1, and send the loads of X k + 2 and of
  // the weights of k + 3 (into the stage just read).
  auto step = [&](uint32_t k, int P) __attribute__((always_inline)) {
    u32x4 *xb = P ? x1_ : x0_;
    u32x4 *wn = P ? ws0_ : ws1_;  // the stage of k + 1 (and k + 3)
    compute(xb);
    if (k + 1 >= nsteps) return;
    if (k + 2 < nsteps) {
      LGMLH_WAIT_VMCNT(NWI);
    } else {
      LGMLH_WAIT_VMCNT(0);
    }
    lds_barrier();
    read_w(wn);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the stage is read before it is reloaded
    if (k + 2 < nsteps) load_x(k + 2, xb);
    if (k + 3 < nsteps) load_w(k + 3, wn);
  };
  if (nsteps > 0) {
    load_x(0, x0_);
    load_w(0, ws0_);
    if (nsteps > 1) {
      load_w(1, ws1_);
      LGMLH_WAIT_VMCNT(NWI);
    } else {
      LGMLH_WAIT_VMCNT(0);
    }
    lds_barrier();
    read_w(ws0_);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    if (nsteps > 1) load_x(1, x1_);
    if (nsteps > 2) load_w(2, ws0_);
  }
  for (uint32_t k = 0; k < nsteps; k += 2) {
    step(k, 0);
    if (k + 1 < nsteps) step(k + 1, 1);
  }

  // acc[a][ct][i] = Y[ct * 16 + r16][(rt0 + a) * 16 + 4 c + i]
  float *const out = nz == 1 ? y : part + (int64_t)z * N * M;
  const int64_t ld = nz == 1 ? ldy : M;
  const bool res = nz == 1 && residual;
  const bool vec = (ld & 3) == 0 && ((uintptr_t)out & 15) == 0 &&
                   (!res || ((ldy & 3) == 0 && ((uintptr_t)residual & 15) == 0));
#pragma unroll
  for (int a = 0; a < R; a++)
#pragma unroll
    for (int ct = 0; ct < NCT; ct++) {
      const int64_t n = ct * 16 + r16, m = (rt0 + a) * 16 + 4 * c;
      if (n >= N) continue;
      if (vec && m + 3 < M) {
        f32x4 v = acc[a][ct];
        if (res) v += *(const f32x4 *)(residual + n * ldy + m);
        *(f32x4 *)(out + n * ld + m) = v;
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (m + i < M) {
          float v = acc[a][ct][i];
          if (res) v += residual[n * ldy + m + i];
          out[n * ld + m + i] = v;
        }
    }
}

// The partial sums of a split-K product, added in the canonical order
// (Pending::sum): pairs of splits, then the pairs in order, then the
// residual.
__global__ void splitk_reduce_kernel(Pending pd, float *__restrict__ y, int64_t ldy,
                                     const float *__restrict__ residual) {
  const int64_t total = pd.rows * pd.cols, M = pd.cols;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    int64_t n = e / M, m = e % M;
    float v = pd.sum(n, m);
    if (residual) v += residual[n * ldy + m];
    y[n * ldy + m] = v;
  }
}

// X (f32 or f16 rows of K) -> planes of the form xf; one thread per 8 values
// (the lanes of a 256-value block are consecutive and leave together).
__global__ void xsplit_kernel(const void *__restrict__ x, int xtype, int64_t N, int64_t K,
                              f16 *__restrict__ planes, int64_t Npad, int xf) {
  const int64_t per_row = K / 8;  // a multiple of 32: groups never straddle rows
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= N * per_row) return;   // whole groups of 4 lanes leave together
  const int64_t n = t / per_row, k0 = (t % per_row) * 8;
  float v[8];
  if (xtype == LGMLH_F32) {
    const f32x4 *p = (const f32x4 *)((const float *)x + n * K + k0);
    f32x4 a = p[0], b = p[1];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  } else {
    f16x8 h = *(const f16x8 *)((const f16 *)x + n * K + k0);
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (float)h[e];
  }
  act_store8(xf, planes, Npad, K, n, k0, v);
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
// the same sum in the same order for any batch size. Returns the number of
// splits (each of sb_per_split K steps, the last may be shorter). Their
// sums add up in a fixed association: consecutive pairs (SPLIT_PAIR) first,
// then the pairs in order, so that a workgroup may run both splits of a
// pair itself (see launch_q) with the same result.
constexpr int SPLIT_PAIR = 2;
constexpr int SPLIT_ROWS = 128;  // the row unit of the split count
int splits_for(int64_t M, int64_t K, int64_t N, int *sb_per_split = nullptr) {
  (void)N;
  const int64_t NSB = K / QK_K;
  const int64_t tiles = (M + SPLIT_ROWS - 1) / SPLIT_ROWS;
  // About one workgroup of SPLIT_ROWS rows per CU (256), at least 2 K steps
  // per split so the pipeline has a step to overlap.
  int64_t want = (256 + tiles / 2) / tiles;
  const int64_t maxs = NSB / 2 > 1 ? NSB / 2 : 1;
  if (want > maxs) want = maxs;
  if (want < 1) want = 1;
  const int64_t spb = (NSB + want - 1) / want;
  if (sb_per_split) *sb_per_split = (int)spb;
  return (int)((NSB + spb - 1) / spb);
}

// Split-K partial sums of a call (0 when K is not split).
size_t partial_bytes(int type, int64_t M, int64_t K, int64_t N) {
  if (type == LGMLH_F32) return 0;
  int s = splits_for(M, K, N);
  return s == 1 ? 0 : (size_t)s * N * M * 4;
}

static size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

size_t workspace_for(int type, int64_t M, int64_t K, int64_t N) {
  if (type == LGMLH_F32) return 0;
  return align256(split_bytes(N, K)) + partial_bytes(type, M, K, N);
}

// Launch a quantized product; returns the partials it leaves in part (0:
// the product is in y) and, in *group, how many consecutive partials make a
// pair sum (2: one per split; 1: one per folded pair).
template <int TYPE, bool Q8>
static int launch_q(const void *w, int64_t M, int64_t K, const f16 *xs, int64_t N, float *y,
                    int64_t ldy, const float *res, float *part, bool defer, hipStream_t st,
                    int *group) {
  int spb = 0;
  const int splits = splits_for(M, K, N, &spb);
  const int64_t Npad = split_npad(N);
  if constexpr (Q8) {
    if (N <= 64) {  // decode-sized: the streamed-weight kernel, unfolded splits
      constexpr int WV = qs_waves(TYPE), R = qs_rt(TYPE);
      const int wrows = WV * R * 16;
      dim3 grid((unsigned)((M + wrows - 1) / wrows), (unsigned)splits);
#define LGMLH_STREAM(NCT_)                                                                  \
  hipLaunchKernelGGL((qstream_kernel<TYPE, NCT_, WV, R>), grid, dim3(WV * 64), 0, st,       \
                     (const uint8_t *)w, M, K, xs, Npad, N, y, ldy, res, splits, spb, part)
      if (N <= 16)
        LGMLH_STREAM(1);
      else if (N <= 32)
        LGMLH_STREAM(2);
      else
        LGMLH_STREAM(4);
#undef LGMLH_STREAM
      *group = SPLIT_PAIR;
      if (splits > 1 && !defer) {
        int64_t total = N * M;
        unsigned blocks = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
        Pending pd{part, splits, N, M};
        pd.group = SPLIT_PAIR;
        hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, pd, y, ldy, res);
      }
      return splits > 1 ? splits : 0;
    }
  }
  // Column tiles of 64, or of 16 / 32 for a batch that small (the same sums
  // per element: only the columns a workgroup carries change). A decode-
  // sized product (N <= 64) with fewer than 200 workgroups of rows and
  // splits takes tiles of 16: more workgroups, and for Q4_K / Q6_K two per
  // CU (C5's dense products 6.81 -> 6.49 ms per step, C4's Q8_0 ones 1.96
  // -> 1.85; at 256, C2's gate|up, 224 workgroups, lost 20%). A prefill-
  // sized batch keeps wide tiles, so each weight fragment is dequantized
  // once for 64 columns. Q4_K's wide tiles run two 4-wave workgroups per
  // CU themselves, so for Q4_K the bound is 100 (C2's q|k|v and wo at 160
  // and 128: decode +1.2%).
  int nct = N <= 16 ? 1 : N <= 32 ? 2 : WG_COLS / 16;
  const int64_t small_wg = TYPE == LGMLH_Q4_K ? 100 : 200;
  if (N <= 64 && (int64_t)((M + WG_ROWS - 1) / WG_ROWS) * splits < small_wg) nct = 1;
  const int cols = 16 * nct;
  const int wrows = gemm_waves(TYPE, nct, Q8) * RT_PER_WAVE * 16;  // rows per workgroup
  const int64_t tiles = ((N + cols - 1) / cols) * ((M + wrows - 1) / wrows);
  // With 8192 workgroups or more (16 rounds of two per CU), a workgroup
  // runs both splits of a pair: half the partial sums (none for a product
  // of two splits) to write and read back. Same sums either way. Below
  // that, one split per workgroup finishes sooner, and that outweighs the
  // consumers' reads of twice the partials (C2's 512-token prefill pass:
  // products 16.1 -> 15.2 ms, the rms_norm and rope consumers 1.85 ->
  // 2.29 ms, the pass 0.4 ms shorter than with pairs from 512 tiles).
  const int fold =
      splits > 1 && nct == 4 && TYPE != LGMLH_Q8_0 && tiles * splits >= 8192 ? SPLIT_PAIR : 1;
  const int nz = (splits + fold - 1) / fold;
  *group = fold == 1 ? SPLIT_PAIR : 1;
  dim3 grid((unsigned)((N + cols - 1) / cols), (unsigned)((M + wrows - 1) / wrows),
            (unsigned)nz);
#define LGMLH_PLAIN(NCT_)                                                                  \
  hipLaunchKernelGGL((qgemm_kernel<TYPE, NCT_, false, Q8>), grid, dim3(gemm_waves(TYPE, NCT_, Q8) * 64), \
                     0, st,                                                                \
                     (const uint8_t *)w, M, K, xs, Npad, N, y, ldy, res, nz, spb, fold,    \
                     part, Gather{})
  if (nct == 1)
    LGMLH_PLAIN(1);
  else if (nct == 2)
    LGMLH_PLAIN(2);
  else
    LGMLH_PLAIN(4);
#undef LGMLH_PLAIN
  if (nz > 1 && !defer) {
    int64_t total = N * M;
    unsigned blocks = (unsigned)((total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096);
    Pending pd{part, nz, N, M};
    pd.group = *group;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, st, pd, y, ldy, res);
  }
  return nz > 1 ? nz : 0;
}

// The X form a quantized product takes: the split planes (exact), or in
// ggml's arithmetic the weight type's vec_dot_type (Q8_K / Q8_0).
int xf_for(int type, int act) {
  if (act != LGMLH_ACT_GGML || type == LGMLH_F32) return XF_SPLIT;
  return type == LGMLH_Q8_0 ? XF_Q80 : XF_Q8K;
}

// Quantized product on X planes in the form xf (split.h, N rows of K):
// XF_SPLIT, or xf_for(type, LGMLH_ACT_GGML). part holds the split-K partial
// sums (partial_bytes). With `deferred` given, a split product leaves its
// partials in part and *deferred describes them (added in the canonical
// order by the consumer, Pending::sum, which also adds the residual);
// otherwise they are reduced here (*deferred stays empty).
int mul_mat_split(int type, const void *w, int64_t M, int64_t K, const f16 *xs, int64_t N,
                  float *y, int64_t ldy, const float *residual, float *part, size_t part_bytes,
                  hipStream_t st, Pending *deferred, int xf) {
  if (deferred) *deferred = Pending{};
  if (xf != XF_SPLIT && xf != xf_for(type, LGMLH_ACT_GGML)) {
    set_error("mul_mat: X form %d does not suit weight type %d", xf, type);
    return LGMLH_EINVAL;
  }
  const bool q8 = xf != XF_SPLIT;
  if (!w || !xs || !y || M <= 0 || K <= 0 || N < 0 || ldy < M || K % QK_K) {
    set_error("mul_mat: bad arguments (M %lld, K %lld)", (long long)M, (long long)K);
    return LGMLH_EINVAL;
  }
  if (N == 0) return LGMLH_OK;
  int splits = splits_for(M, K, N);
  if (splits > 1 && (!part || part_bytes < partial_bytes(type, M, K, N))) {
    set_error("mul_mat: workspace too small for %d K splits", splits);
    return LGMLH_ENOMEM;
  }
  const bool defer = deferred && splits > 1;
  int nz = 0, group = 1;
  switch (type) {
#define LGMLH_Q(T_)                                                                          \
  (q8 ? launch_q<T_, true>(w, M, K, xs, N, y, ldy, residual, part, defer, st, &group)        \
      : launch_q<T_, false>(w, M, K, xs, N, y, ldy, residual, part, defer, st, &group))
    case LGMLH_Q4_K: nz = LGMLH_Q(LGMLH_Q4_K); break;
    case LGMLH_Q6_K: nz = LGMLH_Q(LGMLH_Q6_K); break;
    case LGMLH_Q8_0: nz = LGMLH_Q(LGMLH_Q8_0); break;
#undef LGMLH_Q
    default:
      set_error("mul_mat: type %d not supported", type);
      return LGMLH_EINVAL;
  }
  if (defer && nz > 1) {
    *deferred = Pending{part, nz, N, M};
    deferred->group = group;
  }
  return hip_check(hipGetLastError(), "mul_mat");
}

template <int TYPE, int NCT, bool Q8>
static void launch_grouped(const void *w, int64_t M, int64_t K, const f16 *xs, int64_t Npad,
                           const Gather &gt, int max_tiles, float *y, hipStream_t st) {
  const int NSB = (int)(K / QK_K);
  const int wrows = gemm_waves(TYPE, NCT, Q8) * RT_PER_WAVE * 16;
  dim3 grid((unsigned)max_tiles, (unsigned)((M + wrows - 1) / wrows), 1);
  hipLaunchKernelGGL((qgemm_kernel<TYPE, NCT, true, Q8>), grid, dim3(gemm_waves(TYPE, NCT, Q8) * 64), 0, st,
                     (const uint8_t *)w, M, K, xs, Npad, (int64_t)0, y, M, (const float *)nullptr,
                     1, NSB, 1, (float *)nullptr, gt);
}

// Grouped product (mul_mat_id): for each column tile of the grouping (see
// Gather), Y rows of its picks = expert matrix x X rows, K unsplit. w holds
// n_expert repacked matrices of M rows, expert_bytes apart; xs the split
// planes of the X rows (Npad rows). tile_cols is 16 or 64, the tile width
// the grouping was made for; max_tiles bounds the tiles in use. xf: the
// planes' form (as mul_mat_split).
int mul_mat_grouped(int type, const void *w, int64_t expert_bytes, int64_t M, int64_t K,
                    const f16 *xs, int64_t Npad, int n_used, int U, const int32_t *sorted,
                    const int4 *tiles, const int32_t *n_tiles, int max_tiles, int tile_cols,
                    float *y, hipStream_t st, int xf) {
  if (xf != XF_SPLIT && xf != xf_for(type, LGMLH_ACT_GGML)) {
    set_error("mul_mat_id: X form %d does not suit weight type %d", xf, type);
    return LGMLH_EINVAL;
  }
  const bool q8 = xf != XF_SPLIT;
  if (!w || !xs || !y || M <= 0 || K <= 0 || K % QK_K || (tile_cols != 16 && tile_cols != 64)) {
    set_error("mul_mat_id: bad arguments (M %lld, K %lld)", (long long)M, (long long)K);
    return LGMLH_EINVAL;
  }
  if (max_tiles <= 0) return LGMLH_OK;
  Gather gt;
  gt.sorted = sorted;
  gt.tiles = tiles;
  gt.n_tiles = n_tiles;
  gt.expert_bytes = expert_bytes;
  gt.n_used = n_used;
  gt.U = U;
#define LGMLH_GROUPED(T_)                                                                    \
  (tile_cols == 16                                                                           \
       ? (q8 ? launch_grouped<T_, 1, true>(w, M, K, xs, Npad, gt, max_tiles, y, st)          \
             : launch_grouped<T_, 1, false>(w, M, K, xs, Npad, gt, max_tiles, y, st))        \
       : (q8 ? launch_grouped<T_, 4, true>(w, M, K, xs, Npad, gt, max_tiles, y, st)          \
             : launch_grouped<T_, 4, false>(w, M, K, xs, Npad, gt, max_tiles, y, st)))
  switch (type) {
    case LGMLH_Q4_K: LGMLH_GROUPED(LGMLH_Q4_K); break;
    case LGMLH_Q6_K: LGMLH_GROUPED(LGMLH_Q6_K); break;
    case LGMLH_Q8_0: LGMLH_GROUPED(LGMLH_Q8_0); break;
    default:
      set_error("mul_mat_id: type %d not supported", type);
      return LGMLH_EINVAL;
  }
#undef LGMLH_GROUPED
  return hip_check(hipGetLastError(), "mul_mat_id");
}

// X -> planes of the form xf (xs holds split_bytes(N, K)).
int split_x(const void *x, int xtype, int64_t N, int64_t K, f16 *xs, hipStream_t st, int xf) {
  if (K % QK_K || (xtype != LGMLH_F32 && xtype != LGMLH_F16)) {
    set_error("split: bad arguments");
    return LGMLH_EINVAL;
  }
  int64_t total = N * (K / 8);
  if (total == 0) return LGMLH_OK;
  hipLaunchKernelGGL(xsplit_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x,
                     xtype, N, K, xs, split_npad(N), xf);
  return hip_check(hipGetLastError(), "split");
}

// f32 weights on f32 X.
int mul_mat_f32(const float *w, int64_t M, int64_t K, const float *x, int64_t N, float *y,
                int64_t ldy, const float *residual, hipStream_t st) {
  if (!w || !x || !y || M <= 0 || K <= 0 || N < 0 || ldy < M) {
    set_error("mul_mat: bad arguments");
    return LGMLH_EINVAL;
  }
  if (N == 0) return LGMLH_OK;
  dim3 grid((unsigned)((M + 15) / 16), (unsigned)((N + 15) / 16));
  hipLaunchKernelGGL(f32gemm_kernel, grid, dim3(256), 0, st, w, M, K, x, N, y, ldy, residual);
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

static int mul_mat_entry(int act, int type, const void *w, int64_t M, int64_t K, const void *x,
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
  if (!x || (xtype != LGMLH_F32 && xtype != LGMLH_F16)) {
    set_error("mul_mat: x must be f32 or f16");
    return LGMLH_EINVAL;
  }
  const float *res = epi == LGMLH_EPI_ADD ? residual : nullptr;
  hipStream_t st = as_stream(stream);
  if (type == LGMLH_F32) {
    if (xtype != LGMLH_F32) {
      set_error("mul_mat: f32 weights take f32 x");
      return LGMLH_EINVAL;
    }
    return mul_mat_f32((const float *)w, M, K, (const float *)x, N, y, M, res, st);
  }
  if (K <= 0 || K % QK_K || M <= 0 || N < 0) {
    set_error("mul_mat: bad shape (M %lld, K %lld, N %lld)", (long long)M, (long long)K,
              (long long)N);
    return LGMLH_EINVAL;
  }
  size_t need = workspace_for(type, M, K, N);
  if (!workspace || ws_bytes < need) {
    set_error("mul_mat: workspace of %zu bytes, need %zu", ws_bytes, need);
    return LGMLH_ENOMEM;
  }
  if (N == 0) return LGMLH_OK;
  f16 *xs = (f16 *)workspace;
  size_t xb = align256(split_bytes(N, K));
  const int xf = xf_for(type, act);
  LGMLH_TRY(split_x(x, xtype, N, K, xs, st, xf));
  return mul_mat_split(type, w, M, K, xs, N, y, M, res, (float *)((char *)workspace + xb),
                       ws_bytes - xb, st, nullptr, xf);
}

extern "C" int lgmlh_mul_mat(int type, const void *w, int64_t M, int64_t K, const void *x,
                             int xtype, int64_t N, float *y, int epi, const float *residual,
                             void *workspace, size_t ws_bytes, void *stream) {
  return mul_mat_entry(LGMLH_ACT_EXACT, type, w, M, K, x, xtype, N, y, epi, residual, workspace,
                       ws_bytes, stream);
}

extern "C" int lgmlh_mul_mat_ggml(int type, const void *w, int64_t M, int64_t K, const void *x,
                                  int xtype, int64_t N, float *y, int epi,
                                  const float *residual, void *workspace, size_t ws_bytes,
                                  void *stream) {
  return mul_mat_entry(LGMLH_ACT_GGML, type, w, M, K, x, xtype, N, y, epi, residual, workspace,
                       ws_bytes, stream);
}

// ggml's activation blocks of X (N, K) f32 for a product with weight type
// `type`: Q8_K (q, d, bsums) for Q4_K / Q6_K, Q8_0 (q, d as f16 bits) for
// Q8_0. One thread per 8 values.
__global__ void act_quant_kernel(const float *__restrict__ x, int64_t N, int64_t K, int xf,
                                 int8_t *__restrict__ q, void *__restrict__ d,
                                 int16_t *__restrict__ bsums) {
  const int64_t per_row = K / 8;
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= N * per_row) return;  // whole blocks of lanes leave together
  const int64_t n = t / per_row, k0 = (t % per_row) * 8;
  float v[8], qv[8], dd;
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = x[n * K + k0 + e];
  if (xf == XF_Q8K) {
    float bs;
    q8k_block8(v, qv, dd, bs);
    if ((k0 & 15) == 0) bsums[n * (K / 16) + (k0 >> 4)] = (int16_t)bs;
    if ((k0 & 255) == 0) ((float *)d)[n * (K / 256) + (k0 >> 8)] = dd;
  } else {
    uint16_t dh;
    q80_block8(v, qv, dd, dh);
    if ((k0 & 31) == 0) ((uint16_t *)d)[n * (K / 32) + (k0 >> 5)] = dh;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) q[n * K + k0 + e] = (int8_t)qv[e];
}

extern "C" int lgmlh_quantize_act(int type, const float *x, int64_t N, int64_t K, int8_t *q,
                                  void *d, int16_t *bsums, void *stream) {
  const int xf = xf_for(type, LGMLH_ACT_GGML);
  const int64_t qb = xf == XF_Q80 ? 32 : QK_K;
  if (xf == XF_SPLIT || !x || !q || !d || (xf == XF_Q8K && !bsums) || N < 0 || K <= 0 ||
      K % qb) {
    set_error("quantize_act: bad arguments (type %d, K %lld)", type, (long long)K);
    return LGMLH_EINVAL;
  }
  const int64_t total = N * (K / 8);
  if (total == 0) return LGMLH_OK;
  hipLaunchKernelGGL(act_quant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     as_stream(stream), x, N, K, xf, q, d, bsums);
  return hip_check(hipGetLastError(), "quantize_act");
}

// ---- the entry point that allocates nothing -----------------------------------
// lgmlh_mul_mat_noalloc runs lgmlh_mul_mat's kernels with their workspace
// (the split X planes and the split-K partial sums) in `scratch`, a
// file-scope device array, instead of a caller's workspace: for callers
// that cannot allocate (code under HIP graph capture, serving loops that
// forbid hipMalloc). Every GPU the library runs on holds its own copy of
// the array until the process ends. In host code `scratch` names a host
// stand-in, never a device address: the device address comes from
// hipGetSymbolAddress, once per device with that device current, and only
// that address reaches kernels. Nothing in the workspace needs to start at
// zero (every byte a kernel reads was written by the same call), so no call
// clears it. Calls that overlap on one GPU (two streams, two threads) race
// for the array.
namespace lgmlh {
constexpr size_t SCRATCH_BYTES = size_t(32) << 20;  // 32 MiB per GPU
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

// The device address of this device's scratch, or nullptr (error set).
static void *scratch_ptr() {
  constexpr int MAX_DEV = 64;
  static std::mutex mu;
  static void *ptrs[MAX_DEV];
  int dev = 0;
  if (hip_check(hipGetDevice(&dev), "mul_mat_noalloc: device") != LGMLH_OK) return nullptr;
  if (dev < 0 || dev >= MAX_DEV) {
    set_error("mul_mat_noalloc: device %d past the %d this library tracks", dev, MAX_DEV);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    if (hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "mul_mat_noalloc: scratch") !=
        LGMLH_OK)
      return nullptr;
    ptrs[dev] = p;
  }
  return ptrs[dev];
}
}  // namespace lgmlh

extern "C" size_t lgmlh_mul_mat_noalloc_limit(void) { return SCRATCH_BYTES; }

extern "C" int lgmlh_mul_mat_noalloc(int type, const void *w, int64_t M, int64_t K,
                                     const void *x, int xtype, int64_t N, float *y, int epi,
                                     const float *residual, void *stream) {
  if (type != LGMLH_F32 && (M <= 0 || K <= 0 || N < 0 || K % QK_K)) {
    set_error("mul_mat_noalloc: bad shape (M %lld, K %lld, N %lld)", (long long)M,
              (long long)K, (long long)N);
    return LGMLH_EINVAL;
  }
  const size_t need = type == LGMLH_F32 ? 0 : workspace_for(type, M, K, N);
  if (need > SCRATCH_BYTES) {
    set_error("mul_mat_noalloc: this product needs %zu bytes of workspace; the static scratch "
              "holds %zu (use lgmlh_mul_mat with a workspace)", need, SCRATCH_BYTES);
    return LGMLH_ENOMEM;
  }
  void *ws = scratch_ptr();
  if (!ws) return LGMLH_EHIP;
  return lgmlh_mul_mat(type, w, M, K, x, xtype, N, y, epi, residual, ws, SCRATCH_BYTES, stream);
}
