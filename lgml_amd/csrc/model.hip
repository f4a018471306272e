// One forward pass of a dense llama / qwen3 decoder over a planned ubatch:
// the launches that ggml's graph compute runs for the graph that
// transformer.lua forward (:2285-2365) builds, with the per-sequence
// attention loop of attention_batch (:2389-2416) replaced by one paged
// attention launch for all sequences.
#include <math.h>

#include "common.h"
#include "quant.h"

namespace lgmlh {

int mul_mat_ldy(int type, const void *w, int64_t M, int64_t K, const void *x, int xtype,
                int64_t N, float *y, int64_t ldy, const float *residual, float *part,
                size_t part_bytes, hipStream_t st);
size_t partial_bytes(int type, int64_t M, int64_t K, int64_t N);
int get_rows_dev(int type, const void *table, int64_t n_cols, const int32_t *ids, int64_t n,
                 float *out, hipStream_t st);

// rms_norm(x[rows[j]]) * w for the logit rows (get_rows + head norm).
template <typename OutT>
__global__ void rms_norm_rows_kernel(const float *__restrict__ x, const int32_t *__restrict__ rows,
                                     int64_t n, float eps, const float *__restrict__ w,
                                     OutT *__restrict__ out) {
  __shared__ double part[256];
  const float *xr = x + (int64_t)rows[blockIdx.x] * n;
  double s = 0;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += (double)xr[i] * (double)xr[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  float mean = (float)(part[0] / (double)n);
  float scale = 1.0f / sqrtf(mean + eps);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = xr[i] * scale;
    if (w) v = v * w[i];
    out[(int64_t)blockIdx.x * n + i] = (OutT)v;
  }
}

struct Carve {
  char *p;
  size_t left;
  bool ok;
  void *take(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes > left) {
      ok = false;
      return nullptr;
    }
    void *r = p;
    p += bytes;
    left -= bytes;
    return r;
  }
};

struct Sizes {
  int64_t N, E, H, Hkv, D, F, V, W, n_out;
  size_t gemm_ws, attn_ws;
};

static Sizes sizes_of(const lgmlh_model *m, int64_t n_tokens, int64_t n_items, int n_out) {
  Sizes z;
  z.N = n_tokens;
  z.E = m->n_embd;
  z.H = m->n_head;
  z.Hkv = m->n_head_kv;
  z.D = m->head_dim;
  z.F = m->n_ff;
  z.V = m->n_vocab;
  z.W = (z.H + 2 * z.Hkv) * z.D;
  z.n_out = n_out;
  size_t g = 0;
  auto upd = [&](int t, int64_t M, int64_t K, int64_t N) {
    size_t w = partial_bytes(t, M, K, N);
    if (w > g) g = w;
  };
  for (int il = 0; il < m->n_layer; il++) {
    const lgmlh_layer &L = m->layers[il];
    upd(L.wqkv_type, L.wqkv_rows, z.E, z.N);
    if (L.wv) upd(L.wv_type, z.W - L.wqkv_rows, z.E, z.N);
    upd(L.wo_type, z.E, z.H * z.D, z.N);
    upd(L.wgu_type, 2 * z.F, z.E, z.N);
    upd(L.wdown_type, z.E, z.F, z.N);
  }
  upd(m->output_type, z.V, z.E, n_out);
  z.gemm_ws = g;
  z.attn_ws = (size_t)n_items * z.Hkv * (16 * z.D + 32) * sizeof(float);
  return z;
}

static size_t ws_bytes_of(const Sizes &z) {
  size_t b = 0;
  auto add = [&](size_t x) { b += (x + 255) & ~size_t(255); };
  add(z.N * z.E * 4);        // x (residual stream)
  add(z.N * z.E * 4);        // normed x (f16 or f32)
  add(z.N * z.W * 4);        // [q | k | v]
  add(z.N * z.H * z.D * 4);  // roped q
  add(z.N * z.H * z.D * 4);  // attention out
  add(z.N * 2 * z.F * 4);    // [gate | up]
  add(z.N * z.F * 4);        // silu(gate) * up
  add(z.n_out * z.E * 4);    // normed logit rows
  add(z.attn_ws);
  add(z.gemm_ws);
  return b + 256;
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" size_t lgmlh_forward_workspace(const lgmlh_model *m, const lgmlh_plan_info *info,
                                          int n_out) {
  if (!m || !info || !m->layers) return 0;
  return ws_bytes_of(sizes_of(m, info->n_tokens, info->n_items, n_out));
}

namespace {
// Records an event pair around a launch group when the trace asks for it.
struct Span {
  lgmlh_trace *t;
  hipStream_t st;
  int slot;
  Span(lgmlh_trace *tr, int kind, hipStream_t s) : t(tr), st(s), slot(-1) {
    if (!t || !(t->kinds & kind) || t->used >= t->capacity) return;
    slot = t->used++;
    if (t->kind) t->kind[slot] = kind;
    (void)hipEventRecord((hipEvent_t)t->events[2 * slot], st);
  }
  ~Span() {
    if (slot >= 0) (void)hipEventRecord((hipEvent_t)t->events[2 * slot + 1], st);
  }
};
}  // namespace

extern "C" int lgmlh_forward(const lgmlh_model *m, const lgmlh_ubatch *ub,
                             const int32_t *out_rows, int n_out, float *logits, void *workspace,
                             size_t ws_bytes, lgmlh_trace *trace, void *stream) {
  if (!m || !ub || !logits || !workspace || !m->layers || m->n_layer <= 0 ||
      m->n_head_kv != ub->n_head_kv) {
    set_error("forward: bad arguments");
    return LGMLH_EINVAL;
  }
  if (!out_rows) {
    out_rows = ub->logit_rows;
    n_out = ub->n_seq;
  }
  hipStream_t st = as_stream(stream);
  Sizes z = sizes_of(m, ub->n_tokens, ub->n_items, n_out);
  size_t need = ws_bytes_of(z);
  if (ws_bytes < need) {
    set_error("forward: workspace of %zu bytes, need %zu", ws_bytes, need);
    return LGMLH_ENOMEM;
  }
  if (z.N == 0) return LGMLH_OK;
  uintptr_t base = ((uintptr_t)workspace + 255) & ~uintptr_t(255);
  Carve cv{(char *)base, ws_bytes - (size_t)(base - (uintptr_t)workspace), true};
  float *x = (float *)cv.take(z.N * z.E * 4);
  void *xn = cv.take(z.N * z.E * 4);
  float *qkv = (float *)cv.take(z.N * z.W * 4);
  float *q = (float *)cv.take(z.N * z.H * z.D * 4);
  float *att = (float *)cv.take(z.N * z.H * z.D * 4);
  float *gu = (float *)cv.take(z.N * 2 * z.F * 4);
  void *act = cv.take(z.N * z.F * 4);
  void *xo = cv.take(z.n_out * z.E * 4);
  void *aws = cv.take(z.attn_ws);
  float *gws = (float *)cv.take(z.gemm_ws);
  if (!cv.ok) {
    set_error("forward: workspace carve failed");
    return LGMLH_ENOMEM;
  }
  const float scale = m->attn_scale > 0 ? m->attn_scale : 1.0f / sqrtf((float)z.D);

#define GEMM(...)                                  \
  do {                                             \
    Span sp_(trace, LGMLH_TRACE_GEMM, st);         \
    LGMLH_TRY(mul_mat_ldy(__VA_ARGS__));           \
  } while (0)
  // token embeddings (get_rows, transformer.lua:2309); the ids were range
  // checked when the plan was made.
  LGMLH_TRY(get_rows_dev(m->tok_embd_type, m->tok_embd, z.E, ub->ids, z.N, x, st));
  for (int il = 0; il < m->n_layer; il++) {
    const lgmlh_layer &L = m->layers[il];
    // Activations stay f32: the GEMM splits them into f16 hi + lo itself.
    const int at = LGMLH_F32;
    LGMLH_TRY(lgmlh_rms_norm(x, z.N, z.E, m->eps, L.attn_norm, xn, at, st));
    GEMM(L.wqkv_type, L.wqkv, L.wqkv_rows, z.E, xn, at, z.N, qkv, z.W, nullptr,
                          gws, z.gemm_ws, st);
    if (L.wv) {
      GEMM(L.wv_type, L.wv, z.W - L.wqkv_rows, z.E, xn, at, z.N,
                            qkv + L.wqkv_rows, z.W, nullptr, gws, z.gemm_ws, st);
    }
    LGMLH_TRY(lgmlh_qkv_rope_store(qkv, z.N, (int)z.H, (int)z.Hkv, (int)z.D, m->n_rot,
                                   m->rope_neox, m->rope_base, m->rope_freqs, L.q_norm, L.k_norm,
                                   m->eps, ub->pos, L.kpool, L.vpool, m->n_cells, ub->cells, q,
                                   st));
    {
      Span sp(trace, LGMLH_TRACE_ATTN, st);
      LGMLH_TRY(lgmlh_paged_attention(q, (int)z.H, (int)z.Hkv, (int)z.D, scale, L.kpool,
                                      L.vpool, ub, att, aws, z.attn_ws, st));
    }
    GEMM(L.wo_type, L.wo, z.E, z.H * z.D, att, LGMLH_F32, z.N, x, z.E, x, gws,
                          z.gemm_ws, st);
    const int ft = LGMLH_F32;
    LGMLH_TRY(lgmlh_rms_norm(x, z.N, z.E, m->eps, L.ffn_norm, xn, ft, st));
    GEMM(L.wgu_type, L.wgu, 2 * z.F, z.E, xn, ft, z.N, gu, 2 * z.F, nullptr,
                          gws, z.gemm_ws, st);
    const int dt = LGMLH_F32;
    LGMLH_TRY(lgmlh_swiglu(gu, z.N, z.F, act, dt, st));
    GEMM(L.wdown_type, L.wdown, z.E, z.F, act, dt, z.N, x, z.E, x, gws,
                          z.gemm_ws, st);
  }
  // head (transformer.lua:2094-2104) on the logit rows (:2349-2350)
  const int ot = LGMLH_F32;
  if (n_out > 0) {
    if (ot == LGMLH_F16)
      hipLaunchKernelGGL(rms_norm_rows_kernel<f16>, dim3(n_out), dim3(256), 0, st, x, out_rows,
                         z.E, m->eps, m->output_norm, (f16 *)xo);
    else
      hipLaunchKernelGGL(rms_norm_rows_kernel<float>, dim3(n_out), dim3(256), 0, st, x, out_rows,
                         z.E, m->eps, m->output_norm, (float *)xo);
    LGMLH_TRY(hip_check(hipGetLastError(), "forward: head norm"));
    GEMM(m->output_type, m->output, z.V, z.E, xo, ot, n_out, logits, z.V,
                          nullptr, gws, z.gemm_ws, st);
  }
#undef GEMM
  return LGMLH_OK;
}
