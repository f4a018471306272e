// One forward pass of a llama / qwen3 / qwen3moe decoder over a planned ubatch:
// the launches that ggml's graph compute runs for the graph that
// transformer.lua forward (:2285-2365) builds, with the per-sequence
// attention loop of attention_batch (:2389-2416) replaced by one paged
// attention launch for all sequences.
#include <math.h>

#include "common.h"
#include "moe.h"
#include "quant.h"
#include "split.h"

namespace lgmlh {

int mul_mat_f32(const float *w, int64_t M, int64_t K, const float *x, int64_t N, float *y,
                int64_t ldy, const float *residual, hipStream_t st);
int paged_attention_dev(const float *q, int n_head, int n_head_kv, int head_dim, float scale,
                        const void *kpool, const void *vpool, const lgmlh_ubatch *ub, float *out,
                        f16 *planes, int64_t npad, void *workspace, size_t workspace_bytes,
                        hipStream_t st, int xf);
bool attn_q8k_fits(int head_dim, int G);
int rms_norm_dev(float *x, const int32_t *rows, int64_t n_rows, int64_t n, float eps,
                 const float *w, float *out, f16 *planes, hipStream_t st, Pending pend,
                 bool writeback, int xf);
int swiglu_dev(const float *gu, int64_t n, int64_t F, float *out, f16 *planes, hipStream_t st,
               Pending pend, int gelu, int xf);
int softcap_dev(float *x, int64_t n, float cap, hipStream_t st);
int qkv_rope_store_dev(float *qkv, int64_t n, int n_head, int n_head_kv, int head_dim, int n_rot,
                       int neox, float freq_base, const float *freq_factors, const float *q_norm,
                       const float *k_norm, float eps, const int32_t *pos, void *kpool,
                       void *vpool, int64_t n_cells, const int64_t *cells, float *q_out,
                       void *stream, Pending pa, Pending pb, int vmode, const float *table);
int rope_table_dev(const int32_t *pos, int64_t n, int n_rot, float freq_base,
                   const float *freq_factors, float *table, hipStream_t st);
size_t partial_bytes(int type, int64_t M, int64_t K, int64_t N);
int get_rows_dev(int type, const void *table, int64_t n_cols, const int32_t *ids, int64_t n,
                 float *out, hipStream_t st, float scale);
constexpr int QKV_V_FROM_K = 1, QKV_V_NORM = 2;

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
  size_t gemm_ws, gemm_ws_v, attn_ws, split_ws;
  // a layer whose V product takes X in another form than its q|k product
  // (ggml arithmetic, Q8_0 beside a K-quant): planes of its own
  bool v_own;
  // routed experts: experts, picks per token, expert width, picks, tile width
  bool moe;
  int NE, NU, tc;
  int64_t FX, P;
  // rope angle tables of the pass: distinct settings, the widest n_rot
  int n_rope, rot;
};

static bool isq(int type) { return type != LGMLH_F32; }

// A layer's rope setting (rotated dimensions, base, frequency factors).
struct RopeKey {
  int n_rot;
  float base;
  const float *ff;
  bool operator==(const RopeKey &o) const {
    return n_rot == o.n_rot && base == o.base && ff == o.ff;
  }
};
constexpr int MAX_ROPE = 8;  // distinct settings with a table of their own

// A layer's attention shape: its own head size, KV heads and rotated
// dimensions where it sets them (gemma's sliding and global layers differ,
// transformer.lua:215-235), else the model's; W = the row width of [q|k|v].
struct LDims {
  int D, Hkv, n_rot;
  int64_t W;
};
static LDims dims_of(const lgmlh_model *m, const lgmlh_layer &L) {
  LDims d;
  d.D = L.head_dim > 0 ? L.head_dim : m->head_dim;
  d.Hkv = L.n_head_kv > 0 ? L.n_head_kv : m->n_head_kv;
  d.n_rot = L.n_rot > 0 ? L.n_rot : L.head_dim > 0 ? L.head_dim : m->n_rot;
  d.W = (int64_t)(m->n_head + 2 * d.Hkv) * d.D;
  return d;
}

static RopeKey rope_key(const lgmlh_model *m, const lgmlh_layer &L) {
  return RopeKey{dims_of(m, L).n_rot, L.rope_base > 0 ? L.rope_base : m->rope_base,
                 L.rope_freqs ? L.rope_freqs : m->rope_freqs};
}

// The distinct rope settings of the model's layers, in layer order (at most
// MAX_ROPE: further ones make their angles in the layer's own kernel).
static int rope_keys(const lgmlh_model *m, RopeKey (&keys)[MAX_ROPE]) {
  int n = 0;
  for (int il = 0; il < m->n_layer; il++) {
    const RopeKey k = rope_key(m, m->layers[il]);
    bool seen = false;
    for (int j = 0; j < n; j++) seen = seen || keys[j] == k;
    if (!seen && n < MAX_ROPE) keys[n++] = k;
  }
  return n;
}

// The V product of layer L takes its X planes apart from the q|k product's.
static bool v_own_planes(const lgmlh_model *m, const lgmlh_layer &L) {
  return L.wv && isq(L.wv_type) && isq(L.wqkv_type) &&
         xf_for(L.wv_type, m->act) != xf_for(L.wqkv_type, m->act);
}

static Sizes sizes_of(const lgmlh_model *m, int64_t n_tokens, int64_t n_items, int n_out) {
  Sizes z;
  z.v_own = false;
  for (int il = 0; il < m->n_layer; il++) z.v_own = z.v_own || v_own_planes(m, m->layers[il]);
  z.N = n_tokens;
  z.E = m->n_embd;
  z.H = m->n_head;
  z.Hkv = m->n_head_kv;
  z.D = m->head_dim;
  z.F = m->n_ff;
  z.V = m->n_vocab;
  // the widest layer sizes the buffers (z.D: the largest head, z.W the
  // widest [q|k|v] row)
  z.W = 0;
  size_t attn_unit = 0;  // floats of an item's partial state per KV head set
  for (int il = 0; il < m->n_layer; il++) {
    const LDims d = dims_of(m, m->layers[il]);
    if (d.W > z.W) z.W = d.W;
    if (d.D > z.D) z.D = d.D;
    const size_t u = (size_t)d.Hkv * (16 * d.D + 32);
    if (u > attn_unit) attn_unit = u;
  }
  z.n_out = n_out;
  size_t g = 0, gv = 0;
  auto upd = [&](int t, int64_t M, int64_t K, int64_t N) {
    size_t w = partial_bytes(t, M, K, N);
    if (w > g) g = w;
  };
  z.moe = false;
  for (int il = 0; il < m->n_layer; il++) z.moe = z.moe || m->layers[il].gate_inp != nullptr;
  z.NE = z.moe ? m->n_expert : 0;
  z.NU = z.moe ? m->n_used : 0;
  z.FX = z.moe ? m->n_ff_exp : 0;
  z.P = z.N * z.NU;
  z.tc = z.moe ? moe_tile_cols(z.P, z.NE) : 16;
  for (int il = 0; il < m->n_layer; il++) {
    const lgmlh_layer &L = m->layers[il];
    const LDims d = dims_of(m, L);
    upd(L.wqkv_type, L.wqkv_rows, z.E, z.N);
    if (L.wv) {
      // pending beside the [q|k] partials: a region of its own
      size_t w = partial_bytes(L.wv_type, d.W - L.wqkv_rows, z.E, z.N);
      if (w > gv) gv = w;
    }
    upd(L.wo_type, z.E, z.H * d.D, z.N);
    if (!L.gate_inp) {
      upd(L.wgu_type, 2 * z.F, z.E, z.N);
      upd(L.wdown_type, z.E, z.F, z.N);
    }
  }
  upd(m->output_type, z.V, z.E, n_out);
  z.gemm_ws = g;
  z.gemm_ws_v = gv;
  int64_t kmax = z.E > z.F ? z.E : z.F;
  if (z.H * z.D > kmax) kmax = z.H * z.D;
  if (z.FX > kmax) kmax = z.FX;
  int64_t rmax = z.N > n_out ? z.N : n_out;
  if (z.P > rmax) rmax = z.P;  // the expert activations of the picks
  z.split_ws = split_bytes(rmax, kmax);
  z.attn_ws = (size_t)n_items * attn_unit * sizeof(float);
  RopeKey keys[MAX_ROPE];
  z.n_rope = rope_keys(m, keys);
  z.rot = 0;
  for (int j = 0; j < z.n_rope; j++)
    if (keys[j].n_rot > z.rot) z.rot = keys[j].n_rot;
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
  add(z.N * z.E * 4);        // a post-normed product (gemma), pending
  add(z.split_ws);           // X planes of the current product
  if (z.v_own) add(split_bytes(z.N, z.E));  // X planes of a V product of its own form
  add(z.attn_ws);
  add((size_t)z.n_rope * z.N * z.rot * 4);  // rope angle tables
  add(z.gemm_ws);
  add(z.gemm_ws_v);
  if (z.moe) {
    add((size_t)router_splits(z.E) * z.N * z.NE * 4);  // router partials
    add(z.P * 4);                                        // ids
    add(z.P * 4);                                        // weights
    add(group_bytes(z.P, z.NE, z.tc));                   // grouping
    add(z.P * 2 * z.FX * 4);                             // [gate | up] of the picks
    add(z.P * z.FX * 4);                                 // f32 activations (f32 experts)
    add(z.P * z.E * 4);                                  // expert outputs (pending)
  }
  return b + 256;
}

}  // namespace lgmlh

using namespace lgmlh;

extern "C" size_t lgmlh_forward_workspace(const lgmlh_model *m, const lgmlh_plan_info *info,
                                          const lgmlh_plan_info *info_ring, int n_out) {
  if (!m || !info || !m->layers) return 0;
  int items = info->n_items;
  if (info_ring && info_ring->n_items > items) items = info_ring->n_items;
  return ws_bytes_of(sizes_of(m, info->n_tokens, items, n_out));
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

// A side stream (default priority) and two events per host thread, device
// and caller stream (up to SIDE_PER_DEV caller streams), for a product that
// runs beside another product of the same pass; null when none can be made
// (the caller stays on its stream). Passes on different caller streams get
// different side streams, so that one's side products never queue behind
// another's.
struct Side {
  hipStream_t caller = nullptr;
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  bool failed = false;
};
constexpr int SIDE_MAX_DEV = 16, SIDE_PER_DEV = 4;
thread_local Side sides[SIDE_MAX_DEV][SIDE_PER_DEV];

Side *side_of(hipStream_t caller) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= SIDE_MAX_DEV) return nullptr;
  Side *free_slot = nullptr;
  for (Side &sd : sides[dev]) {
    if ((sd.s || sd.failed) && sd.caller == caller) return sd.failed ? nullptr : &sd;
    if (!sd.s && !sd.failed && !free_slot) free_slot = &sd;
  }
  if (!free_slot) return nullptr;
  Side &sd = *free_slot;
  sd.caller = caller;
  if (hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&sd.join, hipEventDisableTiming) != hipSuccess) {
    (void)hipGetLastError();
    if (sd.s) (void)hipStreamDestroy(sd.s);
    if (sd.fork) (void)hipEventDestroy(sd.fork);
    sd.s = nullptr;
    sd.fork = sd.join = nullptr;
    sd.failed = true;
    return nullptr;
  }
  return &sd;
}
}  // namespace

// The calling thread's side streams and events on the current device, made
// by its passes with a V product of its own type, are destroyed (after the
// work queued on each stream ends); later passes make them again.
extern "C" int lgmlh_forward_release(void) {
  int dev = 0;
  LGMLH_TRY(hip_check(hipGetDevice(&dev), "forward_release: device"));
  if (dev < 0 || dev >= SIDE_MAX_DEV) return LGMLH_OK;
  for (Side &sd : sides[dev]) {
    if (sd.s) {
      LGMLH_TRY(hip_check(hipStreamSynchronize(sd.s), "forward_release: sync"));
      LGMLH_TRY(hip_check(hipStreamDestroy(sd.s), "forward_release: stream"));
      sd.s = nullptr;
    }
    if (sd.fork) {
      LGMLH_TRY(hip_check(hipEventDestroy(sd.fork), "forward_release: event"));
      sd.fork = nullptr;
    }
    if (sd.join) {
      LGMLH_TRY(hip_check(hipEventDestroy(sd.join), "forward_release: event"));
      sd.join = nullptr;
    }
    sd = Side{};
  }
  return LGMLH_OK;
}

extern "C" int lgmlh_forward(const lgmlh_model *m, const lgmlh_ubatch *ub,
                             const lgmlh_ubatch *ub_ring, const int32_t *out_rows, int n_out,
                             float *logits, void *workspace, size_t ws_bytes, lgmlh_trace *trace,
                             void *stream) {
  if (!m || !ub || !logits || !workspace || !m->layers || m->n_layer <= 0) {
    set_error("forward: bad arguments");
    return LGMLH_EINVAL;
  }
  if (m->act != LGMLH_ACT_EXACT && m->act != LGMLH_ACT_GGML) {
    set_error("forward: act %d is neither LGMLH_ACT_EXACT nor LGMLH_ACT_GGML", m->act);
    return LGMLH_EINVAL;
  }
  for (int il = 0; il < m->n_layer; il++) {
    const lgmlh_layer &L = m->layers[il];
    if (L.swa && (!ub_ring || ub_ring->ring <= 0 || ub_ring->n_tokens != ub->n_tokens)) {
      set_error("forward: layer %d slides and needs the pass's ring plan", il);
      return LGMLH_EINVAL;
    }
    // each plan is made for the KV heads of the layers that attend through it
    const int hkv = dims_of(m, L).Hkv;
    if ((L.swa ? ub_ring : ub)->n_head_kv != hkv) {
      set_error("forward: layer %d has %d KV heads; its plan was made for %d", il, hkv,
                (L.swa ? ub_ring : ub)->n_head_kv);
      return LGMLH_EINVAL;
    }
  }
  if (!out_rows) {
    out_rows = ub->logit_rows;
    n_out = ub->n_seq;
  }
  hipStream_t st = as_stream(stream);
  const int items = ub_ring && ub_ring->n_items > ub->n_items ? ub_ring->n_items : ub->n_items;
  Sizes z = sizes_of(m, ub->n_tokens, items, n_out);
  size_t need = ws_bytes_of(z);
  if (ws_bytes < need) {
    set_error("forward: workspace of %zu bytes, need %zu", ws_bytes, need);
    return LGMLH_ENOMEM;
  }
  if (z.N == 0) return LGMLH_OK;
  uintptr_t base = ((uintptr_t)workspace + 255) & ~uintptr_t(255);
  Carve cv{(char *)base, ws_bytes - (size_t)(base - (uintptr_t)workspace), true};
  float *x = (float *)cv.take(z.N * z.E * 4);
  float *xn = (float *)cv.take(z.N * z.E * 4);
  float *qkv = (float *)cv.take(z.N * z.W * 4);
  float *q = (float *)cv.take(z.N * z.H * z.D * 4);
  float *att = (float *)cv.take(z.N * z.H * z.D * 4);
  float *gu = (float *)cv.take(z.N * 2 * z.F * 4);
  float *act = (float *)cv.take(z.N * z.F * 4);
  float *xo = (float *)cv.take(z.n_out * z.E * 4);
  float *ao = (float *)cv.take(z.N * z.E * 4);
  f16 *xs = (f16 *)cv.take(z.split_ws);
  f16 *xs_v = z.v_own ? (f16 *)cv.take(split_bytes(z.N, z.E)) : nullptr;
  void *aws = cv.take(z.attn_ws);
  float *rtab = (float *)cv.take((size_t)z.n_rope * z.N * z.rot * 4);
  float *gws = (float *)cv.take(z.gemm_ws);
  float *gws_v = (float *)cv.take(z.gemm_ws_v);
  float *rpart = nullptr, *mwts = nullptr, *gu_e = nullptr, *act_e = nullptr, *y_e = nullptr;
  int32_t *mids = nullptr;
  GroupOut go{};
  if (z.moe) {
    rpart = (float *)cv.take((size_t)router_splits(z.E) * z.N * z.NE * 4);
    mids = (int32_t *)cv.take(z.P * 4);
    mwts = (float *)cv.take(z.P * 4);
    void *gb = cv.take(group_bytes(z.P, z.NE, z.tc));
    gu_e = (float *)cv.take(z.P * 2 * z.FX * 4);
    act_e = (float *)cv.take(z.P * z.FX * 4);
    y_e = (float *)cv.take(z.P * z.E * 4);
    if (gb) go = group_carve(gb, z.P, z.NE, z.tc);
  }
  if (!cv.ok) {
    set_error("forward: workspace carve failed");
    return LGMLH_ENOMEM;
  }


  // The X form of a quantized product (split planes, or ggml's Q8_K / Q8_0
  // blocks under LGMLH_ACT_GGML).
  auto xfo = [&](int type) { return xf_for(type, m->act); };
  // A product on X given as f32 rows (f32 weights) or as planes (quantized
  // weights, xs unless given); the producer wrote the form(s) the weights
  // take. A quantized product split over K leaves its partial sums pending
  // (pd): the next kernel that reads y adds them in the canonical order,
  // then the residual.
  auto gemm_on = [&](hipStream_t s, int type, const void *w, int64_t M, int64_t K,
                     const float *xf, int64_t N, float *y, int64_t ldy, const float *res,
                     float *part, size_t part_bytes, Pending &pd,
                     const f16 *planes = nullptr) -> int {
    Span sp(trace, LGMLH_TRACE_GEMM, s);
    pd = Pending{};
    if (type == LGMLH_F32) return mul_mat_f32((const float *)w, M, K, xf, N, y, ldy, res, s);
    return mul_mat_split(type, w, M, K, planes ? planes : xs, N, y, ldy, res, part, part_bytes,
                         s, &pd, xfo(type));
  };
  auto gemm = [&](int type, const void *w, int64_t M, int64_t K, const float *xf, int64_t N,
                  float *y, int64_t ldy, const float *res, float *part, size_t part_bytes,
                  Pending &pd) -> int {
    return gemm_on(st, type, w, M, K, xf, N, y, ldy, res, part, part_bytes, pd);
  };
  // A product whose output goes to the residual stream x: added into x by
  // the GEMM (or left pending, the consumer adds it), or, with a post norm
  // or an output scale (gemma), left pending in ao: the next norm adds
  // rms_norm(product) * post to x, then scales.
  auto out_product = [&](int type, const void *w, int64_t K, const float *xf, const float *post,
                         float oscale, Pending &pd) -> int {
    if (!post && oscale == 0.0f)
      return gemm(type, w, z.E, K, xf, z.N, x, z.E, x, gws, z.gemm_ws, pd);
    LGMLH_TRY(gemm(type, w, z.E, K, xf, z.N, ao, z.E, nullptr, gws, z.gemm_ws, pd));
    if (!pd.splits) pd = Pending{ao, 1, z.N, z.E};
    pd.post = post;
    pd.scale = oscale;
    return LGMLH_OK;
  };
  Pending p_qk, p_v, p_o, p_gu, p_down;
  // token embeddings (get_rows, transformer.lua:2309; times the gemma
  // embedding scale, :2304-2306); the ids were range checked when the plan
  // was made.
  LGMLH_TRY(get_rows_dev(m->tok_embd_type, m->tok_embd, z.E, ub->ids, z.N, x, st,
                         m->embd_scale));
  // the rope angles of every token, once per setting for all its layers
  RopeKey rkeys[MAX_ROPE];
  const int n_rope = rope_keys(m, rkeys);
  for (int j = 0; j < n_rope; j++)
    LGMLH_TRY(rope_table_dev(ub->pos, z.N, rkeys[j].n_rot, rkeys[j].base, rkeys[j].ff,
                             rtab + (size_t)j * z.N * z.rot, st));
  for (int il = 0; il < m->n_layer; il++) {
    const lgmlh_layer &L = m->layers[il];
    const LDims d = dims_of(m, L);
    const float scale = m->attn_scale > 0 ? m->attn_scale : 1.0f / sqrtf((float)d.D);
    const bool v_sep = L.wv != nullptr;
    const bool v_own = v_own_planes(m, L);
    const bool qin_q = isq(L.wqkv_type) || (v_sep && isq(L.wv_type));
    const bool qin_f = !isq(L.wqkv_type) || (v_sep && !isq(L.wv_type)) || v_own;
    // x += the previous layer's down product, then attn_norm (planes in
    // the form of the first quantized product; a V product of another
    // form gets its own from the f32 rows)
    LGMLH_TRY(rms_norm_dev(x, nullptr, z.N, z.E, m->eps, L.attn_norm, qin_f ? xn : nullptr,
                           qin_q ? xs : nullptr, st, p_down, true,
                           xfo(isq(L.wqkv_type) ? L.wqkv_type : L.wv_type)));
    if (v_own) LGMLH_TRY(split_x(xn, LGMLH_F32, z.N, z.E, xs_v, st, xfo(L.wv_type)));
    // A V matrix of its own type (a more_bits layer's Q6_K) is a small
    // product that leaves most CUs idle: it runs on a side stream beside
    // the q|k product (not while tracing, whose events time one stream).
    p_v = Pending{};
    Side *sd = v_sep && !trace ? side_of(st) : nullptr;
    if (sd) {
      LGMLH_TRY(hip_check(hipEventRecord(sd->fork, st), "forward: fork"));
      LGMLH_TRY(hip_check(hipStreamWaitEvent(sd->s, sd->fork, 0), "forward: fork"));
      LGMLH_TRY(gemm_on(sd->s, L.wv_type, L.wv, d.W - L.wqkv_rows, z.E, xn, z.N,
                        qkv + L.wqkv_rows, d.W, nullptr, gws_v, z.gemm_ws_v, p_v,
                        v_own ? xs_v : nullptr));
      LGMLH_TRY(hip_check(hipEventRecord(sd->join, sd->s), "forward: join"));
    }
    LGMLH_TRY(gemm(L.wqkv_type, L.wqkv, L.wqkv_rows, z.E, xn, z.N, qkv, d.W, nullptr, gws,
                   z.gemm_ws, p_qk));
    if (sd) {
      LGMLH_TRY(hip_check(hipStreamWaitEvent(st, sd->join, 0), "forward: join"));
    } else if (v_sep) {
      LGMLH_TRY(gemm_on(st, L.wv_type, L.wv, d.W - L.wqkv_rows, z.E, xn, z.N, qkv + L.wqkv_rows,
                        d.W, nullptr, gws_v, z.gemm_ws_v, p_v, v_own ? xs_v : nullptr));
    }
    // a sliding layer keeps its K / V in the sequences' rings (rows_swa,
    // transformer.lua:2469-2476) and attends through the ring plan
    const lgmlh_ubatch *lub = L.swa ? ub_ring : ub;
    const int vmode = (L.v_from_k ? QKV_V_FROM_K : 0) | (m->gemma ? QKV_V_NORM : 0);
    const RopeKey rk = rope_key(m, L);
    const float *tab = nullptr;
    for (int j = 0; j < n_rope; j++)
      if (rkeys[j] == rk) tab = rtab + (size_t)j * z.N * z.rot;
    LGMLH_TRY(qkv_rope_store_dev(qkv, z.N, (int)z.H, d.Hkv, d.D, d.n_rot, m->rope_neox, rk.base,
                                 rk.ff, L.q_norm, L.k_norm, m->eps, ub->pos, L.kpool, L.vpool,
                                 L.swa ? m->ring_cells : m->n_cells, lub->cells, q, st, p_qk, p_v,
                                 vmode, tab));
    // a quantized output product takes its X (split planes, ggml's Q8_0
    // blocks, or its Q8_K blocks when a block's heads are of one KV head's
    // group) from the attention (and merge) kernels themselves; heads too
    // small for that have theirs made from the f32 rows
    const int xo = xfo(L.wo_type);
    const bool oq = isq(L.wo_type),
               o_split = oq && (xo == XF_Q8K ? attn_q8k_fits(d.D, (int)z.H / d.Hkv) : d.D >= 32);
    {
      Span sp(trace, LGMLH_TRACE_ATTN, st);
      LGMLH_TRY(paged_attention_dev(q, (int)z.H, d.Hkv, d.D, scale, L.kpool, L.vpool,
                                    lub, o_split ? nullptr : att, o_split ? xs : nullptr,
                                    split_npad(z.N), aws, z.attn_ws, st, xo));
    }
    if (oq && !o_split)
      LGMLH_TRY(split_x(att, LGMLH_F32, z.N, z.H * d.D, xs, st, xfo(L.wo_type)));
    LGMLH_TRY(out_product(L.wo_type, L.wo, z.H * d.D, att, L.post_attn_norm, 0.0f, p_o));
    if (L.gate_inp) {
      // routed experts (transformer.lua:2054-2068, M.moe :1989-2027): x +=
      // attention out, then ffn_norm for the router (f32) and the experts
      const bool gq = isq(L.exp_gu_type), dq = isq(L.exp_down_type);
      LGMLH_TRY(rms_norm_dev(x, nullptr, z.N, z.E, m->eps, L.ffn_norm, xn, gq ? xs : nullptr,
                             st, p_o, true, xfo(L.exp_gu_type)));
      {
        Span sp(trace, LGMLH_TRACE_GEMM, st);
        LGMLH_TRY(router_logits(L.gate_inp, z.NE, z.E, xn, z.N, rpart, st));
      }
      LGMLH_TRY(moe_route_dev(rpart, router_splits(z.E), z.N, z.NE, z.NU, m->gating,
                              m->norm_topk, m->expert_scale, mids, mwts, &go, st));
      {
        Span sp(trace, LGMLH_TRACE_EXPERTS, st);
        LGMLH_TRY(experts_dev(L.exp_gu_type, L.exp_gu, z.NE, 2 * z.FX, z.E, xn, xs,
                              split_npad(z.N), 1, mids, z.N, z.NU, go, gu_e, st,
                              xfo(L.exp_gu_type)));
      }
      // swiglu_split on the picks' rows; their split planes replace x's
      LGMLH_TRY(swiglu_dev(gu_e, z.P, z.FX, dq ? nullptr : act_e, dq ? xs : nullptr, st,
                           Pending{}, 0, xfo(L.exp_down_type)));
      {
        Span sp(trace, LGMLH_TRACE_EXPERTS, st);
        LGMLH_TRY(experts_dev(L.exp_down_type, L.exp_down, z.NE, z.E, z.FX, act_e, xs,
                              split_npad(z.P), z.NU, mids, z.N, z.NU, go, y_e, st,
                              xfo(L.exp_down_type)));
      }
      // the weighted sum of the picks (g:mul, sum_picks) is added to x by
      // the next norm
      p_down = Pending{y_e, z.NU, z.N, z.E, mwts};
      continue;
    }
    // x += attention out, then ffn_norm
    LGMLH_TRY(rms_norm_dev(x, nullptr, z.N, z.E, m->eps, L.ffn_norm,
                           isq(L.wgu_type) ? nullptr : xn, isq(L.wgu_type) ? xs : nullptr, st,
                           p_o, true, xfo(L.wgu_type)));
    LGMLH_TRY(gemm(L.wgu_type, L.wgu, 2 * z.F, z.E, xn, z.N, gu, 2 * z.F, nullptr, gws,
                   z.gemm_ws, p_gu));
    // SwiGLU, or GeGLU on gemma (transformer.lua:2048)
    LGMLH_TRY(swiglu_dev(gu, z.N, z.F, isq(L.wdown_type) ? nullptr : act,
                         isq(L.wdown_type) ? xs : nullptr, st, p_gu, m->gemma,
                         xfo(L.wdown_type)));
    LGMLH_TRY(out_product(L.wdown_type, L.wdown, z.F, act, L.post_ffn_norm, L.out_scale, p_down));
  }
  // head (transformer.lua:2094-2104) on the logit rows (:2349-2350); the last
  // down product is added to those rows only (x is not needed afterwards)
  if (n_out > 0) {
    const bool oq = isq(m->output_type);
    LGMLH_TRY(rms_norm_dev(x, out_rows, n_out, z.E, m->eps, m->output_norm, oq ? nullptr : xo,
                           oq ? xs : nullptr, st, p_down, false, xfo(m->output_type)));
    // the logits are the output: a split head product is reduced here
    Span sp(trace, LGMLH_TRACE_GEMM, st);
    if (oq)
      LGMLH_TRY(mul_mat_split(m->output_type, m->output, z.V, z.E, xs, n_out, logits, z.V,
                              nullptr, gws, z.gemm_ws, st, nullptr, xfo(m->output_type)));
    else
      LGMLH_TRY(mul_mat_f32((const float *)m->output, z.V, z.E, xo, n_out, logits, z.V, nullptr,
                            st));
    // the final logit softcap (transformer.lua:2097-2099)
    if (m->softcap > 0) LGMLH_TRY(softcap_dev(logits, (int64_t)n_out * z.V, m->softcap, st));
  }
  return LGMLH_OK;
}
