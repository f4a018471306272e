/*
 * CPU oracle for the lgml ragged decode/prefill path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library (lgml_amd/)
 * links, loads or calls this code. Only tests/, the smoke check in
 * __graft_entry__.py and the cpu_baseline leg of bench.py use it, and
 * only as the checker or the CPU baseline, never as the thing measured.
 *
 * Semantics: fp32 values, f64 reductions, f16 (round to nearest even)
 * KV storage, closed-form Q4_K / Q6_K / Q8_0 dequantization; activations
 * exact, or (orc_model.act_quant, orc_mul_mat_q8) quantized per block as
 * ggml's CPU backend does for quantized weights. Each function cites the reference file:line
 * whose behaviour it restates (paths under the lgml tree).
 */
#ifndef LGML_ORACLE_H
#define LGML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids of the weight formats the path uses. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q6_K = 14 };

/* ---- random numbers ---------------------------------------------------- */
/* test/tiny.lua:16-22: x <- x*6364136223846793005 + 1442695040888963407,
 * u = (x >> 11) / 2^53. state is advanced in place. */
double orc_lcg_next(uint64_t *state);
/* Fill n floats with lo + (hi - lo) * u, computed in double and rounded
 * to f32, as test_qwen_moe.lua:77-86 and gguf.lua:41-50 store them. */
void orc_lcg_fill(uint64_t *state, float *out, int64_t n, double lo, double hi);
/* src/lgml.c:3064-3079,3130-3136: splitmix64 unit numbers and the
 * Box-Muller "normal" fill (two draws per value, cos branch). */
void orc_fill_normal(uint64_t *seed, float *out, int64_t n, double mean, double sd);
void orc_fill_uniform(uint64_t *seed, float *out, int64_t n, double a, double b);
/* One raw splitmix64 draw (the state advanced in place). */
uint64_t orc_splitmix64(uint64_t *state);
/* orc_fill_normal's values for a fresh seed, in parallel; and the same
 * values quantized row by row (rows x cols) into `type`. */
void orc_gen_normal(uint64_t seed, float *out, int64_t n, double mean, double sd, int n_threads);
int64_t orc_gen_normal_quant(uint64_t seed, int type, int64_t rows, int64_t cols, double mean,
    double sd, void *out, int n_threads);

/* ---- f16 ----------------------------------------------------------------- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_row(const float *x, uint16_t *y, int64_t n);
void orc_f16_to_f32_row(const uint16_t *x, float *y, int64_t n);

/* ---- quantized formats --------------------------------------------------- */
int64_t orc_row_size(int type, int64_t n);
/* Dequantize n values (a multiple of the block size) of one row. */
int orc_dequantize_row(int type, const void *src, float *dst, int64_t n);
/* The oracle's own deterministic quantizer (format-exact, not ggml's
 * search). Returns bytes written. */
int64_t orc_quantize_row(int type, const float *src, void *dst, int64_t n);

/* ---- dense model --------------------------------------------------------- */
typedef struct {
	int type;           /* ORC_* */
	const void *data;   /* rows of `cols` values in `type` */
} orc_tensor;

typedef struct {
	orc_tensor attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, gate, up, down;
	/* Routed experts (qwen3moe): gate_inp (n_expert, n_embd) router;
	 * gate_exps / up_exps n_expert matrices (n_ff_exp, n_embd), down_exps
	 * n_expert matrices (n_embd, n_ff_exp), each expert's rows contiguous.
	 * A layer with gate_inp.data set has no dense FFN. */
	orc_tensor gate_inp, gate_exps, up_exps, down_exps;
	/* gemma (transformer.lua:300-333): post-attention and post-FFN norms
	 * (data NULL = none), the layer output scale (0 = none). swa: a
	 * sliding-window layer (its K/V in the sequence's ring, the window
	 * mask). head_dim, n_head_kv, n_rot, rope_base: this layer's attention
	 * shape and rope (0 = the model's); rope_freqs: its frequency factors
	 * (NULL = none). A gemma layer with wv.data NULL takes V = the raw K
	 * (:1779). */
	orc_tensor post_attn_norm, post_ffn_norm;
	float out_scale;
	int swa, head_dim, n_head_kv, n_rot;
	float rope_base;
	const float *rope_freqs;
} orc_layer;

/* Expert gating functions (transformer.lua:32-35). */
enum { ORC_GATING_SOFTMAX = 1, ORC_GATING_SIGMOID = 2 };

typedef struct {
	int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_rot;
	float eps, rope_base, attn_scale; /* attn_scale 0 means 1/sqrt(head_dim) */
	int rope_neox;                    /* 0 normal (llama), 1 neox (qwen3, gemma) */
	const float *rope_freqs;          /* n_rot/2 factors or NULL */
	orc_tensor tok_embd, output, output_norm;
	const orc_layer *layers;
	/* MoE hyperparameters (transformer.lua:160-170): experts, picks per
	 * token, expert FFN width, gating, norm_topk, expert_scale. */
	int n_expert, n_used, n_ff_exp, gating, norm_topk;
	float expert_scale;
	/* gemma (transformer.lua:171-183): V rms-normed, GeGLU, embeddings
	 * times embd_scale (0 = none), logits softcap * tanh(l / softcap)
	 * (0 = none); n_swa: the sliding window of swa layers. */
	int gemma, n_swa;
	float embd_scale, softcap;
	/* 0: exact products (f32 activations, f64 sums over dequantized
	 * weights); 1: ggml's CPU arithmetic for quantized weights (X quantized
	 * to Q8_K / Q8_0 per block, integer block dots; orc_mul_mat_q8). */
	int act_quant;
} orc_model;

/* One ubatch over a paged pool. Sequence s owns tokens
 * [off_s, off_s + seq_n[s]) of ids (off_s = sum of earlier seq_n), at
 * positions seq_npast[s] + j. Position p of sequence s lives in pool cell
 * block_tab[s * max_blocks + p / block] * block + p % block.
 * kpool[l], vpool[l] are (cap, n_head_kv * head_dim) f16 rows.
 * logits gets one row per out_rows entry (token indices into the ubatch).
 * hidden_out, when not NULL, gets the final-normed rows (n_out, n_embd). */
typedef struct {
	int n_seq, max_blocks, block;
	const int32_t *seq_n, *seq_npast, *block_tab;
	const int32_t *ids;
	int n_out;
	const int32_t *out_rows;
	/* Sliding-window layers keep a ring of ring_blocks blocks per
	 * sequence: position p of sequence s lives in cell
	 * ring_tab[s * ring_blocks + (p / block) % ring_blocks] * block +
	 * p % block of those layers' pools (rows_swa = p % ring,
	 * transformer.lua:2469-2476, with ring = ring_blocks * block). */
	int ring_blocks;
	const int32_t *ring_tab;
} orc_batch;

int orc_forward(const orc_model *m, uint16_t *const *kpool, uint16_t *const *vpool,
    int64_t cap, const orc_batch *b, float *logits, int n_threads);

/* Paged attention alone (the flash_attn / fill_blocks pair, per sequence).
 * q: (N, H, D) f32 in ubatch order. out: (N, H, D) f32. Causal over the
 * sequence's own positions 0..npast+j. */
int orc_paged_attention(const float *q, const uint16_t *kpool, const uint16_t *vpool,
    int H, int Hkv, int D, float scale, const orc_batch *b, float *out, int n_threads);
/* The same over the sequences' rings with a sliding window
 * (tensor_fill_mask window + ring, src/lgml.c:2873-2935): query j sees
 * positions max(0, p - window + 1)..p, p = npast + j. */
int orc_paged_attention_swa(const float *q, const uint16_t *kpool, const uint16_t *vpool,
    int H, int Hkv, int D, float scale, int window, const orc_batch *b, float *out,
    int n_threads);

/* graph:flash_attn (src/lgml.c:2121-2170) with an explicit mask: the
 * published algorithm of ggml_flash_attn_ext (ggml, the un-vendored
 * subproject pinned at 0f1fa6109ad6f11d51dc0ab6f8e599258a393e1c). For
 * query row t of head h and column j: s = scale * q.k_j; with softcap > 0
 * s = softcap * tanh(s / softcap); then s += slope_h * mask[h % mask_heads]
 * [t][j] (slope 1, or ALiBi's with max_bias > 0). A -inf mask drops the
 * column; a row with every column dropped gives zeros. o = softmax(s) v.
 * q (H, T, D) f32; k, v element (hk, j, d) at [hk * hs + j * rs + d] f16;
 * mask (mask_heads, mask_rows >= T, n_kv) f16 or NULL; out (T, H, D).
 * Head h reads kv head h / (H / Hkv). Scores and sums in f64. */
int orc_flash_attn(const float *q, int H, int T, int D, const uint16_t *k, const uint16_t *v,
    int Hkv, int n_kv, int64_t k_rs, int64_t k_hs, int64_t v_rs, int64_t v_hs,
    const uint16_t *mask, int mask_heads, int mask_rows, float scale, float max_bias,
    float softcap, float *out, int n_threads);

/* ggml_set_rows (src/lgml.c:1937-1969): dst[ids[j]] = f16(src[j]). */
int orc_set_rows_f16(uint16_t *dst, int64_t dst_rows, int64_t row, const float *src,
    const int64_t *ids, int64_t n);

/* Y (N, M) = X (N, K) W^T, W rows in `type` (ggml mul_mat convention,
 * src/lgml.c:1811-1839). f64 accumulation. */
int orc_mul_mat(int type, const void *w, int64_t M, int64_t K, const float *x, int64_t N,
    float *y, int n_threads);

/* ggml's CPU mul_mat for a quantized weight (src/lgml.c:1811-1839 on the
 * CPU backend [ggml]): each X row quantized to the weight type's
 * vec_dot_type (Q8_K for Q4_K / Q6_K, Q8_0 for Q8_0), then integer dot
 * products per block, scaled by the f32 products of the block scales, the
 * blocks added in f64. f32 weights: orc_mul_mat. */
int orc_mul_mat_q8(int type, const void *w, int64_t M, int64_t K, const float *x, int64_t N,
    float *y, int n_threads);
/* quantize_row_q8_K_ref [ggml]: per 256 values d (f32), q (int8), 16 sums
 * of 16 q. K a multiple of 256. */
void orc_quantize_q8_K(const float *x, int64_t K, int8_t *q, float *d, int16_t *bsums);
/* quantize_row_q8_0_ref [ggml]: per 32 values d (f16 bits), q (int8). */
void orc_quantize_q8_0_act(const float *x, int64_t K, int8_t *q, uint16_t *d);

/* The router of M.moe (transformer.lua:1998-2008): probs = soft_max (or
 * sigmoid) of each logits row (n_expert values, f64 sums); ids = the
 * n_used largest, largest first (argsort_top_k, src/ops_nn.c:266-286),
 * chosen on the logits (the gating is monotone), ties to the smaller
 * index; w = probs[ids], divided by max(sum, 6.103515625e-5) when
 * norm_topk, then times scale. ids, w: (n, n_used). */
int orc_moe_route(const float *logits, int64_t n, int n_expert, int n_used, int gating,
    int norm_topk, float scale, int32_t *ids, float *w);

/* ggml_mul_mat_id via graph:mul_mat_id (src/ops_nn.c:322-362): w holds
 * n_expert matrices (M, K) of `type`; row (t, j) of y (T, n_used, M) is
 * w[ids[t][j]] times x[t][j % U] (x is (T, U, K)). f64 accumulation.
 * Returns -1 on an id outside [0, n_expert). */
int orc_mul_mat_id(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const float *x, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    int n_threads);
/* The same with ggml's CPU arithmetic (orc_mul_mat_q8 per expert). */
int orc_mul_mat_id_q8(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const float *x, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    int n_threads);

/* The forward's row ops, one by one: rms_norm of rows of n values
 * (graph:rms_norm, src/lgml.c:1633; w may be NULL); rope of rows of
 * n_heads x D at pos[r] (graph:rope, src/lgml.c:2004-2081; ff may be NULL);
 * silu(g) u or, with use_gelu, gelu(g) u (transformer.lua:2048). */
void orc_rms_norm(const float *x, float *y, int64_t rows, int64_t n, float eps, const float *w);
void orc_rope(float *x, int64_t rows, int n_heads, int D, int n_rot, int neox, float base,
    const float *ff, const int32_t *pos);
void orc_glu(const float *g, const float *u, float *out, int64_t n, int use_gelu);

/* Greedy first-max argmax (src/sample.c:914-925). */
int32_t orc_argmax(const float *v, int64_t n);

#ifdef __cplusplus
}
#endif
#endif
