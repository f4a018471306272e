/*
 * lgml_hip: MI355X (gfx950) kernels for lgml's ragged continuous-batching
 * decode/prefill path, behind a plain C ABI.
 *
 * Every entry point takes plain pointers and sizes, returns an int status
 * (LGMLH_OK = 0, negative on error, text in lgmlh_last_error()), never
 * longjmps, and never allocates device or host memory: callers pass
 * buffers and workspaces whose sizes the *_bytes / *_workspace functions
 * report. (One exception, stated at lgmlh_forward: a side stream and two
 * events per host thread, device and caller stream, made once and released
 * by lgmlh_forward_release.) Device pointers are HIP device addresses;
 * `stream` is a hipStream_t (NULL = the null stream). Calls on one stream
 * are ordered; calls on different streams that share a workspace race.
 *
 * Reference citations are paths under the lgml tree (mischief/lgml).
 */
#ifndef LGML_HIP_H
#define LGML_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LGMLH_ABI_VERSION 7

enum {
	LGMLH_OK = 0,
	LGMLH_EINVAL = -1, /* bad argument or shape (luaL_error "... shape mismatch") */
	LGMLH_ENOMEM = -2, /* workspace or buffer too small */
	LGMLH_EHIP = -3,   /* a HIP runtime call failed */
	LGMLH_EFULL = -4,  /* kv pool full (transformer.lua:975, "kv pool full") */
	LGMLH_ERANGE = -5  /* an index (cell, id, position) out of range */
};

/* Weight / element types, numbered as ggml's type ids. */
enum { LGMLH_F32 = 0, LGMLH_F16 = 1, LGMLH_Q8_0 = 8, LGMLH_Q4_K = 12, LGMLH_Q6_K = 14 };

/* Text of the last error on this thread (never NULL). */
const char *lgmlh_last_error(void);
int lgmlh_abi_version(void);

/* Bytes of one row of n values in `type` (src/lgml.c:3603-3619 row_size). */
int64_t lgmlh_row_size(int type, int64_t n);

/* ===================================================================== *
 * Paged KV pool.
 *
 * Replaces the pool tensors pool.k[il] / pool.v[il] of M:pool
 * (lua/lgml/transformer.lua:678-705), (cap, Hkv*D) f16 rows, with an
 * MI355X layout of 64-cell blocks (BLOCK, transformer.lua:30):
 *   K: [block][kv_head][cell % 64][D]   (a 64 x D tile per block and head)
 *   V: [block][kv_head][D][cell % 64]   (the same tile, transposed)
 * Cell c of the reference lives in block c / 64 at offset c % 64, so the
 * reference's cell ids (seq_cells, transformer.lua:1126-1133) are used
 * unchanged. One layer's K (or V) takes lgmlh_kv_layer_bytes bytes.
 * ===================================================================== */
int64_t lgmlh_kv_layer_bytes(int64_t n_cells, int n_head_kv, int head_dim);

/* The KV scatter of attention_batch (transformer.lua:2403-2409): two
 * graph:set_rows (src/lgml.c:1937-1969) into the pool. k_src, v_src are
 * (n, Hkv*D) f32 rows, stored as f16 (round to nearest even) at cells[j].
 * Errors: LGMLH_ERANGE (checked on the host) if a cell id is outside
 * [0, n_cells) -- the host copy h_cells is required for that check. */
int lgmlh_kv_store(void *kpool, void *vpool, int64_t n_cells, int n_head_kv, int head_dim,
    const float *k_src, const float *v_src, const int64_t *cells, const int64_t *h_cells,
    int64_t n, void *stream);

/* Read cells back as (n, Hkv*D) f16 rows in the reference row layout
 * (which = 0: K, 1: V). For tests, snapshots and host spill. */
int lgmlh_kv_gather(const void *pool, int which, int64_t n_cells, int n_head_kv, int head_dim,
    const int64_t *cells, int64_t n, uint16_t *out, void *stream);

/* Copy the first n cells of block src to block dst in one layer's K and V
 * (M.copy_block, transformer.lua:989-1007, without the host round trip). */
int lgmlh_kv_copy_block(void *kpool, void *vpool, int64_t n_cells, int n_head_kv, int head_dim,
    int32_t src, int32_t dst, int n, void *stream);

/* Bytes of one 64-cell block of one layer's K (or V): 64 * Hkv * D * 2. A
 * pool block's cells in all layers (M.block_bytes, transformer.lua:
 * 1036-1042) are that times the number of pool tensors. */
int64_t lgmlh_kv_block_bytes(int n_head_kv, int head_dim);

/* M.copy_block_host (transformer.lua:1044-1060) in one launch: block
 * `block` of every pool tensor pools[0..n_pools) (a DEVICE array of the
 * tensors' addresses, e.g. K and V of each layer in order) to host memory
 * (out = 1) or back (out = 0), tensor p at host + p * lgmlh_kv_block_bytes.
 * host must be device-accessible (pinned: hipHostMalloc, or device memory)
 * and 16-byte aligned. The spill / unspill of E:spill_block / E:unspill
 * (engine.lua:1845-1868). */
int lgmlh_kv_block_host(void *const *pools, int n_pools, int64_t n_cells, int n_head_kv,
    int head_dim, int32_t block, void *host, int out, void *stream);

/* pool_grow (transformer.lua:831-908) on the device: a pool of old_cells
 * into a new tensor of new_cells (both multiples of 64), cell ids kept
 * (the block layout makes the old pool a prefix of the new); the new
 * cells start zeroed. No host round trip. */
int lgmlh_kv_grow(const void *old_pool, int64_t old_cells, void *new_pool, int64_t new_cells,
    int n_head_kv, int head_dim, void *stream);

/* Plain ggml_set_rows on a row-major f16 tensor: dst[ids[j]] = f16(src[j])
 * (src/lgml.c:1937-1969). h_ids is the host copy for the range check. */
int lgmlh_set_rows_f16(uint16_t *dst, int64_t dst_rows, int64_t row, const float *src,
    const int64_t *ids, const int64_t *h_ids, int64_t n, void *stream);

/* ===================================================================== *
 * Pool bookkeeping (host): lua/lgml/kvpool.lua in C. All state lives in
 * one caller buffer of lgmlh_kvpool_bytes(blocks, size) bytes. Block ids
 * count from 0; priorities are LOW 0, NORMAL 1, HIGH 2 (kvpool.lua:25).
 * Lua's pairs() order leaves exact ties of evict / longest_kid open; here
 * they go to the lowest block id.
 * ===================================================================== */
size_t lgmlh_kvpool_bytes(int32_t blocks, int32_t size);
/* M.new (kvpool.lua:65-72): blocks of size cells, cap usable. */
int lgmlh_kvpool_init(void *mem, size_t bytes, int32_t blocks, int32_t size, int32_t cap);
/* P:take (kvpool.lua:102-116): the lowest free block from min up, else the
 * lowest one; -1 when none is free below cap. */
int32_t lgmlh_kvpool_take(void *pool, int32_t min);
/* P:evict (kvpool.lua:139-160): the cached block of the lowest priority,
 * least recently used, deepest; it loses its key. -1 when none. */
int32_t lgmlh_kvpool_evict(void *pool);
/* The block the next lgmlh_kvpool_evict takes (-1 if none) and its
 * priority, nothing changed: the on_evict moment of kvpool.lua:149-152,
 * when the owner copies a keyed block's cells out before it loses its key. */
int32_t lgmlh_kvpool_victim(void *pool, int32_t *prio);
/* P:ref / P:unref / P:refs_of (kvpool.lua:165-205). */
int lgmlh_kvpool_ref(void *pool, int32_t b, int prio);
int lgmlh_kvpool_unref(void *pool, int32_t b);
int32_t lgmlh_kvpool_refs_of(void *pool, int32_t b);
/* P:publish (kvpool.lua:217-226): 1 when b got the key, 0 when b or the
 * key already had one. P:publish_part (:239-249) likewise. */
int lgmlh_kvpool_publish(void *pool, int32_t b, const char *key, const char *parent,
    int32_t depth, const int32_t *tokens, int32_t n, int prio);
int lgmlh_kvpool_publish_part(void *pool, int32_t b, const char *parent, int32_t depth,
    const int32_t *tokens, int32_t n, int prio);
/* P:key_of (kvpool.lua:254-256): 0 none, 1 a key (64 hex digits + NUL to
 * out), 2 the partial-block marker. */
int lgmlh_kvpool_key_of(void *pool, int32_t b, char *out);
/* P:lookup (kvpool.lua:261-263): the block with key, or -1. */
int32_t lgmlh_kvpool_lookup(void *pool, const char *key);
/* P:longest_kid (kvpool.lua:273-285) on tokens[0..max): block or -1, and
 * the shared token count in *shared. */
int32_t lgmlh_kvpool_longest_kid(void *pool, const char *parent, const int32_t *tokens,
    int32_t max, int32_t *shared);
/* P:set_cap (kvpool.lua:289-293). */
int lgmlh_kvpool_set_cap(void *pool, int32_t cap);
/* out[8]: n, size, cap, used, low, cached, tick, evicted. */
int lgmlh_kvpool_stats(void *pool, int64_t *out);
/* M.key (kvpool.lua:51-59): sha256 hex of parent "," t0 "," t1 ... (65 bytes). */
int lgmlh_block_key(const char *parent, const int32_t *tokens, int32_t n, char *out);

/* ===================================================================== *
 * Ubatch plan: the packing of fill_batch / batch_inputs
 * (transformer.lua:2433-2551) plus the attention work list.
 *
 * A pass runs n_seq sequences; sequence s has seq_n[s] tokens at positions
 * seq_npast[s] + j and a block table of max_blocks entries
 * (block_tab[s * max_blocks + i] = block of positions [64 i, 64 i + 64)).
 * lgmlh_plan fills one host buffer that the caller copies to the device
 * unchanged; lgmlh_plan_bind turns a device copy into the device views.
 * ===================================================================== */
typedef struct {
	int32_t n_seq, n_tokens, max_blocks, block;
	int32_t n_items, n_merge, rows, n_head_kv; /* attention work sizes */
	int64_t bytes;                             /* bytes of the plan buffer */
	/* byte offsets of the arrays inside the plan buffer */
	int64_t off_ids, off_pos, off_cells, off_seq_off, off_npast, off_block_tab, off_logit_rows,
	    off_items, off_merge;
	int32_t window, ring;  /* a ring plan (lgmlh_plan_ring): window, ring blocks; else 0 */
	/* items [0, n_single) are query groups on their own; the rest come in
	 * shared runs of consecutive items, {first item, count} at off_shared */
	int32_t n_single, n_shared;
	int64_t off_shared;
	int64_t off_order; /* [n_single] dispatch order of the items on their own */
} lgmlh_plan_info;

typedef struct {
	int32_t n_seq, n_tokens, max_blocks, block;
	int32_t n_items, n_merge, rows, n_head_kv;
	const int32_t *ids;        /* [n_tokens] token ids, sequences in pass order */
	const int32_t *pos;        /* [n_tokens] n_past + j (fill_batch :2446-2451) */
	const int64_t *cells;      /* [n_tokens] pool cells (seq_cells) */
	const int32_t *seq_off;    /* [n_seq + 1] first token of each sequence */
	const int32_t *seq_npast;  /* [n_seq] */
	const int32_t *block_tab;  /* [n_seq * max_blocks] */
	const int32_t *logit_rows; /* [n_seq] off + n - 1 (batch_inputs :2540-2545) */
	const int32_t *items;      /* [n_items * 4] attention work items */
	const int32_t *merge;      /* [n_merge * 4] split-merge groups */
	int32_t window, ring;      /* ring plans: the window and the ring's blocks; else 0 */
	int32_t n_single, n_shared;
	const int32_t *shared;     /* [n_shared * 2] {first item, count} of each shared run */
	/* [n_single] the items on their own in the order the attention kernel
	 * starts them (longest run first, then by index); NULL: index order.
	 * Only which workgroup runs an item depends on it, not its result. */
	const int32_t *order;
} lgmlh_ubatch;

/* Plan a pass. G = n_head / n_head_kv; blocks_per_split bounds the KV
 * blocks one work item reads (0 = the default, 16): a query group's blocks
 * go into the fewest such runs, of lengths that differ by at most one. A
 * sequence with several query groups in the pass (a prompt chunk) takes
 * them in sets of up to 8 consecutive groups with the runs of the set's
 * last token, so that one workgroup reads each block once for the set. The
 * work list depends only on each sequence's own tokens, so a sequence is
 * computed the same way alone or in any batch. With buf NULL only info is
 * filled (sizes); otherwise buf must hold info->bytes. Errors:
 * LGMLH_ERANGE when a block id that a position needs is outside
 * [0, pool_blocks) (the fill_blocks "position ... is in no column" error,
 * src/lgml.c:3003-3008), or a position passes 65535 blocks. */
int lgmlh_plan(int n_seq, const int32_t *seq_n, const int32_t *seq_npast,
    const int32_t *block_tab, int max_blocks, int64_t pool_blocks, const int32_t *ids,
    int n_head, int n_head_kv, int blocks_per_split, void *buf, size_t buf_bytes,
    lgmlh_plan_info *info);
/* The plan of a pass over the sliding-window layers (transformer.lua:
 * 2464-2476, tensor_fill_mask with window and ring, src/lgml.c:2873-2935):
 * sequence s keeps a ring of ring_blocks blocks, ring_tab[s * ring_blocks
 * + i]; position p lives in cell ring_tab[s * ring_blocks + (p / 64) %
 * ring_blocks] * 64 + p % 64 (rows_swa = p % ring, ring = 64 ring_blocks
 * cells). Query p sees positions max(0, p - window + 1)..p. The ring must
 * hold window - 1 + seq_n[s] cells (the "tokens in one pass" error of
 * transformer.lua:1544-1546, LGMLH_ERANGE). block_tab / max_blocks of the
 * resulting plan are the ring tables; items hold logical block ranges. */
int lgmlh_plan_ring(int n_seq, const int32_t *seq_n, const int32_t *seq_npast,
    const int32_t *ring_tab, int ring_blocks, int64_t pool_blocks, int window, const int32_t *ids,
    int n_head, int n_head_kv, int blocks_per_split, void *buf, size_t buf_bytes,
    lgmlh_plan_info *info);
/* Device views of a plan buffer at dev (a device copy of buf). */
int lgmlh_plan_bind(const lgmlh_plan_info *info, const void *dev, lgmlh_ubatch *ub);

/* ===================================================================== *
 * Paged GQA attention: the per-sequence graph:flash_attn
 * (src/lgml.c:2121-2170) over the fill_blocks mask (src/lgml.c:2936-3017)
 * of attention_batch (transformer.lua:2389-2416), for all sequences of a
 * pass in one launch. Query row t (sequence s, position npast + j) sees
 * exactly the cells of positions 0..npast+j of s, read through its block
 * table; other cells are never read (the mask made them -inf).
 * q: (n_tokens, H, D) f32; out: (n_tokens, H, D) f32 written in place in
 * pass order (the concat chain of :2413 is not needed). K/V from the pool
 * layout above. scale: 1/sqrt(D) for llama (transformer.lua:1845).
 * D in {64, 128, 256}; H a multiple of Hkv with H/Hkv in {1, 2, 4, 8, 16}.
 * ===================================================================== */
size_t lgmlh_attention_workspace(const lgmlh_plan_info *info, int head_dim);
int lgmlh_paged_attention(const float *q, int n_head, int n_head_kv, int head_dim, float scale,
    const void *kpool, const void *vpool, const lgmlh_ubatch *ub, float *out, void *workspace,
    size_t workspace_bytes, void *stream);

/* graph:flash_attn(q, k, v, mask, scale, max_bias, softcap)
 * (src/lgml.c:2121-2170) over strided K / V views with an explicit mask:
 * the compatibility entry for attention outside the paged pool (e.g. M.attend
 * on kv.for_flash views, kv.lua:141-147, under fill_causal / fill_mask
 * masks, src/lgml.c:2836-2935). For query row t of head h and column j:
 * s = scale q.k_j; with softcap > 0, s = softcap tanh(s / softcap); then
 * s += slope_h mask[h % mask_heads][t][j] (slope 1, or ALiBi's when
 * max_bias > 0); out = softmax(s) v. A -inf mask drops the column; a row
 * with every column dropped gives zeros. q (H, T, D) f32; K / V element
 * (hk, j, d) at k[hk * k_head_stride + j * k_row_stride + d] f16 (strides
 * in elements, K 16-byte aligned with strides multiples of 8); mask
 * (mask_heads, mask_rows >= T, n_kv) contiguous f16 or NULL; out (T, H, D)
 * f32 (heads and tokens swapped, as the reference returns). Head h reads
 * kv head h / (H / Hkv). D a multiple of 8 up to 256. */
int lgmlh_flash_attn(const float *q, int n_head, int n_tokens, int head_dim, const uint16_t *k,
    const uint16_t *v, int n_head_kv, int n_kv, int64_t k_row_stride, int64_t k_head_stride,
    int64_t v_row_stride, int64_t v_head_stride, const uint16_t *mask, int mask_heads,
    int mask_rows, float scale, float max_bias, float softcap, float *out, void *stream);

/* ===================================================================== *
 * Weight matrix products: graph:mul_mat (src/lgml.c:1811-1839), ggml
 * convention: W (M, K) rows of `type`, X (N, K) -> Y (N, M) f32.
 * Quantized weights are first repacked (once, at load) from the ggml
 * block layout into row tiles of 16 rows (as ggml's CPU backend repacks
 * into interleaved buffers); the values are the same bytes, permuted.
 * F32 weights are used in place (no repack).
 * ===================================================================== */
int64_t lgmlh_repacked_bytes(int type, int64_t M, int64_t K);
int lgmlh_repack(int type, int64_t M, int64_t K, const void *src, void *dst, void *stream);

/* Dequantize rows [0, M) of a ggml-layout matrix to f32 (M, K); the
 * closed form of the block format, bit-exact with the CPU reference. */
int lgmlh_dequantize(int type, const void *src, int64_t M, int64_t K, float *out, void *stream);

enum { LGMLH_EPI_NONE = 0, LGMLH_EPI_ADD = 1 };

/* Workspace of a call: the split-K partial sums (0 bytes when K is not
 * split). Its contents need no initialisation. */
size_t lgmlh_mul_mat_workspace(int type, int64_t M, int64_t K, int64_t N);
/* y = X W^T (+ residual when epi == LGMLH_EPI_ADD; residual may alias y).
 * x is f32 or f16 (xtype). Quantized types take the repacked w. The
 * result of an output element does not depend on N or on the other rows
 * of X (fixed summation order), so a row gives the same bits alone or in
 * any batch. */
int lgmlh_mul_mat(int type, const void *w, int64_t M, int64_t K, const void *x, int xtype,
    int64_t N, float *y, int epi, const float *residual, void *workspace, size_t ws_bytes,
    void *stream);

/* Activation arithmetic of quantized products. LGMLH_ACT_EXACT: X stays
 * f32-accurate (f16 hi + lo halves against exact integer weights).
 * LGMLH_ACT_GGML: the reference CPU path's arithmetic [ggml mul_mat on the
 * CPU backend]: each X row is first quantized to the weight type's
 * vec_dot_type -- Q8_K (256-value blocks: f32 d, int8 q, 16 sums of 16) for
 * Q4_K / Q6_K, Q8_0 (32-value blocks: f16 d, int8 q) for Q8_0 -- and the
 * products are integer block dots scaled by d_w d_x. f32 weights take f32
 * X in either mode. */
enum { LGMLH_ACT_EXACT = 0, LGMLH_ACT_GGML = 1 };

/* lgmlh_mul_mat in LGMLH_ACT_GGML arithmetic: graph:mul_mat
 * (src/lgml.c:1811-1839) as the reference's CPU backend computes it.
 * Same arguments, workspace and batch invariance as lgmlh_mul_mat. */
int lgmlh_mul_mat_ggml(int type, const void *w, int64_t M, int64_t K, const void *x, int xtype,
    int64_t N, float *y, int epi, const float *residual, void *workspace, size_t ws_bytes,
    void *stream);
/* The activation blocks of LGMLH_ACT_GGML for X (N, K) f32 and a weight
 * of `type` (quantize_row_q8_K / quantize_row_q8_0 of ggml's CPU path, as
 * the vec_dot_type conversion before mul_mat, src/lgml.c:1811-1839):
 * Q4_K / Q6_K: q (N, K) int8, d (N, K / 256) f32, bsums (N, K / 16) int16;
 * Q8_0: q (N, K) int8, d (N, K / 32) f16 bits, bsums unused (may be NULL).
 * Device pointers. */
int lgmlh_quantize_act(int type, const float *x, int64_t N, int64_t K, int8_t *q, void *d,
    int16_t *bsums, void *stream);

/* lgmlh_mul_mat without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc). It has no counterpart in the reference. The workspace lives
 * in a static device array of lgmlh_mul_mat_noalloc_limit() bytes (32 MiB)
 * that each GPU holds until the process ends; a product whose
 * lgmlh_mul_mat_workspace exceeds it fails with LGMLH_ENOMEM. Calls that
 * overlap on one GPU (other streams or threads) race for the array.
 * Results are those of lgmlh_mul_mat, bit for bit. */
size_t lgmlh_mul_mat_noalloc_limit(void);
int lgmlh_mul_mat_noalloc(int type, const void *w, int64_t M, int64_t K, const void *x,
    int xtype, int64_t N, float *y, int epi, const float *residual, void *stream);

/* ===================================================================== *
 * Routed experts (qwen3moe): the router of M.moe (transformer.lua:
 * 1989-2027) and graph:mul_mat_id (src/ops_nn.c:322-362) with the weighted
 * sum of the picks (experts / sum_picks, transformer.lua:1875-1910).
 * ===================================================================== */
/* Expert gating functions, as gguf expert_gating_func numbers
 * (transformer.lua:32-35). */
enum { LGMLH_GATING_SOFTMAX = 1, LGMLH_GATING_SIGMOID = 2 };

/* The router tail of M.moe (transformer.lua:1998-2008): for each row of
 * logits (n, n_expert) f32, probs = soft_max (or sigmoid); ids (n, n_used)
 * = the n_used largest, largest first (g:argsort_top_k,
 * src/ops_nn.c:266-286), ties to the smaller index, chosen on the logits
 * (the gating is monotone); weights (n, n_used) = probs[ids]
 * (get_rows), divided by max(sum, 6.103515625e-5) when norm_topk, then
 * times scale (expert_scale). n_expert <= 512, n_used <= 16,
 * n * n_used <= 8192. */
int lgmlh_moe_route(const float *logits, int64_t n, int n_expert, int n_used, int gating,
    int norm_topk, float scale, int32_t *ids, float *weights, void *stream);

/* Workspace of lgmlh_mul_mat_id (the grouping of the picks by expert and,
 * for quantized weights, the split X). Its contents need no
 * initialisation. */
size_t lgmlh_mul_mat_id_workspace(int type, int64_t n_expert, int64_t M, int64_t K, int64_t T,
    int64_t U, int n_used);
/* graph:mul_mat_id (src/ops_nn.c:322-362): w holds n_expert matrices
 * (M, K) of `type`, each repacked (lgmlh_repack) and stored one after the
 * other, lgmlh_repacked_bytes(type, M, K) apart (f32: M * K floats
 * apart); x (T, U, K) f32 (or f16 for quantized w); ids (T, n_used) i32
 * on the device; row (t, j) of y (T, n_used, M) f32 = w[ids[t, j]] times
 * x[t, j % U]. U is 1 or n_used. Each expert's rows are read once per
 * 16 (or 64) of its picks; an expert nobody picked costs nothing. ids
 * outside [0, n_expert) give rows of zeros (the reference asserts).
 * n_expert <= 512, T * n_used <= 8192. */
int lgmlh_mul_mat_id(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const void *x, int xtype, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    void *workspace, size_t ws_bytes, void *stream);
/* lgmlh_mul_mat_id in LGMLH_ACT_GGML arithmetic (ggml_mul_mat_id on the
 * CPU backend, src/ops_nn.c:322-362): each X row quantized to the expert
 * type's vec_dot_type, integer block dots. Same arguments and workspace. */
int lgmlh_mul_mat_id_ggml(int type, const void *w, int64_t n_expert, int64_t M, int64_t K,
    const void *x, int xtype, int64_t U, const int32_t *ids, int64_t T, int n_used, float *y,
    void *workspace, size_t ws_bytes, void *stream);
/* The tail of experts / sum_picks (transformer.lua:1888,1894-1910) and the
 * residual add of ffn (:2079): out[t] = y[t, 0] w[t, 0] + y[t, 1] w[t, 1]
 * + ... (+ residual[t]), products and sums in pick order. y (T, n_used, M),
 * weights (T, n_used); residual may be NULL or alias out. */
int lgmlh_moe_sum(const float *y, const float *weights, int64_t T, int n_used, int64_t M,
    const float *residual, float *out, void *stream);

/* ===================================================================== *
 * Dense-layer ops around the hot ops (transformer.lua:1754-1789,
 * 1859-1872, 2042-2104).
 * ===================================================================== */
/* get_rows of a (rows, n_cols) table in `type` (ggml layout): out f32. */
int lgmlh_get_rows(int type, const void *table, int64_t n_rows, int64_t n_cols,
    const int32_t *ids, const int32_t *h_ids, int64_t n, float *out, void *stream);
/* rms_norm(x) * w per row (graph:rms_norm, src/lgml.c:1633); out f32 or f16. */
int lgmlh_rms_norm(const float *x, int64_t n_rows, int64_t n, float eps, const float *w,
    void *out, int out_type, void *stream);
/* The qkv tail (transformer.lua:1776-1788): optional per-head rms_norm with
 * q_norm / k_norm, rope (graph:rope, src/lgml.c:2004-2081: mode normal or
 * neox, freq factors), then the KV store of k and v at cells. q is roped
 * in place. qkv is (n, (H + 2 Hkv) * D) f32 with [q | k | v] per row. A
 * cell outside [0, n_cells) is not written (cells are device data here). */
int lgmlh_qkv_rope_store(float *qkv, int64_t n, int n_head, int n_head_kv, int head_dim,
    int n_rot, int neox, float freq_base, const float *freq_factors, const float *q_norm,
    const float *k_norm, float eps, const int32_t *pos, void *kpool, void *vpool,
    int64_t n_cells, const int64_t *cells, float *q_out, void *stream);
/* silu(g) * u (transformer.lua:2048) for gu = (n, 2F) rows [g | u]; out f32 or f16. */
int lgmlh_swiglu(const float *gu, int64_t n, int64_t F, void *out, int out_type, void *stream);
/* gelu(g) * u, the gemma FFN (graph:geglu_split, src/ops_nn.c:165-172;
 * transformer.lua:2048): gelu in ggml's tanh form. Same layout as swiglu. */
int lgmlh_geglu(const float *gu, int64_t n, int64_t F, void *out, int out_type, void *stream);
/* The final logit softcap (transformer.lua:2097-2099): x = cap * tanh(x *
 * (1 / cap)) in place, n values. */
int lgmlh_softcap(float *x, int64_t n, float cap, void *stream);
/* Greedy id of each row: the first index of the maximum (src/sample.c:914-925). */
int lgmlh_argmax(const float *x, int64_t n_rows, int64_t n_cols, int32_t *out, void *stream);

/* Seeded random-init weights in a ggml layout (rows x cols of `type`,
 * F32 / Q4_K / Q6_K / Q8_0): N(mean, sd) values of tensor:fill("normal")
 * (src/lgml.c:3130-3136, splitmix64 + Box-Muller, value i from draws
 * 2i+1 and 2i+2 after seed) quantized by this library's own quantizer
 * (the role of lgml.quantize, src/quant.c:107). */
int lgmlh_gen_normal(uint64_t seed, int type, int64_t rows, int64_t cols, double mean, double sd,
    void *out, void *stream);

/* ===================================================================== *
 * One forward pass of a llama / qwen3 / qwen3moe model over a planned ubatch:
 * transformer.lua forward (:2285-2365) with the batched attention of
 * attention_batch (:2389-2416), for every sequence of the pass at once.
 * Weights are device pointers: quantized matrices repacked, f32 in place.
 * wqkv holds the rows of [wq | wk | wv] (or [wq | wk] with wv separate
 * when its type differs, as in the Q4_K_M mix); wgu holds [gate | up].
 * ===================================================================== */
typedef struct {
	const float *attn_norm, *ffn_norm, *q_norm, *k_norm; /* q/k_norm may be NULL */
	int wqkv_type, wv_type, wo_type, wgu_type, wdown_type;
	int64_t wqkv_rows;       /* rows of wqkv: (H + 2 Hkv) D, or (H + Hkv) D */
	const void *wqkv, *wv, *wo, *wgu, *wdown; /* wv NULL when inside wqkv */
	void *kpool, *vpool;     /* this layer's pool tensors */
	/* Routed experts (transformer.lua:2054-2068), used when gate_inp is set
	 * (wgu / wdown are then unused): the router (n_expert, n_embd) f32;
	 * exp_gu n_expert matrices [gate | up] (2 n_ff_exp, n_embd) and
	 * exp_down n_expert matrices (n_embd, n_ff_exp), as lgmlh_mul_mat_id
	 * takes them. */
	const float *gate_inp;
	int exp_gu_type, exp_down_type;
	const void *exp_gu, *exp_down;
	/* Gemma and sliding-window layers (transformer.lua:171-183,215-235,
	 * 300-333). swa: K / V in the ring pools (kpool / vpool hold ring
	 * blocks), attention through the ring plan. v_from_k: wqkv holds
	 * [wq | wk] only and V is the raw K (:1779). post_attn_norm /
	 * post_ffn_norm: rms-norm weights of the attention / FFN outputs before
	 * the residual add (NULL = none). out_scale: the layer output scale
	 * (0 = none). rope_base / rope_freqs: this layer's rope (0 / NULL = the
	 * model's). */
	int swa, v_from_k;
	const float *post_attn_norm, *post_ffn_norm;
	float out_scale, rope_base;
	const float *rope_freqs;
	/* This layer's head size, KV heads and rotated dimensions (0 = the
	 * model's; n_rot 0 with head_dim set = head_dim): gemma's sliding and
	 * global layers differ (transformer.lua:215-235). The plan a layer
	 * attends through (the ring plan for a sliding layer) must be made for
	 * its KV heads; its pool tensors hold rows of n_head_kv x head_dim. */
	int head_dim, n_head_kv, n_rot;
} lgmlh_layer;

typedef struct {
	int n_layer, n_embd, n_head, n_head_kv, head_dim, n_ff, n_vocab, n_rot, rope_neox;
	float eps, rope_base, attn_scale; /* attn_scale 0: 1 / sqrt(head_dim) */
	const float *rope_freqs;          /* n_rot / 2 factors or NULL */
	int tok_embd_type, output_type;
	const void *tok_embd;             /* ggml row layout (get_rows) */
	const void *output;               /* repacked (or f32) */
	const float *output_norm;
	int64_t n_cells;                  /* pool cells per layer */
	const lgmlh_layer *layers;        /* host array of n_layer */
	/* MoE (transformer.lua:160-170): experts, picks per token, expert FFN
	 * width, LGMLH_GATING_*, norm_topk, expert_scale. */
	int n_expert, n_used, n_ff_exp, gating, norm_topk;
	float expert_scale;
	/* Gemma (transformer.lua:171-183): V rms-normed, GeGLU FFN, embeddings
	 * times embd_scale (0 = none), logits softcapped (softcap 0 = none).
	 * ring_cells: cells of each sliding layer's ring pools. */
	int gemma;
	float embd_scale, softcap;
	int64_t ring_cells;
	/* LGMLH_ACT_EXACT or LGMLH_ACT_GGML: the arithmetic of every quantized
	 * weight product of the pass (the router stays f32). */
	int act;
} lgmlh_model;

/* Workspace bytes of lgmlh_forward for a plan and n_out logit rows. Its
 * contents need no initialisation; one workspace (grown when a larger pass
 * needs more) serves passes of any size on one stream. */
size_t lgmlh_forward_workspace(const lgmlh_model *m, const lgmlh_plan_info *info,
    const lgmlh_plan_info *info_ring, int n_out);
/* Optional timing: hipEvent_t handles (created by the caller), two per
 * slot, recorded on the pass's stream right before and after each traced
 * launch group. kinds: LGMLH_TRACE_ATTN (paged attention + merge, one slot
 * per layer), LGMLH_TRACE_GEMM (each dense weight product and the MoE
 * router), LGMLH_TRACE_EXPERTS (each grouped expert product). used counts
 * slots; a pass stops recording when capacity runs out. */
enum { LGMLH_TRACE_ATTN = 1, LGMLH_TRACE_GEMM = 2, LGMLH_TRACE_EXPERTS = 4 };
typedef struct {
	void *const *events; /* 2 * capacity hipEvent_t */
	int32_t capacity, used, kinds;
	int32_t *kind;       /* per slot: the kind recorded (may be NULL) */
} lgmlh_trace;

/* Run the pass: logits (n_out, n_vocab) f32 for the ubatch rows out_rows
 * (device; NULL = ub->logit_rows with n_out = n_seq). ids must be in range
 * (checked by the caller's plan, h_ids) -- the kernel reads them unchecked.
 * ub_ring: the ring plan of the same pass (lgmlh_plan_ring), needed when
 * a layer slides (NULL otherwise). trace may be NULL. A layer whose V
 * matrix has a type of its own runs that product on a side stream beside
 * the q|k product (not while tracing): the first such pass on a host
 * thread, device and caller stream creates that side stream (non-blocking,
 * default priority) and two events, kept until lgmlh_forward_release or
 * the process ends; passes on different caller streams (up to 4 per
 * thread and device) get side streams of their own, so that neither's side
 * products queue behind the other's. If creating them fails, or a fifth
 * caller stream asks, the pass runs on the caller's stream alone. */
int lgmlh_forward(const lgmlh_model *m, const lgmlh_ubatch *ub, const lgmlh_ubatch *ub_ring,
    const int32_t *out_rows, int n_out, float *logits, void *workspace, size_t ws_bytes,
    lgmlh_trace *trace, void *stream);
/* Destroy the side streams and events that lgmlh_forward made for the
 * calling thread on the current device (after the work queued on each
 * stream ends); nothing to do when it made none. A later pass makes them
 * again. For hosts that tear a thread's device context down (the
 * counterpart of backend:close / the backend's last release,
 * src/lgml.c:50-66,535-545). */
int lgmlh_forward_release(void);

#ifdef __cplusplus
}
#endif
#endif
