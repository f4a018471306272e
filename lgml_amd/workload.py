"""Model shapes, weight-type policy and synthetic workloads of the benchmark
configurations (seeds recorded with each result).

Integers (lengths, ids, budgets) come from the reference's test LCG
(test/tiny.lua:16-22); weights from lgmlh_gen_normal (tensor:fill
"normal", src/lgml.c:3130-3136)."""

SHAPES = {
    # C2: Llama-3-8B shape, Q4_K_M mix, f16 KV.
    "c2": dict(arch="llama", n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128,
               n_ff=14336, n_vocab=128256, rope_base=5e5, eps=1e-5, n_rot=128, rope_neox=0,
               attn_scale=0.0, wtype="q4_K_M"),
    # C5: 30B-A3B-shaped qwen3moe, Q4_K, 128 experts of width 768, top-8.
    "c5": dict(arch="qwen3moe", n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, head_dim=128,
               n_ff=768, n_vocab=151936, rope_base=1e6, eps=1e-6, n_rot=128, rope_neox=1,
               attn_scale=0.0, wtype="q4_K", n_expert=128, n_used=8, n_ff_exp=768, gating=1,
               norm_topk=True, expert_scale=1.0),
    # C4: Gemma-4-style, 26 layers, 5 sliding-window (1024-token ring per
    # slot) : 1 global, head 256, Q8_0, tied output, logit softcap 30.
    "c4": dict(arch="gemma4", n_layer=26, n_embd=2560, n_head=8, n_head_kv=4, head_dim=256,
               n_ff=10240, n_vocab=262144, rope_base=1e6, eps=1e-6, n_rot=256, rope_neox=1,
               attn_scale=1.0, wtype="q8_0", gemma=True, n_swa=1024, swa_period=6,
               rope_base_swa=1e4, softcap=30.0, embd_scale=50.596443),
}

F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14


def more_bits(i, n):
    """lua/lgml/convert.lua:123-126: layers that get Q6_K in the _M mixes."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def policy(wtype, n_layer):
    """lua/lgml/convert.lua:128-165: weight type of matrix `name` of `layer`
    (None for the embeddings / output)."""
    def ty(name, layer):
        if wtype == "f32" or name == "gate_inp":  # the router stays f32
            return F32
        if wtype == "q8_0":
            return Q8_0
        if wtype == "q4_K":
            return Q4_K
        if name == "output":
            return Q6_K
        if layer is not None and name in ("wv", "down", "down_exps") and more_bits(layer, n_layer):
            return Q6_K
        return Q4_K
    return ty


class Lcg:
    """test/tiny.lua:16-22: x <- x * 6364136223846793005 + 1442695040888963407
    (mod 2^64), u = (x >> 11) / 2^53."""

    def __init__(self, seed):
        self.x = seed % 2**64

    def next(self):
        self.x = (self.x * 6364136223846793005 + 1442695040888963407) % 2**64
        return (self.x >> 11) / 2.0**53

    def int(self, lo, hi):
        """U[lo, hi] inclusive."""
        return lo + int(self.next() * (hi - lo + 1))


def gemma_layer(hp, il):
    """Layer il of a gemma shape (transformer.lua:215-235; the layer layout
    of test/test_gemma4.lua:116-128): it slides unless il % swa_period ==
    swa_period - 1. Sliding layers: rope base rope_base_swa, an attn_v.
    Global layers: rope base rope_base, proportional rope (factors 1 for
    the first head_dim / 4 pairs, 1e30 after: those pairs stay unrotated),
    V = the raw K. Layer output scales 0.8 + 0.05 (il % 7)."""
    import numpy as np
    D, per = hp["head_dim"], hp["swa_period"]
    swa = il % per != per - 1
    L = {"swa": int(swa), "rope_base": hp["rope_base_swa"] if swa else hp["rope_base"],
         "out_scale": float(np.float32(0.8 + 0.05 * (il % 7))), "has_wv": swa}
    if not swa:
        L["rope_freqs"] = np.array([1.0 if i <= D // 4 else 1e30 for i in range(1, D // 2 + 1)],
                                   np.float32)
    return L


def ring_blocks(hp, max_ubatch):
    """64-cell blocks of each sequence's ring (transformer.lua:575-581: the
    ring holds n_swa - 1 + ubatch positions)."""
    return (hp["n_swa"] - 1 + max_ubatch + 63) // 64


def expected_experts(hp, n_tokens):
    """Distinct experts a layer reads for n_tokens tokens under uniform
    routing: NE (1 - (1 - k / NE) ** n_tokens) (125.9 of 128 at 64 tokens)."""
    NE, k = hp["n_expert"], hp["n_used"]
    return NE * (1.0 - (1.0 - k / NE) ** n_tokens)


def weight_bytes(hp, n_tokens=64):
    """Bytes of the weights a decode step of n_tokens reads (all layer
    matrices and the output head; the embedding table is read only at the
    ubatch's ids; routed experts: the expected distinct experts per layer;
    gemma global layers have no attn_v)."""
    E, H, Hkv, D, F, V, L = (hp[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff",
                                             "n_vocab", "n_layer"))
    ty = policy(hp["wtype"], L)
    size = {F32: 4.0, Q8_0: 34 / 32, Q4_K: 144 / 256, Q6_K: 210 / 256}
    b = size[ty("output", None)] * V * E
    moe = bool(hp.get("n_expert"))
    for il in range(L):
        b += size[ty("wq", il)] * H * D * E + size[ty("wk", il)] * Hkv * D * E
        if not hp.get("gemma") or gemma_layer(hp, il)["has_wv"]:
            b += size[ty("wv", il)] * Hkv * D * E
        b += size[ty("wo", il)] * E * H * D
        if moe:
            FX = hp["n_ff_exp"]
            b += 4.0 * hp["n_expert"] * E  # router
            b += expected_experts(hp, n_tokens) * (
                (size[ty("gate_exps", il)] + size[ty("up_exps", il)]) * FX * E +
                size[ty("down_exps", il)] * E * FX)
        else:
            b += size[ty("gate", il)] * F * E + size[ty("up", il)] * F * E
            b += size[ty("down", il)] * E * F
    return int(b)


def expert_bytes(hp, n_tokens=64):
    """The routed-expert part of weight_bytes (0 for a dense model)."""
    if not hp.get("n_expert"):
        return 0
    ty = policy(hp["wtype"], hp["n_layer"])
    size = {F32: 4.0, Q8_0: 34 / 32, Q4_K: 144 / 256, Q6_K: 210 / 256}
    E, FX = hp["n_embd"], hp["n_ff_exp"]
    return int(sum(expected_experts(hp, n_tokens) * (
        (size[ty("gate_exps", il)] + size[ty("up_exps", il)]) * FX * E +
        size[ty("down_exps", il)] * E * FX) for il in range(hp["n_layer"])))
