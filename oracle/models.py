"""Model weight builders for the oracle and the GPU path.

TEST INFRASTRUCTURE: the tiny models regenerate the reference's test
fixtures exactly, so the oracle can be pinned against its golden rows;
the config builders make the seeded random-init models that the tests
and bench.py feed to both the oracle and the GPU library.

A weights dict: {"tok_embd": (arr, type), "output": ..., "output_norm":
..., "rope_freqs": arr or None, "layers": [{name: (arr, type)}]} where a
quantized arr is uint8 (rows, row_bytes) and an f32 arr is (rows, cols).
"""
import math

import numpy as np

from . import core

LAYER_KEYS = ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm", "gate", "up",
              "down")


def ref_tiny(arch):
    """The tiny llama / qwen3 / qwen3moe of test/test_qwen_moe.lua:66-200 (build()).

    Seed #arch * 7919 (:70); tensors drawn in the order build() lists them
    (:140-195); w(): U(-s, s), s = gain * sqrt(3 / fan_in) (:88-91); norms
    U(0.9, 1.1) (:92-94); llama rope_freqs U(1, 8) x D/2 (:143-147). All
    stored as f32 (gguf.lua:41-50). Shapes: E=64, H=4, HKV=2, D=16,
    FF=2E, 2 layers, vocab 259 (:41-64,66,96-104), eps 1e-6, base 1e6.
    qwen3moe layers replace the dense FFN by X=8 experts of width F=32,
    USED=2 picks (:66,116-118,183-191): ffn_gate_inp (X, E) gain 3, then
    ffn_gate_exps / ffn_up_exps (X, F, E) and ffn_down_exps (X, E, F);
    softmax gating with norm_topk (transformer.lua:162-165 defaults).
    """
    assert arch in ("llama", "qwen3", "qwen3moe")
    E, H, HKV, D = 64, 4, 2, 16
    X, USED, FX = 8, 2, 32
    nv = 256 + 3
    r = core.Lcg(len(arch) * 7919)

    def w(rows, cols, gain=1.0):
        s = gain * math.sqrt(3.0 / cols)
        return (r.fill(rows * cols, -s, s).reshape(rows, cols), core.F32)

    def norm(d):
        return (r.fill(d, 0.9, 1.1), core.F32)

    out = {}
    out["tok_embd"] = w(nv, E, 3.0)
    out["output_norm"] = norm(E)
    out["output"] = w(nv, E)
    out["rope_freqs"] = None
    if arch == "llama":
        out["rope_freqs"] = r.fill(D // 2, 1.0, 8.0)
    layers = []
    for _ in range(2):
        L = {}
        L["attn_norm"] = norm(E)
        L["wq"] = w(H * D, E)
        L["wk"] = w(HKV * D, E)
        L["wv"] = w(HKV * D, E)
        L["wo"] = w(E, H * D)
        if arch != "llama":
            L["q_norm"] = norm(D)
            L["k_norm"] = norm(D)
        L["ffn_norm"] = norm(E)
        if arch == "qwen3moe":
            L["gate_inp"] = w(X, E, 3.0)
            L["gate_exps"] = w(X * FX, E)
            L["up_exps"] = w(X * FX, E)
            s = math.sqrt(3.0 / FX)
            L["down_exps"] = (r.fill(X * E * FX, -s, s).reshape(X * E, FX), core.F32)
        else:
            L["gate"] = w(2 * E, E)
            L["up"] = w(2 * E, E)
            L["down"] = w(E, 2 * E)
        layers.append(L)
    out["layers"] = layers
    hp = dict(arch=arch, n_layer=2, n_embd=E, n_head=H, n_head_kv=HKV, head_dim=D, n_ff=2 * E,
              n_vocab=nv, n_rot=D, eps=1e-6, rope_base=1e6, rope_neox=0 if arch == "llama" else 1,
              attn_scale=0.0)
    if arch == "qwen3moe":
        hp.update(n_expert=X, n_used=USED, n_ff_exp=FX, gating=core.GATING_SOFTMAX,
                  norm_topk=True, expert_scale=1.0)
    return hp, out


def ref_tiny_gemma4():
    """The tiny gemma4 "dense" model of test/test_gemma4.lua:38-174 (build("dense")).

    Seed #"dense" * 7919 (:58); tensors drawn in the order build() lists
    them (:120-171): w() is U(-s, s), s = gain * sqrt(3 / fan_in) (:72-79);
    norms U(0.8, 1.2) (:80-82). E=64, H=4, FF=96, vocab 289 (bpe_vocab
    gemma4_kv: 9 specials, 255 byte tokens, 13 chars, 10 merges, 2 more).
    Layer 0 slides (window 6, head 16, 2 KV heads, rope base 1e4); layer 1
    is global (head 32, 1 KV head, rope base 1e6, proportional rope: freq
    factors 1 for the first half of the pairs, 1e30 after (:123-128), no
    attn_v: V is the raw K). Layer output scales 0.8 + 0.3 i (:168), logit
    softcap 30, embeddings times sqrt(64), attention scale 1, tied output
    (transformer.lua:171-183,408).
    """
    E, H, D, DS, FF, NSWA = 64, 4, 32, 16, 96, 6
    nv = 9 + 255 + 13 + 10 + 2
    r = core.Lcg(len("dense") * 7919)

    def w(rows, cols, gain=1.0):
        s = gain * math.sqrt(3.0 / cols)
        return (r.fill(rows * cols, -s, s).reshape(rows, cols), core.F32)

    def norm(d):
        return (r.fill(d, 0.8, 1.2), core.F32)

    out = {"tok_embd": w(nv, E, 0.3), "output_norm": norm(E), "rope_freqs": None}
    out["output"] = out["tok_embd"]
    freqs = np.array([1.0 if i <= D // 4 else 1e30 for i in range(1, D // 2 + 1)], np.float32)
    swa, hkv = [True, False], [2, 1]
    layers = []
    for i in range(2):
        d = DS if swa[i] else D
        L = {"swa": int(swa[i]), "head_dim": d, "n_head_kv": hkv[i], "n_rot": d,
             "rope_base": 1e4 if swa[i] else 1e6}
        if not swa[i]:
            L["rope_freqs"] = freqs
        L["attn_norm"] = norm(E)
        L["wq"] = w(H * d, E)
        L["wk"] = w(hkv[i] * d, E)
        L["k_norm"] = norm(d)
        if swa[i]:
            L["wv"] = w(hkv[i] * d, E)
        L["wo"] = w(E, H * d)
        L["q_norm"] = norm(d)
        L["post_attn_norm"] = norm(E)
        L["ffn_norm"] = norm(E)
        L["gate"] = w(FF, E)
        L["up"] = w(FF, E)
        L["down"] = w(E, FF)
        L["post_ffn_norm"] = norm(E)
        L["out_scale"] = float(np.float32(0.8 + 0.3 * i))
        layers.append(L)
    out["layers"] = layers
    hp = dict(arch="gemma4", n_layer=2, n_embd=E, n_head=H, n_head_kv=hkv[1], head_dim=D,
              n_ff=FF, n_vocab=nv, n_rot=D, eps=1e-6, rope_base=1e6, rope_neox=1,
              attn_scale=1.0, gemma=True, n_swa=NSWA, embd_scale=float(np.float32(math.sqrt(E))),
              softcap=30.0)
    return hp, out


# Named model shapes of BASELINE.json's configs.
SHAPES = {
    # C1: tiny llama-style f32 model runnable on CPU.
    "c1": dict(arch="llama", n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_ff=688,
               n_vocab=512, rope_base=1e4, eps=1e-6, wtype="f32"),
    # C2: Llama-3-8B shape, Q4_K_M mix, f16 KV.
    "c2": dict(arch="llama", n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128,
               n_ff=14336, n_vocab=128256, rope_base=5e5, eps=1e-5, wtype="q4_K_M"),
    # C5: a 30B-A3B-shaped qwen3moe (Qwen3-30B-A3B sizes: vocab 151936, rope
    # base 1e6, eps 1e-6, q/k norms), 128 experts of width 768, top-8
    # softmax routing with norm_topk; Q4_K weights, f32 router.
    "c5": dict(arch="qwen3moe", n_layer=48, n_embd=2048, n_head=32, n_head_kv=4, head_dim=128,
               n_ff=768, n_vocab=151936, rope_base=1e6, eps=1e-6, wtype="q4_K", n_expert=128,
               n_used=8, n_ff_exp=768, gating=1, norm_topk=True, expert_scale=1.0),
    # C4: a Gemma-4-style model: 5 sliding-window layers (1024-token window,
    # rope base 1e4) to 1 global layer (rope base 1e6, proportional rope, V
    # from the raw K), q/k norms, V norm, post norms, GeGLU, layer output
    # scales, tied output, logit softcap 30; Q8_0 weights.
    "c4": dict(arch="gemma4", n_layer=26, n_embd=2560, n_head=8, n_head_kv=4, head_dim=256,
               n_ff=10240, n_vocab=262144, rope_base=1e6, eps=1e-6, wtype="q8_0", gemma=True,
               n_swa=1024, swa_period=6, rope_base_swa=1e4, softcap=30.0),
}


def gemma_layer(hp, il):
    """Per-layer structure of a gemma shape (transformer.lua:215-235,
    test/test_gemma4.lua:116-128): layer il slides unless il % swa_period
    == swa_period - 1; sliding layers use rope_base_swa and have attn_v;
    global layers use rope_base with proportional rope (factors 1 for the
    first head_dim / 4 pairs, 1e30 after) and take V from the raw K. Layer
    output scales 0.8 + 0.05 (il % 7)."""
    D, per = hp["head_dim"], hp["swa_period"]
    swa = il % per != per - 1
    L = {"swa": int(swa), "rope_base": hp["rope_base_swa"] if swa else hp["rope_base"],
         "out_scale": float(np.float32(0.8 + 0.05 * (il % 7))), "has_wv": swa}
    if not swa:
        L["rope_freqs"] = np.array([1.0 if i <= D // 4 else 1e30 for i in range(1, D // 2 + 1)],
                                   np.float32)
    return L


def more_bits(i, n):
    """lua/lgml/convert.lua:123-126: layers that get Q6_K in the _M mixes."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def weight_type(wtype, name, layer, n_layer):
    """lua/lgml/convert.lua:128-165 policies: 1-D tensors and the router
    stay f32; q4_K_M gives output Q6_K and attn_v / ffn_down (also the
    expert ffn_down_exps) Q6_K on more_bits layers."""
    if wtype == "f32" or name == "gate_inp":
        return core.F32
    if wtype == "q8_0":
        return core.Q8_0
    if wtype == "q4_K":
        return core.Q4_K
    if wtype == "q4_K_M":
        if name == "output":
            return core.Q6_K
        if layer is not None and name in ("wv", "down", "down_exps") and more_bits(layer, n_layer):
            return core.Q6_K
        return core.Q4_K
    raise ValueError(wtype)


def build(shape, seed=1234, n_layer=None, init="uniform"):
    """Seeded random-init weights for a named shape.

    init "uniform": C1's U(-s, s), s = sqrt(3 / fan_in) (as tiny.lua:102-108),
    norms U(0.9, 1.1), drawn from the reference LCG.
    init "normal": N(0, 0.02) weights from the reference splitmix64 +
    Box-Muller fill (src/lgml.c:3130-3136), one seed per tensor (seed + i),
    norms 1.0; quantized per the shape's weight policy. A MoE router is
    N(0, 1/sqrt(n_embd)), so that the logits of a unit-rms row are N(0, 1).
    n_layer overrides the depth (reduced-depth parity runs keep the width).
    """
    hp = dict(SHAPES[shape]) if isinstance(shape, str) else dict(shape)
    if n_layer is not None:
        hp["n_layer"] = n_layer
    hp.setdefault("n_rot", hp["head_dim"])
    hp["rope_neox"] = 0 if hp["arch"] == "llama" else 1
    gemma = hp["arch"] == "gemma4"
    # gemma: attention scale 1, embeddings times sqrt(n_embd) rounded to f32
    # (transformer.lua:171-183)
    hp["attn_scale"] = 1.0 if gemma else 0.0
    if gemma:
        hp["embd_scale"] = float(np.float32(math.sqrt(hp["n_embd"])))
    E, H, Hkv, D, F, V = (hp[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff",
                                          "n_vocab"))
    nl = hp["n_layer"]
    full_layers = SHAPES[shape]["n_layer"] if isinstance(shape, str) else nl
    wt = hp["wtype"]
    lcg = core.Lcg(seed)
    counter = [0]

    def mat(name, rows, cols, layer=None, gain=1.0):
        ty = weight_type(wt, name, layer, full_layers)
        if init == "uniform":
            s = gain * math.sqrt(3.0 / cols)
            x = lcg.fill(rows * cols, -s, s).reshape(rows, cols)
        else:
            counter[0] += 1
            tseed = seed * 1000003 + counter[0]
            sd = 1.0 / math.sqrt(E) if name == "gate_inp" else 0.02
            if ty == core.F32:
                return (core.gen_normal(rows * cols, 0.0, sd, tseed).reshape(rows, cols), ty)
            return (core.gen_normal_quant(ty, rows, cols, 0.0, sd, tseed), ty)
        if ty == core.F32:
            return (x, ty)
        return (core.quantize(ty, x), ty)

    def norm(d, mean=1.0):
        if init == "uniform":
            return (lcg.fill(d, 0.9 * mean, 1.1 * mean), core.F32)
        if gemma:  # norm weights N(mean, mean / 10): the post norms are then visible
            counter[0] += 1
            return (core.gen_normal(d, mean, 0.1 * mean, seed * 1000003 + counter[0]), core.F32)
        return (np.ones(d, np.float32), core.F32)

    # gemma attends at scale 1 to rms-normed q and k: q / k norm weights of
    # mean D^(-1/4) give scores of unit scale, as trained weights keep them
    # (with weights near 1 the scores of random heads have sd sqrt(D) = 16,
    # every softmax is nearly one-hot and a 1-ulp change of any weight moves
    # 6-layer logits by ~5e-3)
    qk_mean = D ** -0.25 if gemma else 1.0

    w = {}
    w["tok_embd"] = mat("tok_embd", V, E)
    w["output_norm"] = norm(E)
    # gemma ties the output to the embeddings (transformer.lua:408)
    w["output"] = w["tok_embd"] if gemma else mat("output", V, E)
    w["rope_freqs"] = None
    layers = []
    for il in range(nl):
        L = {}
        g = gemma_layer(hp, il) if gemma else {}
        L["attn_norm"] = norm(E)
        L["wq"] = mat("wq", H * D, E, il)
        L["wk"] = mat("wk", Hkv * D, E, il)
        if g.get("has_wv", True):
            L["wv"] = mat("wv", Hkv * D, E, il)
        L["wo"] = mat("wo", E, H * D, il)
        if hp["arch"] in ("qwen3", "qwen3moe", "gemma4"):
            L["q_norm"] = norm(D, qk_mean)
            L["k_norm"] = norm(D, qk_mean)
        if gemma:
            L["post_attn_norm"] = norm(E)
            L["post_ffn_norm"] = norm(E)
            for k in ("swa", "rope_base", "out_scale", "rope_freqs"):
                if k in g:
                    L[k] = g[k]
        L["ffn_norm"] = norm(E)
        if hp.get("n_expert"):
            NE, FX = hp["n_expert"], hp["n_ff_exp"]
            L["gate_inp"] = mat("gate_inp", NE, E, il)
            L["gate_exps"] = mat("gate_exps", NE * FX, E, il)
            L["up_exps"] = mat("up_exps", NE * FX, E, il)
            L["down_exps"] = mat("down_exps", NE * E, FX, il)
        else:
            L["gate"] = mat("gate", F, E, il)
            L["up"] = mat("up", F, E, il)
            L["down"] = mat("down", E, F, il)
        layers.append(L)
    w["layers"] = layers
    return hp, w
