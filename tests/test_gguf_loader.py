"""The gguf loader (lgml_amd/gguf.py) end to end on the CPU.

The reference's tiny llama / qwen3 / qwen3moe / gemma4 models are written
as gguf files with the key-values and tensor names of its own tests
(test/test_qwen_moe.lua:65-200, test/test_gemma4.lua:84-174, encoded as
test/gguf.lua does), loaded back with lgml_amd.gguf.load, and run on the
oracle: they must reproduce the reference's golden rows (REF.llama,
REF.qwen3, REF.qwen3moe, REF.dense; TOL 2e-3 and the greedy ids). That pins
the key mapping (M.config), the tensor names and orientation (M.load /
M.load_layer), rope_freqs on llama vs the global gemma layers only, V = K
where a gemma layer has no attn_v, per-layer KV heads and head sizes, the
layer output scale tensor and the tied output. Quantized tensors come
back with their bytes unchanged.
"""
import numpy as np
import pytest

from lgml_amd import gguf
from oracle import core, models
from tests import gguf_util as gw
from tests import test_oracle_golden as tg


def tensors_of(arch, hp, w, gemma=False):
    """(name, torch shape, data, type) of a weights dict, as the reference's
    tests name them."""
    ts = []

    def t(name, key_or_arr, shape=None, ty=core.F32):
        arr = key_or_arr
        ts.append((name, list(shape if shape is not None else arr.shape), arr, ty))

    E = hp["n_embd"]
    t("token_embd.weight", w["tok_embd"][0])
    t("output_norm.weight", w["output_norm"][0])
    if not gemma:
        t("output.weight", w["output"][0])
    if w.get("rope_freqs") is not None:
        t("rope_freqs.weight", np.asarray(w["rope_freqs"], np.float32))
    if gemma:
        glob = [L for L in w["layers"] if not L["swa"]][0]
        t("rope_freqs.weight", np.asarray(glob["rope_freqs"], np.float32))
    names = {"attn_norm": "attn_norm", "wq": "attn_q", "wk": "attn_k", "wv": "attn_v",
             "wo": "attn_output", "q_norm": "attn_q_norm", "k_norm": "attn_k_norm",
             "ffn_norm": "ffn_norm", "gate": "ffn_gate", "up": "ffn_up", "down": "ffn_down",
             "gate_inp": "ffn_gate_inp", "post_attn_norm": "post_attention_norm",
             "post_ffn_norm": "post_ffw_norm"}
    for i, L in enumerate(w["layers"]):
        p = "blk.%d." % i
        for k, n in names.items():
            if k in L:
                t(p + n + ".weight", L[k][0])
        if "gate_exps" in L:
            X, F = hp["n_expert"], hp["n_ff_exp"]
            t(p + "ffn_gate_exps.weight", L["gate_exps"][0], (X, F, E))
            t(p + "ffn_up_exps.weight", L["up_exps"][0], (X, F, E))
            t(p + "ffn_down_exps.weight", L["down_exps"][0], (X, E, F))
        if gemma:
            t(p + "layer_output_scale.weight", np.array([L["out_scale"]], np.float32))
    return ts


def kv_qwen(arch, hp):
    """test/test_qwen_moe.lua:100-118 (the tokenizer keys left out)."""
    a = arch
    kv = [("general.architecture", gw.STRING, a), ("general.name", gw.STRING, "tiny " + a),
          (a + ".block_count", gw.U32, hp["n_layer"]), (a + ".context_length", gw.U32, 4096),
          (a + ".embedding_length", gw.U32, hp["n_embd"]),
          (a + ".feed_forward_length", gw.U32, 2 * hp["n_embd"]),
          (a + ".attention.head_count", gw.U32, hp["n_head"]),
          (a + ".attention.head_count_kv", gw.U32, hp["n_head_kv"]),
          (a + ".attention.key_length", gw.U32, hp["head_dim"]),
          (a + ".attention.value_length", gw.U32, hp["head_dim"]),
          (a + ".attention.layer_norm_rms_epsilon", gw.F32V, 1e-6),
          (a + ".rope.freq_base", gw.F32V, 1e6)]
    if hp.get("n_expert"):
        kv += [(a + ".expert_count", gw.U32, hp["n_expert"]),
               (a + ".expert_used_count", gw.U32, hp["n_used"]),
               (a + ".expert_feed_forward_length", gw.U32, hp["n_ff_exp"])]
    if a == "llama":
        kv.append((a + ".rope.dimension_count", gw.U32, hp["head_dim"]))
    return kv


def kv_gemma4(hp, w):
    """test/test_gemma4.lua:91-112 for the dense model."""
    a = "gemma4"
    L0 = w["layers"]
    swa = [bool(L["swa"]) for L in L0]
    D = [L for L in L0 if not L["swa"]][0]["head_dim"]
    DS = [L for L in L0 if L["swa"]][0]["head_dim"]
    return [("general.architecture", gw.STRING, a), ("general.name", gw.STRING, "tiny gemma4"),
            (a + ".block_count", gw.U32, hp["n_layer"]), (a + ".context_length", gw.U32, 256),
            (a + ".embedding_length", gw.U32, hp["n_embd"]),
            (a + ".feed_forward_length", gw.U32, hp["n_ff"]),
            (a + ".attention.head_count", gw.U32, hp["n_head"]),
            (a + ".attention.head_count_kv", (gw.ARRAY, gw.I32), [L["n_head_kv"] for L in L0]),
            (a + ".attention.key_length", gw.U32, D), (a + ".attention.value_length", gw.U32, D),
            (a + ".attention.key_length_swa", gw.U32, DS),
            (a + ".attention.value_length_swa", gw.U32, DS),
            (a + ".attention.layer_norm_rms_epsilon", gw.F32V, 1e-6),
            (a + ".attention.sliding_window", gw.U32, hp["n_swa"]),
            (a + ".attention.sliding_window_pattern", (gw.ARRAY, gw.BOOL), swa),
            (a + ".attention.shared_kv_layers", gw.U32, 0),
            (a + ".rope.dimension_count", gw.U32, D), (a + ".rope.dimension_count_swa", gw.U32, DS),
            (a + ".rope.freq_base", gw.F32V, 1e6), (a + ".rope.freq_base_swa", gw.F32V, 1e4),
            (a + ".final_logit_softcapping", gw.F32V, 30.0),
            (a + ".embedding_length_per_layer_input", gw.U32, 0)]


def check_rows(d, ref, rows):
    idx = [i - 1 for i in d["idx_1based"]]
    err = max(max(abs(float(g[i]) - v) for i, v in zip(idx, r["v"])) for r, g in zip(ref, rows))
    assert err < d["tol"], err
    assert all(core.argmax(g) == r["best"] for r, g in zip(ref, rows))


@pytest.mark.parametrize("arch", ["llama", "qwen3", "qwen3moe"])
def test_loaded_tiny_models_reproduce_the_golden_rows(oracle_lib, tmp_path, arch):
    hp, w = models.ref_tiny(arch)
    path = str(tmp_path / ("%s.gguf" % arch))
    gw.write(path, kv_qwen(arch, hp), tensors_of(arch, hp, w))
    hp2, w2 = gguf.load(path)
    assert hp2["n_vocab"] == hp["n_vocab"] and hp2["rope_neox"] == hp["rope_neox"]
    check_rows(*tg.run_rows(arch, model=(hp2, w2)))


def test_loaded_tiny_gemma4_reproduces_the_golden_rows(oracle_lib, tmp_path):
    hp, w = models.ref_tiny_gemma4()
    path = str(tmp_path / "gemma4.gguf")
    gw.write(path, kv_gemma4(hp, w), tensors_of("gemma4", hp, w, gemma=True))
    hp2, w2 = gguf.load(path)
    assert w2["output"] is w2["tok_embd"] and "wv" not in w2["layers"][1]
    assert [L["n_head_kv"] for L in w2["layers"]] == [2, 1]
    assert w2["layers"][0].get("rope_freqs") is None and w2["rope_freqs"] is None
    check_rows(*tg.run_gemma4_rows(model=(hp2, w2)))


def test_quantized_tensors_load_byte_exact(tmp_path):
    rng = np.random.default_rng(0)
    ts = []
    want = {}
    for name, ty, shape in (("a.weight", core.Q4_K, (48, 512)), ("b.weight", core.Q8_0, (16, 256)),
                            ("c.weight", core.Q6_K, (4, 7, 256))):
        rows = int(np.prod(shape[:-1]))
        q = core.quantize(ty, rng.standard_normal((rows, shape[-1])).astype(np.float32))
        ts.append((name, list(shape), q, ty))
        want[name] = q
    path = str(tmp_path / "q.gguf")
    gw.write(path, [("general.architecture", gw.STRING, "llama")], ts)
    g = gguf.GGUF(path)
    for name, q in want.items():
        got = g.tensor(name)
        assert got.shape == q.shape and np.array_equal(got, q), name
    assert g.tensors["c.weight"][0] == (256, 7, 4)


def test_bad_files_are_refused(tmp_path):
    p = tmp_path / "x.gguf"
    p.write_bytes(b"GGML" + bytes(60))
    with pytest.raises(gguf.GGUFError):
        gguf.GGUF(str(p))
    gw.write(str(p), [("general.architecture", gw.STRING, "mamba")], [])
    with pytest.raises(gguf.GGUFError, match="unknown architecture"):
        gguf.load(str(p))
