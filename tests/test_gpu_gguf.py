"""A model loaded from a gguf file (quantized Q4_K_M tensors, the ggml
bytes unchanged) gives the same logits on the device, bit for bit, as the
same weights handed to DeviceModel directly."""
import numpy as np
import pytest

from oracle import core, models
from tests import gguf_util as gw
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHAPE = dict(arch="llama", n_layer=2, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, n_ff=1024,
             n_vocab=2048, rope_base=5e5, eps=1e-5, wtype="q4_K_M")


def c2_like_gguf(path):
    hp, w = models.build(dict(SHAPE), seed=9, init="normal")
    E, H, Hkv, D, F, V = (hp[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff",
                                          "n_vocab"))
    ts = [("token_embd.weight", [V, E]) + w["tok_embd"],
          ("output_norm.weight", [E]) + w["output_norm"],
          ("output.weight", [V, E]) + w["output"]]
    shapes = {"attn_q": ("wq", [H * D, E]), "attn_k": ("wk", [Hkv * D, E]),
              "attn_v": ("wv", [Hkv * D, E]), "attn_output": ("wo", [E, H * D]),
              "ffn_gate": ("gate", [F, E]), "ffn_up": ("up", [F, E]), "ffn_down": ("down", [E, F]),
              "attn_norm": ("attn_norm", [E]), "ffn_norm": ("ffn_norm", [E])}
    for i, L in enumerate(w["layers"]):
        for n, (k, sh) in shapes.items():
            ts.append(("blk.%d.%s.weight" % (i, n), sh) + L[k])
    a = "llama"
    kv = [("general.architecture", gw.STRING, a), (a + ".block_count", gw.U32, hp["n_layer"]),
          (a + ".context_length", gw.U32, 8192), (a + ".embedding_length", gw.U32, E),
          (a + ".feed_forward_length", gw.U32, F), (a + ".attention.head_count", gw.U32, H),
          (a + ".attention.head_count_kv", gw.U32, Hkv),
          (a + ".attention.layer_norm_rms_epsilon", gw.F32V, hp["eps"]),
          (a + ".rope.freq_base", gw.F32V, hp["rope_base"])]
    gw.write(path, kv, ts)
    return hp, w


def test_gguf_model_equals_the_direct_model(tmp_path):
    from lgml_amd import runtime
    path = str(tmp_path / "m.gguf")
    hp, w = c2_like_gguf(path)
    assert {w["layers"][1]["wv"][1], w["output"][1]} == {core.Q6_K}  # the _M mix
    a = runtime.DeviceModel(hp, w, 1024)
    b = runtime.load_gguf(path, 1024)
    assert b.hp["n_vocab"] == hp["n_vocab"] and b.hp["rope_neox"] == 0
    ids = np.array(lcg_ints(11, 37, 0, hp["n_vocab"]), np.int32)
    bt = np.array([[0, 1]], np.int32)
    la = a.forward(a.plan([37], [0], bt, ids)).cpu().numpy()
    lb = b.forward(b.plan([37], [0], bt, ids)).cpu().numpy()
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
