"""GGUF weights for the HIP path: the metadata, tensor table and tensor
bytes of a gguf file (the role of lgml.gguf / gload.c, src/lgml.c:872-984),
the model config of transformer.lua's M.config (:122-250) and the weight
set of M.load / M.load_layer (:272-435), for the llama, qwen3, qwen3moe and
gemma4 architectures, in the weights-dict form DeviceModel and the tests
take.

The file is memory-mapped; tensors are numpy views of it. Quantized
tensors (Q4_K, Q6_K, Q8_0) stay in their ggml bytes as uint8 (rows,
row_bytes), for lgmlh_repack; f32 tensors are (rows, cols) float32; f16
matrices are widened to f32 (the products take f32 or quantized weights).
Shapes follow ggml: ne[0] is the row length, the other dimensions count
rows (an expert tensor (ne0, ne1, n_expert) is n_expert * ne1 rows,
expert-major).
"""
import math
import mmap
import struct

import numpy as np

from . import hip

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types (the gguf format)
U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f",
           BOOL: "<B", U64: "<Q", I64: "<q", F64: "<d"}

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
SUPPORTED = {F32, F16, Q8_0, Q4_K, Q6_K}

# gating values of <arch>.expert_gating_func (transformer.lua:32-35)
GATING_SOFTMAX, GATING_SIGMOID = 1, 2


class GGUFError(ValueError):
    pass


class _Reader:
    def __init__(self, buf):
        self.buf, self.off = buf, 0

    def take(self, fmt):
        v = struct.unpack_from(fmt, self.buf, self.off)[0]
        self.off += struct.calcsize(fmt)
        return v

    def string(self):
        n = self.take("<Q")
        s = bytes(self.buf[self.off:self.off + n]).decode("utf-8")
        self.off += n
        return s

    def value(self, t):
        if t == STRING:
            return self.string()
        if t == ARRAY:
            et, n = self.take("<I"), self.take("<Q")
            return [self.value(et) for _ in range(n)]
        if t not in _SCALAR:
            raise GGUFError("gguf: unknown value type %d" % t)
        v = self.take(_SCALAR[t])
        return bool(v) if t == BOOL else v


class GGUF:
    """A gguf file: .meta (key -> value), .tensors (name -> (ne, type,
    offset)), .tensor(name) (a numpy view)."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            self.mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        r = _Reader(self.mm)
        if bytes(self.mm[:4]) != GGUF_MAGIC:
            raise GGUFError("%s: not a gguf file" % path)
        r.off = 4
        self.version = r.take("<I")
        if self.version not in (2, 3):
            raise GGUFError("%s: gguf version %d not supported" % (path, self.version))
        n_tensors, n_kv = r.take("<Q"), r.take("<Q")
        self.meta = {}
        for _ in range(n_kv):
            k = r.string()
            self.meta[k] = r.value(r.take("<I"))
        self.tensors = {}
        self.order = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.take("<I")
            ne = tuple(r.take("<Q") for _ in range(nd))
            ty, off = r.take("<I"), r.take("<Q")
            self.tensors[name] = (ne, ty, off)
            self.order.append(name)
        align = int(self.meta.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data = (r.off + align - 1) // align * align

    def has(self, name):
        return name in self.tensors

    def tensor(self, name):
        """The tensor as a numpy view: f32 (rows, ne0) or (ne0,) for 1-D,
        f16 likewise, quantized uint8 (rows, row_bytes)."""
        if name not in self.tensors:
            raise GGUFError("%s: no tensor %s" % (self.path, name))
        ne, ty, off = self.tensors[name]
        if ty not in SUPPORTED:
            raise GGUFError("%s: tensor %s has type %d (f32, f16, Q8_0, Q4_K, Q6_K are "
                            "supported)" % (self.path, name, ty))
        rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
        rb = hip.lib().lgmlh_row_size(ty, ne[0]) if ty not in (F32, F16) else ne[0] * (
            4 if ty == F32 else 2)
        if rb <= 0:
            raise GGUFError("%s: row of %d values does not fit type %d" % (name, ne[0], ty))
        start = self.data + off
        raw = np.frombuffer(self.mm, np.uint8, count=rows * rb, offset=start)
        if ty == F32:
            a = raw.view(np.float32)
        elif ty == F16:
            a = raw.view(np.float16)
        else:
            return raw.reshape(rows, rb)
        return a.reshape(rows, ne[0]) if len(ne) > 1 else a

    def close(self):
        self.mm.close()


# Settings the metadata does not hold, per architecture (transformer.lua:61-78)
FAMILY = {
    "llama": dict(rope_neox=0, qk_norm=False),
    "qwen3": dict(rope_neox=1, qk_norm=True),
    "qwen3moe": dict(rope_neox=1, qk_norm=True),
    "gemma4": dict(rope_neox=1, qk_norm=True, gemma=True),
}


def config(meta):
    """M.config (transformer.lua:122-250) for llama / qwen3 / qwen3moe /
    gemma4: the hp dict, with per-layer fields in hp["layers"]."""
    a = meta.get("general.architecture")
    fam = FAMILY.get(a)
    if fam is None:
        raise GGUFError("transformer: unknown architecture %s" % a)

    def k(s, default=None):
        v = meta.get(a + "." + s)
        return default if v is None else v

    n_layer = k("block_count") - k("nextn_predict_layers", 0)
    n_embd, n_head = k("embedding_length"), k("attention.head_count")
    head_dim = k("attention.key_length") or n_embd // n_head
    hkv = k("attention.head_count_kv", n_head)
    hp = dict(arch=a, n_layer=n_layer, n_embd=n_embd, n_head=n_head,
              n_head_kv=hkv[0] if isinstance(hkv, list) else hkv, head_dim=head_dim,
              n_rot=k("rope.dimension_count", head_dim),
              eps=float(k("attention.layer_norm_rms_epsilon")),
              rope_base=float(k("rope.freq_base", 10000.0)), n_ctx=k("context_length"),
              n_vocab=k("vocab_size"), rope_neox=fam["rope_neox"], qk_norm=fam["qk_norm"],
              gemma=fam.get("gemma", False), attn_scale=0.0, n_ff=k("feed_forward_length"))
    n_expert = k("expert_count")
    if n_expert:
        hp.update(n_expert=n_expert, n_used=k("expert_used_count"),
                  n_ff_exp=k("expert_feed_forward_length"),
                  gating=k("expert_gating_func", GATING_SOFTMAX),
                  norm_topk=bool(k("expert_weights_norm", True)),
                  expert_scale=float(k("expert_weights_scale", 1.0)))
        if hp["gating"] not in (GATING_SOFTMAX, GATING_SIGMOID):
            raise GGUFError("%s: expert gating %s not supported" % (a, hp["gating"]))
    swa = k("attention.sliding_window_pattern")
    if hp["gemma"]:
        if not isinstance(swa, list) or len(swa) != n_layer:
            raise GGUFError("%s: need a sliding_window_pattern entry per layer" % a)
        if k("attention.shared_kv_layers", 0) or k("embedding_length_per_layer_input", 0):
            raise GGUFError("%s: shared KV layers and per-layer inputs are not supported" % a)
        hp.update(head_dim_swa=k("attention.key_length_swa"),
                  rope_base_swa=float(k("rope.freq_base_swa", 10000.0)),
                  n_swa=k("attention.sliding_window"),
                  softcap=float(k("final_logit_softcapping", 0.0)),
                  embd_scale=float(np.float32(math.sqrt(n_embd))), attn_scale=1.0)
        hp["n_rot_swa"] = k("rope.dimension_count_swa", hp["head_dim_swa"])
    layers = []
    for i in range(n_layer):
        s = bool(swa[i]) if hp["gemma"] else False
        layers.append(dict(swa=int(s), head_dim=hp["head_dim_swa"] if s else head_dim,
                           n_head_kv=hkv[i] if isinstance(hkv, list) else hkv,
                           n_rot=hp["n_rot_swa"] if s else hp["n_rot"],
                           rope_base=hp["rope_base_swa"] if s else hp["rope_base"],
                           freqs=not s))
    hp["layers"] = layers
    return hp


def _mat(g, name):
    """A weight matrix as (array, ggml type) for the weights dict."""
    a = g.tensor(name)
    ty = g.tensors[name][1]
    if ty == F16:
        return (a.astype(np.float32), F32)
    return (a, ty)


def _vec(g, name):
    return (np.asarray(g.tensor(name), np.float32).reshape(-1), F32)


def load(path):
    """M.load (transformer.lua:388-435) + M.load_layer (:272-380): (hp,
    weights dict). The output weight falls back to the token embedding."""
    g = GGUF(path)
    hp = config(g.meta)

    def get(name):
        if not g.has(name):
            raise GGUFError("%s: %s" % (path, name))
        return name

    w = {"tok_embd": _mat(g, get("token_embd.weight")),
         "output_norm": _vec(g, get("output_norm.weight"))}
    w["output"] = _mat(g, "output.weight") if g.has("output.weight") else w["tok_embd"]
    rope_freqs = (np.asarray(g.tensor("rope_freqs.weight"), np.float32).reshape(-1)
                  if g.has("rope_freqs.weight") else None)
    if hp["n_vocab"] is None:  # the rows of the output (or embedding) matrix
        out_name = "output.weight" if g.has("output.weight") else "token_embd.weight"
        hp["n_vocab"] = int(g.tensors[out_name][0][1])
    w["rope_freqs"] = None if hp["gemma"] else rope_freqs
    layers = []
    for i, d in enumerate(hp["layers"]):
        p = "blk.%d." % i
        L = {"attn_norm": _vec(g, get(p + "attn_norm.weight")),
             "wq": _mat(g, get(p + "attn_q.weight")), "wk": _mat(g, get(p + "attn_k.weight")),
             "wo": _mat(g, get(p + "attn_output.weight"))}
        if g.has(p + "attn_v.weight"):
            L["wv"] = _mat(g, p + "attn_v.weight")
        elif not hp["gemma"]:
            get(p + "attn_v.weight")  # required outside gemma (V = K on gemma global layers)
        if hp["qk_norm"]:
            L["q_norm"] = _vec(g, get(p + "attn_q_norm.weight"))
            L["k_norm"] = _vec(g, get(p + "attn_k_norm.weight"))
        L["ffn_norm"] = _vec(g, get(p + "ffn_norm.weight"))
        if hp["gemma"]:
            L["post_attn_norm"] = _vec(g, get(p + "post_attention_norm.weight"))
            L["post_ffn_norm"] = _vec(g, get(p + "post_ffw_norm.weight"))
            if g.has(p + "layer_output_scale.weight"):
                L["out_scale"] = float(np.asarray(g.tensor(p + "layer_output_scale.weight"),
                                                  np.float32).reshape(-1)[0])
            L.update(swa=d["swa"], head_dim=d["head_dim"], n_head_kv=d["n_head_kv"],
                     n_rot=d["n_rot"], rope_base=d["rope_base"])
            if d["freqs"] and rope_freqs is not None:
                L["rope_freqs"] = rope_freqs
        if hp.get("n_expert") and not hp["gemma"]:
            L["gate_inp"] = _mat(g, get(p + "ffn_gate_inp.weight"))
            for nm, t in (("gate_exps", "ffn_gate_exps"), ("up_exps", "ffn_up_exps"),
                          ("down_exps", "ffn_down_exps")):
                L[nm] = _mat(g, get(p + t + ".weight"))
        else:
            L["gate"] = _mat(g, get(p + "ffn_gate.weight"))
            L["up"] = _mat(g, get(p + "ffn_up.weight"))
            L["down"] = _mat(g, get(p + "ffn_down.weight"))
        layers.append(L)
    w["layers"] = layers
    if hp["n_ff"] is None:
        hp["n_ff"] = hp.get("n_ff_exp", 0)
    # the arrays are views of the mapped file and keep it open
    return hp, w
