"""ctypes bindings of oracle/liboracle.so (the C restatement).

TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and bench.py's
cpu_baseline leg as the checker, never by the shipped library.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
BLOCK_BYTES = {Q4_K: (256, 144), Q6_K: (256, 210), Q8_0: (32, 34), F32: (1, 4), F16: (1, 2)}

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class Tensor(C.Structure):
    _fields_ = [("type", C.c_int), ("data", C.c_void_p)]


TENSOR_FIELDS = ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm", "gate",
                 "up", "down", "gate_inp", "gate_exps", "up_exps", "down_exps", "post_attn_norm",
                 "post_ffn_norm")


class Layer(C.Structure):
    _fields_ = [(n, Tensor) for n in TENSOR_FIELDS[:15]] + \
               [("post_attn_norm", Tensor), ("post_ffn_norm", Tensor), ("out_scale", C.c_float),
                ("swa", C.c_int), ("head_dim", C.c_int), ("n_head_kv", C.c_int),
                ("n_rot", C.c_int), ("rope_base", C.c_float), ("rope_freqs", C.c_void_p)]


class Model(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_embd", C.c_int), ("n_head", C.c_int),
                ("n_head_kv", C.c_int), ("head_dim", C.c_int), ("n_ff", C.c_int),
                ("n_vocab", C.c_int), ("n_rot", C.c_int), ("eps", C.c_float),
                ("rope_base", C.c_float), ("attn_scale", C.c_float), ("rope_neox", C.c_int),
                ("rope_freqs", C.c_void_p), ("tok_embd", Tensor), ("output", Tensor),
                ("output_norm", Tensor), ("layers", C.POINTER(Layer)),
                ("n_expert", C.c_int), ("n_used", C.c_int), ("n_ff_exp", C.c_int),
                ("gating", C.c_int), ("norm_topk", C.c_int), ("expert_scale", C.c_float),
                ("gemma", C.c_int), ("n_swa", C.c_int), ("embd_scale", C.c_float),
                ("softcap", C.c_float), ("act_quant", C.c_int)]


class Batch(C.Structure):
    _fields_ = [("n_seq", C.c_int), ("max_blocks", C.c_int), ("block", C.c_int),
                ("seq_n", C.c_void_p), ("seq_npast", C.c_void_p), ("block_tab", C.c_void_p),
                ("ids", C.c_void_p), ("n_out", C.c_int), ("out_rows", C.c_void_p),
                ("ring_blocks", C.c_int), ("ring_tab", C.c_void_p)]


def _declare(L):
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
    L.orc_lcg_next.argtypes = [C.POINTER(C.c_uint64)]
    L.orc_lcg_next.restype = C.c_double
    L.orc_lcg_fill.argtypes = [C.POINTER(C.c_uint64), vp, i64, C.c_double, C.c_double]
    L.orc_fill_normal.argtypes = [C.POINTER(C.c_uint64), vp, i64, C.c_double, C.c_double]
    L.orc_fill_uniform.argtypes = [C.POINTER(C.c_uint64), vp, i64, C.c_double, C.c_double]
    L.orc_gen_normal.argtypes = [C.c_uint64, vp, i64, C.c_double, C.c_double, i32]
    L.orc_gen_normal_quant.argtypes = [C.c_uint64, i32, i64, i64, C.c_double, C.c_double, vp, i32]
    L.orc_gen_normal_quant.restype = i64
    L.orc_f32_to_f16_row.argtypes = [vp, vp, i64]
    L.orc_f16_to_f32_row.argtypes = [vp, vp, i64]
    L.orc_row_size.argtypes = [i32, i64]
    L.orc_row_size.restype = i64
    L.orc_dequantize_row.argtypes = [i32, vp, vp, i64]
    L.orc_quantize_row.argtypes = [i32, vp, vp, i64]
    L.orc_quantize_row.restype = i64
    L.orc_forward.argtypes = [C.POINTER(Model), vp, vp, i64, C.POINTER(Batch), vp, i32]
    L.orc_paged_attention.argtypes = [vp, vp, vp, i32, i32, i32, C.c_float, C.POINTER(Batch),
                                      vp, i32]
    L.orc_paged_attention_swa.argtypes = [vp, vp, vp, i32, i32, i32, C.c_float, i32,
                                          C.POINTER(Batch), vp, i32]
    L.orc_flash_attn.argtypes = [vp, i32, i32, i32, vp, vp, i32, i32, i64, i64, i64, i64, vp,
                                 i32, i32, C.c_float, C.c_float, C.c_float, vp, i32]
    L.orc_set_rows_f16.argtypes = [vp, i64, i64, vp, vp, i64]
    L.orc_mul_mat.argtypes = [i32, vp, i64, i64, vp, i64, vp, i32]
    L.orc_mul_mat_q8.argtypes = [i32, vp, i64, i64, vp, i64, vp, i32]
    L.orc_mul_mat_id_q8.argtypes = [i32, vp, i64, i64, i64, vp, i64, vp, i64, i32, vp, i32]
    L.orc_quantize_q8_K.argtypes = [vp, i64, vp, vp, vp]
    L.orc_quantize_q8_0_act.argtypes = [vp, i64, vp, vp]
    L.orc_moe_route.argtypes = [vp, i64, i32, i32, i32, i32, C.c_float, vp, vp]
    L.orc_mul_mat_id.argtypes = [i32, vp, i64, i64, i64, vp, i64, vp, i64, i32, vp, i32]
    L.orc_splitmix64.argtypes = [C.POINTER(C.c_uint64)]
    L.orc_splitmix64.restype = C.c_uint64
    L.orc_rms_norm.argtypes = [vp, vp, i64, i64, C.c_float, vp]
    L.orc_rope.argtypes = [vp, i64, i32, i32, i32, i32, C.c_float, vp, vp]
    L.orc_glu.argtypes = [vp, vp, vp, i64, i32]
    L.orc_argmax.argtypes = [vp, i64]
    L.orc_argmax.restype = C.c_int32


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class Lcg:
    """test/tiny.lua:16-22 seeded uniform numbers in [0, 1)."""

    def __init__(self, seed):
        self.state = C.c_uint64(seed & (2**64 - 1))

    def next(self):
        return lib().orc_lcg_next(C.byref(self.state))

    def fill(self, n, lo, hi):
        out = np.empty(n, np.float32)
        lib().orc_lcg_fill(C.byref(self.state), _p(out), n, lo, hi)
        return out


def fill_normal(n, mean, sd, seed):
    """src/lgml.c:3130-3136 tensor:fill("normal", mean, sd, seed)."""
    s = C.c_uint64(seed & (2**64 - 1))
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(C.byref(s), _p(out), n, mean, sd)
    return out


def threads():
    """OpenMP threads for the oracle: OMP_NUM_THREADS, else up to 16 cores."""
    return int(os.environ.get("OMP_NUM_THREADS") or min(16, os.cpu_count() or 1))


def gen_normal(n, mean, sd, seed):
    """fill_normal's values (same seed), generated in parallel."""
    out = np.empty(n, np.float32)
    lib().orc_gen_normal(seed & (2**64 - 1), _p(out), n, mean, sd, threads())
    return out


def gen_normal_quant(t, rows, cols, mean, sd, seed):
    """gen_normal(rows * cols) quantized row by row; uint8 (rows, row_size)."""
    out = np.empty((rows, row_size(t, cols)), np.uint8)
    if lib().orc_gen_normal_quant(seed & (2**64 - 1), t, rows, cols, mean, sd, _p(out),
                                  threads()) < 0:
        raise ValueError("gen_normal_quant failed")
    return out


def fill_uniform(n, a, b, seed):
    s = C.c_uint64(seed & (2**64 - 1))
    out = np.empty(n, np.float32)
    lib().orc_fill_uniform(C.byref(s), _p(out), n, a, b)
    return out


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_row(_p(x), _p(y), x.size)
    return y


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().orc_f16_to_f32_row(_p(h), _p(y), h.size)
    return y


def row_size(t, n):
    return lib().orc_row_size(t, n)


def quantize(t, x):
    """Quantize a (rows, K) f32 matrix row by row; returns uint8 (rows, row_size)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    rs = row_size(t, K)
    out = np.zeros((rows, rs), np.uint8)
    for r in range(rows):
        if lib().orc_quantize_row(t, _p(x[r]), _p(out[r]), K) != rs:
            raise ValueError("quantize failed")
    return out


def dequantize(t, q, K):
    q = np.ascontiguousarray(q, np.uint8).reshape(-1, row_size(t, K))
    out = np.empty((q.shape[0], K), np.float32)
    for r in range(q.shape[0]):
        if lib().orc_dequantize_row(t, _p(q[r]), _p(out[r]), K) != 0:
            raise ValueError("dequantize failed")
    return out


def mul_mat(t, w, M, K, x, nthreads=None):
    x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]
    y = np.empty((N, M), np.float32)
    w = np.ascontiguousarray(w)
    if lib().orc_mul_mat(t, _p(w), M, K, _p(x), N, _p(y), nthreads or threads()) != 0:
        raise ValueError("mul_mat failed")
    return y


def mul_mat_q8(t, w, M, K, x, nthreads=None):
    """ggml's CPU mul_mat for a quantized weight: X quantized per block to the
    weight type's vec_dot_type (Q8_K / Q8_0), integer block dots."""
    x = np.ascontiguousarray(x, np.float32)
    N = x.shape[0]
    y = np.empty((N, M), np.float32)
    w = np.ascontiguousarray(w)
    if lib().orc_mul_mat_q8(t, _p(w), M, K, _p(x), N, _p(y), nthreads or threads()) != 0:
        raise ValueError("mul_mat_q8 failed")
    return y


def quantize_q8_K(x):
    """quantize_row_q8_K_ref of each row of x (rows, K): q int8 (rows, K),
    d f32 (rows, K/256), bsums int16 (rows, K/16)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    d = np.empty((rows, K // 256), np.float32)
    bs = np.empty((rows, K // 16), np.int16)
    for r in range(rows):
        lib().orc_quantize_q8_K(_p(x[r]), K, _p(q[r]), _p(d[r]), _p(bs[r]))
    return q, d, bs


def quantize_q8_0_act(x):
    """quantize_row_q8_0_ref of each row of x (rows, K): q int8 (rows, K), d
    f16 bits (rows, K/32)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    d = np.empty((rows, K // 32), np.uint16)
    for r in range(rows):
        lib().orc_quantize_q8_0_act(_p(x[r]), K, _p(q[r]), _p(d[r]))
    return q, d


GATING_SOFTMAX, GATING_SIGMOID = 1, 2


def moe_route(logits, n_used, gating=GATING_SOFTMAX, norm_topk=True, scale=1.0):
    """Router picks (ids i32 (n, n_used)) and weights (f32) of logits (n, n_expert)."""
    lg = np.ascontiguousarray(logits, np.float32)
    n, ne = lg.shape
    ids = np.empty((n, n_used), np.int32)
    w = np.empty((n, n_used), np.float32)
    if lib().orc_moe_route(_p(lg), n, ne, n_used, gating, int(bool(norm_topk)), scale, _p(ids),
                           _p(w)) != 0:
        raise ValueError("moe_route failed")
    return ids, w


def mul_mat_id(t, w, n_expert, M, K, x, ids, nthreads=None, act_quant=False):
    """y (T, n_used, M): row (t, j) = w[ids[t, j]] x[t, j % U], x (T, U, K);
    act_quant: ggml's CPU arithmetic (mul_mat_q8) per expert."""
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.int32)
    T, n_used = ids.shape
    U = x.shape[1] if x.ndim == 3 else 1
    y = np.empty((T, n_used, M), np.float32)
    w = np.ascontiguousarray(w)
    fn = lib().orc_mul_mat_id_q8 if act_quant else lib().orc_mul_mat_id
    if fn(t, _p(w), n_expert, M, K, _p(x), U, _p(ids), T, n_used, _p(y),
          nthreads or threads()) != 0:
        raise ValueError("mul_mat_id failed")
    return y


def splitmix64(seed, n):
    """n raw splitmix64 draws from seed (src/lgml.c:3064-3079)."""
    s = C.c_uint64(seed & (2**64 - 1))
    return [int(lib().orc_splitmix64(C.byref(s))) for _ in range(n)]


def rms_norm(x, eps, w=None):
    """graph:rms_norm (src/lgml.c:1633) of each row of x (rows, n), times w."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    wv = None if w is None else np.ascontiguousarray(w, np.float32)
    lib().orc_rms_norm(_p(x), _p(y), x.shape[0], x.shape[1], eps,
                       None if wv is None else _p(wv))
    return y


def rope(x, n_heads, D, n_rot, neox, base, pos, ff=None):
    """graph:rope (src/lgml.c:2004-2081) of rows (rows, n_heads * D) at pos."""
    y = np.ascontiguousarray(x, np.float32).copy()
    pos = np.ascontiguousarray(pos, np.int32)
    ffv = None if ff is None else np.ascontiguousarray(ff, np.float32)
    lib().orc_rope(_p(y), y.shape[0], n_heads, D, n_rot, int(neox), base,
                   None if ffv is None else _p(ffv), _p(pos))
    return y


def glu(g, u, gelu=False):
    """silu(g) u, or gelu(g) u (transformer.lua:2048), elementwise."""
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().orc_glu(_p(g), _p(u), _p(out), g.size, int(bool(gelu)))
    return out


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return int(lib().orc_argmax(_p(v), v.size))


class BatchDesc:
    """Keeps the arrays of an orc_batch alive."""

    def __init__(self, seq_n, seq_npast, block_tab, block, ids, out_rows, ring_tab=None):
        """ring_tab: (n_seq, ring_blocks) block ids of each sequence's ring
        (the cells of sliding-window layers), or None."""
        self.seq_n = np.ascontiguousarray(seq_n, np.int32)
        self.seq_npast = np.ascontiguousarray(seq_npast, np.int32)
        bt = np.ascontiguousarray(block_tab, np.int32)
        if bt.ndim == 1:
            bt = bt.reshape(len(self.seq_n), -1)
        self.block_tab = bt
        self.ids = np.ascontiguousarray(ids, np.int32)
        self.out_rows = np.ascontiguousarray(out_rows, np.int32)
        self.c = Batch(len(self.seq_n), bt.shape[1], block, _p(self.seq_n), _p(self.seq_npast),
                       _p(self.block_tab), _p(self.ids), len(self.out_rows), _p(self.out_rows))
        if ring_tab is not None:
            rt = np.ascontiguousarray(ring_tab, np.int32)
            if rt.ndim == 1:
                rt = rt.reshape(len(self.seq_n), -1)
            self.ring_tab = rt
            self.c.ring_blocks = rt.shape[1]
            self.c.ring_tab = _p(rt)


def paged_attention(q, kpool, vpool, H, Hkv, D, scale, batch, nthreads=None):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty_like(q)
    rc = lib().orc_paged_attention(_p(q), _p(kpool), _p(vpool), H, Hkv, D, scale,
                                   C.byref(batch.c), _p(out), nthreads or threads())
    if rc:
        raise ValueError("paged_attention failed")
    return out


def paged_attention_swa(q, kpool, vpool, H, Hkv, D, scale, window, batch, nthreads=None):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty_like(q)
    rc = lib().orc_paged_attention_swa(_p(q), _p(kpool), _p(vpool), H, Hkv, D, scale, window,
                                       C.byref(batch.c), _p(out), nthreads or threads())
    if rc:
        raise ValueError("paged_attention_swa failed")
    return out


def flash_attn(q, k, v, n_head_kv, mask=None, scale=1.0, max_bias=0.0, softcap=0.0,
               k_strides=None, v_strides=None, n_kv=None, nthreads=None):
    """graph:flash_attn (src/lgml.c:2121-2170) on f16 K / V. q (H, T, D) f32.
    k, v: uint16 arrays (f16 bits) holding element (hk, j, d) at [hk *
    head_stride + j * row_stride + d] of the flattened array; strides
    (row_stride, head_stride) default to a contiguous (Hkv, n_kv, D) layout
    (n_kv = k.shape[-2]). mask: (mask_heads, rows, n_kv) or (rows, n_kv)
    f16 bits, or None. Returns (T, H, D) f32."""
    q = np.ascontiguousarray(q, np.float32)
    H, T, D = q.shape
    kf = np.ascontiguousarray(k).reshape(-1)
    vf = np.ascontiguousarray(v).reshape(-1)
    if n_kv is None:
        n_kv = k.shape[-2]
    if k_strides is None:
        k_strides = (D, n_kv * D)
    if v_strides is None:
        v_strides = (D, n_kv * D)
    mh, mr, mp = 0, 0, None
    if mask is not None:
        m = np.ascontiguousarray(mask)
        if m.ndim == 2:
            m = m[None]
        mh, mr = m.shape[0], m.shape[1]
        assert m.shape[2] == n_kv, "the mask has a column per kv row"
        mp = m
    out = np.zeros((T, H, D), np.float32)
    rc = lib().orc_flash_attn(_p(q), H, T, D, _p(kf), _p(vf), n_head_kv, n_kv, k_strides[0],
                              k_strides[1], v_strides[0], v_strides[1],
                              _p(mp) if mp is not None else None, mh, mr, scale, max_bias,
                              softcap, _p(out), nthreads or threads())
    if rc:
        raise ValueError("flash_attn failed")
    return out


def set_rows_f16(dst, src, ids):
    src = np.ascontiguousarray(src, np.float32)
    ids = np.ascontiguousarray(ids, np.int64)
    if lib().orc_set_rows_f16(_p(dst), dst.shape[0], dst.shape[1], _p(src), _p(ids),
                              len(ids)) != 0:
        raise ValueError("set_rows: id out of range")


class OracleModel:
    """Wraps a weights dict (see oracle.models) as an orc_model."""

    def __init__(self, hp, w):
        self.hp, self.w = hp, w
        self._keep = []
        L = hp["n_layer"]
        self.layers = (Layer * L)()
        for il in range(L):
            lw = w["layers"][il]
            Ly = self.layers[il]
            for f in TENSOR_FIELDS:
                t = lw.get(f)
                if t is not None:
                    arr, ty = t
                    arr = np.ascontiguousarray(arr)
                    self._keep.append(arr)
                    setattr(Ly, f, Tensor(ty, _p(arr).value))
            # per-layer attention shape / rope / gemma scalars
            for f in ("out_scale", "swa", "head_dim", "n_head_kv", "n_rot", "rope_base"):
                if lw.get(f) is not None:
                    setattr(Ly, f, lw[f])
            if lw.get("rope_freqs") is not None:
                rf = np.ascontiguousarray(lw["rope_freqs"], np.float32)
                self._keep.append(rf)
                Ly.rope_freqs = _p(rf).value
        self.c = Model()
        for k in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                  "n_rot", "rope_neox"):
            setattr(self.c, k, int(hp[k]))
        self.c.eps, self.c.rope_base = hp["eps"], hp["rope_base"]
        self.c.attn_scale = hp.get("attn_scale", 0.0)
        rf = w.get("rope_freqs")
        if rf is not None:
            rf = np.ascontiguousarray(rf, np.float32)
            self._keep.append(rf)
            self.c.rope_freqs = _p(rf).value
        for f in ("tok_embd", "output", "output_norm"):
            arr, ty = w[f]
            arr = np.ascontiguousarray(arr)
            self._keep.append(arr)
            setattr(self.c, f, Tensor(ty, _p(arr).value))
        self.c.layers = self.layers
        for k in ("n_expert", "n_used", "n_ff_exp"):
            setattr(self.c, k, int(hp.get(k, 0)))
        self.c.gating = int(hp.get("gating", GATING_SOFTMAX))
        self.c.gemma = int(bool(hp.get("gemma", False)))
        self.c.n_swa = int(hp.get("n_swa", 0))
        self.c.embd_scale = float(hp.get("embd_scale", 0.0))
        self.c.softcap = float(hp.get("softcap", 0.0))
        self.c.norm_topk = int(bool(hp.get("norm_topk", True)))
        self.c.expert_scale = float(hp.get("expert_scale", 1.0))
        self.c.act_quant = int(bool(hp.get("act_quant", False)))

    def forward(self, kpools, vpools, batch, nthreads=None):
        """kpools/vpools: lists of (cap, Hkv*D) uint16 arrays (f16 bits), updated in place."""
        L = self.hp["n_layer"]
        kp = (C.c_void_p * L)(*[_p(a).value for a in kpools])
        vp = (C.c_void_p * L)(*[_p(a).value for a in vpools])
        cap = kpools[0].shape[0]
        out = np.empty((len(batch.out_rows), self.hp["n_vocab"]), np.float32)
        rc = lib().orc_forward(C.byref(self.c), kp, vp, cap, C.byref(batch.c), _p(out),
                               nthreads or threads())
        if rc:
            raise ValueError("orc_forward failed: %d" % rc)
        return out
