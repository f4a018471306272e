"""ctypes binding of liblgml_hip.so (the C ABI in include/lgml_hip.h).

Device memory and streams come from torch (ROCm): a device buffer is a
torch tensor and its data_ptr() is passed to the library; the stream is
torch's current HIP stream. The library must be built
(`python -m lgml_amd.build`); importing this module without it raises.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblgml_hip.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
OK, EINVAL, ENOMEM, EHIP, EFULL, ERANGE = 0, -1, -2, -3, -4, -5
EPI_NONE, EPI_ADD = 0, 1
ACT_EXACT, ACT_GGML = 0, 1

# Every symbol include/lgml_hip.h declares.
SYMBOLS = (
    "lgmlh_last_error", "lgmlh_abi_version", "lgmlh_row_size", "lgmlh_kv_layer_bytes",
    "lgmlh_kv_store", "lgmlh_kv_gather", "lgmlh_kv_copy_block", "lgmlh_set_rows_f16",
    "lgmlh_kv_block_bytes", "lgmlh_kv_block_host", "lgmlh_kv_grow", "lgmlh_kvpool_victim",
    "lgmlh_plan", "lgmlh_plan_bind", "lgmlh_attention_workspace", "lgmlh_paged_attention",
    "lgmlh_flash_attn",
    "lgmlh_repacked_bytes", "lgmlh_repack", "lgmlh_dequantize", "lgmlh_mul_mat_workspace",
    "lgmlh_mul_mat", "lgmlh_get_rows", "lgmlh_rms_norm", "lgmlh_qkv_rope_store",
    "lgmlh_swiglu", "lgmlh_argmax", "lgmlh_forward_workspace", "lgmlh_forward",
    "lgmlh_kvpool_bytes", "lgmlh_kvpool_init", "lgmlh_kvpool_take", "lgmlh_kvpool_evict",
    "lgmlh_kvpool_ref", "lgmlh_kvpool_unref", "lgmlh_kvpool_refs_of", "lgmlh_kvpool_publish",
    "lgmlh_kvpool_publish_part", "lgmlh_kvpool_key_of", "lgmlh_kvpool_lookup",
    "lgmlh_kvpool_longest_kid", "lgmlh_kvpool_set_cap", "lgmlh_kvpool_stats", "lgmlh_block_key",
    "lgmlh_gen_normal", "lgmlh_moe_route", "lgmlh_mul_mat_id_workspace", "lgmlh_mul_mat_id",
    "lgmlh_moe_sum", "lgmlh_plan_ring", "lgmlh_geglu", "lgmlh_softcap",
    "lgmlh_mul_mat_noalloc_limit", "lgmlh_mul_mat_noalloc", "lgmlh_mul_mat_ggml",
    "lgmlh_mul_mat_id_ggml", "lgmlh_quantize_act", "lgmlh_forward_release",
)
GATING_SOFTMAX, GATING_SIGMOID = 1, 2
TRACE_ATTN, TRACE_GEMM, TRACE_EXPERTS = 1, 2, 4


class LgmlhError(RuntimeError):
    def __init__(self, rc, msg):
        super().__init__("lgml_hip error %d: %s" % (rc, msg))
        self.rc = rc


class PlanInfo(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_seq", "n_tokens", "max_blocks", "block", "n_items",
                                         "n_merge", "rows", "n_head_kv")] + \
               [(n, C.c_int64) for n in ("bytes", "off_ids", "off_pos", "off_cells", "off_seq_off",
                                         "off_npast", "off_block_tab", "off_logit_rows",
                                         "off_items", "off_merge")] + \
               [("window", C.c_int32), ("ring", C.c_int32), ("n_single", C.c_int32),
                ("n_shared", C.c_int32), ("off_shared", C.c_int64), ("off_order", C.c_int64)]


class Ubatch(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("n_seq", "n_tokens", "max_blocks", "block", "n_items",
                                         "n_merge", "rows", "n_head_kv")] + \
               [(n, C.c_void_p) for n in ("ids", "pos", "cells", "seq_off", "seq_npast",
                                          "block_tab", "logit_rows", "items", "merge")] + \
               [("window", C.c_int32), ("ring", C.c_int32), ("n_single", C.c_int32),
                ("n_shared", C.c_int32), ("shared", C.c_void_p), ("order", C.c_void_p)]


class Layer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("wqkv_type", C.c_int), ("wv_type", C.c_int),
                ("wo_type", C.c_int), ("wgu_type", C.c_int), ("wdown_type", C.c_int),
                ("wqkv_rows", C.c_int64), ("wqkv", C.c_void_p), ("wv", C.c_void_p),
                ("wo", C.c_void_p), ("wgu", C.c_void_p), ("wdown", C.c_void_p),
                ("kpool", C.c_void_p), ("vpool", C.c_void_p), ("gate_inp", C.c_void_p),
                ("exp_gu_type", C.c_int), ("exp_down_type", C.c_int), ("exp_gu", C.c_void_p),
                ("exp_down", C.c_void_p), ("swa", C.c_int), ("v_from_k", C.c_int),
                ("post_attn_norm", C.c_void_p), ("post_ffn_norm", C.c_void_p),
                ("out_scale", C.c_float), ("rope_base", C.c_float), ("rope_freqs", C.c_void_p),
                ("head_dim", C.c_int), ("n_head_kv", C.c_int), ("n_rot", C.c_int)]


class Trace(C.Structure):
    _fields_ = [("events", C.POINTER(C.c_void_p)), ("capacity", C.c_int32), ("used", C.c_int32),
                ("kinds", C.c_int32), ("kind", C.POINTER(C.c_int32))]


class Model(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim",
                                       "n_ff", "n_vocab", "n_rot", "rope_neox")] + \
               [("eps", C.c_float), ("rope_base", C.c_float), ("attn_scale", C.c_float),
                ("rope_freqs", C.c_void_p), ("tok_embd_type", C.c_int), ("output_type", C.c_int),
                ("tok_embd", C.c_void_p), ("output", C.c_void_p), ("output_norm", C.c_void_p),
                ("n_cells", C.c_int64), ("layers", C.POINTER(Layer))] + \
               [(n, C.c_int) for n in ("n_expert", "n_used", "n_ff_exp", "gating", "norm_topk")] + \
               [("expert_scale", C.c_float), ("gemma", C.c_int), ("embd_scale", C.c_float),
                ("softcap", C.c_float), ("ring_cells", C.c_int64), ("act", C.c_int)]


_lib = None


def lib():
    """The loaded library; raises if it was not built (no CPU fallback)."""
    global _lib
    if _lib is None:
        # torch first: its HIP runtime (soname libamdhip64.so.7) is then the
        # one this library binds to, so one runtime serves the process.
        import torch  # noqa: F401
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("lgml_amd: %s is missing; run `python -m lgml_amd.build`" % LIB_PATH)
        L = C.CDLL(LIB_PATH)
        _declare(L)
        _lib = L
    return _lib


def _declare(L):
    vp, i64, i32, sz = C.c_void_p, C.c_int64, C.c_int, C.c_size_t
    sig = {
        "lgmlh_last_error": ([], C.c_char_p),
        "lgmlh_abi_version": ([], i32),
        "lgmlh_row_size": ([i32, i64], i64),
        "lgmlh_kv_layer_bytes": ([i64, i32, i32], i64),
        "lgmlh_kv_store": ([vp, vp, i64, i32, i32, vp, vp, vp, vp, i64, vp], i32),
        "lgmlh_kv_gather": ([vp, i32, i64, i32, i32, vp, i64, vp, vp], i32),
        "lgmlh_kv_copy_block": ([vp, vp, i64, i32, i32, C.c_int32, C.c_int32, i32, vp], i32),
        "lgmlh_kv_block_bytes": ([i32, i32], i64),
        "lgmlh_kv_block_host": ([vp, i32, i64, i32, i32, C.c_int32, vp, i32, vp], i32),
        "lgmlh_kv_grow": ([vp, i64, vp, i64, i32, i32, vp], i32),
        "lgmlh_set_rows_f16": ([vp, i64, i64, vp, vp, vp, i64, vp], i32),
        "lgmlh_plan": ([i32, vp, vp, vp, i32, i64, vp, i32, i32, i32, vp, sz,
                        C.POINTER(PlanInfo)], i32),
        "lgmlh_plan_bind": ([C.POINTER(PlanInfo), vp, C.POINTER(Ubatch)], i32),
        "lgmlh_plan_ring": ([i32, vp, vp, vp, i32, i64, i32, vp, i32, i32, i32, vp, sz,
                             C.POINTER(PlanInfo)], i32),
        "lgmlh_attention_workspace": ([C.POINTER(PlanInfo), i32], sz),
        "lgmlh_flash_attn": ([vp, i32, i32, i32, vp, vp, i32, i32, i64, i64, i64, i64, vp, i32,
                              i32, C.c_float, C.c_float, C.c_float, vp, vp], i32),
        "lgmlh_paged_attention": ([vp, i32, i32, i32, C.c_float, vp, vp, C.POINTER(Ubatch), vp,
                                   vp, sz, vp], i32),
        "lgmlh_repacked_bytes": ([i32, i64, i64], i64),
        "lgmlh_repack": ([i32, i64, i64, vp, vp, vp], i32),
        "lgmlh_dequantize": ([i32, vp, i64, i64, vp, vp], i32),
        "lgmlh_mul_mat_workspace": ([i32, i64, i64, i64], sz),
        "lgmlh_mul_mat": ([i32, vp, i64, i64, vp, i32, i64, vp, i32, vp, vp, sz, vp], i32),
        "lgmlh_mul_mat_ggml": ([i32, vp, i64, i64, vp, i32, i64, vp, i32, vp, vp, sz, vp], i32),
        "lgmlh_quantize_act": ([i32, vp, i64, i64, vp, vp, vp, vp], i32),
        "lgmlh_mul_mat_noalloc_limit": ([], sz),
        "lgmlh_mul_mat_noalloc": ([i32, vp, i64, i64, vp, i32, i64, vp, i32, vp, vp], i32),
        "lgmlh_get_rows": ([i32, vp, i64, i64, vp, vp, i64, vp, vp], i32),
        "lgmlh_rms_norm": ([vp, i64, i64, C.c_float, vp, vp, i32, vp], i32),
        "lgmlh_qkv_rope_store": ([vp, i64, i32, i32, i32, i32, i32, C.c_float, vp, vp, vp,
                                  C.c_float, vp, vp, vp, i64, vp, vp, vp], i32),
        "lgmlh_swiglu": ([vp, i64, i64, vp, i32, vp], i32),
        "lgmlh_geglu": ([vp, i64, i64, vp, i32, vp], i32),
        "lgmlh_softcap": ([vp, i64, C.c_float, vp], i32),
        "lgmlh_argmax": ([vp, i64, i64, vp, vp], i32),
        "lgmlh_forward_workspace": ([C.POINTER(Model), C.POINTER(PlanInfo), C.POINTER(PlanInfo),
                                     i32], sz),
        "lgmlh_forward": ([C.POINTER(Model), C.POINTER(Ubatch), C.POINTER(Ubatch), vp, i32, vp,
                           vp, sz, C.POINTER(Trace), vp], i32),
        "lgmlh_forward_release": ([], i32),
        "lgmlh_kvpool_bytes": ([C.c_int32, C.c_int32], sz),
        "lgmlh_kvpool_init": ([vp, sz, C.c_int32, C.c_int32, C.c_int32], i32),
        "lgmlh_kvpool_take": ([vp, C.c_int32], C.c_int32),
        "lgmlh_kvpool_evict": ([vp], C.c_int32),
        "lgmlh_kvpool_victim": ([vp, C.POINTER(C.c_int32)], C.c_int32),
        "lgmlh_kvpool_ref": ([vp, C.c_int32, i32], i32),
        "lgmlh_kvpool_unref": ([vp, C.c_int32], i32),
        "lgmlh_kvpool_refs_of": ([vp, C.c_int32], C.c_int32),
        "lgmlh_kvpool_publish": ([vp, C.c_int32, C.c_char_p, C.c_char_p, C.c_int32, vp, C.c_int32,
                                  i32], i32),
        "lgmlh_kvpool_publish_part": ([vp, C.c_int32, C.c_char_p, C.c_int32, vp, C.c_int32, i32],
                                      i32),
        "lgmlh_kvpool_key_of": ([vp, C.c_int32, vp], i32),
        "lgmlh_kvpool_lookup": ([vp, C.c_char_p], C.c_int32),
        "lgmlh_kvpool_longest_kid": ([vp, C.c_char_p, vp, C.c_int32, C.POINTER(C.c_int32)],
                                     C.c_int32),
        "lgmlh_kvpool_set_cap": ([vp, C.c_int32], i32),
        "lgmlh_kvpool_stats": ([vp, vp], i32),
        "lgmlh_block_key": ([C.c_char_p, vp, C.c_int32, vp], i32),
        "lgmlh_gen_normal": ([C.c_uint64, i32, i64, i64, C.c_double, C.c_double, vp, vp], i32),
        "lgmlh_moe_route": ([vp, i64, i32, i32, i32, i32, C.c_float, vp, vp, vp], i32),
        "lgmlh_mul_mat_id_workspace": ([i32, i64, i64, i64, i64, i64, i32], sz),
        "lgmlh_mul_mat_id": ([i32, vp, i64, i64, i64, vp, i32, i64, vp, i64, i32, vp, vp, sz, vp],
                             i32),
        "lgmlh_mul_mat_id_ggml": ([i32, vp, i64, i64, i64, vp, i32, i64, vp, i64, i32, vp, vp, sz,
                                   vp], i32),
        "lgmlh_moe_sum": ([vp, vp, i64, i32, i64, vp, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res


def check(rc):
    if rc != OK:
        raise LgmlhError(rc, lib().lgmlh_last_error().decode())
    return rc


def last_error():
    return lib().lgmlh_last_error().decode()


def ptr(t):
    """Device (or host) address of a torch tensor / numpy array, or None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream
