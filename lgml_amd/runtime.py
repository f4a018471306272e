"""Host driver of the HIP path: device weights, the KV pool, ubatch plans
and forward passes (the roles of transformer.lua's load / M:pool /
batch_inputs / run_batch, lua/lgml/transformer.lua:380-435,678-705,
2502-2624), over the C ABI of liblgml_hip.so.

Weights arrive as a dict of numpy arrays in ggml layouts:
{"tok_embd": (arr, type), "output": ..., "output_norm": (f32, F32),
 "rope_freqs": f32 or None, "layers": [{"attn_norm", "wq", "wk", "wv",
 "wo", "ffn_norm", "gate", "up", "down", optional "q_norm", "k_norm"}]},
quantized arrays as uint8 (rows, row_bytes), f32 as (rows, cols).
"""
import ctypes as C

import numpy as np
import torch

from . import hip
from .hip import check, ptr, stream

DEV = "cuda"


def _dev(arr):
    """Copy a numpy array to a new device tensor (bytes preserved)."""
    a = np.ascontiguousarray(arr)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy())
    return t.to(DEV)


def _empty(nbytes):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=DEV)


def _zeros(nbytes):
    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device=DEV)


def repack_concat(parts, K):
    """Repack weight matrices of one type (each (rows, row_bytes) in ggml
    layout, rows a multiple of 16) into one device matrix [p0 | p1 | ...]."""
    ty = parts[0][1]
    assert all(p[1] == ty for p in parts)
    rows = [p[0].shape[0] for p in parts]
    M = sum(rows)
    L = hip.lib()
    if ty == hip.F32:
        return _dev(np.concatenate([np.ascontiguousarray(p[0], np.float32) for p in parts])), ty, M
    total = L.lgmlh_repacked_bytes(ty, M, K)
    if total < 0:
        raise ValueError("cannot repack type %d (%d x %d)" % (ty, M, K))
    out = _empty(total)
    off = 0
    for (arr, _), r in zip(parts, rows):
        assert r % 16 == 0, "fused matrices need rows in multiples of 16"
        src = _dev(arr)
        nb = L.lgmlh_repacked_bytes(ty, r, K)
        check(L.lgmlh_repack(ty, r, K, ptr(src), out.data_ptr() + off, stream()))
        off += nb
    return out, ty, M


class Plan:
    """A planned ubatch (lgmlh_plan), copied to the device."""

    def __init__(self, seq_n, seq_npast, block_tab, ids, n_head, n_head_kv, pool_blocks,
                 blocks_per_split=0):
        L = hip.lib()
        self.seq_n = np.ascontiguousarray(seq_n, np.int32)
        self.seq_npast = np.ascontiguousarray(seq_npast, np.int32)
        bt = np.ascontiguousarray(block_tab, np.int32)
        if bt.ndim == 1:
            bt = bt.reshape(len(self.seq_n), -1)
        self.block_tab = bt
        self.ids = np.ascontiguousarray(ids, np.int32)
        assert len(self.ids) == int(self.seq_n.sum())
        self.info = hip.PlanInfo()
        args = (len(self.seq_n), ptr(self.seq_n), ptr(self.seq_npast), ptr(bt), bt.shape[1],
                int(pool_blocks), ptr(self.ids), n_head, n_head_kv, blocks_per_split)
        check(L.lgmlh_plan(*args, None, 0, C.byref(self.info)))
        self.host = np.zeros(self.info.bytes, np.uint8)
        check(L.lgmlh_plan(*args, ptr(self.host), self.host.nbytes, C.byref(self.info)))
        self.dev = torch.from_numpy(self.host).to(DEV)
        self.ub = hip.Ubatch()
        check(L.lgmlh_plan_bind(C.byref(self.info), self.dev.data_ptr(), C.byref(self.ub)))

    def host_array(self, off, n, dtype):
        return self.host[off:off + n * np.dtype(dtype).itemsize].view(dtype)

    @property
    def cells(self):
        return self.host_array(self.info.off_cells, self.info.n_tokens, np.int64)

    @property
    def logit_rows(self):
        return self.host_array(self.info.off_logit_rows, self.info.n_seq, np.int32)


class DeviceModel:
    """A dense llama / qwen3 model on the device with its paged KV pool."""

    def __init__(self, hp, w, n_cells):
        L = hip.lib()
        self.hp = hp
        E, H, Hkv, D = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        F, V = hp["n_ff"], hp["n_vocab"]
        self.n_cells = int(n_cells)
        assert self.n_cells % 64 == 0
        self._keep = []

        def keep(t):
            self._keep.append(t)
            return t

        kvb = L.lgmlh_kv_layer_bytes(self.n_cells, Hkv, D)
        self.kpools, self.vpools = [], []
        self.layers = (hip.Layer * hp["n_layer"])()
        for il, lw in enumerate(w["layers"]):
            Ly = self.layers[il]
            Ly.attn_norm = keep(_dev(np.asarray(lw["attn_norm"][0], np.float32))).data_ptr()
            Ly.ffn_norm = keep(_dev(np.asarray(lw["ffn_norm"][0], np.float32))).data_ptr()
            for nm in ("q_norm", "k_norm"):
                if lw.get(nm) is not None:
                    setattr(Ly, nm, keep(_dev(np.asarray(lw[nm][0], np.float32))).data_ptr())
            qk = [lw["wq"], lw["wk"]]
            if lw["wv"][1] == lw["wq"][1] == lw["wk"][1]:
                t, ty, M = repack_concat(qk + [lw["wv"]], E)
                Ly.wv = None
            else:
                t, ty, M = repack_concat(qk, E)
                tv, tyv, _ = repack_concat([lw["wv"]], E)
                Ly.wv, Ly.wv_type = keep(tv).data_ptr(), tyv
            Ly.wqkv, Ly.wqkv_type, Ly.wqkv_rows = keep(t).data_ptr(), ty, M
            t, ty, _ = repack_concat([lw["wo"]], H * D)
            Ly.wo, Ly.wo_type = keep(t).data_ptr(), ty
            t, ty, _ = repack_concat([lw["gate"], lw["up"]], E)
            Ly.wgu, Ly.wgu_type = keep(t).data_ptr(), ty
            t, ty, _ = repack_concat([lw["down"]], F)
            Ly.wdown, Ly.wdown_type = keep(t).data_ptr(), ty
            kp, vp = keep(_zeros(kvb)), keep(_zeros(kvb))
            self.kpools.append(kp)
            self.vpools.append(vp)
            Ly.kpool, Ly.vpool = kp.data_ptr(), vp.data_ptr()
        m = hip.Model()
        for k in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                  "n_rot", "rope_neox"):
            setattr(m, k, int(hp[k]))
        m.eps, m.rope_base = hp["eps"], hp["rope_base"]
        m.attn_scale = hp.get("attn_scale", 0.0)
        if w.get("rope_freqs") is not None:
            m.rope_freqs = keep(_dev(np.asarray(w["rope_freqs"], np.float32))).data_ptr()
        arr, ty = w["tok_embd"]
        m.tok_embd, m.tok_embd_type = keep(_dev(arr)).data_ptr(), ty
        t, ty, _ = repack_concat([w["output"]], E)
        m.output, m.output_type = keep(t).data_ptr(), ty
        m.output_norm = keep(_dev(np.asarray(w["output_norm"][0], np.float32))).data_ptr()
        m.n_cells = self.n_cells
        m.layers = self.layers
        self.m = m
        self.ws = None
        self.ws_bytes = 0

    @property
    def pool_blocks(self):
        return self.n_cells // 64

    def plan(self, seq_n, seq_npast, block_tab, ids, blocks_per_split=0):
        ids = np.ascontiguousarray(ids, np.int32)
        if len(ids) and (ids.min() < 0 or ids.max() >= self.hp["n_vocab"]):
            raise ValueError("token id out of range [0, %d)" % self.hp["n_vocab"])
        return Plan(seq_n, seq_npast, block_tab, ids, self.hp["n_head"], self.hp["n_head_kv"],
                    self.pool_blocks, blocks_per_split)

    def workspace(self, plan, n_out):
        need = hip.lib().lgmlh_forward_workspace(C.byref(self.m), C.byref(plan.info), n_out)
        if need > self.ws_bytes:
            # zero-filled when (re)allocated: the split-K counters start at 0
            # and every pass leaves them at 0
            self.ws = _zeros(need)
            self.ws_bytes = need
        return self.ws

    def forward(self, plan, out_rows=None, logits=None):
        """Logits (n_out, vocab) f32 on the device for out_rows (ubatch token
        indices; default the last token of each sequence)."""
        if out_rows is None:
            n_out, rows = plan.info.n_seq, None
        else:
            rows = torch.as_tensor(np.ascontiguousarray(out_rows, np.int32)).to(DEV)
            n_out = rows.numel()
        ws = self.workspace(plan, n_out)
        if logits is None:
            logits = torch.empty((n_out, self.hp["n_vocab"]), dtype=torch.float32, device=DEV)
        check(hip.lib().lgmlh_forward(C.byref(self.m), C.byref(plan.ub), ptr(rows), n_out,
                                      logits.data_ptr(), ws.data_ptr(), self.ws_bytes, stream()))
        return logits

    def gather_kv(self, layer, cells, which=0):
        """Cells of a layer's K (0) or V (1) as (n, Hkv*D) f16 bits (uint16)."""
        cells = np.ascontiguousarray(cells, np.int64)
        dc = torch.from_numpy(cells).to(DEV)
        out = torch.empty((len(cells), self.hp["n_head_kv"] * self.hp["head_dim"]),
                          dtype=torch.int16, device=DEV)
        pool = (self.kpools if which == 0 else self.vpools)[layer]
        check(hip.lib().lgmlh_kv_gather(pool.data_ptr(), which, self.n_cells,
                                        self.hp["n_head_kv"], self.hp["head_dim"],
                                        dc.data_ptr(), len(cells), out.data_ptr(), stream()))
        return out.cpu().numpy().view(np.uint16)
