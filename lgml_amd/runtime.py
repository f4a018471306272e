"""Host driver of the HIP path: device weights, the KV pool, ubatch plans
and forward passes (the roles of transformer.lua's load / M:pool /
batch_inputs / run_batch, lua/lgml/transformer.lua:380-435,678-705,
2502-2624), over the C ABI of liblgml_hip.so.

Weights arrive as a dict of numpy arrays in ggml layouts:
{"tok_embd": (arr, type), "output": ..., "output_norm": (f32, F32),
 "rope_freqs": f32 or None, "layers": [{"attn_norm", "wq", "wk", "wv",
 "wo", "ffn_norm", "gate", "up", "down", optional "q_norm", "k_norm"}]},
quantized arrays as uint8 (rows, row_bytes), f32 as (rows, cols). Gemma
layers add "post_attn_norm", "post_ffn_norm" and the scalars "swa",
"rope_base", "out_scale", optional "rope_freqs"; a layer without "wv"
takes V from the raw K; "output" may be the "tok_embd" entry (tied).
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
    """Repack weight matrices of one type into one device matrix
    [p0 | p1 | ...]. Each part is (arr, type) with arr a numpy array (ggml
    layout: uint8 (rows, row_bytes), or f32 (rows, K)) or (dev, type, rows)
    with dev a device uint8 tensor in the same layout. Rows of fused parts
    come in multiples of 16 (whole row tiles)."""
    ty = parts[0][1]
    assert all(p[1] == ty for p in parts)
    rows = [p[2] if len(p) > 2 else p[0].shape[0] for p in parts]
    M = sum(rows)
    L = hip.lib()

    def on_dev(p):
        return p[0] if len(p) > 2 else _dev(p[0])

    if ty == hip.F32:
        return torch.cat([on_dev(p) for p in parts]), ty, M
    total = L.lgmlh_repacked_bytes(ty, M, K)
    if total < 0:
        raise ValueError("cannot repack type %d (%d x %d)" % (ty, M, K))
    out = _empty(total)
    off = 0
    for p, r in zip(parts, rows):
        assert r % 16 == 0 or len(parts) == 1, "fused matrices need rows in multiples of 16"
        src = on_dev(p)
        nb = L.lgmlh_repacked_bytes(ty, r, K)
        check(L.lgmlh_repack(ty, r, K, ptr(src), out.data_ptr() + off, stream()))
        off += nb
    torch.cuda.current_stream().synchronize()  # sources may go
    return out, ty, M


def repack_experts(gate, up, n_expert, K):
    """n_expert matrices of R rows each (gate: (arr, type) or (dev, type,
    rows) with n_expert * R rows, expert-major) repacked one after the other,
    as lgmlh_mul_mat_id takes them; with up given, each expert's matrix is
    [gate_e | up_e] (2R rows). R must be a multiple of 16."""
    g, ty, rows = repack_concat([gate], K)
    R = rows // n_expert
    assert R * n_expert == rows and R % 16 == 0
    if up is None:
        return g, ty
    u, tyu, _ = repack_concat([up], K)
    assert tyu == ty, "gate and up experts must share a type"
    return torch.stack([g.view(n_expert, -1), u.view(n_expert, -1)], 1).reshape(-1), ty


def router_sd(hp):
    """Router weights N(0, 1 / sqrt(n_embd)): logits of a unit-rms h are then
    N(0, 1) (BASELINE.json's MoE config)."""
    return 1.0 / float(np.sqrt(hp["n_embd"]))


def generated_weights(hp, seed, policy):
    """A weights source for DeviceModel that makes each matrix on the device
    with lgmlh_gen_normal: N(0, 0.02) (the router N(0, 1/sqrt(n_embd))), one
    seed per tensor in draw order; norms are 1. policy(name, layer) gives
    the weight type."""
    counter = [0]

    def get(name, layer, rows, cols):
        ty = policy(name, layer)
        counter[0] += 1
        nb = hip.lib().lgmlh_row_size(ty, cols) * rows
        t = _empty(nb)
        sd = router_sd(hp) if name == "gate_inp" else 0.02
        check(hip.lib().lgmlh_gen_normal(seed * 1000003 + counter[0], ty, rows, cols, 0.0, sd,
                                         t.data_ptr(), stream()))
        return (t, ty, rows)

    return get


def load_gguf(path, n_cells, ring_cells=0):
    """A DeviceModel from a gguf file (lgml_amd.gguf.load: llama, qwen3,
    qwen3moe, gemma4; a gemma4 model's sliding and global layers keep their
    own head sizes and KV head counts)."""
    from . import gguf
    hp, w = gguf.load(path)
    return DeviceModel(hp, w, n_cells, ring_cells)


class Plan:
    """A planned ubatch (lgmlh_plan), copied to the device. With ring_tab
    (n_seq, ring_blocks) and window, the plan of the sliding-window layers
    over the sequences' rings (lgmlh_plan_ring); pool_blocks is then the
    ring pools' block count. .ring: the pass's ring plan, if any."""

    def __init__(self, seq_n, seq_npast, block_tab, ids, n_head, n_head_kv, pool_blocks,
                 blocks_per_split=0, ring_tab=None, window=0):
        L = hip.lib()
        self.ring = None
        self.seq_n = np.ascontiguousarray(seq_n, np.int32)
        self.seq_npast = np.ascontiguousarray(seq_npast, np.int32)
        bt = np.ascontiguousarray(block_tab, np.int32)
        if bt.ndim == 1:
            bt = bt.reshape(len(self.seq_n), -1)
        self.block_tab = bt
        self.ids = np.ascontiguousarray(ids, np.int32)
        assert len(self.ids) == int(self.seq_n.sum())
        self.info = hip.PlanInfo()
        if ring_tab is None:
            fn = L.lgmlh_plan
            args = (len(self.seq_n), ptr(self.seq_n), ptr(self.seq_npast), ptr(bt), bt.shape[1],
                    int(pool_blocks), ptr(self.ids), n_head, n_head_kv, blocks_per_split)
        else:
            fn = L.lgmlh_plan_ring
            args = (len(self.seq_n), ptr(self.seq_n), ptr(self.seq_npast), ptr(bt), bt.shape[1],
                    int(pool_blocks), int(window), ptr(self.ids), n_head, n_head_kv,
                    blocks_per_split)
        check(fn(*args, None, 0, C.byref(self.info)))
        # pinned host memory: the upload is an asynchronous copy on the
        # stream, so the host does not wait for the work queued before it
        self._pinned = torch.empty(self.info.bytes, dtype=torch.uint8, pin_memory=True)
        self.host = self._pinned.numpy()
        check(fn(*args, ptr(self.host), self.host.nbytes, C.byref(self.info)))
        self.dev = self._pinned.to(DEV, non_blocking=True)
        self.ub = hip.Ubatch()
        check(L.lgmlh_plan_bind(C.byref(self.info), self.dev.data_ptr(), C.byref(self.ub)))

    def host_array(self, off, n, dtype):
        return self.host[off:off + n * np.dtype(dtype).itemsize].view(dtype)

    def dev_ids(self):
        """The pass's token ids on the device (int32), as the forward reads
        them."""
        n = self.info.n_tokens
        return self.dev[self.info.off_ids:self.info.off_ids + 4 * n].view(torch.int32)

    @property
    def cells(self):
        return self.host_array(self.info.off_cells, self.info.n_tokens, np.int64)

    @property
    def logit_rows(self):
        return self.host_array(self.info.off_logit_rows, self.info.n_seq, np.int32)


class EventTrace:
    """HIP events (torch.cuda.Event handles) that lgmlh_forward records around
    the launch groups of the kinds asked for, on the pass's own stream."""

    def __init__(self, capacity, kinds=hip.TRACE_ATTN):
        self.events = [torch.cuda.Event(enable_timing=True) for _ in range(2 * capacity)]
        for e in self.events:  # torch creates the HIP event on first record
            e.record()
        torch.cuda.synchronize()
        self.handles = (C.c_void_p * (2 * capacity))(*[e.cuda_event for e in self.events])
        self.kinds_arr = (C.c_int32 * capacity)()
        self.c = hip.Trace(self.handles, capacity, 0, kinds, self.kinds_arr)

    def reset(self):
        self.c.used = 0

    def times_ms(self, kind):
        """Elapsed ms of every recorded slot of one kind (synchronizes)."""
        torch.cuda.synchronize()
        out = []
        for i in range(self.c.used):
            if self.kinds_arr[i] == kind:
                out.append(self.events[2 * i].elapsed_time(self.events[2 * i + 1]))
        return out


class DeviceModel:
    """A llama / qwen3 / qwen3moe / gemma model on the device with its paged
    KV pool (and, for sliding-window layers, ring pools)."""

    def __init__(self, hp, w, n_cells, ring_cells=0, kv_initial=0):
        """w: a weights dict of numpy arrays, or a callable source
        w(name, layer, rows, cols) -> (device tensor, type, rows) such as
        generated_weights() (gemma layers then follow workload.gemma_layer).
        ring_cells: cells of each sliding layer's ring pools (a multiple of
        64; the sequences' ring tables index its blocks). kv_initial: the
        paged pool starts at this many cells and grows (grow_pool) up to
        n_cells, as the reference's pool starts at KV_INITIAL and doubles
        (engine.lua:49, transformer.lua:831-908); 0: n_cells from the start."""
        from . import workload
        L = hip.lib()
        self.hp = hp
        E, H, Hkv, D = hp["n_embd"], hp["n_head"], hp["n_head_kv"], hp["head_dim"]
        F, V = hp["n_ff"], hp["n_vocab"]
        self.max_cells = int(n_cells)
        self.n_cells = int(kv_initial) if kv_initial else self.max_cells
        self.ring_cells = int(ring_cells)
        assert self.n_cells % 64 == 0 and self.ring_cells % 64 == 0
        assert self.max_cells % 64 == 0 and self.n_cells <= self.max_cells
        self._keep = []
        gen = callable(w)
        gemma = bool(hp.get("gemma"))

        def layer_info(il):
            if not gemma:
                return {}
            if gen:
                return workload.gemma_layer(hp, il)
            lw = w["layers"][il]
            return {k: lw[k] for k in ("swa", "rope_base", "out_scale", "rope_freqs") if k in lw}

        def keep(t):
            self._keep.append(t)
            return t

        def mat(name, layer, rows, cols):
            if gen:
                return w(name, layer, rows, cols)
            return w["layers"][layer][name] if layer is not None else w[name]

        def vec(name, layer, n):
            if gen:
                # norms 1; gemma's q / k norms D^(-1/4): scores of unit scale
                # at attention scale 1
                v = D ** -0.25 if gemma and name in ("q_norm", "k_norm") else 1.0
                return keep(torch.full((n,), v, dtype=torch.float32, device=DEV)).data_ptr()
            arr = w["layers"][layer][name][0] if layer is not None else w[name][0]
            return keep(_dev(np.asarray(arr, np.float32))).data_ptr()

        self.kpools, self.vpools = [], []
        self.layers = (hip.Layer * hp["n_layer"])()
        qk_norm = hp["arch"] in ("qwen3", "qwen3moe", "gemma4")
        NE = hp.get("n_expert", 0)
        self.swa = []
        self.dims = []  # (head_dim, n_head_kv) per layer
        rope_dev = {}  # the bytes of a layer's rope factors -> their device copy
        for il in range(hp["n_layer"]):
            Ly = self.layers[il]
            g = layer_info(il)
            # this layer's head size and KV heads (gemma's sliding and global
            # layers differ, transformer.lua:215-235)
            lw = w["layers"][il] if not gen else {}
            Dl, Hl = int(lw.get("head_dim") or D), int(lw.get("n_head_kv") or Hkv)
            Ly.head_dim, Ly.n_head_kv = Dl, Hl
            Ly.n_rot = int(lw.get("n_rot") or 0)
            self.dims.append((Dl, Hl))
            Ly.attn_norm = vec("attn_norm", il, E)
            Ly.ffn_norm = vec("ffn_norm", il, E)
            for nm in ("q_norm", "k_norm"):
                if (gen and qk_norm) or (not gen and w["layers"][il].get(nm) is not None):
                    setattr(Ly, nm, vec(nm, il, Dl))
            if gemma:
                for nm in ("post_attn_norm", "post_ffn_norm"):
                    if gen or w["layers"][il].get(nm) is not None:
                        setattr(Ly, nm, vec(nm, il, E))
                Ly.out_scale = g.get("out_scale", 0.0)
                Ly.rope_base = g.get("rope_base", 0.0)
                if g.get("rope_freqs") is not None:
                    # layers with the same factors share one device copy (and
                    # so one rope angle table per pass)
                    rf = np.ascontiguousarray(g["rope_freqs"], np.float32)
                    key = rf.tobytes()
                    if key not in rope_dev:
                        rope_dev[key] = keep(_dev(rf)).data_ptr()
                    Ly.rope_freqs = rope_dev[key]
            Ly.swa = int(g.get("swa", 0))
            self.swa.append(bool(Ly.swa))
            if Ly.swa and self.ring_cells <= 0:
                raise ValueError("layer %d slides: the model needs ring_cells" % il)
            has_wv = g.get("has_wv", True) if gen else "wv" in w["layers"][il]
            wq, wk = mat("wq", il, H * Dl, E), mat("wk", il, Hl * Dl, E)
            wv = mat("wv", il, Hl * Dl, E) if has_wv else None
            if wv is None:
                # V is the raw K (transformer.lua:1779): wqkv holds [wq | wk]
                t, ty, M = repack_concat([wq, wk], E)
                Ly.wv, Ly.v_from_k = None, 1
            elif wv[1] == wq[1] == wk[1]:
                t, ty, M = repack_concat([wq, wk, wv], E)
                Ly.wv = None
            else:
                t, ty, M = repack_concat([wq, wk], E)
                tv, tyv, _ = repack_concat([wv], E)
                Ly.wv, Ly.wv_type = keep(tv).data_ptr(), tyv
            Ly.wqkv, Ly.wqkv_type, Ly.wqkv_rows = keep(t).data_ptr(), ty, M
            del wq, wk, wv
            t, ty, _ = repack_concat([mat("wo", il, E, H * Dl)], H * Dl)
            Ly.wo, Ly.wo_type = keep(t).data_ptr(), ty
            if NE:
                # routed experts: the router stays f32 (convert.lua:135-137)
                FX = hp["n_ff_exp"]
                gi = mat("gate_inp", il, NE, E)
                assert gi[1] == hip.F32, "the router is f32"
                Ly.gate_inp = keep(gi[0] if gen else _dev(np.asarray(gi[0], np.float32))).data_ptr()
                t, ty = repack_experts(mat("gate_exps", il, NE * FX, E),
                                       mat("up_exps", il, NE * FX, E), NE, E)
                Ly.exp_gu, Ly.exp_gu_type = keep(t).data_ptr(), ty
                t, ty = repack_experts(mat("down_exps", il, NE * E, FX), None, NE, FX)
                Ly.exp_down, Ly.exp_down_type = keep(t).data_ptr(), ty
            else:
                t, ty, _ = repack_concat([mat("gate", il, F, E), mat("up", il, F, E)], E)
                Ly.wgu, Ly.wgu_type = keep(t).data_ptr(), ty
                t, ty, _ = repack_concat([mat("down", il, E, F)], F)
                Ly.wdown, Ly.wdown_type = keep(t).data_ptr(), ty
            # the pool tensors live in kpools / vpools (grow_pool replaces them)
            kvb_l = L.lgmlh_kv_layer_bytes(self.ring_cells if Ly.swa else self.n_cells, Hl, Dl)
            kp = _zeros(kvb_l)
            vp = _zeros(kvb_l)
            self.kpools.append(kp)
            self.vpools.append(vp)
            Ly.kpool, Ly.vpool = kp.data_ptr(), vp.data_ptr()
        # the paged layers share one head shape, and so do the sliding ones:
        # each kind attends through one plan (made for its KV heads), and
        # the block copies take one row layout per pool kind
        kinds = {sw: {d for d, s_ in zip(self.dims, self.swa) if s_ == sw} for sw in (False, True)}
        for sw, ds in kinds.items():
            if len(ds) > 1:
                raise ValueError("%s layers with head shapes %s: one (head_dim, n_head_kv) per kind"
                                 % ("sliding" if sw else "paged", sorted(ds)))
        self.paged_dims = next(iter(kinds[False])) if kinds[False] else (D, Hkv)
        self.ring_dims = next(iter(kinds[True])) if kinds[True] else (D, Hkv)
        m = hip.Model()
        for k in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_vocab",
                  "n_rot", "rope_neox"):
            setattr(m, k, int(hp[k]))
        m.eps, m.rope_base = hp["eps"], hp["rope_base"]
        m.attn_scale = hp.get("attn_scale", 0.0)
        if not gen and w.get("rope_freqs") is not None:
            m.rope_freqs = keep(_dev(np.asarray(w["rope_freqs"], np.float32))).data_ptr()
        te = mat("tok_embd", None, V, E)
        if gen:
            ted = keep(te[0])
        else:
            ted = keep(_dev(te[0]))
        m.tok_embd, m.tok_embd_type = ted.data_ptr(), te[1]
        if gemma or (not gen and w["output"] is w["tok_embd"]):
            # tied output (transformer.lua:408): the head reads a repacked
            # copy of the embedding table
            t, ty, _ = repack_concat([(ted, te[1], V)], E)
        else:
            t, ty, _ = repack_concat([mat("output", None, V, E)], E)
        m.output, m.output_type = keep(t).data_ptr(), ty
        m.output_norm = vec("output_norm", None, E)
        m.n_cells = self.n_cells
        m.ring_cells = self.ring_cells
        m.layers = self.layers
        # hp["act_quant"]: the reference CPU path's arithmetic for quantized
        # weights (X quantized to Q8_K / Q8_0 per block, integer block dots)
        m.act = hip.ACT_GGML if hp.get("act_quant") else hip.ACT_EXACT
        if gemma:
            m.gemma = 1
            m.embd_scale = hp.get("embd_scale", 0.0)
            m.softcap = hp.get("softcap", 0.0)
        if NE:
            m.n_expert, m.n_used, m.n_ff_exp = NE, hp["n_used"], hp["n_ff_exp"]
            m.gating = hp.get("gating", hip.GATING_SOFTMAX)
            m.norm_topk = int(bool(hp.get("norm_topk", True)))
            m.expert_scale = hp.get("expert_scale", 1.0)
        self.m = m
        self.ws = None
        self.ws_bytes = 0
        self._side_ws = {}  # workspaces of passes run concurrently on other streams
        # the pool tensors of the paged layers as a device array (K, V of
        # each layer in order), for the one-launch block copies to host
        # memory (lgmlh_kv_block_host)
        ptrs = []
        for il in range(hp["n_layer"]):
            if not self.swa[il]:
                ptrs += [self.kpools[il].data_ptr(), self.vpools[il].data_ptr()]
        self.n_pools = len(ptrs)
        self.pools_dev = torch.tensor(ptrs or [0], dtype=torch.int64, device=DEV)
        self.block_bytes_all = self.n_pools * L.lgmlh_kv_block_bytes(self.paged_dims[1],
                                                                     self.paged_dims[0])

    @property
    def pool_blocks(self):
        return self.n_cells // 64

    @property
    def max_blocks(self):
        return self.max_cells // 64

    def grow_pool(self, cells=None):
        """pool_grow (transformer.lua:831-908): the paged pool tensors of
        every layer to `cells` cells (default twice the present, at most
        max_cells); the new tensors hold the old cells (lgmlh_kv_grow) and
        zeros after them. Returns the new cell count (unchanged at the
        ceiling). Sliding layers' rings keep their size."""
        cells = min(self.max_cells, cells or 2 * self.n_cells)
        if cells <= self.n_cells:
            return self.n_cells
        L, hp = hip.lib(), self.hp
        D, Hkv = self.paged_dims
        nb = L.lgmlh_kv_layer_bytes(cells, Hkv, D)
        for il in range(hp["n_layer"]):
            if self.swa[il]:
                continue
            for pools, attr in ((self.kpools, "kpool"), (self.vpools, "vpool")):
                old = pools[il]
                new = _empty(nb)
                check(L.lgmlh_kv_grow(old.data_ptr(), self.n_cells, new.data_ptr(), cells, Hkv, D,
                                      stream()))
                pools[il] = new
                setattr(self.layers[il], attr, new.data_ptr())
        # the old tensors are freed once the copies are done
        torch.cuda.current_stream().synchronize()
        self.n_cells = cells
        self.m.n_cells = cells
        ptrs = []
        for il in range(hp["n_layer"]):
            if not self.swa[il]:
                ptrs += [self.kpools[il].data_ptr(), self.vpools[il].data_ptr()]
        self.pools_dev = torch.tensor(ptrs or [0], dtype=torch.int64, device=DEV)
        return cells

    ring_blocks_per_split = 0  # the ring plans' run length (0: as blocks_per_split; 12 for heads of 256)

    def plan(self, seq_n, seq_npast, block_tab, ids, blocks_per_split=0, ring_tab=None):
        """The pass's plan; with sliding layers also its ring plan (.ring)
        over ring_tab (n_seq, ring blocks), the sequences' rings.
        blocks_per_split 0: for heads of 256 (their kernel holds one wave per
        SIMD), runs of 28 KV blocks over the paged pool (fewer, longer items
        stay within one round of waves) and of 12 through the rings (a
        window's few blocks over more waves; with the longest runs started
        first, C4 7172 -> 7462 tok/s against 32 and 16; 24 / 26 / 30 and
        10 / 14 are no better); else runs of 12 (C2 decode 7263 -> 7407
        tok/s against 16; 10: 7383, 8: 7088). The run length is fixed per
        model, so split points still depend on a sequence's own length
        only."""
        ids = np.ascontiguousarray(ids, np.int32)
        ring_bps = self.ring_blocks_per_split or blocks_per_split
        if not ring_bps and self.hp["head_dim"] >= 256:
            ring_bps = 12
        if not blocks_per_split and self.hp["head_dim"] >= 256:
            blocks_per_split = 28
        elif not blocks_per_split:
            blocks_per_split = 12
        if len(ids) and (ids.min() < 0 or ids.max() >= self.hp["n_vocab"]):
            raise ValueError("token id out of range [0, %d)" % self.hp["n_vocab"])
        p = Plan(seq_n, seq_npast, block_tab, ids, self.hp["n_head"], self.paged_dims[1],
                 self.pool_blocks, blocks_per_split)
        if any(self.swa):
            if ring_tab is None:
                raise ValueError("the model has sliding-window layers: pass ring_tab")
            p.ring = Plan(seq_n, seq_npast, ring_tab, ids, self.hp["n_head"],
                          self.ring_dims[1], self.ring_cells // 64, ring_bps,
                          ring_tab=ring_tab, window=self.hp["n_swa"])
        return p

    def workspace(self, plan, n_out, slot=0):
        """The forward's workspace; slot > 0: one of its own, for a pass that
        runs at the same time as slot 0's on another stream."""
        need = hip.lib().lgmlh_forward_workspace(
            C.byref(self.m), C.byref(plan.info),
            C.byref(plan.ring.info) if plan.ring is not None else None, n_out)
        if slot:
            ws = self._side_ws.get(slot)
            if ws is None or ws.numel() < need:
                ws = self._side_ws[slot] = _empty(need)
            return ws, ws.numel()
        if need > self.ws_bytes:
            self.ws = _empty(need)
            self.ws_bytes = need
        return self.ws, self.ws_bytes

    def forward(self, plan, out_rows=None, logits=None, trace=None, slot=0):
        """Logits (n_out, vocab) f32 on the device for out_rows (ubatch token
        indices; default the last token of each sequence), on the current
        stream. trace: an EventTrace to time launch groups with HIP events.
        slot: the workspace (see workspace())."""
        if out_rows is None:
            n_out, rows = plan.info.n_seq, None
        else:
            rows = torch.as_tensor(np.ascontiguousarray(out_rows, np.int32)).to(DEV)
            n_out = rows.numel()
        ws, ws_bytes = self.workspace(plan, n_out, slot)
        if logits is None:
            logits = torch.empty((n_out, self.hp["n_vocab"]), dtype=torch.float32, device=DEV)
        check(hip.lib().lgmlh_forward(C.byref(self.m), C.byref(plan.ub),
                                      C.byref(plan.ring.ub) if plan.ring is not None else None,
                                      ptr(rows), n_out, logits.data_ptr(), ws.data_ptr(),
                                      ws_bytes,
                                      C.byref(trace.c) if trace is not None else None, stream()))
        return logits

    def gather_kv(self, layer, cells, which=0):
        """Cells of a layer's K (0) or V (1) as (n, Hkv*D) f16 bits (uint16)
        (ring cells for a sliding layer)."""
        cells = np.ascontiguousarray(cells, np.int64)
        dc = torch.from_numpy(cells).to(DEV)
        D, Hkv = self.dims[layer]
        out = torch.empty((len(cells), Hkv * D), dtype=torch.int16, device=DEV)
        pool = (self.kpools if which == 0 else self.vpools)[layer]
        n = self.ring_cells if self.swa[layer] else self.n_cells
        check(hip.lib().lgmlh_kv_gather(pool.data_ptr(), which, n, Hkv, D,
                                        dc.data_ptr(), len(cells), out.data_ptr(), stream()))
        return out.cpu().numpy().view(np.uint16)
