"""CPU checks of the C ABI: the library loads, exports every function that
include/lgml_hip.h declares, and its host-only entry points (sizes, the
ubatch plan) behave; no GPU compute is called here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import kvpool as kp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "lgml_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lgmlh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def hip():
    from lgml_amd import build, hip
    if not os.path.exists(hip.LIB_PATH):
        build.build()
    hip.lib()
    return hip


def test_exports_every_declared_symbol(hip):
    names = declared()
    assert len(names) >= 20
    L = hip.lib()
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing
    assert sorted(hip.SYMBOLS) == names
    assert L.lgmlh_abi_version() == 7


def test_struct_layouts_match_the_header(hip, tmp_path):
    """The ctypes mirrors of lgmlh_layer / lgmlh_model / lgmlh_ubatch /
    lgmlh_plan_info have the C layout (gcc on the header: size and every
    field offset)."""
    import shutil
    import subprocess
    if not shutil.which("gcc"):
        pytest.skip("no gcc")
    structs = {"lgmlh_layer": hip.Layer, "lgmlh_model": hip.Model, "lgmlh_ubatch": hip.Ubatch,
               "lgmlh_plan_info": hip.PlanInfo, "lgmlh_trace": hip.Trace}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "lgml_hip.h"',
             'int main(void) {']
    for cn, py in structs.items():
        lines.append('printf("%s %%zu\\n", sizeof(%s));' % (cn, cn))
        for f, _ in py._fields_:
            lines.append('printf("%s.%s %%zu\\n", offsetof(%s, %s));' % (cn, f, cn, f))
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    out = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for cn, py in structs.items():
        assert int(out[cn]) == C.sizeof(py), cn
        for f, _ in py._fields_:
            assert int(out["%s.%s" % (cn, f)]) == getattr(py, f).offset, (cn, f)


def test_moe_entry_points_check_arguments(hip):
    """Host-side argument checks of the MoE entry points (no GPU work)."""
    L = hip.lib()
    # the grouping and the split X grow with the picks; f32 needs no split X
    a = L.lgmlh_mul_mat_id_workspace(hip.Q4_K, 128, 1536, 2048, 64, 1, 8)
    b = L.lgmlh_mul_mat_id_workspace(hip.Q4_K, 128, 1536, 2048, 128, 1, 8)
    f = L.lgmlh_mul_mat_id_workspace(hip.F32, 128, 1536, 2048, 64, 1, 8)
    assert 0 < f < a < b
    dummy = C.c_void_p(16)
    # bad shapes / types are refused before any device work
    assert L.lgmlh_mul_mat_id(hip.Q4_K, dummy, 128, 768, 100, dummy, hip.F32, 1, dummy, 4, 8,
                              dummy, dummy, 1 << 30, None) == hip.EINVAL
    assert b"256" in L.lgmlh_last_error()
    assert L.lgmlh_mul_mat_id(hip.Q4_K, dummy, 1000, 768, 256, dummy, hip.F32, 1, dummy, 4, 8,
                              dummy, dummy, 1 << 30, None) == hip.EINVAL
    assert L.lgmlh_mul_mat_id(hip.Q4_K, dummy, 128, 768, 256, dummy, hip.F32, 3, dummy, 4, 8,
                              dummy, dummy, 1 << 30, None) == hip.EINVAL
    assert L.lgmlh_mul_mat_id(hip.Q4_K, dummy, 128, 768, 256, dummy, hip.F32, 1, dummy, 4, 8,
                              dummy, dummy, 16, None) == hip.ENOMEM
    assert L.lgmlh_mul_mat_id(hip.Q4_K, dummy, 128, 768, 256, dummy, hip.F32, 1, dummy, 2000, 8,
                              dummy, dummy, 1 << 30, None) == hip.EINVAL
    assert L.lgmlh_moe_route(dummy, 4, 128, 17, 1, 1, 1.0, dummy, dummy, None) == hip.EINVAL
    assert L.lgmlh_moe_route(dummy, 4, 128, 8, 3, 1, 1.0, dummy, dummy, None) == hip.EINVAL
    assert L.lgmlh_moe_route(dummy, 4, 4, 8, 1, 1, 1.0, dummy, dummy, None) == hip.EINVAL


def test_sizes(hip):
    L = hip.lib()
    assert L.lgmlh_row_size(hip.Q4_K, 4096) == 16 * 144
    assert L.lgmlh_row_size(hip.Q6_K, 4096) == 16 * 210
    assert L.lgmlh_row_size(hip.Q8_0, 4096) == 128 * 34
    assert L.lgmlh_row_size(hip.Q4_K, 100) == -1
    assert L.lgmlh_kv_layer_bytes(4096, 8, 128) == 4096 * 8 * 128 * 2
    assert L.lgmlh_kv_layer_bytes(100, 8, 128) == -1
    assert L.lgmlh_repacked_bytes(hip.Q4_K, 4096, 4096) == 4096 * 16 * 144
    assert L.lgmlh_repacked_bytes(hip.Q6_K, 1000, 4096) == 63 * 16 * 16 * 210
    # split-K workspace does not depend on the batch size beyond the rows it holds
    a = L.lgmlh_mul_mat_workspace(hip.Q4_K, 4096, 4096, 64)
    b = L.lgmlh_mul_mat_workspace(hip.Q4_K, 4096, 4096, 128)
    assert a > 0 and b > a


def plan(hip, seq_n, npast, bt, ids, H, Hkv, pool_blocks, bps=0):
    L = hip.lib()
    info = hip.PlanInfo()
    bt = np.ascontiguousarray(bt, np.int32)
    args = (len(seq_n), np.ascontiguousarray(seq_n, np.int32).ctypes.data,
            np.ascontiguousarray(npast, np.int32).ctypes.data, bt.ctypes.data, bt.shape[1],
            pool_blocks, np.ascontiguousarray(ids, np.int32).ctypes.data, H, Hkv, bps)
    keep = [np.ascontiguousarray(seq_n, np.int32), np.ascontiguousarray(npast, np.int32),
            np.ascontiguousarray(ids, np.int32)]
    args = (len(seq_n), keep[0].ctypes.data, keep[1].ctypes.data, bt.ctypes.data, bt.shape[1],
            pool_blocks, keep[2].ctypes.data, H, Hkv, bps)
    rc = L.lgmlh_plan(*args, None, 0, C.byref(info))
    if rc:
        return rc, None, None
    buf = np.zeros(info.bytes, np.uint8)
    rc = L.lgmlh_plan(*args, buf.ctypes.data, buf.nbytes, C.byref(info))
    return rc, info, buf


def arr(buf, off, n, dt):
    return buf[off:off + n * np.dtype(dt).itemsize].view(dt)


def test_plan_packs_like_fill_batch(hip):
    # Two interleaved sequences (blocks from the pool restatement), one
    # decode token and one 70-token chunk.
    p = kp.Pool(64, 64)
    a, b = kp.Seq(p), kp.Seq(p)
    for n in (50, 100, 150):
        kp.reserve(a, n)
        kp.reserve(b, n)
    kp.reserve(a, 151)
    kp.reserve(b, 220)
    bt = np.full((2, 4), -1, np.int32)
    bt[0, :len(a.blocks)] = a.blocks
    bt[1, :len(b.blocks)] = b.blocks
    ids = np.arange(71, dtype=np.int32) + 7
    rc, info, buf = plan(hip, [1, 70], [150, 150], bt, ids, 32, 8, 64, bps=2)
    assert rc == 0 and info.n_tokens == 71 and info.n_seq == 2
    assert list(arr(buf, info.off_ids, 71, np.int32)) == list(ids)
    assert list(arr(buf, info.off_pos, 71, np.int32)) == [150] + list(range(150, 220))
    want = kp.seq_cells(a.blocks, 64, 150, 1) + kp.seq_cells(b.blocks, 64, 150, 70)
    assert list(arr(buf, info.off_cells, 71, np.int64)) == want
    assert list(arr(buf, info.off_logit_rows, 2, np.int32)) == [0, 70]
    assert list(arr(buf, info.off_seq_off, 3, np.int32)) == [0, 1, 71]
    items = arr(buf, info.off_items, 4 * info.n_items, np.int32).reshape(-1, 4)
    # every (token group, block) pair up to the group's last position is covered once
    seen = {}
    groups = {}
    for s, tok0, nt, blk in items:
        lo, hi = blk & 0xffff, blk >> 16
        groups.setdefault((int(s), int(tok0)), set()).add(int(nt) >> 5)
        assert 1 <= (nt & 31) <= 16 // 4
        key = (int(s), int(tok0))
        seen.setdefault(key, []).append((lo, hi))
        assert hi - lo <= 2
    for (s, tok0), runs in seen.items():
        runs.sort()
        assert runs[0][0] == 0 and all(runs[i][1] == runs[i + 1][0] for i in range(len(runs) - 1))
    assert info.n_merge == sum(1 for r in seen.values() if len(r) > 1)
    # one merge group per split token group (numbered from 1), 0 for one split;
    # its runs are `stride` items apart, in order
    mg = arr(buf, info.off_merge, 4 * info.n_merge, np.int32).reshape(-1, 4)
    for key, runs in seen.items():
        (g,) = groups[key]
        if len(runs) == 1:
            assert g == 0
        else:
            first, ns, tok0, f = mg[g - 1]
            assert ns == len(runs) and tok0 == key[1]
            stride = f >> 8
            got = [(items[first + j * stride][3] & 0xffff, items[first + j * stride][3] >> 16)
                   for j in range(ns)]
            assert all(items[first + j * stride][1] == tok0 for j in range(ns))
            assert got == sorted(runs)
    # the decode token's items come first (on their own); the chunk's 18
    # groups of 4 tokens come in shared sets of 8, 8, 2 with the runs of
    # each set's last token
    assert info.n_single == len(seen[(0, 0)])
    assert all(items[i][0] == 0 for i in range(info.n_single))
    sh = arr(buf, info.off_shared, 2 * info.n_shared, np.int32).reshape(-1, 2)
    covered = []
    for first, n in sh:
        assert 1 <= n <= 8
        blk = {int(items[first + m][3]) for m in range(n)}
        assert len(blk) == 1 and all(items[first + m][0] == 1 for m in range(n))
        assert [items[first + m][1] for m in range(n)] == [items[first][1] + 4 * m
                                                          for m in range(n)]
        covered += range(first, first + n)
    assert sorted(covered) == list(range(info.n_single, info.n_items))
    for (s, tok0), runs in seen.items():
        if s == 1:
            set0 = 1 + ((tok0 - 1) // 32) * 32
            last = min(set0 + 32, 71) - 1  # the set's last token
            assert max(hi for _, hi in runs) == (150 + last - 1) // 64 + 1


def test_plan_order_starts_the_longest_runs_first(hip):
    """The items on their own come in `order` by run length, longest first,
    ties by index: a permutation of [0, n_single). Shared-run items are not
    in it."""
    rng = np.random.default_rng(7)
    seq_n = [1] * 40 + [37]
    npast = list(rng.integers(0, 64 * 30, size=40)) + [500]
    nb = [(p + n + 63) // 64 for p, n in zip(npast, seq_n)]
    bt = np.full((len(seq_n), max(nb)), -1, np.int32)
    nxt = 0
    for s, k in enumerate(nb):
        bt[s, :k] = np.arange(nxt, nxt + k)
        nxt += k
    for bps in (0, 5, 12):
        rc, info, buf = plan(hip, seq_n, npast, bt, np.zeros(sum(seq_n), np.int32), 32, 8, nxt,
                             bps=bps)
        assert rc == 0
        items = arr(buf, info.off_items, 4 * info.n_items, np.int32).reshape(-1, 4)
        order = list(arr(buf, info.off_order, info.n_single, np.int32))
        assert sorted(order) == list(range(info.n_single))
        length = lambda i: (int(items[i][3]) >> 16) - (int(items[i][3]) & 0xffff)
        want = sorted(range(info.n_single), key=lambda i: (-length(i), i))
        assert order == want
        assert info.n_single < info.n_items  # the chunk's shared runs stay out
        assert info.off_order >= info.off_shared + 8 * info.n_shared
        assert info.bytes >= info.off_order + 4 * info.n_single


def test_plan_errors(hip):
    bt = np.array([[3, -1]], np.int32)
    rc, _, _ = plan(hip, [1], [64], bt, [0], 4, 2, 16)  # position 64 needs block table[1]
    assert rc == hip.ERANGE
    rc, _, _ = plan(hip, [1], [0], np.array([[16]], np.int32), [0], 4, 2, 16)  # block 16 >= pool
    assert rc == hip.ERANGE
    rc, _, _ = plan(hip, [1], [0], np.array([[1]], np.int32), [0], 6, 4, 16)  # H % Hkv
    assert rc == hip.EINVAL
    assert "plan" in hip.last_error()


def plan_ring(hip, seq_n, npast, ring_tab, window, ids, H, Hkv, pool_blocks, bps=0):
    L = hip.lib()
    info = hip.PlanInfo()
    keep = [np.ascontiguousarray(seq_n, np.int32), np.ascontiguousarray(npast, np.int32),
            np.ascontiguousarray(ring_tab, np.int32), np.ascontiguousarray(ids, np.int32)]
    args = (len(seq_n), keep[0].ctypes.data, keep[1].ctypes.data, keep[2].ctypes.data,
            keep[2].shape[1], pool_blocks, window, keep[3].ctypes.data, H, Hkv, bps)
    rc = L.lgmlh_plan_ring(*args, None, 0, C.byref(info))
    if rc:
        return rc, None, None
    buf = np.zeros(info.bytes, np.uint8)
    rc = L.lgmlh_plan_ring(*args, buf.ctypes.data, buf.nbytes, C.byref(info))
    return rc, info, buf


def test_ring_plan_maps_positions_into_the_rings(hip):
    """lgmlh_plan_ring: position p of sequence s goes to ring_tab[s, (p / 64)
    % R] * 64 + p % 64 (rows_swa = p % ring, transformer.lua:2469-2476), and
    each query group's runs cover the logical blocks from its window's start
    to its last position exactly once."""
    W, R = 100, 3  # 192 ring cells: a pass of up to 93 tokens
    ring_tab = np.array([[7, 2, 5], [0, 9, 4], [1, 3, 8]], np.int32)
    seq_n, npast = [1, 40, 93], [1000, 37, 0]
    ids = np.arange(sum(seq_n), dtype=np.int32)
    rc, info, buf = plan_ring(hip, seq_n, npast, ring_tab, W, ids, 8, 4, 10, bps=1)
    assert rc == 0 and info.window == W and info.ring == R and info.max_blocks == R
    cells = arr(buf, info.off_cells, info.n_tokens, np.int64)
    t = 0
    for s, (n, p0) in enumerate(zip(seq_n, npast)):
        for j in range(n):
            p = p0 + j
            assert cells[t] == ring_tab[s, (p // 64) % R] * 64 + p % 64
            t += 1
    assert list(arr(buf, info.off_block_tab, 9, np.int32)) == list(ring_tab.reshape(-1))
    items = arr(buf, info.off_items, 4 * info.n_items, np.int32).reshape(-1, 4)
    runs = {}
    for s, tok0, nt, blk in items:
        runs.setdefault((int(s), int(tok0), int(nt) & 31), []).append((blk & 0xffff, blk >> 16))
    offs = np.cumsum([0] + seq_n)
    for (s, tok0, nt), rr in runs.items():
        rr.sort()
        pf = npast[s] + tok0 - offs[s]
        pl = pf + nt - 1
        assert rr[0][0] == max(0, pf - W + 1) // 64 and rr[-1][1] == pl // 64 + 1
        assert all(rr[i][1] == rr[i + 1][0] for i in range(len(rr) - 1))
        lens = [hi - lo for lo, hi in rr]
        assert max(lens) - min(lens) <= 1 and max(lens) <= 1  # balanced runs, at most bps
    # every token is in exactly one group
    assert sorted(t0 + k for (_, t0, nt) in runs for k in range(nt)) == list(range(sum(seq_n)))
    # ring plans have every item on its own, started longest run first
    assert info.n_single == info.n_items and info.n_shared == 0
    rc, info, buf = plan_ring(hip, seq_n, npast, ring_tab, W, ids, 8, 4, 10, bps=2)
    assert rc == 0
    items = arr(buf, info.off_items, 4 * info.n_items, np.int32).reshape(-1, 4)
    order = list(arr(buf, info.off_order, info.n_single, np.int32))
    length = lambda i: (int(items[i][3]) >> 16) - (int(items[i][3]) & 0xffff)
    assert order == sorted(range(info.n_single), key=lambda i: (-length(i), i))
    assert len({length(i) for i in range(info.n_single)}) > 1


def test_ring_plan_errors(hip):
    tab = np.array([[0, 1]], np.int32)
    # 2 blocks = 128 cells: window 100 leaves room for 29 tokens in one pass
    assert plan_ring(hip, [29], [500], tab, 100, np.zeros(29), 4, 2, 4)[0] == 0
    assert plan_ring(hip, [30], [500], tab, 100, np.zeros(30), 4, 2, 4)[0] == hip.ERANGE
    assert "ring" in hip.last_error()
    # ring blocks outside the pool
    assert plan_ring(hip, [1], [70], np.array([[0, 4]], np.int32), 100, [0], 4, 2, 4)[0] == \
        hip.ERANGE
    # no window
    assert plan_ring(hip, [1], [0], tab, 0, [0], 4, 2, 4)[0] == hip.EINVAL


def test_flash_attn_checks_arguments(hip):
    """Host-side argument checks of lgmlh_flash_attn (no GPU work)."""
    L = hip.lib()
    d = C.c_void_p(256)
    # head size not a multiple of 8; max_bias without a mask
    assert L.lgmlh_flash_attn(d, 4, 1, 20, d, d, 2, 8, 20, 160, 20, 160, None, 0, 0, 1.0, 0.0,
                              0.0, d, None) == hip.EINVAL
    assert L.lgmlh_flash_attn(d, 4, 1, 16, d, d, 2, 8, 16, 128, 16, 128, None, 0, 0, 1.0, 8.0,
                              0.0, d, None) == hip.EINVAL
    assert "max_bias" in hip.last_error()
    # mask planes must divide the heads
    assert L.lgmlh_flash_attn(d, 4, 1, 16, d, d, 2, 8, 16, 128, 16, 128, d, 3, 1, 1.0, 0.0,
                              0.0, d, None) == hip.EINVAL
