"""Pins the CPU oracle against the reference's llama.cpp golden rows.

REF.llama / REF.qwen3 / REF.qwen3moe (test/test_qwen_moe.lua:202-273, fixture
tests/golden/ref_logits.json): logits at 8 vocab indices plus the argmax of
14 rows (two prompt batches, then 6 greedy decode ids), TOL 2e-3 absolute
max error and argmax on every row (test_qwen_moe.lua:378-400,1019-1023).
"""
import json
import os

import numpy as np
import pytest

from oracle import core, models

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_logits.json")


def run_rows(arch, block_tab=None, cap=64, block=64, model=None):
    """The golden passes of arch on the tiny model (or on model = (hp, w))."""
    hp, w = model if model is not None else models.ref_tiny(arch)
    m = core.OracleModel(hp, w)
    d = json.load(open(GOLDEN))
    ref = d["rows"][arch]
    L, row = hp["n_layer"], hp["n_head_kv"] * hp["head_dim"]
    kp = [np.zeros((cap, row), np.uint16) for _ in range(L)]
    vp = [np.zeros((cap, row), np.uint16) for _ in range(L)]
    if block_tab is None:
        block_tab = list(range(cap // block))
    nb = sum(len(b) for b in d["batches"])
    passes = d["batches"] + [[r["id"]] for r in ref[nb:]]
    rows, npast = [], 0
    for ids in passes:
        b = core.BatchDesc([len(ids)], [npast], [block_tab], block, ids, list(range(len(ids))))
        rows.extend(m.forward(kp, vp, b))
        npast += len(ids)
    return d, ref, rows


@pytest.mark.parametrize("arch", ["llama", "qwen3", "qwen3moe"])
def test_oracle_matches_llama_cpp_rows(oracle_lib, arch):
    d, ref, rows = run_rows(arch)
    idx = [i - 1 for i in d["idx_1based"]]
    assert len(rows) == len(ref) == 14
    err = 0.0
    for r, got in zip(ref, rows):
        err = max(err, max(abs(float(got[i]) - v) for i, v in zip(idx, r["v"])))
        assert core.argmax(got) == r["best"], "argmax differs from llama.cpp"
    assert err < d["tol"], "max logit error %.3g" % err


def test_oracle_pool_layout_does_not_change_rows(oracle_lib):
    """Scattered blocks (cells out of position order) give the same rows as
    the identity layout: the mask semantics of fill_blocks hide cell ids."""
    _, _, a = run_rows("qwen3", block_tab=[0, 1], cap=128, block=64)
    _, _, b = run_rows("qwen3", block_tab=[3, 1, 0, 2], cap=256, block=16)
    assert np.array_equal(np.array(a), np.array(b))


def test_greedy_stream_follows_reference(oracle_lib):
    """generate.greedy semantics (lua/lgml/generate.lua:19-34): each decode id
    of the golden rows is the argmax of the row before it."""
    d, ref, rows = run_rows("llama")
    nb = sum(len(b) for b in d["batches"])
    for i in range(nb, len(ref)):
        assert ref[i]["id"] == core.argmax(rows[i - 1])


GOLDEN_G4 = os.path.join(os.path.dirname(__file__), "golden", "ref_gemma4.json")


def run_gemma4_rows(block=64, ring_blocks=1, model=None):
    """The tiny gemma4 rows: the two prompt batches, then the greedy ids.
    Global layers use a paged pool; the sliding layer a ring of
    ring_blocks blocks of `block` cells (it must hold window - 1 + 20)."""
    hp, w = model if model is not None else models.ref_tiny_gemma4()
    m = core.OracleModel(hp, w)
    d = json.load(open(GOLDEN_G4))
    ref = d["rows"]["dense"]
    cap = 256
    kp = [np.zeros((cap, L["n_head_kv"] * L["head_dim"]), np.uint16) for L in w["layers"]]
    vp = [np.zeros((cap, L["n_head_kv"] * L["head_dim"]), np.uint16) for L in w["layers"]]
    block_tab = list(range(64 // block))            # positions 0..63: cells 0..63
    ring_tab = [cap // block - 1 - i for i in range(ring_blocks)]  # the ring from the top
    nb = sum(len(b) for b in d["batches"])
    passes = d["batches"] + [[r["id"]] for r in ref[nb:]]
    rows, npast = [], 0
    for ids in passes:
        b = core.BatchDesc([len(ids)], [npast], [block_tab], block, ids, list(range(len(ids))),
                           ring_tab=[ring_tab])
        rows.extend(m.forward(kp, vp, b))
        npast += len(ids)
    return d, ref, rows


def test_oracle_matches_gemma4_rows(oracle_lib):
    """REF.dense of test/test_gemma4.lua:192-224: a sliding layer (window 6,
    a 20-token prompt longer than it) and a global one; TOL 2e-3 + argmax."""
    d, ref, rows = run_gemma4_rows()
    idx = [i - 1 for i in d["idx_1based"]]
    assert len(rows) == len(ref) == 31
    err = 0.0
    for r, got in zip(ref, rows):
        err = max(err, max(abs(float(got[i]) - v) for i, v in zip(idx, r["v"])))
        assert core.argmax(got) == r["best"], "argmax differs from llama.cpp"
    assert err < d["tol"], "max logit error %.3g" % err


def test_oracle_ring_wraps_give_the_same_rows(oracle_lib):
    """A ring of 7 blocks of 4 cells (28 >= window - 1 + 20) wraps at
    position 28; the rows equal those of an unwrapped ring bit for bit
    (rows_swa = p % ring, transformer.lua:2469-2476)."""
    _, _, a = run_gemma4_rows(block=64, ring_blocks=1)
    _, _, b = run_gemma4_rows(block=4, ring_blocks=7)
    assert np.array_equal(np.array(a), np.array(b))
