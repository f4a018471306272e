"""Pins the oracle's routed experts (orc_moe_route, orc_mul_mat_id).

The whole MoE layer is pinned end to end by the reference's llama.cpp rows
of the tiny qwen3moe (tests/test_oracle_golden.py, REF.qwen3moe of
test/test_qwen_moe.lua:242-257). Here, each piece is checked on its own
against a brute-force numpy statement of the reference semantics
(soft_max / sigmoid, argsort_top_k, get_rows, the norm_topk division and
clamp, expert_scale: transformer.lua:1998-2008; mul_mat_id row (t, j) =
w[ids[t, j]] x[t, j % U]: src/ops_nn.c:322-362). The golden rows also
reject planted mistakes in the MoE hyperparameters.
"""
import numpy as np
import pytest

from oracle import core, models


def np_route(lg, k, gating=1, norm_topk=True, scale=1.0):
    lg = np.asarray(lg, np.float64)
    if gating == 1:
        e = np.exp(lg - lg.max(axis=1, keepdims=True))
        p = e / e.sum(axis=1, keepdims=True)
    else:
        p = 1.0 / (1.0 + np.exp(-lg))
    # largest first, ties to the smaller index: a stable sort of -logits
    ids = np.argsort(-lg, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p.astype(np.float32), ids, axis=1).astype(np.float64)
    if norm_topk:
        s = np.maximum(w.sum(axis=1, keepdims=True).astype(np.float32), np.float32(6.103515625e-5))
        w = w / s
    return ids, (w * scale).astype(np.float32)


@pytest.mark.parametrize("ne,k,gating,norm,scale", [
    (128, 8, 1, True, 1.0), (8, 2, 1, True, 1.0), (60, 4, 1, False, 1.0), (128, 8, 2, True, 2.5),
    (512, 16, 1, True, 1.0), (16, 16, 2, False, 1.0), (3, 1, 1, True, 1.0)])
def test_route_matches_numpy(oracle_lib, ne, k, gating, norm, scale):
    rng = np.random.default_rng(ne * 31 + k)
    lg = rng.standard_normal((37, ne)).astype(np.float32) * 2
    lg[0, :] = 0.5                      # all tied: ids 0..k-1 in order
    lg[1, ::2] = lg[1, 1::2][:len(lg[1, ::2])]  # pairs of equal logits
    ids, w = core.moe_route(lg, k, gating, norm, scale)
    ri, rw = np_route(lg, k, gating, norm, scale)
    assert np.array_equal(ids, ri)
    assert list(ids[0]) == list(range(k))
    np.testing.assert_allclose(w, rw, rtol=1e-6, atol=0)
    if norm and scale == 1.0:
        np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-5)


def test_route_norm_clamp(oracle_lib):
    """Sigmoid gates far below 6.1e-5 in sum: divided by the clamp, not the sum."""
    lg = np.full((2, 16), -40.0, np.float32)
    lg[1, 3] = -30.0
    ids, w = core.moe_route(lg, 4, core.GATING_SIGMOID, True)
    p = 1.0 / (1.0 + np.exp(40.0))
    np.testing.assert_allclose(w[0], np.float32(p) / np.float32(6.103515625e-5), rtol=1e-6)
    assert ids[1, 0] == 3 and list(ids[0]) == [0, 1, 2, 3]


@pytest.mark.parametrize("ty", [core.F32, core.Q4_K, core.Q6_K, core.Q8_0])
@pytest.mark.parametrize("U", [1, 4])
def test_mul_mat_id_matches_per_pick_products(oracle_lib, ty, U):
    rng = np.random.default_rng(ty * 10 + U)
    NE, M, K, T, k = 6, 32, 256, 9, 4
    wf = rng.standard_normal((NE * M, K)).astype(np.float32) * 0.1
    w = wf if ty == core.F32 else core.quantize(ty, wf)
    deq = wf if ty == core.F32 else core.dequantize(ty, w, K)
    x = rng.standard_normal((T, U, K)).astype(np.float32)
    ids = rng.integers(0, NE, size=(T, k)).astype(np.int32)
    ids[0] = [2, 2, 2, 2]  # one expert picked several times by a token
    y = core.mul_mat_id(ty, w, NE, M, K, x, ids)
    for t in range(T):
        for j in range(k):
            e = ids[t, j]
            want = deq[e * M:(e + 1) * M].astype(np.float64) @ x[t, j % U].astype(np.float64)
            np.testing.assert_allclose(y[t, j], want, rtol=1e-5, atol=1e-5)


def test_mul_mat_id_rejects_bad_ids(oracle_lib):
    w = np.zeros((4 * 8, 32), np.float32)
    x = np.zeros((2, 1, 32), np.float32)
    with pytest.raises(ValueError):
        core.mul_mat_id(core.F32, w, 4, 8, 32, x, np.array([[0, 4], [1, 2]], np.int32))


@pytest.mark.parametrize("mod", [dict(norm_topk=False), dict(gating=core.GATING_SIGMOID),
                                 dict(n_used=1), dict(expert_scale=0.9)])
def test_planted_moe_mistakes_fail_the_golden_rows(oracle_lib, monkeypatch, mod):
    """A changed routing rule moves the tiny qwen3moe's logits far past the
    golden tolerance: the rows pin each of these hyperparameters."""
    from tests import test_oracle_golden as tg
    orig = models.ref_tiny

    def patched(arch):
        hp, w = orig(arch)
        hp.update(mod)
        return hp, w

    monkeypatch.setattr(models, "ref_tiny", patched)
    d, ref, rows = tg.run_rows("qwen3moe")
    idx = [i - 1 for i in d["idx_1based"]]
    err = max(max(abs(float(g[i]) - v) for i, v in zip(idx, r["v"])) for r, g in zip(ref, rows))
    assert err > 20 * d["tol"], err
