"""GPU parity of the sliding-window ring path and the gemma layers.

Ring attention (lgmlh_plan_ring + lgmlh_paged_attention) against the
oracle's orc_paged_attention_swa (pinned by a brute-force window mask and
the tiny gemma4 rows, tests/test_oracle_gemma.py) at head sizes 64 / 128 /
256, decode and prefill groups, windows that wrap the ring, split and
unsplit runs: within 1e-4 max relative error (the bar is 2e-3). GeGLU and
the logit softcap against their closed forms. Whole C4-shaped passes
(full width: 2560, 8 / 4 heads of 256, Q8_0, vocab 262144, tied output;
reduced depth, a 100-token window so that a few hundred tokens wrap the
rings) against the oracle: logits within 2e-3, greedy tokens identical.
A sequence alone and in a batch gives the same bits through the rings.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import core, models
from tests.gpu_util import Schedule, lcg_ints, oracle_pools, rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def L():
    from lgml_amd import hip
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return hip.lib()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def st():
    return torch.cuda.current_stream().cuda_stream


def ring_case(H, Hkv, D, seqs, R, seed, n_blocks):
    """Random q and pools; sequence s owns ring blocks perm[s R:(s + 1) R]."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_blocks).astype(np.int32)
    ring_tab = perm[:len(seqs) * R].reshape(len(seqs), R)
    N = sum(n for n, _ in seqs)
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    cells = n_blocks * 64
    kpool = core.f32_to_f16_bits(rng.standard_normal((cells, Hkv * D)).astype(np.float32))
    vpool = core.f32_to_f16_bits(rng.standard_normal((cells, Hkv * D)).astype(np.float32))
    return q, kpool, vpool, ring_tab


def gpu_ring_attention(L, q, kpool_rows, vpool_rows, H, Hkv, D, seqs, ring_tab, window, scale,
                       bps=0):
    from lgml_amd import hip, runtime
    n_cells = kpool_rows.shape[0]
    seq_n = [n for n, _ in seqs]
    npast = [p for _, p in seqs]
    plan = runtime.Plan(seq_n, npast, ring_tab, np.zeros(sum(seq_n), np.int32), H, Hkv,
                        n_cells // 64, bps, ring_tab=ring_tab, window=window)
    assert plan.info.ring == ring_tab.shape[1] and plan.info.window == window
    kb = L.lgmlh_kv_layer_bytes(n_cells, Hkv, D)
    kp = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    vp = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    allc = np.arange(n_cells, dtype=np.int64)
    kf = dev(core.f16_bits_to_f32(kpool_rows))
    vf = dev(core.f16_bits_to_f32(vpool_rows))
    cd = dev(allc)
    hip.check(L.lgmlh_kv_store(kp.data_ptr(), vp.data_ptr(), n_cells, Hkv, D, kf.data_ptr(),
                               vf.data_ptr(), cd.data_ptr(), allc.ctypes.data, n_cells, st()))
    out = torch.full(q.shape, float("nan"), dtype=torch.float32, device="cuda")
    wsb = L.lgmlh_attention_workspace(C.byref(plan.info), D)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    qd = dev(q)
    hip.check(L.lgmlh_paged_attention(qd.data_ptr(), H, Hkv, D, scale, kp.data_ptr(),
                                      vp.data_ptr(), C.byref(plan.ub), out.data_ptr(),
                                      ws.data_ptr(), wsb, st()))
    return out.cpu().numpy()


# (window, ring blocks, sequences (n, npast)): the C4 window with its ring
# for 512-token passes, and a 100-token window in a 3-block ring whose
# windows straddle block and ring boundaries.
RING_CASES = [
    (1024, 24, [(1, 0), (1, 63), (1, 1023), (1, 1024), (1, 5000), (37, 2000), (512, 3000),
                (16, 1530), (1, 16383)]),
    (100, 3, [(1, 1000), (40, 37), (93, 0), (16, 150), (1, 99), (1, 100), (5, 190)]),
]


@pytest.mark.parametrize("H,Hkv,D", [(8, 4, 256), (32, 8, 128), (4, 2, 64), (4, 2, 16)])
@pytest.mark.parametrize("case", range(len(RING_CASES)))
def test_ring_attention_matches_oracle(L, H, Hkv, D, case):
    window, R, seqs = RING_CASES[case]
    n_blocks = len(seqs) * R + 5
    q, kpool, vpool, ring_tab = ring_case(H, Hkv, D, seqs, R, seed=D + case, n_blocks=n_blocks)
    scale = 1.0 if D == 256 else 1.0 / np.sqrt(D)
    b = core.BatchDesc([n for n, _ in seqs], [p for _, p in seqs], np.zeros((len(seqs), 1)), 64,
                       np.zeros(len(q), np.int32), [], ring_tab=ring_tab)
    want = core.paged_attention_swa(q, kpool, vpool, H, Hkv, D, scale, window, b)
    for bps in (0, 1, 3):
        print("ring attention H=%d Hkv=%d D=%d window=%d bps=%d" % (H, Hkv, D, window, bps),
              flush=True)
        got = gpu_ring_attention(L, q, kpool, vpool, H, Hkv, D, seqs, ring_tab, window, scale,
                                 bps)
        assert np.isfinite(got).all()
        e = rel_err(got.reshape(len(q) * H, D), want.reshape(len(q) * H, D))
        assert e < 1e-4, (bps, e)


def test_ring_attention_alone_equals_batched(L):
    H, Hkv, D, window, R = 8, 4, 256, 1024, 24
    seqs = [(1, 100), (1, 7000), (9, 1500), (1, 5)]
    q, kpool, vpool, ring_tab = ring_case(H, Hkv, D, seqs, R, seed=11, n_blocks=4 * R)
    got = gpu_ring_attention(L, q, kpool, vpool, H, Hkv, D, seqs, ring_tab, window, 1.0, 2)
    off = 0
    for i, (n, p) in enumerate(seqs):
        alone = gpu_ring_attention(L, q[off:off + n], kpool, vpool, H, Hkv, D, [(n, p)],
                                   ring_tab[i:i + 1], window, 1.0, 2)
        assert np.array_equal(alone.view(np.uint32), got[off:off + n].view(np.uint32)), i
        off += n


def test_geglu_and_softcap_closed_forms(L):
    from lgml_amd import hip
    rng = np.random.default_rng(7)
    n, F = 5, 1000
    gu = (rng.standard_normal((n, 2 * F)) * 3).astype(np.float32)
    gd = dev(gu)
    out = torch.empty((n, F), dtype=torch.float32, device="cuda")
    hip.check(L.lgmlh_geglu(gd.data_ptr(), n, F, out.data_ptr(), hip.F32, st()))
    g, u = gu[:, :F].astype(np.float64), gu[:, F:].astype(np.float64)
    # ggml's tanh gelu: 0.5 x (1 + tanh(sqrt(2 / pi) x (1 + 0.044715 x^2)))
    want = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * g * (1 + 0.044715 * g * g))) * u
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=2e-6, atol=1e-6)
    x = (rng.standard_normal(4097) * 40).astype(np.float32)
    xd = dev(x)
    hip.check(L.lgmlh_softcap(xd.data_ptr(), len(x), 30.0, st()))
    np.testing.assert_allclose(xd.cpu().numpy(), 30.0 * np.tanh(x.astype(np.float64) / 30.0),
                               rtol=2e-6, atol=2e-6)


def c4_small(n_layer, swa_period, seed, n_swa=100):
    """The C4 shape at full width, reduced depth and window."""
    shape = dict(models.SHAPES["c4"], n_layer=n_layer, swa_period=swa_period, n_swa=n_swa)
    return models.build(shape, seed=seed, init="normal")


def run_gemma(hp, w, n_cells, prompts, steps, ubatch=512):
    """Prefill every prompt in one pass (each at most ubatch tokens), then
    greedy decode steps batched over every sequence, on the GPU and the
    oracle; both continue on the oracle's token. Sequence s owns ring
    blocks s R .. s R + R - 1."""
    from lgml_amd import runtime
    assert max(len(p) for p in prompts) <= ubatch
    R = (hp["n_swa"] - 1 + min(ubatch, max(len(p) for p in prompts)) + 63) // 64
    # the oracle keeps every layer in n_cells cells: the rings must fit
    assert len(prompts) * R * 64 <= n_cells
    gm = runtime.DeviceModel(hp, w, n_cells, ring_cells=len(prompts) * R * 64)
    om = core.OracleModel(hp, w)
    kp, vp = oracle_pools(hp, n_cells)
    sch = Schedule(n_cells // 64, len(prompts))
    ring_all = np.arange(len(prompts) * R, dtype=np.int32).reshape(len(prompts), R)
    which = list(range(len(prompts)))
    npast = [0] * len(prompts)
    cur = [list(p) for p in prompts]
    errs, same = [], True
    for step in range(steps + 1):
        for s in which:
            sch.grow(s, npast[s] + len(cur[s]))
        bt = sch.table(which)
        seq_n = [len(cur[s]) for s in which]
        ids = np.concatenate([np.array(cur[s], np.int32) for s in which])
        rt = ring_all[which]
        print("gemma pass %d: seq_n %s npast %s" % (step, seq_n, [npast[s] for s in which]),
              flush=True)
        plan = gm.plan(seq_n, [npast[s] for s in which], bt, ids, ring_tab=rt)
        lg = gm.forward(plan).cpu().numpy()
        b = core.BatchDesc(seq_n, [npast[s] for s in which], bt, 64, ids, plan.logit_rows,
                           ring_tab=rt)
        lo = om.forward(kp, vp, b)
        errs.append(rel_err(lg, lo))
        for i, s in enumerate(which):
            same = same and int(np.argmax(lg[i])) == core.argmax(lo[i])
            npast[s] += len(cur[s])
            cur[s] = [core.argmax(lo[i])]
    return errs, same


def test_c4_shape_reduced_depth_windows_wrap():
    """5 sliding layers and 1 global (the C4 pattern), prompts of 5..260
    tokens (the 100-token window wraps the 6-block rings), 8 greedy steps."""
    hp, w = c4_small(6, 6, seed=4)
    assert [L.get("swa") for L in w["layers"]] == [1, 1, 1, 1, 1, 0]
    assert "wv" not in w["layers"][5] and w["output"] is w["tok_embd"]
    lens = [5, 37, 150, 260]
    prompts = [lcg_ints(2000 + i, n, 0, hp["n_vocab"]) for i, n in enumerate(lens)]
    errs, same = run_gemma(hp, w, 2048, prompts, 8)
    assert max(errs) < 2e-3, errs
    assert same


def test_c4_batched_pass_equals_lone_pass():
    from lgml_amd import runtime
    hp, w = c4_small(2, 2, seed=8)
    R = 6
    gm = runtime.DeviceModel(hp, w, 2048, ring_cells=3 * R * 64)
    prompts = [lcg_ints(300 + i, n, 0, hp["n_vocab"]) for i, n in enumerate([9, 140, 3])]
    ids = np.concatenate([np.array(p, np.int32) for p in prompts])
    bt = np.array([[0, 1, 2], [3, 4, 5], [6, 7, 8]], np.int32)
    rt = np.arange(3 * R, dtype=np.int32).reshape(3, R)
    lb = gm.forward(gm.plan([9, 140, 3], [0, 0, 0], bt, ids, ring_tab=rt)).cpu().numpy()
    for s, p in enumerate(prompts):
        la = gm.forward(gm.plan([len(p)], [0], bt[s:s + 1], np.array(p, np.int32),
                                ring_tab=rt[s:s + 1])).cpu().numpy()
        assert np.array_equal(la.view(np.uint32), lb[s:s + 1].view(np.uint32)), s
