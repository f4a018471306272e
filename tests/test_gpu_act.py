"""GPU parity of ggml's CPU arithmetic for quantized weights (LGMLH_ACT_GGML)
against the oracle's act_quant mode, through the C ABI.

Bit-exact: the activation blocks (Q8_K q / d / bsums, Q8_0 q / d) of the
same f32 rows. Tolerance: products within 1e-5 of orc_mul_mat_q8 (the block
dots are exact integers on both sides; only the f32 scale products and the
order of the block sums differ). Whole passes: at the oracle's own
conditioning in this arithmetic (faithful_run), since a one-ulp change
moves these models' logits by 1-10% under X quantization. Batch
invariance: a row alone and in a batch give the same bits.
"""
import numpy as np
import pytest

from oracle import core, models
from tests.gpu_util import lcg_ints, rel_err
from tests.test_gpu_kernels import L, dev, st  # noqa: F401 (fixture)
from tests.test_gpu_model import run_both

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def act_rows(K, n, seed):
    """Rows with the cases the quantizers must get right: an all-zero
    block, a block whose largest |x| appears twice with both signs, a
    negative max, ties at iscale = 1, tiny and large scales."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, K)) * rng.uniform(1e-3, 30, (n, 1))).astype(np.float32)
    x[0, :256] = 0
    x[1, 3], x[1, 10] = -50.0, 50.0
    x[2, :256] = np.round(rng.uniform(-126, 126, 256) * 2) / 2  # halves: ties
    x[2, 5] = -127.0
    if K >= 512:
        x[3, 256:288] = 0
        x[3, 300] = 127.0
        x[3, 301:305] = [2.5, -2.5, 0.5, 1.5]
    return x


@pytest.mark.parametrize("ty", [core.Q4_K, core.Q8_0])
def test_quantize_act_bit_exact(L, ty):
    from lgml_amd import hip
    K, n = 1024, 37
    x = act_rows(K, n, 1)
    qd = torch.empty((n, K), dtype=torch.int8, device="cuda")
    if ty == core.Q8_0:
        dd = torch.empty((n, K // 32), dtype=torch.int16, device="cuda")
        bs = None
    else:
        dd = torch.empty((n, K // 256), dtype=torch.float32, device="cuda")
        bs = torch.empty((n, K // 16), dtype=torch.int16, device="cuda")
    xd = dev(x)
    hip.check(L.lgmlh_quantize_act(ty, xd.data_ptr(), n, K, qd.data_ptr(), dd.data_ptr(),
                                   bs.data_ptr() if bs is not None else None, st()))
    if ty == core.Q8_0:
        q, d = core.quantize_q8_0_act(x)
        assert np.array_equal(dd.cpu().numpy().view(np.uint16), d)
    else:
        q, d, b = core.quantize_q8_K(x)
        assert np.array_equal(dd.cpu().numpy().view(np.uint32), d.view(np.uint32))
        assert np.array_equal(bs.cpu().numpy(), b)
    assert np.array_equal(qd.cpu().numpy(), q)


def run_mul_mat_ggml(L, ty, w, M, K, x):
    from lgml_amd import hip
    N = x.shape[0]
    nb = L.lgmlh_repacked_bytes(ty, M, K)
    rp = torch.empty(nb, dtype=torch.uint8, device="cuda")
    wd = dev(w)
    hip.check(L.lgmlh_repack(ty, M, K, wd.data_ptr(), rp.data_ptr(), st()))
    ws_n = L.lgmlh_mul_mat_workspace(ty, M, K, N)
    ws = torch.zeros(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty((N, M), dtype=torch.float32, device="cuda")
    xd = dev(x)
    hip.check(L.lgmlh_mul_mat_ggml(ty, rp.data_ptr(), M, K, xd.data_ptr(), hip.F32, N,
                                   y.data_ptr(), hip.EPI_NONE, None, ws.data_ptr(), ws_n, st()))
    return y.cpu().numpy()


# The shapes of test_gpu_kernels' product test: 16-, 32- and 64-column
# kernels, split and unsplit K, 4- and 8-wave workgroups; and (4096, 4096)
# at N = 4096, where a workgroup runs both splits of a pair.
@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K, core.Q8_0])
@pytest.mark.parametrize("MK", [(512, 1024), (256, 4096), (48, 768), (25600, 1024),
                                (51200, 256), (12800, 1024)])
def test_mul_mat_ggml_parity_and_batch_invariance(L, ty, MK):
    M, K = MK
    big = M * K > 4_000_000
    wf = core.fill_normal(M * K, 0, 0.02, 7).reshape(M, K)
    w = core.quantize(ty, wf)
    x = act_rows(K, 130, 8)
    ys = {}
    for N in ((17, 32, 64, 130) if big else (1, 3, 17, 32, 40, 64, 70, 130)):
        y = ys[N] = run_mul_mat_ggml(L, ty, w, M, K, x[:N])
        want = core.mul_mat_q8(ty, w, M, K, x[:N])
        assert rel_err(y, want) < 1e-5, (N, rel_err(y, want))
        if N in (32, 130):
            for j in ((0, 63, 64, 129) if N == 130 else (0, 16, 31)):
                alone = run_mul_mat_ggml(L, ty, w, M, K, x[j:j + 1])
                assert np.array_equal(alone[0].view(np.uint32), y[j].view(np.uint32)), j
    # every batch size (the decode kernels at N <= 64, the wide one above)
    # gives each row the same bits
    for N, y in ys.items():
        assert np.array_equal(y.view(np.uint32), ys[130][:N].view(np.uint32)), N


@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K])
def test_mul_mat_ggml_folded_pairs(L, ty):
    # N = 4096: 8192 workgroups of single splits or more (Q4_K 16384, Q6_K
    # 8192), so a workgroup runs both splits of a pair
    M, K, N = 4096, 4096, 4096
    w = core.quantize(ty, core.fill_normal(M * K, 0, 0.02, 17).reshape(M, K))
    x = core.fill_normal(N * K, 0, 1, 18).reshape(N, K)
    y = run_mul_mat_ggml(L, ty, w, M, K, x)
    y130 = run_mul_mat_ggml(L, ty, w, M, K, x[:130])
    assert np.array_equal(y[:130].view(np.uint32), y130.view(np.uint32))
    rows = [0, 65, 300, N - 1]
    want = core.mul_mat_q8(ty, w, M, K, x[rows])
    assert rel_err(y[rows], want) < 1e-5


def test_mul_mat_id_ggml(L):
    from lgml_amd import hip
    NE, M, K, T, U, nu = 16, 768, 2048, 40, 1, 8
    wf = core.fill_normal(NE * M * K, 0, 0.02, 21).reshape(NE * M, K)
    w = core.quantize(core.Q4_K, wf)
    x = core.fill_normal(T * K, 0, 1, 22).reshape(T, 1, K)
    rng = np.random.default_rng(3)
    ids = np.stack([rng.permutation(NE)[:nu] for _ in range(T)]).astype(np.int32)
    eb = L.lgmlh_repacked_bytes(core.Q4_K, M, K)
    rp = torch.empty(NE * eb, dtype=torch.uint8, device="cuda")
    for e in range(NE):
        src = dev(w[e * M:(e + 1) * M])
        hip.check(L.lgmlh_repack(core.Q4_K, M, K, src.data_ptr(), rp.data_ptr() + e * eb, st()))
    ws_n = L.lgmlh_mul_mat_id_workspace(core.Q4_K, NE, M, K, T, U, nu)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda")
    y = torch.empty((T, nu, M), dtype=torch.float32, device="cuda")
    xd, idd = dev(x), dev(ids)
    hip.check(L.lgmlh_mul_mat_id_ggml(core.Q4_K, rp.data_ptr(), NE, M, K, xd.data_ptr(), hip.F32,
                                      U, idd.data_ptr(), T, nu, y.data_ptr(), ws.data_ptr(), ws_n,
                                      st()))
    want = core.mul_mat_id(core.Q4_K, w, NE, M, K, x, ids, act_quant=True)
    assert rel_err(y.cpu().numpy().reshape(T * nu, M), want.reshape(T * nu, M)) < 1e-5


def _rms(a):
    return float(np.sqrt(np.mean(np.square(np.asarray(a, np.float64)))))


def faithful_run(hp, w, n_cells, prompts, steps):
    """Whole passes of the GPU in ggml arithmetic (G) beside three oracle
    runs, all fed the greedy ids of F: F the oracle in ggml arithmetic, E the
    oracle in exact arithmetic, P the oracle in ggml arithmetic with layer
    0's attn_norm one ulp up (x (1 + 2^-23)). ggml's arithmetic is not
    continuous in X (a q flips at a rounding boundary), and on these random
    models a one-ulp change moves the logits by 1-10% (test_oracle_act), so
    G is held to F's own conditioning rather than to 2e-3: per pass, |G - F|
    <= 2 |P - F| (as close as F is to itself one ulp away), and |G - E| >=
    |F - E| / 2 (G carries the quantization: an exact-arithmetic G would
    sit at |G - E| ~ 1e-4). Distances are rms over the logits, relative to
    rms(E)."""
    from lgml_amd import runtime
    from tests.gpu_util import Schedule, oracle_pools
    gm = runtime.DeviceModel(dict(hp, act_quant=True), w, n_cells)
    wp = dict(w, layers=[dict(L) for L in w["layers"]])
    a, t = w["layers"][0]["attn_norm"]
    wp["layers"][0]["attn_norm"] = ((a * np.float32(1 + 2**-23)).astype(np.float32), t)
    oms = {"F": core.OracleModel(dict(hp, act_quant=True), w),
           "E": core.OracleModel(dict(hp, act_quant=False), w),
           "P": core.OracleModel(dict(hp, act_quant=True), wp)}
    pools = {k: oracle_pools(hp, n_cells) for k in oms}
    sch = Schedule(n_cells // 64, len(prompts))
    which = list(range(len(prompts)))
    npast = [0] * len(prompts)
    cur = [list(p) for p in prompts]
    rows = []
    for step in range(steps + 1):
        for s in which:
            sch.grow(s, npast[s] + len(cur[s]))
        bt = sch.table(which)
        seq_n = [len(cur[s]) for s in which]
        ids = np.concatenate([np.array(cur[s], np.int32) for s in which])
        plan = gm.plan(seq_n, npast, bt, ids)
        lg = gm.forward(plan).cpu().numpy()
        b = core.BatchDesc(seq_n, npast, bt, 64, ids, plan.logit_rows)
        lo = {k: om.forward(*pools[k], b) for k, om in oms.items()}
        den = _rms(lo["E"])
        rows.append(dict(gf=_rms(lg - lo["F"]) / den, ge=_rms(lg - lo["E"]) / den,
                         fe=_rms(lo["F"] - lo["E"]) / den, pf=_rms(lo["P"] - lo["F"]) / den,
                         rel=rel_err(lg, lo["F"])))
        for i, s in enumerate(which):
            npast[s] += len(cur[s])
            cur[s] = [core.argmax(lo["F"][i])]
    for r in rows:
        print("G-F %.3g  P-F %.3g  G-E %.3g  F-E %.3g  (max rel G-F %.3g)" % (
            r["gf"], r["pf"], r["ge"], r["fe"], r["rel"]), flush=True)
    return rows


def check_faithful(rows):
    for r in rows:
        assert r["gf"] <= 2 * r["pf"], r
        assert r["ge"] >= 0.5 * r["fe"], r


def test_c2_shape_reduced_depth_ggml():
    hp, w = models.build("c2", seed=2, n_layer=2, init="normal")
    lens = [5, 70, 1, 130, 33, 64]
    prompts = [lcg_ints(2000 + i, n, 0, hp["n_vocab"]) for i, n in enumerate(lens)]
    check_faithful(faithful_run(hp, w, 4096, prompts, 4))


def test_c5_shape_reduced_depth_ggml():
    hp, w = models.build("c5", seed=5, n_layer=2, init="normal")
    lens = [9, 40, 3, 77]
    prompts = [lcg_ints(5000 + i, n, 0, hp["n_vocab"]) for i, n in enumerate(lens)]
    check_faithful(faithful_run(hp, w, 2048, prompts, 3))


def test_batched_pass_equals_lone_pass_ggml():
    from lgml_amd import runtime
    from tests.gpu_util import Schedule
    hp, w = models.build("c2", seed=3, n_layer=2, init="normal")
    hp = dict(hp, act_quant=True)
    gm_b = runtime.DeviceModel(hp, w, 2048)
    gm_a = runtime.DeviceModel(hp, w, 2048)
    prompts = [lcg_ints(3000 + i, n, 0, hp["n_vocab"]) for i, n in enumerate([9, 40, 3])]
    sch = Schedule(32, 3)
    for s, p in enumerate(prompts):
        sch.grow(s, len(p) + 1)
    bt = sch.table([0, 1, 2])
    ids = np.concatenate([np.array(p, np.int32) for p in prompts])
    lb = gm_b.forward(gm_b.plan([9, 40, 3], [0, 0, 0], bt, ids)).cpu().numpy()
    for s, p in enumerate(prompts):
        la = gm_a.forward(gm_a.plan([len(p)], [0], bt[s:s + 1], np.array(p, np.int32)))
        assert np.array_equal(la.cpu().numpy()[0].view(np.uint32), lb[s].view(np.uint32))
