"""GPU parity of the single kernels against the CPU oracle, through the C ABI.

Bit-exact: KV store (f32 -> f16 RNE), gather, block copy, dequantization,
plan cells. Tolerance: attention and weight products within 2e-3 max
relative error of the oracle's f64 result; the
kernels keep weights exact and split f32 activations into f16 hi + lo, so
they also meet 1e-5 (products) and 1e-4 (attention). Batch invariance: a
row alone and in a batch give the same bits.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import core
from tests.gpu_util import rel_err

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


def test_kv_store_gather_bit_exact(L):
    from lgml_amd import hip
    Hkv, D, cells_n = 8, 128, 4096
    rng = np.random.default_rng(1)
    n = 200
    k = rng.standard_normal((n, Hkv * D)).astype(np.float32) * 3
    v = rng.standard_normal((n, Hkv * D)).astype(np.float32)
    # edge values: f16 subnormals, ties, overflow to inf, tiny -> 0
    edge = np.array([6e-8, 3e-8, 2.98e-8, 65519.0, 65520.0, 1e6, -1e6, 1e-9, 1.00048828125,
                     1.000732421875, -0.0, 5.96e-8], np.float32)
    k[0, :len(edge)] = edge
    v[1, :len(edge)] = edge
    cells = rng.choice(cells_n // 2, n, replace=False).astype(np.int64)
    kb = L.lgmlh_kv_layer_bytes(cells_n, Hkv, D)
    kp, vp = torch.zeros(kb, dtype=torch.uint8, device="cuda"), torch.zeros(kb, dtype=torch.uint8, device="cuda")
    dk, dv, dc = dev(k), dev(v), dev(cells)
    hip.check(L.lgmlh_kv_store(kp.data_ptr(), vp.data_ptr(), cells_n, Hkv, D, dk.data_ptr(),
                               dv.data_ptr(), dc.data_ptr(), cells.ctypes.data, n, st()))
    for which, src, pool in ((0, k, kp), (1, v, vp)):
        out = torch.empty((n, Hkv * D), dtype=torch.int16, device="cuda")
        hip.check(L.lgmlh_kv_gather(pool.data_ptr(), which, cells_n, Hkv, D, dc.data_ptr(), n,
                                    out.data_ptr(), st()))
        got = out.cpu().numpy().view(np.uint16)
        want = core.f32_to_f16_bits(src)
        assert np.array_equal(got, want)
        assert np.array_equal(got, src.astype(np.float16).view(np.uint16))
    # a cell out of range is an error, checked on the host
    bad = cells.copy()
    bad[3] = cells_n
    rc = L.lgmlh_kv_store(kp.data_ptr(), vp.data_ptr(), cells_n, Hkv, D, dk.data_ptr(),
                          dv.data_ptr(), dc.data_ptr(), bad.ctypes.data, n, st())
    assert rc == hip.ERANGE
    # copy_block: first 37 cells of block of cells[5] to a free block
    src_b = int(cells[5] // 64)
    used = set((cells // 64).tolist())
    dst_b = next(b for b in range(cells_n // 64) if b not in used)
    hip.check(L.lgmlh_kv_copy_block(kp.data_ptr(), vp.data_ptr(), cells_n, Hkv, D, src_b, dst_b,
                                    37, st()))
    sc = np.arange(src_b * 64, src_b * 64 + 64, dtype=np.int64)
    dcs = np.arange(dst_b * 64, dst_b * 64 + 64, dtype=np.int64)
    for which, pool in ((0, kp), (1, vp)):
        def g(c):
            o = torch.empty((64, Hkv * D), dtype=torch.int16, device="cuda")
            cd = dev(c)
            hip.check(L.lgmlh_kv_gather(pool.data_ptr(), which, cells_n, Hkv, D,
                                        cd.data_ptr(), 64, o.data_ptr(), st()))
            return o.cpu().numpy()
        a, b = g(sc), g(dcs)
        assert np.array_equal(a[:37], b[:37]) and np.all(b[37:] == 0)


@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K, core.Q8_0])
def test_dequantize_bit_exact(L, ty):
    from lgml_amd import hip
    M, K = 96, 1024
    x = core.fill_normal(M * K, 0, 0.02, 5).reshape(M, K)
    q = core.quantize(ty, x)
    # also raw random bytes with finite f16 scales
    rng = np.random.default_rng(2)
    raw = rng.integers(0, 256, size=q.shape, dtype=np.uint8)
    bs = {core.Q4_K: 144, core.Q6_K: 210, core.Q8_0: 34}[ty]
    for blk in range(q.shape[1] // bs):
        o = blk * bs
        if ty == core.Q6_K:
            raw[:, o + 208:o + 210] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
        else:
            raw[:, o:o + 2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
            if ty == core.Q4_K:
                raw[:, o + 2:o + 4] = np.frombuffer(np.float16(0.003).tobytes(), np.uint8)
    for data in (q, raw):
        out = torch.empty((M, K), dtype=torch.float32, device="cuda")
        dd = dev(data)
        hip.check(L.lgmlh_dequantize(ty, dd.data_ptr(), M, K, out.data_ptr(), st()))
        want = core.dequantize(ty, data, K)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def run_mul_mat(L, ty, w, M, K, x, xtype=None):
    from lgml_amd import hip
    N = x.shape[0]
    nb = L.lgmlh_repacked_bytes(ty, M, K)
    rp = torch.empty(nb, dtype=torch.uint8, device="cuda")
    wd = dev(w)
    hip.check(L.lgmlh_repack(ty, M, K, wd.data_ptr(), rp.data_ptr(), st()))
    ws_n = L.lgmlh_mul_mat_workspace(ty, M, K, N)
    ws = torch.zeros(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty((N, M), dtype=torch.float32, device="cuda")
    xt = xtype if xtype is not None else hip.F32
    xd = dev(x.astype(np.float16) if xt == hip.F16 else x)
    hip.check(L.lgmlh_mul_mat(ty, rp.data_ptr(), M, K, xd.data_ptr(), xt, N, y.data_ptr(),
                              hip.EPI_NONE, None, ws.data_ptr(), ws_n, st()))
    return y.cpu().numpy()


# Column tiles per workgroup (gemm.hip launch_q): 16 for N <= 16, 32 for
# N <= 32, else 64; but a product of N <= 64 with fewer than 200 workgroups
# of row tiles x K splits (Q4_K: 100) takes 16. The small shapes run the
# 16-column kernel at N <= 64 and the 64-column one at N = 70 and 130; the
# large ones, (25600, 1024) = 100 row tiles x 2 splits and (51200, 256) =
# 200 x 1, run the 32- and 64-column kernels at N = 17 / 32 and 64 / 130;
# (12800, 1024) = 50 x 2 runs Q4_K's 64-column kernel at N = 64 and the
# others' 16-column one.
@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K, core.Q8_0, core.F32])
@pytest.mark.parametrize("MK", [(512, 1024), (256, 4096), (48, 768), (25600, 1024),
                                (51200, 256), (12800, 1024)])
def test_mul_mat_parity_and_batch_invariance(L, ty, MK):
    M, K = MK
    if ty != core.F32 and K % 256:
        pytest.skip("quantized K must be a multiple of 256")
    big = M * K > 4_000_000
    if big and ty == core.F32:
        pytest.skip("the column tiles are a quantized-product choice")
    wf = core.fill_normal(M * K, 0, 0.02, 7).reshape(M, K)
    w = wf if ty == core.F32 else core.quantize(ty, wf)
    deq = wf if ty == core.F32 else core.dequantize(ty, w, K)
    x = core.fill_normal(130 * K, 0, 1, 8).reshape(130, K)
    for N in ((17, 32, 64, 130) if big else (1, 3, 17, 32, 64, 70, 130)):
        y = run_mul_mat(L, ty, w, M, K, x[:N])
        want = core.mul_mat(core.F32, deq, M, K, x[:N])
        assert rel_err(y, want) < 2e-3, (N, rel_err(y, want))
        assert rel_err(y, want) < 1e-5, (N, rel_err(y, want))
        if N in (32, 130):  # a 16-column launch alone, the 32- / 64-column one batched
            for j in ((0, 63, 64, 129) if N == 130 else (0, 16, 31)):
                alone = run_mul_mat(L, ty, w, M, K, x[j:j + 1])
                assert np.array_equal(alone[0].view(np.uint32), y[j].view(np.uint32)), j


# At large batches a workgroup runs both K splits of a pair (gemm.hip
# launch_q: Q4_K / Q6_K with 64-column tiles and at least 8192 workgroups
# of single splits: column tiles x row blocks of 128 (Q4_K) or 256 (Q6_K)
# rows x splits); its sums are the same as with one workgroup per split,
# bit for bit. (4096, 4096): 8 splits, 4 pairs; (4096, 3584): 7 splits,
# the last pair a single split; (16384, 1024): 2 splits, one pair, written
# straight to y (and, with the residual, over it in place). N is the
# smallest multiple of 64 that reaches 8192 workgroups.
FOLD_N = {(core.Q4_K, (4096, 4096)): 2048, (core.Q4_K, (4096, 3584)): 2368,
          (core.Q4_K, (16384, 1024)): 2048, (core.Q6_K, (4096, 4096)): 4096,
          (core.Q6_K, (4096, 3584)): 4736, (core.Q6_K, (16384, 1024)): 4096}


@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K])
@pytest.mark.parametrize("MK", [(4096, 4096), (4096, 3584), (16384, 1024)])
def test_mul_mat_folded_split_pairs(L, ty, MK):
    from lgml_amd import hip
    M, K = MK
    N = FOLD_N[(ty, MK)]
    wf = core.fill_normal(M * K, 0, 0.02, 17).reshape(M, K)
    w = core.quantize(ty, wf)
    x = core.fill_normal(N * K, 0, 1, 18).reshape(N, K)
    y = run_mul_mat(L, ty, w, M, K, x)
    y130 = run_mul_mat(L, ty, w, M, K, x[:130])  # one workgroup per split
    assert np.array_equal(y[:130].view(np.uint32), y130.view(np.uint32))
    alone = run_mul_mat(L, ty, w, M, K, x[N - 1:N])
    assert np.array_equal(alone[0].view(np.uint32), y[N - 1].view(np.uint32))
    rows = [0, 65, 300, N - 1]
    want = core.mul_mat(core.F32, core.dequantize(ty, w, K), M, K, x[rows])
    assert rel_err(y[rows], want) < 1e-5, rel_err(y[rows], want)
    # the residual added in place (y is the residual)
    nb = L.lgmlh_repacked_bytes(ty, M, K)
    rp = torch.empty(nb, dtype=torch.uint8, device="cuda")
    wd = dev(w)
    hip.check(L.lgmlh_repack(ty, M, K, wd.data_ptr(), rp.data_ptr(), st()))
    res = core.fill_normal(N * M, 0, 1, 19).reshape(N, M)
    yd = dev(res.copy())
    ws_n = L.lgmlh_mul_mat_workspace(ty, M, K, N)
    ws = torch.zeros(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    xd = dev(x)
    hip.check(L.lgmlh_mul_mat(ty, rp.data_ptr(), M, K, xd.data_ptr(), hip.F32, N, yd.data_ptr(),
                              hip.EPI_ADD, yd.data_ptr(), ws.data_ptr(), ws_n, st()))
    assert np.array_equal(yd.cpu().numpy(), (y + res).astype(np.float32))


def test_mul_mat_f32_input_and_residual(L):
    from lgml_amd import hip
    M, K, N = 512, 1024, 9
    wf = core.fill_normal(M * K, 0, 0.02, 9).reshape(M, K)
    w = core.quantize(core.Q4_K, wf)
    x = core.fill_normal(N * K, 0, 1, 10).reshape(N, K)
    x = x.astype(np.float16).astype(np.float32)  # values an f16 input can hold
    y16 = run_mul_mat(L, core.Q4_K, w, M, K, x, hip.F16)
    y32 = run_mul_mat(L, core.Q4_K, w, M, K, x, hip.F32)
    assert np.array_equal(y16, y32)  # an f16 x is the f32 x with a zero lo part
    nb = L.lgmlh_repacked_bytes(core.Q4_K, M, K)
    rp = torch.empty(nb, dtype=torch.uint8, device="cuda")
    wd = dev(w)
    hip.check(L.lgmlh_repack(core.Q4_K, M, K, wd.data_ptr(), rp.data_ptr(), st()))
    res = core.fill_normal(N * M, 0, 1, 11).reshape(N, M)
    yd = dev(res.copy())
    ws_n = L.lgmlh_mul_mat_workspace(core.Q4_K, M, K, N)
    ws = torch.zeros(max(ws_n, 1), dtype=torch.uint8, device="cuda")
    xd = dev(x)
    hip.check(L.lgmlh_mul_mat(core.Q4_K, rp.data_ptr(), M, K, xd.data_ptr(), hip.F32, N,
                              yd.data_ptr(), hip.EPI_ADD, yd.data_ptr(), ws.data_ptr(), ws_n,
                              st()))
    assert np.array_equal(yd.cpu().numpy(), (y32 + res).astype(np.float32))


def make_attn_case(H, Hkv, D, seqs, seed, n_cells=8192):
    """seqs: list of (n, npast). Random q, pool; scattered block tables."""
    rng = np.random.default_rng(seed)
    nblocks = n_cells // 64
    perm = rng.permutation(nblocks)
    bts, used = [], 0
    for n, npast in seqs:
        nb = (npast + n + 63) // 64
        bts.append(perm[used:used + nb])
        used += nb
    assert used <= nblocks
    mb = max(len(b) for b in bts)
    bt = np.full((len(seqs), mb), -1, np.int32)
    for i, b in enumerate(bts):
        bt[i, :len(b)] = b
    N = sum(n for n, _ in seqs)
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    kpool = core.f32_to_f16_bits(rng.standard_normal((n_cells, Hkv * D)).astype(np.float32))
    vpool = core.f32_to_f16_bits(rng.standard_normal((n_cells, Hkv * D)).astype(np.float32))
    return q, kpool, vpool, bt


def gpu_attention(L, q, kpool_rows, vpool_rows, H, Hkv, D, seqs, bt, bps=0, n_cells=8192,
                  order=True):
    from lgml_amd import hip, runtime
    seq_n = [n for n, _ in seqs]
    npast = [p for _, p in seqs]
    ids = np.zeros(sum(seq_n), np.int32)
    plan = runtime.Plan(seq_n, npast, bt, ids, H, Hkv, n_cells // 64, bps)
    if not order:
        plan.ub.order = None  # the items on their own start in index order
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
    scale = 1.0 / np.sqrt(D)
    qd = dev(q)
    hip.check(L.lgmlh_paged_attention(qd.data_ptr(), H, Hkv, D, scale, kp.data_ptr(),
                                      vp.data_ptr(), C.byref(plan.ub), out.data_ptr(),
                                      ws.data_ptr(), wsb, st()))
    return out.cpu().numpy(), plan


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (4, 2, 64), (8, 4, 256), (16, 16, 64),
                                     (4, 2, 16), (8, 1, 32)])
def test_paged_attention_parity(L, H, Hkv, D):
    seqs = [(1, 0), (1, 63), (1, 64), (1, 200), (37, 0), (1, 1500), (5, 61), (64, 130), (1, 3000)]
    q, kpool, vpool, bt = make_attn_case(H, Hkv, D, seqs, seed=H + D)
    for bps in (0, 1, 3):
        got, plan = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, bps)
        b = core.BatchDesc([n for n, _ in seqs], [p for _, p in seqs], bt, 64,
                           np.zeros(len(q), np.int32), [])
        want = core.paged_attention(q, kpool, vpool, H, Hkv, D, 1.0 / np.sqrt(D), b)
        assert np.isfinite(got).all()
        e = rel_err(got.reshape(len(q) * H, D), want.reshape(len(q) * H, D))
        assert e < 2e-3 and e < 1e-4, (bps, e)


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (32, 4, 128), (4, 2, 64), (4, 2, 16),
                                     (8, 2, 32)])
def test_paged_attention_prompt_chunks(L, H, Hkv, D):
    """Prompt chunks run in shared sets of 8 query groups (one workgroup
    reads each K / V block once for the set, lgmlh_plan): a 512-token chunk
    deep in its prompt, sets cut short (37 and 40 tokens), a decode token
    beside them; runs of 16 blocks and of 3 (merges of interleaved items)."""
    seqs = [(512, 2500), (1, 700), (37, 3000), (40, 63)]
    q, kpool, vpool, bt = make_attn_case(H, Hkv, D, seqs, seed=H + Hkv + D, n_cells=16384)
    for bps in (0, 3):
        got, plan = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, bps, n_cells=16384)
        assert plan.info.n_shared > 0 and plan.info.n_single > 0
        b = core.BatchDesc([n for n, _ in seqs], [p for _, p in seqs], bt, 64,
                           np.zeros(len(q), np.int32), [])
        want = core.paged_attention(q, kpool, vpool, H, Hkv, D, 1.0 / np.sqrt(D), b)
        assert np.isfinite(got).all()
        e = rel_err(got.reshape(len(q) * H, D), want.reshape(len(q) * H, D))
        assert e < 1e-4, (bps, e)
        off = 0
        for i, (n, p) in enumerate(seqs):  # alone: the same bits
            alone, _ = gpu_attention(L, q[off:off + n], kpool, vpool, H, Hkv, D, [(n, p)],
                                     bt[i:i + 1], bps, n_cells=16384)
            assert np.array_equal(alone.view(np.uint32), got[off:off + n].view(np.uint32)), i
            off += n


def test_paged_attention_more_splits_than_kept_weights(L):
    """A group split into more runs (68) than the merge keeps weights for in
    LDS (64): the last runs' weights are recomputed from m and M."""
    H, Hkv, D = 8, 2, 128
    seqs = [(1, 4300), (3, 4400)]
    q, kpool, vpool, bt = make_attn_case(H, Hkv, D, seqs, seed=77, n_cells=16384)
    got, plan = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, 1, n_cells=16384)
    b = core.BatchDesc([n for n, _ in seqs], [p for _, p in seqs], bt, 64,
                       np.zeros(len(q), np.int32), [])
    want = core.paged_attention(q, kpool, vpool, H, Hkv, D, 1.0 / np.sqrt(D), b)
    assert np.isfinite(got).all()
    assert rel_err(got.reshape(len(q) * H, D), want.reshape(len(q) * H, D)) < 1e-4


def test_paged_attention_alone_equals_batched(L):
    H, Hkv, D = 32, 8, 128
    seqs = [(1, 100), (1, 2000), (9, 700), (1, 5)]
    q, kpool, vpool, bt = make_attn_case(H, Hkv, D, seqs, seed=3)
    got, _ = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, bps=2)
    off = 0
    for i, (n, p) in enumerate(seqs):
        alone, _ = gpu_attention(L, q[off:off + n], kpool, vpool, H, Hkv, D, [(n, p)],
                                 bt[i:i + 1], bps=2)
        assert np.array_equal(alone.view(np.uint32), got[off:off + n].view(np.uint32)), i
        off += n


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (8, 4, 256)])
def test_paged_attention_order_changes_no_bits(L, H, Hkv, D):
    """The plan's dispatch order (longest runs first) only changes which
    workgroup runs an item: the same bits as index order, with runs of
    mixed lengths and merges."""
    seqs = [(1, 63), (1, 700), (1, 3000), (4, 1500), (1, 64), (1, 2100), (9, 400)]
    q, kpool, vpool, bt = make_attn_case(H, Hkv, D, seqs, seed=H * D)
    for bps in (0, 5):
        a, plan = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, bps)
        b, _ = gpu_attention(L, q, kpool, vpool, H, Hkv, D, seqs, bt, bps, order=False)
        items = plan.host_array(plan.info.off_items, 4 * plan.info.n_single, np.int32)
        lengths = [(int(it[3]) >> 16) - (int(it[3]) & 0xffff) for it in items.reshape(-1, 4)]
        assert len(set(lengths)) > 1  # the order is not the index order
        assert np.isfinite(a).all()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), bps


def test_plan_cells_and_errors(L):
    from lgml_amd import hip, runtime
    from oracle import kvpool as kp
    bt = np.array([[5, 2, 9], [0, 1, -1]], np.int32)
    plan = runtime.Plan([3, 2], [126, 60], bt, np.array([1, 2, 3, 4, 5], np.int32), 4, 2, 16)
    want = kp.seq_cells([5, 2, 9], 64, 126, 3) + kp.seq_cells([0, 1], 64, 60, 2)
    assert list(plan.cells) == want
    assert list(plan.logit_rows) == [2, 4]
    with pytest.raises(hip.LgmlhError):
        runtime.Plan([3, 2], [126, 127], bt, np.zeros(5, np.int32), 4, 2, 16)  # seq 1 needs a 3rd block
    with pytest.raises(hip.LgmlhError):
        runtime.Plan([3], [126], bt[:1], np.zeros(3, np.int32), 4, 2, 9)  # block 9 past the pool
