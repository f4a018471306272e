"""GPU parity of the standalone entry points around the hot ops, through the
C ABI, against the oracle and closed forms.

- lgmlh_argmax: greedy = the first index of the maximum as src/sample.c:
  914-925 states it (m = x[0]; x[i] replaces m only when x[i] > m): ties
  keep the first index, a NaN at index 0 gives 0, a NaN elsewhere is never
  taken, all -inf gives 0. Expected indices are written out per case and
  also checked against the oracle's restatement (orc_argmax).
- lgmlh_set_rows_f16: the plain ggml_set_rows drop-in (src/lgml.c:
  1937-1969), bit-exact f32 -> f16 round to nearest even (numpy's IEEE
  conversion) on edge values, rows untouched elsewhere, range errors.
- lgmlh_rms_norm (f32, f16 out), lgmlh_swiglu / lgmlh_geglu,
  lgmlh_qkv_rope_store, lgmlh_get_rows: against the oracle's row ops (the
  ones its golden-pinned forward runs).
- lgmlh_gen_normal: bit-exact against the oracle generator (splitmix64 +
  Box-Muller, pinned by splitmix64's published outputs) and its quantizers:
  the bench's weights are the oracle's weights.
"""
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


def argmax_dev(L, x):
    from lgml_amd import hip
    x = np.ascontiguousarray(x, np.float32)
    out = torch.empty(x.shape[0], dtype=torch.int32, device="cuda")
    xd = dev(x)  # held: a freed temporary's memory goes to the next upload
    hip.check(L.lgmlh_argmax(xd.data_ptr(), x.shape[0], x.shape[1], out.data_ptr(), st()))
    return out.cpu().numpy().tolist()


@pytest.mark.parametrize("n", [128256, 1001, 262144, 5])
def test_argmax_first_max_and_nan(L, n):
    rng = np.random.default_rng(n)
    rows, want = [], []

    def case(x, w):
        rows.append(x.astype(np.float32))
        want.append(w)

    x = rng.standard_normal(n).astype(np.float32)
    case(x, int(np.argmax(x)))                          # random
    t = np.zeros(n, np.float32)
    hot = sorted({min(3, n - 1), n // 2, n - 1})
    t[hot] = 7.0
    case(t, hot[0])                                     # ties: the first
    case(np.full(n, -np.inf, np.float32), 0)            # all -inf
    z = np.zeros(n, np.float32)
    z[0] = -0.0
    case(z, 0)                                          # -0 == +0: a tie
    a = rng.standard_normal(n).astype(np.float32)
    a[0] = np.nan
    a[n - 1] = 100.0
    case(a, 0)                                          # NaN at 0 decides the row
    if n > 4352:
        # NaN at index 256: the first element of thread 64's float4 slice
        # (and lane 0 of wave 1); the maximum sits at 4352, that thread's
        # next float4 (1024 threads x 4 values further)
        b = rng.standard_normal(n).astype(np.float32)
        b[256] = np.nan
        b[4352] = 50.0
        case(b, 4352)
        c = rng.standard_normal(n).astype(np.float32)
        c[1:: 97] = np.nan                              # NaNs spread over every thread
        c[n - 2] = 60.0
        case(c, n - 2)
    d = np.full(n, np.nan, np.float32)
    d[0] = -5.0
    case(d, 0)                                          # only x[0] is a number
    e = rng.standard_normal(n).astype(np.float32)
    e[n - 1] = np.inf
    e[min(2, n - 1)] = np.inf
    case(e, min(2, n - 1))                              # +inf: the first
    x = np.stack(rows)
    got = argmax_dev(L, x)
    assert got == want
    assert [core.argmax(r) for r in rows] == want       # the oracle's restatement agrees


def test_set_rows_f16_bit_exact(L):
    from lgml_amd import hip
    rows, row, n = 1000, 384, 130
    rng = np.random.default_rng(3)
    src = (rng.standard_normal((n, row)) * 4).astype(np.float32)
    edge = np.array([6e-8, 3e-8, 2.98e-8, 65519.0, 65520.0, 1e6, -1e6, 1e-9, 1.00048828125,
                     1.000732421875, -0.0, 5.96e-8, np.inf, -np.inf], np.float32)
    src[0, :len(edge)] = edge
    ids = rng.choice(rows, n, replace=False).astype(np.int64)
    dst = torch.zeros((rows, row), dtype=torch.int16, device="cuda")
    dsrc, dids = dev(src), dev(ids)
    hip.check(L.lgmlh_set_rows_f16(dst.data_ptr(), rows, row, dsrc.data_ptr(), dids.data_ptr(),
                                   ids.ctypes.data, n, st()))
    got = dst.cpu().numpy().view(np.uint16)
    want = np.zeros((rows, row), np.uint16)
    want[ids] = src.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    ora = np.zeros((rows, row), np.uint16)
    core.set_rows_f16(ora, src, ids)
    assert np.array_equal(got, ora)
    bad = ids.copy()
    bad[5] = rows
    dbad = dev(bad)
    rc = L.lgmlh_set_rows_f16(dst.data_ptr(), rows, row, dsrc.data_ptr(), dbad.data_ptr(),
                              bad.ctypes.data, n, st())
    assert rc == hip.ERANGE
    bad[5] = -1
    assert L.lgmlh_set_rows_f16(dst.data_ptr(), rows, row, dsrc.data_ptr(), dbad.data_ptr(),
                                bad.ctypes.data, n, st()) == hip.ERANGE
    assert np.array_equal(dst.cpu().numpy().view(np.uint16), want)  # nothing written


@pytest.mark.parametrize("n", [4096, 2560, 2048, 64])
@pytest.mark.parametrize("rows", [37, 600])  # past 512 rows: n / 8 threads per row
def test_rms_norm_f32_and_f16(L, n, rows):
    from lgml_amd import hip
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((rows, n)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    want = core.rms_norm(x, 1e-6, w)
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    dx, dw = dev(x), dev(w)
    hip.check(L.lgmlh_rms_norm(dx.data_ptr(), rows, n, 1e-6, dw.data_ptr(), out.data_ptr(),
                               hip.F32, st()))
    got = out.cpu().numpy()
    assert rel_err(got, want) < 1e-6
    # a row gives the same bits in either launch shape
    few = torch.empty((3, n), dtype=torch.float32, device="cuda")
    hip.check(L.lgmlh_rms_norm(dx.data_ptr(), 3, n, 1e-6, dw.data_ptr(), few.data_ptr(), hip.F32,
                               st()))
    assert np.array_equal(few.cpu().numpy().view(np.uint32), got[:3].view(np.uint32))
    o16 = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    hip.check(L.lgmlh_rms_norm(dx.data_ptr(), rows, n, 1e-6, dw.data_ptr(), o16.data_ptr(),
                               hip.F16, st()))
    g16 = o16.cpu().numpy().view(np.uint16).astype(np.int32)
    w16 = got.astype(np.float16).view(np.uint16).astype(np.int32)
    assert np.array_equal(g16, w16)  # f16 of the kernel's own f32 values
    # without a weight
    hip.check(L.lgmlh_rms_norm(dx.data_ptr(), rows, n, 1e-5, None, out.data_ptr(), hip.F32,
                               st()))
    assert rel_err(out.cpu().numpy(), core.rms_norm(x, 1e-5)) < 1e-6


@pytest.mark.parametrize("gelu", [False, True])
def test_swiglu_geglu(L, gelu):
    from lgml_amd import hip
    n, F = 19, 14336 if not gelu else 10240
    rng = np.random.default_rng(5 + gelu)
    gu = (rng.standard_normal((n, 2 * F)) * 3).astype(np.float32)
    gu[0, :6] = [0.0, -0.0, 30.0, -30.0, 1e-8, -100.0]
    want = core.glu(gu[:, :F], gu[:, F:], gelu)
    fn = L.lgmlh_geglu if gelu else L.lgmlh_swiglu
    out = torch.empty((n, F), dtype=torch.float32, device="cuda")
    dgu = dev(gu)
    hip.check(fn(dgu.data_ptr(), n, F, out.data_ptr(), hip.F32, st()))
    got = out.cpu().numpy()
    assert rel_err(got, want) < 1e-6
    o16 = torch.empty((n, F), dtype=torch.float16, device="cuda")
    hip.check(fn(dgu.data_ptr(), n, F, o16.data_ptr(), hip.F16, st()))
    assert np.array_equal(o16.cpu().numpy().view(np.uint16),
                          got.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("shape", [
    # H, Hkv, D, neox, q/k norm, base, freq factors
    (32, 8, 128, False, False, 5e5, True),    # llama-3 (rope_freqs)
    (32, 4, 128, True, True, 1e6, False),     # qwen3 / qwen3moe
    (8, 4, 256, True, True, 1e4, False),      # gemma heads
])
def test_qkv_rope_store(L, shape):
    from lgml_amd import hip
    H, Hkv, D, neox, qk, base, use_ff = shape
    n, n_cells = 45, 4096
    W = (H + 2 * Hkv) * D
    rng = np.random.default_rng(H + D)
    qkv = rng.standard_normal((n, W)).astype(np.float32)
    pos = rng.integers(0, 20000, n).astype(np.int32)
    pos[:3] = [0, 1, 65535]
    cells = rng.choice(n_cells, n, replace=False).astype(np.int64)
    qn = rng.uniform(0.8, 1.2, D).astype(np.float32) if qk else None
    kn = rng.uniform(0.8, 1.2, D).astype(np.float32) if qk else None
    ff = rng.uniform(1.0, 8.0, D // 2).astype(np.float32) if use_ff else None
    eps = 1e-6
    kb = L.lgmlh_kv_layer_bytes(n_cells, Hkv, D)
    kp = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    vp = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    q_out = torch.empty((n, H * D), dtype=torch.float32, device="cuda")
    dq = dev(qkv)
    keep = [dev(a) if a is not None else None for a in (ff, qn, kn)]
    p = [t.data_ptr() if t is not None else None for t in keep]
    dc, dpos = dev(cells), dev(pos)
    hip.check(L.lgmlh_qkv_rope_store(dq.data_ptr(), n, H, Hkv, D, D, int(neox), base, p[0], p[1],
                                     p[2], eps, dpos.data_ptr(), kp.data_ptr(), vp.data_ptr(),
                                     n_cells, dc.data_ptr(), q_out.data_ptr(), st()))
    q = qkv[:, :H * D].reshape(n * H, D)
    k = qkv[:, H * D:(H + Hkv) * D].reshape(n * Hkv, D)
    v = qkv[:, (H + Hkv) * D:]
    if qk:
        q = core.rms_norm(q, eps, qn)
        k = core.rms_norm(k, eps, kn)
    qw = core.rope(q.reshape(n, H * D), H, D, D, neox, base, pos, ff)
    kw = core.rope(k.reshape(n, Hkv * D), Hkv, D, D, neox, base, pos, ff)
    assert rel_err(q_out.cpu().numpy(), qw) < 1e-6
    # V has no norm and no rope: its f16 bits at exactly these cells
    for which, pool, want in ((0, kp, kw), (1, vp, v)):
        out = torch.empty((n, Hkv * D), dtype=torch.int16, device="cuda")
        hip.check(L.lgmlh_kv_gather(pool.data_ptr(), which, n_cells, Hkv, D, dc.data_ptr(), n,
                                    out.data_ptr(), st()))
        got = out.cpu().numpy().view(np.uint16)
        w16 = want.astype(np.float16).view(np.uint16)
        if which == 1:
            assert np.array_equal(got, w16)
        else:
            # rope's cos / sin: the device's f32 math and the host libm may
            # differ in the last bit, one f16 ulp at most after rounding
            diff = np.abs(got.astype(np.int32) - w16.astype(np.int32))
            assert diff.max() <= 1 and (diff == 0).mean() > 0.999
    # no other cell was written
    others = np.setdiff1d(np.arange(n_cells), cells)
    for which, pool in ((0, kp), (1, vp)):
        sel = others[::7]
        out = torch.empty((len(sel), Hkv * D), dtype=torch.int16, device="cuda")
        dsel = dev(sel.astype(np.int64))
        hip.check(L.lgmlh_kv_gather(pool.data_ptr(), which, n_cells, Hkv, D, dsel.data_ptr(),
                                    len(sel), out.data_ptr(), st()))
        assert not out.cpu().numpy().any()


@pytest.mark.parametrize("ty", [core.F32, core.F16, core.Q8_0, core.Q4_K, core.Q6_K])
def test_get_rows(L, ty):
    from lgml_amd import hip
    rows, cols, n = 300, 512, 77
    wf = core.fill_normal(rows * cols, 0, 0.5, 17).reshape(rows, cols)
    if ty == core.F32:
        table, deq = wf, wf
    elif ty == core.F16:
        table = wf.astype(np.float16).view(np.uint16)
        deq = wf.astype(np.float16).astype(np.float32)
    else:
        table = core.quantize(ty, wf)
        deq = core.dequantize(ty, table, cols)
    rng = np.random.default_rng(ty)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[:3] = [0, rows - 1, 0]
    out = torch.empty((n, cols), dtype=torch.float32, device="cuda")
    dt, dids = dev(table), dev(ids)
    hip.check(L.lgmlh_get_rows(ty, dt.data_ptr(), rows, cols, dids.data_ptr(), ids.ctypes.data,
                               n, out.data_ptr(), st()))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), deq[ids].view(np.uint32))
    bad = ids.copy()
    bad[9] = rows
    dbad = dev(bad)
    assert L.lgmlh_get_rows(ty, dt.data_ptr(), rows, cols, dbad.data_ptr(), bad.ctypes.data,
                            n, out.data_ptr(), st()) == hip.ERANGE


@pytest.mark.parametrize("case", [
    (core.F32, 64, 4096, 0.0, 0.02), (core.Q4_K, 256, 4096, 0.0, 0.02),
    (core.Q6_K, 128, 4096, 0.0, 0.02), (core.Q8_0, 160, 2560, 0.0, 0.02),
    (core.Q4_K, 64, 14336, 0.0, 0.02), (core.F32, 16, 2048, 0.0, 1.0 / np.sqrt(2048)),
])
def test_gen_normal_matches_oracle(L, case):
    from lgml_amd import hip
    ty, rows, cols, mean, sd = case
    seed = 20261201 * 1000003 + rows + ty
    nb = core.row_size(ty, cols) * rows
    out = torch.empty(nb, dtype=torch.uint8, device="cuda")
    hip.check(L.lgmlh_gen_normal(seed, ty, rows, cols, mean, sd, out.data_ptr(), st()))
    got = out.cpu().numpy()
    if ty == core.F32:
        want = core.gen_normal(rows * cols, mean, sd, seed).view(np.uint8)
    else:
        want = core.gen_normal_quant(ty, rows, cols, mean, sd, seed).reshape(-1)
    assert np.array_equal(got, want)
