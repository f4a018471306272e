"""GPU parity of lgmlh_flash_attn (graph:flash_attn over strided K / V
views with an explicit mask) against the oracle's orc_flash_attn (pinned in
tests/test_oracle_flash.py), within 1e-5 max relative error (the bar is
2e-3): head sizes 16..256, GQA, random and causal masks with broadcast
planes, softcap, ALiBi, a fully masked row, pool-row views with strides.
Under the fill_blocks mask over the pool rows it equals the paged kernel
(lgmlh_paged_attention) on the same cells.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import core, kvpool as kp
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


def gpu_flash(L, q, k, v, Hkv, n_kv, k_strides, v_strides, mask, scale, max_bias=0.0,
              softcap=0.0):
    from lgml_amd import hip
    H, T, D = q.shape
    qd, kd, vd = dev(q), dev(k), dev(v)
    md = dev(mask) if mask is not None else None
    mh, mr = (mask.shape[0], mask.shape[1]) if mask is not None else (0, 0)
    out = torch.full((T, H, D), float("nan"), dtype=torch.float32, device="cuda")
    hip.check(L.lgmlh_flash_attn(qd.data_ptr(), H, T, D, kd.data_ptr(), vd.data_ptr(), Hkv, n_kv,
                                 k_strides[0], k_strides[1], v_strides[0], v_strides[1],
                                 md.data_ptr() if md is not None else None, mh, mr, scale,
                                 max_bias, softcap, out.data_ptr(), st()))
    return out.cpu().numpy()


CASES = [  # H, Hkv, T, D, n_kv, mask kind, softcap, max_bias
    (4, 2, 5, 16, 37, "random", 0.0, 0.0),
    (8, 8, 3, 32, 200, "causal", 0.0, 0.0),
    (8, 2, 17, 64, 129, "random", 20.0, 0.0),
    (12, 4, 4, 80, 70, "random", 0.0, 8.0),
    (32, 8, 9, 128, 300, "causal", 0.0, 0.0),
    (8, 4, 2, 256, 1100, "random", 0.0, 0.0),
    (4, 1, 6, 128, 65, None, 0.0, 0.0),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_flash_attn_matches_oracle(L, case):
    H, Hkv, T, D, n_kv, kind, softcap, max_bias = CASES[case]
    rng = np.random.default_rng(10 + case)
    q = (rng.standard_normal((H, T, D)) * 0.5).astype(np.float32)
    k = core.f32_to_f16_bits(rng.standard_normal((Hkv, n_kv, D)).astype(np.float32))
    v = core.f32_to_f16_bits(rng.standard_normal((Hkv, n_kv, D)).astype(np.float32))
    mask = None
    if kind == "random":
        planes = 2 if H % 2 == 0 else 1
        m = rng.standard_normal((planes, T + 1, n_kv)).astype(np.float32)
        m[rng.random(m.shape) < 0.4] = -np.inf
        m[-1, T - 1, :] = -np.inf  # a fully masked row
        mask = core.f32_to_f16_bits(m)
    elif kind == "causal":
        m = np.where(np.arange(n_kv)[None, :] <= n_kv - T + np.arange(T)[:, None], 0.0, -np.inf)
        mask = core.f32_to_f16_bits(m[None].astype(np.float32))
    scale = 1.0 / np.sqrt(D)
    print("flash_attn case %d: H=%d Hkv=%d T=%d D=%d n_kv=%d mask=%s softcap=%g max_bias=%g" % (
        case, H, Hkv, T, D, n_kv, kind, softcap, max_bias), flush=True)
    got = gpu_flash(L, q, k, v, Hkv, n_kv, (D, n_kv * D), (D, n_kv * D), mask, scale, max_bias,
                    softcap)
    want = core.flash_attn(q, k, v, Hkv, mask, scale, max_bias, softcap)
    assert np.isfinite(got).all()
    assert rel_err(got.reshape(T * H, D) + 1e-30, want.reshape(T * H, D) + 1e-30) < 1e-5
    if kind == "random":
        assert not got[T - 1, H - 1].any()  # the fully masked row is zeros


def test_flash_attn_on_pool_rows_equals_paged_attention(L):
    """The same cells as plain (cap, Hkv * D) rows under fill_blocks masks
    and as the block pool through the plan give the same outputs."""
    from lgml_amd import hip, runtime
    rng = np.random.default_rng(3)
    H, Hkv, D, B, cap = 32, 8, 128, 64, 2048
    pool = kp.Pool(cap // B, B)
    seqs = [kp.Seq(pool) for _ in range(3)]
    seq_n, npast = [1, 9, 1], [700, 100, 5]
    for s in seqs:
        kp.reserve(s, 65)
    for s, n, p in zip(seqs, seq_n, npast):
        kp.reserve(s, n + p)
    bt = np.full((3, max(len(s.blocks) for s in seqs)), -1, np.int32)
    for i, s in enumerate(seqs):
        bt[i, :len(s.blocks)] = s.blocks
    krows = core.f32_to_f16_bits(rng.standard_normal((cap, Hkv * D)).astype(np.float32))
    vrows = core.f32_to_f16_bits(rng.standard_normal((cap, Hkv * D)).astype(np.float32))
    N = sum(seq_n)
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    # the paged kernel on the block pool
    plan = runtime.Plan(seq_n, npast, bt, np.zeros(N, np.int32), H, Hkv, cap // B)
    kb = L.lgmlh_kv_layer_bytes(cap, Hkv, D)
    kpd = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    vpd = torch.zeros(kb, dtype=torch.uint8, device="cuda")
    allc = np.arange(cap, dtype=np.int64)
    kf, vf, cd = dev(core.f16_bits_to_f32(krows)), dev(core.f16_bits_to_f32(vrows)), dev(allc)
    hip.check(L.lgmlh_kv_store(kpd.data_ptr(), vpd.data_ptr(), cap, Hkv, D, kf.data_ptr(),
                               vf.data_ptr(), cd.data_ptr(), allc.ctypes.data, cap, st()))
    paged = torch.empty((N, H, D), dtype=torch.float32, device="cuda")
    wsb = L.lgmlh_attention_workspace(C.byref(plan.info), D)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
    qd = dev(q)
    hip.check(L.lgmlh_paged_attention(qd.data_ptr(), H, Hkv, D, 1.0 / np.sqrt(D), kpd.data_ptr(),
                                      vpd.data_ptr(), C.byref(plan.ub), paged.data_ptr(),
                                      ws.data_ptr(), wsb, st()))
    paged = paged.cpu().numpy()
    off = 0
    for i, (n, p) in enumerate(zip(seq_n, npast)):
        m16 = core.f32_to_f16_bits(kp.fill_blocks(n, cap, p, B, list(seqs[i].blocks)))[None]
        qh = np.ascontiguousarray(q[off:off + n].transpose(1, 0, 2))
        got = gpu_flash(L, qh, krows, vrows, Hkv, cap, (Hkv * D, D), (Hkv * D, D), m16,
                        1.0 / np.sqrt(D))
        assert rel_err(got.reshape(n * H, D), paged[off:off + n].reshape(n * H, D)) < 1e-5, i
        off += n
