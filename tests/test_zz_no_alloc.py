"""lgmlh_mul_mat_noalloc (the entry point that allocates nothing: its
workspace is a static device array) against lgmlh_mul_mat with a caller
workspace, through the C ABI: bit-identical outputs on two calls in a row,
the second with a smaller input (the array keeps the first call's contents),
for each quantized type, split and unsplit K, with and without the residual
epilogue; a product whose workspace exceeds the array is refused."""
import numpy as np
import pytest

from oracle import core

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


def repacked(L, ty, M, K, seed):
    from lgml_amd import hip
    wf = core.fill_normal(M * K, 0, 0.02, seed).reshape(M, K)
    w = core.quantize(ty, wf)
    wd = dev(w)
    rp = torch.empty(L.lgmlh_repacked_bytes(ty, M, K), dtype=torch.uint8, device="cuda")
    hip.check(L.lgmlh_repack(ty, M, K, wd.data_ptr(), rp.data_ptr(), st()))
    torch.cuda.synchronize()
    return rp


def both(L, ty, rp, M, K, x, res=None):
    """(lgmlh_mul_mat, lgmlh_mul_mat_noalloc) outputs of one product."""
    from lgml_amd import hip
    N = x.shape[0]
    xd = dev(x)
    epi = hip.EPI_ADD if res is not None else hip.EPI_NONE
    outs = []
    for noalloc in (False, True):
        y = dev(res.copy()) if res is not None else torch.full((N, M), np.nan, device="cuda")
        rptr = y.data_ptr() if res is not None else None  # the residual aliases y
        if noalloc:
            hip.check(L.lgmlh_mul_mat_noalloc(ty, rp.data_ptr(), M, K, xd.data_ptr(), hip.F32, N,
                                              y.data_ptr(), epi, rptr, st()))
        else:
            n = L.lgmlh_mul_mat_workspace(ty, M, K, N)
            ws = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
            hip.check(L.lgmlh_mul_mat(ty, rp.data_ptr(), M, K, xd.data_ptr(), hip.F32, N,
                                      y.data_ptr(), epi, rptr, ws.data_ptr(), n, st()))
        outs.append(y.cpu().numpy())
    return outs


@pytest.mark.parametrize("ty", [core.Q4_K, core.Q6_K, core.Q8_0])
def test_noalloc_equals_workspace_path(L, ty):
    # (M, K, N): the first is split over K (down-shaped), the second smaller
    # and unsplit, the third a decode-sized split product again
    cases = [(4096, 14336, 64), (512, 1024, 9), (1024, 4096, 33)]
    for i, (M, K, N) in enumerate(cases):
        rp = repacked(L, ty, M, K, 40 + i)
        x = core.fill_normal(N * K, 0, 1, 50 + i).reshape(N, K)
        a, b = both(L, ty, rp, M, K, x)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (M, K, N)
        res = core.fill_normal(N * M, 0, 1, 60 + i).reshape(N, M)
        a, b = both(L, ty, rp, M, K, x, res)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (M, K, N, "residual")


def test_noalloc_refuses_past_its_limit(L):
    from lgml_amd import hip
    limit = L.lgmlh_mul_mat_noalloc_limit()
    M, K = 4096, 14336
    N = 1024  # split planes alone: 1024 x 14336 x 4.125 B > 32 MiB
    assert L.lgmlh_mul_mat_workspace(core.Q4_K, M, K, N) > limit
    y = torch.empty((1, 1), device="cuda")
    rc = L.lgmlh_mul_mat_noalloc(core.Q4_K, y.data_ptr(), M, K, y.data_ptr(), hip.F32, N,
                                 y.data_ptr(), hip.EPI_NONE, None, st())
    assert rc == hip.ENOMEM
    assert b"static scratch" in L.lgmlh_last_error()
