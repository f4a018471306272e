"""Pins the oracle's sliding-window ring attention and gemma layers.

The tiny gemma4 model's llama.cpp rows (REF.dense of
test/test_gemma4.lua:192-224, tests/test_oracle_golden.py) pin the whole
forward: the window-6 ring, proportional rope, V from the raw K, the V
norm, post norms, GeGLU, layer output scales, the embedding scale. Here,
planted mistakes in each of those must fail the rows, and the windowed ring
attention is checked against a brute-force numpy statement of the mask of
tensor_fill_mask (src/lgml.c:2873-2935). The logit softcap is not pinned by
the rows (30 tanh(l / 30) is within 2e-3 of l at these logits): its closed
form is checked where it is computed (tests/test_gpu_gemma.py).
"""
import numpy as np
import pytest

from oracle import core, models


def gemma_err(monkeypatch, fhp=None, fw=None):
    from tests import test_oracle_golden as tg
    orig = models.ref_tiny_gemma4

    def patched():
        hp, w = orig()
        if fhp:
            fhp(hp)
        if fw:
            fw(w)
        return hp, w

    monkeypatch.setattr(models, "ref_tiny_gemma4", patched)
    d, ref, rows = tg.run_gemma4_rows()
    idx = [i - 1 for i in d["idx_1based"]]
    return max(max(abs(float(g[i]) - v) for i, v in zip(idx, r["v"])) for r, g in zip(ref, rows))


def _pop(key, layer=None):
    def f(w):
        for i, L in enumerate(w["layers"]):
            if layer is None or i == layer:
                L.pop(key, None)
    return f


@pytest.mark.parametrize("name,fhp,fw", [
    ("window 5", lambda hp: hp.update(n_swa=5), None),
    ("window 7", lambda hp: hp.update(n_swa=7), None),
    ("no window", lambda hp: hp.update(n_swa=1000), None),
    ("SiLU for GeGLU, no V norm", lambda hp: hp.update(gemma=False), None),
    ("no embedding scale", lambda hp: hp.update(embd_scale=0.0), None),
    ("attention scale 1/sqrt(D)", lambda hp: hp.update(attn_scale=0.0), None),
    ("no post-attention norm", None, _pop("post_attn_norm")),
    ("no post-FFN norm", None, _pop("post_ffn_norm")),
    ("no layer output scale", None, lambda w: [L.update(out_scale=0.0) for L in w["layers"]]),
    ("no proportional rope", None, _pop("rope_freqs", 1)),
])
def test_planted_gemma_mistakes_fail_the_rows(oracle_lib, monkeypatch, name, fhp, fw):
    assert gemma_err(monkeypatch, fhp, fw) > 4 * 2e-3, name


def np_swa(q, kf, vf, H, Hkv, D, scale, window, seq_n, npast, cell):
    """Brute force: query j of sequence s (position p) sees positions
    max(0, p - window + 1)..p, read at cell(s, pos)."""
    out = np.zeros_like(q, dtype=np.float64)
    t, G = 0, H // Hkv
    for s, (n, p0) in enumerate(zip(seq_n, npast)):
        for j in range(n):
            p = p0 + j
            ks = list(range(max(0, p - window + 1), p + 1))
            for h in range(H):
                kh = h // G
                K = np.array([kf[cell(s, kp), kh * D:(kh + 1) * D] for kp in ks], np.float64)
                Vv = np.array([vf[cell(s, kp), kh * D:(kh + 1) * D] for kp in ks], np.float64)
                sc = K @ q[t, h].astype(np.float64) * scale
                e = np.exp(sc - sc.max())
                out[t, h] = (e / e.sum()) @ Vv
            t += 1
    return out


def test_swa_ring_attention_matches_brute_force(oracle_lib):
    rng = np.random.default_rng(3)
    H, Hkv, D, block, ring_blocks, window = 4, 2, 32, 8, 3, 10
    seq_n, npast = [1, 5, 3], [40, 17, 2]
    cap = 128
    ring_tab = np.array([[4, 9, 1], [7, 2, 12], [0, 5, 14]], np.int32)
    kp = rng.integers(0x3000, 0x3c00, size=(cap, Hkv * D)).astype(np.uint16)
    vp = rng.integers(0x3000, 0x3c00, size=(cap, Hkv * D)).astype(np.uint16)
    q = rng.standard_normal((sum(seq_n), H, D)).astype(np.float32)
    b = core.BatchDesc(seq_n, npast, np.zeros((3, 1), np.int32), block, np.zeros(sum(seq_n)),
                       [0], ring_tab=ring_tab)
    got = core.paged_attention_swa(q, kp, vp, H, Hkv, D, 0.2, window, b)

    def cell(s, p):
        return ring_tab[s, (p // block) % ring_blocks] * block + p % block

    want = np_swa(q, core.f16_bits_to_f32(kp), core.f16_bits_to_f32(vp), H, Hkv, D, 0.2, window,
                  seq_n, npast, cell)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_c4_synthetic_model_is_well_conditioned(oracle_lib):
    """The tolerance of the C4 GPU parity test rests on this: the synthetic
    C4-shaped model (reduced depth and vocabulary) moves its logits by far
    less than 2e-3 when one weight vector changes by 1 ulp, so an f32
    implementation that differs from the oracle only in rounding order
    stays within the bar."""
    from tests.gpu_util import Schedule, rel_err
    shape = dict(models.SHAPES["c4"], n_swa=100, n_vocab=2048, n_layer=3, swa_period=3)
    hp, w = models.build(shape, seed=4, init="normal")
    lens = [5, 37, 150]
    n_cells = 1024

    def run(w):
        om = core.OracleModel(hp, w)
        kp = [np.zeros((n_cells, 4 * 256), np.uint16) for _ in range(3)]
        vp = [np.zeros((n_cells, 4 * 256), np.uint16) for _ in range(3)]
        sch = Schedule(n_cells // 64, len(lens))
        for s, n in enumerate(lens):
            sch.grow(s, n)
        rt = np.arange(12, dtype=np.int32).reshape(3, 4)
        ids = (np.arange(sum(lens)) * 7919 % hp["n_vocab"]).astype(np.int32)
        b = core.BatchDesc(lens, [0, 0, 0], sch.table([0, 1, 2]), 64, ids,
                           list(np.cumsum(lens) - 1), ring_tab=rt)
        return om.forward(kp, vp, b)

    a = run(w)
    w2 = dict(w, layers=[dict(L) for L in w["layers"]])
    for L in w2["layers"]:
        x, t = L["attn_norm"]
        L["attn_norm"] = (np.nextafter(x, np.float32(2)), t)
    assert rel_err(run(w2), a) < 1e-4
