"""Pins the oracle's flash_attn with an explicit mask (orc_flash_attn).

- Under the fill_blocks mask (src/lgml.c:2936-3017, restated in
  oracle/kvpool.py and pinned by test_kvpool.lua's hand example) over the
  whole pool, flash_attn per sequence equals orc_paged_attention, which
  the reference's golden rows pin (tests/test_oracle_golden.py): scale,
  GQA head mapping, masking and the (tokens, heads, d) output layout.
- ALiBi slopes recovered from the outputs match the ALiBi paper's
  get_slopes (a different statement: the closest power of two's geometric
  sequence, then every other slope of twice as many heads).
- A row with every column masked gives zeros; mask planes broadcast over
  heads (plane h % mask_heads).
- The softcap's place (inside the scale, before the mask) follows ggml's
  published flash_attn_ext; no reference test holds a softcapped
  attention, so that order is parity unpinned (checked against a numpy
  statement only).
"""
import math

import numpy as np

from oracle import core, kvpool as kp


def test_flash_attn_with_fill_blocks_mask_equals_paged_attention(oracle_lib):
    rng = np.random.default_rng(1)
    H, Hkv, D, B, cap = 8, 2, 32, 64, 1024
    pool = kp.Pool(cap // B, B)
    seqs = [kp.Seq(pool) for _ in range(3)]
    seq_n, npast = [1, 7, 3], [130, 60, 0]
    for s, n, p in zip(seqs, seq_n, npast):
        kp.reserve(s, 40)
    for s, n, p in zip(seqs, seq_n, npast):
        kp.reserve(s, n + p)
    bt = np.full((3, max(len(s.blocks) for s in seqs)), -1, np.int32)
    for i, s in enumerate(seqs):
        bt[i, :len(s.blocks)] = s.blocks
    kpool = core.f32_to_f16_bits(rng.standard_normal((cap, Hkv * D)).astype(np.float32))
    vpool = core.f32_to_f16_bits(rng.standard_normal((cap, Hkv * D)).astype(np.float32))
    N = sum(seq_n)
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    b = core.BatchDesc(seq_n, npast, bt, B, np.zeros(N, np.int32), [])
    want = core.paged_attention(q, kpool, vpool, H, Hkv, D, 0.17, b)
    off = 0
    for i, (n, p) in enumerate(zip(seq_n, npast)):
        mask = kp.fill_blocks(n, cap, p, B, list(seqs[i].blocks))
        m16 = core.f32_to_f16_bits(mask)
        qh = np.ascontiguousarray(q[off:off + n].transpose(1, 0, 2))  # (H, n, D)
        got = core.flash_attn(qh, kpool, vpool, Hkv, m16, 0.17, k_strides=(Hkv * D, D),
                              v_strides=(Hkv * D, D), n_kv=cap)
        np.testing.assert_allclose(got, want[off:off + n], rtol=1e-6, atol=1e-7)
        off += n


def paper_slopes(n_heads, max_bias=8.0):
    """ALiBi (Press et al., get_slopes): for a power of two n, the geometric
    sequence start = 2^(-max_bias / n), slope_i = start^(i+1); otherwise the
    slopes of the closest power of two, then every other slope of twice
    that many heads."""
    def pow2(n):
        start = 2.0 ** (-max_bias / n)
        return [start ** (i + 1) for i in range(n)]
    if math.log2(n_heads).is_integer():
        return pow2(n_heads)
    c = 2 ** math.floor(math.log2(n_heads))
    return pow2(c) + pow2(2 * c)[0::2][:n_heads - c]


def test_alibi_slopes_match_the_paper(oracle_lib):
    H, D, n_kv = 12, 8, 4
    q = np.zeros((H, 1, D), np.float32)  # scores 0: s_j = slope * mask_j
    k = np.zeros((1, n_kv, D), np.uint16)
    v = np.zeros((1, n_kv, D), np.float32)
    v[0, :, 0] = [1, 0, 0, 0]
    v[0, :, 1] = [0, 1, 0, 0]
    mvals = np.array([[0.0, -1.0, -2.0, -3.0]], np.float32)
    got = core.flash_attn(q, k, core.f32_to_f16_bits(v), 1, core.f32_to_f16_bits(mvals),
                          1.0, max_bias=8.0)
    # w1 / w0 = exp(-slope)
    slopes = -np.log(got[0, :, 1].astype(np.float64) / got[0, :, 0])
    np.testing.assert_allclose(slopes, paper_slopes(H), rtol=1e-5)


def np_flash(q, k, v, mask, scale, softcap, G):
    H, T, D = q.shape
    out = np.zeros((T, H, D))
    for h in range(H):
        for t in range(T):
            s = scale * (k[h // G].astype(np.float64) @ q[h, t].astype(np.float64))
            if softcap > 0:
                s = softcap * np.tanh(s / softcap)
            m = mask[h % mask.shape[0], t].astype(np.float64)
            keep = np.isfinite(m)
            if not keep.any():
                continue
            s = np.where(keep, s + m, -np.inf)
            w = np.exp(s - s[keep].max())
            out[t, h] = (w / w.sum()) @ v[h // G].astype(np.float64)
    return out


def test_softcap_broadcast_and_fully_masked_rows(oracle_lib):
    rng = np.random.default_rng(2)
    H, Hkv, T, D, n_kv = 4, 2, 5, 16, 37
    q = (rng.standard_normal((H, T, D)) * 3).astype(np.float32)
    kf = rng.standard_normal((Hkv, n_kv, D)).astype(np.float16)
    vf = rng.standard_normal((Hkv, n_kv, D)).astype(np.float16)
    mask = rng.standard_normal((2, T + 2, n_kv)).astype(np.float16)
    mask[rng.random(mask.shape) < 0.3] = -np.inf
    mask[1, 3, :] = -np.inf  # row 3 of plane 1: heads 1, 3 see nothing
    for softcap in (0.0, 5.0):
        got = core.flash_attn(q, kf.view(np.uint16), vf.view(np.uint16), Hkv,
                              mask.view(np.uint16), 0.4, softcap=softcap)
        want = np_flash(q, kf, vf, mask, 0.4, softcap, H // Hkv)
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
        assert not got[3, 1].any() and not got[3, 3].any() and got[3, 0].any()
