"""Pins the oracle's f16 conversion, RNGs and quantized block formats.

f16: numpy's IEEE round-to-nearest-even conversion on a sweep of f32 bit
patterns. Q4_K / Q6_K / Q8_0: hand-built blocks whose values follow the
public block layout (stated in each test), the Q8_0 bytes of the
reference's writer test (test_convert.lua:322-335: 1.5 x 64), and the
quantize->dequantize rmse bounds of test_convert.lua:287-310.
"""
import struct

import numpy as np

from oracle import core


def test_f16_matches_numpy_rne(oracle_lib):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    # plus the edge cases: subnormal boundary, ties, overflow, inf/nan, zero
    extra = np.array([0, 0x80000000, 0x33000000, 0x33000001, 0x32ffffff, 0x387fc000,
                      0x38800000, 0x477fe000, 0x477fefff, 0x477ff000, 0x7f800000, 0xff800000,
                      0x3f800000, 0x3f801000, 0x3f803000, 0x3f802fff],
                     np.uint32)
    bits = np.concatenate([bits, extra])
    f = bits.view(np.float32)
    want = f.astype(np.float16).view(np.uint16)
    got = core.f32_to_f16_bits(f)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7c00) == 0x7c00) and np.all((got[nan] & 0x3ff) != 0)
    # f16 -> f32 is exact for every f16 value
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    fh = core.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(fh[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_lcg_sequence(oracle_lib):
    # x <- x * 6364136223846793005 + 1442695040888963407 mod 2^64; u = (x >> 11) / 2^53
    r = core.Lcg(12345)
    x = 12345
    for _ in range(1000):
        x = (x * 6364136223846793005 + 1442695040888963407) % 2**64
        assert r.next() == (x >> 11) / 2.0**53


# splitmix64's published outputs (Vigna's splitmix64.c, the generator that
# seeds xoshiro): seed 1234567 and seed 0 (0xe220a8397b1dcdaf first).
SPLITMIX_1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                    4593380528125082431, 16408922859458223821]
SPLITMIX_0 = [0xe220a8397b1dcdaf]


def test_splitmix64_published_vectors(oracle_lib):
    assert core.splitmix64(1234567, 5) == SPLITMIX_1234567
    assert core.splitmix64(0, 1) == SPLITMIX_0


def test_fill_normal_is_box_muller_of_the_draws(oracle_lib):
    # tensor:fill("normal", mean, sd, seed) (src/lgml.c:3130-3136): value i
    # takes draws 2i+1, 2i+2 as u = (draw >> 11) / 2^53 and is
    # mean + sd sqrt(-2 ln u1) cos(2 pi u2), in double, stored as f32.
    # The draws come from the splitmix64 pinned above; math.log / math.cos
    # (the platform libm) give the closed form.
    import math
    for seed, mean, sd in ((1234567, 0.0, 0.02), (0, 1.5, 3.0), (20261201, -0.25, 1.0)):
        n = 64
        draws = core.splitmix64(seed, 2 * n)
        got = core.fill_normal(n, mean, sd, seed)
        par = core.gen_normal(n, mean, sd, seed)
        for i in range(n):
            u1 = (draws[2 * i] >> 11) / 2.0**53
            u2 = (draws[2 * i + 1] >> 11) / 2.0**53
            want = np.float32(mean + sd * math.sqrt(-2.0 * math.log(u1 if u1 > 0 else 1e-300)) *
                              math.cos(6.283185307179586 * u2))
            assert got[i] == want, (seed, i)
            assert par[i] == want, (seed, i)  # the parallel generator: same values


def test_splitmix_normal_statistics(oracle_lib):
    v = core.fill_normal(200_000, 0.0, 0.02, 99)
    assert abs(float(v.mean())) < 2e-4
    assert abs(float(v.std()) - 0.02) < 2e-4
    u = core.fill_uniform(200_000, -1.0, 1.0, 5)
    assert -1 <= u.min() and u.max() < 1 and abs(float(u.mean())) < 1e-2


def f16(x):
    return struct.unpack("<H", np.float16(x).tobytes())[0]


def test_q4k_hand_block(oracle_lib):
    # Q4_K: {f16 d, f16 dmin, 12 scale bytes, 128 qs}. Groups g = v // 32;
    # groups 0..3 take scale s[g] & 63 and min s[g+4] & 63; groups 4..7
    # take scale (s[g+4] & 15) | (s[g-4] >> 6) << 4 and min
    # (s[g+4] >> 4) | (s[g] >> 6) << 4. Value v's 4-bit q is in byte
    # 32 * (v // 64) + v % 32, low nibble when v % 64 < 32.
    d, dmin = 0.5, 0.25
    sc = [1, 2, 3, 63, 17, 33, 48, 5]
    mn = [0, 7, 1, 2, 20, 40, 0, 63]
    s = [0] * 12
    for g in range(4):
        s[g] = sc[g] | ((sc[g + 4] >> 4) << 6)
        s[g + 4] = mn[g] | ((mn[g + 4] >> 4) << 6)
        s[g + 8] = (sc[g + 4] & 15) | ((mn[g + 4] & 15) << 4)
    qs = bytes(((b * 7) % 16) | (((b * 5 + 3) % 16) << 4) for b in range(128))
    blk = struct.pack("<HH", f16(d), f16(dmin)) + bytes(s) + qs
    got = core.dequantize(core.Q4_K, np.frombuffer(blk, np.uint8), 256)[0]
    want = []
    for v in range(256):
        g, byte = v // 32, qs[32 * (v // 64) + v % 32]
        q = byte & 15 if v % 64 < 32 else byte >> 4
        want.append(np.float32(d * sc[g]) * np.float32(q) - np.float32(dmin * mn[g]))
    assert np.array_equal(got, np.array(want, np.float32))


def test_q6k_hand_block(oracle_lib):
    # Q6_K: {ql[128], qh[64], i8 scales[16], f16 d}. Value v: half h = v // 128,
    # r = v % 128, quarter t = r // 32, l = r % 32; low 4 bits in
    # ql[64h + l + 32 * (t & 1)] (low nibble for t < 2), high 2 bits in
    # qh[32h + l] >> 2t; q = bits - 32; y = d * scales[v // 16] * q.
    d = 0.125
    ql = bytes((b * 11 + 1) % 256 for b in range(128))
    qh = bytes((b * 29 + 7) % 256 for b in range(64))
    scales = [(-1) ** i * (i * 9 % 128) for i in range(16)]
    blk = ql + qh + struct.pack("<16b", *scales) + struct.pack("<H", f16(d))
    got = core.dequantize(core.Q6_K, np.frombuffer(blk, np.uint8), 256)[0]
    want = []
    for v in range(256):
        h, r = v // 128, v % 128
        t, l = r // 32, r % 32
        lo = ql[64 * h + l + 32 * (t & 1)]
        lo = lo & 15 if t < 2 else lo >> 4
        hb = (qh[32 * h + l] >> (2 * t)) & 3
        q = (lo | (hb << 4)) - 32
        want.append(np.float32(np.float32(d) * np.float32(scales[v // 16])) * np.float32(q))
    assert np.array_equal(got, np.array(want, np.float32))


def test_q8_0_writer_bytes(oracle_lib):
    # test_convert.lua:322-335 quantizes 64 values of 1.5 to q8_0: two
    # blocks {f16 d = 1.5 / 127, 32 x int8 127}.
    q = core.quantize(core.Q8_0, np.full((1, 64), 1.5, np.float32))[0].tobytes()
    blk = struct.pack("<H", f16(1.5 / 127)) + bytes([127] * 32)
    assert q == blk * 2
    back = core.dequantize(core.Q8_0, np.frombuffer(q, np.uint8), 64)[0]
    assert np.all(np.abs(back - 1.5) < 0.02)


def test_roundtrip_rmse_bounds(oracle_lib):
    # test_convert.lua:287 BOUND = { q8_0 = 0.01, q6_K = 0.02, q4_K = 0.08 } (rmse / rms)
    x = core.fill_normal(64 * 4096, 0.0, 0.02, 3).reshape(64, 4096)
    rms = float(np.sqrt(np.mean(x.astype(np.float64) ** 2)))
    for t, bound in ((core.Q8_0, 0.01), (core.Q6_K, 0.02), (core.Q4_K, 0.08)):
        back = core.dequantize(t, core.quantize(t, x), 4096)
        rmse = float(np.sqrt(np.mean((back.astype(np.float64) - x) ** 2)))
        assert rmse / rms < bound, (t, rmse / rms)
        assert core.row_size(t, 4096) == {core.Q8_0: 128 * 34, core.Q6_K: 16 * 210,
                                          core.Q4_K: 16 * 144}[t]


def test_mul_mat_matches_numpy(oracle_lib):
    x = core.fill_normal(5 * 512, 0, 1, 11).reshape(5, 512)
    for t in (core.F32, core.Q4_K, core.Q6_K, core.Q8_0):
        wf = core.fill_normal(48 * 512, 0, 0.02, 12).reshape(48, 512)
        w = wf if t == core.F32 else core.quantize(t, wf)
        deq = wf if t == core.F32 else core.dequantize(t, w, 512)
        y = core.mul_mat(t, w, 48, 512, x)
        ref = (x.astype(np.float64) @ deq.astype(np.float64).T)
        assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)
