"""Pins the pool bookkeeping restatement (oracle/kvpool.py) with the
known-answer tests of the reference: test/test_kvpool.lua:22-52 (fill_blocks
mask on a hand example) and :55-132 (keys, cached blocks, eviction order,
priorities, take(min), default_seqs), plus the block-table invariants of
transformer.lua (reserve sorts new blocks; truncate copy-on-write)."""
import hashlib

import numpy as np
import pytest

from oracle import kvpool as kp


def test_fill_blocks_hand_example():
    # Block size 2: positions 0-1 in block 3 (cells 6, 7), 2-3 in block 1
    # (cells 2, 3). The window starts at cell 0. (test_kvpool.lua:22-52)
    m = kp.fill_blocks(3, 8, n_past=1, block=2, blocks=[3, 1], lo=0)
    want = [{6, 7}, {6, 7, 2}, {6, 7, 2, 3}]
    for r in range(3):
        for c in range(8):
            assert (m[r, c] == 0) == (c in want[r])
            assert m[r, c] == 0 or m[r, c] == -np.inf
    m2 = kp.fill_blocks(3, 8, n_past=1, block=2, blocks=[3, 1], lo=0, causal=False)
    assert m2[0, 2] == 0 and m2[0, 3] == 0
    with pytest.raises(ValueError):
        kp.fill_blocks(3, 8, n_past=1, block=2, blocks=[3])
    with pytest.raises(ValueError):
        kp.fill_blocks(3, 8, n_past=1, block=2, blocks=[3, 1], lo=4)


def test_key_is_sha256_of_joined_tokens():
    toks = [101, 102, 103, 104]
    assert kp.key("r", toks, 1, 4) == hashlib.sha256(b"r,101,102,103,104").hexdigest()
    assert kp.key("r", toks, 1, 4) != kp.key("s", toks, 1, 4)
    assert kp.key("r", toks, 2, 2) == hashlib.sha256(b"r,102,103").hexdigest()


def test_pool_known_answers():
    # test_kvpool.lua:55-132, step by step.
    a = kp.Pool(8, 4)
    toks = [100 + i for i in range(1, 13)]

    def chain(root, lst, t):
        parent = root
        for i, b in enumerate(lst, 1):
            k = kp.key(parent, t, (i - 1) * 4 + 1, 4)
            a.publish(b, k, parent, i, t[(i - 1) * 4:i * 4])
            parent = k
        return parent

    A = [a.take(), a.take(), a.take()]
    B = [a.take(), a.take()]
    chain("r", A, toks)
    chain("r", B, [7, 7, 7, 7, 8, 8, 8, 8])
    assert a.lookup(kp.key("r", toks, 1, 4)) == A[0]
    assert not a.publish(a.take(), kp.key("r", toks, 1, 4), "r", 1, [])
    a.unref(5)
    for b in reversed(A):
        a.unref(b)
    for b in reversed(B):
        a.unref(b)
    assert a.used == 0 and a.cached == 5
    kid, part = a.longest_kid(kp.key("r", toks, 1, 4), [105, 106, 0], 1, 3)
    assert kid == A[1] and part == 2
    hit = a.lookup(kp.key("r", toks, 1, 4))
    a.ref(hit)
    assert a.cached == 4 and a.used == 1
    a.unref(hit)
    got = [a.take(), a.take(), a.take()]
    assert got == [5, 6, 7], "free blocks go before cached ones"
    assert a.take() is None
    order = [a.evict() for _ in range(5)]
    assert order == [A[2], A[1], B[1], B[0], A[0]]
    assert a.evict() is None and a.cached == 0 and a.lookup(kp.key("r", toks, 1, 4)) is None
    for b in order:
        a.unref(b)
    assert [a.take(3), a.take(3), a.take(3)] == [3, 4, 0], "take prefers blocks from min up"
    p = kp.Pool(3, 4)
    hi, lo, mid = p.take(), p.take(), p.take()
    p.publish(hi, "h", "r", 1, [], kp.HIGH)
    p.publish(lo, "l", "r", 1, [], kp.LOW)
    p.publish(mid, "m", "r", 1, [], kp.NORMAL)
    p.unref(hi)
    p.unref(mid)
    p.unref(lo)
    assert [p.evict(), p.evict(), p.evict()] == [lo, mid, hi]
    q = kp.Pool(2, 4)
    s1 = q.take()
    q.publish(s1, "s", "r", 1, [], kp.LOW)
    q.ref(s1, kp.HIGH)
    q.unref(s1)
    q.unref(s1)
    assert q.info[s1]["prio"] == kp.HIGH
    assert [kp.default_seqs(1000, f) for f in (0, 50, 100, 900)] == [4, 4, 2, 1]


def test_reserve_sorts_and_interleaves():
    # Two sequences growing in turns interleave their blocks; each call's
    # new blocks come in cell order (transformer.lua:963-981).
    p = kp.Pool(64, 64)
    a, b = kp.Seq(p), kp.Seq(p)
    for n in range(50, 151, 50):
        kp.reserve(a, n)
        kp.reserve(b, n)
    assert a.blocks == [0, 2, 4] and b.blocks == [1, 3, 5]
    c = kp.Seq(p)
    kp.reserve(c, 64 * 5)
    assert c.blocks == sorted(c.blocks) == [6, 7, 8, 9, 10]
    assert kp.seq_cells(a.blocks, 64, 62, 4) == [62, 63, 128, 129]
    lo, w = kp.seq_window(a.blocks, 64, 150, 64 * 64)
    assert lo == 0 and w == 512


def test_truncate_copy_on_write_and_share():
    p = kp.Pool(16, 4)
    a = kp.Seq(p)
    kp.reserve(a, 10)
    a.n_past = 10
    kb = [p.publish(a.blocks[0], "k1", "r", 1, [1, 2, 3, 4])]
    assert kb == [True]
    b = kp.Seq(p)
    kp.share(b, a.blocks[:2], ["k1", None])
    assert b.n_past == 8 and p.refs_of(a.blocks[1]) == 2
    copies = []
    kp.truncate(b, 6, copy_block=lambda s, d, n: copies.append((s, d, n)))
    # The shared partial block was copied, the keyed first block kept.
    assert copies == [(a.blocks[1], b.blocks[1], 2)] and b.blocks[0] == a.blocks[0]
    assert p.refs_of(a.blocks[1]) == 1 and b.n_past == 6
    kp.truncate(a, 0)
    assert a.blocks == [] and p.key_of(0) == "k1"
