"""The native KV pool (lgmlh_kvpool_*, lgml_amd.kvpool) against the reference's
known answers (test/test_kvpool.lua:55-132) and, step by step, against the
oracle restatement of lua/lgml/kvpool.lua on seeded random operation
sequences. Host code: runs without a GPU."""
import hashlib
import random

import pytest

from oracle import kvpool as okp

pytest.importorskip("torch")


@pytest.fixture(scope="module")
def nkp():
    from lgml_amd import kvpool
    return kvpool


def test_block_key_is_sha256_of_joined_tokens(nkp):
    toks = [101, 102, 103, 104]
    assert nkp.key("r", toks, 1, 4) == hashlib.sha256(b"r,101,102,103,104").hexdigest()
    assert nkp.key("r", toks, 2, 2) == hashlib.sha256(b"r,102,103").hexdigest()
    parent = hashlib.sha256(b"x").hexdigest()
    assert nkp.key(parent, [-5, 0, 7]) == hashlib.sha256((parent + ",-5,0,7").encode()).hexdigest()
    assert nkp.key("r", []) == hashlib.sha256(b"r").hexdigest()


def test_native_pool_known_answers(nkp):
    # test_kvpool.lua:55-132, as tests/test_oracle_kvpool.py restates them.
    a = nkp.Pool(8, 4)
    toks = [100 + i for i in range(1, 13)]

    def chain(root, lst, t):
        parent = root
        for i, b in enumerate(lst, 1):
            k = nkp.key(parent, t, (i - 1) * 4 + 1, 4)
            assert a.publish(b, k, parent, i, t[(i - 1) * 4:i * 4])
            parent = k
        return parent

    A = [a.take(), a.take(), a.take()]
    B = [a.take(), a.take()]
    assert A + B == [0, 1, 2, 3, 4]
    chain("r", A, toks)
    chain("r", B, [7, 7, 7, 7, 8, 8, 8, 8])
    assert a.lookup(nkp.key("r", toks, 1, 4)) == A[0]
    assert not a.publish(a.take(), nkp.key("r", toks, 1, 4), "r", 1, [])
    a.unref(5)
    for b in reversed(A):
        a.unref(b)
    for b in reversed(B):
        a.unref(b)
    assert a.used == 0 and a.cached == 5
    kid, part = a.longest_kid(nkp.key("r", toks, 1, 4), [105, 106, 0], 1, 3)
    assert kid == A[1] and part == 2
    hit = a.lookup(nkp.key("r", toks, 1, 4))
    a.ref(hit)
    assert a.cached == 4 and a.used == 1
    a.unref(hit)
    assert [a.take(), a.take(), a.take()] == [5, 6, 7], "free blocks go before cached ones"
    assert a.take() is None
    order = [a.evict() for _ in range(5)]
    assert order == [A[2], A[1], B[1], B[0], A[0]]
    assert a.evict() is None and a.cached == 0 and a.lookup(nkp.key("r", toks, 1, 4)) is None
    for b in order:
        a.unref(b)
    assert [a.take(3), a.take(3), a.take(3)] == [3, 4, 0], "take prefers blocks from min up"
    p = nkp.Pool(3, 4)
    hi, lo, mid = p.take(), p.take(), p.take()
    p.publish(hi, "h" * 64, "r", 1, [], nkp.HIGH)
    p.publish(lo, "1" * 64, "r", 1, [], nkp.LOW)
    p.publish(mid, "2" * 64, "r", 1, [], nkp.NORMAL)
    p.unref(hi)
    p.unref(mid)
    p.unref(lo)
    assert [p.evict(), p.evict(), p.evict()] == [lo, mid, hi]
    # ref raises the priority (kvpool.lua:165-178): a LOW block referenced
    # at HIGH outlives a NORMAL one
    q = nkp.Pool(2, 4)
    s1, s2 = q.take(), q.take()
    q.publish(s1, "3" * 64, "r", 1, [], nkp.LOW)
    q.publish(s2, "4" * 64, "r", 1, [], nkp.NORMAL)
    q.ref(s1, nkp.HIGH)
    q.unref(s1)
    q.unref(s1)
    q.unref(s2)
    assert [q.evict(), q.evict()] == [s2, s1]
    assert [nkp.default_seqs(1000, f) for f in (0, 50, 100, 900)] == [4, 4, 2, 1]


def _key(i):
    return hashlib.sha256(b"k%d" % i).hexdigest()


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_native_pool_follows_the_oracle(nkp, seed):
    rng = random.Random(seed)
    n = 24
    o, nat = okp.Pool(n, 4), nkp.Pool(n, 4)
    parents = ["root"] + [_key(i) for i in range(8)]
    nkeys = 0
    for step in range(3000):
        op = rng.choice(["take", "take_min", "evict", "ref", "unref", "unref", "publish",
                         "part", "lookup", "kid", "cap"])
        held = sorted(o.refs)
        cached = sorted(b for b in o.keys if b not in o.refs)
        if op == "take":
            assert nat.take() == o.take(), step
        elif op == "take_min":
            m = rng.randrange(n)
            assert nat.take(m) == o.take(m), step
        elif op == "evict":
            # victim names the block evict takes (the on_evict moment)
            v = nat.victim()
            got = nat.evict()
            assert got == o.evict(), step
            assert (v[0] if v else None) == got, step
        elif op == "ref" and (held or cached):
            b = rng.choice(held + cached)
            pr = rng.choice([nkp.LOW, nkp.NORMAL, nkp.HIGH])
            o.ref(b, pr)
            nat.ref(b, pr)
        elif op == "unref" and held:
            b = rng.choice(held)
            o.unref(b)
            nat.unref(b)
        elif op == "publish" and held:
            b = rng.choice(held)
            parent = rng.choice(parents)
            if rng.random() < 0.3 and o.bykey:
                k = rng.choice(sorted(o.bykey))  # a key already taken
            else:
                k = _key(1000 + nkeys)
                nkeys += 1
            toks = [rng.randrange(5) for _ in range(4)]
            pr = rng.choice([nkp.LOW, nkp.NORMAL, nkp.HIGH])
            depth = rng.randrange(1, 6)
            assert nat.publish(b, k, parent, depth, toks, pr) == o.publish(b, k, parent, depth, toks, pr), step
            if len(parents) < 40 and rng.random() < 0.5:
                parents.append(k)
        elif op == "part" and held:
            b = rng.choice(held)
            parent = rng.choice(parents)
            toks = [rng.randrange(5) for _ in range(rng.randrange(0, 4))]
            assert nat.publish_part(b, parent, 1, toks) == o.publish_part(b, parent, 1, toks), step
        elif op == "lookup" and o.bykey:
            k = rng.choice(sorted(o.bykey) + [_key(99999)])
            assert nat.lookup(k) == o.lookup(k), step
        elif op == "kid":
            parent = rng.choice(parents)
            toks = [rng.randrange(5) for _ in range(6)]
            assert nat.longest_kid(parent, toks, 1, 4) == o.longest_kid(parent, toks, 1, 4), step
        elif op == "cap" and rng.random() < 0.1:
            c = rng.randrange(n // 2, n + 1)
            o.set_cap(c)
            nat.set_cap(c)
        assert (nat.used, nat.cached, nat.cap) == (o.used, o.cached, o.cap), (step, op)
        for b in range(n):
            assert nat.refs_of(b) == o.refs_of(b), (step, op, b)
            kn, ko = nat.key_of(b), o.key_of(b)
            assert kn == ko, (step, op, b)
