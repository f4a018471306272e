"""Block-table parity of the engine's pool sequences (lgml_amd.engine.PoolSeqs
over the native pool) against the oracle's restatement of transformer.lua's
pool helpers (oracle/kvpool.py): new_block :934-958, reserve :963-981,
truncate :1084-1108 (copy-on-write of a shared or keyed partial block),
share :1116-1123, free_seq :784-803, with publish / eviction of
kvpool.lua.

One seeded stream of operations (reference LCG, test/tiny.lua:16-22) runs
on both sides; after every operation the block table of every sequence,
the refcount and key of every block, the pool's used count, the
copy-on-write copies (src, dst, cells) and any "kv pool full" must be
identical. The oracle pool is pinned by the kvpool KATs
(tests/test_oracle_kvpool.py); this runs on the CPU (no device call: the
block copies are recorded, not made).
"""
import pytest

from oracle import core, kvpool as okp

B = 64


class _Model:
    """What PoolSeqs reads of a device model: the pool's size."""

    def __init__(self, blocks):
        self.pool_blocks = blocks
        self.n_cells = blocks * B
        self.hp = {"n_head_kv": 1, "head_dim": 8}


def _engine_side(blocks):
    from lgml_amd import engine
    ps = engine.PoolSeqs(_Model(blocks))
    copies = []
    ps.copy_block = lambda src, dst, n: copies.append((src, dst, n))
    return engine, ps, copies


@pytest.mark.parametrize("seed,blocks", [(11, 24), (12, 40), (13, 9), (14, 64)])
def test_pool_seqs_follow_the_oracle(seed, blocks):
    engine, ps, e_copies = _engine_side(blocks)
    opool = okp.Pool(blocks, B)
    o_copies = []
    ocopy = lambda src, dst, n: o_copies.append((src, dst, n))  # noqa: E731
    rng = core.Lcg(seed)

    def ri(lo, hi):  # U[lo, hi]
        return lo + int(rng.next() * (hi - lo + 1))

    eseqs, oseqs, toks = [], [], []
    full = [0, 0]

    def both(fe, fo):
        """Run one operation on both sides; both raise PoolFull or neither."""
        re = ro = None
        try:
            fe()
        except engine.PoolFull as e:
            re = e
        try:
            fo()
        except okp.PoolFull as e:
            ro = e
        assert (re is None) == (ro is None), (re, ro)
        if re is not None:
            full[0] += 1

    def check():
        pairs = [(a, b) for a, b in zip(eseqs, oseqs) if a is not None]
        assert [a.blocks for a, _ in pairs] == [b.blocks for _, b in pairs]
        assert [a.n_past for a, _ in pairs] == [b.n_past for _, b in pairs]
        assert [a.keys for a, _ in pairs] == [b.keys for _, b in pairs]
        for b in range(blocks):
            assert ps.alloc.refs_of(b) == opool.refs_of(b), b
            assert ps.alloc.key_of(b) == opool.key_of(b), b
        assert ps.alloc.used == opool.used
        assert ps.alloc.evicted == opool.stats["evicted"]
        assert e_copies == o_copies

    for step in range(600):
        op = ri(0, 9)
        live = [i for i in range(len(eseqs)) if eseqs[i] is not None]
        if op <= 1 or not live:
            prio = ri(0, 2)
            eseqs.append(engine.Seq(ps, prio))
            oseqs.append(okp.Seq(opool, prio))
            toks.append([ri(0, 50) for _ in range(ri(1, 6) * B + ri(0, B - 1))])
        elif op <= 4:  # grow (a prompt chunk or decode steps)
            i = live[ri(0, len(live) - 1)]
            n = min(eseqs[i].n_past + ri(1, 200), len(toks[i]) + 300)
            both(lambda: ps.reserve(eseqs[i], n), lambda: okp.reserve(oseqs[i], n))
            if len(eseqs[i].blocks) * B >= n:
                eseqs[i].n_past = oseqs[i].n_past = n
        elif op == 5:  # publish the full prompt blocks (E:publish)
            i = live[ri(0, len(live) - 1)]
            c, oc = eseqs[i], oseqs[i]
            upto = min(c.n_past, len(toks[i])) // B
            for j in range(len(c.keys) + 1, upto + 1):
                parent = c.keys[j - 2] if j >= 2 else "lgml:"
                k = okp.key(parent, toks[i], (j - 1) * B + 1, B)
                t = toks[i][(j - 1) * B:j * B]
                c.keys.append(k)
                oc.keys.append(k)
                assert (ps.alloc.publish(c.blocks[j - 1], k, parent, j, t, c.prio) ==
                        opool.publish(oc.blocks[j - 1], k, parent, j, t, oc.prio))
        elif op == 6:  # a new sequence shares another's keyed prefix blocks
            i = live[ri(0, len(live) - 1)]
            nk = len(eseqs[i].keys)
            if nk:
                m = ri(1, nk)
                prio = ri(0, 2)
                eseqs.append(engine.Seq(ps, prio))
                oseqs.append(okp.Seq(opool, prio))
                toks.append(list(toks[i][:m * B]) + [ri(0, 50) for _ in range(ri(1, 100))])
                ps.share(eseqs[-1], eseqs[i].blocks[:m], eseqs[i].keys[:m])
                okp.share(oseqs[-1], oseqs[i].blocks[:m], oseqs[i].keys[:m])
        elif op <= 8:  # truncate (a rewind; CoW when the block is shared or keyed)
            i = live[ri(0, len(live) - 1)]
            n = ri(0, eseqs[i].n_past)
            both(lambda: ps.truncate(eseqs[i], n), lambda: okp.truncate(oseqs[i], n, ocopy))
        else:  # free_seq
            i = live[ri(0, len(live) - 1)]
            ps.free(eseqs[i])
            okp.truncate(oseqs[i], 0, ocopy)
            eseqs[i] = oseqs[i] = None
        check()
    assert len(e_copies) > 0, "the stream never copied a shared partial block"
    assert full[0] > 0 or blocks >= 40, "the small pools should fill"
    assert ps.alloc.evicted > 0 or blocks >= 40, "the small pools should evict cached blocks"
