"""C3 against the oracle: sequences on a shared,
refcounted prefix, their suffixes prefilled in chunks mixed into the
decode passes, at the C2 width (d 4096, 32 / 8 heads of 128, FFN 14336,
vocab 128256, Q4_K_M) and 1 layer.

The engine (prefix_cache=True: E:cached_blocks / E:attach_blocks /
E:publish, lua/lgml/engine.lua:1829-1892,2038-2077) runs the passes; the
oracle replays every pass from the engine's own plan (sequence lengths,
positions, block tables, ids, logit rows) on pools of its own, and mirrors
each copy-on-write block copy the engine makes. Every pass's logits must be
within 2e-3 of the oracle's, the greedy ids (the device argmax) identical,
and the prefix blocks must carry the expected reference counts
(test/test_slots.lua:272-316: a shared prefix is referenced by every
sequence on it).
"""
import numpy as np
import pytest

from oracle import core, models
from tests.gpu_util import lcg_ints, oracle_pools, rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def test_c3_shared_prefix_against_oracle():
    from lgml_amd import engine, runtime
    hp, w = models.build("c2", seed=31, n_layer=1, init="normal")
    V = hp["n_vocab"]
    n_cells = 96 * 64
    gm = runtime.DeviceModel(hp, w, n_cells)
    om = core.OracleModel(hp, w)
    kp, vp = oracle_pools(hp, n_cells)
    n_req = 8
    # decode tokens plus at most 64 prompt tokens per pass, in chunks of 64
    eng = engine.Engine(gm, n_req + 1, ubatch=64, prefix_cache=True, max_tokens=n_req + 64)

    # mirror the engine's block copies (the partial prefix block) on the oracle pools
    dev_copy = eng.seqs.copy_block

    def copy_both(src, dst, n):
        dev_copy(src, dst, n)
        for pool in kp + vp:
            pool[dst * 64:dst * 64 + n] = pool[src * 64:src * 64 + n]
    eng.seqs.copy_block = copy_both

    errs, same, n_pass = [], [True], [0]

    def step():
        got = eng.step()
        pl = eng.last_plan
        b = core.BatchDesc(pl.seq_n, pl.seq_npast, pl.block_tab, 64, pl.host_array(
            pl.info.off_ids, pl.info.n_tokens, np.int32), pl.logit_rows)
        lo = om.forward(kp, vp, b)
        lg = eng.last_logits.cpu().numpy()
        errs.append(rel_err(lg, lo))
        sampled = {id(r) for r in got}
        for i, r in enumerate(eng.last_entries):
            if id(r) in sampled:
                same[0] = same[0] and r.out[-1] == core.argmax(lo[i])
        n_pass[0] += 1
        return got

    prefix = lcg_ints(7000, 3 * 64, 0, V)  # 3 full blocks
    r0 = engine.Request(prefix + lcg_ints(7001, 1, 0, V), 1)
    eng.submit(r0)
    while not r0.done:
        step()
    lens = [5 + (17 * i) % 60 for i in range(n_req)]
    reqs = []
    for i in range(n_req):
        if i == 3:
            # shares 2 full blocks and 22 cells of the third: a copy-on-write copy
            p = prefix[:150] + lcg_ints(7100 + i, lens[i], 0, V)
        else:
            p = prefix + lcg_ints(7100 + i, lens[i], 0, V)
        r = engine.Request(p, 4)
        eng.submit(r)
        reqs.append(r)
    fed = [r.fed for r in reqs]
    assert fed == [192 if i != 3 else 150 for i in range(n_req)], fed
    blocks = [r.seq.blocks[:3] for r in reqs]
    shared = [b for b in blocks[0]]
    assert all(bl[:2] == shared[:2] for bl in blocks)
    assert all(bl[2] == shared[2] for i, bl in enumerate(blocks) if i != 3)
    assert blocks[3][2] != shared[2]  # its own copy of the partial block
    refs = [eng.seqs.alloc.refs_of(b) for b in shared]
    assert refs == [n_req, n_req, n_req - 1], refs
    assert eng.hit_blocks == 2 * n_req + (n_req - 1)
    while not all(r.done for r in reqs):
        step()
    assert all(len(r.out) == 4 for r in reqs)
    print("c3: %d passes, max rel err %.3g" % (n_pass[0], max(errs)), flush=True)
    assert max(errs) < 2e-3, errs
    assert same[0]
    # every sequence released its blocks: the prefix blocks are cached (keyed),
    # not referenced
    assert [eng.seqs.alloc.refs_of(b) for b in shared] == [0, 0, 0]
    assert all(eng.seqs.alloc.key_of(b) for b in shared)


def test_c3_at_its_own_shape():
    """C3 at its shape, 1 layer at the C2 attention width: 64 requests on one
    2048-token system prefix (32 keyed blocks, each referenced by every
    sequence on it: refcounts reach 64), suffixes U[16, 512] drawn with the
    bench's LCG and seed, each pass at most 64 decode tokens plus one
    512-token prompt chunk (E:prefill_batched's chunks mixed into the decode
    ubatch, engine.lua:2213-2255). Every pass is replayed on the oracle from
    the engine's own plan: logits within 2e-3 and identical greedy ids."""
    from lgml_amd import engine, runtime, workload
    # the C2 attention width (d 4096, 32 / 8 heads of 128) at 1 layer; an
    # FFN of 1024 and a vocab of 8192 keep the oracle's replay of ~40 passes
    # of up to 576 tokens short (the sharing, chunking and attention do not
    # depend on them)
    hp, w = models.build(dict(models.SHAPES["c2"], n_ff=1024, n_vocab=8192), seed=33,
                         n_layer=1, init="normal")
    V, S, P = hp["n_vocab"], 64, 2048
    rng = workload.Lcg(20261201)
    prefix = [rng.int(0, V - 1) for _ in range(P)]
    suffix = [rng.int(16, 512) for _ in range(S)]
    n_cells = (P + S * (512 + 64) + 4 * 512 + 63) // 64 * 64
    gm = runtime.DeviceModel(hp, w, n_cells)
    om = core.OracleModel(hp, w)
    kp, vp = oracle_pools(hp, n_cells)
    eng = engine.Engine(gm, S + 1, ubatch=512, prefix_cache=True, max_tokens=S + 512)
    errs, same, n_pass, most = [], [True], [0], [0]

    def step():
        got = eng.step()
        pl = eng.last_plan
        ids = pl.host_array(pl.info.off_ids, pl.info.n_tokens, np.int32)
        b = core.BatchDesc(pl.seq_n, pl.seq_npast, pl.block_tab, 64, ids, pl.logit_rows)
        lo = om.forward(kp, vp, b)
        lg = eng.last_logits.cpu().numpy()
        errs.append(rel_err(lg, lo))
        sampled = {id(r) for r in got}
        for i, r in enumerate(eng.last_entries):
            if id(r) in sampled:
                same[0] = same[0] and r.out[-1] == core.argmax(lo[i])
        n_pass[0] += 1
        most[0] = max(most[0], len(ids))
        print("c3 pass %d: %d tokens, %d sequences, rel err %.3g" % (
            n_pass[0], len(ids), len(pl.seq_n), errs[-1]), flush=True)

    r0 = engine.Request(prefix + [rng.int(0, V - 1)], 1)
    eng.submit(r0)
    while not r0.done:
        step()
    reqs = []
    for i in range(S):
        r = engine.Request(prefix + [rng.int(0, V - 1) for _ in range(suffix[i])], 2)
        eng.submit(r)
        reqs.append(r)
    assert all(r.fed == P for r in reqs)  # the whole prefix attached
    shared = reqs[0].seq.blocks[:P // 64]
    assert all(r.seq.blocks[:P // 64] == shared for r in reqs)
    assert [eng.seqs.alloc.refs_of(b) for b in shared] == [S] * (P // 64)
    while not all(r.done for r in reqs):
        step()
    print("c3 at shape: %d passes (up to %d tokens), max rel err %.3g" % (
        n_pass[0], most[0], max(errs)), flush=True)
    assert most[0] > 512  # 512-token chunks beside decode tokens
    assert max(errs) < 2e-3, errs
    assert same[0]
