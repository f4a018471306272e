"""C3: prefix sharing through the engine.

Requests that start with a prompt already in the pool attach its cached
blocks (E:attach_blocks, lua/lgml/engine.lua:2038-2077): full blocks are
shared with a reference count, the best partial match is copied, only the
rest of the prompt runs, in chunks mixed into the decode passes. Every
request must sample the same tokens with the same logits, bit for bit, as
without sharing (the shared KV is what the request would have computed:
the pass is batch invariant).
"""
import numpy as np
import pytest

from oracle import models
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def run(hp, w, prompts, prefix_cache, n_samples=4, ubatch=64):
    from lgml_amd import engine, runtime
    gm = runtime.DeviceModel(hp, w, 64 * 64)
    eng = engine.Engine(gm, len(prompts), ubatch=ubatch, prefix_cache=prefix_cache)
    reqs = [engine.Request(p, 10 ** 6) for p in prompts]
    got = {id(r): [] for r in reqs}
    info = {}

    def step():
        done = eng.step()
        lg = eng.last_logits.cpu().numpy()
        for i, r in enumerate(eng.last_entries):
            if r in done:
                got[id(r)].append((r.out[-1], lg[i].copy()))

    eng.submit(reqs[0])
    while reqs[0].fed < len(reqs[0].prompt):  # the first prompt runs alone and publishes
        step()
    for r in reqs[1:]:
        eng.submit(r)
    info["fed_at_submit"] = [r.fed for r in reqs[1:]]
    info["refs"] = [eng.seqs.alloc.refs_of(b) for b in reqs[0].seq.blocks[:2]]
    while min(len(got[id(r)]) for r in reqs) < n_samples:
        step()
    info["hit_blocks"] = eng.hit_blocks
    return [got[id(r)][:n_samples] for r in reqs], info


def test_c3_prefix_sharing_is_bit_exact_with_unshared():
    hp, w = models.build("c2", seed=5, n_layer=2, init="normal")
    V = hp["n_vocab"]
    prefix = lcg_ints(5000, 130, 0, V)
    prompts = [prefix + lcg_ints(5001, 40, 0, V),
               prefix + lcg_ints(5002, 70, 0, V),
               prefix[:100] + lcg_ints(5003, 25, 0, V),
               prefix + lcg_ints(5004, 3, 0, V)]
    shared, info = run(hp, w, prompts, True)
    plain, info0 = run(hp, w, prompts, False)
    # r1, r3 share the 2 full prefix blocks; r2 shares block 1 and copies the
    # 36 cells of block 2 it has in common (longest_kid over r0's block 2)
    assert info["fed_at_submit"] == [128, 100, 128], info
    assert info["refs"] == [4, 3], info
    assert info["hit_blocks"] == 5 and info0["hit_blocks"] == 0
    for a, b in zip(shared, plain):
        for (ta, la), (tb, lb) in zip(a, b):
            assert ta == tb
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
