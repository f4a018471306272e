"""The run-ahead engine (Engine(run_ahead=True), the mode bench.py runs):
each step queues the next pass before reading back the previous one, and a
decode token goes from one pass to the next on the device (copied into the
next plan's ids). Joining requests start one pass later than with the
synchronous engine, so the passes are batched differently; every request
must still sample the same tokens with the same logits, bit for bit (a
sequence's results do not depend on its batch), and end after exactly its
budget. Covered: prompt chunks mixed into decode passes, budgets that end
requests at different passes, slots taken by queued requests, prefix
sharing (blocks published as their pass is read back), and a model with
sliding-window rings (the ring plan's ids take the device tokens too); and
the same with each pass run as two halves at once on two streams (a half's
decode tokens may come from either half of the previous pass).
"""
import numpy as np
import pytest

from oracle import models
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def serve(gm, prompts, budgets, n_slots, run_ahead, ubatch=64, prefix_cache=False, streams=1,
          expect_err=()):
    """All requests through one engine, queued ones joining as slots free;
    per request its (token, logits) samples in order. Requests whose index
    is in expect_err must end with "kv pool full"."""
    from lgml_amd import engine
    eng = engine.Engine(gm, n_slots, ubatch=ubatch, prefix_cache=prefix_cache,
                        run_ahead=run_ahead, streams=streams)
    reqs = [engine.Request(p, b) for p, b in zip(prompts, budgets)]
    queue = list(reqs)
    got = {id(r): [] for r in reqs}

    def record(done):
        if not done:
            return
        lg = eng.last_logits.cpu().numpy()
        for i, r in enumerate(eng.last_entries):
            if r in done:
                got[id(r)].append((r.out[-1], lg[i].copy()))

    passes = 0
    while queue or eng.active or eng.waiting:
        while queue and len(eng.active) < n_slots:
            eng.submit(queue.pop(0))
        record(eng.step())
        passes += 1
        assert passes < 1000
    record(eng.drain())
    for i, r in enumerate(reqs):
        if i in expect_err:
            assert r.done and r.err and "kv pool full" in r.err, r.err
        else:
            assert r.done and r.err is None and len(r.out) == r.max_new, (r.err, len(r.out))
    return [got[id(r)] for i, r in enumerate(reqs) if i not in expect_err]


def same(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert len(x) == len(y)
        for (ta, la), (tb, lb) in zip(x, y):
            assert ta == tb
            assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))


def test_run_ahead_equals_sync_with_joins_and_prefix_sharing():
    from lgml_amd import runtime
    hp, w = models.build("c2", seed=11, n_layer=2, init="normal")
    V = hp["n_vocab"]
    prefix = lcg_ints(6000, 130, 0, V)
    prompts = [lcg_ints(6001, 150, 0, V), prefix + lcg_ints(6002, 20, 0, V),
               lcg_ints(6003, 5, 0, V), prefix + lcg_ints(6004, 70, 0, V),
               lcg_ints(6005, 1, 0, V), prefix[:90] + lcg_ints(6006, 9, 0, V)]
    budgets = [7, 3, 12, 1, 5, 4]
    for pc in (False, True):
        print("run-ahead vs sync, prefix_cache=%s" % pc, flush=True)
        a = serve(runtime.DeviceModel(hp, w, 64 * 64), prompts, budgets, 3, False,
                  prefix_cache=pc)
        b = serve(runtime.DeviceModel(hp, w, 64 * 64), prompts, budgets, 3, True,
                  prefix_cache=pc)
        same(a, b)
        print("run-ahead on two streams vs sync, prefix_cache=%s" % pc, flush=True)
        c = serve(runtime.DeviceModel(hp, w, 64 * 64), prompts, budgets, 3, True,
                  prefix_cache=pc, streams=2)
        same(a, c)


def test_run_ahead_equals_sync_with_rings():
    from lgml_amd import runtime
    shape = dict(models.SHAPES["c4"], n_layer=2, swa_period=2, n_swa=100)
    hp, w = models.build(shape, seed=12, init="normal")
    V = hp["n_vocab"]
    prompts = [lcg_ints(6100 + i, n, 0, V) for i, n in enumerate([3, 90, 140, 17])]
    budgets = [6, 2, 5, 9]
    R = 3  # (n_swa - 1 + ubatch) / 64 blocks per slot
    print("run-ahead vs sync, rings", flush=True)
    a = serve(runtime.DeviceModel(hp, w, 2048, ring_cells=2 * R * 64), prompts, budgets, 2,
              False)
    b = serve(runtime.DeviceModel(hp, w, 2048, ring_cells=2 * R * 64), prompts, budgets, 2,
              True)
    same(a, b)
    print("run-ahead on two streams vs sync, rings", flush=True)
    c = serve(runtime.DeviceModel(hp, w, 2048, ring_cells=2 * R * 64), prompts, budgets, 2,
              True, streams=2)
    same(a, c)


def test_run_ahead_pool_full_mid_prompt():
    """A prompt longer than the pool waits while other requests run (its
    earlier chunks may still be in flight when the pool fills) and, once
    alone, ends with "kv pool full" (engine.lua:2229-2234); the other
    requests sample as with the synchronous engine."""
    from lgml_amd import runtime
    hp, w = models.build("c2", seed=13, n_layer=2, init="normal")
    V = hp["n_vocab"]
    prompts = [lcg_ints(6200, 100, 0, V), lcg_ints(6201, 800, 0, V), lcg_ints(6202, 30, 0, V)]
    budgets = [5, 3, 6]
    print("run-ahead vs sync, a prompt longer than the pool", flush=True)
    a = serve(runtime.DeviceModel(hp, w, 12 * 64), prompts, budgets, 2, False, expect_err=(1,))
    b = serve(runtime.DeviceModel(hp, w, 12 * 64), prompts, budgets, 2, True, expect_err=(1,))
    same(a, b)
