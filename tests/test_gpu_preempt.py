"""A full pool makes a request wait, not end (test/test_slots.lua:200-256;
E:flush / E:victim / E:preempt, lua/lgml/engine.lua:1193-1243,1410-1448).

C1's tiny llama (f32, vocab 512) on a pool of 12 blocks (768 cells) with 2
slots: a request of a 300-token prompt and one of a 100-token prompt, each
decoding 400 tokens, need 19 blocks together. Expected, as the reference
test states it:
- both replies are whole (400 tokens) and at least one request waited;
- the replies start as the replies alone (the passes are batch invariant,
  so every token before the first wait is the lone run's token; after a
  wait the cells come back through a prefill, which may round differently);
- with the short request at high priority, the normal one waits for it and
  the high one never waits;
- a request alone that outgrows the pool ends with "kv pool full".
"""
import numpy as np
import pytest

from oracle import models
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

N_NEW = 400


@pytest.fixture(scope="module")
def c1():
    return models.build("c1", seed=71)


def prompts(hp):
    V = hp["n_vocab"]
    return lcg_ints(8100, 300, 0, V), lcg_ints(8101, 100, 0, V)


def run(hp, w, reqs_spec, blocks, run_ahead, slots=2):
    from lgml_amd import engine, kvpool, runtime
    gm = runtime.DeviceModel(hp, w, blocks * 64)
    eng = engine.Engine(gm, slots, ubatch=128, run_ahead=run_ahead)
    reqs = [engine.Request(p, N_NEW, prio if prio is not None else kvpool.NORMAL)
            for p, prio in reqs_spec]
    for r in reqs:
        eng.submit(r)
    for _ in range(20 * N_NEW):
        if all(r.done for r in reqs):
            break
        eng.step()
    eng.drain()
    for _ in range(4 * N_NEW):  # a drained engine may still hold waiting requests
        if all(r.done for r in reqs):
            break
        eng.step()
        eng.drain()
    return eng, reqs


def first_diff(a, b):
    k = 0
    while k < min(len(a), len(b)) and a[k] == b[k]:
        k += 1
    return k


@pytest.mark.parametrize("run_ahead", [False, True])
def test_full_pool_makes_a_request_wait(c1, run_ahead):
    hp, w = c1
    pa, pb = prompts(hp)
    alone = []
    for p in (pa, pb):
        _, (r,) = run(hp, w, [(p, None)], 64, run_ahead, slots=1)
        assert r.done and r.err is None and len(r.out) == N_NEW
        alone.append(r.out)
    eng, (ra, rb) = run(hp, w, [(pa, None), (pb, None)], 12, run_ahead)
    print("preemptions %d, waits %s" % (eng.preemptions, eng.waits), flush=True)
    assert ra.done and rb.done and ra.err is None and rb.err is None
    assert len(ra.out) == N_NEW and len(rb.out) == N_NEW
    assert eng.preemptions >= 1
    # the pool fills after about 180 decode steps: everything before is the
    # lone run's, token for token
    assert first_diff(ra.out, alone[0]) >= 150, first_diff(ra.out, alone[0])
    assert first_diff(rb.out, alone[1]) >= 150, first_diff(rb.out, alone[1])
    assert not eng.active and not eng.waiting
    assert eng.seqs.alloc.used == 0  # every block given back


@pytest.mark.parametrize("run_ahead", [False, True])
def test_the_normal_request_waits_for_the_high_one(c1, run_ahead):
    from lgml_amd import kvpool
    hp, w = c1
    pa, pb = prompts(hp)
    eng, (ra, rb) = run(hp, w, [(pa, kvpool.NORMAL), (pb, kvpool.HIGH)], 12, run_ahead)
    print("preemptions %d, waits %s" % (eng.preemptions, eng.waits), flush=True)
    assert len(ra.out) == N_NEW and len(rb.out) == N_NEW and ra.err is None and rb.err is None
    assert eng.waits.get(kvpool.NORMAL, 0) >= 1
    assert eng.waits.get(kvpool.HIGH, 0) == 0
    assert rb.waits == 0 and ra.waits >= 1


@pytest.mark.parametrize("run_ahead", [False, True])
def test_alone_a_full_pool_ends_the_reply(c1, run_ahead):
    hp, w = c1
    pa, _ = prompts(hp)
    eng, (r,) = run(hp, w, [(pa, None)], 8, run_ahead, slots=1)
    assert r.done and r.err is not None and "kv pool full" in r.err
    assert len(r.out) < N_NEW
    assert eng.preemptions == 0
    assert eng.seqs.alloc.used == 0
