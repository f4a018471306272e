"""Scheduler corners of the continuous-batching engine (lgml_amd.engine).

- A model with sliding-window rings: a request that lets its cells go
  checkpoints its slot's rings to host memory (E:checkpoint_slot,
  lua/lgml/engine.lua:2103-2116; the rings of M:snapshot,
  transformer.lua:1450-1471) and, when it attaches all of its tokens again,
  restores them into its new slot (M:restore, :1473-1511), so its reply is
  the uninterrupted one token for token; on a full pool it waits instead of
  ending (test/test_slots.lua:200-256).
- A request that ends publishes its reply's blocks (engine.lua:1042-1052,
  E:publish_tail :1906-1918), so a follow-up turn that repeats prompt and
  reply attaches them (E:pick_slot / E:reuse, :1704-1819) and runs only the
  new tokens, with the same tokens as a fresh run.
- The pool starts small and doubles (KV_INITIAL, engine.lua:49; new_block's
  grow branch and pool_grow, transformer.lua:831-958): replies equal those
  on a pool of full size from the start.
"""
import numpy as np
import pytest

from oracle import models
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

# a gemma-style model with a sliding layer (window 64) and a global one
GEMMA_TINY = dict(arch="gemma4", n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64,
                  n_ff=512, n_vocab=512, rope_base=1e6, eps=1e-6, wtype="f32", gemma=True,
                  n_swa=64, swa_period=2, rope_base_swa=1e4, softcap=30.0)
UB = 128
R = (64 - 1 + UB + 63) // 64  # ring blocks per slot for passes of UB tokens


def drive(eng, reqs, limit=20000):
    for _ in range(limit):
        if all(r.done for r in reqs):
            break
        eng.step()
    eng.drain()
    for _ in range(limit):
        if all(r.done for r in reqs):
            break
        eng.step()
        eng.drain()


def gemma_run(hp, w, specs, blocks, slots, preempt_at=None, run_ahead=True):
    """specs: (prompt, n_new); preempt_at: (request index, tokens out) at
    which that request is made to let its cells go."""
    from lgml_amd import engine, runtime
    gm = runtime.DeviceModel(hp, w, blocks * 64, ring_cells=slots * R * 64)
    eng = engine.Engine(gm, slots, ubatch=UB, run_ahead=run_ahead)
    reqs = [engine.Request(p, n) for p, n in specs]
    for r in reqs:
        eng.submit(r)
    done_pre = False
    for _ in range(20000):
        if all(r.done for r in reqs):
            break
        if preempt_at and not done_pre:
            r = reqs[preempt_at[0]]
            if len(r.out) >= preempt_at[1]:
                r.preempt = True  # lets go at the next launch with nothing in flight
                done_pre = True
        eng.step()
    drive(eng, reqs)
    return eng, reqs


def first_diff(a, b):
    k = 0
    while k < min(len(a), len(b)) and a[k] == b[k]:
        k += 1
    return k


@pytest.fixture(scope="module")
def gemma():
    return models.build(GEMMA_TINY, seed=91, init="normal")


def test_ring_model_resumes_with_its_rings(gemma):
    """A request of a ring model that lets go mid-reply while the pool keeps
    its blocks: on resume it attaches all of its tokens, its rings come back
    from the checkpoint, and the reply is the uninterrupted one, token for
    token. The other request ends meanwhile (that is what wakes it)."""
    hp, w = gemma
    V = hp["n_vocab"]
    pa, pb = lcg_ints(9100, 150, 0, V), lcg_ints(9101, 40, 0, V)
    _, (alone,) = gemma_run(hp, w, [(pa, 120)], 64, 1)
    eng, (ra, rb) = gemma_run(hp, w, [(pa, 120), (pb, 30)], 64, 2, preempt_at=(0, 20))
    assert ra.err is None and rb.err is None and len(ra.out) == 120
    assert ra.waits == 1 and eng.preemptions == 1
    assert ra.out == alone.out, first_diff(ra.out, alone.out)
    assert ra.ring_ckpt is None


def test_ring_model_waits_on_a_full_pool(gemma):
    """test_slots.lua:200-256 on a ring model: two requests that outgrow the
    pool together; one waits (its rings checkpointed; its blocks may be
    taken meanwhile, then it runs again from the start) and both replies
    are whole. Before the pool fills, each reply is its lone run's."""
    hp, w = gemma
    V = hp["n_vocab"]
    pa, pb = lcg_ints(9200, 300, 0, V), lcg_ints(9201, 100, 0, V)
    lone = [gemma_run(hp, w, [(p, 300)], 64, 1)[1][0].out for p in (pa, pb)]
    eng, (ra, rb) = gemma_run(hp, w, [(pa, 300), (pb, 300)], 14, 2)
    print("ring model: preemptions %d" % eng.preemptions, flush=True)
    assert ra.err is None and rb.err is None
    assert len(ra.out) == 300 and len(rb.out) == 300
    assert eng.preemptions >= 1
    assert first_diff(ra.out, lone[0]) >= 100 and first_diff(rb.out, lone[1]) >= 100
    assert not eng.waiting and eng.seqs.alloc.used == 0


def test_follow_up_turn_attaches_the_reply():
    """A finished request's prompt and reply stay keyed in the pool; the next
    turn (prompt + reply + new text) attaches them: it runs only the tokens
    after the cached ones, and its reply equals a fresh run's."""
    from lgml_amd import engine, runtime
    hp, w = models.build("c1", seed=93)
    V = hp["n_vocab"]
    p1 = lcg_ints(9300, 100, 0, V)
    gm = runtime.DeviceModel(hp, w, 64 * 64)
    eng = engine.Engine(gm, 2, ubatch=128, prefix_cache=True)
    ra = engine.Request(p1, 50)
    eng.submit(ra)
    drive(eng, [ra])
    turn2 = p1 + ra.out + lcg_ints(9301, 10, 0, V)
    rb = engine.Request(turn2, 20)
    eng.submit(rb)
    # the cells of prompt + reply but the reply's last token (which never ran)
    assert rb.fed == len(p1) + len(ra.out) - 1, rb.fed
    drive(eng, [rb])
    gm2 = runtime.DeviceModel(hp, w, 64 * 64)
    eng2 = engine.Engine(gm2, 1, ubatch=256)
    fresh = engine.Request(turn2, 20)
    eng2.submit(fresh)
    drive(eng2, [fresh])
    assert rb.out == fresh.out, first_diff(rb.out, fresh.out)


@pytest.mark.parametrize("run_ahead", [False, True])
def test_pool_grows_from_kv_initial(run_ahead):
    """The pool starts at 4 blocks and doubles as the requests need cells
    (4 -> 8 -> 16 blocks); the replies equal those of a pool allocated
    whole from the start, and nothing waits."""
    from lgml_amd import engine, runtime
    hp, w = models.build("c1", seed=95)
    V = hp["n_vocab"]
    specs = [(lcg_ints(9500, 300, 0, V), 200), (lcg_ints(9501, 100, 0, V), 200)]
    outs = []
    for kv_initial in (0, 256):
        gm = runtime.DeviceModel(hp, w, 1024 * 64, kv_initial=kv_initial)
        eng = engine.Engine(gm, 2, ubatch=128, run_ahead=run_ahead)
        reqs = [engine.Request(p, n) for p, n in specs]
        for r in reqs:
            eng.submit(r)
        drive(eng, reqs)
        assert all(r.err is None and len(r.out) == n for r, (_, n) in zip(reqs, specs))
        assert eng.preemptions == 0
        if kv_initial:
            print("pool grew %d times to %d cells" % (eng.seqs.grows, gm.n_cells), flush=True)
            assert eng.seqs.grows >= 2 and gm.n_cells >= 16 * 64
        outs.append([r.out for r in reqs])
    assert outs[0] == outs[1]
