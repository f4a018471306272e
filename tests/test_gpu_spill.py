"""Block spill / restore and pool growth on the device (the fourth "next"
row: M.copy_block_host, E:spill_block / E:unspill, pool_grow).

- lgmlh_kv_block_host copies one block of every pool tensor to pinned host
  memory and back, bit for bit.
- lgmlh_kv_grow keeps every cell of a grown pool and zeroes the new ones.
- The engine scenario of test/test_slots.lua:158-170: a pool of 768 cells
  and a RAM store of 4 blocks. Request a (460 prompt tokens) runs, then b
  evicts a's cached blocks, which spill to RAM; a's prompt again finds its
  7 full blocks in the pool and in RAM (448 tokens cached, at least 3 from
  RAM) and samples the same tokens with the same logits, bit for bit, as a
  fresh cache.
"""
import numpy as np
import pytest

from oracle import models
from tests.gpu_util import lcg_ints

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def st():
    return torch.cuda.current_stream().cuda_stream


def test_block_host_round_trip_and_grow():
    from lgml_amd import hip
    L = hip.lib()
    Hkv, D, cells, n_pools = 8, 128, 1024, 6
    lb = L.lgmlh_kv_layer_bytes(cells, Hkv, D)
    bb = L.lgmlh_kv_block_bytes(Hkv, D)
    assert bb == 64 * Hkv * D * 2
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    pools = [torch.randint(0, 255, (lb,), dtype=torch.uint8, device="cuda", generator=g)
             for _ in range(n_pools)]
    before = [p.clone() for p in pools]
    ptrs = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64, device="cuda")
    host = torch.zeros(n_pools * bb, dtype=torch.uint8, pin_memory=True)
    hip.check(L.lgmlh_kv_block_host(ptrs.data_ptr(), n_pools, cells, Hkv, D, 5, host.data_ptr(),
                                    1, st()))
    torch.cuda.synchronize()
    for i, p in enumerate(before):
        assert torch.equal(host[i * bb:(i + 1) * bb], p[5 * bb:6 * bb].cpu()), i
    # back into block 9 of every tensor: block 9 now equals block 5, nothing else moved
    hip.check(L.lgmlh_kv_block_host(ptrs.data_ptr(), n_pools, cells, Hkv, D, 9, host.data_ptr(),
                                    0, st()))
    torch.cuda.synchronize()
    for p, q in zip(pools, before):
        want = q.clone()
        want[9 * bb:10 * bb] = q[5 * bb:6 * bb]
        assert torch.equal(p, want)
    # grow: the old pool is a prefix of the new one, the new cells are zero
    new = torch.full((L.lgmlh_kv_layer_bytes(3 * cells, Hkv, D),), 7, dtype=torch.uint8,
                     device="cuda")
    hip.check(L.lgmlh_kv_grow(pools[0].data_ptr(), cells, new.data_ptr(), 3 * cells, Hkv, D,
                              st()))
    torch.cuda.synchronize()
    assert torch.equal(new[:lb], pools[0]) and not new[lb:].any()
    assert L.lgmlh_kv_grow(pools[0].data_ptr(), cells, new.data_ptr(), cells - 64, Hkv, D,
                           st()) == hip.EINVAL


def chat(eng, prompt, n):
    """Run one request to completion; its (token, logits) per sampled step."""
    from lgml_amd import engine
    r = engine.Request(prompt, n)
    eng.submit(r)
    fed_at_submit = r.fed
    rows = []
    while not r.done:
        got = eng.step()
        if r in got:
            i = eng.last_entries.index(r)
            rows.append((r.out[-1], eng.last_logits[i].cpu().numpy().copy()))
    return rows, fed_at_submit


def test_evicted_blocks_spill_to_ram_and_come_back_bit_exact():
    from lgml_amd import engine, runtime
    hp, w = models.build("c2", seed=7, n_layer=2, init="normal")
    V = hp["n_vocab"]
    a = lcg_ints(7000, 460, 0, V)
    b = lcg_ints(7001, 470, 0, V)
    a2 = a + lcg_ints(7002, 5, 0, V)
    gm = runtime.DeviceModel(hp, w, 768)
    eng = engine.Engine(gm, 2, prefix_cache=True, ram=4 * gm.block_bytes_all)
    chat(eng, a, 3)
    chat(eng, b, 3)
    assert eng.ram.stats["spilled"] >= 3, eng.ram.stats
    rows, fed = chat(eng, a2, 4)
    assert fed == 448 and eng.ram.stats["unspilled"] >= 3 and eng.from_ram >= 3, (
        fed, eng.ram.stats, eng.from_ram)
    fresh = engine.Engine(runtime.DeviceModel(hp, w, 768), 2)
    want, fed0 = chat(fresh, a2, 4)
    assert fed0 == 0
    for (ta, la), (tb, lb) in zip(rows, want):
        assert ta == tb
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
