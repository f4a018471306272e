"""The RAM store of spilled pool blocks (lgml_amd.engine.RamStore), on the
CPU: the behaviour of prompt_cache.lua's block entries -- P:spill skips a
key it holds and a block that does not fit the budget (:195-207), P:room
drops entries until one fits (:178-190), P:evict drops the lowest priority
first, then the least recently spilled (`before`, :132-136; :140-176),
P:unspill takes the entry out (:212-221). The device copies are covered by
tests/test_gpu_spill.py."""
from lgml_amd.engine import RamStore


def store(ram):
    filled = []
    s = RamStore(ram, alloc=lambda n: bytearray(n))
    return s, filled


def spill(s, key, prio, n=10):
    return s.spill(key, "p", 1, [1, 2], prio, n, lambda buf: buf.__setitem__(0, 7))


def test_spill_budget_and_skips():
    s, _ = store(0)
    assert not spill(s, "a", 1) and not s.blocks  # no RAM: nothing spills
    s, _ = store(25)
    assert spill(s, "a", 1) and spill(s, "b", 1)
    assert not spill(s, "a", 2)  # held already
    assert not spill(s, "big", 1, n=26)  # larger than the whole budget
    assert s.bytes == 20 and s.blocks["a"].buf[0] == 7


def test_room_drops_lowest_priority_then_oldest():
    s, _ = store(30)
    spill(s, "a", 1)
    spill(s, "b", 0)
    spill(s, "c", 1)
    spill(s, "d", 1)  # full: b goes (lowest priority)
    assert sorted(s.blocks) == ["a", "c", "d"]
    spill(s, "e", 2)  # then a (priority 1, spilled first)
    assert sorted(s.blocks) == ["c", "d", "e"]
    assert s.stats == {"spilled": 5, "unspilled": 0, "evicted": 2} and s.bytes == 30


def test_unspill_takes_the_entry_out():
    s, _ = store(30)
    spill(s, "a", 1)
    e = s.unspill("a")
    assert e.key == "a" and e.parent == "p" and e.depth == 1 and e.tokens == [1, 2]
    assert s.unspill("a") is None and s.bytes == 0 and s.stats["unspilled"] == 1
