"""Request.history across preemptions (CPU: no pass runs).

E:preempt (engine.lua:1193-1243) rebuilds a waiting request's tokens from
the cells its sequence holds plus what did not run (slot.tokens + rest,
:1194-1195). A request may wait more than once; its history must then
still be the prompt and every sample but the last, once each.
"""
from lgml_amd.engine import Request


def _prefill(r, sample):
    """The whole feed runs; its last pass samples one token."""
    r.fed = len(r.feed)
    r.out.append(sample)


def test_history_through_two_decode_preemptions():
    prompt = [1, 2, 3, 4, 5]
    r = Request(prompt, max_new=20)
    _prefill(r, 100)
    r.out += [101, 102]                       # two decode passes
    hist, rest = r.history()
    assert hist == prompt + [100, 101] and rest == [102]
    r.feed, r.fed = hist + rest, 0            # let_go: wait, then run the feed again
    _prefill(r, 103)                          # ... whose last pass samples 103
    r.out += [104]
    hist, rest = r.history()
    assert hist == prompt + [100, 101, 102, 103] and rest == [104]
    r.feed, r.fed = hist + rest, 0            # a second wait
    r.fed = 3                                 # preempted again mid re-prefill
    hist, rest = r.history()
    assert hist == prompt[:3] and rest == prompt[3:] + [100, 101, 102, 103, 104]
    r.feed, r.fed = hist + rest, 0
    _prefill(r, 105)
    hist, rest = r.history()
    assert hist == prompt + [100, 101, 102, 103, 104] and rest == [105]
    assert len(hist) + len(rest) == len(prompt) + len(r.out)


def test_history_while_prefilling():
    r = Request([7, 8, 9, 10], max_new=4)
    r.fed = 2
    assert r.history() == ([7, 8], [9, 10])
