"""Restatement of the KV pool bookkeeping and cell mapping (pure Python).

TEST INFRASTRUCTURE ONLY: the checker for lgml_amd's native pool
(lgml_amd/csrc/host/kvpool.cpp) and for the GPU ubatch descriptors.

Follows lua/lgml/kvpool.lua (whole file), the block helpers of
lua/lgml/transformer.lua (reserve :963-981, truncate :1084-1108, share
:1116-1123, seq_cells :1126-1133, seq_window :1154-1172, PAD :25) and
tensor:fill_blocks (src/lgml.c:2936-3017).
"""
import hashlib

import numpy as np

LOW, NORMAL, HIGH = 0, 1, 2  # kvpool.lua:25
SEQS = 4  # kvpool.lua:28
PAD = 256  # transformer.lua:25


def default_seqs(pool, fixed):
    """kvpool.lua:37-42."""
    if fixed <= 0:
        return SEQS
    return max(1, min(SEQS, pool // 4 // fixed))


def key(parent, tokens, i=1, n=None):
    """kvpool.lua:51-59: sha256 hex of parent .. "," .. tokens[i..j] joined by ","."""
    j = i + n - 1 if n is not None else len(tokens)
    parts = [parent] + [str(t) for t in tokens[i - 1:j]]
    return hashlib.sha256(",".join(parts).encode()).hexdigest()


class Pool:
    """kvpool.lua:65-72 (M.new) and the P methods."""

    def __init__(self, blocks, size, cap=None):
        self.n, self.size = blocks, size
        self.cap = blocks if cap is None else cap
        self.refs, self.used, self.low = {}, 0, 0
        self.keys, self.bykey, self.info, self.kids = {}, {}, {}, {}
        self.cached, self.tick = 0, 0
        self.stats = {"evicted": 0, "hits": 0, "hit_blocks": 0}
        self.on_evict = None

    def _take_at(self, b):  # :84-91
        self.refs[b] = 1
        self.used += 1
        if b == self.low:
            self.low = b + 1
        return b

    def take(self, min_=None):  # :102-116
        frm = max(self.low, min_ or 0)
        for b in range(frm, self.cap):
            if b not in self.refs and b not in self.keys:
                return self._take_at(b)
        for b in range(self.low, min(frm, self.cap)):
            if b not in self.refs and b not in self.keys:
                return self._take_at(b)
        self.low = self.cap
        return None

    def _unkey(self, b):  # :119-133
        k = self.keys.pop(b)
        info = self.info.pop(b)
        if self.bykey.get(k) == b:
            del self.bykey[k]
        kids = self.kids.get(info["parent"])
        if kids is not None:
            kids.pop(b, None)
            if not kids:
                del self.kids[info["parent"]]

    def evict(self):  # :139-160
        best = None
        # Lua pairs() order is unspecified; the minimum under (prio, used,
        # -depth) is unique except for exact ties, broken here by lowest id.
        for b in sorted(self.info):
            info = self.info[b]
            if b in self.refs or b >= self.cap:
                continue
            if best is None or info["prio"] < bp or (info["prio"] == bp and (
                    info["used"] < bu or (info["used"] == bu and info["depth"] > bd))):
                best, bp, bu, bd = b, info["prio"], info["used"], info["depth"]
        if best is None:
            return None
        if self.on_evict and self.keys[best] != "part":
            self.on_evict(best, self.keys[best], self.info[best])
        self._unkey(best)
        self.cached -= 1
        self.stats["evicted"] += 1
        self.refs[best] = 1
        self.used += 1
        return best

    def ref(self, b, prio=None):  # :165-178
        r = self.refs.get(b)
        if r is None:
            assert b in self.keys, "kvpool: ref of a free block"
            self.cached -= 1
            self.used += 1
            r = 0
        self.refs[b] = r + 1
        info = self.info.get(b)
        if info is not None:
            info["prio"] = max(info["prio"], NORMAL if prio is None else prio)

    def unref(self, b):  # :183-198
        assert b in self.refs, "kvpool: unref of a free block"
        r = self.refs[b] - 1
        if r > 0:
            self.refs[b] = r
            return
        del self.refs[b]
        self.used -= 1
        if b in self.keys:
            self.tick += 1
            self.info[b]["used"] = self.tick
            self.cached += 1
        elif b < self.low:
            self.low = b

    def refs_of(self, b):  # :203-205
        return self.refs.get(b, 0)

    def publish(self, b, k, parent, depth, tokens, prio=None):  # :217-226
        if b in self.keys or k in self.bykey:
            return False
        self.keys[b], self.bykey[k] = k, b
        self.info[b] = {"parent": parent, "depth": depth, "tokens": list(tokens),
                        "used": self.tick, "prio": NORMAL if prio is None else prio}
        self.kids.setdefault(parent, {})[b] = True
        return True

    def publish_part(self, b, parent, depth, tokens, prio=None):  # :239-249
        if b in self.keys or len(tokens) == 0:
            return False
        self.keys[b] = "part"
        self.info[b] = {"parent": parent, "depth": depth, "tokens": list(tokens),
                        "used": self.tick, "prio": NORMAL if prio is None else prio}
        self.kids.setdefault(parent, {})[b] = True
        return True

    def key_of(self, b):
        return self.keys.get(b)

    def lookup(self, k):  # :261-263
        return self.bykey.get(k)

    def longest_kid(self, parent, tokens, i, max_):  # :273-285
        best, bn = None, 0
        # Lua pairs() order: ties go to the lowest block id here.
        for b in sorted(self.kids.get(parent, {})):
            t, k = self.info[b]["tokens"], 0
            while k < max_ and k < len(t) and i - 1 + k < len(tokens) and t[k] == tokens[i - 1 + k]:
                k += 1
            if k > bn:
                best, bn = b, k
        return best, bn

    def set_cap(self, cap):  # :289-293
        assert cap <= self.n, "kvpool: cap past the pool"
        self.cap = cap
        self.low = min(self.low, cap)


class PoolFull(Exception):
    pass


class Seq:
    """A pool sequence's block table (transformer.lua:716-725, M:seq)."""

    def __init__(self, pool, prio=None):
        self.pool, self.blocks, self.keys, self.n_past, self.prio = pool, [], [], 0, prio


def new_block(pool, c, min_, pressure=None):
    """transformer.lua:934-958 without pool growth: a free block, else a
    cached one, else one that pressure frees."""
    b = pool.take(min_)
    if b is not None:
        return b
    b = pool.evict()
    if b is None and pressure is not None:
        pressure(pool, c)
        b = pool.take(min_)
        if b is None:
            b = pool.evict()
    return b


def reserve(c, n, pressure=None):
    """transformer.lua:963-981: blocks for positions [0, n); the new blocks
    of one call are sorted so cells stay in position order."""
    p, B = c.pool, c.pool.size
    first = len(c.blocks)
    while len(c.blocks) * B < n:
        last = c.blocks[-1] if c.blocks else None
        b = new_block(p, c, None if last is None else last + 1, pressure)
        if b is None:
            raise PoolFull("kv pool full: %d of %d cells in use" % (p.used * B, p.n * B))
        c.blocks.append(b)
    if len(c.blocks) - first > 1:
        c.blocks[first:] = sorted(c.blocks[first:])


def truncate(c, n, copy_block=None):
    """transformer.lua:1084-1108 (copy-on-write of a shared partial block)."""
    p, B = c.pool, c.pool.size
    keep = (n + B - 1) // B
    while len(c.blocks) > keep:
        p.unref(c.blocks.pop())
    del c.keys[n // B:]
    last = c.blocks[keep - 1] if keep >= 1 and len(c.blocks) >= keep else None
    if n % B != 0 and last is not None and (p.refs_of(last) > 1 or p.key_of(last)):
        prev = c.blocks[keep - 2] if keep >= 2 else None
        b = new_block(p, c, None if prev is None else prev + 1)
        if b is None:
            raise PoolFull("kv pool full")
        if copy_block:
            copy_block(last, b, n % B)
        c.blocks[keep - 1] = b
        p.unref(last)
    c.n_past = min(c.n_past, n)


def share(c, blocks, keys):
    """transformer.lua:1116-1123."""
    assert not c.blocks, "share: the sequence has blocks"
    for i, b in enumerate(blocks):
        c.pool.ref(b, c.prio)
        c.blocks.append(b)
        c.keys.append(keys[i])
    c.n_past = len(blocks) * c.pool.size


def seq_cells(blocks, B, frm, n):
    """transformer.lua:1126-1133: cell(p) = blocks[p // B] * B + p % B."""
    return [blocks[p // B] * B + p % B for p in range(frm, frm + n)]


def seq_window(blocks, B, n_kv, cap):
    """transformer.lua:1154-1172: the PAD-aligned pool window [lo, lo+w)."""
    nb = (n_kv + B - 1) // B
    lo, hi = None, 0
    for i in range(nb):
        s = blocks[i] * B
        lo = s if lo is None or s < lo else lo
        e = s + B if i < nb - 1 else s + (n_kv - 1) % B + 1
        hi = max(hi, e)
    lo = lo // PAD * PAD
    hi = min(cap, (hi + PAD - 1) // PAD * PAD)
    return lo, hi - lo


def fill_blocks(rows, n_kv, n_past, block, blocks, lo=0, causal=True):
    """src/lgml.c:2936-3017: additive mask (rows, n_kv) over window columns."""
    need = (n_past + rows + block - 1) // block
    if len(blocks) < need:
        raise ValueError("fill_blocks: too few blocks")
    m = np.full((rows, n_kv), -np.inf, np.float32)
    p = 0
    for i in range(rows):
        if i > 0:
            m[i] = m[i - 1]
        last = n_past + i if causal else n_past + rows - 1
        while p <= last:
            col = blocks[p // block] * block - lo + p % block
            if col < 0 or col >= n_kv:
                raise ValueError("fill_blocks: position %d is in no column" % p)
            m[i, col] = 0.0
            p += 1
    return m
