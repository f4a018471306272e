"""KV pool bookkeeping over the native pool (lgmlh_kvpool_* in the C ABI):
the lua/lgml/kvpool.lua API -- new, take, evict, ref, unref, refs_of,
publish, publish_part, key_of, lookup, longest_kid, set_cap, key,
default_seqs -- with block ids from 0 and None where Lua returns nil."""
import ctypes as C

import numpy as np

from . import hip

LOW, NORMAL, HIGH = 0, 1, 2  # kvpool.lua:25
SEQS = 4  # kvpool.lua:28


def default_seqs(pool, fixed):
    """kvpool.lua:37-42."""
    if fixed <= 0:
        return SEQS
    return max(1, min(SEQS, pool // 4 // fixed))


def key(parent, tokens, i=1, n=None):
    """kvpool.lua:51-59: the block key of tokens[i..i+n-1] (1-based i) after parent."""
    j = i + n - 1 if n is not None else len(tokens)
    t = np.ascontiguousarray(tokens[i - 1:j], np.int32)
    out = C.create_string_buffer(65)
    hip.check(hip.lib().lgmlh_block_key(parent.encode(), t.ctypes.data, len(t), out))
    return out.value.decode()


def _toks(tokens):
    return np.ascontiguousarray(list(tokens) if not isinstance(tokens, np.ndarray) else tokens,
                                np.int32)


class Pool:
    """M.new (kvpool.lua:65-72): blocks of size cells, cap usable."""

    def __init__(self, blocks, size, cap=None):
        L = hip.lib()
        cap = blocks if cap is None else cap
        nb = L.lgmlh_kvpool_bytes(blocks, size)
        self.mem = (C.c_uint8 * nb)()
        hip.check(L.lgmlh_kvpool_init(self.mem, nb, blocks, size, cap))
        self.n, self.size = blocks, size

    def _stats(self):
        out = (C.c_int64 * 8)()
        hip.check(hip.lib().lgmlh_kvpool_stats(self.mem, out))
        return list(out)

    cap = property(lambda self: self._stats()[2])
    used = property(lambda self: self._stats()[3])
    low = property(lambda self: self._stats()[4])
    cached = property(lambda self: self._stats()[5])
    evicted = property(lambda self: self._stats()[7])

    def take(self, min_=None):
        b = hip.lib().lgmlh_kvpool_take(self.mem, min_ or 0)
        return None if b < 0 else b

    def evict(self):
        b = hip.lib().lgmlh_kvpool_evict(self.mem)
        return None if b < 0 else b

    def victim(self):
        """(block, prio) that the next evict takes, or None; nothing changes
        (the on_evict moment of kvpool.lua:149-152)."""
        prio = C.c_int32(0)
        b = hip.lib().lgmlh_kvpool_victim(self.mem, C.byref(prio))
        return None if b < 0 else (b, prio.value)

    def ref(self, b, prio=None):
        hip.check(hip.lib().lgmlh_kvpool_ref(self.mem, b, NORMAL if prio is None else prio))

    def unref(self, b):
        hip.check(hip.lib().lgmlh_kvpool_unref(self.mem, b))

    def refs_of(self, b):
        return hip.lib().lgmlh_kvpool_refs_of(self.mem, b)

    def publish(self, b, k, parent, depth, tokens, prio=None):
        t = _toks(tokens)
        rc = hip.lib().lgmlh_kvpool_publish(self.mem, b, k.encode(), parent.encode(), depth,
                                            t.ctypes.data, len(t), NORMAL if prio is None else prio)
        hip.check(min(rc, 0))
        return rc == 1

    def publish_part(self, b, parent, depth, tokens, prio=None):
        t = _toks(tokens)
        rc = hip.lib().lgmlh_kvpool_publish_part(self.mem, b, parent.encode(), depth,
                                                 t.ctypes.data, len(t),
                                                 NORMAL if prio is None else prio)
        hip.check(min(rc, 0))
        return rc == 1

    def key_of(self, b):
        out = C.create_string_buffer(65)
        rc = hip.lib().lgmlh_kvpool_key_of(self.mem, b, out)
        return None if rc == 0 else ("part" if rc == 2 else out.value.decode())

    def lookup(self, k):
        b = hip.lib().lgmlh_kvpool_lookup(self.mem, k.encode())
        return None if b < 0 else b

    def longest_kid(self, parent, tokens, i, max_):
        t = _toks(tokens[i - 1:i - 1 + max_])
        shared = C.c_int32(0)
        b = hip.lib().lgmlh_kvpool_longest_kid(self.mem, parent.encode(), t.ctypes.data, len(t),
                                               C.byref(shared))
        return (None if b < 0 else b), shared.value

    def set_cap(self, cap):
        hip.check(hip.lib().lgmlh_kvpool_set_cap(self.mem, cap))
