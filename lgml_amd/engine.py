"""Pool sequences and the continuous-batching scheduler of the HIP path.

Sequences over one paged pool follow lua/lgml/transformer.lua's pool
helpers -- new_block (:934-958), reserve (:963-981), truncate (:1084-1108,
copy-on-write of a shared partial block, here a device block copy),
share (:1116-1123), seq_cells (:1126-1133) -- over the native pool
bookkeeping (lgml_amd.kvpool). Engine.flush restates E:flush
(lua/lgml/engine.lua:1423-1506): the pending decode steps and prompt
chunks of all slots run as one pass, and blocks are taken for each entry
in arrival order first (a full pool: see below). Prompts go in chunks of at most ubatch tokens
(E:prefill_batched, :2213-2255, ubatch 512, :57). Greedy sampling is the
first maximum (src/sample.c:914-925) on the device.

With prefix_cache, a request attaches the cached blocks of its prompt
before its first pass (E:attach / E:cached_blocks / E:attach_blocks,
engine.lua:2010-2077): the full blocks whose chained keys it finds are
shared, the best partial match is copied into a block of its own, and only
the rest of the prompt runs. Full prompt blocks get keys as their prefill
completes (E:publish, :1829-1841), so later requests can share them.

A pass carries at most max_tokens tokens (a MoE model: 8192 / n_used,
the picks one routing pass groups): decode tokens always go, prompt chunks
are cut to what is left, and a request with no room waits for the next
pass (E:flush itself is bounded by the memory budget, engine.lua:1477-1486).

With ram > 0 (and prefix_cache), keyed blocks that the pool evicts spill
to a RAM store (E:spill_block / E:unspill, engine.lua:1843-1868; the block
entries of prompt_cache.lua's store, :132-222): one launch copies the
block's cells in every layer to pinned host memory, and a later request
whose prompt key misses the pool takes them back before it attaches.

A model with sliding-window layers gives each slot a ring of its own in
the ring pools (M:cache's per-slot rings, transformer.lua:575-600): slot
i owns ring blocks i R .. i R + R - 1, R = ring_cells / 64 / n_slots, and
a request holds a slot from submit to finish.

A full pool makes a request wait, not end (E:flush, E:victim, E:preempt,
engine.lua:1193-1243,1410-1448): when an entry gets no block, a running
request of lower priority (the lowest, the least recently started) lets
its cells go and the entry runs in a later pass; with no such request,
the entry's own request lets its cells go and waits, unless it runs
alone (then its reply ends with "kv pool full"). A request that lets its
cells go publishes the keys of its blocks (E:publish_tail, :1906-1918),
gives up its slot and waits; when another request ends it takes a slot
again, attaches what is still cached of its tokens (pool or RAM store)
and runs the rest. The reference's E:pool_pressure (:1122-1140) first
takes the cells of idle slots; here a request that ends gives its blocks
back at once (keyed ones stay cached and are evicted first), so no idle
slot holds cells. A sliding-window ring cannot be rebuilt from cached
blocks, so a request of a model with rings checkpoints its slot's rings to
pinned host memory when it lets go (E:checkpoint_slot, :2103-2116) and
restores them into its new slot when it attaches exactly the tokens it had;
otherwise it runs again from the start.

The pool can start small (DeviceModel kv_initial) and grow: a reserve that
finds no free block doubles the pool tensors up to their ceiling before it
evicts (new_block's grow branch, transformer.lua:934-958, pool_grow
:831-908).

With prefix_cache, a request that ends publishes the keys of its prompt and
reply blocks, so a follow-up turn that repeats them attaches them.
"""
import ctypes as C

import numpy as np
import torch

from . import hip, kvpool
from .hip import check, stream

UBATCH = 512  # lua/lgml/engine.lua:57
BLOCK = 64    # lua/lgml/transformer.lua:30


class PoolFull(RuntimeError):
    pass


class Seq:
    """A sequence on the pool (M:seq, transformer.lua:716-725)."""

    def __init__(self, pool, prio=kvpool.NORMAL):
        self.pool, self.blocks, self.keys, self.n_past, self.prio = pool, [], [], 0, prio


class PoolSeqs:
    """Block tables of the sequences on one device model's pool."""

    def __init__(self, model, pressure=None):
        self.model = model
        # blocks up to the model's ceiling, usable up to its present size
        self.alloc = kvpool.Pool(getattr(model, "max_blocks", model.pool_blocks), BLOCK,
                                 cap=model.pool_blocks)
        self.pressure = pressure
        self.on_evict = None  # on_evict(block, key, prio), kvpool.lua:149-152
        self.grows = 0

    def evict(self):
        """P:evict (kvpool.lua:139-160), telling on_evict about a keyed block
        first, while its cells and key are still there."""
        if self.on_evict is not None:
            v = self.alloc.victim()
            if v is not None:
                k = self.alloc.key_of(v[0])
                if k is not None and k != "part":
                    self.on_evict(v[0], k, v[1])
        return self.alloc.evict()

    def new_block(self, c, min_):
        """new_block (transformer.lua:934-958): a free block, else a new one
        when the pool can grow (the model's pool tensors doubled, up to its
        ceiling), else a cached one, else one that pressure frees for c."""
        b = self.alloc.take(min_)
        if b is not None:
            return b
        m = self.model
        if getattr(m, "max_cells", m.n_cells) > m.n_cells:
            m.grow_pool()
            self.alloc.set_cap(m.pool_blocks)
            self.grows += 1
            return self.alloc.take(min_)
        b = self.evict()
        if b is None and self.pressure is not None:
            self.pressure(self, c)
            b = self.alloc.take(min_)
            if b is None:
                b = self.evict()
        return b

    def reserve(self, c, n):
        """transformer.lua:963-981: blocks for positions [0, n); the new
        blocks of one call go in cell order."""
        first = len(c.blocks)
        while len(c.blocks) * BLOCK < n:
            last = c.blocks[-1] if c.blocks else None
            b = self.new_block(c, None if last is None else last + 1)
            if b is None:
                raise PoolFull("kv pool full: %d of %d cells in use" % (
                    self.alloc.used * BLOCK, self.model.n_cells))
            c.blocks.append(b)
        if len(c.blocks) - first > 1:
            c.blocks[first:] = sorted(c.blocks[first:])

    def copy_block(self, src, dst, n):
        """M.copy_block (transformer.lua:989-1007) on the device, every layer."""
        m = self.model
        D, Hkv = getattr(m, "paged_dims", (m.hp["head_dim"], m.hp["n_head_kv"]))
        for il, (kp, vp) in enumerate(zip(m.kpools, m.vpools)):
            if getattr(m, "swa", None) and m.swa[il]:
                continue  # ring pools hold no pool blocks
            check(hip.lib().lgmlh_kv_copy_block(kp.data_ptr(), vp.data_ptr(), m.n_cells, Hkv, D,
                                                src, dst, n, stream()))

    def truncate(self, c, n):
        """transformer.lua:1084-1108."""
        keep = (n + BLOCK - 1) // BLOCK
        while len(c.blocks) > keep:
            self.alloc.unref(c.blocks.pop())
        del c.keys[n // BLOCK:]
        last = c.blocks[keep - 1] if keep >= 1 and len(c.blocks) >= keep else None
        if n % BLOCK and last is not None and (self.alloc.refs_of(last) > 1 or
                                               self.alloc.key_of(last)):
            prev = c.blocks[keep - 2] if keep >= 2 else None
            b = self.new_block(c, None if prev is None else prev + 1)
            if b is None:
                raise PoolFull("kv pool full")
            self.copy_block(last, b, n % BLOCK)
            c.blocks[keep - 1] = b
            self.alloc.unref(last)
        c.n_past = min(c.n_past, n)

    def share(self, c, blocks, keys):
        """transformer.lua:1116-1123."""
        assert not c.blocks, "share: the sequence has blocks"
        for b, k in zip(blocks, keys):
            self.alloc.ref(b, c.prio)
            c.blocks.append(b)
            c.keys.append(k)
        c.n_past = len(blocks) * BLOCK

    def free(self, c):
        """M:free_seq (transformer.lua:784-803): give the blocks back."""
        self.truncate(c, 0)


def seq_cells(c, frm, n):
    """transformer.lua:1126-1133."""
    return [c.blocks[p // BLOCK] * BLOCK + p % BLOCK for p in range(frm, frm + n)]


class RamEntry:
    __slots__ = ("key", "parent", "depth", "tokens", "prio", "buf", "bytes", "used")

    def __init__(self, **kw):
        for k, v in kw.items():
            setattr(self, k, v)


class RamStore:
    """The spilled-block part of the prompt cache's RAM store
    (prompt_cache.lua:132-222): entries by key under a byte budget, room
    made by dropping the entry of the lowest priority, then the least
    recently spilled (`before`, :132-136). Buffers are pinned host memory
    the device reads and writes directly."""

    def __init__(self, ram_bytes, alloc=None):
        """alloc(nbytes): the buffer of a spilled block (default: pinned
        host memory)."""
        self.ram = int(ram_bytes)
        self.alloc = alloc or (lambda n: torch.empty(n, dtype=torch.uint8, pin_memory=True))
        self.blocks = {}
        self.bytes = 0
        self.tick = 0
        self.stats = {"spilled": 0, "unspilled": 0, "evicted": 0}

    def evict(self):
        """P:evict (:140-176) over the block entries."""
        if not self.blocks:
            return False
        lru = min(self.blocks.values(), key=lambda e: (e.prio, e.used))
        del self.blocks[lru.key]
        self.bytes -= lru.bytes
        self.stats["evicted"] += 1
        return True

    def room(self, nbytes):
        """P:room (:178-190)."""
        if nbytes > self.ram:
            return False
        while self.bytes + nbytes > self.ram:
            if not self.evict():
                return False
        return True

    def spill(self, key, parent, depth, tokens, prio, nbytes, fill):
        """P:spill (:195-207): fill(buf) copies the cells into a new pinned
        buffer of nbytes."""
        if self.ram <= 0 or key in self.blocks or not self.room(nbytes):
            return False
        buf = self.alloc(nbytes)
        fill(buf)
        self.tick += 1
        self.blocks[key] = RamEntry(key=key, parent=parent, depth=depth, tokens=list(tokens),
                                    prio=prio, buf=buf, bytes=nbytes, used=self.tick)
        self.bytes += nbytes
        self.stats["spilled"] += 1
        return True

    def unspill(self, key):
        """P:unspill (:212-221): the entry, out of the store, or None."""
        e = self.blocks.pop(key, None)
        if e is None:
            return None
        self.bytes -= e.bytes
        self.stats["unspilled"] += 1
        return e


class Request:
    def __init__(self, prompt, max_new, prio=kvpool.NORMAL):
        self.prompt = list(prompt)
        self.max_new = max_new
        self.prio = prio
        self.out = []
        self.seq = None
        # the tokens to run before decoding: the prompt, or after a wait the
        # tokens so far and the rest (E:preempt's toks)
        self.feed = list(prompt)
        self.fed = 0       # feed tokens run so far
        self.err = None
        self.done = False
        self.preempt = False  # lets its cells go at the next chance
        self.started = 0      # submit order (E:victim: the least recently started)
        self.waits = 0        # times it let its cells go
        self.wait_mark = 0    # the engine's count of ended requests when it began to wait
        self.ring_ckpt = None  # (position, pinned bytes) of its rings while it waits
        # run-ahead engines: sampled tokens of passes not yet read back, the
        # (pass, row) holding the latest one on the device, and whether the
        # request takes part in no further pass
        self.n_inflight = 0
        self.tok_src = None
        self.finishing = False

    def pending(self, ubatch):
        """The ids of this request's next pass: a prompt chunk or one token."""
        if self.fed < len(self.feed):
            return self.feed[self.fed:self.fed + ubatch]
        return [self.out[-1]]

    def history(self):
        """(the tokens whose cells the sequence holds, the tokens that did
        not run) with no pass in flight: the feed run so far and the fed
        samples; the rest of the feed, or the last sample."""
        if self.fed < len(self.feed):
            return self.feed[:self.fed], self.feed[self.fed:]
        # decoding: the feed is the prompt and a prefix of out (after a wait),
        # all of it run; the sequence holds the prompt and every sample but
        # the last (E:preempt's slot.tokens + rest, engine.lua:1194-1195)
        return self.prompt + self.out[:-1], self.out[-1:]


class _Half:
    """The part of a pass in flight that runs on one stream (run-ahead
    engines): its plan, logits, sampled ids (device, pinned host) and the
    event after their copy."""
    __slots__ = ("plan", "logits", "ids_dev", "ids_host", "event", "entries")


class _Pass:
    """A pass in flight: its halves (one, or two on two streams) and its
    entries (request, tokens, prompt chunk?, sampled?) in pass order."""
    __slots__ = ("halves", "entries")


ROOT_KEY = "lgml:"  # E:root_key (engine.lua:1823-1825) without adapters


class Engine:
    """Slots over one pool; step() runs one batched pass (E:flush)."""

    def __init__(self, model, n_slots, ubatch=UBATCH, blocks_per_split=0, trace=None,
                 prefix_cache=False, max_tokens=None, ram=0, run_ahead=False, streams=1):
        self.model = model
        self.run_ahead = run_ahead
        if streams not in (1, 2) or (streams == 2 and not run_ahead):
            raise ValueError("streams: 1, or 2 with run_ahead")
        # streams=2: a pass runs as two halves (alternate entries) at once,
        # the second on a side stream of default priority
        self.n_streams = streams
        self._side = torch.cuda.Stream() if streams == 2 else None
        self._inflight = None
        self.launched_plan = None
        self.launched_plans = []
        self.last_plans = []
        self._last_halves = None
        nu = model.hp.get("n_used", 0) if model.hp.get("n_expert") else 0
        self.max_tokens = max_tokens or (8192 // nu if nu else None)
        self.seqs = PoolSeqs(model)
        self.prefix_cache = prefix_cache
        self.hits = self.hit_blocks = 0
        self.n_slots = n_slots
        self.ubatch = ubatch
        self.bps = blocks_per_split
        self.active = []   # requests in arrival order
        self.trace = trace
        self.passes = self.rows = self.tokens = 0
        self.last_plan = None
        self.last_logits = None
        self._ids = torch.empty(0, dtype=torch.int32, device="cuda")
        self.ring_blocks = 0
        if any(getattr(model, "swa", [])):
            if prefix_cache:
                raise ValueError("prefix sharing covers the paged pool only, not the rings")
            self.ring_blocks = model.ring_cells // BLOCK // n_slots
            need = model.hp["n_swa"] - 1 + ubatch
            if self.ring_blocks * BLOCK < need:
                # "tokens in one pass; the ring takes" (transformer.lua:1544-1546)
                raise ValueError("rings of %d cells per slot; a pass of %d tokens needs %d" % (
                    self.ring_blocks * BLOCK, ubatch, need))
        self.free_slots = list(range(n_slots))
        # the RAM tier of evicted prompt blocks (engine.lua:618-629)
        self.ram = RamStore(ram) if ram > 0 and prefix_cache else None
        self.infos = {}  # key -> (parent, depth, tokens) of the blocks published here
        self.from_ram = 0
        # requests that let their cells go, in the order they did, and the
        # counts of E:preempt (engine.lua:1203-1206)
        self.waiting = []
        self.preemptions = 0
        self.waits = {}
        self._ended = 0     # requests that ended so far (a waiting request wakes on a later one)
        self._submitted = 0
        if self.ram is not None:
            self.seqs.on_evict = self.spill_block

    def submit(self, req):
        if len(self.active) >= self.n_slots:
            raise RuntimeError("no free slot")
        req.slot = self.free_slots.pop(0)
        req.seq = Seq(self.seqs, req.prio)
        self._submitted += 1
        req.started = self._submitted
        self.active.append(req)
        if self.prefix_cache:
            req.fed = self.attach(req)
            req.seq.n_past = req.fed
        return req

    # -- prefix sharing ------------------------------------------------------
    # -- the RAM tier --------------------------------------------------------
    def block_host(self, b, buf, out):
        m = self.model
        check(hip.lib().lgmlh_kv_block_host(m.pools_dev.data_ptr(), m.n_pools, m.n_cells,
                                            m.paged_dims[1], m.paged_dims[0], b, buf.data_ptr(),
                                            1 if out else 0, stream()))

    def spill_block(self, b, key, prio):
        """E:spill_block (engine.lua:1843-1850): copy the cells of a keyed
        block that the pool evicts to the RAM store."""
        info = self.infos.pop(key, None)
        if info is None:
            return
        self.ram.spill(key, info[0], info[1], info[2], prio, self.model.block_bytes_all,
                       lambda buf: self.block_host(b, buf, True))

    def unspill(self, key, last, prio):
        """E:unspill (engine.lua:1852-1868): a spilled block back in the pool
        after block last, published again, with one reference; or None."""
        e = self.ram.unspill(key) if self.ram is not None else None
        if e is None:
            return None
        b = self.seqs.new_block(None, None if last is None else last + 1)
        if b is not None:
            self.block_host(b, e.buf, False)
            # the buffer goes with the entry: the copy must be done first
            torch.cuda.current_stream().synchronize()
            self.seqs.alloc.publish(b, key, e.parent, e.depth, e.tokens, max(e.prio, prio))
            self.infos[key] = (e.parent, e.depth, e.tokens)
            self.from_ram += 1
        return b

    def cached_blocks(self, prompt, max_, prio):
        """E:cached_blocks (engine.lua:1873-1892): the cached blocks holding the
        first full blocks of prompt (at most max_ tokens), each referenced;
        spilled blocks come back from the RAM store."""
        alloc, blocks, keys, parent = self.seqs.alloc, [], [], ROOT_KEY
        while (len(blocks) + 1) * BLOCK <= max_:
            k = kvpool.key(parent, prompt, len(blocks) * BLOCK + 1, BLOCK)
            b = alloc.lookup(k)
            if b is not None:
                alloc.ref(b, prio)
            else:
                b = self.unspill(k, blocks[-1] if blocks else None, prio)
                if b is None:
                    break
            blocks.append(b)
            keys.append(k)
            parent = k
        return blocks, keys

    def attach(self, req):
        """E:attach_blocks (engine.lua:2038-2077) for a new request: returns
        the number of prompt tokens already in the cache."""
        prompt, c, alloc = req.feed, req.seq, self.seqs.alloc
        max_ = len(prompt) - 1  # at least one prompt token must run
        blocks, keys = self.cached_blocks(prompt, max_, c.prio)
        try:
            m = len(blocks) * BLOCK
            kid, part = alloc.longest_kid(keys[-1] if keys else ROOT_KEY, prompt, m + 1,
                                          min(BLOCK - 1, max_ - m))
            if m + part <= 0:
                return 0
            self.seqs.share(c, blocks, keys)
            if part > 0:
                alloc.ref(kid)  # hold it while the copy takes a new block
                try:
                    self.seqs.reserve(c, m + part)
                    self.seqs.copy_block(kid, c.blocks[len(blocks)], part)
                    c.n_past = m + part
                except PoolFull:
                    part = 0
                    c.n_past = m
                alloc.unref(kid)
            self.hits += 1
            self.hit_blocks += len(blocks)
            return m + part
        finally:
            for b in blocks:  # E:drop_held
                alloc.unref(b)

    def publish(self, req):
        """E:publish (engine.lua:1829-1841): keys for the full prompt blocks
        of the request that have none yet."""
        self.publish_tokens(req, req.feed)

    def publish_tokens(self, req, tokens):
        """Keys for the full blocks of the sequence's tokens (a prefix of
        tokens) that have none yet."""
        c, alloc = req.seq, self.seqs.alloc
        upto = min(c.n_past, len(tokens)) // BLOCK
        for i in range(len(c.keys) + 1, upto + 1):
            parent = c.keys[i - 2] if i >= 2 else ROOT_KEY
            k = kvpool.key(parent, tokens, (i - 1) * BLOCK + 1, BLOCK)
            c.keys.append(k)
            toks = tokens[(i - 1) * BLOCK:i * BLOCK]
            if alloc.publish(c.blocks[i - 1], k, parent, i, toks, c.prio):
                self.infos[k] = (parent, i, list(toks))

    def finish(self, req):
        """A request ends: with prefix_cache, its cells keep the keys of its
        tokens so far (the prompt and the reply but its last sample: the
        reference keeps them in the idle slot and publishes its tail when
        it reuses the slot, engine.lua:1042-1052, E:publish_tail
        :1906-1918), so a follow-up prompt that repeats them attaches them
        (E:pick_slot / E:reuse, :1704-1819); then its blocks go back (the
        keyed ones stay cached until evicted)."""
        if self.prefix_cache and req.seq is not None and not self.ring_blocks:
            hist, _ = req.history()
            if req.seq.n_past == len(hist):
                self.publish_tail(req, hist)
        self.seqs.free(req.seq)
        self.free_slots.append(req.slot)
        req.done = True
        self.active.remove(req)
        self._ended += 1

    # -- a full pool ------------------------------------------------------------
    def victim(self, req):
        """E:victim (engine.lua:1410-1420): a running request of lower
        priority than req whose cells can go: the lowest priority, the least
        recently started first; or None."""
        best = None
        for q in self.active:
            if (q is not req and not q.preempt and not q.finishing and q.prio < req.prio and
                    (best is None or (q.prio, q.started) < (best.prio, best.started))):
                best = q
        return best

    def on_full(self, req, err):
        """An entry of req got no block (E:flush, engine.lua:1436-1448, and
        the callers of E:preempt, :2230-2233,3178-3187): a running request of
        lower priority lets its cells go and req runs in a later pass; with
        none, req itself lets its cells go and waits, or, alone or on a model
        with rings, its reply ends. Returns True when req ended."""
        v = self.victim(req)
        if v is not None:
            v.preempt = True
            return False
        running = sum(1 for q in self.active if not q.preempt and not q.finishing)
        if running < 2:
            req.err = str(err)
            return True
        req.preempt = True
        return False

    def publish_tail(self, req, tokens):
        """E:publish_tail (engine.lua:1906-1918): keys for the full blocks of
        the sequence's tokens, and the partial-block marker of its last
        block, so that the request finds its cells again."""
        c, alloc = req.seq, self.seqs.alloc
        self.publish_tokens(req, tokens)
        n = min(c.n_past, len(tokens))
        i = n // BLOCK  # the partial block's index (0-based)
        if n % BLOCK and i < len(c.blocks) and len(c.keys) == i:
            alloc.publish_part(c.blocks[i], c.keys[i - 1] if i else ROOT_KEY, i + 1,
                               tokens[i * BLOCK:n], c.prio)

    def ring_bytes(self, slot):
        """The bytes of slot's ring blocks in every sliding layer's K and V
        ring pools (device uint8 views, in layer order)."""
        m, R = self.model, self.ring_blocks
        bb = hip.lib().lgmlh_kv_block_bytes(m.ring_dims[1], m.ring_dims[0])
        views = []
        for il, swa in enumerate(m.swa):
            if swa:
                for pool in (m.kpools[il], m.vpools[il]):
                    views.append(pool[slot * R * bb:(slot + 1) * R * bb])
        return views

    def checkpoint_ring(self, req):
        """E:checkpoint_slot (engine.lua:2103-2116, M:snapshot's sliding
        rings, transformer.lua:1450-1471): the slot's rings, the part of a
        sequence that cannot be rebuilt from cached blocks, to pinned host
        memory at the sequence's position."""
        views = self.ring_bytes(req.slot)
        buf = torch.empty(sum(v.numel() for v in views), dtype=torch.uint8, pin_memory=True)
        o = 0
        for v in views:
            buf[o:o + v.numel()].copy_(v, non_blocking=True)
            o += v.numel()
        torch.cuda.current_stream().synchronize()
        req.ring_ckpt = (req.seq.n_past, buf)

    def restore_ring(self, req):
        """M:restore of the rings (transformer.lua:1473-1511) into the new
        slot's ring blocks: the checkpoint holds the rings at its position,
        so it serves only a sequence that attached exactly that many tokens."""
        _, buf = req.ring_ckpt
        o = 0
        for v in self.ring_bytes(req.slot):
            v.copy_(buf[o:o + v.numel()], non_blocking=True)
            o += v.numel()
        torch.cuda.current_stream().synchronize()

    def let_go(self, req):
        """E:preempt (engine.lua:1193-1243), with no pass of req in flight: it
        publishes its blocks' keys, checkpoints its rings (a model with
        sliding layers), lets its cells and slot go and waits; its feed
        becomes its tokens so far and the rest."""
        hist, rest = req.history()
        assert req.seq.n_past == len(hist), (req.seq.n_past, len(hist))
        if self.ring_blocks:
            self.checkpoint_ring(req)
        self.publish_tail(req, hist)
        self.seqs.free(req.seq)
        self.free_slots.append(req.slot)
        self.active.remove(req)
        req.seq, req.slot = None, None
        req.feed, req.fed = hist + rest, 0
        req.preempt = req.finishing = False
        req.tok_src = None
        req.waits += 1
        req.wait_mark = self._ended
        self.waiting.append(req)
        self.preemptions += 1
        self.waits[req.prio] = self.waits.get(req.prio, 0) + 1

    def resume(self):
        """The waiting requests take a slot again, in the order they began to
        wait, once a request has ended after they began (E:preempt's wait,
        engine.lua:1223-1242, woken by E:slot_freed, :1284-1291): each
        attaches what is still cached of its tokens and runs the rest. A
        resumed request counts as started now (E:pick_slot's `best.used =
        self.tick`, :1753), so E:victim does not pick it first again. Only
        ends wake a waiter: a request that lets go frees cells for the one
        that needed them, which a waiter taking them back would undo."""
        for req in [q for q in self.waiting if self._ended > q.wait_mark]:
            if not self.free_slots:
                break
            self.waiting.remove(req)
            req.slot = self.free_slots.pop(0)
            req.seq = Seq(self.seqs, req.prio)
            self._submitted += 1
            req.started = self._submitted
            self.active.append(req)
            req.fed = self.attach(req)
            req.seq.n_past = req.fed
            ck = getattr(req, "ring_ckpt", None)
            if ck is not None:
                if req.fed == ck[0]:
                    self.restore_ring(req)
                else:
                    # the rings are at the checkpoint's position: without all
                    # of its tokens the sequence runs again from the start
                    self.seqs.free(req.seq)
                    req.seq = Seq(self.seqs, req.prio)
                    req.fed = 0
                req.ring_ckpt = None

    def step(self):
        """One pass over every active request; returns the requests that got
        a token. Requests whose budget is spent finish.

        A run-ahead engine launches the next pass first and then reads back
        the one launched by the previous call: it returns that pass's
        requests (last_plan, last_entries and last_logits are that pass's),
        and a decode token goes from one pass to the next on the device. The
        passes' contents do not depend on the sampled values (budgets end
        requests), so only the joining of new requests lags one pass; each
        sequence's results are the same (they do not depend on the batch)."""
        if not self.run_ahead:
            return self._step_sync()
        nxt = self._launch()
        got = self._complete(self._inflight) if self._inflight is not None else []
        self._inflight = nxt
        return got

    def drain(self):
        """Read back the pass in flight (run-ahead engines); its requests."""
        p, self._inflight = self._inflight, None
        return self._complete(p) if p is not None else []

    def _launch(self):
        """Plan and queue one pass from the launched state (positions and
        prompt progress advance at launch); None when nothing runs."""
        # requests that must let their cells go do so once nothing of theirs
        # is in flight; then the waiting ones may come back
        for r in [q for q in self.active if q.preempt and not q.finishing and not q.n_inflight]:
            self.let_go(r)
        self.resume()
        entries = []
        left = self.max_tokens if self.max_tokens else 1 << 62
        n_dec = sum(1 for r in self.active
                    if not r.finishing and not r.preempt and r.fed >= len(r.feed))
        for r in list(self.active):
            if r.finishing or r.preempt:
                continue
            src = None
            if r.fed < len(r.feed):
                room = left - n_dec
                if room <= 0:
                    continue
                ids = r.feed[r.fed:r.fed + min(self.ubatch, room)]
            else:
                n_dec -= 1
                if r.tok_src is not None:
                    ids, src = [0], r.tok_src  # the token is still on the device
                else:
                    ids = [r.out[-1]]
            left -= len(ids)
            try:
                self.seqs.reserve(r.seq, r.seq.n_past + len(ids))
            except PoolFull as e:
                if self.on_full(r, e):
                    if r.n_inflight:
                        r.finishing = True
                    else:
                        self.finish(r)
                continue
            entries.append((r, ids, src))
        # a request whose cells must go drops out of the pass (E:flush,
        # engine.lua:1450-1456)
        entries = [e for e in entries if not e[0].preempt]
        for r in [q for q in self.active if q.preempt and not q.finishing and not q.n_inflight]:
            self.let_go(r)
        if not entries:
            return None
        groups = [entries]
        if self.n_streams == 2 and len(entries) >= 2:
            groups = [entries[0::2], entries[1::2]]
        main = torch.cuda.current_stream()
        if len(groups) > 1:
            # the side stream starts after all the work queued so far
            ev = torch.cuda.Event()
            ev.record(main)
            self._side.wait_event(ev)
        p = _Pass()
        p.halves, p.entries = [], []
        for gi, ents in enumerate(groups):
            st = main if gi == 0 else self._side
            with torch.cuda.stream(st):
                p.halves.append(self._launch_half(ents, gi, main))
        if len(groups) > 1:
            # and the main stream goes on after both halves
            ev = torch.cuda.Event()
            ev.record(self._side)
            main.wait_event(ev)
        self.launched_plans = [h.plan for h in p.halves]
        self.launched_plan = self.launched_plans[0]
        for h in p.halves:
            for row, (r, x, _) in enumerate(h.entries):
                r.seq.n_past += len(x)
                prompt = r.fed < len(r.feed)
                sampled = True
                if prompt:
                    r.fed += len(x)
                    sampled = r.fed >= len(r.feed)  # mid-prompt chunk: not sampled
                if sampled:
                    r.n_inflight += 1
                    r.tok_src = (h, row)
                    if len(r.out) + r.n_inflight >= r.max_new:
                        r.finishing = True
                p.entries.append((r, len(x), prompt, sampled, h, row))
        return p

    def _launch_half(self, entries, slot, main):
        """Plan and queue the entries on the current stream."""
        seq_n = [len(ids) for _, ids, _ in entries]
        npast = [r.seq.n_past for r, _, _ in entries]
        mb = max(len(r.seq.blocks) for r, _, _ in entries)
        bt = np.full((len(entries), mb), -1, np.int32)
        for i, (r, _, _) in enumerate(entries):
            bt[i, :len(r.seq.blocks)] = r.seq.blocks
        ids = np.concatenate([np.asarray(x, np.int32) for _, x, _ in entries])
        ring_tab = None
        if self.ring_blocks:
            R = self.ring_blocks
            ring_tab = np.array([np.arange(r.slot * R, (r.slot + 1) * R) for r, _, _ in entries],
                                np.int32)
        plan = self.model.plan(seq_n, npast, bt, ids, self.bps, ring_tab=ring_tab)
        # decode tokens still on the device: copied into the plan's ids
        # (and the ring plan's) from the previous pass's samples
        off = np.cumsum([0] + seq_n[:-1])
        by_src = {}
        for i, (_, _, src) in enumerate(entries):
            if src is not None:
                by_src.setdefault(id(src[0]), (src[0], [], []))
                by_src[id(src[0])][1].append(int(off[i]))
                by_src[id(src[0])][2].append(src[1])
        cur = torch.cuda.current_stream()
        for h, dst, rows in by_src.values():
            di = torch.from_numpy(np.array(dst, np.int64)).pin_memory().to("cuda", non_blocking=True)
            ri = torch.from_numpy(np.array(rows, np.int64)).pin_memory().to("cuda", non_blocking=True)
            h.ids_dev.record_stream(cur)  # the source may come from the other stream
            vals = h.ids_dev.index_select(0, ri)
            plan.dev_ids().index_copy_(0, di, vals)
            if plan.ring is not None:
                plan.ring.dev_ids().index_copy_(0, di, vals)
        logits = self.model.forward(plan, trace=self.trace, slot=slot)
        n = len(entries)
        h = _Half()
        h.plan, h.logits, h.entries = plan, logits, entries
        h.ids_dev = torch.empty(n, dtype=torch.int32, device="cuda")
        check(hip.lib().lgmlh_argmax(logits.data_ptr(), n, self.model.hp["n_vocab"],
                                     h.ids_dev.data_ptr(), stream()))
        h.ids_host = torch.empty(n, dtype=torch.int32, pin_memory=True)
        h.ids_host.copy_(h.ids_dev, non_blocking=True)
        h.event = torch.cuda.Event()
        h.event.record()
        return h

    def _complete(self, p):
        """Read back a launched pass: its sampled tokens, prefix-cache keys of
        its prompt chunks, and the requests that end with it."""
        toks = {}
        for h in p.halves:
            h.event.synchronize()
            toks[id(h)] = h.ids_host.numpy()
        self.last_plans = [h.plan for h in p.halves]
        self.last_plan = self.last_plans[0]
        self._last_halves = p.halves
        self._last_logits = None
        self.last_entries = [r for r, _, _, _, _, _ in p.entries]
        self.passes += 1
        self.rows += len(p.entries)
        self.tokens += sum(n for _, n, _, _, _, _ in p.entries)
        got = []
        for r, _, prompt, sampled, h, row in p.entries:
            if r.done:
                continue  # ended at launch (a pool-full reserve) with only a prompt chunk in flight
            if prompt and self.prefix_cache and r.seq is not None:
                self.publish(r)  # (a request that let its cells go has no sequence)
            if sampled:
                r.out.append(int(toks[id(h)][row]))
                r.n_inflight -= 1
                if r.tok_src is not None and r.tok_src[0] is h:
                    r.tok_src = None
                got.append(r)
            if r.finishing and r.n_inflight == 0 and not r.done:
                self.finish(r)
        return got

    @property
    def last_logits(self):
        """Logits of the last pass read back, rows in last_entries order."""
        if self._last_logits is None and self._last_halves:
            hs = self._last_halves
            self._last_logits = hs[0].logits if len(hs) == 1 else torch.cat(
                [h.logits for h in hs])
        return self._last_logits

    @last_logits.setter
    def last_logits(self, v):
        self._last_logits = v
        self._last_halves = None

    def _step_sync(self):
        self.resume()
        entries = []
        left = self.max_tokens if self.max_tokens else 1 << 62
        n_dec = sum(1 for r in self.active if r.fed >= len(r.feed))
        for r in list(self.active):
            if r.preempt:
                continue
            ids = r.pending(self.ubatch)
            if r.fed < len(r.feed):
                # a prompt chunk takes what the decode tokens leave
                room = left - n_dec
                if room <= 0:
                    continue
                ids = ids[:room]
            else:
                n_dec -= 1
            left -= len(ids)
            try:
                self.seqs.reserve(r.seq, r.seq.n_past + len(ids))
            except PoolFull as e:
                if self.on_full(r, e):
                    self.finish(r)
                continue
            entries.append((r, ids))
        # the requests whose cells go drop out of the pass and wait (E:flush,
        # engine.lua:1450-1456)
        for r in [q for q in self.active if q.preempt]:
            self.let_go(r)
        entries = [(r, ids) for r, ids in entries if r.seq is not None]
        if not entries:
            return []
        seq_n = [len(ids) for _, ids in entries]
        npast = [r.seq.n_past for r, _ in entries]
        mb = max(len(r.seq.blocks) for r, _ in entries)
        bt = np.full((len(entries), mb), -1, np.int32)
        for i, (r, _) in enumerate(entries):
            bt[i, :len(r.seq.blocks)] = r.seq.blocks
        ids = np.concatenate([np.asarray(x, np.int32) for _, x in entries])
        ring_tab = None
        if self.ring_blocks:
            R = self.ring_blocks
            ring_tab = np.array([np.arange(r.slot * R, (r.slot + 1) * R) for r, _ in entries],
                                np.int32)
        plan = self.model.plan(seq_n, npast, bt, ids, self.bps, ring_tab=ring_tab)
        self.last_plan = self.launched_plan = plan
        self.last_plans = self.launched_plans = [plan]
        self.last_entries = [r for r, _ in entries]
        logits = self.model.forward(plan, trace=self.trace)
        self.last_logits = logits
        if self._ids.numel() < len(entries):
            self._ids = torch.empty(len(entries), dtype=torch.int32, device="cuda")
        check(hip.lib().lgmlh_argmax(logits.data_ptr(), len(entries), self.model.hp["n_vocab"],
                                     self._ids.data_ptr(), stream()))
        nxt = self._ids[:len(entries)].cpu().numpy()
        self.passes += 1
        self.rows += len(entries)
        self.tokens += int(sum(seq_n))
        got = []
        for (r, x), tok in zip(entries, nxt):
            r.seq.n_past += len(x)
            if r.fed < len(r.feed):
                r.fed += len(x)
                if self.prefix_cache:
                    self.publish(r)
                if r.fed < len(r.feed):
                    continue  # mid-prompt chunk: its logits are not sampled
            r.out.append(int(tok))
            got.append(r)
            if len(r.out) >= r.max_new:
                self.finish(r)
        return got
