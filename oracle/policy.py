"""Pure-Python restatement of ExpertPool's slot bookkeeping (no I/O).

TEST INFRASTRUCTURE ONLY (the checker for the pool policy of the product).

Follows engine_v3.py:214-236 (state), :303-311 (protect window),
:313-374 (_alloc, sampled LFU/LRU/asis eviction), :376-380 (_touch),
:383-396 (prefetch), :398-454 (acquire), :456-464 (stats).

The reference runs fills on worker threads and learns of their completion
when `_read_task` returns (engine_v3.py:292-301).  Here completion is an
explicit call, `complete(key)`, so that a recorded sequence of
prefetch/acquire/complete calls replays deterministically.  An acquire of a
key whose prefetch is still pending is the reference's "wait" branch
(engine_v3.py:423-446): the key is touched in the loop and again after the
wait, and counts as a prefetch hit.

Parity status: pinned by hand-derived known answers on tiny pools (free list
popped from the end, stride-7919 sampling order, young-entry protection,
pinned/pending exclusion, exhaustion), by invariants on random traces, and
against `prefetch_simulator` below, a restatement of the reference's own
second model of the same pool (tests/test_policy.py).
"""
from __future__ import annotations

from collections import defaultdict

SAMPLE = 24            # engine_v3.py:322
STRIDE = 7919          # engine_v3.py:336
YOUNG = 1 << 30        # engine_v3.py:349


class PoolExhausted(RuntimeError):
    pass


class PolicyOracle:
    def __init__(self, n_slots: int, evict: str = "lfu", depth: int = 1,
                 window: int | None = None):
        self.n_slots = n_slots
        self.evict = evict
        # engine_v3.py:310-311; explicit `window` for small hand-made cases
        self.window = 24 * max(1, depth) if window is None else window
        self.slot_of = {}
        self.key_of = [None] * n_slots
        self.freq = defaultdict(int)
        self.free = list(range(n_slots))
        self.pending = set()
        self.from_prefetch = set()
        self.pinned = set()
        self.clock = 0
        self.born = {}
        self.last_use = {}
        self.use_clock = 0
        self.n_prefetch_hit = 0
        self.n_cache_hit = 0
        self.n_miss = 0
        self.n_prefetch_bail = 0
        self.n_prefetch_issued = 0
        self.fills = []          # (key, slot, kind) in issue order

    # engine_v3.py:313-374
    def _alloc(self, key):
        self.clock += 1
        if self.free:
            slot = self.free.pop()
        else:
            victim = best = None
            n = self.n_slots
            start = self.clock % n
            seen = 0
            for j in range(n):
                sidx = (start + j * STRIDE) % n
                k = self.key_of[sidx]
                if k is None or sidx in self.pinned or k in self.pending:
                    continue
                young = self.clock - self.born.get(k, 0) < self.window
                if self.evict == "asis":
                    base = 0
                elif self.evict == "lru":
                    base = self.last_use.get(k, 0)
                else:
                    base = self.freq.get(k, 0)
                f = base + (YOUNG if young else 0)
                if best is None or f < best:
                    best, victim = f, sidx
                seen += 1
                if seen >= SAMPLE and best is not None and best < YOUNG:
                    break
            if victim is None:
                raise PoolExhausted("pool exhausted: every slot pinned or pending")
            vk = self.key_of[victim]
            self.from_prefetch.discard(vk)
            self.born.pop(vk, None)
            self.last_use.pop(vk, None)
            self.freq.pop(vk, None)
            del self.slot_of[vk]
            slot = victim
        self.key_of[slot] = key
        self.slot_of[key] = slot
        self.born[key] = self.clock
        return slot

    # engine_v3.py:376-380
    def _touch(self, key):
        self.use_clock += 1
        self.last_use[key] = self.use_clock
        self.freq[key] += 1

    # engine_v3.py:383-396
    def prefetch(self, layer, experts):
        for e in experts:
            key = (layer, int(e))
            if key in self.slot_of or key in self.pending:
                continue
            try:
                slot = self._alloc(key)
            except PoolExhausted:
                self.n_prefetch_bail += 1
                return
            self.n_prefetch_issued += 1
            self.pending.add(key)
            self.fills.append((key, slot, "prefetch"))

    # engine_v3.py:292-301 (the worker's epilogue)
    def complete(self, key):
        if key in self.pending:
            self.pending.discard(key)
            self.from_prefetch.add(key)

    # engine_v3.py:398-454
    def acquire(self, layer, experts):
        n = len(experts)
        slots = [None] * n
        waits, issue = [], []
        for i, e in enumerate(experts):
            key = (layer, int(e))
            pend = key in self.pending
            slot = self.slot_of.get(key)
            missed = False
            if not pend and slot is None:
                slot = self._alloc(key)
                self.pinned.add(slot)
                self._touch(key)
                issue.append((i, key, slot))
                missed = True
            elif slot is not None:
                self.pinned.add(slot)
                self._touch(key)
            if pend:
                waits.append((i, key))
            elif slot is not None and not missed:
                early = key in self.from_prefetch
                self.from_prefetch.discard(key)
                self.n_prefetch_hit += 1 if early else 0
                self.n_cache_hit += 0 if early else 1
                slots[i] = slot
            if missed:
                slots[i] = slot
        for _, key, slot in issue:
            self.fills.append((key, slot, "miss"))
        for i, key in waits:
            # the prefetch worker finished first (its epilogue), then acquire
            self.complete(key)
            self.pending.discard(key)
            self.from_prefetch.discard(key)
            slots[i] = self.slot_of[key]
            self.pinned.add(slots[i])
            self._touch(key)
            self.n_prefetch_hit += 1
        self.n_miss += len(issue)
        self.pinned = set(s for s in slots if s is not None)
        return slots

    def stats(self):
        tot = self.n_prefetch_hit + self.n_cache_hit + self.n_miss
        return dict(total=tot, prefetch=self.n_prefetch_hit,
                    cache=self.n_cache_hit, miss=self.n_miss,
                    bail=self.n_prefetch_bail, issued=self.n_prefetch_issued)


def prefetch_simulator(true, pred, cap: int, mode: str = "lfu", window: int = 24):
    """The reference's prefetch-aware pool simulator (scratchpad/prefetch_sim.py:
    21-94), restated: a second model of ExpertPool written by the reference's
    author, used to cross-check the restatement above.

    true, pred: integer arrays [L, T, k] and [L, T, kp] of expert ids.  Per
    token and layer l: the pin set starts empty; each routed expert of layer
    l is looked up (a hit if resident, else admitted through the sampled
    eviction), recorded as a use and pinned; then every predicted expert of
    layer l + 1 that is not resident is admitted at once (reads complete
    instantly: nothing is ever pending).  Eviction is engine_v3.py's: stride
    7919 from clock % cap over at most SAMPLE unpinned candidates, base
    0 / last use / use count by mode, +2^30 for entries admitted fewer than
    `window` admissions ago; admission is not a use.
    Returns (admissions, hits, accesses)."""
    L, T = len(true), len(true[0])
    E = 1 + max(max(int(e) for row in true for ids in row for e in ids),
                max(int(e) for row in pred for ids in row for e in ids))
    key_at = [None] * cap
    where, uses, born, last = {}, defaultdict(int), {}, {}
    free = list(range(cap))
    clock = tick = admitted = hits = accesses = 0
    pins = set()

    def admit(key):
        nonlocal clock, admitted
        clock += 1
        admitted += 1
        if free:
            slot = free.pop()
        else:
            best, victim, looked = None, None, 0
            for j in range(cap):
                s = (clock % cap + j * STRIDE) % cap
                k = key_at[s]
                if k is None or s in pins:
                    continue
                base = {"asis": 0, "lru": last.get(k, 0)}.get(mode, uses.get(k, 0))
                score = base + (YOUNG if clock - born.get(k, 0) < window else 0)
                if best is None or score < best:
                    best, victim = score, s
                looked += 1
                if looked >= SAMPLE and best < YOUNG:
                    break
            if victim is None:   # every resident entry pinned: first unpinned slot
                victim = next(s for s in range(cap) if s not in pins)
            old = key_at[victim]
            del where[old]
            for d in (born, last, uses):
                d.pop(old, None)
            slot = victim
        key_at[slot] = key
        where[key] = slot
        born[key] = clock
        return slot

    for t in range(T):
        for l in range(L):
            pins = set()
            for e in true[l][t]:
                key = l * E + int(e)
                accesses += 1
                if key in where:
                    hits += 1
                else:
                    admit(key)
                tick += 1
                last[key] = tick
                uses[key] += 1
                pins.add(where[key])
            if l + 1 < L:
                for e in pred[l + 1][t]:
                    key = (l + 1) * E + int(e)
                    if key not in where:
                        admit(key)
    return admitted, hits, accesses
