"""HBM slot pool with the reference's ExpertPool API.

Storage follows engine_v3.py:180-206: one device array per component,
shaped [n_slots, *shape] in its final dtype (uint32 codes are held in int32
tensors, bit-identical), named "{proj}.{part}", exposed as `.views`.

Fills replace ExpertPool._read (engine_v3.py:255-290): a record of the
expert store (pinned host memory or HBM, repacked layout) is copied into
the slot's component rows by hipMemcpyAsync, on a side stream for
prefetches and on the compute stream for demand misses.  Completion is an
event: an acquire of a key whose prefetch is still in flight makes the
compute stream wait on that event instead of blocking the host, and a
prefetch fill waits for the compute work already enqueued, so a slot is
never refilled while a kernel reads it (the guarantee `needs_barrier` gave
with a host sync, engine_v3.py:228-231,601-607).

Bookkeeping (engine_v3.py:213-236, 303-464): (layer, expert) -> slot table,
sampled LFU/LRU eviction with a young-entry window, the free list popped from
the end, pinned slots of the current layer, pending prefetches, hit/miss
statistics.
"""
from __future__ import annotations

import ctypes as C
import os
from collections import defaultdict

import numpy as np
import torch

from . import _lib
from .geometry import Geometry

SAMPLE = 24            # engine_v3.py:322
STRIDE = 7919          # engine_v3.py:336
YOUNG = 1 << 30        # engine_v3.py:349


class HostStore:
    """Pinned host expert store: n_records records of geom.record_bytes in
    the repacked layout (hipHostMalloc through the C ABI)."""

    def __init__(self, geom: Geometry, n_records: int):
        self.geom = geom
        self.n_records = n_records
        self.record_bytes = geom.record_bytes
        self.nbytes = n_records * geom.record_bytes
        p = C.c_void_p()
        _lib.check(_lib.lib().moe_host_alloc(self.nbytes, C.byref(p)))
        self.ptr = p.value
        buf = (C.c_uint8 * self.nbytes).from_address(self.ptr)
        self.array = np.frombuffer(buf, dtype=np.uint8).reshape(n_records, self.record_bytes)

    def close(self):
        if self.ptr:
            self.array = None
            _lib.check(_lib.lib().moe_host_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _torch_dtype(c) -> torch.dtype:
    return torch.int32 if c.dtype == "U32" else torch.bfloat16


class SlotPool:
    """Device arrays of the pool and the C view the kernels read."""

    def __init__(self, geom: Geometry, n_slots: int, device="cuda", store=None):
        self.geom = geom
        self.n_slots = n_slots
        self.device = torch.device(device)
        self.views = {}
        for c in geom.components:
            self.views[c.name] = torch.zeros((n_slots, *c.shape), dtype=_torch_dtype(c),
                                             device=self.device)
        self.pool_bytes = sum(a.numel() * a.element_size() for a in self.views.values())
        self.store = store           # torch uint8 [n_records, record_bytes] or HostStore
        self._view = None

    # -- the C view -------------------------------------------------------
    def _store_ptr(self):
        s = self.store
        if s is None:
            return None, 0, 0
        if isinstance(s, HostStore):
            return s.ptr, s.record_bytes, s.n_records
        assert s.dtype == torch.uint8 and s.dim() == 2 and s.is_contiguous()
        return s.data_ptr(), s.shape[1], s.shape[0]

    def c_view(self) -> _lib.PoolView:
        if self._view is None:
            v = _lib.PoolView()
            v.n_components = self.geom.n_components
            v.n_slots = self.n_slots
            for i, c in enumerate(self.geom.components):
                a = self.views[c.name]
                v.base[i] = a.data_ptr()
                v.slot_bytes[i] = c.nbytes
                v.comp_offset[i] = c.offset
            sp, rb, nr = self._store_ptr()
            if sp is not None and not isinstance(self.store, HostStore):
                v.store, v.record_bytes, v.n_records = sp, rb, nr
            else:
                v.store, v.record_bytes, v.n_records = None, 0, 0
            self._view = v
        return self._view

    # -- fills --------------------------------------------------------------
    def fill(self, records, slots, stream=None, src=None):
        """Copy whole records of the store (or of `src`) into slots."""
        recs = np.ascontiguousarray(np.asarray(records, dtype=np.int64))
        sl = np.ascontiguousarray(np.asarray(slots, dtype=np.int32))
        if recs.shape != sl.shape:
            raise ValueError("records and slots differ in length")
        src = self.store if src is None else src
        if src is None:
            raise ValueError("no store to fill from")
        if isinstance(src, HostStore):
            sp, rb, nr = src.ptr, src.record_bytes, src.n_records
        else:
            sp, rb, nr = src.data_ptr(), src.shape[1], src.shape[0]
        if len(recs) and (recs.min() < 0 or recs.max() >= nr):
            raise ValueError(f"record index outside [0, {nr})")
        _lib.check(_lib.lib().moe_fill_slots(
            C.byref(self.c_view()), sp, rb, recs.ctypes.data, sl.ctypes.data,
            len(sl), _lib.stream_ptr(stream)))

    def read_slot(self, slot: int) -> dict:
        """Host copy of every component of one slot (for verification)."""
        return {n: a[slot].cpu() for n, a in self.views.items()}


class ExpertPool(SlotPool):
    """Fixed pool of expert slots with stream-ordered fills and LFU eviction;
    the API of engine_v3.ExpertPool (engine_v3.py:125-464)."""

    def __init__(self, geom: Geometry, n_slots: int, store, device="cuda",
                 evict: str | None = None, depths=(1,), widen: int = 1,
                 side_stream: torch.cuda.Stream | None = None):
        super().__init__(geom, n_slots, device, store)
        self.n_experts = geom.n_experts
        self.n_layers = geom.n_layers
        self.top_k = geom.top_k
        self.group_size = geom.group_size
        self.bits = geom.bits
        self.blob = geom.record_bytes
        self.depths = tuple(depths)
        self.widen = widen
        self.evict = (evict or os.environ.get("MOE_EVICT", "lfu")).lower()
        self.window = 24 * max(1, self.depths[0])      # engine_v3.py:310-311
        self.slot_of = {}
        self.key_of = [None] * n_slots
        self.freq = defaultdict(int)
        self.free = list(range(n_slots))
        self.pending = {}            # key -> torch.cuda.Event of its fill
        self.from_prefetch = set()
        self.pinned = set()
        self.clock = 0
        self.born = {}
        self.last_use = {}
        self.use_clock = 0
        per_token = self.n_layers * self.top_k * (1 + len(self.depths))
        # Kept for API compatibility; slot reuse is ordered by events here.
        self.needs_barrier = n_slots < per_token * 1.25
        self.n_prefetch_hit = self.n_cache_hit = self.n_miss = 0
        self.n_prefetch_bail = self.n_prefetch_issued = 0
        self.bytes_read = 0
        self.bytes_exposed = 0
        self.side = side_stream if side_stream is not None else torch.cuda.Stream(device=self.device)

    # -- internals (engine_v3.py:313-380) -----------------------------------
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
                raise RuntimeError("pool exhausted: every slot pinned or pending")
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

    def _touch(self, key):
        self.use_clock += 1
        self.last_use[key] = self.use_clock
        self.freq[key] += 1

    def _record(self, key) -> int:
        layer, expert = key
        return layer * self.n_experts + expert

    def complete(self, key):
        """A prefetch fill has finished (engine_v3.py:292-301)."""
        if self.pending.pop(key, None) is not None:
            self.from_prefetch.add(key)

    def poll(self):
        """Retire prefetch fills whose events have completed."""
        for key in [k for k, ev in self.pending.items() if ev.query()]:
            self.complete(key)

    def _read(self, slot, layer, expert, stream=None):
        """Fill one slot now, on `stream` (default: current stream)."""
        self.fill([self._record((layer, expert))], [slot], stream=stream)
        self.bytes_read += self.blob

    # -- public (engine_v3.py:383-464) --------------------------------------
    def prefetch(self, layer, experts):
        """Non-blocking: fill slots a later layer will probably want."""
        self.poll()
        compute = torch.cuda.current_stream(self.device)
        issued = []
        for e in experts:
            key = (layer, int(e))
            if key in self.slot_of or key in self.pending:
                continue
            try:
                slot = self._alloc(key)
            except RuntimeError:
                self.n_prefetch_bail += 1
                break
            self.n_prefetch_issued += 1
            issued.append((key, slot))
        if issued:
            self.side.wait_stream(compute)     # no refill under a running kernel
            self.fill([self._record(k) for k, _ in issued], [s for _, s in issued],
                      stream=self.side)
            ev = torch.cuda.Event()
            ev.record(self.side)
            for key, _ in issued:
                self.pending[key] = ev
            self.bytes_read += len(issued) * self.blob

    def acquire(self, layer, experts):
        """Returns the slot holding each expert.  Misses are filled on the
        compute stream; in-flight prefetches become stream waits."""
        self.poll()
        compute = torch.cuda.current_stream(self.device)
        n = len(experts)
        slots = [None] * n
        waits, issue = [], []
        for i, e in enumerate(experts):
            key = (layer, int(e))
            ev = self.pending.get(key)
            slot = self.slot_of.get(key)
            missed = False
            if ev is None and slot is None:
                slot = self._alloc(key)
                self.pinned.add(slot)
                self._touch(key)
                issue.append((i, key, slot))
                missed = True
            elif slot is not None:
                self.pinned.add(slot)
                self._touch(key)
            if ev is not None:
                waits.append((i, key, ev))
            elif slot is not None and not missed:
                early = key in self.from_prefetch
                self.from_prefetch.discard(key)
                self.n_prefetch_hit += 1 if early else 0
                self.n_cache_hit += 0 if early else 1
                slots[i] = slot
            if missed:
                slots[i] = slot
        self.bytes_exposed += len(issue) * self.blob
        if issue:
            self.fill([self._record(k) for _, k, _ in issue], [s for _, _, s in issue],
                      stream=compute)
            self.bytes_read += len(issue) * self.blob
        for i, key, ev in waits:
            compute.wait_event(ev)
            self.complete(key)
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
                    gb=self.bytes_read / 2 ** 30, bail=self.n_prefetch_bail,
                    issued=self.n_prefetch_issued,
                    exposed_gb=self.bytes_exposed / 2 ** 30)
