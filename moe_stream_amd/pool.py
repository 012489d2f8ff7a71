"""HBM slot pool with the reference's ExpertPool API.

Storage follows engine_v3.py:180-206: one device array per component,
shaped [n_slots, *shape] in its final dtype (uint32 codes are held in int32
tensors, bit-identical), named "{proj}.{part}", exposed as `.views`.

Two layouts of that storage in HBM.  "components": the component arrays
back to back in one allocation (the layout the whole-token decode kernels
require).  "records": slot s holds one whole store record at s x
record_bytes, each component view a strided view into it (the same
[n_slots, *shape] arrays to every reader); ExpertPool's default, since a fill
is then one copy per record.

Fills replace ExpertPool._read (engine_v3.py:255-290): a record of the
expert store (pinned host memory or HBM, repacked layout) is copied into
the slot -- one hipMemcpyAsync per record on the copy engines for the
record layout, copy kernels otherwise -- on a side stream for prefetches
and on the compute stream for demand misses.  Completion is an
event: an acquire of a key whose prefetch is still in flight makes the
compute stream wait on that event instead of blocking the host, and a
prefetch fill first waits for the compute work already enqueued, so a slot
is never refilled while a kernel reads it (the guarantee `needs_barrier`
gave with a host sync, engine_v3.py:228-231,601-607).

Bookkeeping -- the (layer, expert) -> slot table, sampled LFU/LRU eviction
with a young-entry window, pinned and pending slots, hit/miss statistics
(engine_v3.py:213-236, 303-464) -- runs in the native policy
(moe_stream_amd.policy.NativePolicy).
"""
from __future__ import annotations

import ctypes as C
import os
import time

import numpy as np
import torch

from . import _lib
from .geometry import Geometry
from .policy import NativePolicy, PoolExhausted, SlotOf


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


def _norm_device(device) -> torch.device:
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    return d


def _torch_dtype(c) -> torch.dtype:
    return torch.int32 if c.dtype == "U32" else torch.bfloat16


class SlotPool:
    """Device arrays of the pool and the C view the kernels read."""

    def __init__(self, geom: Geometry, n_slots: int, device="cuda", store=None,
                 layout: str = "components"):
        if layout not in ("components", "records"):
            raise ValueError(f"layout {layout!r}: 'components' or 'records'")
        self.geom = geom
        self.n_slots = n_slots
        self.device = _norm_device(device)
        self.layout = layout
        self.views = {}
        if layout == "components":
            # one array per component, [n_slots, *shape] in its final dtype,
            # all in one allocation back to back in component order
            self._buf = torch.zeros(n_slots * geom.payload_bytes, dtype=torch.uint8,
                                    device=self.device)
            for c in geom.components:
                part = self._buf[n_slots * c.offset:n_slots * (c.offset + c.nbytes)]
                self.views[c.name] = part.view(_torch_dtype(c)).view(n_slots, *c.shape)
        else:
            # slot s = store record layout at s * record_bytes; component c at
            # its record offset (16-byte multiples, so every dtype view aligns)
            rb = geom.record_bytes
            self._buf = torch.zeros(n_slots * rb, dtype=torch.uint8, device=self.device)
            for c in geom.components:
                dt = _torch_dtype(c)
                es = torch.empty((), dtype=dt).element_size()
                assert rb % es == 0 and c.offset % es == 0
                inner = [int(np.prod(c.shape[i + 1:])) for i in range(len(c.shape))]
                self.views[c.name] = torch.as_strided(
                    self._buf.view(dt), (n_slots, *c.shape), (rb // es, *inner),
                    c.offset // es)
        self.pool_bytes = sum(a.numel() * a.element_size() for a in self.views.values())
        self.store = store           # torch uint8 [n_records, record_bytes] or HostStore
        self._view = None

    # -- the C view -------------------------------------------------------
    def c_view(self) -> _lib.PoolView:
        if self._view is None:
            v = _lib.PoolView()
            v.n_components = self.geom.n_components
            v.n_slots = self.n_slots
            rec = self.layout == "records"
            for i, c in enumerate(self.geom.components):
                v.base[i] = self.views[c.name].data_ptr()
                v.slot_bytes[i] = self.geom.record_bytes if rec else c.nbytes
                v.comp_offset[i] = c.offset
            s = self.store
            if isinstance(s, torch.Tensor):
                assert s.dtype == torch.uint8 and s.dim() == 2 and s.is_contiguous()
                v.store, v.record_bytes, v.n_records = s.data_ptr(), s.shape[1], s.shape[0]
            else:   # no store, or a host store the kernels must not read over PCIe
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
        if len(sl) and (sl.min() < 0 or sl.max() >= self.n_slots):
            raise ValueError(f"slot outside [0, {self.n_slots})")
        _lib.check(_lib.lib().moe_fill_slots(
            C.byref(self.c_view()), sp, rb, nr, recs.ctypes.data, sl.ctypes.data,
            len(sl), _lib.stream_ptr(stream)))

    def read_slot(self, slot: int) -> dict:
        """Host copy of every component of one slot (for verification)."""
        return {n: a[slot].cpu() for n, a in self.views.items()}


# The reference's defaults (engine_v3.py:59-60): pool slots and fill workers.
N_SLOTS = int(os.environ.get("PF_SLOTS", "3072"))
N_WORKERS = int(os.environ.get("PF_WORKERS", "4"))


def env_depths() -> tuple:
    """Prefetch depths from PF_DEPTH, a comma-separated list (default "1";
    engine_v3.py:61-62): the first is the depth whose recall is tracked and
    which sizes the young-entry window."""
    raw = os.environ.get("PF_DEPTH", "1")
    try:
        d = tuple(int(v) for v in raw.split(","))
    except ValueError:
        raise ValueError(f"PF_DEPTH={raw!r}: a comma-separated list of integers") from None
    if not d or any(v <= 0 for v in d):
        raise ValueError(f"PF_DEPTH={raw!r}: depths must be positive")
    return d


def env_widen() -> int:
    """Speculation width from PF_WIDEN (default 1; engine_v3.py:84): the
    lookahead fetches the top k * PF_WIDEN predicted experts."""
    raw = os.environ.get("PF_WIDEN", "1")
    try:
        w = int(raw)
    except ValueError:
        raise ValueError(f"PF_WIDEN={raw!r}: an integer") from None
    if w <= 0:
        raise ValueError(f"PF_WIDEN={raw!r}: must be positive")
    return w


class ExpertPool(SlotPool):
    """Fixed pool of expert slots with stream-ordered fills and LFU eviction;
    the API of engine_v3.ExpertPool (engine_v3.py:125-464): `prefetch`,
    `acquire`, `stats`, `views`, `slot_of`, `pending`, `pinned`,
    `needs_barrier`, `bytes_read`, `_read`.

    Construction as the reference's, ExpertPool(model_dir, n_slots,
    n_workers) (engine_v3.py:128): `model_dir` holds experts.bin +
    experts_index.json, whose records are loaded into a pinned host store by
    `n_workers` reader threads; fills then cross the host link from there.
    Or ExpertPool(geom, n_slots, store=...) over a store already in pinned
    host memory (HostStore) or HBM (uint8 [n_records, record_bytes])."""

    def __init__(self, model_dir, n_slots: int = N_SLOTS, n_workers: int = N_WORKERS,
                 store=None, device="cuda", evict: str | None = None, depths=None,
                 widen: int | None = None, side_stream: torch.cuda.Stream | None = None,
                 n_layers: int | None = None, layout: str = "records"):
        if isinstance(model_dir, Geometry):
            geom = model_dir
            if store is None:
                raise ValueError("ExpertPool(geom, ...) needs store=")
        else:
            from .store import ExpertStoreFile
            sf = ExpertStoreFile(os.fspath(model_dir))
            geom = sf.geom
            if store is None:
                store = sf.to_host_store(n_workers=n_workers)
            n_layers = n_layers or sf.index.n_layers
        super().__init__(geom, n_slots, device, store, layout=layout)
        self.n_workers = n_workers
        self.n_experts = geom.n_experts
        self.n_layers = n_layers or geom.n_layers
        self.top_k = geom.top_k
        self.group_size = geom.group_size
        self.bits = geom.bits
        self.blob = geom.record_bytes
        # PF_DEPTH / PF_WIDEN from the environment unless given
        self.depths = tuple(depths) if depths is not None else env_depths()
        self.widen = int(widen) if widen is not None else env_widen()
        self.evict = (evict or os.environ.get("MOE_EVICT", "lfu")).lower()
        self.policy = NativePolicy(n_slots, self.n_layers, self.n_experts,
                                   evict=self.evict, depth=self.depths[0])
        self.slot_of = SlotOf(self.policy)
        self.pending = {}            # key -> torch.cuda.Event of its fill
        self.pinned = set()
        per_token = self.n_layers * self.top_k * (1 + len(self.depths))
        # kept for callers; slot reuse is ordered by events, not host syncs
        self.needs_barrier = n_slots < per_token * 1.25
        self.bytes_read = 0
        self.bytes_exposed = 0
        self.side = side_stream if side_stream is not None else torch.cuda.Stream(device=self.device)
        # telemetry of engine_v3.py:238-250, for stream-ordered fills:
        # t_blocked = host seconds inside acquire from issuing its misses to
        # returning; busy_s = device seconds with >= 1 fill in flight (from
        # timing events around every fill batch); depth = mean number of
        # records in flight when a record's fill is issued
        self.t_blocked = 0.0
        self.depth_sum = 0
        self.depth_n = 0
        self._fills = []             # (start event, end event, records) in flight
        self._spans = []             # completed fills: (start ms, end ms) from _t0
        self._busy_done_ms = 0.0     # busy time of spans already merged away
        self._t0 = torch.cuda.Event(enable_timing=True)
        self._t0.record(torch.cuda.current_stream(self.device))

    def _record(self, layer, expert) -> int:
        return layer * self.n_experts + int(expert)

    def _retire_fills(self):
        keep = []
        for a, b, n in self._fills:
            if b.query():
                self._spans.append((self._t0.elapsed_time(a), self._t0.elapsed_time(b)))
            else:
                keep.append((a, b, n))
        self._fills = keep
        if len(self._spans) > 4096:
            self._merge_spans(keep_last=True)

    def _merge_spans(self, keep_last: bool):
        """Fold completed spans into busy time (a union of intervals); with
        keep_last the latest merged interval stays open for later overlaps."""
        spans = sorted(self._spans)
        merged = []
        for a, b in spans:
            if merged and a <= merged[-1][1]:
                merged[-1][1] = max(merged[-1][1], b)
            else:
                merged.append([a, b])
        last = merged.pop() if (keep_last and merged) else None
        self._busy_done_ms += sum(b - a for a, b in merged)
        self._spans = [tuple(last)] if last is not None else []

    def _fill_tracked(self, records, slots, stream):
        """fill() with the telemetry of _read (engine_v3.py:255-262, 286-290)."""
        self._retire_fills()
        inflight = sum(n for _, _, n in self._fills)
        n = len(slots)
        self.depth_sum += n * inflight + n * (n + 1) // 2
        self.depth_n += n
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        self.fill(records, slots, stream=stream)
        b.record(stream)
        self._fills.append((a, b, n))
        self.bytes_read += n * self.blob

    def poll(self):
        """Retire prefetch fills whose events have completed
        (the worker epilogue, engine_v3.py:292-301)."""
        done = [k for k, ev in self.pending.items() if ev.query()]
        for key in done:
            self.pending.pop(key)
            self.policy.complete(*key)

    def _read(self, slot, layer, expert, stream=None):
        """Fill one slot now, on `stream` (default: the current stream)."""
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        self._fill_tracked([self._record(layer, expert)], [slot], s)

    # -- public (engine_v3.py:383-464) --------------------------------------
    def prefetch(self, layer, experts):
        """Non-blocking: fill slots a later layer will probably want; bails
        silently when every slot is pinned or pending."""
        self.poll()
        slots, exps, _ = self.policy.prefetch(layer, experts)
        if len(slots):
            compute = torch.cuda.current_stream(self.device)
            self.side.wait_stream(compute)          # no refill under a running kernel
            try:
                self._fill_tracked([self._record(layer, e) for e in exps], slots, self.side)
                ev = torch.cuda.Event()
                ev.record(self.side)
            except BaseException:
                # no fill (or no event) for these: unmap them so a later
                # acquire refills them instead of reading the slots
                for e in exps:
                    self.policy.cancel(layer, int(e))
                raise
            for e in exps:
                self.pending[(layer, int(e))] = ev

    def acquire(self, layer, experts):
        """The slot holding each expert.  Misses are filled on the compute
        stream; in-flight prefetches become stream waits; raises
        RuntimeError when the pool is exhausted (engine_v3.py:355-356)."""
        self.poll()
        compute = torch.cuda.current_stream(self.device)
        try:
            slots, miss, wait = self.policy.acquire(layer, experts)
        except PoolExhausted as e:
            raise RuntimeError(str(e)) from None
        t0 = time.perf_counter()
        ex = np.asarray(experts).reshape(-1)
        if len(miss):
            self._fill_tracked([self._record(layer, ex[i]) for i in miss], slots[miss], compute)
            self.bytes_exposed += len(miss) * self.blob
        for i in wait:
            ev = self.pending.pop((layer, int(ex[i])), None)
            if ev is not None:
                compute.wait_event(ev)
        self.t_blocked += time.perf_counter() - t0
        self.pinned = set(int(s) for s in slots)
        return [int(s) for s in slots]

    def device_table(self) -> torch.Tensor:
        """int32 [n_layers, n_experts] slot table on the device (-1 = absent)."""
        return torch.from_numpy(self.policy.table()).to(self.device)

    @property
    def busy_s(self) -> float:
        """Device seconds with at least one fill in flight (fills completed
        so far); a float attribute, as the reference's (engine_v3.py:247)."""
        self._retire_fills()
        self._merge_spans(keep_last=True)
        return (self._busy_done_ms + sum(b - a for a, b in self._spans)) / 1e3

    def stats(self):
        """The reference's keys (engine_v3.py:456-464)."""
        s = self.policy.stats()
        return dict(total=s["total"], prefetch=s["prefetch"], cache=s["cache"],
                    miss=s["miss"], blocked=self.t_blocked, gb=self.bytes_read / 2 ** 30,
                    busy_s=self.busy_s, depth=self.depth_sum / max(1, self.depth_n),
                    bail=s["bail"], issued=s["issued"],
                    exposed_gb=self.bytes_exposed / 2 ** 30)
