"""Python handle on the native slot-pool bookkeeping (moe_policy_* in the C
ABI): the ExpertPool table and eviction policy of engine_v3.py:213-464,
running as host C++.  No device calls."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib

EVICT = {"lfu": _lib.MOE_EVICT_LFU, "lru": _lib.MOE_EVICT_LRU,
         "asis": _lib.MOE_EVICT_ASIS}


class PoolExhausted(RuntimeError):
    """Every slot is pinned or pending (engine_v3.py:355-356)."""


class NativePolicy:
    def __init__(self, n_slots: int, n_layers: int, n_experts: int,
                 evict: str = "lfu", depth: int = 1, window: int | None = None):
        self.n_slots, self.n_layers, self.n_experts = n_slots, n_layers, n_experts
        self.window = 24 * max(1, depth) if window is None else window
        h = C.c_void_p()
        _lib.check(_lib.lib().moe_policy_create(n_slots, n_layers, n_experts,
                                                EVICT[evict], self.window, C.byref(h)))
        self._h = h
        cap = max(n_slots, 1)
        self._buf = [np.zeros(cap + 256, dtype=np.int32) for _ in range(4)]

    def close(self):
        if self._h:
            _lib.lib().moe_policy_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ids(self, experts):
        a = np.ascontiguousarray(np.asarray(experts, dtype=np.int32).reshape(-1))
        return a

    def prefetch(self, layer: int, experts):
        """Returns (slots, experts) of the fills to issue, and whether the
        call bailed on exhaustion."""
        e = self._ids(experts)
        fs = np.zeros(max(len(e), 1), dtype=np.int32)
        fe = np.zeros(max(len(e), 1), dtype=np.int32)
        bailed = C.c_int32(0)
        n = _lib.check(_lib.lib().moe_policy_prefetch(
            self._h, int(layer), e.ctypes.data, len(e), fs.ctypes.data, fe.ctypes.data,
            C.byref(bailed)))
        return fs[:n].copy(), fe[:n].copy(), bool(bailed.value)

    def acquire(self, layer: int, experts):
        """Returns (slots, miss positions, wait positions)."""
        e = self._ids(experts)
        n = max(len(e), 1)
        slots = np.zeros(n, dtype=np.int32)
        miss = np.zeros(n, dtype=np.int32)
        wait = np.zeros(n, dtype=np.int32)
        nm, nw = C.c_int32(0), C.c_int32(0)
        rc = _lib.lib().moe_policy_acquire(self._h, int(layer), e.ctypes.data, len(e),
                                           slots.ctypes.data, miss.ctypes.data,
                                           C.byref(nm), wait.ctypes.data, C.byref(nw))
        if rc == _lib.MOE_ERR_EXHAUSTED:
            raise PoolExhausted("pool exhausted: every slot pinned or pending")
        _lib.check(rc)
        return slots[:len(e)].copy(), miss[:nm.value].copy(), wait[:nw.value].copy()

    def complete(self, layer: int, expert: int):
        _lib.check(_lib.lib().moe_policy_complete(self._h, int(layer), int(expert)))

    def cancel(self, layer: int, expert: int):
        """Drop a pending prefetch whose fill was never issued: the key is
        unmapped and its slot freed, so a later acquire refills it."""
        _lib.check(_lib.lib().moe_policy_cancel(self._h, int(layer), int(expert)))

    def lookup(self, layer: int, expert: int) -> int:
        """Slot of (layer, expert), or -1 when it is not resident (the C call
        returns -1 for both an absent key and a bad one, so the range is
        checked here)."""
        layer, expert = int(layer), int(expert)
        if not (0 <= layer < self.n_layers and 0 <= expert < self.n_experts):
            raise _lib.MoeError(_lib.MOE_ERR_INVALID,
                                f"key ({layer}, {expert}) outside [0, {self.n_layers}) x "
                                f"[0, {self.n_experts})")
        return int(_lib.lib().moe_policy_lookup(self._h, layer, expert))

    def is_pending(self, layer: int, expert: int) -> bool:
        return bool(_lib.check(_lib.lib().moe_policy_is_pending(self._h, int(layer), int(expert))))

    def table(self) -> np.ndarray:
        t = np.zeros(self.n_layers * self.n_experts, dtype=np.int32)
        _lib.check(_lib.lib().moe_policy_table(self._h, t.ctypes.data))
        return t.reshape(self.n_layers, self.n_experts)

    def stats(self) -> dict:
        o = np.zeros(8, dtype=np.int64)
        _lib.check(_lib.lib().moe_policy_stats(self._h, o.ctypes.data))
        keys = ("total", "prefetch", "cache", "miss", "bail", "issued", "clock", "use_clock")
        return {k: int(v) for k, v in zip(keys, o)}


class SlotOf:
    """Read-only mapping view (layer, expert) -> slot over the native table,
    for callers of the reference's `pool.slot_of`."""

    def __init__(self, pol: NativePolicy):
        self._p = pol

    def get(self, key, default=None):
        s = self._p.lookup(*key)
        return default if s < 0 else s

    def __getitem__(self, key):
        s = self._p.lookup(*key)
        if s < 0:
            raise KeyError(key)
        return s

    def __contains__(self, key):
        return self._p.lookup(*key) >= 0

    def __len__(self):
        return int((self._p.table() >= 0).sum())
