"""Host-side parts of ExpertPool that need no device: the reference's stats()
key set and the busy-time union of fill spans."""
import types

from moe_stream_amd.pool import ExpertPool

# engine_v3.py:456-464
REFERENCE_STATS_KEYS = {"total", "prefetch", "cache", "miss", "blocked", "gb", "busy_s",
                        "depth", "bail", "issued", "exposed_gb"}


def _spans(spans):
    return types.SimpleNamespace(_spans=list(spans), _busy_done_ms=0.0)


def test_busy_time_is_the_union_of_fill_spans():
    # overlapping, nested, touching and disjoint spans (ms)
    o = _spans([(5.0, 7.0), (0.0, 2.0), (1.0, 3.0), (1.5, 2.5), (3.0, 4.0), (10.0, 11.0)])
    ExpertPool._merge_spans(o, keep_last=False)
    assert o._spans == [] and abs(o._busy_done_ms - (4.0 + 2.0 + 1.0)) < 1e-12
    # keep_last leaves the latest merged interval open for later overlaps
    o = _spans([(0.0, 2.0), (1.0, 3.0), (5.0, 7.0)])
    ExpertPool._merge_spans(o, keep_last=True)
    assert o._spans == [(5.0, 7.0)] and abs(o._busy_done_ms - 3.0) < 1e-12
    o._spans.append((6.0, 9.0))
    ExpertPool._merge_spans(o, keep_last=True)
    assert o._spans == [(5.0, 9.0)] and abs(o._busy_done_ms - 3.0) < 1e-12


def test_stats_keys_and_values():
    """stats() of a pool with no device state behind it (the native policy
    is host-only; fills are stood in by their telemetry): the reference's
    eleven keys, the policy's counters, and busy_s as a float attribute."""
    from moe_stream_amd.policy import NativePolicy
    p = object.__new__(ExpertPool)
    p.policy = NativePolicy(8, 2, 4)
    p.policy.acquire(0, [1, 2])              # 2 misses
    p.policy.acquire(0, [1])                 # 1 cache hit
    slots, exps, _ = p.policy.prefetch(1, [3])
    p.policy.complete(1, 3)
    p.policy.acquire(1, [3])                 # 1 prefetch hit
    p.t_blocked, p.bytes_read, p.bytes_exposed = 0.25, 3 * 2 ** 30, 2 ** 29
    p.depth_sum, p.depth_n = 6, 4
    p._fills, p._spans, p._busy_done_ms = [], [(0.0, 2.0), (1.0, 4.0)], 1000.0
    s = p.stats()
    assert set(s) == REFERENCE_STATS_KEYS
    assert (s["total"], s["prefetch"], s["cache"], s["miss"]) == (4, 1, 1, 2)
    assert (s["issued"], s["bail"]) == (1, 0)
    assert s["blocked"] == 0.25 and s["gb"] == 3.0 and s["exposed_gb"] == 0.5
    assert s["depth"] == 1.5
    assert abs(s["busy_s"] - 1.004) < 1e-12            # 1000 ms + the union [0, 4] ms
    assert isinstance(p.busy_s, float) and abs(p.busy_s - 1.004) < 1e-12


def test_record_layout_views_address_whole_records():
    """The record layout on host memory: slot s holds a store record at
    s * record_bytes, every component view reads its bytes at the record's
    component offset, and the C view carries one base with slot stride =
    record size (the form moe_fill_slots copies with one call per record)."""
    import numpy as np
    import torch
    from moe_stream_amd import geometry as G
    from moe_stream_amd.pool import SlotPool
    for geom in (G.SMALL, G.GPT_OSS_120B):
        n = 3
        pool = SlotPool(geom, n, "cpu", layout="records")
        rb = geom.record_bytes
        rng = np.random.default_rng(5)
        recs = rng.integers(0, 256, (n, rb), dtype=np.uint8)
        pool._buf.copy_(torch.from_numpy(recs.reshape(-1)))
        v = pool.c_view()
        base = pool._buf.data_ptr()
        for i, c in enumerate(geom.components):
            got = pool.views[c.name]
            assert tuple(got.shape) == (n, *c.shape)
            for s in range(n):
                b = got[s].contiguous().view(torch.uint8).numpy().reshape(-1)
                np.testing.assert_array_equal(b, recs[s, c.offset:c.offset + c.nbytes])
            assert v.base[i] == base + c.offset and v.slot_bytes[i] == rb
            assert v.comp_offset[i] == c.offset
    try:
        SlotPool(G.SMALL, 2, "cpu", layout="rows")
    except ValueError:
        pass
    else:
        raise AssertionError("unknown layout accepted")
