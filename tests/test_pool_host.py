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


def test_stats_keys_are_the_reference_keys():
    import inspect
    src = inspect.getsource(ExpertPool.stats)
    for k in REFERENCE_STATS_KEYS:
        assert f"{k}=" in src, k
