"""Slot-pool bookkeeping: the oracle restatement pinned by hand-derived known
answers on tiny pools, then the native C++ policy checked against the
oracle, call for call, on random traces.  Host only (no device calls)."""
import numpy as np
import pytest

from moe_stream_amd.policy import NativePolicy, PoolExhausted
from oracle.policy import PolicyOracle, prefetch_simulator
from oracle.policy import PoolExhausted as OracleExhausted


# --------------------------------------------------- oracle known answers --
A, B, C, D = 10, 11, 12, 13
def test_free_list_pops_from_the_end():
    # engine_v3.py:218,324-325: free = list(range(n)); free.pop()
    p = PolicyOracle(3)
    assert [p.acquire(0, [e])[0] for e in (5, 6, 7)] == [2, 1, 0]


def _lfu_lru_scene(mode):
    # A, B, C admitted to slots 2, 1, 0; B used 3 more times early, then A
    # and C once each; C's acquire leaves slot 0 pinned.  A miss on D at
    # clock 4 scans slots 1, 0, 2 (start 4 % 3, stride 7919 % 3 = 2).
    p = PolicyOracle(3, evict=mode, window=1)
    for e in (A, B, C):
        p.acquire(0, [e])
    for _ in range(3):
        p.acquire(0, [B])
    p.acquire(0, [A])
    p.acquire(0, [C])
    return p, p.acquire(0, [D])[0]


def test_eviction_lfu_lru_asis_known_answers():
    # LFU: B freq 4 vs A freq 2 -> A (slot 2) goes
    p, s = _lfu_lru_scene("lfu")
    assert s == 2 and (0, A) not in p.slot_of and (0, B) in p.slot_of
    # LRU: B last used at 6 vs A at 7 -> B (slot 1) goes
    p, s = _lfu_lru_scene("lru")
    assert s == 1 and (0, B) not in p.slot_of
    # asis: every score 0, the first candidate seen (slot 1) goes
    p, s = _lfu_lru_scene("asis")
    assert s == 1


def _young_scene(window):
    p = PolicyOracle(3, window=window)
    p.acquire(0, [A])
    p.acquire(0, [A])
    p.acquire(0, [A])           # A: slot 2, born 1, freq 3
    p.prefetch(1, [B])          # B: slot 1, born 2, freq 0
    p.complete((1, B))
    p.acquire(0, [C])           # C: slot 0, pinned
    p.prefetch(1, [D])          # clock 4: scan slots 1, 0, 2
    return p


def test_young_entries_are_protected():
    # window 3: B (age 2) is young, +2^30, so A (freq 3) is the victim
    p = _young_scene(3)
    assert p.slot_of[(1, D)] == 2 and (1, B) in p.slot_of
    # window 1: B is old and has the lowest frequency
    p = _young_scene(1)
    assert p.slot_of[(1, D)] == 1 and (0, A) in p.slot_of


def test_pending_is_not_evictable_and_exhaustion():
    p = PolicyOracle(1)
    p.prefetch(0, [1])                       # the only slot, in flight
    with pytest.raises(OracleExhausted):
        p.acquire(1, [2])
    p2 = PolicyOracle(1)
    p2.prefetch(0, [1])
    p2.prefetch(2, [3])                      # silent bail
    assert p2.stats()["bail"] == 1 and p2.stats()["issued"] == 1


def test_hit_accounting():
    p = PolicyOracle(4)
    p.prefetch(1, [5])
    assert p.acquire(1, [5]) == [3]          # waited on the pending prefetch
    assert p.freq[(1, 5)] == 2               # touched in the loop and after the wait
    p.prefetch(1, [6])
    p.complete((1, 6))
    p.acquire(1, [6])                        # completed prefetch: prefetch hit
    p.acquire(1, [6])                        # now a cache hit
    p.acquire(1, [7])                        # demand miss
    assert p.stats() == dict(total=4, prefetch=2, cache=1, miss=1, bail=0, issued=2)
    assert p.pinned == {p.slot_of[(1, 7)]}


# ------------------------------------------------ native against oracle --
def _run_trace(seed, n_slots, evict, n_layers=6, n_experts=24, steps=400):
    rng = np.random.default_rng(seed)
    o = PolicyOracle(n_slots, evict=evict, window=24)
    n = NativePolicy(n_slots, n_layers, n_experts, evict=evict, window=24)
    pending = []
    for step in range(steps):
        layer = int(rng.integers(n_layers))
        op = rng.random()
        if op < 0.35:
            ex = rng.choice(n_experts, size=int(rng.integers(1, 6)), replace=False)
            before = len(o.fills)
            bailed_before = o.n_prefetch_bail
            o.prefetch(layer, ex)
            fs, fe, bailed = n.prefetch(layer, ex)
            exp = [(k[1], s) for k, s, _ in o.fills[before:]]
            assert list(zip(fe.tolist(), fs.tolist())) == exp, step
            assert bailed == (o.n_prefetch_bail > bailed_before)
            pending += [(layer, int(e)) for e in fe]
        elif op < 0.5 and pending:
            key = pending.pop(int(rng.integers(len(pending))))
            o.complete(key)
            n.complete(*key)
        else:
            ex = rng.choice(n_experts, size=int(rng.integers(1, 5)), replace=False)
            try:
                so = o.acquire(layer, ex)
            except OracleExhausted:
                with pytest.raises(PoolExhausted):
                    n.acquire(layer, ex)
                break
            sn, miss, wait = n.acquire(layer, ex)
            assert sn.tolist() == so, step
        assert n.stats()["total"] == o.stats()["total"]
        for key, slot in o.slot_of.items():
            assert n.lookup(*key) == slot
        assert int((n.table() >= 0).sum()) == len(o.slot_of) <= n_slots
    so, sn = o.stats(), n.stats()
    for k in ("total", "prefetch", "cache", "miss", "bail", "issued"):
        assert so[k] == sn[k], k
    assert sn["clock"] == o.clock and sn["use_clock"] == o.use_clock
    return so


@pytest.mark.parametrize("evict", ["lfu", "lru", "asis"])
@pytest.mark.parametrize("n_slots", [7, 40, 150])
def test_native_policy_matches_oracle(evict, n_slots):
    for seed in range(3):
        _run_trace(1000 * n_slots + seed, n_slots, evict)


def test_native_policy_rejects_bad_keys():
    n = NativePolicy(4, 2, 3)
    with pytest.raises(Exception):
        n.acquire(2, [0])
    with pytest.raises(Exception):
        n.prefetch(0, [3])


# ------------------------------- against the reference's pool simulator --
def _zipf_trace(rng, L, T, E, k, kp, recall):
    """Routed ids [L, T, k] from a Zipf-like popularity, and predictions
    [L, T, kp] that keep each routed id with probability `recall` and fill
    the rest with popular ids (as the lookahead does)."""
    pop = 1.0 / np.arange(1, E + 1) ** 1.1
    pop /= pop.sum()
    true = np.zeros((L, T, k), dtype=np.int64)
    pred = np.zeros((L, T, kp), dtype=np.int64)
    for l in range(L):
        perm = rng.permutation(E)      # each layer its own popular experts
        for t in range(T):
            ids = perm[rng.choice(E, size=k, replace=False, p=pop)]
            true[l, t] = ids
            keep = [int(e) for e in ids if rng.random() < recall]
            rest = [int(e) for e in perm[rng.choice(E, size=2 * kp, replace=False, p=pop)]
                    if int(e) not in keep]
            pred[l, t] = (keep + rest)[:kp]
    return true, pred


@pytest.mark.parametrize("evict", ["lfu", "lru", "asis"])
@pytest.mark.parametrize("cap", [40, 96, 300])
def test_policy_matches_reference_pool_simulator(evict, cap):
    """Driven in the simulator's order (per token and layer: pins cleared,
    acquire of the routed ids, then prefetch of the next layer's predicted
    ids with each fill completed at once), the native policy and the oracle
    admit exactly as many entries and hit exactly as often as the
    reference's second model of the pool (scratchpad/prefetch_sim.py:21-94),
    for every eviction mode and pool sizes from tight to roomy."""
    rng = np.random.default_rng(cap * 7 + len(evict))
    L, T, E, k, kp = 6, 40, 64, 8, 8
    true, pred = _zipf_trace(rng, L, T, E, k, kp, recall=0.8)
    want = prefetch_simulator(true, pred, cap, evict)
    n = NativePolicy(cap, L, E, evict=evict)
    o = PolicyOracle(cap, evict=evict)
    for t in range(T):
        for l in range(L):
            n.acquire(l, [])           # the simulator's pin set starts empty
            o.acquire(l, [])
            n.acquire(l, true[l, t])
            o.acquire(l, true[l, t].tolist())
            if l + 1 < L:
                for e in pred[l + 1, t]:   # one at a time, each read done at once
                    _, fe, bailed = n.prefetch(l + 1, [int(e)])
                    assert not bailed
                    for x in fe:
                        n.complete(l + 1, int(x))
                    o.prefetch(l + 1, [int(e)])
                    if (l + 1, int(e)) in o.pending:
                        o.complete((l + 1, int(e)))
    sn, so = n.stats(), o.stats()
    admitted, hits, accesses = want
    assert sn["total"] == so["total"] == accesses == L * T * k
    assert sn["issued"] + sn["miss"] == so["issued"] + so["miss"] == admitted
    assert sn["prefetch"] + sn["cache"] == so["prefetch"] + so["cache"] == hits
    assert 0 < hits < accesses


def test_cancel_unmaps_a_pending_prefetch():
    """A prefetch whose fill was never issued is cancelled: the key is no
    longer mapped or pending, its slot goes back to the free list (the next
    allocation pops it from the end), and a later acquire of it is a miss
    that refills it instead of a wait on a fill that does not exist."""
    n = NativePolicy(4, 2, 8)
    slots, exps, _ = n.prefetch(1, [5, 6])
    assert list(exps) == [5, 6] and list(slots) == [3, 2]
    n.cancel(1, 6)
    assert not n.is_pending(1, 6) and n.lookup(1, 6) == -1
    assert n.is_pending(1, 5) and n.lookup(1, 5) == 3
    with pytest.raises(Exception):
        n.cancel(1, 6)          # no longer pending
    s, miss, wait = n.acquire(1, [6, 5])
    assert list(miss) == [0] and list(wait) == [1]
    assert s[0] == 2            # the freed slot, popped from the end again
    assert s[1] == 3
    st = n.stats()
    assert st["miss"] == 1 and st["prefetch"] == 1


def test_slot_of_view_absent_keys():
    """pool.slot_of-style lookups of keys that are not resident give the
    default / False / KeyError, not an error from the library."""
    from moe_stream_amd.policy import SlotOf
    n = NativePolicy(4, 2, 8)
    v = SlotOf(n)
    assert v.get((0, 3)) is None and v.get((0, 3), -7) == -7
    assert (0, 3) not in v
    with pytest.raises(KeyError):
        v[(0, 3)]
    n.acquire(0, [3])
    assert (0, 3) in v and v[(0, 3)] == 3 and v.get((0, 3)) == 3
    with pytest.raises(Exception):
        n.lookup(2, 0)          # layer out of range
