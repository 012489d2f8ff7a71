"""The streaming pool end to end: a pinned host store feeding a slot pool
smaller than the model, prefetch driven by the lookahead (engine_v3.py:
493-609).  Outputs must equal the HBM-resident stack's on the same seeds
(residency never changes a result), the host store must hold the same bytes
as the device store, and fills from an on-disk store must give the same
results as fills from HBM."""
import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import store as S
from moe_stream_amd import synth
from moe_stream_amd.block import MoEBlock
from moe_stream_amd.pool import ExpertPool
from moe_stream_amd.stack import DecodeStack, StreamingStack

pytestmark = pytest.mark.gpu

L = 4


@pytest.fixture(scope="module")
def stacks():
    geom = G.QWEN3_30B_A3B
    dec = DecodeStack(geom, L, 512, "cuda", seed=20260601, zipf_s=1.1)
    st = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1)
    xs = synth.hidden_states(6, L, geom.d_model, "cuda", 20260602)
    return geom, dec, st, xs


def test_host_store_equals_device_store(stacks):
    geom, dec, st, _ = stacks
    for r in (0, 1, 200, L * 128 - 1):
        a = dec.store[r].cpu().numpy()
        np.testing.assert_array_equal(st.store.array[r], a)


def test_streaming_equals_resident_stack(stacks):
    geom, dec, st, xs = stacks
    for t in range(xs.shape[0]):
        dec.run_token(xs[t], use_graph=False)
        y = st.token(xs[t])
        torch.cuda.synchronize()
        assert torch.equal(y, dec.y), t
    s = st.pool.stats()
    assert s["total"] == xs.shape[0] * L * 8
    assert s["miss"] + s["prefetch"] + s["cache"] == s["total"]
    assert s["prefetch"] > 0 and s["miss"] > 0        # 40 slots: evictions happen
    assert st.pool.bytes_read == (s["issued"] + s["miss"]) * geom.record_bytes
    assert 0.0 <= st.recall() <= 1.0


@pytest.mark.parametrize("layout", ["records", "components"])
def test_native_engine_equals_resident_stack(stacks, layout):
    """The engine loop in the library (moe_engine_layer): same outputs as the
    HBM-resident stack, the policy's statistics and byte counts consistent,
    with fills by the copy engines (slots holding whole records) or by copy
    kernels (component arrays)."""
    geom, dec, _, xs = stacks
    st = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1, native=True,
                        pool_layout=layout)
    for t in range(xs.shape[0]):
        dec.run_token(xs[t], use_graph=False)
        y = st.token(xs[t])
        torch.cuda.synchronize()
        assert torch.equal(y, dec.y), t
    s = st.pool.stats()
    c = st.engine_counters()
    assert s["total"] == xs.shape[0] * L * 8
    assert s["miss"] + s["prefetch"] + s["cache"] == s["total"]
    assert s["prefetch"] > 0 and s["miss"] > 0
    assert c["bytes_read"] == (s["issued"] + s["miss"]) * geom.record_bytes
    assert c["bytes_exposed"] == s["miss"] * geom.record_bytes
    assert 0 < c["recall_hit"] <= c["recall_total"] == xs.shape[0] * (L - 1) * 8
    st.close()


def test_native_engine_matches_python_loop(stacks):
    """The same token sequence through MoEBlock.streaming_call and through
    the library's engine loop, fresh pools: identical outputs and lookups.
    (Hit/miss splits may differ: when a prefetch retires depends on when its
    fill's event completes.)"""
    geom, _, _, xs = stacks
    py = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1)
    na = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1, native=True)
    for t in range(xs.shape[0]):
        a = py.token(xs[t])
        b = na.token(xs[t])
        torch.cuda.synchronize()
        assert torch.equal(a, b), t
    sp, sn = py.pool.stats(), na.pool.stats()
    assert sp["total"] == sn["total"] == xs.shape[0] * L * 8
    assert sn["miss"] + sn["prefetch"] + sn["cache"] == sn["total"]
    na.close()


@pytest.mark.parametrize("depths", [(1, 2), (2, 1, 3)])
def test_native_engine_depth_list_equals_resident_stack(stacks, depths):
    """A list of prefetch depths (the reference's PF_DEPTH, engine_v3.py:61,
    509-527) through the library's engine loop (moe_engine_layer_depths) and
    through MoEBlock.streaming_call: outputs equal the HBM-resident stack's,
    prefetches are issued, recall counts the first depth only."""
    geom, dec, _, xs = stacks
    na = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1, native=True,
                        depths=depths)
    py = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1, depths=depths)
    one = StreamingStack(geom, L, 40, "cuda", seed=20260601, zipf_s=1.1, native=True)
    for t in range(xs.shape[0]):
        dec.run_token(xs[t], use_graph=False)
        a = na.token(xs[t])
        b = py.token(xs[t])
        one.token(xs[t])
        torch.cuda.synchronize()
        assert torch.equal(a, dec.y), t
        assert torch.equal(b, dec.y), t
    s, s1 = na.pool.stats(), one.pool.stats()
    c = na.engine_counters()
    assert s["total"] == xs.shape[0] * L * 8
    assert s["miss"] + s["prefetch"] + s["cache"] == s["total"]
    assert c["bytes_read"] == (s["issued"] + s["miss"]) * geom.record_bytes
    # the first depth's target layers are the only ones counted for recall
    assert c["recall_total"] == xs.shape[0] * (L - depths[0]) * 8
    assert s["issued"] > 0 and s1["issued"] > 0
    na.close()
    one.close()


@pytest.mark.parametrize("depths", [(1,), (1, 2)])
def test_native_engine_gptoss_equals_resident_stack(depths):
    """The engine loop on the gpt-oss geometry (top-4, projection biases,
    clamped SwiGLU, biased router, top-k then softmax): the decode kernels
    take the slot refs in their kernel arguments there too, and the outputs
    are those of the HBM-resident stack bit for bit, with one prefetch depth
    and with a depth list (the further depth's router carries its bias)."""
    geom, Lg = G.GPT_OSS_120B, 2 if len(depths) == 1 else 3
    dec = DecodeStack(geom, Lg, 256, "cuda", seed=20260611, zipf_s=None, router_bias=True)
    st = StreamingStack(geom, Lg, 16, "cuda", seed=20260611, zipf_s=None, router_bias=True,
                        native=True, depths=depths)
    xs = synth.hidden_states(5, Lg, geom.d_model, "cuda", 20260612)
    for t in range(xs.shape[0]):
        dec.run_token(xs[t], use_graph=False)
        y = st.token(xs[t])
        torch.cuda.synchronize()
        assert torch.equal(y, dec.y), t
    s = st.pool.stats()
    assert s["total"] == xs.shape[0] * Lg * 4
    assert s["miss"] > 0
    st.close()


def test_on_disk_store_feeds_the_pool(tmp_path):
    geom = G.SMALL
    recs = synth.make_store(geom, geom.n_layers * geom.n_experts, "cuda", 20260603)
    S.write_store(str(tmp_path), geom, recs.cpu().numpy())
    f = S.ExpertStoreFile(str(tmp_path), base=G.SMALL)
    host = f.to_host_store()
    W, _ = synth.router_weights(geom, geom.n_layers, "cuda", 20260604)
    xs = synth.hidden_states(3, geom.n_layers, geom.d_model, "cuda", 20260605)
    outs = []
    for src in (host, recs):
        pool = ExpertPool(geom, 16, store=src, n_layers=geom.n_layers)
        blocks = []
        for i in range(geom.n_layers):
            blocks.append(MoEBlock(i, geom, pool, W[i], None, blocks))
        outs.append([blocks[i](xs[t, i:i + 1]) for t in range(3) for i in range(geom.n_layers)])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    host.close()


def test_expert_pool_reference_constructor(tmp_path):
    """ExpertPool(model_dir, n_slots, n_workers), the reference's signature
    (engine_v3.py:128): the store directory is read into pinned memory by the
    workers, acquire fills the pool from it byte for byte, and stats() has
    the reference's keys (engine_v3.py:456-464) with the fill telemetry."""
    from test_pool_host import REFERENCE_STATS_KEYS
    geom = G.SMALL
    recs = synth.make_store(geom, geom.n_layers * geom.n_experts, "cuda", 20260621)
    S.write_store(str(tmp_path), geom, recs.cpu().numpy())
    pool = ExpertPool(str(tmp_path), 12, 3)
    assert pool.n_slots == 12 and pool.n_workers == 3 and pool.n_layers == geom.n_layers
    assert pool.blob == geom.record_bytes and pool.group_size == 64 and pool.bits == 4
    pool.prefetch(1, [4, 5])
    slots = pool.acquire(0, [3, 7, 9])
    slots1 = pool.acquire(1, [4, 5, 6])
    torch.cuda.synchronize()
    for layer, es, ss in ((0, [3, 7, 9], slots), (1, [4, 5, 6], slots1)):
        for e, sl in zip(es, ss):
            got = pool.read_slot(sl)
            for c in geom.components:
                want = recs[layer * geom.n_experts + e, c.offset:c.offset + c.nbytes]
                assert torch.equal(got[c.name].contiguous().view(torch.uint8).reshape(-1),
                                   want.cpu()), (layer, e, c.name)
    s = pool.stats()
    assert set(s) == REFERENCE_STATS_KEYS
    assert s["total"] == 6 and s["miss"] == 4 and s["prefetch"] == 2
    assert s["blocked"] >= 0.0 and s["busy_s"] > 0.0 and s["depth"] >= 1.0
    assert abs(s["gb"] * 2 ** 30 - 6 * geom.record_bytes) < 1
    pool.store.close()
