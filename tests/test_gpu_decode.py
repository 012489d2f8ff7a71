"""GPU parity of the batch-1 expert block and the router against the oracle.

Inputs are the seeded synthetic workloads; the oracle runs on the same bytes
copied back from the device.  Bars: routed ids equal as sets (ties at the
k-th rank excused), FFN outputs within 2e-2 max relative error of both the
fp64 oracle and the MLX-emulation oracle."""
import numpy as np
import pytest
import torch

from moe_stream_amd import _lib, ops
from moe_stream_amd import geometry as G
from oracle import numerics as N

from helpers import TOL, Layer, bf16_randn, bf16_values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen_layer():
    # config 1: 128 experts in a 256-slot pool at a seeded permutation
    return Layer(G.QWEN3_30B_A3B, 256, seed=20260001)


def _check_route_and_block(layer, x, label):
    g = layer.geom
    bufs = ops.route(x, layer.W, layer.bias, g.routing, g.norm_topk_prob, g.top_k,
                     table=layer.table)
    out32 = torch.zeros((1, g.d_model), dtype=torch.float32, device="cuda")
    out = torch.zeros((1, g.d_model), dtype=torch.bfloat16, device="cuda")
    ops.ffn_decode(layer.pool, bufs.slot_refs, bufs.scores, x, out=out, out_f32=out32)
    torch.cuda.synchronize()
    ops.check_device_error()
    ids = bufs.ids[0].cpu().numpy()
    sc = bufs.scores[0].cpu().numpy().astype(np.float64)
    refs = bufs.slot_refs[0].cpu().numpy()
    x64 = bf16_values(x[0])
    ref_ids, ref_sc, ranked = layer.route_oracle(x64, "mlx")
    assert N.ids_match(ranked, ref_ids, ids), (label, sorted(ids), sorted(ref_ids))
    assert len(set(ids.tolist())) == g.top_k
    np.testing.assert_array_equal(refs, layer.perm[ids])
    if set(ids.tolist()) == set(ref_ids.tolist()):
        # scores are bf16 values; allow one bf16 ulp of rounding-order difference
        ref_by_id = dict(zip(ref_ids.tolist(), ref_sc.tolist()))
        exp = np.array([ref_by_id[int(e)] for e in ids])
        assert np.all(np.abs(sc - exp) <= N.bf16_ulp(exp) * 1.01), (label, sc, exp)
    if g.routing == _lib.MOE_ROUTE_SOFTMAX_TOPK and g.norm_topk_prob:
        assert abs(sc.sum() - 1.0) < 2e-2
    y64 = layer.block_oracle(x64, ids, sc, "f64")
    ymlx = layer.block_oracle(x64, ids, sc, "mlx")
    e64 = N.rel_err(out32.cpu().numpy()[0], y64)
    emlx = N.rel_err(bf16_values(out[0]), ymlx)
    print(f"{label}: rel err vs f64 {e64:.2e}, bf16 out vs MLX-emulation {emlx:.2e}")
    assert e64 < TOL and emlx < TOL, (label, e64, emlx)
    return e64, emlx


def test_qwen3_layer_config1(qwen_layer):
    x = bf16_randn((1, 2048), seed=20260011)
    _check_route_and_block(qwen_layer, x, "qwen3 cfg1")


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_qwen3_layer_more_tokens(qwen_layer, seed):
    x = bf16_randn((1, 2048), seed=20260100 + seed)
    _check_route_and_block(qwen_layer, x, f"qwen3 seed {seed}")


def test_gptoss_layer():
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260003, router_bias=True)
    for s in range(2):
        x = bf16_randn((1, 2880), seed=20260300 + s)
        _check_route_and_block(layer, x, f"gpt-oss seed {s}")
    del layer
    torch.cuda.empty_cache()


def test_store_refs_equal_pool_refs(qwen_layer):
    """Reading an expert from the store (ref < 0) or from its pool slot gives
    bit-identical outputs: the result does not depend on residency."""
    x = bf16_randn((1, 2048), seed=20260021)
    ids = torch.tensor([[3, 17, 40, 77, 90, 101, 5, 127]], dtype=torch.int32)
    sc = torch.tensor([[.3, .2, .1, .1, .1, .1, .05, .05]], dtype=torch.float32).cuda()
    pool_refs = torch.tensor(qwen_layer.perm[ids.numpy()], dtype=torch.int32).cuda()
    store_refs = (-(ids.long() + 1)).to(torch.int32).cuda()
    a = ops.ffn_decode(qwen_layer.pool, pool_refs, sc, x)
    b = ops.ffn_decode(qwen_layer.pool, store_refs, sc, x)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_permutation_invariance_and_determinism(qwen_layer):
    """Output unchanged (bit-exact in fp32 up to summation order of the
    combine) when the (slot, score) pairs are permuted; bit-identical across
    runs."""
    x = bf16_randn((1, 2048), seed=20260022)
    ids = np.array([9, 2, 66, 31, 120, 45, 88, 12])
    sc = np.array([.25, .2, .15, .1, .1, .1, .05, .05], dtype=np.float32)
    refs = torch.tensor(qwen_layer.perm[ids][None], dtype=torch.int32).cuda()
    s = torch.tensor(sc[None]).cuda()
    o1 = torch.zeros((1, 2048), dtype=torch.float32, device="cuda")
    o2 = torch.zeros_like(o1)
    o3 = torch.zeros_like(o1)
    ops.ffn_decode(qwen_layer.pool, refs, s, x, out_f32=o1)
    ops.ffn_decode(qwen_layer.pool, refs, s, x, out_f32=o2)
    p = np.random.default_rng(0).permutation(8)
    ops.ffn_decode(qwen_layer.pool, refs[:, p].contiguous(), s[:, p].contiguous(), x,
                   out_f32=o3)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert N.rel_err(o3.cpu().numpy(), o1.cpu().numpy()) < 1e-5


def test_small_T_matches_per_token(qwen_layer):
    """T tokens in one call equal T single-token calls."""
    T, k = 4, 8
    x = bf16_randn((T, 2048), seed=20260023)
    rng = np.random.default_rng(1)
    ids = np.stack([rng.permutation(128)[:k] for _ in range(T)])
    refs = torch.tensor(qwen_layer.perm[ids], dtype=torch.int32).cuda()
    sc = torch.tensor(rng.dirichlet(np.ones(k), T), dtype=torch.float32).cuda()
    yT = ops.ffn_decode(qwen_layer.pool, refs, sc, x)
    y1 = torch.cat([ops.ffn_decode(qwen_layer.pool, refs[t:t + 1].contiguous(),
                                   sc[t:t + 1].contiguous(), x[t:t + 1].contiguous())
                    for t in range(T)])
    torch.cuda.synchronize()
    assert torch.equal(yT, y1)


def test_out_of_range_ref_is_reported_not_faulting(qwen_layer):
    """A slot ref past the pool (or a store record past the store) is skipped
    by the kernels and reported as MOE_ERR_DEVICE."""
    x = bf16_randn((1, 2048), seed=20260024)
    refs = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 100000]], dtype=torch.int32).cuda()
    sc = torch.full((1, 8), 0.125, dtype=torch.float32).cuda()
    ops.ffn_decode(qwen_layer.pool, refs, sc, x)
    with pytest.raises(_lib.MoeError) as ei:
        ops.check_device_error()
    assert ei.value.code == _lib.MOE_ERR_DEVICE
    ops.check_device_error()   # cleared


@pytest.mark.parametrize("T", [1, 3])
def test_split_halves_equal_one_call(qwen_layer, T):
    """moe_ffn_decode_up then moe_ffn_decode_down, each its own call (the
    second on another stream that waits for the first), give the bytes of
    moe_ffn_decode; T=3 takes the kernels that group pairs per expert."""
    g = qwen_layer.geom
    x = bf16_randn((T, 2048), seed=20260030 + T)
    bufs = ops.route(x, qwen_layer.W, None, g.routing, g.norm_topk_prob, g.top_k,
                     table=qwen_layer.table)
    ref32 = torch.zeros((T, 2048), dtype=torch.float32, device="cuda")
    ref = torch.zeros((T, 2048), dtype=torch.bfloat16, device="cuda")
    ops.ffn_decode(qwen_layer.pool, bufs.slot_refs, bufs.scores, x, out=ref, out_f32=ref32)
    ws = ops.ffn_decode_up(qwen_layer.pool, bufs.slot_refs, x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    out32 = torch.zeros((T, 2048), dtype=torch.float32, device="cuda")
    with torch.cuda.stream(side):
        out = ops.ffn_decode_down(qwen_layer.pool, bufs.slot_refs, bufs.scores, ws,
                                  out_f32=out32, stream=side)
    torch.cuda.synchronize()
    ops.check_device_error()
    assert out is out32
    assert torch.equal(out32, ref32)
    out_b = ops.ffn_decode_down(qwen_layer.pool, bufs.slot_refs, bufs.scores, ws)
    torch.cuda.synchronize()
    assert torch.equal(out_b, ref)
    with pytest.raises(_lib.MoeError):   # a workspace too small for T x k
        ops.ffn_decode_down(qwen_layer.pool, bufs.slot_refs, bufs.scores, ws[:256])


def test_split_halves_gptoss():
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260033, router_bias=True)
    g = layer.geom
    x = bf16_randn((1, g.d_model), seed=20260034)
    bufs = ops.route(x, layer.W, layer.bias, g.routing, g.norm_topk_prob, g.top_k,
                     table=layer.table)
    ref = ops.ffn_decode(layer.pool, bufs.slot_refs, bufs.scores, x)
    ws = ops.ffn_decode_up(layer.pool, bufs.slot_refs, x)
    out = ops.ffn_decode_down(layer.pool, bufs.slot_refs, bufs.scores, ws)
    torch.cuda.synchronize()
    ops.check_device_error()
    assert torch.equal(out, ref)
    del layer
    torch.cuda.empty_cache()


def test_slot_lookup(qwen_layer):
    """slot_refs = table[ids] for ids of any count (several 256-thread
    blocks and a ragged last one); refs < 0 (experts not resident) are
    counted into miss; an id outside [0, E) is reported, not read."""
    rng = np.random.default_rng(20260035)
    table = qwen_layer.perm.astype(np.int32).copy()
    table[rng.choice(128, 10, replace=False)] = -1
    t_dev = torch.tensor(table, device="cuda")
    for n in (1, 300, 4096 + 7):
        ids = rng.integers(0, 128, n).astype(np.int32)
        miss = torch.zeros(1, dtype=torch.int32, device="cuda")
        refs = ops.slot_lookup(t_dev, torch.tensor(ids, device="cuda"), miss)
        torch.cuda.synchronize()
        ops.check_device_error()
        np.testing.assert_array_equal(refs.cpu().numpy(), table[ids])
        assert int(miss.item()) == int((table[ids] < 0).sum())
    ids = torch.tensor([3, 128, 5], dtype=torch.int32, device="cuda")
    refs = ops.slot_lookup(t_dev, ids)
    torch.cuda.synchronize()
    with pytest.raises(_lib.MoeError) as ei:
        ops.check_device_error()
    assert ei.value.code == _lib.MOE_ERR_DEVICE
    ops.check_device_error()   # cleared
    assert refs.cpu().tolist() == [table[3], 0, table[5]]


def test_events_order_streams_and_time(qwen_layer):
    """The event entry points as a caller orders slot reuse across streams
    (needs_barrier, engine_v3.py:228-231): the block runs on a side stream
    between two recorded events; the current stream waits on the second and
    then reads the output, which equals the same block run in order; the
    event reports done and a non-negative elapsed time."""
    import ctypes as C
    L = _lib.lib()
    g = qwen_layer.geom
    x = bf16_randn((1, 2048), seed=20260036)
    bufs = ops.route(x, qwen_layer.W, None, g.routing, g.norm_topk_prob, g.top_k,
                     table=qwen_layer.table)
    ref = ops.ffn_decode(qwen_layer.pool, bufs.slot_refs, bufs.scores, x)
    out = torch.zeros((1, 2048), dtype=torch.bfloat16, device="cuda")
    ev0, ev1 = C.c_void_p(), C.c_void_p()
    _lib.check(L.moe_event_create(C.byref(ev0)))
    _lib.check(L.moe_event_create(C.byref(ev1)))
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        _lib.check(L.moe_event_record(ev0, side.cuda_stream))
        ops.ffn_decode(qwen_layer.pool, bufs.slot_refs, bufs.scores, x, out=out, stream=side)
        _lib.check(L.moe_event_record(ev1, side.cuda_stream))
        _lib.check(L.moe_stream_wait_event(torch.cuda.current_stream().cuda_stream, ev1))
        copy = out.clone()   # on the current stream, ordered after the block
        torch.cuda.synchronize()
        ops.check_device_error()
        assert L.moe_event_query(ev1) == 1
        ms = C.c_float(-1.0)
        _lib.check(L.moe_event_elapsed_ms(ev0, ev1, C.byref(ms)))
        assert 0.0 <= ms.value < 1000.0, ms.value
        assert torch.equal(copy, ref)
        with pytest.raises(_lib.MoeError):
            _lib.check(L.moe_event_record(None, side.cuda_stream))
    finally:
        _lib.check(L.moe_event_destroy(ev0))
        _lib.check(L.moe_event_destroy(ev1))
