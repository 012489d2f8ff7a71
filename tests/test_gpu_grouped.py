"""GPU parity of the multi-token path: the MFMA router for T > 16 tokens and
the grouped bf16 MFMA expert block, against the oracle on the same bytes,
against the decode kernels on the same slot refs, and through the
properties the grouping must not change (token order, residency, pair
order inside a group)."""
import numpy as np
import pytest
import torch

from moe_stream_amd import _lib, ops, synth
from moe_stream_amd import geometry as G
from oracle import numerics as N

from helpers import TOL, Layer, bf16_bits, bf16_randn, bf16_values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def qwen_layer():
    layer = Layer(G.QWEN3_30B_A3B, 256, seed=20260041)
    # Zipf(1.1) expert popularity on the router logits, as in the prefill workload
    logpop = synth.zipf_log_popularity(1, 128, 1.1, seed=20260042)
    layer.bias = synth.bf16_bias_from_log(logpop, "cuda")[0].contiguous()
    return layer


def _route_many(layer, x, k_pred=0, W_next=None):
    g = layer.geom
    bufs = ops.route(x, layer.W, layer.bias, g.routing, g.norm_topk_prob, g.top_k,
                     W_next=W_next, k_pred=k_pred, table=layer.table)
    torch.cuda.synchronize()
    return bufs


def _check_ids(layer, x, bufs):
    """Every token's ids equal the oracle's as sets (ties excused); scores
    within one bf16 ulp where the sets agree; refs = table[ids]."""
    g = layer.geom
    X = bf16_values(x)
    Wb = bf16_bits(layer.W)
    bb = None if layer.bias is None else bf16_bits(layer.bias)
    Z = N.router_logits(X, Wb, bb, "mlx")
    ids = bufs.ids.cpu().numpy()
    sc = bufs.scores.cpu().numpy().astype(np.float64)
    refs = bufs.slot_refs.cpu().numpy()
    exact = 0
    for t in range(X.shape[0]):
        if g.routing == 0:
            rid, rsc, ranked = N.top_k_experts(Z[t], g.top_k, g.norm_topk_prob, "mlx")
        else:
            rid, rsc, ranked = N.top_k_route(Z[t], g.top_k, "mlx")
        assert N.ids_match(ranked, rid, ids[t]), (t, sorted(ids[t]), sorted(rid))
        if set(ids[t].tolist()) == set(rid.tolist()):
            exact += 1
            by = dict(zip(rid.tolist(), rsc.tolist()))
            exp = np.array([by[int(e)] for e in ids[t]])
            assert np.all(np.abs(sc[t] - exp) <= N.bf16_ulp(exp) * 1.01), (t, sc[t], exp)
    np.testing.assert_array_equal(refs, layer.perm[ids])
    return ids, sc, exact


def test_route_many_tokens_matches_oracle(qwen_layer):
    T = 100   # not a multiple of the 16-token MFMA tile
    x = bf16_randn((T, 2048), seed=20260043)
    W_next, _ = synth.router_weights(qwen_layer.geom, 1, "cuda", 20260044)
    W_next = W_next[0].contiguous()
    bufs = _route_many(qwen_layer, x, k_pred=16, W_next=W_next)
    ids, sc, exact = _check_ids(qwen_layer, x, bufs)
    assert exact >= 0.9 * T
    # lookahead: top-16 of the raw bf16 logits of the next router
    Zn = N.router_logits(bf16_values(x), bf16_bits(W_next), None, "mlx")
    pred = bufs.pred.cpu().numpy()
    for t in range(T):
        assert N.ids_match(Zn[t], N.top_k_indices(Zn[t], 16), pred[t])
    assert int(bufs.miss.item()) == 0


def test_route_many_tokens_gptoss_matches_oracle():
    """gpt-oss routing on the MFMA router: top-4 of the raw biased logits
    over d_model 2880, 100 tokens (a ragged last 16-token tile), with a
    biased lookahead router ranking the top 8 of the next layer."""
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260054, router_bias=True)
    g = layer.geom
    T = 100
    x = bf16_randn((T, g.d_model), seed=20260055)
    Wn, bn = synth.router_weights(g, 1, "cuda", 20260056, with_bias=True)
    Wn, bn = Wn[0].contiguous(), bn[0].contiguous()
    bufs = ops.route(x, layer.W, layer.bias, g.routing, g.norm_topk_prob, g.top_k,
                     W_next=Wn, bias_next=bn, k_pred=8, table=layer.table)
    torch.cuda.synchronize()
    ids, sc, exact = _check_ids(layer, x, bufs)
    assert exact >= 0.9 * T
    Zn = N.router_logits(bf16_values(x), bf16_bits(Wn), bf16_bits(bn), "mlx")
    pred = bufs.pred.cpu().numpy()
    for t in range(T):
        assert N.ids_match(Zn[t], N.top_k_indices(Zn[t], 8), pred[t]), t
    assert int(bufs.miss.item()) == 0
    del layer
    torch.cuda.empty_cache()


def test_route_many_equals_fused_small_T(qwen_layer):
    """The MFMA router (T > 16) and the fused router (T <= 16) select the
    same experts for the same tokens (their fp32 logits differ only in
    summation order)."""
    g = qwen_layer.geom
    x = bf16_randn((32, 2048), seed=20260045)
    many = _route_many(qwen_layer, x)
    a = many.ids.cpu().numpy()
    Z = N.router_logits(bf16_values(x), bf16_bits(qwen_layer.W),
                        bf16_bits(qwen_layer.bias), "mlx")
    same = 0
    for h in range(2):
        few = _route_many(qwen_layer, x[16 * h:16 * h + 16].contiguous())
        b = few.ids.cpu().numpy()
        for t in range(16):
            if set(a[16 * h + t].tolist()) == set(b[t].tolist()):
                same += 1
            else:   # a near-tie at the k-th rank: both must be valid selections
                _, _, ranked = N.top_k_experts(Z[16 * h + t], g.top_k, True, "mlx")
                assert N.ids_match(ranked, b[t], a[16 * h + t])
    assert same >= 30


def _grouped_vs_oracle(layer, x, label, n_check=None):
    g = layer.geom
    bufs = _route_many(layer, x)
    T = x.shape[0]
    out32 = torch.zeros((T, g.d_model), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, g.d_model), dtype=torch.bfloat16, device="cuda")
    ops.ffn_grouped(layer.pool, bufs.slot_refs, bufs.scores, x, out=out, out_f32=out32)
    torch.cuda.synchronize()
    ops.check_device_error()
    ids = bufs.ids.cpu().numpy()
    sc = bufs.scores.cpu().numpy().astype(np.float64)
    n = T if n_check is None else n_check
    X = bf16_values(x)[:n]
    kind = "qwen3" if not g.has_proj_bias else "gptoss"
    y64 = N.moe_block_batch(X, ids[:n], sc[:n], layer.expert, kind, "f64",
                            g.alpha, g.limit)
    ymlx = N.moe_block_batch(X, ids[:n], sc[:n], layer.expert, kind, "mlx",
                             g.alpha, g.limit)
    o32 = out32.cpu().numpy()
    ob = bf16_values(out)
    e64 = max(N.rel_err(o32[t], y64[t]) for t in range(n))
    emlx = max(N.rel_err(ob[t], ymlx[t]) for t in range(n))
    print(f"{label}: worst-token rel err vs f64 {e64:.2e}, bf16 out vs MLX-emulation "
          f"{emlx:.2e}")
    assert e64 < TOL and emlx < TOL, (label, e64, emlx)
    return bufs, out, out32


def test_grouped_qwen3_matches_oracle(qwen_layer):
    x = bf16_randn((48, 2048), seed=20260046)
    _grouped_vs_oracle(qwen_layer, x, "qwen3 grouped T=48")


@pytest.mark.parametrize("T", [5, 12])
def test_grouped_few_tokens_matches_oracle(qwen_layer, T):
    """A few tokens per call (a verification step): ops.ffn takes the grouped
    MFMA block above 4 tokens, whose tiles then hold one to a few rows."""
    assert T > ops.GROUPED_MIN_TOKENS
    x = bf16_randn((T, 2048), seed=20260060 + T)
    bufs, out, out32 = _grouped_vs_oracle(qwen_layer, x, f"qwen3 grouped T={T}")
    y = ops.ffn(qwen_layer.pool, bufs.slot_refs, bufs.scores, x)
    torch.cuda.synchronize()
    assert torch.equal(y, out)


@pytest.mark.parametrize("T", [17, 33])
def test_grouped_just_past_the_fused_router_matches_oracle(qwen_layer, T):
    """One token past a whole number of 16-token router tiles: the MFMA
    router's last tile holds a single real token (its other rows clamp to it
    and are never stored), and the grouped block sees tiles of one row."""
    x = bf16_randn((T, 2048), seed=20260070 + T)
    bufs, _, _ = _grouped_vs_oracle(qwen_layer, x, f"qwen3 grouped T={T}")
    _check_ids(qwen_layer, x, bufs)


def test_grouped_gptoss_matches_oracle():
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260047, router_bias=True)
    x = bf16_randn((40, 2880), seed=20260048)
    _grouped_vs_oracle(layer, x, "gpt-oss grouped T=40", n_check=12)
    del layer
    torch.cuda.empty_cache()


def test_grouped_gptoss_full_tiles_match_oracle():
    """gpt-oss geometry with 64-row tiles: 160 tokens all routed to experts
    0 and 1 (plus two others each), so those two slots hold 160 rows each
    (tiles of 64, 64 and 32 rows) and every row-block count of both kernels
    runs; the first tokens' rows lie in full tiles."""
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260051, router_bias=True)
    g = layer.geom
    T = 160
    rng = np.random.default_rng(20260052)
    ids = np.zeros((T, g.top_k), dtype=np.int64)
    for t in range(T):
        ids[t] = [0, 1] + list(rng.choice(np.arange(2, g.n_experts), g.top_k - 2, replace=False))
    sc = rng.random((T, g.top_k)).astype(np.float32)
    sc = (sc / sc.sum(axis=1, keepdims=True)).astype(np.float32)
    refs = layer.table[torch.tensor(ids, device="cuda")].to(torch.int32).contiguous()
    scores = torch.tensor(sc, device="cuda")
    x = bf16_randn((T, g.d_model), seed=20260053)
    out32 = torch.zeros((T, g.d_model), dtype=torch.float32, device="cuda")
    ops.ffn_grouped(layer.pool, refs, scores, x, out_f32=out32)
    torch.cuda.synchronize()
    ops.check_device_error()
    n = 12
    y64 = N.moe_block_batch(bf16_values(x)[:n], ids[:n], sc[:n].astype(np.float64),
                            layer.expert, "gptoss", "f64", g.alpha, g.limit)
    o32 = out32.cpu().numpy()
    e64 = max(N.rel_err(o32[t], y64[t]) for t in range(n))
    print(f"gpt-oss grouped, 64-row tiles: worst-token rel err vs f64 {e64:.2e}")
    assert e64 < TOL, e64
    del layer
    torch.cuda.empty_cache()


def test_grouped_full_size_equals_decode(qwen_layer):
    """512 tokens x top-8 with Zipf skew (4096 pairs): the grouped MFMA block
    matches the fp64 oracle on every token, and the decode kernels on the
    same refs.  Both paths round the [pairs, d_ff] intermediate to bf16, so a
    different fp32 summation order can move an intermediate by one bf16 ulp
    (2^-8 relative); the cross-path bar is half of that."""
    g = qwen_layer.geom
    x = bf16_randn((512, 2048), seed=20260049)
    bufs = _route_many(qwen_layer, x)
    ids = bufs.ids.cpu().numpy()
    counts = np.bincount(ids.ravel(), minlength=128)
    assert counts.max() > 64        # the skew gives multi-tile groups
    yg = torch.zeros((512, g.d_model), dtype=torch.float32, device="cuda")
    yd = torch.zeros_like(yg)
    ops.ffn_grouped(qwen_layer.pool, bufs.slot_refs, bufs.scores, x, out_f32=yg)
    for c in range(0, 512, 16):
        ops.ffn_decode(qwen_layer.pool, bufs.slot_refs[c:c + 16].contiguous(),
                       bufs.scores[c:c + 16].contiguous(), x[c:c + 16].contiguous(),
                       out_f32=yd[c:c + 16])
    torch.cuda.synchronize()
    ops.check_device_error()
    a, b = yg.cpu().numpy(), yd.cpu().numpy()
    diffs = np.array([N.rel_err(a[t], b[t]) for t in range(512)])
    sc = bufs.scores.cpu().numpy().astype(np.float64)
    y64 = N.moe_block_batch(bf16_values(x), ids, sc, qwen_layer.expert, "qwen3", "f64")
    e64 = max(N.rel_err(a[t], y64[t]) for t in range(512))
    print(f"512 tokens: grouped vs f64 oracle worst {e64:.2e}; grouped vs decode "
          f"worst {diffs.max():.2e}, median {np.median(diffs):.2e}")
    assert e64 < TOL
    assert diffs.max() < 2e-3


def test_grouped_token_order_residency_and_determinism(qwen_layer):
    """Permuting tokens permutes the output rows bit-exactly; store refs and
    pool refs give bit-identical outputs; repeated calls are bit-identical."""
    g = qwen_layer.geom
    T = 96
    x = bf16_randn((T, 2048), seed=20260050)
    bufs = _route_many(qwen_layer, x)
    y1 = ops.ffn_grouped(qwen_layer.pool, bufs.slot_refs, bufs.scores, x)
    y2 = ops.ffn_grouped(qwen_layer.pool, bufs.slot_refs, bufs.scores, x)
    p = torch.tensor(np.random.default_rng(3).permutation(T), device="cuda")
    yp = ops.ffn_grouped(qwen_layer.pool, bufs.slot_refs[p].contiguous(),
                         bufs.scores[p].contiguous(), x[p].contiguous())
    store_refs = (-(bufs.ids.long() + 1)).to(torch.int32)
    mixed = torch.where(torch.arange(T, device="cuda")[:, None] % 2 == 0,
                        bufs.slot_refs, store_refs).contiguous()
    ym = ops.ffn_grouped(qwen_layer.pool, mixed, bufs.scores, x)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(yp, y1[p])
    assert torch.equal(ym, y1)


def test_grouped_repeated_calls_with_mixed_tile_keys_bit_identical(qwen_layer):
    """A key with one full 64-row tile and a small remainder tile: the
    grouping scatters its pairs over the two tiles in a different order every
    call (its scatter cursors are atomics), and the outputs stay
    bit-identical: a row's result does not depend on the tile it lands in."""
    g = qwen_layer.geom
    T = 76
    rng = np.random.default_rng(20260053)
    ids = np.stack([np.concatenate([[7], rng.permutation(np.arange(8, 128))[:g.top_k - 1]])
                    for _ in range(T)])   # expert 7 in every token: 76 pairs = 64 + 12
    refs = torch.tensor(qwen_layer.perm[ids], dtype=torch.int32, device="cuda")
    sc = torch.tensor(rng.dirichlet(np.ones(g.top_k), T).astype(np.float32), device="cuda")
    x = bf16_randn((T, 2048), seed=20260054)
    ys = [ops.ffn_grouped(qwen_layer.pool, refs, sc, x) for _ in range(4)]
    torch.cuda.synchronize()
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


@pytest.mark.parametrize("T,k,rows_per_expert", [(1, 4, None), (17, 4, None),
                                                 (64, 1, 64), (65, 1, 65), (130, 2, None)])
def test_grouped_ragged_tiles_small_geometry(T, k, rows_per_expert):
    """Tile edges: a single pair, one expert with exactly 64 / 65 rows, groups
    spanning several tiles; small geometry (d_model 256, d_ff 128)."""
    layer = Layer(G.SMALL, 24, seed=20260051)
    E = layer.geom.n_experts
    rng = np.random.default_rng(T * 10 + k)
    if rows_per_expert is not None:
        ids = np.full((T, k), 5)
    else:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    sc = rng.dirichlet(np.ones(k), T).astype(np.float32)
    x = bf16_randn((T, 256), seed=20260052 + T)
    refs = torch.tensor(layer.perm[ids], dtype=torch.int32, device="cuda")
    s = torch.tensor(sc, device="cuda")
    y = torch.zeros((T, 256), dtype=torch.float32, device="cuda")
    ops.ffn_grouped(layer.pool, refs, s, x, out_f32=y)
    torch.cuda.synchronize()
    ops.check_device_error()
    y64 = N.moe_block_batch(bf16_values(x), ids, sc.astype(np.float64), layer.expert,
                            "qwen3", "f64")
    err = max(N.rel_err(y.cpu().numpy()[t], y64[t]) for t in range(T))
    assert err < TOL, err


def test_grouped_out_of_range_ref_reported_not_faulting(qwen_layer):
    """A ref outside the pool and store is skipped (its pair contributes
    zero) and reported as MOE_ERR_DEVICE; the other tokens are unaffected."""
    T = 20
    x = bf16_randn((T, 2048), seed=20260053)
    bufs = _route_many(qwen_layer, x)
    good = ops.ffn_grouped(qwen_layer.pool, bufs.slot_refs, bufs.scores, x)
    torch.cuda.synchronize()
    bad_refs = bufs.slot_refs.clone()
    bad_refs[3, 2] = 1 << 20
    bad = ops.ffn_grouped(qwen_layer.pool, bad_refs, bufs.scores, x)
    torch.cuda.synchronize()
    with pytest.raises(_lib.MoeError) as ei:
        ops.check_device_error()
    assert ei.value.code == _lib.MOE_ERR_DEVICE
    keep = torch.arange(T, device="cuda") != 3
    assert torch.equal(bad[keep], good[keep])


@pytest.mark.parametrize("T,block,expect", [(4, "auto", "decode"), (8, "auto", "grouped"),
                                            (64, "grouped", "grouped")])
def test_multi_token_stack_graph_replays_equal_eager(T, block, expect):
    """The multi-token stack (router + expert block per layer, 4 layers)
    captured once as a HIP graph and replayed for several steps, with eager
    work of the same stack between the replays: every replay routes and
    computes exactly what the eager launches do.  `auto` picks the block
    ops.ffn picks for T tokens."""
    from moe_stream_amd.stack import PrefillStack
    st = PrefillStack(G.QWEN3_30B_A3B, 4, 256, T, "cuda", block=block,
                      seed=20260070 + T, zipf_s=1.1)
    assert st.block == expect
    xs = synth.hidden_states(3 * T, st.L, 2048, "cuda", 20260071 + T).view(3, T, st.L, 2048)
    st.x_in.copy_(xs[0].transpose(0, 1))
    st.capture()
    for i in range(3):
        x_step = xs[i].transpose(0, 1).contiguous()
        st.run_step(x_step, use_graph=False)
        torch.cuda.synchronize()
        ids = torch.stack([b.ids for b in st.bufs]).clone()
        y_ref = st.y.clone()
        st.run_step(x_step, use_graph=True)
        torch.cuda.synchronize()
        ops.check_device_error()
        assert torch.equal(torch.stack([b.ids for b in st.bufs]), ids), i
        assert torch.equal(st.y, y_ref), i
    Lx = 1                       # ops.ffn runs the same block at this T
    y = ops.ffn(st.pool, st.bufs[Lx].slot_refs, st.bufs[Lx].scores, st.x_in[Lx])
    torch.cuda.synchronize()
    assert torch.equal(y, st.y[Lx])
    del st
    torch.cuda.empty_cache()
