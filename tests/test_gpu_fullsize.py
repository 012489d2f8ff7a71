"""The benchmark configurations at their real size.

* 48-layer Qwen3-30B-A3B-shaped decode stack, 3072 slots over the 6144
  (layer, expert) pairs, Zipf(1.1) router bias: the whole-token kernel
  (cooperative and ordinary launches) equals the per-layer launches bit for
  bit over 8 consecutive tokens (epochs 1..8 and beyond), all 48 layers;
  ids and outputs of layers 0, 23 and 47 against the oracle on two tokens.
* 36-layer gpt-oss-120b-shaped stack, 2304 slots over 4608 pairs, biased
  router: the per-layer graph replayed over 4 tokens equals the eager
  launches; layers 0 and 35 against the oracle; the whole-token kernel
  (cooperative and ordinary launches) equals the per-layer launches bit for
  bit over 4 tokens, all 36 layers.
* The 48-layer prefill stack (512 tokens per layer, grouped MFMA block,
  3072-slot pool, Zipf(1.1)): the captured graph replays exactly what the
  eager launches compute; routing and outputs of layers 0, 23 and 47 against
  the oracle on a sample of 64 tokens each.
* The streaming pool on the 48-layer stack: a 2048-slot pool fed from a
  pinned host store of all 6144 records by the native engine loop, 16 tokens,
  bit-exact against the HBM-resident stack, with consistent pool and engine
  counters.

Reference: engine_v3.py:493-609 (the per-layer loop), engine_120b.py:78-149.
"""
import gc

import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import ops, synth
from moe_stream_amd.stack import DecodeStack, PrefillStack, StreamingStack
from oracle import layout as OL
from oracle import numerics as N

from helpers import TOL, bf16_bits, bf16_values

pytestmark = pytest.mark.gpu


def _free():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _layer_oracle(stack, x_tok, l, ids, scores, y):
    """Routing of layer l (ids as a set, ties excused) and its output against
    the fp64 and MLX-emulation oracles, from the store bytes."""
    g = stack.geom
    Wb = bf16_bits(stack.W[l])
    bb = None if stack.bias is None else bf16_bits(stack.bias[l])
    x64 = bf16_values(x_tok[l])
    z = N.router_logits(x64, Wb, bb, "mlx")
    if g.routing == 0:
        ref_ids, _, ranked = N.top_k_experts(z, g.top_k, g.norm_topk_prob, "mlx")
    else:
        ref_ids, _, ranked = N.top_k_route(z, g.top_k, "mlx")
    assert N.ids_match(ranked, ref_ids, ids), (l, sorted(ids), sorted(ref_ids))
    kind = "gptoss" if g.has_proj_bias else "qwen3"
    exps = [OL.split_record(stack.store[l * stack.E + int(e)].cpu().numpy(), g.d_model,
                            g.d_ff, g.has_proj_bias) for e in ids]
    sc = np.asarray(scores, dtype=np.float64)
    yv = bf16_values(y)
    for mode in ("f64", "mlx"):
        ref = N.moe_block(x64, exps, sc, kind=kind, mode=mode, alpha=g.alpha, limit=g.limit)
        err = N.rel_err(yv, ref)
        print(f"layer {l}: rel err vs {mode} oracle {err:.2e}", flush=True)
        assert err < TOL, (l, mode, err)


@pytest.fixture(scope="module")
def qwen3_stack():
    """The headline decode workload: 48 layers, 3072 slots, Zipf(1.1)."""
    print("building the 48-layer Qwen3 stack (16.3 GB store, 8.2 GB pool)", flush=True)
    st = DecodeStack(G.QWEN3_30B_A3B, 48, 3072, "cuda", zipf_s=1.1)
    yield st
    del st
    _free()


def test_qwen3_48l_persistent_equals_per_layer(qwen3_stack):
    st = qwen3_stack
    xs = synth.hidden_states(8, st.L, st.geom.d_model, "cuda", synth.SEED_BASE + 200)
    st.reset_persistent()
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        for ordinary in (False, True):
            st.token_persistent(xs[t], ordinary=ordinary)
            st.check_persistent()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
            np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
            np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
            np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
            assert torch.equal(st.p_y, y_ref), (t, ordinary)
        print(f"token {t}: persistent == per-layer over 48 layers (epoch {st.p_epoch})",
              flush=True)
    assert st.p_epoch == 2 * xs.shape[0]
    assert int(st.p_miss.sum()) > 0          # some routed experts read from the store


def test_qwen3_48l_layers_against_oracle(qwen3_stack):
    st = qwen3_stack
    xs = synth.hidden_states(2, st.L, st.geom.d_model, "cuda", synth.SEED_BASE + 201)
    for t in range(2):
        st.token_persistent(xs[t])
        st.check_persistent()
        ids = st.p_ids.cpu().numpy()
        sc = st.p_scores.cpu().numpy()
        for l in (0, 23, 47):
            _layer_oracle(st, xs[t], l, ids[l], sc[l], st.p_y[l])


def test_qwen3_48l_streaming_native_equals_resident(qwen3_stack):
    """A 2048-slot pool over a pinned host store of all 6144 records, the
    engine loop in the library, 16 tokens: every layer output equals the
    HBM-resident stack's; the policy and engine counters agree."""
    dec = qwen3_stack
    g = dec.geom
    print("building the pinned host store (6144 records, 16.3 GB)", flush=True)
    st = StreamingStack(g, 48, 2048, "cuda", zipf_s=1.1, native=True)
    try:
        for r in (0, 3071, 6143):
            np.testing.assert_array_equal(st.store.array[r], dec.store[r].cpu().numpy())
        n_tok = 16
        xs = synth.hidden_states(n_tok, 48, g.d_model, "cuda", synth.SEED_BASE + 400)
        for t in range(n_tok):
            dec.run_token(xs[t], use_graph=False)
            y = st.token(xs[t])
            torch.cuda.synchronize()
            assert torch.equal(y, dec.y), t
        ops.check_device_error()
        s = st.pool.stats()
        c = st.engine_counters()
        print(f"streaming: {s}, engine {c}", flush=True)
        assert s["total"] == n_tok * 48 * 8
        assert s["miss"] + s["prefetch"] + s["cache"] == s["total"]
        assert s["prefetch"] > 0 and s["cache"] > 0
        assert c["bytes_read"] == (s["issued"] + s["miss"]) * g.record_bytes
        assert c["bytes_exposed"] == s["miss"] * g.record_bytes
        assert 0 < c["recall_hit"] <= c["recall_total"] == n_tok * 47 * 8
    finally:
        st.close()
        st.store.close()
        del st
        _free()


@pytest.fixture(scope="module")
def gptoss_stack():
    """The gpt-oss decode workload: 36 layers, 2304 slots, biased router."""
    print("building the 36-layer gpt-oss stack (64.6 GB store, 32.3 GB pool)", flush=True)
    st = DecodeStack(G.GPT_OSS_120B, 36, 2304, "cuda", zipf_s=None, router_bias=True)
    yield st
    del st
    _free()


def test_gptoss_36l_graph_equals_eager_and_oracle(gptoss_stack):
    st = gptoss_stack
    g = st.geom
    xs = synth.hidden_states(4, st.L, g.d_model, "cuda", synth.SEED_BASE + 300)
    st.capture()
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        torch.cuda.synchronize()
        ref = st.routed(), st.y.clone()
        st.run_token(xs[t], use_graph=True)
        torch.cuda.synchronize()
        ops.check_device_error()
        for a, b in zip(st.routed(), ref[0]):
            np.testing.assert_array_equal(a, b)
        assert torch.equal(st.y, ref[1]), t
        print(f"token {t}: graph replay == eager over 36 layers", flush=True)
    ids, sc, refs, _ = st.routed()
    assert (refs < 0).any() and (refs >= 0).any()    # pool and store both read
    for l in (0, 35):
        _layer_oracle(st, xs[-1], l, ids[l], sc[l], st.y[l])


def test_gptoss_36l_persistent_equals_per_layer(gptoss_stack):
    """The gpt-oss whole-token kernel (stack_wide_kernel) at full size: every
    layer's ids, scores, refs, lookahead and output equal the per-layer
    launches bit for bit, with cooperative and ordinary launches."""
    st = gptoss_stack
    assert st.persistent_supported()
    xs = synth.hidden_states(4, st.L, st.geom.d_model, "cuda", synth.SEED_BASE + 301)
    st.reset_persistent()
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        for ordinary in (False, True):
            st.token_persistent(xs[t], ordinary=ordinary)
            st.check_persistent()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
            np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
            np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
            np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
            assert torch.equal(st.p_y, y_ref), (t, ordinary)
        print(f"token {t}: gpt-oss persistent == per-layer over 36 layers "
              f"(epoch {st.p_epoch})", flush=True)
    assert st.p_epoch == 2 * xs.shape[0]


def test_qwen3_prefill_48l_graph_and_oracle():
    """The prefill workload at full size: 48 layers x 512 tokens, top-8 with
    Zipf(1.1) skew, 3072-slot pool.  The captured graph (router + grouped
    block per layer) replays the eager launches exactly; at layers 0, 23
    and 47 the routing of 64 sampled tokens matches the oracle (ids as sets,
    ties excused) and their outputs are within the FFN tolerance of the
    fp64 and MLX-emulation oracles."""
    print("building the 48-layer prefill stack (512 tokens per layer)", flush=True)
    T = 512
    st = PrefillStack(G.QWEN3_30B_A3B, 48, 3072, T, "cuda", zipf_s=1.1)
    try:
        g = st.geom
        xs = synth.hidden_states(T, st.L, g.d_model, "cuda", synth.SEED_BASE + 310)
        x_step = xs.transpose(0, 1).contiguous()             # [L, T, D]
        st.run_step(x_step, use_graph=False)
        torch.cuda.synchronize()
        ops.check_device_error()
        ids_e = torch.stack([b.ids for b in st.bufs]).clone()
        y_e = st.y.clone()
        st.capture()
        for rep in range(2):
            st.run_step(x_step, use_graph=True)
            torch.cuda.synchronize()
            ops.check_device_error()
            assert torch.equal(torch.stack([b.ids for b in st.bufs]), ids_e), rep
            assert torch.equal(st.y, y_e), rep
            st.token_eager()                                 # eager work between replays
            torch.cuda.synchronize()
        print("prefill: graph replays == eager over 48 layers x 512 tokens", flush=True)
        counts = st.routed_counts()
        assert counts.max() > 64                             # multi-tile groups
        sample = np.random.default_rng(7).choice(T, 64, replace=False)
        for l in (0, 23, 47):
            X = bf16_values(x_step[l])[sample]
            Z = N.router_logits(X, bf16_bits(st.W[l]), bf16_bits(st.bias[l]), "mlx")
            ids = st.bufs[l].ids.cpu().numpy()[sample]
            sc = st.bufs[l].scores.cpu().numpy()[sample].astype(np.float64)
            for i in range(len(sample)):
                rid, _, ranked = N.top_k_experts(Z[i], g.top_k, g.norm_topk_prob, "mlx")
                assert N.ids_match(ranked, rid, ids[i]), (l, sample[i])
            cache = {}

            def expert(e, l=l, cache=cache):
                if e not in cache:
                    rec = st.store[l * st.E + int(e)].cpu().numpy()
                    cache[e] = OL.split_record(rec, g.d_model, g.d_ff, False)
                return cache[e]
            yv = bf16_values(y_e[l])[sample]
            for mode in ("f64", "mlx"):
                ref = N.moe_block_batch(X, ids, sc, expert, "qwen3", mode)
                err = max(N.rel_err(yv[i], ref[i]) for i in range(len(sample)))
                print(f"prefill layer {l}: worst rel err vs {mode} oracle over "
                      f"{len(sample)} tokens {err:.2e}", flush=True)
                assert err < TOL, (l, mode, err)
    finally:
        del st
        _free()
