"""The whole-token persistent decode against the per-layer launches: same
routed ids, scores, slot refs, lookahead ids, miss counts and bit-identical
layer outputs, over several consecutive tokens (the epoch counters), plus one
layer against the oracle."""
import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import ops, synth
from moe_stream_amd.stack import DecodeStack
from oracle import layout as OL
from oracle import numerics as N

from helpers import TOL, bf16_bits, bf16_values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def stack():
    geom = G.QWEN3_30B_A3B
    # 6 layers, a pool of 384 slots (half the pairs): refs of both signs
    return DecodeStack(geom, 6, 384, "cuda", seed=20260601, zipf_s=1.1)


def test_persistent_equals_per_layer(stack):
    xs = synth.hidden_states(4, stack.L, 2048, "cuda", 20260602)
    for t in range(xs.shape[0]):
        stack.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = stack.routed()
        y_ref = stack.y.clone()
        stack.token_persistent(xs[t])
        torch.cuda.synchronize()
        ops.check_device_error()
        np.testing.assert_array_equal(stack.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(stack.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(stack.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(stack.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(stack.p_y, y_ref), t
    assert int(stack.p_miss.sum()) > 0          # some experts read from the store


def test_persistent_wide_lookahead_equals_per_layer():
    """k_pred = 16 (twice top-k): the lookahead ranks 16 experts, of which
    the kernel stages K and speculates on its spare positions only; every
    output equals the per-layer launches' (a wider k_pred once let spare
    tasks past the spare positions write into the fix-up entries)."""
    st = DecodeStack(G.QWEN3_30B_A3B, 4, 256, "cuda", seed=20260611, zipf_s=1.1, widen=2)
    assert st.k_pred == 16
    xs = synth.hidden_states(4, st.L, 2048, "cuda", 20260612)
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t])
        torch.cuda.synchronize()
        ops.check_device_error()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t
    del st
    torch.cuda.empty_cache()


def test_persistent_narrow_lookahead_equals_per_layer():
    """k_pred = 4 (half of top-k): only positions 0-3 of each layer have a
    predicted expert staged, so the routed experts of the other positions all
    go through the spare positions (lookahead ranks 8 and 9, still ranked) or
    the fix-up pass; every output equals the per-layer launches'."""
    st = DecodeStack(G.QWEN3_30B_A3B, 4, 256, "cuda", seed=20260613, zipf_s=1.1, k_pred=4)
    assert st.k_pred == 4
    xs = synth.hidden_states(3, st.L, 2048, "cuda", 20260614)
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t])
        torch.cuda.synchronize()
        ops.check_device_error()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t
    del st
    torch.cuda.empty_cache()


def test_persistent_unbiased_router_many_misses_equals_per_layer():
    """No router bias and layer inputs far apart (each layer's input adds
    noise ten times its own scale): the lookahead on the previous layer's
    input then predicts few of the routed experts, so most of each layer's 8
    go through the spare positions or the fix-up slots (up to all 8 at once);
    every output still equals the per-layer launches'."""
    st = DecodeStack(G.QWEN3_30B_A3B, 4, 256, "cuda", seed=20260615, zipf_s=None)
    xs = synth.hidden_states(3, st.L, 2048, "cuda", 20260616, step=10.0)
    unstaged = 0
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t])
        torch.cuda.synchronize()
        ops.check_device_error()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t
        unstaged += sum(len(set(ids[l]) - set(pred[l - 1])) for l in range(1, st.L))
    assert unstaged >= 3 * (st.L - 1) * 4   # on average half of the routed experts or more
    del st
    torch.cuda.empty_cache()


def test_graph_replays_equal_eager(stack):
    """The per-layer launches captured once as a HIP graph and replayed for
    several tokens, with eager work of the same stack between the replays:
    every replay routes and computes exactly what the eager launches do (the
    router's per-launch sequence word advances inside the graph too)."""
    xs = synth.hidden_states(4, stack.L, 2048, "cuda", 20260604)
    stack.capture()
    for t in range(xs.shape[0]):
        stack.run_token(xs[t], use_graph=False)
        torch.cuda.synchronize()
        ref = stack.routed(), stack.y.clone()
        stack.run_token(xs[t], use_graph=True)
        torch.cuda.synchronize()
        ops.check_device_error()
        got = stack.routed()
        for a, b in zip(got, ref[0]):
            np.testing.assert_array_equal(a, b)
        assert torch.equal(stack.y, ref[1]), t


def test_persistent_layer_against_oracle(stack):
    xs = synth.hidden_states(1, stack.L, 2048, "cuda", 20260603)
    stack.token_persistent(xs[0])
    torch.cuda.synchronize()
    Wb, bb = bf16_bits(stack.W), bf16_bits(stack.bias)
    store = stack.store
    for l in (0, stack.L - 1):
        x64 = bf16_values(xs[0, l])
        z = N.router_logits(x64, Wb[l], bb[l], "mlx")
        ref_ids, _, ranked = N.top_k_experts(z, 8, True, "mlx")
        ids = stack.p_ids[l].cpu().numpy()
        assert N.ids_match(ranked, ref_ids, ids)
        sc = stack.p_scores[l].cpu().numpy().astype(np.float64)
        exps = [OL.split_record(store[l * 128 + int(e)].cpu().numpy(), 2048, 768, False)
                for e in ids]
        ref = N.moe_block(x64, exps, sc, "qwen3", "mlx")
        assert N.rel_err(bf16_values(stack.p_y[l]), ref) < TOL
        if l + 1 < stack.L:
            zn = N.router_logits(x64, Wb[l + 1], bb[l + 1], "mlx")
            want = N.top_k_indices(zn, stack.k_pred)
            assert N.ids_match(zn, want, stack.p_pred[l].cpu().numpy())


@pytest.fixture(scope="module")
def gptoss_stack():
    geom = G.GPT_OSS_120B
    # 4 layers, 240 slots (under half the pairs): refs of both signs
    st = DecodeStack(geom, 4, 240, "cuda", seed=20260621, zipf_s=None, router_bias=True)
    yield st
    del st
    torch.cuda.empty_cache()


@pytest.mark.parametrize("ordinary", [False, True])
def test_gptoss_persistent_equals_per_layer(gptoss_stack, ordinary):
    """The wide whole-token kernel (gpt-oss geometry: top-4 of raw logits,
    projection biases, clamped SwiGLU) against the per-layer launches:
    routing, lookahead and outputs bit for bit over several tokens, with
    mispredicted experts (fix-ups) and store-resident experts."""
    st = gptoss_stack
    assert st.persistent_supported()
    xs = synth.hidden_states(5, st.L, 2880, "cuda", 20260622 + int(ordinary))
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t], ordinary=ordinary)
        st.check_persistent()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t


@pytest.mark.parametrize("ordinary", [False, True])
def test_gptoss_persistent_many_misses_equals_per_layer(gptoss_stack, ordinary):
    """The wide whole-token kernel with layer inputs far apart (noise ten
    times the input's scale added per layer): the lookahead misses most of
    the 4 routed experts, so most positions take a fix-up expert; routing,
    lookahead and outputs still equal the per-layer launches' bit for bit."""
    st = gptoss_stack
    xs = synth.hidden_states(3, st.L, 2880, "cuda", 20260631 + int(ordinary), step=10.0)
    unstaged = 0
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t], ordinary=ordinary)
        st.check_persistent()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t
        unstaged += sum(len(set(ids[l]) - set(pred[l - 1][:st.k])) for l in range(1, st.L))
    assert unstaged >= 3 * (st.L - 1) * 2   # on average half of the routed experts or more


@pytest.mark.parametrize("k_pred", [2, 8])
def test_gptoss_persistent_lookahead_width_equals_per_layer(k_pred):
    """The wide whole-token kernel with a lookahead narrower (2: positions 2
    and 3 have no staged expert) and wider (8: ranks past top-4 predicted but
    not staged) than top-4: routing, lookahead and outputs equal the
    per-layer launches' bit for bit."""
    st = DecodeStack(G.GPT_OSS_120B, 4, 240, "cuda", seed=20260641, zipf_s=None,
                     router_bias=True, k_pred=k_pred)
    assert st.k_pred == k_pred and st.persistent_supported()
    xs = synth.hidden_states(3, st.L, 2880, "cuda", 20260642 + k_pred)
    for t in range(xs.shape[0]):
        st.run_token(xs[t], use_graph=False)
        ids, sc, refs, pred = st.routed()
        y_ref = st.y.clone()
        st.token_persistent(xs[t])
        st.check_persistent()
        np.testing.assert_array_equal(st.p_ids.cpu().numpy(), ids)
        np.testing.assert_array_equal(st.p_scores.cpu().numpy(), sc)
        np.testing.assert_array_equal(st.p_refs.cpu().numpy(), refs)
        np.testing.assert_array_equal(st.p_pred.cpu().numpy()[:-1], pred[:-1])
        assert torch.equal(st.p_y, y_ref), t
    del st
    torch.cuda.empty_cache()


def test_phase_trace_leaves_outputs_unchanged(stack):
    """moe_stack_trace: a traced launch gives the untraced outputs; each
    traced workgroup stamps every layer's start in order and publishes its
    down rows after the start; a buffer too small is refused; NULL ends it."""
    from moe_stream_amd import _lib
    L = _lib.lib()
    xs = synth.hidden_states(1, stack.L, 2048, "cuda", 20260640)
    stack.token_persistent(xs[0])
    torch.cuda.synchronize()
    y0 = stack.p_y.clone()
    ids0 = stack.p_ids.clone()
    buf = torch.zeros((256, stack.L, 15), dtype=torch.int64, device="cuda")
    try:
        _lib.check(L.moe_stack_trace(buf.data_ptr(), buf.numel() * 8 - 8))
        with pytest.raises(_lib.MoeError):
            stack.token_persistent(xs[0])
        _lib.check(L.moe_stack_trace(buf.data_ptr(), buf.numel() * 8))
        stack.token_persistent(xs[0])
        torch.cuda.synchronize()
        ops.check_device_error()
    finally:
        _lib.check(L.moe_stack_trace(None, 0))
    assert torch.equal(stack.p_y, y0) and torch.equal(stack.p_ids, ids0)
    tr = buf.cpu().numpy()
    ran = tr[:, 0, 0] != 0
    assert ran.sum() >= 128, ran.sum()
    start, down = tr[ran, :, 0], tr[ran, :, 6]
    assert np.all(start > 0) and np.all(np.diff(start, axis=1) >= 0)
    assert np.all(down >= start)
    assert start.max() - start.min() < 100_000_000   # within one second
    stack.token_persistent(xs[0])                     # untraced again
    torch.cuda.synchronize()
    assert torch.equal(stack.p_y, y0)
