"""Pin the numpy oracle (oracle/numerics.py) with checks that do not retype
its formulas: brute force on tiny inputs, closed forms, special cases that
reduce to textbook routines, invariants, and the reference's own constants.
Each check is chosen so that a plausible mistake (wrong nibble order, a
dropped bias term, a transposed operand, a sign slip) fails it."""
import itertools
import math

import numpy as np
import pytest

from oracle import numerics as N


# ---------------------------------------------------------------- bf16 -----
def test_bf16_roundtrip_every_pattern():
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = N.bf16_bits_to_f32(bits)
    finite = np.isfinite(vals)
    back = N.f32_to_bf16_bits(vals[finite])
    np.testing.assert_array_equal(back, bits[finite])


def test_bf16_round_half_to_even_known_answers():
    # 1 + 2^-8 lies exactly between bf16 1.0 and 1 + 2^-7: ties to even -> 1.0
    assert N.bf16r(1.0 + 2 ** -8) == 1.0
    # 1 + 3*2^-8 lies between 1+2^-7 (odd mantissa) and 1+2^-6: -> 1+2^-6
    assert N.bf16r(1.0 + 3 * 2 ** -8) == 1.0 + 2 ** -6
    assert N.bf16r(1.0 + 2 ** -8 + 2 ** -20) == 1.0 + 2 ** -7
    assert N.bf16r(-2.0) == -2.0
    assert N.bf16r(0.1) == np.float32(0.10009765625)   # 0x3DCD
    assert N.f32_to_bf16_bits(1.0) == 0x3F80


# ------------------------------------------------------------- nibbles -----
def test_unpack_nibble_order_known_answer():
    # element i lives in word i>>3 at bit 4*(i&7), low nibble first
    # (kernels.py:135-139, verify_120b.py:95)
    W = np.array([[0x76543210, 0xFEDCBA98]], dtype=np.uint32)
    np.testing.assert_array_equal(N.unpack_u4(W)[0], np.arange(16))


def test_unpack_bruteforce_and_pack_inverse():
    rng = np.random.default_rng(0)
    W = rng.integers(0, 2 ** 32, (5, 4), dtype=np.uint64).astype(np.uint32)
    q = N.unpack_u4(W)
    for o in range(5):
        for i in range(32):
            word = int(W[o, i // 8])
            assert q[o, i] == (word >> (4 * (i % 8))) & 0xF
    np.testing.assert_array_equal(N.pack_u4(q), W)


# ------------------------------------------------------------- dequant -----
def _rand_expert_row(rng, n_out, n_in):
    W = rng.integers(0, 2 ** 32, (n_out, n_in // 8), dtype=np.uint64).astype(np.uint32)
    S = N.f32_to_bf16_bits(np.abs(rng.normal(0, 0.02, (n_out, n_in // 64))))
    B = N.f32_to_bf16_bits(rng.normal(0, 0.02, (n_out, n_in // 64)))
    return W, S, B


def test_dequant_bruteforce():
    rng = np.random.default_rng(1)
    W, S, B = _rand_expert_row(rng, 3, 128)
    d = N.dequant(W, S, B)
    for o, i in itertools.product(range(3), range(128)):
        q = (int(W[o, i // 8]) >> (4 * (i % 8))) & 0xF
        s = float(N.bf16_bits_to_f32(S[o, i // 64]))
        b = float(N.bf16_bits_to_f32(B[o, i // 64]))
        assert d[o, i] == s * q + b


def test_dequant_synthetic_bias_is_centering():
    # the workloads set biases = -8*scale, so w = scale*(q-8) exactly
    rng = np.random.default_rng(2)
    W, S, _ = _rand_expert_row(rng, 4, 64)
    B = N.f32_to_bf16_bits(-8.0 * N.bf16_bits_to_f32(S))
    d = N.dequant(W, S, B)
    q = N.unpack_u4(W).astype(np.float64)
    s = np.repeat(N.bf16_bits_to_f32(S).astype(np.float64), 64, axis=1)
    np.testing.assert_array_equal(d, s * (q - 8))


def test_qmv_equals_dense_dot():
    # the per-group factorised form (kernels.py:141-145) == dense dequant @ x
    rng = np.random.default_rng(3)
    W, S, B = _rand_expert_row(rng, 17, 256)
    x = rng.normal(size=256)
    np.testing.assert_allclose(N.qmv(x, W, S, B), N.dequant(W, S, B) @ x,
                               rtol=1e-12, atol=1e-12)


def test_qmv_known_answers():
    # all codes 9, bias -8*scale: w = scale, so y_o = scale_o * sum(x)
    n_in = 128
    W = np.full((2, n_in // 8), 0x99999999, dtype=np.uint32)
    S = N.f32_to_bf16_bits(np.array([[0.5, 0.5], [0.25, 0.25]]))
    B = N.f32_to_bf16_bits(-8 * N.bf16_bits_to_f32(S))
    x = np.arange(n_in, dtype=np.float64)
    np.testing.assert_allclose(N.qmv(x, W, S, B), [0.5 * x.sum(), 0.25 * x.sum()])
    # a different scale per group: groups must not be swapped
    S2 = N.f32_to_bf16_bits(np.array([[1.0, 2.0]]))
    B2 = N.f32_to_bf16_bits(np.zeros((1, 2)))
    W2 = np.full((1, n_in // 8), 0x11111111, dtype=np.uint32)     # all codes 1
    y = N.qmv(x, W2, S2, B2)[0]
    assert y == 1.0 * x[:64].sum() + 2.0 * x[64:].sum()


# --------------------------------------------------------- activations -----
def test_swiglu_closed_forms():
    g = np.array([0.0, 1.0, -1.0, 10.0, -30.0])
    u = np.array([3.0, 2.0, 2.0, 1.0, 5.0])
    expect = [0.0, 2.0 / (1 + math.exp(-1.0)), -2.0 / (1 + math.e), 10.0 / (1 + math.exp(-10)),
              -30.0 * 5.0 / (1 + math.exp(30.0))]
    np.testing.assert_allclose(N.swiglu(g, u), expect, rtol=1e-13)


def test_swiglu_clamped_special_cases():
    # gate saturates at 7; up clips to [-7, 7]; out = g*sig(1.702 g)*(u+1)
    sig = lambda z: 1 / (1 + math.exp(-z))
    up = np.array([0.0, 100.0, -100.0, -1.0, 2.0])
    gate = np.array([100.0, 7.0, 1.0, 3.0, -2.0])
    expect = [7 * sig(1.702 * 7) * 1.0, 7 * sig(1.702 * 7) * 8.0, 1 * sig(1.702) * -6.0,
              0.0, -2 * sig(-3.404) * 3.0]
    np.testing.assert_allclose(N.swiglu_clamped(up, gate), expect, rtol=1e-13, atol=1e-15)
    # argument order: (up, gate) -- swapping them changes the result
    assert not np.allclose(N.swiglu_clamped(gate, up), expect)


def test_mlx_mode_rounds_to_bf16():
    g = np.linspace(-3, 3, 11)
    u = np.linspace(1, 2, 11)
    y = N.swiglu(g, u, "mlx")
    np.testing.assert_array_equal(y, N.bf16r(y))
    assert N.rel_err(y, N.swiglu(g, u)) < 2 ** -7


# ------------------------------------------------------------- routers -----
def test_top_k_experts_bruteforce():
    rng = np.random.default_rng(5)
    for _ in range(20):
        z = rng.normal(size=128)
        ids, sc, p = N.top_k_experts(z, 8, True)
        full = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
        order = sorted(range(128), key=lambda e: -full[e])[:8]
        assert list(ids) == order
        np.testing.assert_allclose(sc, full[order] / full[order].sum(), rtol=1e-12)
        assert abs(sc.sum() - 1) < 1e-12
        assert len(set(ids.tolist())) == 8


def test_top_k_route_and_lookahead_share_argmax():
    # softmax is monotone: top-k of logits == top-k of probabilities
    # (engine_v3.py:476-482, engine_120b.py:19-22)
    rng = np.random.default_rng(6)
    z = rng.normal(size=128)
    a, _, _ = N.top_k_experts(z, 4, False)
    b, sc, _ = N.top_k_route(z, 4)
    c = N.top_k_indices(z, 4)
    assert list(a) == list(b) == list(c)
    ex = np.exp(z[b] - z[b].max())
    np.testing.assert_allclose(sc, ex / ex.sum(), rtol=1e-12)


def test_router_logits_orientation_and_bias():
    # logits = W @ x + b with W [E, D]: a transposed operand would fail this
    W = np.zeros((3, 4))
    W[0, 1] = 1.0
    W[2, 3] = 2.0
    x = np.array([5.0, 7.0, 11.0, 13.0])
    b = np.array([0.5, -1.0, 0.0])
    z = N.router_logits(x, N.f32_to_bf16_bits(W), N.f32_to_bf16_bits(b))
    np.testing.assert_array_equal(z, [7.5, -1.0, 26.0])


def test_rank_desc_ties_to_lower_index():
    v = np.array([1.0, 3.0, 3.0, 2.0, 3.0])
    assert list(N.rank_desc(v)) == [1, 2, 4, 3, 0]


def test_ids_match_tie_rule():
    v = np.array([5.0, 4.0, 3.0, 3.0, 1.0])
    assert N.ids_match(v, [0, 1, 2], [0, 1, 3])      # exact tie at the boundary
    assert not N.ids_match(v, [0, 1, 2], [0, 1, 4])  # not a tie
    assert not N.ids_match(v, [0, 1, 2], [0, 2, 3])  # drops a sure member
    w = np.array([5.0, 4.0, 3.0, 3.0 - 2 ** -7, 1.0])  # within one bf16 ulp
    assert N.ids_match(w, [0, 1, 2], [0, 1, 3])
    assert not N.ids_match(v, [0, 1, 2], [0, 1, 1])  # duplicate ids


# -------------------------------------------------------------- blocks -----
def _expert(rng, D, F, bias=False):
    e = {}
    for p, (o, i) in (("gate_proj", (F, D)), ("up_proj", (F, D)), ("down_proj", (D, F))):
        W, S, B = _rand_expert_row(rng, o, i)
        e[f"{p}.weight"], e[f"{p}.scales"], e[f"{p}.biases"] = W, S, B
        if bias:
            e[f"{p}.bias"] = N.f32_to_bf16_bits(rng.normal(0, 0.02, o))
    return e


def test_block_dense_reference_qwen3():
    rng = np.random.default_rng(7)
    D, F = 128, 64
    exps = [_expert(rng, D, F) for _ in range(3)]
    x = rng.normal(size=D)
    sc = np.array([0.5, 0.3, 0.2])
    y = N.moe_block(x, exps, sc, "qwen3", "f64")
    ref = np.zeros(D)
    for e, s in zip(exps, sc):
        Wg = N.dequant(e["gate_proj.weight"], e["gate_proj.scales"], e["gate_proj.biases"])
        Wu = N.dequant(e["up_proj.weight"], e["up_proj.scales"], e["up_proj.biases"])
        Wd = N.dequant(e["down_proj.weight"], e["down_proj.scales"], e["down_proj.biases"])
        g, u = Wg @ x, Wu @ x
        ref += s * (Wd @ (g / (1 + np.exp(-g)) * u))
    np.testing.assert_allclose(y, ref, rtol=1e-10, atol=1e-12)
    # the mlx emulation stays within the tolerance of the truth
    assert N.rel_err(N.moe_block(x, exps, sc, "qwen3", "mlx"), ref) < 2e-2


def test_block_dense_reference_gptoss_bias_and_clamp():
    rng = np.random.default_rng(8)
    D, F = 128, 128
    exps = [_expert(rng, D, F, bias=True) for _ in range(2)]
    x = rng.normal(size=D) * 3
    sc = np.array([0.6, 0.4])
    y = N.moe_block(x, exps, sc, "gptoss", "f64")
    ref = np.zeros(D)
    for e, s in zip(exps, sc):
        def proj(p, v):
            W = N.dequant(e[f"{p}.weight"], e[f"{p}.scales"], e[f"{p}.biases"])
            return W @ v + N.bf16_bits_to_f32(e[f"{p}.bias"])
        g = np.minimum(proj("gate_proj", x), 7.0)
        u = np.clip(proj("up_proj", x), -7.0, 7.0)
        h = g / (1 + np.exp(-1.702 * g)) * (u + 1)
        ref += s * proj("down_proj", h)
    np.testing.assert_allclose(y, ref, rtol=1e-10, atol=1e-12)


def test_qmm_rows_equal_qmv():
    rng = np.random.default_rng(11)
    W, S, B = _rand_expert_row(rng, 24, 192)
    X = rng.normal(size=(5, 192))
    Y = N.qmm(X, W, S, B)
    assert Y.shape == (5, 24)
    for t in range(5):
        np.testing.assert_allclose(Y[t], N.qmv(X[t], W, S, B), rtol=1e-12, atol=1e-14)


def test_router_logits_rows_equal_single_token():
    rng = np.random.default_rng(12)
    W = N.f32_to_bf16_bits(rng.normal(0, 0.02, (16, 64)))
    b = N.f32_to_bf16_bits(rng.normal(0, 0.1, 16))
    X = rng.normal(size=(3, 64))
    Z = N.router_logits(X, W, b)
    for t in range(3):
        np.testing.assert_allclose(Z[t], N.router_logits(X[t], W, b), rtol=1e-13)


@pytest.mark.parametrize("kind", ["qwen3", "gptoss"])
def test_block_batch_equals_per_token(kind):
    """The grouped (per-expert batched) restatement equals the per-token
    block on every token, with experts repeating across tokens."""
    rng = np.random.default_rng(13)
    D, F, E, T, k = 128, 64, 6, 9, 3
    exps = [_expert(rng, D, F, bias=(kind == "gptoss")) for _ in range(E)]
    X = rng.normal(size=(T, D))
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    sc = rng.dirichlet(np.ones(k), T)
    for mode in ("f64", "mlx"):
        Y = N.moe_block_batch(X, ids, sc, lambda e: exps[e], kind, mode)
        for t in range(T):
            y = N.moe_block(X[t], [exps[e] for e in ids[t]], sc[t], kind, mode)
            if mode == "f64":
                np.testing.assert_allclose(Y[t], y, rtol=1e-10, atol=1e-12)
            else:   # bf16 rounding points may flip by one ulp on a sum-order change
                assert N.rel_err(Y[t], y) < 2 ** -6


def test_combine_permutation_invariant_and_linear():
    rng = np.random.default_rng(9)
    ys = rng.normal(size=(8, 16))
    s = rng.random(8)
    p = rng.permutation(8)
    np.testing.assert_allclose(N.combine(ys, s), N.combine(ys[p], s[p]), rtol=1e-13)
    np.testing.assert_allclose(N.combine(ys, 2 * s), 2 * N.combine(ys, s), rtol=1e-13)


def test_rel_err_definition():
    # max|a-b| / max|b| (test_kernel.py:68-71)
    assert N.rel_err([1.0, 2.0], [1.0, 4.0]) == pytest.approx(0.5)
