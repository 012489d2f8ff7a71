"""The torch CPU restatement timed by bench.py's CPU baseline, checked
against the numpy oracle: routing (ids as sets, ties excused) and the block
output within the FFN tolerance of both oracle modes, on both geometries."""
import numpy as np
import pytest
import torch

from oracle import cpu_block as CB
from oracle import layout as OL
from oracle import numerics as N

TOL = 2e-2


def _record(rng, D, F, bias):
    rec = {}
    for name, dt, shape, _, _ in OL.components(D, F, bias):
        if dt == np.uint32:
            rec[name] = rng.integers(0, 2 ** 32, shape, dtype=np.uint64).astype(np.uint32)
        elif name.endswith("bias"):
            rec[name] = N.f32_to_bf16_bits(rng.normal(0, 0.02, shape))
        elif name.endswith("scales"):
            rec[name] = N.f32_to_bf16_bits(np.abs(rng.normal(0, 0.02, shape)))
        else:   # quantisation biases: a general value, not only -8 * scale
            rec[name] = N.f32_to_bf16_bits(rng.normal(-0.16, 0.05, shape))
    return rec


@pytest.mark.parametrize("kind,D,F,E,k,routing,norm", [
    ("qwen3", 256, 128, 16, 4, 0, True),
    ("gptoss", 192, 192, 16, 4, 1, False),
])
def test_cpu_layer_matches_oracle(kind, D, F, E, k, routing, norm):
    rng = np.random.default_rng(20260701)
    bias = kind == "gptoss"
    recs = [_record(rng, D, F, bias) for _ in range(E)]
    experts = [CB.Expert(r) for r in recs]
    Wb = N.f32_to_bf16_bits(rng.normal(0, 0.02, (E, D)))
    bb = N.f32_to_bf16_bits(rng.normal(0, 0.02, E)) if bias else None
    W = CB._bits_to_f32(Wb)
    bt = None if bb is None else CB._bits_to_f32(bb)
    for t in range(3):
        xb = N.f32_to_bf16_bits(rng.normal(0, 1, D))
        x64 = N.bf16_bits_to_f32(xb).astype(np.float64)
        ids, sc, y = CB.moe_layer(CB._bits_to_f32(xb), W, bt, lambda e: experts[e], k,
                                  routing, norm, kind)
        z = N.router_logits(x64, Wb, bb, "mlx")
        if routing == 0:
            rid, _, ranked = N.top_k_experts(z, k, norm, "mlx")
        else:
            rid, _, ranked = N.top_k_route(z, k, "mlx")
        assert N.ids_match(ranked, rid, ids.numpy())
        sc64 = sc.double().numpy()
        if routing == 0 and norm:
            assert abs(sc64.sum() - 1) < 2e-2
        for mode in ("f64", "mlx"):
            ref = N.moe_block(x64, [recs[int(e)] for e in ids], sc64, kind=kind, mode=mode)
            assert N.rel_err(y.double().numpy(), ref) < TOL, (kind, t, mode)


def test_quant_matrix_is_dequant_then_dot():
    """The byte-table decode and S*q+B of QuantMatrix against the oracle's
    brute-force dequant, rows of two stacked matrices, one of them with a
    hand-set known answer (all codes 15, S = 1, B = -8: every weight 7)."""
    rng = np.random.default_rng(5)
    D = 128
    w1 = rng.integers(0, 2 ** 32, (3, D // 8), dtype=np.uint64).astype(np.uint32)
    s1 = N.f32_to_bf16_bits(np.abs(rng.normal(0, 0.1, (3, 2))))
    b1 = N.f32_to_bf16_bits(rng.normal(0, 0.1, (3, 2)))
    w2 = np.full((2, D // 8), 0xFFFFFFFF, dtype=np.uint32)
    s2 = N.f32_to_bf16_bits(np.ones((2, 2)))
    b2 = N.f32_to_bf16_bits(np.full((2, 2), -8.0))
    m = CB.QuantMatrix([(w1, s1, b1, None), (w2, s2, b2, None)])
    x = rng.normal(0, 1, D).astype(np.float32)
    y = m.matvec(torch.from_numpy(x)).double().numpy()
    ref = np.concatenate([N.dequant(w1, s1, b1) @ x, N.dequant(w2, s2, b2) @ x])
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
    assert np.allclose(y[3:], 7.0 * x.astype(np.float64).sum(), rtol=1e-5)


@pytest.mark.parametrize("kind,D,F,E,k,routing,norm", [
    ("qwen3", 256, 128, 16, 4, 0, True),
    ("gptoss", 192, 192, 16, 4, 1, False),
])
def test_cpu_layer_batch_matches_oracle_and_per_token(kind, D, F, E, k, routing, norm):
    """The many-token form: routed ids equal the per-token form's token by
    token, outputs within the FFN tolerance of the batched oracle (both
    modes)."""
    rng = np.random.default_rng(20260702)
    bias = kind == "gptoss"
    recs = [_record(rng, D, F, bias) for _ in range(E)]
    experts = [CB.Expert(r) for r in recs]
    Wb = N.f32_to_bf16_bits(rng.normal(0, 0.02, (E, D)))
    bb = N.f32_to_bf16_bits(rng.normal(0, 0.02, E)) if bias else None
    W = CB._bits_to_f32(Wb)
    bt = None if bb is None else CB._bits_to_f32(bb)
    T = 24
    xb = N.f32_to_bf16_bits(rng.normal(0, 1, (T, D)))
    X = CB._bits_to_f32(xb)
    ids, sc, Y = CB.moe_layer_batch(X, W, bt, lambda e: experts[e], k, routing, norm, kind)
    for t in range(T):
        i1, s1, y1 = CB.moe_layer(X[t], W, bt, lambda e: experts[e], k, routing, norm, kind)
        assert set(i1.tolist()) == set(ids[t].tolist()), t
        assert N.rel_err(Y[t].double().numpy(), y1.double().numpy()) < 1e-2, t
    X64 = N.bf16_bits_to_f32(xb).astype(np.float64)
    for mode in ("f64", "mlx"):
        ref = N.moe_block_batch(X64, ids.numpy(), sc.double().numpy(), lambda e: recs[e],
                                kind, mode)
        err = max(N.rel_err(Y[t].double().numpy(), ref[t]) for t in range(T))
        assert err < TOL, (kind, mode, err)
