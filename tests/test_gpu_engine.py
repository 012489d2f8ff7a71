"""The drop-in MoE block over an ExpertPool small enough to evict: routed
outputs against the oracle, byte-exact slot fills (verify_pool.py:64-87),
the pool-size invariance of the outputs (verify_quality.py:88-97), and the
device-resident stack against the engine path."""
import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import synth
from moe_stream_amd.block import MoEBlock
from moe_stream_amd.pool import ExpertPool
from oracle import layout as OL
from oracle import numerics as N

from helpers import TOL, bf16_bits, bf16_values

pytestmark = pytest.mark.gpu

L = 4


@pytest.fixture(scope="module")
def world():
    geom = G.QWEN3_30B_A3B.with_(n_layers=L)
    store = synth.make_store(geom, L * geom.n_experts, "cuda", 20260501)
    W, _ = synth.router_weights(geom, L, "cuda", 20260502)
    xs = synth.hidden_states(3, L, geom.d_model, "cuda", 20260503)
    host = store.cpu().numpy()
    return geom, store, W, xs, host


def _blocks(geom, pool, W):
    blocks = []
    for i in range(L):
        blocks.append(MoEBlock(i, geom, pool, W[i], None, blocks))
    return blocks


def _run(geom, store, W, xs, n_slots):
    pool = ExpertPool(geom, n_slots, store=store, n_layers=L)
    blocks = _blocks(geom, pool, W)
    ys = []
    for t in range(xs.shape[0]):
        ys.append([blocks[i](xs[t, i:i + 1]) for i in range(L)])
    torch.cuda.synchronize()
    return pool, blocks, ys


def test_engine_matches_oracle_and_fills_are_exact(world):
    geom, store, W, xs, host = world
    pool, blocks, ys = _run(geom, store, W, xs, n_slots=24)
    Wb = bf16_bits(W)
    for t in range(xs.shape[0]):
        for i in range(L):
            x64 = bf16_values(xs[t, i])
            z = N.router_logits(x64, Wb[i], None, "mlx")
            ids, sc, probs = N.top_k_experts(z, 8, True, "mlx")
            exps = [OL.split_record(host[i * 128 + e], 2048, 768, False) for e in ids]
            ref = N.moe_block(x64, exps, sc, "qwen3", "mlx")
            err = N.rel_err(bf16_values(ys[t][i][0]), ref)
            assert err < TOL, (t, i, err)
    s = pool.stats()
    assert s["total"] == xs.shape[0] * L * 8
    assert s["miss"] > 0 and s["prefetch"] + s["cache"] > 0
    # every resident slot holds exactly its record's bytes
    table = pool.policy.table()
    checked = 0
    for layer in range(L):
        for e in range(128):
            slot = int(table[layer, e])
            if slot < 0 or (layer, e) in pool.pending:
                continue
            rec = OL.split_record(host[layer * 128 + e], 2048, 768, False)
            for c in geom.components:
                got = pool.views[c.name][slot].contiguous().view(torch.int16).cpu().numpy()
                assert got.tobytes() == rec[c.name].tobytes(), (layer, e, c.name)
            checked += 1
    assert checked > 0


def test_outputs_do_not_depend_on_pool_size(world):
    geom, store, W, xs, _ = world
    _, _, small = _run(geom, store, W, xs, n_slots=24)
    _, _, large = _run(geom, store, W, xs, n_slots=300)
    for a_t, b_t in zip(small, large):
        for a, b in zip(a_t, b_t):
            assert torch.equal(a, b)


def test_lookahead_recall_is_measured(world):
    geom, store, W, xs, _ = world
    _, blocks, _ = _run(geom, store, W, xs, n_slots=300)
    rec = [r for b in blocks for r in b.recall]
    assert rec and all(0.0 <= r <= 1.0 for r in rec)


def test_prefill_through_the_block(world):
    """T = 40 tokens in one call (the prefill path: many-token router, np.unique
    + inverse index build, grouped MFMA block) against the batched oracle."""
    geom, store, W, _, host = world
    # room for layer 1's experts and the lookahead's prefetch of layer 2
    # (each up to all 128 over 40 tokens), both issued before the acquire
    pool = ExpertPool(geom, 300, store=store, n_layers=L)
    blocks = _blocks(geom, pool, W)
    xs = synth.hidden_states(40, L, geom.d_model, "cuda", 20260504)
    x = xs[:, 1].contiguous()                     # 40 tokens at layer 1
    y = blocks[1](x)
    torch.cuda.synchronize()
    X = bf16_values(x)
    Z = N.router_logits(X, bf16_bits(W)[1], None, "mlx")
    ids, sc = [], []
    for t in range(40):
        i, s, _ = N.top_k_experts(Z[t], 8, True, "mlx")
        ids.append(i)
        sc.append(s)
    ref = N.moe_block_batch(X, np.array(ids), np.array(sc),
                            lambda e: OL.split_record(host[1 * 128 + e], 2048, 768, False),
                            "qwen3", "mlx")
    err = max(N.rel_err(bf16_values(y[t]), ref[t]) for t in range(40))
    assert err < TOL, err
