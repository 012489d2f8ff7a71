"""The small-T grouped expert block (2 <= T, T*k <= 256 pairs): pairs grouped
by slot, each distinct expert's codes read once per call and applied to
every token routed to it (the multi-token verification step of
spec.py:192-194).  It must give exactly what T single-token calls give, bit
for bit, and match the batched oracle (moe_block_batch, the reference's
batched gather_qmm of engine_v3.py:588-600) within the FFN tolerance."""
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
    return Layer(G.QWEN3_30B_A3B, 256, seed=20260901)


@pytest.fixture(scope="module")
def gptoss_layer():
    layer = Layer(G.GPT_OSS_120B, 136, seed=20260911, router_bias=True)
    yield layer
    del layer
    torch.cuda.empty_cache()


def _zipf_ids(rng, T, k, E, s=1.1):
    """Per token k distinct experts drawn with Zipf(s) popularity: tokens
    share the hot experts, as routed verification tokens do."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    order = rng.permutation(E)
    return np.stack([order[rng.choice(E, k, replace=False, p=p)] for _ in range(T)])


def _per_token(layer, refs, sc, x):
    T = x.shape[0]
    o = torch.zeros((T, layer.geom.d_model), dtype=torch.bfloat16, device="cuda")
    o32 = torch.zeros((T, layer.geom.d_model), dtype=torch.float32, device="cuda")
    for t in range(T):
        ops.ffn_decode(layer.pool, refs[t:t + 1].contiguous(), sc[t:t + 1].contiguous(),
                       x[t:t + 1].contiguous(), out=o[t:t + 1], out_f32=o32[t:t + 1])
    return o, o32


def _grouped_vs_per_token(layer, ids, sc_np, x, refs=None):
    T, k = ids.shape
    if refs is None:
        refs = torch.tensor(layer.perm[ids], dtype=torch.int32).cuda()
    sc = torch.tensor(sc_np, dtype=torch.float32).cuda()
    y = torch.zeros((T, layer.geom.d_model), dtype=torch.bfloat16, device="cuda")
    y32 = torch.zeros((T, layer.geom.d_model), dtype=torch.float32, device="cuda")
    ops.ffn_decode(layer.pool, refs, sc, x, out=y, out_f32=y32)
    o, o32 = _per_token(layer, refs, sc, x)
    torch.cuda.synchronize()
    assert torch.equal(y, o) and torch.equal(y32, o32)
    return y, y32


@pytest.mark.parametrize("T", [2, 4, 8, 16, 32])
def test_qwen3_grouped_equals_per_token(qwen_layer, T):
    rng = np.random.default_rng(100 + T)
    ids = _zipf_ids(rng, T, 8, 128)
    sc = rng.dirichlet(np.ones(8), T)
    x = bf16_randn((T, 2048), seed=20260920 + T)
    _grouped_vs_per_token(qwen_layer, ids, sc, x)
    distinct = len(np.unique(ids))
    print(f"T={T}: {T * 8} pairs over {distinct} distinct experts")
    assert distinct < T * 8


@pytest.mark.parametrize("T", [2, 4, 8])
def test_qwen3_grouped_against_oracle(qwen_layer, T):
    rng = np.random.default_rng(200 + T)
    ids = _zipf_ids(rng, T, 8, 128)
    sc = rng.dirichlet(np.ones(8), T).astype(np.float32)
    x = bf16_randn((T, 2048), seed=20260930 + T)
    y, y32 = _grouped_vs_per_token(qwen_layer, ids, sc, x)
    X = bf16_values(x)
    for mode, got in (("f64", y32.cpu().numpy()), ("mlx", bf16_values(y))):
        ref = N.moe_block_batch(X, ids, sc.astype(np.float64), qwen_layer.expert, "qwen3", mode)
        for t in range(T):
            err = N.rel_err(got[t], ref[t])
            assert err < TOL, (T, mode, t, err)


def test_gptoss_grouped_equals_per_token_and_oracle(gptoss_layer):
    layer = gptoss_layer
    rng = np.random.default_rng(300)
    for T in (3, 8):
        ids = _zipf_ids(rng, T, 4, 128)
        sc = rng.dirichlet(np.ones(4), T).astype(np.float32)
        x = bf16_randn((T, 2880), seed=20260940 + T)
        y, y32 = _grouped_vs_per_token(layer, ids, sc, x)
        ref = N.moe_block_batch(bf16_values(x), ids, sc.astype(np.float64), layer.expert,
                                "gptoss", "f64")
        for t in range(T):
            assert N.rel_err(y32.cpu().numpy()[t], ref[t]) < TOL


def test_every_token_on_the_same_experts(qwen_layer):
    """Maximal sharing (every token routed to the same 8 experts, one of them
    read from the store, one from the pool): 8 distinct slots serve 128
    pairs; more tokens than one staging pass holds."""
    T = 16
    rng = np.random.default_rng(7)
    ids = np.tile(rng.permutation(128)[:8], (T, 1))
    sc = rng.dirichlet(np.ones(8), T)
    refs = qwen_layer.perm[ids].astype(np.int32)
    refs[:, 3] = -(ids[:, 3] + 1)          # the store record of the same expert
    x = bf16_randn((T, 2048), seed=20260950)
    _grouped_vs_per_token(qwen_layer, ids, sc, x, torch.tensor(refs).cuda())


def test_out_of_range_ref_in_a_group(qwen_layer):
    """An out-of-range ref among the pairs contributes zero and is reported;
    every other pair is computed as in single-token calls."""
    T = 4
    rng = np.random.default_rng(8)
    ids = _zipf_ids(rng, T, 8, 128)
    refs = qwen_layer.perm[ids].astype(np.int32)
    refs[1, 2] = 100000
    refs[3, 5] = 100000
    sc = torch.tensor(rng.dirichlet(np.ones(8), T), dtype=torch.float32).cuda()
    x = bf16_randn((T, 2048), seed=20260960)
    r = torch.tensor(refs).cuda()
    y = ops.ffn_decode(qwen_layer.pool, r, sc, x)
    with pytest.raises(_lib.MoeError) as ei:
        ops.check_device_error()
    assert ei.value.code == _lib.MOE_ERR_DEVICE
    o, _ = _per_token(qwen_layer, r, sc, x)
    with pytest.raises(_lib.MoeError):
        ops.check_device_error()
    torch.cuda.synchronize()
    assert torch.equal(y, o)


@pytest.mark.parametrize("geo", ["qwen3", "gptoss"])
def test_every_token_on_the_same_experts_at_the_limit(qwen_layer, gptoss_layer, geo):
    """Maximal sharing at the small-T kernels' limit (T x k = 256 pairs):
    every token routed to the same experts, so each slot serves T pairs
    (32 for Qwen3, 64 for gpt-oss); outputs equal one call per token."""
    layer = qwen_layer if geo == "qwen3" else gptoss_layer
    g = layer.geom
    T = 256 // g.top_k
    rng = np.random.default_rng(9 + g.top_k)
    ids = np.tile(rng.permutation(g.n_experts)[:g.top_k], (T, 1))
    sc = rng.dirichlet(np.ones(g.top_k), T).astype(np.float32)
    x = bf16_randn((T, g.d_model), seed=20260960 + g.top_k)
    _grouped_vs_per_token(layer, ids, sc, x)
