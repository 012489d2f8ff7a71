"""GPU parity of the reference's fused-kernel entry, kernels.moe_expert_mlp
(kernels.py:231-252), over a flat uint32 pool of repacked records at the
one-layer Qwen3 workload (128 experts, 2048 x 768, top-8): against the fp64
and MLX-emulation oracles, bit-identical to the decode block over the
component pool, chunked above 16 experts, and the ValueError paths."""
import numpy as np
import pytest
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import kernels as K
from moe_stream_amd import ops
from oracle import numerics as N

from helpers import TOL, Layer, bf16_randn, bf16_values

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    return Layer(G.QWEN3_30B_A3B, 256, seed=20260001)


def _flat(layer):
    # the store is [n_records, record_bytes]: as a flat uint32 buffer it is a
    # pool whose slot e holds expert e, the reference's pool_u32
    return layer.store.view(torch.int32).reshape(-1)


def test_moe_expert_mlp_matches_oracle(layer):
    x = bf16_randn((2048,), seed=20260901)
    bufs = ops.route(x.view(1, -1), layer.W, None, 0, True, 8)
    ids = bufs.ids[0].to(torch.int32)
    sc = bufs.scores[0]
    y = K.moe_expert_mlp(_flat(layer), ids, x, sc)
    torch.cuda.synchronize()
    ops.check_device_error()
    assert y.dtype == torch.float32 and y.shape == (2048,)
    x64 = bf16_values(x)
    idn, scn = ids.cpu().numpy(), sc.cpu().numpy().astype(np.float64)
    e64 = N.rel_err(y.cpu().numpy(), layer.block_oracle(x64, idn, scn, "f64"))
    emlx = N.rel_err(y.cpu().numpy(), layer.block_oracle(x64, idn, scn, "mlx"))
    print(f"moe_expert_mlp: rel err vs f64 {e64:.2e}, vs MLX-emulation {emlx:.2e}")
    assert e64 < TOL and emlx < TOL
    # the same kernels over the component pool (slots at the permutation)
    refs = torch.tensor(layer.perm[idn][None], dtype=torch.int32, device="cuda")
    y2 = torch.zeros((1, 2048), dtype=torch.float32, device="cuda")
    ops.ffn_decode(layer.pool, refs, sc.view(1, -1).contiguous(), x.view(1, -1), out_f32=y2)
    torch.cuda.synchronize()
    assert torch.equal(y, y2[0])


def test_moe_expert_mlp_more_experts_than_one_launch(layer):
    """20 active experts: two launches whose fp32 results are summed."""
    x = bf16_randn((2048,), seed=20260902)
    rng = np.random.default_rng(5)
    ids = rng.permutation(128)[:20]
    sc = rng.dirichlet(np.ones(20)).astype(np.float32)
    y = K.moe_expert_mlp(_flat(layer), torch.tensor(ids, dtype=torch.int32),
                         x, torch.tensor(sc))
    torch.cuda.synchronize()
    ref = layer.block_oracle(bf16_values(x), ids, sc.astype(np.float64), "f64")
    assert N.rel_err(y.cpu().numpy(), ref) < TOL


def test_moe_expert_mlp_rejects(layer):
    x = bf16_randn((2048,), seed=20260903)
    with pytest.raises(ValueError, match="slot outside"):
        K.moe_expert_mlp(_flat(layer), torch.tensor([0, 128]), x, torch.tensor([.5, .5]))
    with pytest.raises(ValueError, match="multiple of 4 quant groups"):
        K.moe_expert_mlp(_flat(layer), torch.tensor([0]), x, torch.tensor([1.]), d_ff=700)
    with pytest.raises(ValueError, match="scores"):
        K.moe_expert_mlp(_flat(layer), torch.tensor([0, 1]), x, torch.tensor([1.]))
    # multiples of 4 groups but no compiled kernel: ValueError at the call
    with pytest.raises(ValueError, match="no gfx950 kernel"):
        K.moe_expert_mlp(_flat(layer), torch.tensor([0]), bf16_randn((1024,), seed=1),
                         torch.tensor([1.]), d_model=1024, d_ff=512)
