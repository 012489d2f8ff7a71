"""moe_ffn_decode_static, the entry point that allocates nothing: through
the C ABI, on two calls in a row (the second with fewer tokens, so stale
activations from the first sit in the static scratch), its outputs equal
moe_ffn_decode's bit for bit -- the same kernels, a different activation
buffer -- on the Qwen3 and the gpt-oss geometries."""
import ctypes as C

import pytest
import torch

from moe_stream_amd import _lib, ops
from moe_stream_amd import geometry as G

from helpers import Layer, bf16_randn

pytestmark = pytest.mark.gpu


def _static(layer, refs, scores, x, out, out32):
    g = layer.geom
    T, k = refs.shape
    return _lib.lib().moe_ffn_decode_static(
        C.byref(layer.pool.c_view()), C.byref(g.c_geom()), refs.data_ptr(), scores.data_ptr(),
        x.data_ptr(), T, k, out.data_ptr(), out32.data_ptr(), _lib.stream_ptr())


@pytest.mark.parametrize("geom,seed", [(G.QWEN3_30B_A3B, 20260801), (G.GPT_OSS_120B, 20260811)])
def test_static_scratch_equals_workspace_path(geom, seed):
    layer = Layer(geom, 256 if geom.d_model == 2048 else 160, seed=seed,
                  router_bias=geom.has_proj_bias)
    for call, T in enumerate((5, 2)):
        x = bf16_randn((T, geom.d_model), seed=seed + 10 + call)
        b = ops.route(x, layer.W, layer.bias, geom.routing, geom.norm_topk_prob, geom.top_k,
                      table=layer.table)
        ref = torch.zeros((T, geom.d_model), dtype=torch.bfloat16, device="cuda")
        ref32 = torch.zeros((T, geom.d_model), dtype=torch.float32, device="cuda")
        ops.ffn_decode(layer.pool, b.slot_refs, b.scores, x, out=ref, out_f32=ref32)
        out = torch.full((T, geom.d_model), 7.0, dtype=torch.bfloat16, device="cuda")
        out32 = torch.full((T, geom.d_model), 7.0, dtype=torch.float32, device="cuda")
        _lib.check(_static(layer, b.slot_refs, b.scores, x, out, out32))
        torch.cuda.synchronize()
        ops.check_device_error()
        assert torch.equal(out, ref), (geom.name, call)
        assert torch.equal(out32, ref32), (geom.name, call)


def test_static_scratch_rejects_oversized_calls():
    layer = Layer(G.QWEN3_30B_A3B, 256, seed=20260821)
    limit = _lib.lib().moe_ffn_decode_static_bytes()
    T = limit // (8 * 768 * 2) + 1
    x = torch.zeros((T, 2048), dtype=torch.bfloat16, device="cuda")
    refs = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
    sc = torch.zeros((T, 8), dtype=torch.float32, device="cuda")
    out = torch.zeros((T, 2048), dtype=torch.bfloat16, device="cuda")
    out32 = torch.zeros((T, 2048), dtype=torch.float32, device="cuda")
    assert _static(layer, refs, sc, x, out, out32) == _lib.MOE_ERR_INVALID
    assert b"static scratch" in _lib.lib().moe_last_error()
