"""The MoE block seam: `streaming_call(block, x) -> y` (engine_v3.py:493-609,
engine_120b.py:78-149) on the HBM slot pool and the gfx950 kernels.

The reference's flow per layer is kept: route and speculate in one device
launch, ONE host synchronisation for both results, prefetch the predicted
experts of layer L+d, acquire this layer's experts (misses filled, pending
prefetches waited on as stream dependencies), then the fused expert block.
Nothing is written back to the host except the routed and predicted ids.

For the fully device-resident decode path with no per-layer host round trip
see stack.DecodeStack.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib, ops
from .geometry import Geometry
from .pool import ExpertPool, env_depths, env_widen


def top_k_experts(x: torch.Tensor, W: torch.Tensor, k: int, norm: bool):
    """Qwen3 routing on device: softmax over all experts, top-k of the bf16
    probabilities, renormalised scores (engine_v3.py:467-473).  Returns
    (ids int32 [T,k], scores fp32 [T,k])."""
    b = ops.route(x, W, None, _lib.MOE_ROUTE_SOFTMAX_TOPK, norm, k)
    return b.ids, b.scores


def top_k_route(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, k: int):
    """gpt-oss routing on device: top-k of the raw logits, softmax over the k
    (engine_120b.py:65-70)."""
    b = ops.route(x, W, bias, _lib.MOE_ROUTE_TOPK_SOFTMAX, False, k)
    return b.ids, b.scores


def top_k_indices(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, k: int):
    """Lookahead ids: top-k of the raw logits of a later layer's router on
    this layer's hidden state (engine_v3.py:476-483, engine_120b.py:73-75)."""
    # the route launch ranks the lookahead rows; any k >= 1 router is needed
    b = ops.route(x, W, bias, _lib.MOE_ROUTE_TOPK_SOFTMAX, False, 1,
                  W_next=W, bias_next=bias, k_pred=k)
    return b.pred


class MoEBlock:
    """One layer's MoE block.  `blocks` is the shared list of all layers'
    blocks (the module-level _BLOCKS of the reference), used for the
    lookahead routers of layers L+d."""

    def __init__(self, layer: int, geom: Geometry, pool: ExpertPool,
                 router_W: torch.Tensor, router_bias: torch.Tensor | None,
                 blocks: list, depths=None, widen: int | None = None):
        """depths / widen: the prefetch depths and speculation width; by
        default PF_DEPTH and PF_WIDEN from the environment, as the
        reference's module constants (engine_v3.py:61,84)."""
        self._layer = layer
        self.geom = geom
        self.pool = pool
        self.W = router_W
        self.bias = router_bias
        self.blocks = blocks
        self.depths = tuple(depths) if depths is not None else env_depths()
        self.widen = int(widen) if widen is not None else env_widen()
        self.top_k = geom.top_k
        self.norm_topk_prob = geom.norm_topk_prob
        self.recall = []            # measured lookahead recall, as _RECALL
        self._pred = {}

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return streaming_call(self, x)


_PRED = {}


def streaming_call(self: MoEBlock, x: torch.Tensor) -> torch.Tensor:
    """x bf16 [B, T, D] or [T, D] -> y of the same shape."""
    pool, layer, blocks, g = self.pool, self._layer, self.blocks, self.geom
    shape = x.shape
    xt = x.reshape(-1, shape[-1]).contiguous()
    T, k = xt.shape[0], self.top_k
    # route + one lookahead in a single launch; further depths launch again
    preds = []
    tgt0 = layer + self.depths[0]
    first = blocks[tgt0] if tgt0 < len(blocks) else None
    kp = min(k * self.widen, g.n_experts, 64)
    b = ops.route(xt, self.W, self.bias, g.routing, g.norm_topk_prob, k,
                  W_next=first.W if first is not None else None,
                  bias_next=first.bias if first is not None else None, k_pred=kp)
    if first is not None:
        preds.append((tgt0, self.depths[0], b.pred))
    for d in self.depths[1:]:
        tgt = layer + d
        if tgt < len(blocks):
            preds.append((tgt, d, top_k_indices(xt, blocks[tgt].W, blocks[tgt].bias, kp)))
    # ONE host synchronisation for routing and speculation (engine_v3.py:515)
    host = [b.ids] + [p for _, _, p in preds]
    host = [h.cpu() for h in host]
    ids = host[0].numpy().reshape(-1)
    for (tgt, d, _), p in zip(preds, host[1:]):
        pred = np.unique(p.numpy().reshape(-1))
        if d == self.depths[0]:
            _PRED[(id(pool), tgt)] = set(pred.tolist())
        pool.prefetch(tgt, pred)
    if ids.size == k:
        uniq, inverse = ids, None
    else:
        uniq, inverse = np.unique(ids, return_inverse=True)
    key = (id(pool), layer)
    if key in _PRED:
        want = set(uniq.tolist())
        self.recall.append(len(want & _PRED.pop(key)) / len(want))
    slots = np.asarray(pool.acquire(layer, uniq), dtype=np.int32)
    refs = (slots if inverse is None else slots[inverse]).reshape(T, k)
    refs_d = torch.from_numpy(np.ascontiguousarray(refs)).to(xt.device, non_blocking=True)
    # decode kernels for a few tokens, the grouped MFMA block for prefill
    y = ops.ffn(pool, refs_d, b.scores, xt)
    return y.reshape(shape)
