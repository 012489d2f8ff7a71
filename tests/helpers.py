"""Shared test helpers: build device workloads and evaluate the oracle on the
same bytes (copied back to the host)."""
from __future__ import annotations

import numpy as np
import torch

from moe_stream_amd import geometry as G
from moe_stream_amd import ops, synth
from moe_stream_amd.pool import SlotPool
from oracle import layout as OL
from oracle import numerics as N

TOL = 2e-2   # max relative error for FFN outputs, bf16 with fp32 accumulation


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bf16_values(t: torch.Tensor) -> np.ndarray:
    return N.bf16_bits_to_f32(bf16_bits(t)).astype(np.float64)


class Layer:
    """One MoE layer on device: expert store (one record per expert), a slot
    pool holding the experts at a seeded random placement, router weights."""

    def __init__(self, geom: G.Geometry, n_slots: int, seed: int,
                 router_bias: bool = False, device="cuda"):
        self.geom = geom
        self.store = synth.make_store(geom, geom.n_experts, device, seed)
        self.pool = SlotPool(geom, n_slots, device, store=self.store)
        self.perm = synth.slot_permutation(n_slots, geom.n_experts, seed + 1)
        self.pool.fill(np.arange(geom.n_experts), self.perm)
        W, b = synth.router_weights(geom, 1, device, seed + 2, with_bias=router_bias)
        self.W, self.bias = W[0], (b[0] if b is not None else None)
        self.table = torch.tensor(self.perm, dtype=torch.int32, device=device)
        self._host = {}

    def expert(self, e: int) -> dict:
        """Oracle view of expert e, parsed from the store bytes."""
        if e not in self._host:
            rec = self.store[e].cpu().numpy()
            g = self.geom
            self._host[e] = OL.split_record(rec, g.d_model, g.d_ff, g.has_proj_bias)
        return self._host[e]

    def route_oracle(self, x64, mode="mlx"):
        g = self.geom
        z = N.router_logits(x64, bf16_bits(self.W),
                            None if self.bias is None else bf16_bits(self.bias), mode)
        if g.routing == 0:
            return N.top_k_experts(z, g.top_k, g.norm_topk_prob, mode)
        return N.top_k_route(z, g.top_k, mode)

    def block_oracle(self, x64, ids, scores, mode):
        kind = "qwen3" if not self.geom.has_proj_bias else "gptoss"
        return N.moe_block(x64, [self.expert(int(e)) for e in ids], scores,
                           kind=kind, mode=mode, alpha=self.geom.alpha,
                           limit=self.geom.limit)


def bf16_randn(shape, seed, device="cuda", scale=1.0):
    g = synth.generator(device, seed)
    return (torch.randn(shape, generator=g, device=device) * scale).to(torch.bfloat16)
