"""Seeded synthetic expert stores and router inputs for the benchmark
workloads (no checkpoints are available offline).

Weights: 4-bit codes uniform in 0..15 (uniform 32-bit words), bf16 scales
|N(0, 0.02)|, bf16 quantisation biases -8 * scale, bf16 projection biases
N(0, 0.02) where the geometry has them.  Router weights bf16 N(0, 0.02).
Everything is generated on the target device with torch's seeded generator.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from .geometry import Geometry

SEED_BASE = 20260000


def generator(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def comp_view(store: torch.Tensor, geom: Geometry, name: str) -> torch.Tensor:
    """[n_records, *shape] typed view of one component inside a uint8 record
    store shaped [n_records, record_bytes]."""
    c = geom.comp(name)
    dt = torch.int32 if c.dtype == "U32" else torch.bfloat16
    n = store.shape[0]
    return store[:, c.offset:c.offset + c.nbytes].view(dt).view(n, *c.shape)


def fill_records(store: torch.Tensor, geom: Geometry, gen: torch.Generator,
                 chunk_bytes: int = 256 << 20) -> None:
    """Write synthetic expert weights into every record of `store`."""
    n = store.shape[0]
    chunk = max(1, chunk_bytes // geom.record_bytes)
    for lo in range(0, n, chunk):
        _fill_chunk(store[lo:min(n, lo + chunk)], geom, gen)


def _fill_chunk(part: torch.Tensor, geom: Geometry, gen: torch.Generator) -> None:
    dev = part.device
    for p in ("gate_proj", "up_proj", "down_proj"):
        w = comp_view(part, geom, f"{p}.weight")
        w.copy_(torch.randint(-2**31, 2**31, w.shape, dtype=torch.int64,
                              generator=gen, device=dev).to(torch.int32))
        s = comp_view(part, geom, f"{p}.scales")
        sv = (torch.randn(s.shape, generator=gen, device=dev) * 0.02).abs()
        s.copy_(sv.to(torch.bfloat16))
        b = comp_view(part, geom, f"{p}.biases")
        b.copy_((s.float() * -8.0).to(torch.bfloat16))   # exact: power of 2
        if geom.has_proj_bias:
            pb = comp_view(part, geom, f"{p}.bias")
            pb.copy_((torch.randn(pb.shape, generator=gen, device=dev) * 0.02
                      ).to(torch.bfloat16))


def make_store(geom: Geometry, n_records: int, device, seed: int) -> torch.Tensor:
    store = torch.zeros((n_records, geom.record_bytes), dtype=torch.uint8,
                        device=device)
    fill_records(store, geom, generator(device, seed))
    return store


def make_host_store(geom: Geometry, n_records: int, device, seed: int,
                    chunk_bytes: int = 256 << 20):
    """The records of make_store(geom, n_records, device, seed), byte for
    byte, in a pinned host store: generated chunk by chunk on `device` with
    the same generator sequence and copied down."""
    from .pool import HostStore
    hs = HostStore(geom, n_records)
    gen = generator(device, seed)
    chunk = max(1, chunk_bytes // geom.record_bytes)
    buf = torch.zeros((chunk, geom.record_bytes), dtype=torch.uint8, device=device)
    for lo in range(0, n_records, chunk):
        hi = min(n_records, lo + chunk)
        part = buf[:hi - lo]
        part.zero_()
        _fill_chunk(part, geom, gen)
        torch.from_numpy(hs.array[lo:hi]).copy_(part.cpu())
    del buf
    return hs


def router_weights(geom: Geometry, n_layers: int, device, seed: int,
                   with_bias: bool = False):
    g = generator(device, seed)
    W = (torch.randn((n_layers, geom.n_experts, geom.d_model), generator=g,
                     device=device) * 0.02).to(torch.bfloat16)
    b = None
    if with_bias:
        b = (torch.randn((n_layers, geom.n_experts), generator=g, device=device)
             * 0.02).to(torch.bfloat16)
    return W, b


def zipf_log_popularity(n_layers: int, n_experts: int, s: float,
                        seed: int) -> np.ndarray:
    """Per-layer expert popularity p_e proportional to rank^-s under a seeded
    per-layer permutation; returned as ln p_e (added to router logits)."""
    rng = np.random.default_rng(np.random.SeedSequence(seed))
    ranks = np.arange(1, n_experts + 1, dtype=np.float64)
    p = ranks ** -s
    p /= p.sum()
    out = np.empty((n_layers, n_experts))
    for L in range(n_layers):
        out[L, rng.permutation(n_experts)] = np.log(p)
    return out


def hidden_states(n_tokens: int, n_layers: int, d_model: int, device, seed: int,
                  step: float = 0.1) -> torch.Tensor:
    """Residual-stream inputs per token and layer: h_0 ~ N(0,1) and
    h_{L+1} = h_L + step * N(0,1), stored bf16 [n_tokens, n_layers, d_model]."""
    g = generator(device, seed)
    h0 = torch.randn((n_tokens, 1, d_model), generator=g, device=device)
    inc = torch.randn((n_tokens, n_layers - 1, d_model), generator=g,
                      device=device) * step
    h = torch.cat([h0, h0 + torch.cumsum(inc, dim=1)], dim=1)
    return h.to(torch.bfloat16).contiguous()


def slot_permutation(n_slots: int, n_experts: int, seed: int) -> np.ndarray:
    """expert -> slot placement, rng.permutation(n_slots)[:n_experts]."""
    rng = np.random.default_rng(np.random.SeedSequence(seed))
    return rng.permutation(n_slots)[:n_experts].astype(np.int64)


def popular_pairs(logpop: np.ndarray, per_layer: int) -> list:
    """The `per_layer` most popular experts of every layer, (layer, expert)."""
    out = []
    for L in range(logpop.shape[0]):
        order = np.lexsort((np.arange(logpop.shape[1]), -logpop[L]))
        out += [(L, int(e)) for e in order[:per_layer]]
    return out


def bf16_bias_from_log(logpop: np.ndarray, device) -> torch.Tensor:
    return torch.tensor(logpop, dtype=torch.float32, device=device).to(torch.bfloat16)


def n_bytes_human(n: int) -> str:
    e = int(math.log(max(n, 1), 1024))
    return f"{n / 1024 ** e:.2f} {['B', 'KiB', 'MiB', 'GiB', 'TiB'][e]}"
