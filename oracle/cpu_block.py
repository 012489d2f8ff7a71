"""CPU restatement (not MLX) of the expert hot path in torch, on the host
cores: router + top-k + the k-expert block of one token.

TEST INFRASTRUCTURE ONLY: the CPU-baseline leg of ``bench.py`` times it and
``tests/test_cpu_block.py`` checks it against ``oracle.numerics``; nothing in
the product package imports it.

MLX is not installed on this host or on the GPU host, so the reference's own
CPU backend (``mx.set_default_device(mx.cpu)`` running engine_v3.py:467-473,
588-600 and engine_120b.py:65-70,132-145) cannot run.  This is the same graph
in torch on every visible core, fp32 arithmetic with MLX's bf16 rounding at
each graph edge (router logits and probabilities, each gather_qmm output,
the SwiGLU, the score products and their sum), as ``numerics`` mode "mlx"
states it.  Each 4-bit product dequantises first (codes decoded through a
256-entry byte table, w = S*q + B in fp32, kernels.py:104-106) and then
runs one fp32 matrix-vector product; gate and up share one product.

``moe_layer_batch`` is the many-token form (prefill, speculative
verification): every token routed at once, each routed expert dequantised
once and applied to all rows routed to it by one fp32 matrix product.

Parity: pinned against ``numerics`` (fp64 and MLX-emulation) in
tests/test_cpu_block.py at 2e-2 max relative error, routed ids as sets.
"""
from __future__ import annotations

import numpy as np
import torch

GROUP = 64

# byte -> (low nibble, high nibble) as fp32: element 2j of a byte row is the
# low nibble of byte j (kernels.py:135-139, little-endian words)
_LUT = torch.stack([torch.arange(256) & 15, torch.arange(256) >> 4], dim=1).to(torch.float32)


def _bf16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float32)


def _bits_to_f32(bits: np.ndarray) -> torch.Tensor:
    """bf16 bit patterns (uint16) -> fp32 values."""
    b = torch.from_numpy(np.ascontiguousarray(bits).astype(np.int32))
    return (b << 16).view(torch.float32)


class QuantMatrix:
    """4-bit affine matrices stacked along their output rows ([n_out, n_in]
    in total), held for repeated products: codes as bytes, scales and biases
    as fp32 [n_out, n_in / 64], optional projection biases."""

    def __init__(self, parts):
        """parts: [(weight u32, scales bf16 bits, biases bf16 bits, bias or
        None)], stacked in order."""
        w = np.concatenate([np.ascontiguousarray(p[0]).view(np.uint8) for p in parts])
        self.codes = torch.from_numpy(w.astype(np.int32)).view(-1)   # gather indices
        self.n_out, self.n_in = w.shape[0], w.shape[1] * 2
        self.S = _bits_to_f32(np.concatenate([p[1] for p in parts])).unsqueeze(-1)
        self.B = _bits_to_f32(np.concatenate([p[2] for p in parts])).unsqueeze(-1)
        b = [p[3] for p in parts]
        self.bias = None if b[0] is None else _bits_to_f32(np.concatenate(b))

    def matvec(self, x: torch.Tensor) -> torch.Tensor:
        """fp32 y = deq(W) @ x: the codes decoded through the byte table,
        w = S*q + B in fp32 (kernels.py:104-106), one fp32 matrix-vector
        product."""
        w = torch.index_select(_LUT, 0, self.codes).view(self.n_out, -1, GROUP)
        w.mul_(self.S).add_(self.B)
        return torch.mv(w.view(self.n_out, self.n_in), x)

    def matmul(self, X: torch.Tensor) -> torch.Tensor:
        """fp32 Y = X @ deq(W)^T for the rows X [n, n_in]: the matrix is
        dequantised once for all rows (the batched gather_qmm of the prefill
        path, engine_v3.py:588-600)."""
        w = torch.index_select(_LUT, 0, self.codes).view(self.n_out, -1, GROUP)
        w.mul_(self.S).add_(self.B)
        return X @ w.view(self.n_out, self.n_in).t()


class Expert:
    """One expert from a split record (oracle.layout): gate and up stacked
    into one [2F, D] product, down [D, F]."""

    def __init__(self, rec: dict):
        def part(p):
            return (rec[f"{p}.weight"], rec[f"{p}.scales"], rec[f"{p}.biases"],
                    rec.get(f"{p}.bias"))
        self.gate_up = QuantMatrix([part("gate_proj"), part("up_proj")])
        self.down = QuantMatrix([part("down_proj")])
        self.d_ff = self.gate_up.n_out // 2


def _proj(m: QuantMatrix, x: torch.Tensor) -> torch.Tensor:
    y = _bf16(m.matvec(x))                       # gather_qmm output(s), bf16
    if m.bias is not None:                       # engine_120b.py:136-139
        y = _bf16(y + m.bias)
    return y


def expert_ffn(x: torch.Tensor, e: Expert, kind: str, alpha: float, limit: float):
    gu = _proj(e.gate_up, x)
    gate, up = gu[:e.d_ff], gu[e.d_ff:]
    if kind == "qwen3":                          # silu(g) * u, engine_v3.py:597
        h = _bf16(_bf16(gate * torch.sigmoid(gate)) * up)
    else:                                        # clamped SwiGLU, engine_120b.py:143
        g = torch.clamp(gate, max=limit)
        u = torch.clamp(up, -limit, limit)
        h = _bf16(_bf16(g * torch.sigmoid(alpha * g)) * (u + 1.0))
    return _proj(e.down, h)


def route(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, k: int,
          routing: int, norm: bool):
    """routing 0: softmax over E, top-k, renorm (engine_v3.py:467-473);
    1: top-k of the logits, softmax over the k (engine_120b.py:65-70).
    W fp32 [E, D] holding bf16 values; returns (ids, fp32 scores)."""
    z = W @ x
    if bias is not None:
        z = z + bias
    z = _bf16(z)
    if routing == 0:
        p = _bf16(torch.softmax(z, 0))
        sc, ids = torch.topk(p, k)
        if norm:
            sc = _bf16(sc / _bf16(sc.sum()))
    else:
        zs, ids = torch.topk(z, k)
        sc = _bf16(torch.softmax(zs, 0))
    return ids, sc


def moe_layer(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, experts,
              k: int, routing: int, norm: bool, kind: str, alpha: float = 1.702,
              limit: float = 7.0):
    """One token through one layer: route, then the routed experts' block
    (`experts(e)` -> Expert) and the score-weighted bf16 combine."""
    ids, sc = route(x, W, bias, k, routing, norm)
    y = None
    for j in range(k):
        yj = _bf16(expert_ffn(x, experts(int(ids[j])), kind, alpha, limit) * sc[j])
        y = yj if y is None else y + yj
    return ids, sc, _bf16(y)


def _proj_rows(m: QuantMatrix, X: torch.Tensor) -> torch.Tensor:
    Y = _bf16(m.matmul(X))
    if m.bias is not None:
        Y = _bf16(Y + m.bias)
    return Y


def expert_ffn_rows(X: torch.Tensor, e: Expert, kind: str, alpha: float, limit: float):
    """expert_ffn for the rows X [n, D] routed to one expert."""
    gu = _proj_rows(e.gate_up, X)
    gate, up = gu[:, :e.d_ff], gu[:, e.d_ff:]
    if kind == "qwen3":
        h = _bf16(_bf16(gate * torch.sigmoid(gate)) * up)
    else:
        g = torch.clamp(gate, max=limit)
        u = torch.clamp(up, -limit, limit)
        h = _bf16(_bf16(g * torch.sigmoid(alpha * g)) * (u + 1.0))
    return _proj_rows(e.down, h)


def route_rows(X: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, k: int,
               routing: int, norm: bool):
    """route() for the tokens X [T, D] at once; returns (ids, scores) [T, k]."""
    Z = X @ W.t()
    if bias is not None:
        Z = Z + bias
    Z = _bf16(Z)
    if routing == 0:
        P = _bf16(torch.softmax(Z, 1))
        sc, ids = torch.topk(P, k, dim=1)
        if norm:
            sc = _bf16(sc / _bf16(sc.sum(1, keepdim=True)))
    else:
        zs, ids = torch.topk(Z, k, dim=1)
        sc = _bf16(torch.softmax(zs, 1))
    return ids, sc


def moe_layer_batch(X: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, experts,
                    k: int, routing: int, norm: bool, kind: str, alpha: float = 1.702,
                    limit: float = 7.0):
    """T tokens X [T, D] through one layer: every token routed, each routed
    expert run once over all its rows (`experts(e)` -> Expert), then per
    token the score-weighted bf16 combine in rank order."""
    ids, sc = route_rows(X, W, bias, k, routing, norm)
    T = X.shape[0]
    Y = torch.zeros((T, k, W.shape[1]), dtype=torch.float32)
    for e in torch.unique(ids).tolist():
        t, r = torch.nonzero(ids == e, as_tuple=True)
        Y[t, r] = expert_ffn_rows(X[t], experts(int(e)), kind, alpha, limit)
    P = _bf16(Y * sc.unsqueeze(-1))
    y = P[:, 0]
    for j in range(1, k):
        y = y + P[:, j]
    return ids, sc, _bf16(y)
