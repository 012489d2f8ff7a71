"""Operator-level entry points over the C ABI, on torch device tensors.

These are the calls the MoE blocks make; each validates shapes/dtypes on the
host, then launches on the current stream (or `stream`).
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .geometry import Geometry


def _p(t):
    return None if t is None else t.data_ptr()


def _req(t, dtype, name, numel=None, device=None):
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise TypeError(f"{name}: must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: expected {numel} elements, got {t.numel()}")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: on {t.device}, expected {device}")


class Workspace:
    """Grow-only device scratch buffers, one per purpose and device."""

    def __init__(self):
        self._bufs = {}

    def get(self, key, nbytes: int, device, zero: bool = False) -> torch.Tensor:
        k = (key, str(device))
        b = self._bufs.get(k)
        if b is None or b.numel() < nbytes:
            b = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            self._bufs[k] = b
        return b


_WS = Workspace()


def ffn_decode(pool, slot_refs: torch.Tensor, scores: torch.Tensor,
               x: torch.Tensor, out: torch.Tensor | None = None,
               out_f32: torch.Tensor | None = None, stream=None,
               workspace: torch.Tensor | None = None):
    """Fused expert block for T tokens x k routed experts.

    x bf16 [T, D]; slot_refs int32 [T, k]; scores fp32 [T, k].  Returns bf16
    [T, D] (and fills out_f32 when given)."""
    return _ffn("moe_ffn_decode", "moe_ffn_decode_workspace", "ffn", pool, slot_refs,
                scores, x, out, out_f32, stream, workspace)


def ffn_decode_up(pool, slot_refs: torch.Tensor, x: torch.Tensor,
                  workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """First half of ffn_decode: the gate/up projections and activation of
    every (token, expert) pair into the workspace, which is returned for
    ffn_decode_down (pass the same tensor; it is not shared with ffn_decode's
    cached workspace)."""
    geom: Geometry = pool.geom
    x = x.view(1, -1) if x.dim() == 1 else x
    T, D = x.shape
    if D != geom.d_model:
        raise ValueError(f"x has {D} features, geometry {geom.d_model}")
    k = slot_refs.numel() // T
    _req(x, torch.bfloat16, "x", device=pool.device)
    _req(slot_refs, torch.int32, "slot_refs", T * k, pool.device)
    g = geom.c_geom()
    L = _lib.lib()
    need = L.moe_ffn_decode_workspace(C.byref(g), T, k)
    if need == 0:
        raise ValueError(f"moe_ffn_decode_up: unsupported T={T}, k={k}")
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    _lib.check(L.moe_ffn_decode_up(
        C.byref(pool.c_view()), C.byref(g), _p(slot_refs), _p(x), T, k,
        _p(workspace), workspace.numel(), _lib.stream_ptr(stream)))
    return workspace


def ffn_decode_down(pool, slot_refs: torch.Tensor, scores: torch.Tensor,
                    workspace: torch.Tensor, out: torch.Tensor | None = None,
                    out_f32: torch.Tensor | None = None, stream=None):
    """Second half of ffn_decode: the down projections of the activations
    ffn_decode_up left in `workspace`, weighted by scores and summed per
    token.  slot_refs int32 [T, k] and scores fp32 [T, k] as for ffn_decode."""
    geom: Geometry = pool.geom
    T, k = slot_refs.shape
    D = geom.d_model
    _req(slot_refs, torch.int32, "slot_refs", T * k, pool.device)
    _req(scores, torch.float32, "scores", T * k, pool.device)
    _req(workspace, torch.uint8, "workspace", device=pool.device)
    if out is None and out_f32 is None:
        out = torch.empty((T, D), dtype=torch.bfloat16, device=slot_refs.device)
    if out is not None:
        _req(out, torch.bfloat16, "out", T * D, pool.device)
    if out_f32 is not None:
        _req(out_f32, torch.float32, "out_f32", T * D, pool.device)
    g = geom.c_geom()
    _lib.check(_lib.lib().moe_ffn_decode_down(
        C.byref(pool.c_view()), C.byref(g), _p(slot_refs), _p(scores), T, k,
        _p(out), _p(out_f32), _p(workspace), workspace.numel(),
        _lib.stream_ptr(stream)))
    return out if out is not None else out_f32


def slot_lookup(table: torch.Tensor, ids: torch.Tensor,
                miss: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """slot_refs = table[ids] on device (engine_v3.py:550-552).  table int32
    [E]; ids int32 of any shape.  miss (int32 [1], optional) is incremented
    by the number of refs < 0; an id outside [0, E) gives ref 0 and raises
    the device error flag that check_device_error reports."""
    _req(table, torch.int32, "table")
    _req(ids, torch.int32, "ids", device=table.device)
    if miss is not None:
        _req(miss, torch.int32, "miss", 1, table.device)
    refs = torch.empty_like(ids)
    _lib.check(_lib.lib().moe_slot_lookup(
        _p(table), table.numel(), _p(ids), ids.numel(), _p(refs), _p(miss),
        _lib.stream_ptr(stream)))
    return refs


def ffn_grouped(pool, slot_refs: torch.Tensor, scores: torch.Tensor,
                x: torch.Tensor, out: torch.Tensor | None = None,
                out_f32: torch.Tensor | None = None, stream=None,
                workspace: torch.Tensor | None = None):
    """The expert block for many tokens (prefill): pairs grouped per slot,
    bf16 MFMA per group.  Same arguments and result as ffn_decode."""
    return _ffn("moe_ffn_grouped", "moe_ffn_grouped_workspace", "ffn_grouped", pool,
                slot_refs, scores, x, out, out_f32, stream, workspace)


# Above this many tokens per call the grouped MFMA path runs; at or below it,
# the decode kernels (which group the pairs by slot from 2 tokens on and give
# results bit-identical to one call per token).  Per step of the 48-layer
# Qwen3 stack on one MI355X (HIP graph of router + expert block per layer):
# 4 tokens 2.03 ms (decode kernels) vs 2.02 ms (MFMA block), 8 tokens 2.81
# vs 2.37 ms, 16 tokens 4.35 vs 2.74 ms.
GROUPED_MIN_TOKENS = 4


def ffn(pool, slot_refs, scores, x, out=None, out_f32=None, stream=None):
    """The expert block, choosing the decode or the grouped path by T (the
    decode/prefill split of engine_v3.py:555-600)."""
    T = 1 if x.dim() == 1 else x.shape[0]
    f = ffn_grouped if T > GROUPED_MIN_TOKENS else ffn_decode
    return f(pool, slot_refs, scores, x, out, out_f32, stream)


def _ffn(entry, ws_entry, ws_key, pool, slot_refs, scores, x, out, out_f32, stream,
         workspace):
    geom: Geometry = pool.geom
    if x.dim() == 1:
        x = x.view(1, -1)
    T, D = x.shape
    if D != geom.d_model:
        raise ValueError(f"x has {D} features, geometry {geom.d_model}")
    k = slot_refs.numel() // T
    _req(x, torch.bfloat16, "x", device=pool.device)
    _req(slot_refs, torch.int32, "slot_refs", T * k, pool.device)
    _req(scores, torch.float32, "scores", T * k, pool.device)
    if out is None and out_f32 is None:
        out = torch.empty((T, D), dtype=torch.bfloat16, device=x.device)
    if out is not None:
        _req(out, torch.bfloat16, "out", T * D, pool.device)
    if out_f32 is not None:
        _req(out_f32, torch.float32, "out_f32", T * D, pool.device)
    g = geom.c_geom()
    L = _lib.lib()
    need = getattr(L, ws_entry)(C.byref(g), T, k)
    if need == 0:
        raise ValueError(f"{entry}: unsupported T={T}, k={k}")
    ws = workspace if workspace is not None else _WS.get(ws_key, need, x.device)
    _lib.check(getattr(L, entry)(
        C.byref(pool.c_view()), C.byref(g), _p(slot_refs), _p(scores), _p(x),
        T, k, _p(out), _p(out_f32), _p(ws), ws.numel(), _lib.stream_ptr(stream)))
    return out if out is not None else out_f32


class RouteBuffers:
    """Device outputs of one routing call for T tokens."""

    def __init__(self, T: int, k: int, k_pred: int, device):
        self.ids = torch.zeros((T, k), dtype=torch.int32, device=device)
        self.scores = torch.zeros((T, k), dtype=torch.float32, device=device)
        self.pred = torch.zeros((T, max(k_pred, 1)), dtype=torch.int32, device=device)
        self.slot_refs = torch.zeros((T, k), dtype=torch.int32, device=device)
        self.miss = torch.zeros((1,), dtype=torch.int32, device=device)


def route(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, mode: int,
          renorm: bool, k: int, W_next: torch.Tensor | None = None,
          bias_next: torch.Tensor | None = None, k_pred: int = 0,
          table: torch.Tensor | None = None, bufs: RouteBuffers | None = None,
          stream=None, workspace: torch.Tensor | None = None) -> RouteBuffers:
    """Router + top-k (+ lookahead + slot lookup) on device.

    x bf16 [T, D]; W bf16 [E, D]; bias bf16 [E] or None; table int32 [E]
    (slot refs of this layer) or None."""
    if x.dim() == 1:
        x = x.view(1, -1)
    T, D = x.shape
    E = W.shape[0]
    dev = x.device
    _req(x, torch.bfloat16, "x")
    _req(W, torch.bfloat16, "W", E * D, dev)
    if bias is not None:
        _req(bias, torch.bfloat16, "bias", E, dev)
    if W_next is not None:
        _req(W_next, torch.bfloat16, "W_next", E * D, dev)
        if bias_next is not None:
            _req(bias_next, torch.bfloat16, "bias_next", E, dev)
    if table is not None:
        _req(table, torch.int32, "table", E, dev)
    if bufs is None:
        bufs = RouteBuffers(T, k, k_pred, dev)
    L = _lib.lib()
    need = L.moe_route_workspace(T, E)
    ws = workspace if workspace is not None else _WS.get("route", need, dev, zero=True)
    _lib.check(L.moe_route(
        _p(x), T, D, _p(W), _p(bias), E, mode, int(renorm), k,
        _p(bufs.ids), _p(bufs.scores),
        _p(W_next), _p(bias_next), k_pred if W_next is not None else 0,
        _p(bufs.pred) if W_next is not None else None,
        _p(table), _p(bufs.slot_refs) if table is not None else None,
        _p(bufs.miss), _p(ws), ws.numel(), _lib.stream_ptr(stream)))
    return bufs


def check_device_error(stream=None):
    _lib.check(_lib.lib().moe_check_device_error(_lib.stream_ptr(stream)))
