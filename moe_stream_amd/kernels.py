"""The fused-expert-kernel entry of the reference, `kernels.moe_expert_mlp`
(kernels.py:186-252), and its blob-layout helpers, on the gfx950 decode
kernels.

The reference's fused kernel reads the slot pool as ONE flat uint32 buffer
(each slot one repacked expert record, `blob` words long) and finds every
component of a slot at a constant word offset inside the record
(`LAYOUT_U32`, kernels.py:58-63; `layout_from_index`, kernels.py:255-261).
Here the same flat buffer and offsets become a pool view of the C ABI (one
base pointer per component, the record as the slot stride) and the call runs
`moe_ffn_decode` for one token over the given slots: gate/up, SwiGLU, down
and the score-weighted sum in fp32, result fp32 [d_model] as the
reference's `out` (kernels.py:234-241).  Unlike the Metal kernel's
`atomic_add` the combine runs in a fixed expert order, so the result is
deterministic.

`nsg` and `pad` were launch-shape knobs of the Metal kernel (simdgroups per
threadgroup, threadgroup padding); they are accepted and validated for call
compatibility and do not change the gfx950 launch, whose shape is fixed per
geometry.
"""
from __future__ import annotations

import ctypes as C
import json

import torch

from . import _lib
from . import geometry as G

_PARTS = {"weight": "w", "scales": "s", "biases": "b", "bias": "bias"}


def _layout_of(geom: G.Geometry) -> dict:
    """Word offsets of the components of a record of `geom`, keyed as the
    reference's LAYOUT_U32 ({proj}_{w|s|b}, plus `blob`)."""
    off = {}
    for c in geom.components:
        proj, part = c.name.split(".")
        key = proj.replace("_proj", "") + "_" + _PARTS[part]
        off[key] = c.offset // 4
    off["blob"] = geom.record_bytes // 4
    return off


# The Qwen3-30B-A3B record (kernels.py:58-63): gate_w 0, gate_s 196608,
# gate_b 208896, up_w 221184, up_s 417792, up_b 430080, down_w 442368,
# down_s 638976, down_b 651264, blob 663552 words.
LAYOUT_U32 = _layout_of(G.QWEN3_30B_A3B)


def layout_from_index(path) -> dict:
    """The blob layout in uint32 words from a repacked store's
    experts_index.json (kernels.py:255-261): one entry per component, keyed
    `{proj without _proj}_{first letter of part}`, plus `blob`."""
    with open(path) as f:
        idx = json.load(f)
    off = {c["proj"].replace("_proj", "") + "_" + c["part"][0]: c["offset"] // 4
           for c in idx["components"]}
    off["blob"] = idx["blob_bytes"] // 4
    return off


_CACHE = {}


def build(d_model=2048, d_ff=768, group_size=64, nsg=32, pad=False, layout=LAYOUT_U32):
    """Check one geometry against the compiled kernels and cache its call
    arguments (the reference compiles a Metal kernel per geometry,
    kernels.py:188-228).  ValueError when the dims are not multiples of 4
    quant groups (kernels.py:197-198), when the layout lacks a component or
    misplaces one.  (A geometry with no compiled gfx950 kernel raises
    ValueError at the first call.)"""
    key = (d_model, d_ff, group_size, nsg, bool(pad), tuple(sorted(layout.items())))
    if key in _CACHE:
        return _CACHE[key]
    if d_model % (group_size * 4) or d_ff % (group_size * 4):
        raise ValueError("dims must be a multiple of 4 quant groups")
    if nsg <= 0:
        raise ValueError(f"nsg={nsg} must be positive")
    geom = G.QWEN3_30B_A3B.with_(d_model=d_model, d_ff=d_ff, group_size=group_size)
    names = ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b",
             "down_w", "down_s", "down_b")
    missing = [n for n in names + ("blob",) if n not in layout]
    if missing:
        raise ValueError(f"layout lacks {missing}")
    blob = int(layout["blob"])
    for n, c in zip(names, geom.components):
        w0 = int(layout[n])
        if w0 < 0 or (w0 * 4) % (16 if n.endswith("_w") else 2) or w0 * 4 + c.nbytes > blob * 4:
            raise ValueError(f"layout[{n!r}] = {w0} words: misaligned or outside the "
                             f"{blob}-word blob")
    _CACHE[key] = (geom, [int(layout[n]) for n in names], blob)
    return _CACHE[key]


def moe_expert_mlp(pool_u32, slots, x, scores, d_model=2048, d_ff=768, group_size=64,
                   nsg=32, pad=False, layout=LAYOUT_U32, verbose=False):
    """One launch pair for a whole MoE layer at batch 1 (kernels.py:231-252).

    pool_u32 : uint32 (or int32) device tensor, the flat slot pool: slot s is
               words [s * blob, (s + 1) * blob)
    slots    : integer tensor [E], slot of each active expert
    x        : bfloat16 [d_model]
    scores   : float32 [E], router weights, already normalised
    returns  : float32 [d_model]"""
    geom, offs, blob = build(d_model, d_ff, group_size, nsg, pad, layout)
    if pool_u32.dtype not in (torch.uint32, torch.int32) or not pool_u32.is_cuda:
        raise TypeError("pool_u32: a uint32 device tensor")
    if not pool_u32.is_contiguous():
        raise ValueError("pool_u32: must be contiguous")
    n_slots = pool_u32.numel() // blob
    if n_slots <= 0:
        raise ValueError(f"pool of {pool_u32.numel()} words holds no {blob}-word slot")
    dev = pool_u32.device
    if not torch.is_tensor(slots):
        slots = torch.as_tensor(slots)
    if not torch.is_tensor(scores):
        scores = torch.as_tensor(scores)
    if slots.dtype == torch.uint32:
        slots = slots.view(torch.int32)   # slot indices < 2^31: same bits
    x = x.reshape(-1)
    if x.dtype != torch.bfloat16 or x.numel() != d_model:
        raise ValueError(f"x: bfloat16 [{d_model}]")
    s = slots.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
    E = s.numel()
    sc = scores.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    if sc.numel() != E:
        raise ValueError(f"scores has {sc.numel()} entries, slots {E}")
    if E == 0:
        return torch.zeros(d_model, dtype=torch.float32, device=dev)
    # the active experts are bounds-checked on the host as well as in the
    # kernels (which skip an out-of-range slot and flag the device error)
    if int(s.min()) < 0 or int(s.max()) >= n_slots:
        raise ValueError(f"slot outside [0, {n_slots})")
    v = _lib.PoolView()
    v.n_components = geom.n_components
    v.n_slots = n_slots
    base = pool_u32.data_ptr()
    for i, w0 in enumerate(offs):
        v.base[i] = base + 4 * w0
        v.slot_bytes[i] = 4 * blob
        v.comp_offset[i] = 4 * w0
    v.store, v.record_bytes, v.n_records = None, 0, 0
    g = geom.c_geom()
    xc = x.to(dev).contiguous()
    out = torch.zeros(d_model, dtype=torch.float32, device=dev)
    L = _lib.lib()
    # the decode kernels take up to MOE_MAX_TOPK experts per token: more
    # active experts run as chunks whose fp32 results are summed in order
    step = _lib.MAX_TOPK
    part = torch.empty_like(out) if E > step else out
    for c0 in range(0, E, step):
        n = min(step, E - c0)
        need = L.moe_ffn_decode_workspace(C.byref(g), 1, n)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        rc = L.moe_ffn_decode(
            C.byref(v), C.byref(g), s[c0:c0 + n].data_ptr(), sc[c0:c0 + n].data_ptr(),
            xc.data_ptr(), 1, n, None, part.data_ptr(), ws.data_ptr(), ws.numel(),
            _lib.stream_ptr(None))
        if rc == _lib.MOE_ERR_UNSUPPORTED:
            raise ValueError(f"no gfx950 kernel for d_model={d_model} d_ff={d_ff}: "
                             + L.moe_last_error().decode(errors="replace"))
        _lib.check(rc)
        if part is not out:
            out += part
    if verbose:
        print(f"moe_expert_mlp: d_model={d_model} d_ff={d_ff} E={E} slots={n_slots}")
    return out
