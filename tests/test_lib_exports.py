"""The C-ABI library loads and exports every entry point include/*.h
declares; argument checks fail cleanly before any device call."""
import ctypes as C
import re
from pathlib import Path

import pytest

from moe_stream_amd import _lib
from moe_stream_amd import geometry as G

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported():
    lib = _lib.lib()
    declared = _declared()
    assert declared, "no declarations parsed"
    assert declared == set(_lib.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_version_and_component_bytes():
    lib = _lib.lib()
    assert lib.moe_version() >= 1
    b = (C.c_int64 * 12)()
    g = G.QWEN3_30B_A3B
    n = lib.moe_component_bytes(C.byref(g.c_geom()), b)
    assert n == 9
    assert [b[i] for i in range(9)] == [c.nbytes for c in g.components]
    g = G.GPT_OSS_120B
    assert lib.moe_component_bytes(C.byref(g.c_geom()), b) == 12
    assert sum(b[i] for i in range(12)) == g.payload_bytes


def test_argument_errors_are_reported_without_device_work():
    lib = _lib.lib()
    bad = G.QWEN3_30B_A3B.c_geom()
    bad.bits = 8
    b = (C.c_int64 * 12)()
    assert lib.moe_component_bytes(C.byref(bad), b) == _lib.MOE_ERR_UNSUPPORTED
    assert b"4-bit" in lib.moe_last_error()
    g = G.QWEN3_30B_A3B.c_geom()
    rc = lib.moe_ffn_decode(None, C.byref(g), None, None, None, 1, 8, None, None,
                            None, 0, None)
    assert rc == _lib.MOE_ERR_INVALID
    rc = lib.moe_route(None, 0, 2048, None, None, 128, 0, 1, 8, None, None, None,
                       None, 0, None, None, None, None, None, 0, None)
    assert rc == _lib.MOE_ERR_INVALID and b"T=0" in lib.moe_last_error()
    with pytest.raises(_lib.MoeError):
        _lib.check(rc)
    # the streaming engine's layer calls: a NULL engine is refused before any
    # list is read (the depth-list checks follow the engine check)
    depths = (C.c_int32 * 2)(1, 2)
    rc = lib.moe_engine_layer_depths(None, 0, None, None, None, 0, 1, depths, 2, None, None,
                                     None)
    assert rc == _lib.MOE_ERR_INVALID and b"engine is NULL" in lib.moe_last_error()
    rc = lib.moe_engine_layer(None, 0, None, None, None, 0, 1, None, None, None)
    assert rc == _lib.MOE_ERR_INVALID and b"engine is NULL" in lib.moe_last_error()


def test_workspace_sizes():
    lib = _lib.lib()
    g = G.QWEN3_30B_A3B.c_geom()
    assert lib.moe_ffn_decode_workspace(C.byref(g), 1, 8) >= 8 * 768 * 2
    # up to 16 tokens: a sequence word + (flag, logit) 8-byte entries for the
    # router and the lookahead; more tokens: fp32 logits
    assert lib.moe_route_workspace(1, 128) >= 256 + 2 * 128 * 8
    assert lib.moe_route_workspace(16, 128) >= 256 + 2 * 16 * 128 * 8
    assert lib.moe_route_workspace(17, 128) >= 256 + 2 * 17 * 128 * 4
    for T in (1, 5, 16, 17, 512):
        assert lib.moe_route_workspace(T, 128) % 256 == 0
    assert lib.moe_route_workspace(0, 128) == 0


def _qwen3_view(pad=0, swap_store=False):
    """A pool view over made-up (never dereferenced) addresses: 8 packed
    slots per component, plus a repacked store; `pad` bytes added to every
    slot stride; `swap_store` swaps the record offsets of the gate scales
    and biases (same size, so still a legal view)."""
    g = G.QWEN3_30B_A3B
    v = _lib.PoolView()
    v.n_components, v.n_slots = len(g.components), 8
    for i, c in enumerate(g.components):
        # the component arrays back to back in one allocation
        v.base[i] = 0x10_0000_0000 + v.n_slots * c.offset
        v.slot_bytes[i] = c.nbytes + pad
        v.comp_offset[i] = c.offset
    if swap_store:
        v.comp_offset[1], v.comp_offset[2] = v.comp_offset[2], v.comp_offset[1]
    v.store, v.record_bytes, v.n_records = 0x20_0000_0000, g.record_bytes, 16
    return g, v


def _stack_call(lib, g, v):
    return lib.moe_stack_decode(C.byref(v), C.byref(g.c_geom()), 48, 128, 8, None, None,
                                None, 0, 1, 8, None, None, None, None, None, None, None,
                                1, 0, None, 0, None)


def test_persistent_decode_requires_the_packed_pool_layout():
    """The persistent kernel takes strides and record offsets as constants of
    its geometry: a padded slot stride, reordered store components or another
    record size (legal for the per-call kernels) are rejected before any
    device work."""
    lib = _lib.lib()
    g, v = _qwen3_view(pad=256)
    assert _stack_call(lib, g, v) == _lib.MOE_ERR_UNSUPPORTED
    assert b"packed slots" in lib.moe_last_error()
    g, v = _qwen3_view(swap_store=True)
    assert _stack_call(lib, g, v) == _lib.MOE_ERR_UNSUPPORTED
    assert b"repacked records" in lib.moe_last_error()
    g, v = _qwen3_view()
    v.record_bytes += 16384
    assert _stack_call(lib, g, v) == _lib.MOE_ERR_UNSUPPORTED
    assert b"-byte records" in lib.moe_last_error()
    # the packed layout passes this check; the next argument error reports
    g, v = _qwen3_view()
    assert _stack_call(lib, g, v) == _lib.MOE_ERR_INVALID


def _stack_args(lib, g, v, epoch=1, flags=0, n_layers=48):
    """Every argument of moe_stack_decode valid (made-up, never dereferenced
    device addresses) except what a test changes."""
    fake = 0x30_0000_0000
    ws_bytes = lib.moe_stack_workspace(C.byref(g.c_geom()), n_layers, 128, 8)
    return (C.byref(v), C.byref(g.c_geom()), n_layers, 128, 8, fake, fake, None, 0, 1, 8,
            fake, fake, fake, fake, fake, fake, fake, epoch, flags, fake, ws_bytes, None)


def test_persistent_decode_flags_and_epoch_bound():
    """Unknown launch flags are rejected; the epoch must start at 1 and stay
    below the bound that keeps the per-layer flags (epoch * n_layers + l)
    inside 32 bits -- past it the caller zeroes the workspace and restarts."""
    lib = _lib.lib()
    g, v = _qwen3_view()
    assert lib.moe_stack_decode(*_stack_args(lib, g, v, flags=4)) == _lib.MOE_ERR_INVALID
    assert b"unknown flags" in lib.moe_last_error()
    assert lib.moe_stack_decode(*_stack_args(lib, g, v, epoch=0)) == _lib.MOE_ERR_INVALID
    assert b"epoch must start at 1" in lib.moe_last_error()
    last_ok = (2 ** 32 - 1) // 48 - 1          # (epoch + 1) * 48 <= 2^32 - 1
    assert lib.moe_stack_decode(*_stack_args(lib, g, v, epoch=last_ok + 1)) == \
        _lib.MOE_ERR_INVALID
    assert b"too large" in lib.moe_last_error()
    # the DecodeStack restarts well before that bound
    from moe_stream_amd.stack import DecodeStack
    for L in (1, 48, 4096, 2 ** 20):
        lim = DecodeStack.epoch_limit(L)
        assert lim >= 1 and (lim + 1) * L <= 2 ** 32 - 1


def test_fill_slots_range_checks_records_and_slots():
    """Record indices are checked against the source store's record count
    and slots against the pool on the host, before anything is enqueued."""
    lib = _lib.lib()
    g, v = _qwen3_view()
    recs = (C.c_int64 * 2)(0, 16)          # the view's store holds 16 records
    slots = (C.c_int32 * 2)(0, 1)
    assert lib.moe_fill_slots(C.byref(v), None, 0, 0, recs, slots, 2, None) == \
        _lib.MOE_ERR_INVALID
    assert b"record 16 outside [0, 16)" in lib.moe_last_error()
    src = 0x40_0000_0000
    rb = g.record_bytes
    assert lib.moe_fill_slots(C.byref(v), src, rb, 10, recs, slots, 2, None) == \
        _lib.MOE_ERR_INVALID
    assert b"record 16 outside [0, 10)" in lib.moe_last_error()
    recs[1] = -1
    assert lib.moe_fill_slots(C.byref(v), src, rb, 10, recs, slots, 2, None) == \
        _lib.MOE_ERR_INVALID
    recs[1] = 3
    slots[1] = 8                            # 8 slots in the view
    assert lib.moe_fill_slots(C.byref(v), src, rb, 10, recs, slots, 2, None) == \
        _lib.MOE_ERR_INVALID
    assert b"slot 8 outside [0, 8)" in lib.moe_last_error()
    assert lib.moe_fill_slots(C.byref(v), src, rb, 0, recs, slots, 2, None) == \
        _lib.MOE_ERR_INVALID


def test_static_scratch_decode_rejects_oversized_calls_first():
    """The no-allocation decode checks the activation size against its fixed
    scratch before any device call."""
    lib = _lib.lib()
    assert lib.moe_ffn_decode_static_bytes() == 2 << 20
    g = G.QWEN3_30B_A3B.c_geom()
    T = (2 << 20) // (8 * 768 * 2) + 1
    rc = lib.moe_ffn_decode_static(None, C.byref(g), None, None, None, T, 8, None, None, None)
    assert rc == _lib.MOE_ERR_INVALID and b"static scratch" in lib.moe_last_error()
