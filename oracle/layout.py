"""Restatement of the repacked expert-record layout, for checking.

TEST INFRASTRUCTURE ONLY.

repack.py:35-37,73-82 (Qwen3) and repack_gptoss.py:54-55,139-159 (gpt-oss):
components proj-major over (gate_proj, up_proj, down_proj), part-major over
(weight, scales, biases[, bias]), back to back; the record padded to a whole
number of 16 KiB pages (repack_gptoss.py:159).

Parity status: pinned by the reference's own constants -- kernels.py:58-63
(Qwen3 word offsets), ext/test_pread.py:34 (2,654,208-byte Qwen3 record) and
scratchpad/stage_bench.py:11-12 (gpt-oss segment sizes and 14,024,704-byte
record) -- in tests/test_oracle_layout.py.
"""
from __future__ import annotations

import numpy as np

PAGE = 16384


def components(d_model: int, d_ff: int, proj_bias: bool, group: int = 64):
    """[(name, dtype, shape, offset, nbytes)] in record order."""
    out, off = [], 0
    parts = ["weight", "scales", "biases"] + (["bias"] if proj_bias else [])
    for proj in ("gate_proj", "up_proj", "down_proj"):
        n_out, n_in = (d_model, d_ff) if proj == "down_proj" else (d_ff, d_model)
        for part in parts:
            if part == "weight":
                dt, shape = np.uint32, (n_out, n_in // 8)
            elif part == "bias":
                dt, shape = np.uint16, (n_out,)
            else:
                dt, shape = np.uint16, (n_out, n_in // group)
            nb = int(np.prod(shape)) * np.dtype(dt).itemsize
            out.append((f"{proj}.{part}", dt, shape, off, nb))
            off += nb
    return out


def record_bytes(d_model: int, d_ff: int, proj_bias: bool) -> int:
    c = components(d_model, d_ff, proj_bias)
    payload = c[-1][3] + c[-1][4]
    return -(-payload // PAGE) * PAGE


def split_record(rec: np.ndarray, d_model: int, d_ff: int, proj_bias: bool) -> dict:
    """uint8 record bytes -> {component name: array} (bf16 parts as uint16
    bit patterns)."""
    rec = np.ascontiguousarray(rec, dtype=np.uint8)
    out = {}
    for name, dt, shape, off, nb in components(d_model, d_ff, proj_bias):
        out[name] = rec[off:off + nb].view(dt).reshape(shape)
    return out
