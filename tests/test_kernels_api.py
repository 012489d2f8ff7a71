"""The reference's fused-kernel module interface (kernels.py:58-63,186-261)
on the host: the blob layout constants, `layout_from_index` over a written
store index, and the geometry checks of `build`; the PF_DEPTH / PF_WIDEN
environment defaults (engine_v3.py:61,84).  No device calls."""
import json
import os

import pytest

from moe_stream_amd import geometry as G
from moe_stream_amd import kernels as K
from moe_stream_amd import pool as P
from moe_stream_amd import store as S

# kernels.py:58-63, the reference's own constants
REF_LAYOUT_U32 = dict(blob=663552, gate_w=0, gate_s=196608, gate_b=208896,
                      up_w=221184, up_s=417792, up_b=430080,
                      down_w=442368, down_s=638976, down_b=651264)


def test_layout_u32_is_the_reference_constant():
    assert K.LAYOUT_U32 == REF_LAYOUT_U32


def test_layout_from_index_of_a_written_store(tmp_path):
    idx = S.index_for(G.QWEN3_30B_A3B)
    p = tmp_path / S.INDEX
    p.write_text(json.dumps(idx.to_dict()))
    assert K.layout_from_index(str(p)) == REF_LAYOUT_U32


def test_layout_from_index_of_a_tiny_store(tmp_path):
    # a geometry written end to end with write_store: the index it leaves
    # gives the component word offsets of that geometry's record
    geom = G.SMALL.with_(n_layers=1, n_experts=2)
    import numpy as np
    recs = np.zeros((2, geom.record_bytes), dtype=np.uint8)
    S.write_store(str(tmp_path), geom, recs)
    lay = K.layout_from_index(os.path.join(str(tmp_path), S.INDEX))
    assert lay["blob"] * 4 == geom.record_bytes
    for c in geom.components:
        proj, part = c.name.split(".")
        assert lay[proj.replace("_proj", "") + "_" + part[0]] * 4 == c.offset


@pytest.mark.parametrize("dm,dff", [(2048, 700), (2000, 768), (2880, 2880 + 64)])
def test_build_rejects_dims_not_multiple_of_four_groups(dm, dff):
    with pytest.raises(ValueError, match="multiple of 4 quant groups"):
        K.build(dm, dff)


def test_build_checks_the_layout():
    lay = dict(REF_LAYOUT_U32)
    del lay["down_s"]
    with pytest.raises(ValueError, match="lacks"):
        K.build(layout=lay)
    lay = dict(REF_LAYOUT_U32, up_w=221185)           # not 16-byte aligned
    with pytest.raises(ValueError, match="misaligned"):
        K.build(layout=lay)
    lay = dict(REF_LAYOUT_U32, blob=663552 - 1)       # down_b runs past the blob
    with pytest.raises(ValueError, match="outside"):
        K.build(layout=lay)
    geom, offs, blob = K.build()
    assert blob == 663552 and offs[0] == 0 and offs[-1] == 651264


def test_env_depths_and_widen(monkeypatch):
    monkeypatch.delenv("PF_DEPTH", raising=False)
    monkeypatch.delenv("PF_WIDEN", raising=False)
    assert P.env_depths() == (1,) and P.env_widen() == 1
    monkeypatch.setenv("PF_DEPTH", "2,1,3")
    monkeypatch.setenv("PF_WIDEN", "2")
    assert P.env_depths() == (2, 1, 3) and P.env_widen() == 2
    monkeypatch.setenv("PF_DEPTH", "1,x")
    with pytest.raises(ValueError):
        P.env_depths()
    monkeypatch.setenv("PF_DEPTH", "0")
    with pytest.raises(ValueError):
        P.env_depths()
    monkeypatch.setenv("PF_WIDEN", "0")
    with pytest.raises(ValueError):
        P.env_widen()


def test_moe_block_takes_env_defaults(monkeypatch):
    from moe_stream_amd.block import MoEBlock
    monkeypatch.setenv("PF_DEPTH", "1,2")
    monkeypatch.setenv("PF_WIDEN", "3")
    b = MoEBlock(0, G.QWEN3_30B_A3B, None, None, None, [])
    assert b.depths == (1, 2) and b.widen == 3
    b = MoEBlock(0, G.QWEN3_30B_A3B, None, None, None, [], depths=(2,), widen=1)
    assert b.depths == (2,) and b.widen == 1
