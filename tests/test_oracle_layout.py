"""Record layout of the repacked expert store, pinned by the reference's own
constants, and the product geometry checked against the oracle layout."""
import numpy as np

from moe_stream_amd import geometry as G
from oracle import layout as OL


def test_qwen3_word_offsets_match_kernels_py():
    # kernels.py:58-63 LAYOUT_U32 (uint32 word offsets inside a blob)
    layout = {n: off // 4 for n, _, _, off, _ in OL.components(2048, 768, False)}
    assert layout == {
        "gate_proj.weight": 0, "gate_proj.scales": 196608, "gate_proj.biases": 208896,
        "up_proj.weight": 221184, "up_proj.scales": 417792, "up_proj.biases": 430080,
        "down_proj.weight": 442368, "down_proj.scales": 638976, "down_proj.biases": 651264,
    }
    assert OL.record_bytes(2048, 768, False) == 663552 * 4


def test_qwen3_record_is_2654208_bytes_162_pages():
    # ext/test_pread.py:34 EXPERT_BYTES; repack.py:86-90 (no padding)
    assert OL.record_bytes(2048, 768, False) == 2654208 == 162 * 16384


def test_gptoss_segments_match_stage_bench():
    # scratchpad/stage_bench.py:11-12: [4147200, 259200, 259200, 5760] x 3 + [10624]
    comps = OL.components(2880, 2880, True)
    assert [nb for *_, nb in comps] == [4147200, 259200, 259200, 5760] * 3
    assert OL.record_bytes(2880, 2880, True) == 14024704
    payload = comps[-1][3] + comps[-1][4]
    assert OL.record_bytes(2880, 2880, True) - payload == 10624


def test_product_geometry_matches_oracle_layout():
    for g in (G.QWEN3_30B_A3B, G.GPT_OSS_120B, G.SMALL):
        ref = OL.components(g.d_model, g.d_ff, g.has_proj_bias)
        assert len(ref) == g.n_components
        for (n, dt, shape, off, nb), c in zip(ref, g.components):
            assert (n, tuple(shape), off, nb) == (c.name, tuple(c.shape), c.offset, c.nbytes)
        assert g.record_bytes == OL.record_bytes(g.d_model, g.d_ff, g.has_proj_bias)


def test_record_offset_formula():
    # repack.py:141: (layer * n_experts + expert) * blob_bytes
    g = G.QWEN3_30B_A3B
    assert g.record_offset(3, 5) == (3 * 128 + 5) * 2654208


def test_split_record_roundtrip():
    rng = np.random.default_rng(0)
    rec = rng.integers(0, 256, OL.record_bytes(256, 128, True), dtype=np.uint8)
    parts = OL.split_record(rec, 256, 128, True)
    flat = b"".join(parts[n].tobytes() for n, *_ in OL.components(256, 128, True))
    assert flat == rec[:len(flat)].tobytes()
