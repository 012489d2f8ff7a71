"""The on-disk expert store format (experts.bin + experts_index.json):
round trips, the reference's layout constants, the engine's load-time
checks, and the repack of local safetensors shards."""
import json
import os
import struct

import numpy as np
import pytest

from moe_stream_amd import geometry as G
from moe_stream_amd import store as S

# kernels.py:58-63: word offsets of the Qwen3 blob components and the blob size
LAYOUT_U32 = {"gate_proj.weight": 0, "gate_proj.scales": 196608, "gate_proj.biases": 208896,
              "up_proj.weight": 221184, "up_proj.scales": 417792, "up_proj.biases": 430080,
              "down_proj.weight": 442368, "down_proj.scales": 638976,
              "down_proj.biases": 651264}
BLOB_U32 = 663552


def test_qwen3_index_matches_reference_layout():
    idx = S.index_for(G.QWEN3_30B_A3B)
    for c in idx.components:
        assert c["offset"] == 4 * LAYOUT_U32[f"{c['proj']}.{c['part']}"]
    assert idx.blob_bytes == 4 * BLOB_U32 == 2654208   # ext/test_pread.py:34
    assert idx.blob_bytes % idx.page_size == 0           # 162 pages, no padding


def test_gptoss_index_segments_and_padding():
    # segments [4147200, 259200, 259200, 5760] x 3 + 10624 pad
    # (scratchpad/stage_bench.py:12, repack_gptoss.py:159)
    idx = S.index_for(G.GPT_OSS_120B)
    assert [c["nbytes"] for c in idx.components] == [4147200, 259200, 259200, 5760] * 3
    assert idx.blob_bytes - idx.payload_bytes == 10624
    assert idx.blob_bytes == 14024704


def _small_records(geom, seed=0):
    rng = np.random.default_rng(seed)
    n = geom.n_layers * geom.n_experts
    recs = rng.integers(0, 256, (n, geom.record_bytes), dtype=np.uint8)
    recs[:, geom.payload_bytes:] = 0
    return recs


def test_write_read_round_trip(tmp_path):
    geom = G.SMALL
    recs = _small_records(geom)
    S.write_store(str(tmp_path), geom, recs, model="synthetic")
    d = json.load(open(tmp_path / S.INDEX))
    for key in ("n_layers", "n_experts", "blob_bytes", "page_size", "offset_formula",
                "quantization", "components"):
        assert key in d
    f = S.ExpertStoreFile(str(tmp_path), base=G.SMALL)
    assert f.geom.d_model == 256 and f.geom.d_ff == 128 and not f.geom.has_proj_bias
    assert f.geom.record_bytes == geom.record_bytes
    for layer, e in [(0, 0), (1, 5), (3, 15)]:
        np.testing.assert_array_equal(f.record(layer, e), recs[layer * 16 + e])
    # offset formula: record (l, e) at (l * E + e) * blob_bytes
    raw = open(tmp_path / S.BLOB, "rb").read()
    off = (2 * 16 + 7) * geom.record_bytes
    assert raw[off:off + 64] == recs[2 * 16 + 7][:64].tobytes()


def test_index_validation_catches_holes_and_sizes(tmp_path):
    d = S.index_for(G.SMALL).to_dict()
    bad = json.loads(json.dumps(d))
    bad["components"][1]["offset"] += 16
    with pytest.raises(S.StoreFormatError, match="hole"):
        S.StoreIndex.from_dict(bad)
    bad = json.loads(json.dumps(d))
    bad["components"][0]["nbytes"] += 4
    with pytest.raises(S.StoreFormatError):
        S.StoreIndex.from_dict(bad)
    bad = json.loads(json.dumps(d))
    bad["blob_bytes"] = 1024
    with pytest.raises(S.StoreFormatError, match="overrun"):
        S.StoreIndex.from_dict(bad)
    # a truncated experts.bin is refused at open
    S.write_store(str(tmp_path), G.SMALL, _small_records(G.SMALL))
    with open(tmp_path / S.BLOB, "r+b") as fh:
        fh.truncate(G.SMALL.record_bytes * 10)
    with pytest.raises(S.StoreFormatError, match="bytes"):
        S.ExpertStoreFile(str(tmp_path))


def _write_safetensors(path, tensors):
    """Minimal safetensors writer: {name: (dtype, shape, bytes)}."""
    hdr, off, blobs = {}, 0, []
    for name, (dt, shape, b) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(hdr).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


@pytest.mark.parametrize("bias", [False, True])
def test_repack_safetensors_round_trip(tmp_path, bias):
    geom = G.SMALL.with_(n_layers=2, has_proj_bias=bias)
    rng = np.random.default_rng(7)
    src = tmp_path / "src"
    src.mkdir()
    stacks = {}
    prefix = "experts" if bias else "switch_mlp"
    for layer in range(geom.n_layers):
        tens = {}
        for c in geom.components:
            proj, part = c.name.split(".")
            b = rng.integers(0, 256, geom.n_experts * c.nbytes, dtype=np.uint8).tobytes()
            stacks[(layer, c.name)] = b
            tens[f"model.layers.{layer}.mlp.{prefix}.{proj}.{part}"] = (
                c.dtype, (geom.n_experts, *c.shape), b)
        _write_safetensors(src / f"model-{layer:05d}.safetensors", tens)   # one shard per layer
    out = tmp_path / "store"
    S.repack_safetensors(str(src), str(out), geom)
    f = S.ExpertStoreFile(str(out), base=geom)
    for layer in range(geom.n_layers):
        for e in (0, 3, geom.n_experts - 1):
            rec = f.record(layer, e)
            for c in geom.components:
                want = stacks[(layer, c.name)][e * c.nbytes:(e + 1) * c.nbytes]
                assert rec[c.offset:c.offset + c.nbytes].tobytes() == want
            assert not rec[geom.payload_bytes:].any()   # page padding is zero


def test_repack_rejects_wrong_shapes(tmp_path):
    geom = G.SMALL.with_(n_layers=1)
    src = tmp_path / "src"
    src.mkdir()
    tens = {}
    for c in geom.components:
        proj, part = c.name.split(".")
        shape = (geom.n_experts, *c.shape)
        if c.name == "up_proj.scales":
            shape = (geom.n_experts, c.shape[0], c.shape[1] + 1)
        n = int(np.prod(shape)) * c.elem_bytes
        tens[f"model.layers.0.mlp.switch_mlp.{proj}.{part}"] = (c.dtype, shape, bytes(n))
    _write_safetensors(src / "m.safetensors", tens)
    with pytest.raises(S.StoreFormatError, match="up_proj.scales"):
        S.repack_safetensors(str(src), str(tmp_path / "out"), geom)


def test_read_into_matches_the_records(tmp_path):
    """The pinned-store load of ExpertPool(model_dir, n_slots, n_workers):
    chunked preadv straight into the destination, on several workers, with a
    last chunk shorter than the others."""
    geom = G.SMALL
    recs = _small_records(geom, seed=3)
    S.write_store(str(tmp_path), geom, recs)
    f = S.ExpertStoreFile(str(tmp_path), base=G.SMALL)
    for workers, chunk in ((1, 64), (3, 7), (8, 1)):
        dst = np.zeros_like(recs)
        f.read_into(dst, chunk_records=chunk, n_workers=workers)
        np.testing.assert_array_equal(dst, recs)
    with pytest.raises(ValueError):
        f.read_into(np.zeros((3, geom.record_bytes), dtype=np.uint8))
