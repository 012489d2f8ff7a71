"""The on-disk expert store: `experts.bin` + `experts_index.json`.

Format (repack.py:61-146, repack_gptoss.py:139-168, read by
engine_v3.py:129-175 and engine_120b.py:172-176):

* `experts.bin` -- one record of `blob_bytes` per (layer, expert), at byte
  offset (layer * n_experts + expert) * blob_bytes;
* `experts_index.json` -- {"model", "n_layers", "n_experts", "blob_bytes",
  "page_size", "offset_formula", "quantization": {"group_size", "bits"},
  "components": [{"proj", "part", "dtype", "shape", "offset", "nbytes"}],
  optional "payload_bytes", "top_k"}.  The components tile
  [0, payload) without holes in offset order; the record is padded to
  whole pages.

This module reads and validates that format, loads it into the pinned host
store or an HBM store the slot pool fills from, writes it, and repacks local
MLX-layout safetensors shards into it (no network, no MLX).
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np

from . import geometry as G

INDEX = "experts_index.json"
BLOB = "experts.bin"
DTYPE_BYTES = {"U32": 4, "I32": 4, "F32": 4, "F16": 2, "BF16": 2, "U16": 2, "U8": 1, "I8": 1}


class StoreFormatError(ValueError):
    pass


@dataclass
class StoreIndex:
    n_layers: int
    n_experts: int
    blob_bytes: int
    page_size: int
    group_size: int
    bits: int
    components: list          # dicts sorted by offset
    model: str = ""
    top_k: int | None = None

    @property
    def payload_bytes(self) -> int:
        return sum(c["nbytes"] for c in self.components)

    @classmethod
    def load(cls, path: str) -> "StoreIndex":
        with open(path) as f:
            d = json.load(f)
        return cls.from_dict(d)

    @classmethod
    def from_dict(cls, d: dict) -> "StoreIndex":
        try:
            q = d["quantization"]
            idx = cls(n_layers=int(d.get("n_layers", 48)), n_experts=int(d["n_experts"]),
                      blob_bytes=int(d["blob_bytes"]), page_size=int(d.get("page_size", G.PAGE)),
                      group_size=int(q["group_size"]), bits=int(q["bits"]),
                      components=sorted((dict(c) for c in d["components"]),
                                        key=lambda c: c["offset"]),
                      model=d.get("model", ""), top_k=d.get("top_k"))
        except (KeyError, TypeError) as e:
            raise StoreFormatError(f"experts index: missing or malformed field {e}") from None
        idx.validate()
        return idx

    def validate(self):
        """The engine's load-time checks (engine_v3.py:166-175): components
        contiguous from 0 in offset order, payload within the blob."""
        end = 0
        for c in self.components:
            if c["offset"] != end:
                raise StoreFormatError(f"blob layout has a hole before {c['proj']}.{c['part']}: "
                                       f"{c['offset']} != {end}")
            n = int(np.prod(c["shape"])) * DTYPE_BYTES.get(c["dtype"], 0)
            if n != c["nbytes"]:
                raise StoreFormatError(f"{c['proj']}.{c['part']}: shape {c['shape']} x "
                                       f"{c['dtype']} is {n} bytes, index says {c['nbytes']}")
            end += c["nbytes"]
        if end > self.blob_bytes:
            raise StoreFormatError("components overrun the blob")
        if self.n_layers <= 0 or self.n_experts <= 0:
            raise StoreFormatError("n_layers and n_experts must be positive")

    def to_dict(self) -> dict:
        d = {"model": self.model, "n_layers": self.n_layers, "n_experts": self.n_experts,
             "blob_bytes": self.blob_bytes, "payload_bytes": self.payload_bytes,
             "page_size": self.page_size,
             "offset_formula": "(layer * n_experts + expert) * blob_bytes",
             "quantization": {"group_size": self.group_size, "bits": self.bits},
             "components": self.components}
        if self.top_k is not None:
            d["top_k"] = self.top_k
        return d

    def geometry(self, base: G.Geometry | None = None) -> G.Geometry:
        """The Geometry whose record layout this index describes.  With
        `base`, its routing/activation settings are kept and the shapes are
        checked against it; without, a projection bias means the gpt-oss
        block (clamped SwiGLU, top-k-then-softmax routing), else Qwen3's."""
        comp = {f"{c['proj']}.{c['part']}": c for c in self.components}
        if "gate_proj.weight" not in comp:
            raise StoreFormatError("index has no gate_proj.weight")
        gw = comp["gate_proj.weight"]["shape"]
        d_ff, d_model = int(gw[0]), int(gw[1]) * 32 // self.bits
        has_bias = "gate_proj.bias" in comp
        if base is None:
            base = G.GPT_OSS_120B if has_bias else G.QWEN3_30B_A3B
        geom = base.with_(d_model=d_model, d_ff=d_ff, n_experts=self.n_experts,
                          n_layers=self.n_layers, has_proj_bias=has_bias,
                          group_size=self.group_size, bits=self.bits,
                          top_k=self.top_k or base.top_k)
        if len(geom.components) != len(self.components):
            raise StoreFormatError(f"index has {len(self.components)} components, the "
                                   f"geometry {len(geom.components)}")
        for gc, c in zip(geom.components, self.components):
            name = f"{c['proj']}.{c['part']}"
            if (gc.name != name or tuple(gc.shape) != tuple(c["shape"]) or gc.dtype != c["dtype"]
                    or gc.offset != c["offset"]):
                raise StoreFormatError(f"component {name} {c['dtype']}{c['shape']}@{c['offset']} "
                                       f"differs from the kernels' layout {gc.name} "
                                       f"{gc.dtype}{gc.shape}@{gc.offset}")
        if geom.record_bytes != self.blob_bytes:
            raise StoreFormatError(f"blob_bytes {self.blob_bytes} != {geom.record_bytes} "
                                   f"(payload padded to {G.PAGE}-byte pages)")
        return geom


class ExpertStoreFile:
    """A store directory: its index and a read-only memory map of the blob."""

    def __init__(self, model_dir: str, base: G.Geometry | None = None):
        self.dir = model_dir
        self.index = StoreIndex.load(os.path.join(model_dir, INDEX))
        self.geom = self.index.geometry(base)
        path = os.path.join(model_dir, BLOB)
        n = self.index.n_layers * self.index.n_experts
        size = os.path.getsize(path)
        if size < n * self.index.blob_bytes:
            raise StoreFormatError(f"{path}: {size} bytes, the index needs "
                                   f"{n * self.index.blob_bytes}")
        self.n_records = n
        self.records = np.memmap(path, dtype=np.uint8, mode="r",
                                 shape=(n, self.index.blob_bytes))

    def record(self, layer: int, expert: int) -> np.ndarray:
        return self.records[layer * self.index.n_experts + expert]

    def to_host_store(self, chunk_records: int = 64, n_workers: int = 1):
        """Read every record into pinned host memory (the pool's fill source)."""
        from .pool import HostStore
        hs = HostStore(self.geom, self.n_records)
        self.read_into(hs.array, chunk_records, n_workers)
        return hs

    def read_into(self, dst: np.ndarray, chunk_records: int = 64, n_workers: int = 1):
        """Read every record into dst (uint8 [n_records, blob_bytes], C order):
        contiguous preadv calls of `chunk_records` records straight into it,
        on `n_workers` threads (preadv releases the GIL), as the reference's
        fill workers read (engine_v3.py:255-290)."""
        from concurrent.futures import ThreadPoolExecutor
        rb = self.index.blob_bytes
        if dst.dtype != np.uint8 or dst.shape != (self.n_records, rb) or \
                not dst.flags.c_contiguous:
            raise ValueError(f"dst must be C-contiguous uint8 {(self.n_records, rb)}")
        fd = os.open(os.path.join(self.dir, BLOB), os.O_RDONLY)

        def read(r0):
            r1 = min(self.n_records, r0 + chunk_records)
            view = memoryview(dst[r0:r1].reshape(-1))
            want, got = (r1 - r0) * rb, 0
            while got < want:
                n = os.preadv(fd, [view[got:]], r0 * rb + got)
                if n <= 0:
                    raise IOError(f"short read {got} of {want} at record {r0}")
                got += n

        try:
            starts = range(0, self.n_records, chunk_records)
            if n_workers <= 1:
                for r0 in starts:
                    read(r0)
            else:
                with ThreadPoolExecutor(n_workers, thread_name_prefix="fetch") as ex:
                    list(ex.map(read, starts))
        finally:
            os.close(fd)
        return dst

    def to_device(self, device="cuda", chunk_records: int = 64):
        """Copy every record into an HBM store tensor [n_records, blob_bytes]."""
        import torch
        out = torch.empty((self.n_records, self.index.blob_bytes), dtype=torch.uint8,
                          device=device)
        for r0 in range(0, self.n_records, chunk_records):
            r1 = min(self.n_records, r0 + chunk_records)
            out[r0:r1].copy_(torch.from_numpy(np.ascontiguousarray(self.records[r0:r1])))
        return out


def index_for(geom: G.Geometry, model: str = "", top_k: int | None = None) -> StoreIndex:
    comps = []
    for c in geom.components:
        proj, part = c.name.split(".")
        comps.append({"proj": proj, "part": part, "dtype": c.dtype, "shape": list(c.shape),
                      "offset": c.offset, "nbytes": c.nbytes})
    return StoreIndex(n_layers=geom.n_layers, n_experts=geom.n_experts,
                      blob_bytes=geom.record_bytes, page_size=G.PAGE,
                      group_size=geom.group_size, bits=geom.bits, components=comps,
                      model=model, top_k=top_k if top_k is not None else geom.top_k)


def write_store(out_dir: str, geom: G.Geometry, records, model: str = "") -> StoreIndex:
    """Write `records` (uint8 [n_layers * n_experts, record_bytes], or a
    callable (layer, expert) -> bytes of the record) as experts.bin +
    experts_index.json."""
    os.makedirs(out_dir, exist_ok=True)
    idx = index_for(geom, model)
    n = geom.n_layers * geom.n_experts
    with open(os.path.join(out_dir, BLOB), "wb", buffering=1 << 24) as f:
        for r in range(n):
            rec = records(r // geom.n_experts, r % geom.n_experts) if callable(records) \
                else records[r]
            b = np.asarray(rec, dtype=np.uint8).reshape(-1)
            if b.size != geom.record_bytes:
                raise ValueError(f"record {r} has {b.size} bytes, expected {geom.record_bytes}")
            f.write(b.tobytes())
    with open(os.path.join(out_dir, INDEX), "w") as f:
        json.dump(idx.to_dict(), f, indent=1)
    return idx


# ---------------------------------------------------------------------------
# repack of local safetensors shards (repack.py:61-146 without MLX)
# ---------------------------------------------------------------------------
def read_safetensors_header(path: str):
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
    return hdr, 8 + n


def _expert_tensor_names(layer: int, proj: str, part: str):
    # Qwen3 MLX checkpoints stack experts in switch_mlp (repack.py:72-73);
    # gpt-oss in mlp.experts (repack_gptoss.py:143-144)
    return (f"model.layers.{layer}.mlp.switch_mlp.{proj}.{part}",
            f"model.layers.{layer}.mlp.experts.{proj}.{part}")


def repack_safetensors(src_dir: str, out_dir: str, geom: G.Geometry, model: str = "") -> StoreIndex:
    """Rewrite the stacked per-layer expert tensors of local safetensors
    shards ([n_experts, *shape] each) into one contiguous record per
    (layer, expert).  Layer by layer; shards are memory-mapped."""
    shards = sorted(os.path.join(src_dir, p) for p in os.listdir(src_dir)
                    if p.endswith(".safetensors"))
    if not shards:
        raise FileNotFoundError(f"no .safetensors shards under {src_dir}")
    tensors = {}
    for sp in shards:
        hdr, start = read_safetensors_header(sp)
        for name, meta in hdr.items():
            if name == "__metadata__":
                continue
            s, e = meta["data_offsets"]
            tensors[name] = (sp, start + s, start + e, meta["dtype"], meta["shape"])
    maps = {}

    def stacked(layer, comp):
        proj, part = comp.name.split(".")
        for nm in _expert_tensor_names(layer, proj, part):
            if nm in tensors:
                sp, s, e, dt, shape = tensors[nm]
                if dt != comp.dtype or list(shape) != [geom.n_experts, *comp.shape]:
                    raise StoreFormatError(f"{nm}: {dt}{shape}, expected "
                                           f"{comp.dtype}{[geom.n_experts, *comp.shape]}")
                if sp not in maps:
                    maps[sp] = np.memmap(sp, dtype=np.uint8, mode="r")
                return maps[sp][s:e].reshape(geom.n_experts, comp.nbytes)
        raise StoreFormatError(f"layer {layer}: no tensor for {comp.name}")

    os.makedirs(out_dir, exist_ok=True)
    idx = index_for(geom, model)
    pad = geom.record_bytes - geom.payload_bytes
    with open(os.path.join(out_dir, BLOB), "wb", buffering=1 << 24) as f:
        for layer in range(geom.n_layers):
            parts = [stacked(layer, c) for c in geom.components]
            for e in range(geom.n_experts):
                for p in parts:
                    f.write(p[e].tobytes())
                if pad:
                    f.write(b"\0" * pad)
    with open(os.path.join(out_dir, INDEX), "w") as f:
        json.dump(idx.to_dict(), f, indent=1)
    return idx
