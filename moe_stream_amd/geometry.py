"""Expert geometries and the expert-record layout of the repacked store.

A record holds one expert's components back to back in the order
(gate_proj, up_proj, down_proj) x (weight, scales, biases[, bias])
(repack.py:35-37,73-82; repack_gptoss.py:54-55,139-159), padded up to a
whole number of 16 KiB pages (repack_gptoss.py:159; the Qwen3 record is
exactly 162 pages, repack.py:86-90).  Record (layer, expert) sits at
(layer * n_experts + expert) * record_bytes (repack.py:141).
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import _lib

PAGE = 16384
PROJS = ("gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class Component:
    name: str          # "gate_proj.weight"
    dtype: str         # "U32" or "BF16"
    shape: tuple
    nbytes: int
    offset: int        # inside a record

    @property
    def elem_bytes(self) -> int:
        return 4 if self.dtype == "U32" else 2


@dataclass(frozen=True)
class Geometry:
    name: str
    d_model: int
    d_ff: int
    n_experts: int
    n_layers: int
    top_k: int
    has_proj_bias: bool = False
    act: int = _lib.MOE_ACT_SWIGLU
    routing: int = _lib.MOE_ROUTE_SOFTMAX_TOPK
    norm_topk_prob: bool = True
    alpha: float = 1.702
    limit: float = 7.0
    group_size: int = 64
    bits: int = 4
    components: tuple = field(init=False, repr=False, compare=False)
    payload_bytes: int = field(init=False, repr=False, compare=False)
    record_bytes: int = field(init=False, repr=False, compare=False)

    def __post_init__(self):
        parts = ("weight", "scales", "biases") + (("bias",) if self.has_proj_bias else ())
        comps, off = [], 0
        for p in PROJS:
            out_, in_ = (self.d_model, self.d_ff) if p == "down_proj" else (self.d_ff, self.d_model)
            for part in parts:
                if part == "weight":
                    shape, dt = (out_, in_ * self.bits // 32), "U32"
                elif part == "bias":
                    shape, dt = (out_,), "BF16"
                else:
                    shape, dt = (out_, in_ // self.group_size), "BF16"
                n = 1
                for s in shape:
                    n *= s
                nb = n * (4 if dt == "U32" else 2)
                comps.append(Component(f"{p}.{part}", dt, shape, nb, off))
                off += nb
        object.__setattr__(self, "components", tuple(comps))
        object.__setattr__(self, "payload_bytes", off)
        object.__setattr__(self, "record_bytes", -(-off // PAGE) * PAGE)

    @property
    def n_components(self) -> int:
        return len(self.components)

    def comp(self, name: str) -> Component:
        for c in self.components:
            if c.name == name:
                return c
        raise KeyError(name)

    def record_offset(self, layer: int, expert: int) -> int:
        return (layer * self.n_experts + expert) * self.record_bytes

    def c_geom(self) -> _lib.Geom:
        return _lib.Geom(self.d_model, self.d_ff, self.group_size, self.bits,
                         int(self.has_proj_bias), int(self.act),
                         float(self.alpha), float(self.limit))

    def with_(self, **kw) -> "Geometry":
        d = dict(name=self.name, d_model=self.d_model, d_ff=self.d_ff,
                 n_experts=self.n_experts, n_layers=self.n_layers,
                 top_k=self.top_k, has_proj_bias=self.has_proj_bias,
                 act=self.act, routing=self.routing,
                 norm_topk_prob=self.norm_topk_prob, alpha=self.alpha,
                 limit=self.limit, group_size=self.group_size, bits=self.bits)
        d.update(kw)
        return Geometry(**d)


# Qwen3-30B-A3B: 48 layers x 128 experts, top-8, hidden 2048, expert 768.
QWEN3_30B_A3B = Geometry("qwen3-30b-a3b", d_model=2048, d_ff=768, n_experts=128,
                         n_layers=48, top_k=8)
# gpt-oss-120b: 36 layers x 128 experts, top-4, hidden = expert = 2880,
# projection biases, clamped SwiGLU, top-k-then-softmax routing.
GPT_OSS_120B = Geometry("gpt-oss-120b", d_model=2880, d_ff=2880, n_experts=128,
                        n_layers=36, top_k=4, has_proj_bias=True,
                        act=_lib.MOE_ACT_SWIGLU_CLAMP,
                        routing=_lib.MOE_ROUTE_TOPK_SOFTMAX, norm_topk_prob=False)
# A small geometry with compiled kernels, for fast tests.
SMALL = Geometry("small", d_model=256, d_ff=128, n_experts=16, n_layers=4, top_k=4)
