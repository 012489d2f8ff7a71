"""numpy restatement of the arithmetic on moe-stream's expert hot path.

TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).

Every function cites the reference line it restates.  Two arithmetic modes:

  mode="f64"  -- the mathematical truth: fp64 everywhere, no rounding.
  mode="mlx"  -- MLX-emulation: fp64 arithmetic rounded to bf16 at each MLX
                 graph edge, i.e. wherever the reference materialises a bf16
                 array (gather_qmm outputs, swiglu intermediates, router
                 logits/probabilities, score products and sums).

Parity status (how each function is pinned, see tests/test_oracle_*.py):
  bf16 rounding ....... pinned: round-trip on every bf16 bit pattern, known
                        answers for ties-to-even.
  unpack_u4/pack_u4 ... pinned: brute-force bit loop on tiny rows; the nibble
                        order of kernels.py:135-139 as known answers.
  dequant ............. pinned: brute force element loop; w = s*(q-8) special
                        case of the synthetic workloads.
  qmv / gather_qmm .... pinned: dense dequant-then-dot (np.einsum) and the
                        per-group factorisation of kernels.py:141-145 agree.
  qmm / moe_block_batch pinned: row-by-row equal to qmv / moe_block.
  swiglu (Qwen3) ...... pinned: closed form silu(g)*u on special values.
  swiglu_clamped ...... pinned: saturation/clipping special cases.
  routers ............. pinned: brute-force full sort; invariants (distinct
                        ids, renormed scores sum to 1, softmax monotone).
  combine ............. pinned: permutation invariance, linearity.
  MLX rounding points inside gather_qmm / softmax / compiled swiglu / sum
                        are NOT pinnable without MLX (absent): "parity
                        unpinned" for the exact bf16 rounding points; the
                        tolerance 2e-2 against both modes covers them.
"""
from __future__ import annotations

import numpy as np

GROUP = 64
BITS = 4


# --------------------------------------------------------------------------
# bf16 helpers (bf16 = high half of an fp32 bit pattern; kernels.py:66-72)
# --------------------------------------------------------------------------
def bf16_bits_to_f32(bits) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    b = np.asarray(bits).astype(np.uint32)
    return (b << 16).view(np.float32)


def f32_to_bf16_bits(x) -> np.ndarray:
    """float -> bf16 bits, round to nearest even (NaN kept quiet)."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16r(x) -> np.ndarray:
    """Round to bf16 (via fp32, as an fp32 accumulator rounded on store)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x)).astype(np.float64)


# --------------------------------------------------------------------------
# 4-bit affine quantisation (kernels.py:104-106, 135-139; verify_120b.py:95)
# --------------------------------------------------------------------------
def unpack_u4(W) -> np.ndarray:
    """uint32 [..., n/8] -> codes uint8 [..., n]; element i lives in word
    i>>3 at bit 4*(i&7), low nibble first (kernels.py:135-139)."""
    W = np.asarray(W, dtype=np.uint32)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    q = (W[..., :, None] >> shifts) & np.uint32(0xF)
    return q.reshape(*W.shape[:-1], W.shape[-1] * 8).astype(np.uint8)


def pack_u4(q) -> np.ndarray:
    """Inverse of unpack_u4."""
    q = np.asarray(q, dtype=np.uint32)
    q = q.reshape(*q.shape[:-1], q.shape[-1] // 8, 8)
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)


def dequant(W, S_bits, B_bits, group: int = GROUP) -> np.ndarray:
    """w(o,i) = S[o,i//G]*q(o,i) + B[o,i//G] in fp64 (kernels.py:104-106).
    S_bits/B_bits are bf16 bit patterns [out, in/G]."""
    q = unpack_u4(W).astype(np.float64)
    S = bf16_bits_to_f32(S_bits).astype(np.float64)
    B = bf16_bits_to_f32(B_bits).astype(np.float64)
    S = np.repeat(S, group, axis=-1)
    B = np.repeat(B, group, axis=-1)
    return S * q + B


def qmv(x, W, S_bits, B_bits, group: int = GROUP) -> np.ndarray:
    """One quantised matrix-vector product y = deq(W) @ x, exact fp64.

    Written in the factorised per-group form of kernels.py:141-145,
    y_o = sum_g S_og * sum_{i in g} q_oi x_i + B_og * sum_{i in g} x_i,
    which tests compare against the dense dequant-then-dot form."""
    x = np.asarray(x, dtype=np.float64)
    q = unpack_u4(W).astype(np.float64)
    n_out, n_in = q.shape
    ng = n_in // group
    qg = q.reshape(n_out, ng, group)
    xg = x.reshape(ng, group)
    S = bf16_bits_to_f32(S_bits).astype(np.float64)
    B = bf16_bits_to_f32(B_bits).astype(np.float64)
    qx = np.einsum("ogi,gi->og", qg, xg)
    return (S * qx + B * xg.sum(-1)[None, :]).sum(-1)


def qmm(X, W, S_bits, B_bits, group: int = GROUP) -> np.ndarray:
    """The same product for many rows at once: Y = X @ deq(W).T, exact fp64
    up to summation order (gather_qmm with transpose=True over [.., n, D]
    inputs, engine_v3.py:588-598).  Dense dequant-then-product form."""
    X = np.asarray(X, dtype=np.float64)
    return X @ dequant(W, S_bits, B_bits, group).T


def _qprod(x, W, S_bits, B_bits):
    x = np.asarray(x, dtype=np.float64)
    return qmv(x, W, S_bits, B_bits) if x.ndim == 1 else qmm(x, W, S_bits, B_bits)


def _round(mode, v):
    return bf16r(v) if mode == "mlx" else np.asarray(v, dtype=np.float64)


# --------------------------------------------------------------------------
# activations
# --------------------------------------------------------------------------
def sigmoid(z):
    """1/(1+exp(-z)), evaluated without cancellation for either sign."""
    z = np.asarray(z, dtype=np.float64)
    e = np.exp(-np.abs(z))
    return np.where(z >= 0, 1.0 / (1.0 + e), e / (1.0 + e))


def swiglu(gate, up, mode: str = "f64"):
    """mlx-lm activations.swiglu(gate, x) = silu(gate) * x, used at
    engine_v3.py:597 (fp32 form: test_kernel.py:63)."""
    g = np.asarray(gate, dtype=np.float64)
    u = np.asarray(up, dtype=np.float64)
    if mode == "mlx":
        sg = bf16r(g * bf16r(sigmoid(g)))
        return bf16r(sg * u)
    return g * sigmoid(g) * u


def swiglu_clamped(up, gate, alpha: float = 1.702, limit: float = 7.0,
                   mode: str = "f64"):
    """gpt-oss clamped SwiGLU, called as swiglu(x_up, x_gate) at
    engine_120b.py:143: g=min(gate,limit); u=clip(up,-limit,limit);
    out = g*sigmoid(alpha*g)*(u+1) (engine_120b.py:27-29, HANDOFF.md:886-887)."""
    g = np.minimum(np.asarray(gate, dtype=np.float64), limit)
    u = np.clip(np.asarray(up, dtype=np.float64), -limit, limit)
    if mode == "mlx":
        gs = bf16r(alpha * g)
        og = bf16r(g * bf16r(sigmoid(gs)))
        return bf16r(og * bf16r(u + 1.0))
    return g * sigmoid(alpha * g) * (u + 1.0)


# --------------------------------------------------------------------------
# routing (engine_v3.py:467-483, engine_120b.py:65-75)
# --------------------------------------------------------------------------
def rank_desc(v) -> np.ndarray:
    """Indices sorted by value descending, ties broken by lower index.
    (MLX argpartition leaves the order of ties unspecified; ids are compared
    as sets with the tie rule of ids_match.)"""
    v = np.asarray(v)
    return np.lexsort((np.arange(v.shape[-1]), -v))


def router_logits(x, W_bits, bias_bits=None, mode: str = "f64"):
    """Router linear layer x @ W.T (+ bias), bf16 weights [E, D].  MLX
    materialises a bf16 array, rounded once after the fused add
    (nn.Linear -> addmm).  x is one token [D] or rows [T, D]."""
    x = np.asarray(x, dtype=np.float64)
    W = bf16_bits_to_f32(W_bits).astype(np.float64)
    z = x @ W.T
    if bias_bits is not None:
        z = z + bf16_bits_to_f32(bias_bits).astype(np.float64)
    return _round(mode, z)


def softmax(z, mode: str = "f64"):
    """softmax(z, precise=True): fp32 arithmetic in MLX, bf16 output."""
    z = np.asarray(z, dtype=np.float64)
    e = np.exp(z - z.max(-1, keepdims=True))
    p = e / e.sum(-1, keepdims=True)
    return _round(mode, p)


def top_k_experts(logits, k: int, norm: bool, mode: str = "f64"):
    """Qwen3 routing, engine_v3.py:467-473: softmax over all experts, top-k of
    the probabilities, optional renormalisation.  Returns (ids ranked by
    probability, scores, probs-ranked-on)."""
    p = softmax(logits, mode)
    ids = rank_desc(p)[:k]
    sc = p[ids]
    if norm:
        tot = _round(mode, sc.sum())
        sc = _round(mode, sc / tot)
    return ids, sc, p


def top_k_route(logits, k: int, mode: str = "f64"):
    """gpt-oss routing, engine_120b.py:65-70: top-k of the raw logits, softmax
    over just those k.  Returns (ids, scores, logits-ranked-on)."""
    z = np.asarray(logits, dtype=np.float64)
    ids = rank_desc(z)[:k]
    return ids, softmax(z[ids], mode), z


def top_k_indices(logits, k: int):
    """Lookahead, engine_v3.py:476-483 / engine_120b.py:73-75: top-k of the
    raw logits of layer L+d's router applied to layer L's hidden state."""
    return rank_desc(np.asarray(logits))[:k]


def bf16_ulp(v) -> np.ndarray:
    """Spacing of bf16 numbers at |v|."""
    v = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(v, 1e-38)))
    return np.exp2(e - 7)


def ids_match(ranked_on, ref_ids, got_ids, ulps: float = 1.0) -> bool:
    """Set equality of top-k ids, excusing exact or near (<= `ulps` bf16 ulp)
    ties at the k-th/(k+1)-th boundary in the ranked quantity."""
    v = np.asarray(ranked_on, dtype=np.float64)
    ref = set(int(i) for i in ref_ids)
    got = set(int(i) for i in got_ids)
    if len(got) != len(got_ids) or len(ref) != len(got):
        return False
    if ref == got:
        return True
    k = len(ref)
    order = rank_desc(v)
    vk = v[order[k - 1]]
    tol = ulps * bf16_ulp(vk)
    must = set(int(i) for i in np.nonzero(v > vk + tol)[0])
    may = set(int(i) for i in np.nonzero(v >= vk - tol)[0])
    return must <= got <= may


# --------------------------------------------------------------------------
# the MoE blocks (engine_v3.py:588-600, engine_120b.py:132-145)
# --------------------------------------------------------------------------
def expert_ffn_qwen3(x, e, mode: str = "f64"):
    """One expert of the Qwen3 block.  `e` is a dict of per-expert arrays:
    gate/up/down .weight (u32), .scales/.biases (bf16 bits).  x is one
    token [D] or a batch of rows [n, D]."""
    up = _round(mode, _qprod(x, e["up_proj.weight"], e["up_proj.scales"],
                             e["up_proj.biases"]))
    gate = _round(mode, _qprod(x, e["gate_proj.weight"], e["gate_proj.scales"],
                               e["gate_proj.biases"]))
    h = swiglu(gate, up, mode)
    y = _round(mode, _qprod(h, e["down_proj.weight"], e["down_proj.scales"],
                            e["down_proj.biases"]))
    return y


def expert_ffn_gptoss(x, e, alpha=1.702, limit=7.0, mode: str = "f64"):
    """One expert of the gpt-oss block: each projection adds its bias vector
    after the quantised product (engine_120b.py:136-139)."""
    def proj(name, inp):
        y = _round(mode, _qprod(inp, e[f"{name}.weight"], e[f"{name}.scales"],
                                e[f"{name}.biases"]))
        return _round(mode, y + bf16_bits_to_f32(e[f"{name}.bias"]))
    up = proj("up_proj", x)
    gate = proj("gate_proj", x)
    h = swiglu_clamped(up, gate, alpha, limit, mode)
    return proj("down_proj", h)


def combine(ys, scores, mode: str = "f64"):
    """y = sum_j scores_j * y_j (engine_v3.py:600, engine_120b.py:145)."""
    ys = np.asarray(ys, dtype=np.float64)
    s = np.asarray(scores, dtype=np.float64)
    prod = _round(mode, ys * s[:, None])
    return _round(mode, prod.sum(0))


def moe_block(x, experts, scores, kind: str = "qwen3", mode: str = "f64",
              alpha=1.702, limit=7.0):
    """Whole expert block for one token: `experts` is the list of per-expert
    dicts in routed order, `scores` their routing weights."""
    if kind == "qwen3":
        ys = [expert_ffn_qwen3(x, e, mode) for e in experts]
    else:
        ys = [expert_ffn_gptoss(x, e, alpha, limit, mode) for e in experts]
    return combine(ys, scores, mode)


def moe_block_batch(X, ids, scores, expert, kind: str = "qwen3", mode: str = "f64",
                    alpha=1.702, limit=7.0):
    """The expert block for T tokens: X [T, D], ids/scores [T, k], expert(e)
    -> per-expert dict.  Each expert runs once over all rows routed to it
    (the batched gather_qmm of the prefill path, engine_v3.py:588-600);
    then per token the score-weighted sum over ranks in rank order."""
    X = np.asarray(X, dtype=np.float64)
    ids = np.asarray(ids)
    T, k = ids.shape
    Y = None
    for e in np.unique(ids):
        t, r = np.nonzero(ids == e)
        ex = expert(int(e))
        if kind == "qwen3":
            ye = expert_ffn_qwen3(X[t], ex, mode)
        else:
            ye = expert_ffn_gptoss(X[t], ex, alpha, limit, mode)
        if Y is None:
            Y = np.zeros((T, k, ye.shape[-1]))
        Y[t, r] = ye
    s = np.asarray(scores, dtype=np.float64)
    prod = _round(mode, Y * s[:, :, None])
    return _round(mode, prod.sum(1))


def rel_err(a, b) -> float:
    """max|a-b| / (max|b| + 1e-30) in fp64 (test_kernel.py:68-71)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))
