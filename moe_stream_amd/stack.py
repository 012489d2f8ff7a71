"""Multi-layer bs=1 decode over an HBM-resident slot pool, routing on device.

Per layer L of a token: one launch routes x_L through layer L's router
(top-k, scores), runs layer L+1's router on the same x_L for the lookahead
prediction (top_k_indices, engine_v3.py:509-515) and looks the routed experts
up in the device slot table; then the two expert-block kernels read the
routed slots.  No host round trip per layer: the reference's per-layer
`mx.eval` + `np.array(inds)` + `acquire` (engine_v3.py:515-552) becomes a
device-side table lookup, so a whole token can be captured as one HIP graph.

Residency: a pool of n_slots holds the most popular (layer, expert) pairs;
the slot table maps every pair either to its pool slot (ref >= 0) or, for a
pair not in the pool, to its record in the HBM expert store (ref < 0), which
the kernels read directly.  Both hold identical bytes, so outputs do not
depend on residency (slot-permutation / pool-size invariance).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib, ops, synth
from .geometry import Geometry
from .pool import SlotPool, _norm_device


def routers(geom: Geometry, n_layers: int, device, seed: int, zipf_s: float | None,
            router_bias: bool):
    """Router weights [L, E, D] and bias [L, E] (or None) of the synthetic
    stacks: bf16 N(0, 0.02) weights, optional bf16 N(0, 0.02) bias, plus a
    Zipf(zipf_s) log-popularity per layer on the logits.  Returns (W, bias,
    log-popularity or None)."""
    W, b = synth.router_weights(geom, n_layers, device, seed + 1, with_bias=router_bias)
    logpop = None
    if zipf_s is not None:
        logpop = synth.zipf_log_popularity(n_layers, geom.n_experts, zipf_s, seed + 2)
        zb = synth.bf16_bias_from_log(logpop, device)
        b = zb if b is None else (b.float() + zb.float()).to(torch.bfloat16)
    return W, b, logpop


class DecodeStack:
    def __init__(self, geom: Geometry, n_layers: int, n_slots: int, device="cuda",
                 seed: int = synth.SEED_BASE + 2, zipf_s: float | None = 1.1,
                 router_bias: bool = False, widen: int = 1, resident=None,
                 k_pred: int | None = None):
        self.geom = geom
        self.L = n_layers
        self.E = geom.n_experts
        self.k = geom.top_k
        self.device = _norm_device(device)
        self.widen = widen
        # the lookahead width: k x widen (PF_WIDEN, engine_v3.py:84), or any
        # width the C ABI accepts (1..min(E, 64)), narrower than k included
        self.k_pred = min(self.k * widen, self.E) if k_pred is None else int(k_pred)
        n_rec = n_layers * self.E
        self.store = synth.make_store(geom, n_rec, self.device, seed)
        self.pool = SlotPool(geom, n_slots, self.device, store=self.store)
        self.W, self.bias, self.logpop = routers(geom, n_layers, self.device, seed,
                                                 zipf_s, router_bias)
        # residency: `resident` (layer, expert) pairs in the pool, in a seeded
        # random slot placement; the rest read from the store
        if resident is None:
            if self.logpop is not None:
                resident = synth.popular_pairs(self.logpop, max(1, n_slots // n_layers))
            else:
                rng = np.random.default_rng(seed + 3)
                per = max(1, n_slots // n_layers)
                resident = [(Lx, int(e)) for Lx in range(n_layers)
                            for e in np.sort(rng.permutation(self.E)[:per])]
        resident = resident[:n_slots]
        slots = synth.slot_permutation(n_slots, len(resident), seed + 4)
        table = -(np.arange(n_rec, dtype=np.int64) + 1)
        recs = np.array([Lx * self.E + e for Lx, e in resident], dtype=np.int64)
        table[recs] = slots
        self.table_host = table.reshape(n_layers, self.E).astype(np.int32)
        self.table = torch.tensor(self.table_host, device=self.device)
        self.pool.fill(recs, slots)
        # per-layer device outputs
        self.bufs = [ops.RouteBuffers(1, self.k, self.k_pred, self.device)
                     for _ in range(n_layers)]
        self.route_ws = torch.zeros(_lib.lib().moe_route_workspace(1, self.E),
                                    dtype=torch.uint8, device=self.device)
        g = geom.c_geom()
        import ctypes as C
        self.ffn_ws = torch.zeros(_lib.lib().moe_ffn_decode_workspace(C.byref(g), 1, self.k),
                                  dtype=torch.uint8, device=self.device)
        self.x_in = torch.zeros((n_layers, geom.d_model), dtype=torch.bfloat16,
                                device=self.device)
        self.y = torch.zeros((n_layers, geom.d_model), dtype=torch.bfloat16,
                             device=self.device)
        self.graph = None

    # -- one token ----------------------------------------------------------
    def layer(self, Lx: int, stream=None):
        g = self.geom
        nxt = Lx + 1 < self.L
        b = self.bias[Lx] if self.bias is not None else None
        bn = self.bias[Lx + 1] if (self.bias is not None and nxt) else None
        bufs = self.bufs[Lx]
        ops.route(self.x_in[Lx:Lx + 1], self.W[Lx], b, g.routing,
                  g.norm_topk_prob, self.k,
                  W_next=self.W[Lx + 1] if nxt else None, bias_next=bn,
                  k_pred=self.k_pred, table=self.table[Lx], bufs=bufs,
                  stream=stream, workspace=self.route_ws)
        ops.ffn_decode(self.pool, bufs.slot_refs, bufs.scores,
                       self.x_in[Lx:Lx + 1], out=self.y[Lx:Lx + 1],
                       stream=stream, workspace=self.ffn_ws)

    def token_eager(self, stream=None):
        for Lx in range(self.L):
            self.layer(Lx, stream)

    def capture(self):
        """Capture one token (all layers) as a HIP graph."""
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self.token_eager()          # warm the launch path outside capture
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.token_eager()
        return self.graph

    def run_token(self, x_tok: torch.Tensor, use_graph: bool = True):
        """x_tok: bf16 [n_layers, d_model], the residual stream of one token."""
        self.x_in.copy_(x_tok, non_blocking=True)
        if use_graph and self.graph is not None:
            self.graph.replay()
        else:
            self.token_eager()

    # -- one launch per token ---------------------------------------------
    # geometries and routing rules with a whole-token kernel: (d_model, d_ff,
    # top-k, projection bias, activation, routing)
    PERSISTENT = {(2048, 768, 8, False, _lib.MOE_ACT_SWIGLU, _lib.MOE_ROUTE_SOFTMAX_TOPK),
                  (2880, 2880, 4, True, _lib.MOE_ACT_SWIGLU_CLAMP, _lib.MOE_ROUTE_TOPK_SOFTMAX)}

    # geometries whose whole-token kernel is the faster decode (both, on one
    # MI355X: Qwen3 48 layers about 1,900 against 1,150 tokens/s for the
    # per-layer graph; gpt-oss 36 layers 1,158-1,179 against 1,096-1,120)
    PERSISTENT_PREFERRED = {(2048, 768, 8, False, _lib.MOE_ACT_SWIGLU, _lib.MOE_ROUTE_SOFTMAX_TOPK),
                            (2880, 2880, 4, True, _lib.MOE_ACT_SWIGLU_CLAMP,
                             _lib.MOE_ROUTE_TOPK_SOFTMAX)}

    def persistent_preferred(self) -> bool:
        g = self.geom
        return self.persistent_supported() and \
            (g.d_model, g.d_ff, self.k, g.has_proj_bias, g.act, g.routing) in self.PERSISTENT_PREFERRED

    def persistent_supported(self) -> bool:
        import ctypes as C
        L = _lib.lib()
        g = self.geom
        return L.moe_stack_workspace(C.byref(g.c_geom()), self.L, self.E, self.k) > 0 and \
            (g.d_model, g.d_ff, self.k, g.has_proj_bias, g.act, g.routing) in self.PERSISTENT

    # the launch count after which the persistent workspace is zeroed and the
    # epoch restarts at 1 (the kernel's per-layer flags, epoch * n_layers + l,
    # must stay below 2^32)
    EPOCH_RESTART = 1 << 22

    @staticmethod
    def epoch_limit(n_layers: int) -> int:
        return min(DecodeStack.EPOCH_RESTART, (2 ** 32 - 1) // n_layers - 2)

    def _persistent_buffers(self):
        import ctypes as C
        g = self.geom.c_geom()
        n = _lib.lib().moe_stack_workspace(C.byref(g), self.L, self.E, self.k)
        dev = self.device
        self.p_ws = torch.zeros(n, dtype=torch.uint8, device=dev)
        self.p_epoch = 0
        self.p_ids = torch.zeros((self.L, self.k), dtype=torch.int32, device=dev)
        self.p_scores = torch.zeros((self.L, self.k), dtype=torch.float32, device=dev)
        self.p_refs = torch.zeros((self.L, self.k), dtype=torch.int32, device=dev)
        self.p_pred = torch.zeros((self.L, self.k_pred), dtype=torch.int32, device=dev)
        self.p_miss = torch.zeros((self.L,), dtype=torch.int32, device=dev)
        self.p_y = torch.zeros((self.L, self.geom.d_model), dtype=torch.bfloat16, device=dev)

    def reset_persistent(self, stream=None):
        """Zero the persistent kernel's workspace (on `stream`) and restart
        its epoch at 1: required after a failed launch and before the epoch
        bound."""
        if not hasattr(self, "p_ws"):
            self._persistent_buffers()
            return
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        with torch.cuda.stream(s):
            self.p_ws.zero_()
        self.p_epoch = 0

    def token_persistent(self, x_tok: torch.Tensor, stream=None, ordinary: bool = False):
        """All layers of one token in one launch.  x_tok: bf16 [n_layers,
        d_model]; outputs in p_y, p_ids, p_scores, p_refs, p_pred, p_miss.

        ordinary=False: a cooperative launch.  ordinary=True: an ordinary
        launch, for a caller that guarantees no other kernel runs on the
        device meanwhile; if that guarantee fails, check_persistent() reports
        MOE_ERR_TIMEOUT and the tokens must be run again."""
        import ctypes as C
        if not hasattr(self, "p_ws"):
            self._persistent_buffers()
        if self.p_epoch >= self.epoch_limit(self.L):
            self.reset_persistent(stream)
        x_tok = x_tok.contiguous()
        self.p_epoch += 1
        g = self.geom.c_geom()
        b = self.bias.data_ptr() if self.bias is not None else None
        flags = _lib.MOE_STACK_ORDINARY if ordinary else _lib.MOE_STACK_COOPERATIVE
        try:
            _lib.check(_lib.lib().moe_stack_decode(
                C.byref(self.pool.c_view()), C.byref(g), self.L, self.E, self.k,
                x_tok.data_ptr(), self.W.data_ptr(), b, self.geom.routing,
                int(self.geom.norm_topk_prob), self.k_pred, self.table.data_ptr(),
                self.p_y.data_ptr(), self.p_ids.data_ptr(), self.p_scores.data_ptr(),
                self.p_refs.data_ptr(), self.p_pred.data_ptr(), self.p_miss.data_ptr(),
                self.p_epoch, flags, self.p_ws.data_ptr(), self.p_ws.numel(),
                _lib.stream_ptr(stream)))
        except _lib.MoeError:
            # nothing was launched: the counters still hold the previous
            # epoch, which the next launch must follow
            self.p_epoch -= 1
            raise

    def check_persistent(self, stream=None):
        """Synchronise `stream` and read the device error word.  On an error
        the workspace is reset (the next launch starts at epoch 1) and the
        error is raised: MoeError with code MOE_ERR_TIMEOUT when a launch's
        grid was not resident at once (run those tokens again, cooperatively),
        MOE_ERR_DEVICE for an out-of-range slot reference."""
        rc = _lib.lib().moe_check_device_error(_lib.stream_ptr(stream))
        if rc < 0:
            self.reset_persistent(stream)
            _lib.check(rc)

    def token_persistent_checked(self, x_tok: torch.Tensor, stream=None):
        """One token by an ordinary launch, checked; if its grid was not
        resident at once, the token runs again by a cooperative launch.
        Synchronises `stream` (one host round trip per token).  The per-layer
        miss counts (p_miss, accumulated by the kernel) of a launch that timed
        out come from unfinished routing: they are restored before the retry."""
        if not hasattr(self, "p_ws"):
            self._persistent_buffers()
        s = stream if stream is not None else torch.cuda.current_stream(self.device)
        with torch.cuda.stream(s):
            miss0 = self.p_miss.clone()
        self.token_persistent(x_tok, stream, ordinary=True)
        try:
            self.check_persistent(stream)
        except _lib.MoeError as e:
            if e.code != _lib.MOE_ERR_TIMEOUT:
                raise
            with torch.cuda.stream(s):
                self.p_miss.copy_(miss0)
            self.token_persistent(x_tok, stream, ordinary=False)
            self.check_persistent(stream)
            return "cooperative"
        return "ordinary"

    # -- bookkeeping --------------------------------------------------------
    def expert_bytes_per_token(self) -> int:
        return self.L * self.k * self.geom.payload_bytes

    def routed(self):
        """Host copy of this token's routing: ids, scores, refs, preds."""
        ids = torch.stack([b.ids[0] for b in self.bufs]).cpu().numpy()
        sc = torch.stack([b.scores[0] for b in self.bufs]).cpu().numpy()
        refs = torch.stack([b.slot_refs[0] for b in self.bufs]).cpu().numpy()
        pred = torch.stack([b.pred[0] for b in self.bufs]).cpu().numpy()
        return ids, sc, refs, pred


class PrefillStack(DecodeStack):
    """T tokens per layer through an n_layers stack (the batched/prefill
    path): per layer, the many-token router (bf16 MFMA logits + top-k +
    lookahead + slot lookup) and the grouped MFMA expert block, all on
    device, no host round trip.  The pool, store, routers and residency are
    those of DecodeStack."""

    def __init__(self, geom: Geometry, n_layers: int, n_slots: int, n_tokens: int,
                 device="cuda", block: str = "grouped", **kw):
        """block: "grouped" -- the MFMA block for many tokens (prefill);
        "decode" -- the decode kernels, whose small-T form groups the pairs by
        slot (bit-identical to one call per token); "auto" -- the choice
        ops.ffn makes for n_tokens."""
        if block == "auto":
            block = "grouped" if n_tokens > ops.GROUPED_MIN_TOKENS else "decode"
        super().__init__(geom, n_layers, n_slots, device, **kw)
        import ctypes as C
        self.T = n_tokens
        self.block = block
        dev = self.device
        self.bufs = [ops.RouteBuffers(n_tokens, self.k, self.k_pred, dev)
                     for _ in range(n_layers)]
        self.route_ws = torch.zeros(_lib.lib().moe_route_workspace(n_tokens, self.E),
                                    dtype=torch.uint8, device=dev)
        g = geom.c_geom()
        ws = (_lib.lib().moe_ffn_grouped_workspace if block == "grouped"
              else _lib.lib().moe_ffn_decode_workspace)(C.byref(g), n_tokens, self.k)
        self.ffn_ws = torch.zeros(ws, dtype=torch.uint8, device=dev)
        self.x_in = torch.zeros((n_layers, n_tokens, geom.d_model), dtype=torch.bfloat16,
                                device=dev)
        self.y = torch.zeros((n_layers, n_tokens, geom.d_model), dtype=torch.bfloat16,
                             device=dev)

    def layer(self, Lx: int, stream=None):
        g = self.geom
        nxt = Lx + 1 < self.L
        b = self.bias[Lx] if self.bias is not None else None
        bn = self.bias[Lx + 1] if (self.bias is not None and nxt) else None
        bufs = self.bufs[Lx]
        ops.route(self.x_in[Lx], self.W[Lx], b, g.routing, g.norm_topk_prob, self.k,
                  W_next=self.W[Lx + 1] if nxt else None, bias_next=bn,
                  k_pred=self.k_pred, table=self.table[Lx], bufs=bufs,
                  stream=stream, workspace=self.route_ws)
        f = ops.ffn_grouped if self.block == "grouped" else ops.ffn_decode
        f(self.pool, bufs.slot_refs, bufs.scores, self.x_in[Lx], out=self.y[Lx],
          stream=stream, workspace=self.ffn_ws)

    def run_step(self, x_step: torch.Tensor, use_graph: bool = True):
        """x_step: bf16 [n_layers, T, d_model], the residual stream of T tokens
        at every layer."""
        self.x_in.copy_(x_step, non_blocking=True)
        if use_graph and self.graph is not None:
            self.graph.replay()
        else:
            self.token_eager()

    def pairs_per_layer(self) -> int:
        return self.T * self.k

    def routed_counts(self) -> np.ndarray:
        """Per layer, the number of pairs routed to each expert (host copy)."""
        ids = torch.stack([b.ids for b in self.bufs]).cpu().numpy()
        return np.stack([np.bincount(ids[L].ravel(), minlength=self.E)
                         for L in range(self.L)])


class StreamingStack:
    """The reference's engine loop over a pool smaller than the model: per
    layer, streaming_call (route + lookahead, one host synchronisation,
    prefetch of the predicted layer-L+1 experts, acquire, the expert block;
    engine_v3.py:493-609) on an ExpertPool whose fills come from a pinned
    host store by hipMemcpyAsync (one per record), prefetches on a side
    stream.  Store
    records, routers and inputs are those of DecodeStack with the same seed,
    so the two produce identical outputs."""

    def __init__(self, geom: Geometry, n_layers: int, n_slots: int, device="cuda",
                 seed: int = synth.SEED_BASE + 2, zipf_s: float | None = 1.1,
                 router_bias: bool = False, widen: int = 1, host_store=None,
                 evict: str | None = None, native: bool = False,
                 pool_layout: str = "records", depths=(1,)):
        """native: run each layer's engine loop in the library
        (moe_engine_layer) instead of MoEBlock.streaming_call; same policy,
        fills and kernels, no Python frame between a layer's steps.
        pool_layout: "records" (a fill is one copy-engine copy per record) or
        "components" (copy-kernel fills).
        depths: the prefetch depths (the reference's PF_DEPTH list,
        engine_v3.py:61), each layer L's hidden state predicting layer L+d."""
        from .block import MoEBlock
        from .pool import ExpertPool
        self.geom = geom
        self.L = n_layers
        self.E = geom.n_experts
        self.k = geom.top_k
        self.device = _norm_device(device)
        self.store = host_store if host_store is not None else \
            synth.make_host_store(geom, n_layers * self.E, self.device, seed)
        self.depths = tuple(int(d) for d in depths)
        if not self.depths or min(self.depths) <= 0 or len(self.depths) > 4:
            raise ValueError(f"depths {depths!r}: 1 to 4 positive layer offsets")
        self.pool = ExpertPool(geom, n_slots, store=self.store, device=self.device, evict=evict,
                               widen=widen, n_layers=n_layers, layout=pool_layout,
                               depths=self.depths)
        self.W, self.bias, self.logpop = routers(geom, n_layers, self.device, seed,
                                                 zipf_s, router_bias)
        self.blocks = []
        for Lx in range(n_layers):
            self.blocks.append(MoEBlock(Lx, geom, self.pool, self.W[Lx],
                                        None if self.bias is None else self.bias[Lx],
                                        self.blocks, depths=self.depths, widen=widen))
        self.native = native
        self._engine = None
        if native:
            from .pool import HostStore
            if not isinstance(self.store, HostStore):
                raise ValueError("the native engine fills from a pinned host store")
            self.k_pred = min(self.k * widen, self.E, 64)
            self._compute = torch.cuda.current_stream(self.device)
            h = C.c_void_p()
            g = geom.c_geom()
            _lib.check(_lib.lib().moe_engine_create(
                C.byref(self.pool.c_view()), C.byref(g), n_layers, self.E, self.k,
                self.k_pred, self.pool.policy._h, self.store.ptr, self.store.record_bytes,
                self.store.n_records, _lib.stream_ptr(self._compute),
                _lib.stream_ptr(self.pool.side), C.byref(h)))
            self._engine = h

    def close(self):
        if self._engine:
            _lib.lib().moe_engine_destroy(self._engine)
            self._engine = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def token(self, x_tok: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """x_tok: bf16 [n_layers, d_model]; returns y bf16 [n_layers, d_model]."""
        if out is None:
            out = torch.empty_like(x_tok)
        if self._engine:
            return self._token_native(x_tok, out)
        for Lx, blk in enumerate(self.blocks):
            out[Lx:Lx + 1] = blk(x_tok[Lx:Lx + 1])
        return out

    def _layer_args(self):
        """Per layer: (router, router bias, next router, next bias) pointers."""
        if getattr(self, "_largs", None) is None:
            W, b, L = self.W, self.bias, self.L
            ptr = lambda t: None if t is None else t.data_ptr()
            self._largs = [(W[Lx].data_ptr(), ptr(None if b is None else b[Lx]),
                            W[Lx + 1].data_ptr() if Lx + 1 < L else None,
                            ptr(None if (b is None or Lx + 1 >= L) else b[Lx + 1]))
                           for Lx in range(L)]
        return self._largs

    def _depth_args(self):
        """Per layer: (router, router bias, depths, routers and biases of
        the target layers) for moe_engine_layer_depths; a target past the
        last layer has a NULL router."""
        if getattr(self, "_dargs", None) is None:
            W, b, L, n = self.W, self.bias, self.L, len(self.depths)
            ptr = lambda t: None if t is None else t.data_ptr()
            depths = (C.c_int32 * n)(*self.depths)
            self._dargs = []
            for Lx in range(L):
                tg = [Lx + d for d in self.depths]
                wl = (C.c_void_p * n)(*[W[t].data_ptr() if t < L else None for t in tg])
                bl = None if b is None else \
                    (C.c_void_p * n)(*[b[t].data_ptr() if t < L else None for t in tg])
                self._dargs.append((W[Lx].data_ptr(), ptr(None if b is None else b[Lx]),
                                    depths, wl, bl))
        return self._dargs

    def _token_native(self, x_tok, out):
        assert x_tok.is_contiguous() and out.is_contiguous()
        assert x_tok.dtype == out.dtype == torch.bfloat16
        assert x_tok.shape == out.shape == (self.L, self.geom.d_model)
        step = self.geom.d_model * 2
        eng, g = self._engine, self.geom
        mode, renorm = g.routing, int(g.norm_topk_prob)
        x0, y0 = x_tok.data_ptr(), out.data_ptr()
        if self.depths == (1,):
            layer = _lib.lib().moe_engine_layer
            for Lx, (w, b, wn, bn) in enumerate(self._layer_args()):
                rc = layer(eng, Lx, x0 + Lx * step, w, b, mode, renorm, wn, bn, y0 + Lx * step)
                if rc < 0:
                    _lib.check(rc)
            return out
        layer, n = _lib.lib().moe_engine_layer_depths, len(self.depths)
        for Lx, (w, b, depths, wl, bl) in enumerate(self._depth_args()):
            rc = layer(eng, Lx, x0 + Lx * step, w, b, mode, renorm, depths, n, wl, bl,
                       y0 + Lx * step)
            if rc < 0:
                _lib.check(rc)
        return out

    def engine_counters(self) -> dict:
        v = (C.c_int64 * 5)()
        _lib.check(_lib.lib().moe_engine_counters(self._engine, v))
        return dict(bytes_read=v[0], bytes_exposed=v[1], recall_hit=v[2], recall_total=v[3],
                    pending=v[4])

    def recall(self) -> float:
        if self._engine:
            c = self.engine_counters()
            return c["recall_hit"] / c["recall_total"] if c["recall_total"] else float("nan")
        r = [v for b in self.blocks for v in b.recall]
        return float(np.mean(r)) if r else float("nan")
