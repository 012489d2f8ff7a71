#!/usr/bin/env python3
"""MoE decode tok/s (bs=1, 48 layers) + achieved HBM GB/s of the
gather-dequant-GEMV kernels against the MI355X peak.

Workload (default): a 48-layer stack of Qwen3-30B-A3B-shaped MoE blocks (128
experts, hidden 2048, expert 768, top-8, 4-bit affine group 64), no
attention, bs=1 decode of 64 consecutive tokens; a 3072-slot HBM pool over the
6144 (layer, expert) pairs with the HBM expert store behind it; router logits
biased by a Zipf(1.1) per-layer popularity; residual h += 0.1*N(0,1) per
layer.  One step = the 64 tokens.  Synthetic seeded weights and inputs.

Prints ONE JSON line (rank 0).  `--gpus N` with N > 1 is refused: this build
measures one GPU.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0   # MI355X HBM3E, 8 TB/s
PCIE_PEAK_GBS = 64.0    # MI355X host interface, PCIe 5.0 x16, one direction


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--workload", default="qwen3-48l",
                    choices=["qwen3-48l", "gptoss-36l", "qwen3-prefill", "qwen3-stream",
                             "qwen3-verify", "qwen3-layer", "hbm-copy"],
                    help="qwen3-prefill: 512 tokens per layer through the grouped "
                         "MFMA path; qwen3-verify: 8 tokens per layer (a speculative "
                         "verification step) through the expert block ops.ffn picks, "
                         "against the same tokens decoded one at a time; "
                         "qwen3-stream: 256 decode tokens over a 2048-slot "
                         "pool fed from a pinned host store; qwen3-layer: one layer at "
                         "batch 1 (256-slot pool); hbm-copy: a 1 GiB device "
                         "copy, the achievable HBM rate and the known-size reference "
                         "for the FETCH_SIZE / WRITE_SIZE counters (secondary "
                         "measurements, not the headline)")
    ap.add_argument("--mode", default="auto", choices=["auto", "persistent", "graph", "eager"],
                    help="persistent: one launch per token; graph/eager: 3 launches per layer; "
                         "auto: the faster of the two for the geometry")
    ap.add_argument("--launch", default="ordinary", choices=["ordinary", "cooperative"],
                    help="persistent mode: the bench owns the GPU, so an ordinary launch "
                         "(checked after the timed steps; if a launch timed out the steps "
                         "are measured again with cooperative launches)")
    ap.add_argument("--cpu-repeats", type=int, default=96,
                    help="timed layer-blocks of the CPU baseline")
    ap.add_argument("--cpu-layers", type=int, default=2,
                    help="qwen3-prefill / qwen3-verify: timed many-token layer-blocks of "
                         "the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="default workload: skip the other configurations (one layer, "
                         "gpt-oss 36 layers, prefill, verification, streaming) that follow "
                         "the headline in the same JSON line")
    ap.add_argument("--engine", default="native", choices=["native", "python"],
                    help="qwen3-stream: the per-layer engine loop in the library "
                         "(moe_engine_layer) or in Python (MoEBlock.streaming_call)")
    ap.add_argument("--pool-layout", default="records", choices=["records", "components"],
                    help="qwen3-stream: slots holding whole records (fills by the copy "
                         "engines, one copy per record) or component arrays (fills by "
                         "copy kernels)")
    ap.add_argument("--depths", default="1",
                    help="qwen3-stream: the prefetch depths, comma-separated (the "
                         "reference's PF_DEPTH list), e.g. 1,2")
    ap.add_argument("--verify-block", default="auto", choices=["auto", "grouped", "decode"],
                    help="qwen3-verify: the expert block (auto: the one ops.ffn picks for "
                         "8 tokens, the grouped MFMA block; decode: the small-T decode "
                         "kernels, bit-identical to one-token calls)")
    ap.add_argument("--profile-tokens", type=int, default=8,
                    help="tokens of the kernel-timing pass after the timed steps")
    return ap.parse_args()


def workload(args, device):
    from moe_stream_amd import geometry as G
    from moe_stream_amd.stack import DecodeStack
    if args.workload == "qwen3-48l":
        geom, L, slots = G.QWEN3_30B_A3B, 48, 3072
        stack = DecodeStack(geom, L, slots, device, zipf_s=1.1)
        cfg = {"workload": "qwen3-30b-a3b-moe-stack", "layers": L, "experts": 128,
               "d_model": 2048, "d_ff": 768, "top_k": 8, "pool_slots": slots,
               "pairs": L * 128, "quant": "4-bit affine g64, bf16 scales/biases",
               "router_bias": "zipf(1.1) log-popularity", "global_batch": 1,
               "tokens_per_step": args.tokens}
    else:
        geom, L, slots = G.GPT_OSS_120B, 36, 2304
        stack = DecodeStack(geom, L, slots, device, zipf_s=None, router_bias=True)
        cfg = {"workload": "gpt-oss-120b-moe-stack", "layers": L, "experts": 128,
               "d_model": 2880, "d_ff": 2880, "top_k": 4, "pool_slots": slots,
               "pairs": L * 128, "quant": "4-bit affine g64 + bf16 proj bias",
               "activation": "clamped swiglu a=1.702 limit=7", "global_batch": 1,
               "tokens_per_step": args.tokens}
    return stack, cfg


MFMA_BF16_PEAK_TFS = 2500.0   # MI355X dense bf16 MFMA

# HBM bytes per launch measured with the L2 FETCH_SIZE / WRITE_SIZE counters
# (each scaled by its reading for a copy of known size); the summary and the
# commands that produced it are in the named file.
TRAFFIC_FILES = {("qwen3-48l", "persistent"): "profiles/stack_decode_qwen3_48l_traffic.md"}


def measured_traffic(workload, mode):
    import re
    name = TRAFFIC_FILES.get((workload, mode))
    if name is None:
        return None, None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), name)
    try:
        m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", open(path).read(), re.M)
    except OSError:
        return None, None
    return (int(m.group(1)), name) if m else (None, None)


def _prefill_roofline(flops, wbytes, block_s, block_ms):
    """The grouped block's roofline against its binding floor: the larger of
    the MFMA time (bf16 FLOPs at the dense peak) and the weight read (each
    distinct routed expert's payload once, at the HBM peak)."""
    t_mfma = flops / (MFMA_BF16_PEAK_TFS * 1e12)
    t_hbm = wbytes / (HBM_PEAK_GBS * 1e9)
    tflops = flops / block_s / 1e12
    gbs = wbytes / block_s / 1e9
    r = {"kernel": "expert block (group + gate/up + down + combine)", "traffic": None,
         "floors_us_per_step": {"mfma": round(t_mfma * 1e6, 1), "hbm": round(t_hbm * 1e6, 1)},
         "mfma_TFLOPs": round(tflops, 2), "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFS, 4),
         "weight_read_GBs": round(gbs, 1), "flops_per_step": flops,
         "avg_block_us": round(float(block_ms.mean()) * 1e3, 2)}
    if t_hbm >= t_mfma:
        r.update(bound="hbm", achieved=round(gbs, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                 frac=round(gbs / HBM_PEAK_GBS, 4))
    else:
        r.update(bound="mfma", achieved=round(tflops, 2), peak=MFMA_BF16_PEAK_TFS,
                 unit="TFLOP/s", frac=round(tflops / MFMA_BF16_PEAK_TFS, 4))
    return r


def prefill(args):
    """48 layers x 512 tokens through the grouped MFMA path: per layer the
    many-token router and the grouped expert block.  One step = the 512
    tokens through all 48 layers.  Reports tokens/s, the expert block's
    algorithmic TFLOP/s against the bf16 MFMA peak, and the bytes of the
    distinct experts the step reads against HBM peak."""
    import torch
    from moe_stream_amd import geometry as G
    from moe_stream_amd import ops, synth
    from moe_stream_amd.stack import PrefillStack
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, L, slots = args.tokens if args.tokens != 64 else 512, 48, 3072
    geom = G.QWEN3_30B_A3B
    stack = PrefillStack(geom, L, slots, T, dev, zipf_s=1.1)
    xs = synth.hidden_states(T, L, geom.d_model, dev, synth.SEED_BASE + 300)  # [T, L, D]
    x_step = xs.transpose(0, 1).contiguous()                                   # [L, T, D]
    stack.x_in.copy_(x_step)
    s = torch.cuda.current_stream()
    ev = []

    def step(timed=False):
        for Lx in range(L):
            if timed:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            nxt = Lx + 1 < L
            bufs = stack.bufs[Lx]
            ops.route(stack.x_in[Lx], stack.W[Lx], stack.bias[Lx], geom.routing,
                      geom.norm_topk_prob, stack.k,
                      W_next=stack.W[Lx + 1] if nxt else None,
                      bias_next=stack.bias[Lx + 1] if nxt else None,
                      k_pred=stack.k_pred, table=stack.table[Lx], bufs=bufs,
                      workspace=stack.route_ws)
            if timed:
                a.record(s)
            ops.ffn_grouped(stack.pool, bufs.slot_refs, bufs.scores, stack.x_in[Lx],
                            out=stack.y[Lx], workspace=stack.ffn_ws)
            if timed:
                b.record(s)
                ev.append((a, b))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step(timed=True)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ops.check_device_error()
    gpu_ms = e0.elapsed_time(e1)
    counts = stack.routed_counts()                     # [L, E] pairs per expert
    pairs = int(counts.sum())
    distinct = int((counts > 0).sum())
    flops = 2.0 * pairs * geom.d_model * geom.d_ff * 3   # gate, up, down
    block_ms = np.array([a.elapsed_time(b) for a, b in ev]).reshape(args.steps, L)
    block_s = block_ms.sum(1).mean() / 1e3
    tflops = flops / block_s / 1e12
    wbytes = distinct * geom.payload_bytes
    out = {"metric": "MoE prefill tok/s (512 tokens x 48 layers, grouped bf16 MFMA)",
           "value": round(T * args.steps / (gpu_ms / 1e3), 1), "unit": "tok/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(gpu_ms / args.steps, 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "qwen3-30b-a3b-moe-stack-prefill", "layers": L,
                      "tokens_per_layer": T, "top_k": stack.k, "pool_slots": slots,
                      "router_bias": "zipf(1.1) log-popularity",
                      "pairs_per_layer": pairs // L,
                      "distinct_experts_per_layer": round(distinct / L, 1),
                      "max_pairs_per_expert": int(counts.max()),
                      "parallelism": "none (1 GPU)"},
           "roofline": _prefill_roofline(flops, wbytes, block_s, block_ms),
           "expert_weight_GBs": round(wbytes / block_s / 1e9, 1),
           "wall_s": round(wall, 3)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_batch(stack, x_step, args.cpu_layers)
    return out


def verify(args):
    """A speculative verification step (gamma + 1 = 8 draft tokens, the
    multi-token call of spec.py:192-194) on the 48-layer Qwen3 stack: per
    layer the router for the 8 tokens and the expert block ops.ffn picks
    for 8 tokens (the grouped MFMA block; `--verify-block decode` runs the
    small-T decode kernels instead), each distinct expert's weights read once
    for every token routed to it, the 48 layers captured as one HIP graph.
    Interleaved in the same run: the same 8 tokens decoded one at a time by
    the whole-token kernel.  One step = one verification; value = verified
    tokens per second."""
    import torch
    from moe_stream_amd import geometry as G
    from moe_stream_amd import ops, synth
    from moe_stream_amd.stack import PrefillStack
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T = args.tokens if args.tokens != 64 else 8
    L, slots, geom = 48, 3072, G.QWEN3_30B_A3B
    stack = PrefillStack(geom, L, slots, T, dev, block=args.verify_block, zipf_s=1.1)
    n_steps = args.warmup + args.steps
    xs = synth.hidden_states(T * n_steps, L, geom.d_model, dev, synth.SEED_BASE + 500)
    xs = xs.view(n_steps, T, L, geom.d_model)
    stack.x_in.copy_(xs[0].transpose(0, 1))
    stack.capture()
    s = torch.cuda.current_stream()
    ver_ms, seq_ms, distinct = [], [], []
    for i in range(n_steps):
        x_step = xs[i].transpose(0, 1).contiguous()          # [L, T, D]
        a, b, c = (torch.cuda.Event(enable_timing=True) for _ in range(3))
        stack.x_in.copy_(x_step)
        a.record(s)
        stack.graph.replay()
        b.record(s)
        for t in range(T):                                   # one token at a time
            stack.token_persistent(xs[i, t], ordinary=True)
        c.record(s)
        c.synchronize()
        if i >= args.warmup:
            ver_ms.append(a.elapsed_time(b))
            seq_ms.append(b.elapsed_time(c))
            distinct.append(int((stack.routed_counts() > 0).sum()))
    stack.check_persistent()
    ops.check_device_error()
    ver, seq = float(np.median(ver_ms)), float(np.median(seq_ms))
    wbytes = float(np.mean(distinct)) * geom.payload_bytes
    block = stack.block
    out = {"metric": "MoE speculative verification tok/s (8 tokens x 48 layers)",
           "value": round(T / (ver / 1e3), 1), "unit": "tok/s", "n_gpus": 1,
           "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ver, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "qwen3-30b-a3b-moe-stack-verify", "layers": L,
                      "tokens_per_step": T, "top_k": stack.k, "pool_slots": slots,
                      "router_bias": "zipf(1.1) log-popularity",
                      "launch": "one HIP graph per step: route + the expert block per layer",
                      "expert_block": ("grouped bf16 MFMA" if block == "grouped"
                                       else "small-T decode kernels (pairs grouped by slot)"),
                      "parallelism": "none (1 GPU)"},
           "ms_per_verify": round(ver, 4),
           "ms_same_tokens_one_at_a_time": round(seq, 4),
           "speedup_vs_one_at_a_time": round(seq / ver, 3),
           "pairs_per_layer": T * stack.k,
           "distinct_experts_per_layer": round(float(np.mean(distinct)) / L, 2),
           "expert_bytes_per_verify": int(wbytes),
           "expert_GBs": round(wbytes / (ver * 1e-3) / 1e9, 1),
           "roofline": {"bound": "hbm", "kernel": "expert blocks of the step (router + "
                        "expert block per layer, one graph)",
                        "achieved": round(wbytes / (ver * 1e-3) / 1e9, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(wbytes / (ver * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "traffic": None,
                        "bytes": "distinct routed experts x payload, summed over layers"}}
    if not args.no_cpu:
        x_step = xs[n_steps - 1].transpose(0, 1).contiguous()
        out["cpu_baseline"] = cpu_baseline_batch(stack, x_step, args.cpu_layers)
    return out


def hbm_copy(args):
    """A 1 GiB device-to-device copy (1 GiB read + 1 GiB written per launch,
    4x the 256 MB last-level cache) and a 1 GiB sum (read only): the
    achievable HBM rates on this GPU, and the launch of known size that
    scales the L2 FETCH_SIZE / WRITE_SIZE counters into bytes."""
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)
    acc = src.view(torch.float32)
    res = {}
    for name, fn, nbytes in (("copy", lambda: dst.copy_(src), 2 * n),
                             ("read", lambda: acc.sum(), n)):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / args.steps
        res[name] = {"bytes_per_launch": nbytes, "avg_us": round(ms * 1e3, 1),
                     "GBs": round(nbytes / (ms * 1e-3) / 1e9, 1)}
    out = {"metric": "achievable HBM GB/s (device copy, device sum)",
           "value": res["copy"]["GBs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "higher_is_better": True, "dtype": "u8",
           "data": "synthetic", "config": {"workload": "hbm-copy-1GiB"},
           "peak": HBM_PEAK_GBS, **res}
    return out


def stream(args):
    """The streaming pool end to end: 48 Qwen3-shaped layers, a pinned host
    store of all 6144 records, a 2048-slot HBM pool with LFU eviction and
    lookahead-driven prefetch on a side stream, the per-layer engine loop
    with one host synchronisation per layer.  One step = `--tokens` decode
    tokens (default 256) after `--warmup` warm-up tokens.  Reports tok/s,
    pool hit rate, bytes copied per token and the measured H2D rate."""
    import torch
    from moe_stream_amd import geometry as G
    from moe_stream_amd import synth
    from moe_stream_amd.stack import StreamingStack
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    geom, L, slots = G.QWEN3_30B_A3B, 48, 2048
    n_tok = args.tokens if args.tokens != 64 else 256
    t_build = time.perf_counter()
    native = args.engine == "native"
    depths = tuple(int(d) for d in args.depths.split(","))
    st = StreamingStack(geom, L, slots, dev, zipf_s=1.1, native=native,
                        pool_layout=args.pool_layout, depths=depths)
    t_build = time.perf_counter() - t_build

    def bytes_read():
        return st.engine_counters()["bytes_read"] if native else st.pool.bytes_read
    xs = synth.hidden_states(n_tok + args.warmup, L, geom.d_model, dev, synth.SEED_BASE + 400)
    # pinned host -> HBM copy rate on this box (1 GiB, one hipMemcpyAsync)
    h = torch.empty(1 << 30, dtype=torch.uint8).pin_memory()
    d = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    d.copy_(h, non_blocking=True)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    d.copy_(h, non_blocking=True)
    b.record()
    torch.cuda.synchronize()
    h2d = (1 << 30) / (a.elapsed_time(b) * 1e-3) / 1e9
    del h, d
    for t in range(args.warmup):
        st.token(xs[t])
    torch.cuda.synchronize()
    s0 = st.pool.stats()
    b0 = bytes_read()
    y = torch.empty((L, geom.d_model), dtype=torch.bfloat16, device=dev)
    t0 = time.perf_counter()
    for t in range(args.warmup, args.warmup + n_tok):
        st.token(xs[t], out=y)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    from moe_stream_amd import ops
    ops.check_device_error()
    s1 = st.pool.stats()
    d = {k: s1[k] - s0[k] for k in ("total", "prefetch", "cache", "miss", "bail", "issued")}
    copied = bytes_read() - b0
    out = {"metric": "MoE streaming decode tok/s (bs=1, 48 layers, 2048-slot pool, "
                     "pinned host store)",
           "value": round(n_tok / wall, 2), "unit": "tok/s", "n_gpus": 1, "steps": 1,
           "warmup": args.warmup, "ms_per_step": round(wall * 1e3, 3),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic",
           "config": {"workload": "qwen3-30b-a3b-moe-stack-streaming", "layers": L,
                      "pool_slots": slots, "store_records": L * geom.n_experts,
                      "record_bytes": geom.record_bytes, "tokens": n_tok,
                      "evict": st.pool.evict, "prefetch": f"lookahead depths {','.join(map(str, depths))}, widen 1",
                      "pool_layout": args.pool_layout,
                      "fills": ("hipMemcpyAsync per record (copy engines)"
                                if args.pool_layout == "records" else "copy kernels"),
                      "engine": ("moe_engine_layer (library)" if native
                                 else "MoEBlock.streaming_call (Python)"),
                      "router_bias": "zipf(1.1) log-popularity",
                      "parallelism": "none (1 GPU)"},
           "hit_rate": round((d["prefetch"] + d["cache"]) / max(1, d["total"]), 4),
           "lookups": d, "bytes_copied_per_token": int(copied / n_tok),
           "lookahead_recall": round(st.recall(), 4), "h2d_GBs": round(h2d, 1),
           "build_s": round(t_build, 1)}
    # the loop's binding resource is the host link: the bytes copied per
    # second against the link's published rate (PCIe 5.0 x16, one direction)
    link = copied / wall / 1e9
    out["roofline"] = {"bound": "host link", "kernel": "slot fills (hipMemcpyAsync per "
                       "record, pinned host -> HBM)", "achieved": round(link, 2),
                       "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                       "frac": round(link / PCIE_PEAK_GBS, 4), "traffic": None,
                       "measured_h2d_GBs": round(h2d, 1)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(st, xs[args.warmup:], args.cpu_repeats)
    st.close()
    st.store.close()
    return out


def single_layer(args):
    """One Qwen3-30B-A3B-shaped MoE layer at batch 1 (128 experts in a
    256-slot pool at a seeded random placement, router softmax top-8 with
    renormalised scores, one bf16 N(0, 1) token per call): 64 calls of the
    layer on 64 different tokens (router kernel + the two decode kernels
    each) captured as one HIP graph, replayed back to back.  Reports the
    time per call and the HBM rate of its bytes (8 routed experts' payload +
    the router rows)."""
    import torch
    from moe_stream_amd import geometry as G
    from moe_stream_amd import ops, synth
    from moe_stream_amd.pool import SlotPool
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    geom = G.QWEN3_30B_A3B
    store = synth.make_store(geom, geom.n_experts, dev, synth.SEED_BASE + 600)
    pool = SlotPool(geom, 256, dev, store=store)
    perm = synth.slot_permutation(256, geom.n_experts, synth.SEED_BASE + 601)
    pool.fill(np.arange(geom.n_experts), perm)
    W, _ = synth.router_weights(geom, 1, dev, synth.SEED_BASE + 602)
    table = torch.tensor(perm, dtype=torch.int32, device=dev)
    n = 64
    xs = synth.hidden_states(n, 1, geom.d_model, dev, synth.SEED_BASE + 603)[:, 0]
    bufs = ops.RouteBuffers(1, geom.top_k, 0, dev)
    ws_r = torch.zeros(_lib_fn("moe_route_workspace")(1, geom.n_experts), dtype=torch.uint8,
                       device=dev)
    g = geom.c_geom()
    ws_f = torch.zeros(_lib_fn("moe_ffn_decode_workspace")(C.byref(g), 1, geom.top_k),
                       dtype=torch.uint8, device=dev)
    y = torch.empty((1, geom.d_model), dtype=torch.bfloat16, device=dev)

    def calls():
        for i in range(n):
            x = xs[i:i + 1]
            ops.route(x, W[0], None, geom.routing, geom.norm_topk_prob, geom.top_k,
                      table=table, bufs=bufs, workspace=ws_r)
            ops.ffn_decode(pool, bufs.slot_refs, bufs.scores, x, out=y, workspace=ws_f)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        calls()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls()
    reps = args.steps * n
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(args.steps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    ops.check_device_error()
    us = a.elapsed_time(b) * 1e3 / reps
    nbytes = geom.top_k * geom.payload_bytes + geom.n_experts * geom.d_model * 2
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"value": round(gbs, 1), "unit": "GB/s", "us_per_layer": round(us, 3),
           "layers_per_s": round(1e6 / us, 1),
           "config": {"workload": "qwen3-30b-a3b-moe-layer", "experts": 128, "d_model": 2048,
                      "d_ff": 768, "top_k": 8, "pool_slots": 256, "tokens": 1,
                      "launch": f"{n} layer calls (router + gate/up + down each) in one "
                                f"HIP graph, {args.steps} replays"},
           "roofline": {"bound": "hbm", "kernel": "route_kernel + ffn_gate_up_kernel + "
                        "ffn_down_kernel (one layer)", "achieved": round(gbs, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                        "bytes_per_layer": nbytes}}
    if not args.no_cpu:
        import torch as _t
        from oracle import cpu_block as CB
        from oracle import layout as OL
        threads = len(os.sched_getaffinity(0))
        _t.set_num_threads(threads)
        ex = {e: CB.Expert(OL.split_record(store[e].cpu().numpy(), geom.d_model, geom.d_ff,
                                           False)) for e in range(geom.n_experts)}
        Wc = W[0].float().cpu()
        xh = xs.float().cpu()
        ms = []
        for i in range(args.cpu_repeats + 3):
            t0 = time.perf_counter()
            CB.moe_layer(xh[i % n], Wc, None, lambda e: ex[e], geom.top_k, geom.routing,
                         geom.norm_topk_prob, "qwen3")
            if i >= 3:
                ms.append((time.perf_counter() - t0) * 1e3)
        med = float(np.median(ms))
        out["cpu_baseline"] = {"value": round(nbytes / (med * 1e-3) / 1e9, 3), "unit": "GB/s",
                               "us_per_layer": round(med * 1e3, 1), "cores": threads,
                               "kind": "port",
                               "label": "CPU restatement (not MLX): torch on the host cores",
                               "sample": f"{len(ms)} single-token layer calls (router + "
                                         "top-8 + 8 experts), 3 warm-up; median"}
    del pool, store
    return out


def _lib_fn(name):
    from moe_stream_amd import _lib
    return getattr(_lib.lib(), name)


def time_dominant_kernel(stack, xs, n_tok):
    """Average duration of the gate/up dequant-GEMV kernel, each launch
    bracketed by HIP events on the stream it runs on."""
    import torch
    from moe_stream_amd import _lib, ops
    L = _lib.lib()
    g = stack.geom.c_geom()
    view = stack.pool.c_view()
    s = torch.cuda.current_stream()
    sp = _lib.stream_ptr(s)
    pairs = []
    for t in range(n_tok):
        stack.x_in.copy_(xs[t])
        for Lx in range(stack.L):
            nxt = Lx + 1 < stack.L
            b = stack.bias[Lx] if stack.bias is not None else None
            bn = stack.bias[Lx + 1] if (stack.bias is not None and nxt) else None
            bufs = stack.bufs[Lx]
            ops.route(stack.x_in[Lx:Lx + 1], stack.W[Lx], b, stack.geom.routing,
                      stack.geom.norm_topk_prob, stack.k,
                      W_next=stack.W[Lx + 1] if nxt else None, bias_next=bn,
                      k_pred=stack.k_pred, table=stack.table[Lx], bufs=bufs,
                      workspace=stack.route_ws)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            _lib.check(L.moe_ffn_decode_up(C.byref(view), C.byref(g),
                                           bufs.slot_refs.data_ptr(),
                                           stack.x_in[Lx:Lx + 1].data_ptr(), 1, stack.k,
                                           stack.ffn_ws.data_ptr(), stack.ffn_ws.numel(), sp))
            e1.record(s)
            _lib.check(L.moe_ffn_decode_down(C.byref(view), C.byref(g),
                                             bufs.slot_refs.data_ptr(),
                                             bufs.scores.data_ptr(), 1, stack.k,
                                             stack.y[Lx:Lx + 1].data_ptr(), None,
                                             stack.ffn_ws.data_ptr(), stack.ffn_ws.numel(), sp))
            pairs.append((e0, e1))
    torch.cuda.synchronize()
    ms = [a.elapsed_time(b) for a, b in pairs]
    return float(np.mean(ms)), float(np.median(ms)), len(ms)


def _record(stack, idx):
    """Store record idx as host bytes (a device store or a pinned host store)."""
    arr = getattr(stack.store, "array", None)
    return arr[idx] if arr is not None else stack.store[idx].cpu().numpy()


def cpu_baseline_batch(stack, x_step, n_layers):
    """The many-token expert path on the host cores: oracle.cpu_block's
    moe_layer_batch (every token routed at once, each routed expert
    dequantised once and applied to all its rows by one fp32 matrix product,
    MLX's bf16 rounding points; not MLX), `n_layers` layer-blocks of the
    stack spread over its layers, each timed on its own with the routed
    experts read from the store before its timer starts.  tok/s = T tokens /
    (n_layers_of_stack x median layer-block time)."""
    import torch
    from oracle import cpu_block as CB
    from oracle import layout as OL
    g = stack.geom
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    kind = "gptoss" if g.has_proj_bias else "qwen3"
    T = x_step.shape[1]
    layers = np.linspace(0, stack.L - 1, n_layers).round().astype(int).tolist()
    ms = []
    for i, Lx in enumerate([layers[0]] + layers):       # the first run is a warm-up
        X = x_step[Lx].float().cpu()
        W = stack.W[Lx].float().cpu()
        b = None if stack.bias is None else stack.bias[Lx].float().cpu()
        ids, _ = CB.route_rows(X, W, b, g.top_k, g.routing, g.norm_topk_prob)
        ex = {int(e): CB.Expert(OL.split_record(_record(stack, Lx * stack.E + int(e)),
                                                g.d_model, g.d_ff, g.has_proj_bias))
              for e in torch.unique(ids).tolist()}
        t0 = time.perf_counter()
        CB.moe_layer_batch(X, W, b, lambda e: ex[e], g.top_k, g.routing,
                           g.norm_topk_prob, kind, g.alpha, g.limit)
        if i > 0:
            ms.append((time.perf_counter() - t0) * 1e3)
        del ex
    ms = np.array(ms)
    med = float(np.median(ms))
    return {"value": round(T / (stack.L * med * 1e-3), 3), "unit": "tok/s", "cores": threads,
            "kind": "port", "label": "CPU restatement (not MLX): torch on the host cores, "
            "experts dequantised once per layer-block",
            "layer_ms": {"median": round(med, 2), "min": round(float(ms.min()), 2),
                         "max": round(float(ms.max()), 2)},
            "sample": f"{len(ms)} layer-blocks of {T} tokens (router + top-{g.top_k} + the "
                      f"routed experts) at layers {layers}, 1 warm-up; tok/s = {T} / "
                      f"({stack.L} x median layer time)"}


def cpu_baseline(stack, xs, repeats, gpu_token=None):
    """The expert path on the host cores: oracle.cpu_block, a torch CPU
    restatement of the reference graph (router + top-k + the k-expert block,
    dequantise then fp32 matrix-vector products, MLX's bf16 rounding points;
    not MLX, which is not installed), on every visible core.

    `repeats` layer-blocks of the same stack, walking the layers of
    consecutive tokens (so the routed experts change from repeat to repeat),
    each timed on its own; median and p10/p90 over them, after 3 warm-up
    repeats.  The experts a repeat routes to are read from the store before
    its timer starts (the reference's pool holds them resident).  With
    `gpu_token(t)`, one GPU token runs before every CPU repeat, its launch
    timed by events, so the two arms interleave."""
    import torch
    from oracle import cpu_block as CB
    from oracle import layout as OL
    g = stack.geom
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    kind = "gptoss" if g.has_proj_bias else "qwen3"
    W = stack.W.float().cpu()
    B = None if stack.bias is None else stack.bias.float().cpu()
    xh = xs.float().cpu()
    cache = {}

    def expert(Lx, e):
        key = (Lx, e)
        if key not in cache:
            if len(cache) >= 64:
                cache.pop(next(iter(cache)))
            cache[key] = CB.Expert(OL.split_record(_record(stack, Lx * stack.E + e),
                                                   g.d_model, g.d_ff, g.has_proj_bias))
        return cache[key]

    cpu_ms, gpu_us = [], []
    warm = 3
    for r in range(repeats + warm):
        t, Lx = divmod(r, stack.L)
        t %= xh.shape[0]
        x = xh[t, Lx]
        b = None if B is None else B[Lx]
        ids, _ = CB.route(x, W[Lx], b, g.top_k, g.routing, g.norm_topk_prob)
        for e in ids.tolist():          # resident before the timer starts
            expert(Lx, e)
        if gpu_token is not None:
            us = gpu_token(t)
            if r >= warm:
                gpu_us.append(us)
        t0 = time.perf_counter()
        CB.moe_layer(x, W[Lx], b, lambda e: cache[(Lx, e)], g.top_k, g.routing,
                     g.norm_topk_prob, kind, g.alpha, g.limit)
        if r >= warm:
            cpu_ms.append((time.perf_counter() - t0) * 1e3)
    ms = np.array(cpu_ms)
    p10, med, p90 = np.percentile(ms, [10, 50, 90])

    def tok_s(layer_ms):
        return round(1e3 / (layer_ms * stack.L), 3)
    out = {"value": tok_s(med), "unit": "tok/s",
           "cores": threads, "kind": "port",
           "label": "CPU restatement (not MLX): torch on the host cores",
           "os_cpu_count": os.cpu_count(), "sched_affinity": threads,
           "torch_threads": torch.get_num_threads(),
           "layer_ms": {"median": round(med, 3), "p10": round(p10, 3), "p90": round(p90, 3)},
           "tok_s_p10_p90": [tok_s(p90), tok_s(p10)],
           "repeats": len(ms),
           "sample": f"{len(ms)} layer-blocks (router + top-k + {g.top_k} experts) of the "
                     f"same {stack.L}-layer stack, consecutive layers of "
                     f"{(repeats + warm - 1) // stack.L + 1} tokens, {warm} warm-up repeats; "
                     f"tok/s = 1 / ({stack.L} x median layer time)"}
    if gpu_us:
        q = np.percentile(np.array(gpu_us), [10, 50, 90])
        out["gpu_interleaved_us_per_token"] = {"median": round(q[1], 2), "p10": round(q[0], 2),
                                               "p90": round(q[2], 2), "n": len(gpu_us)}
    return out


def decode(args):
    """The decode stacks (bs=1, one token at a time): the 48-layer Qwen3
    stack (the headline) or the 36-layer gpt-oss stack."""
    import torch
    from moe_stream_amd import synth
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stack, cfg = workload(args, dev)
    xs = synth.hidden_states(args.tokens, stack.L, stack.geom.d_model, dev,
                             synth.SEED_BASE + 200)
    mode = args.mode
    if mode == "auto":
        mode = "persistent" if stack.persistent_preferred() else "graph"
    if mode == "persistent" and not stack.persistent_supported():
        mode = "graph"
    if mode == "graph":
        stack.capture()
    torch.cuda.synchronize()
    launch_ev = []          # (start, end) events around every persistent launch
    ordinary = args.launch == "ordinary"

    def step(timed=False):
        for t in range(args.tokens):
            if mode == "persistent":
                if timed:
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    stack.token_persistent(xs[t], ordinary=ordinary)
                    b.record()
                    launch_ev.append((a, b))
                else:
                    stack.token_persistent(xs[t], ordinary=ordinary)
            else:
                stack.run_token(xs[t], mode == "graph")

    def measure():
        for _ in range(args.warmup):
            step()
        for b in stack.bufs:
            b.miss.zero_()
        if mode == "persistent":
            stack.p_miss.zero_()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            step(timed=True)
        e1.record()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, e0.elapsed_time(e1)

    wall, gpu_ms = measure()
    from moe_stream_amd import _lib, ops
    launch_note = None
    if mode == "persistent":
        try:
            stack.check_persistent()
        except _lib.MoeError as e:
            if e.code != _lib.MOE_ERR_TIMEOUT or not ordinary:
                raise
            # another kernel held CUs: measure again with cooperative launches
            launch_note = "ordinary launch timed out; measured with cooperative launches"
            ordinary = False
            launch_ev.clear()
            wall, gpu_ms = measure()
            stack.check_persistent()
    ms_per_step = gpu_ms / args.steps
    tok_s = args.tokens * args.steps / (gpu_ms / 1e3)
    ops.check_device_error()
    if mode == "persistent":
        misses = int(stack.p_miss.sum().item())
    else:
        misses = int(sum(int(b.miss.item()) for b in stack.bufs))
    lookups = args.steps * args.tokens * stack.L * stack.k
    cfg["pool_hit_rate"] = round(1.0 - misses / lookups, 4)
    cfg["launch"] = {"persistent": ("one ordinary launch per token (all layers)" if ordinary
                                    else "one cooperative launch per token (all layers)"),
                     "graph": "one HIP graph per token, 3 launches per layer",
                     "eager": "3 launches per layer"}[mode]
    if launch_note:
        cfg["launch_note"] = launch_note
    cfg["parallelism"] = "none (1 GPU)"
    cfg["seq_len"] = 1

    router_bytes = (stack.L + (stack.L - 1)) * stack.E * stack.geom.d_model * 2
    if mode == "persistent":
        # the dominant kernel is the whole-token kernel: expert payload of the
        # routed experts + router and lookahead rows, per launch
        ms = np.array([a.elapsed_time(b) for a, b in launch_ev])
        avg_ms, med_ms, n = float(ms.mean()), float(np.median(ms)), len(ms)
        per_launch = stack.expert_bytes_per_token() + router_bytes
        kname = "stack_decode_kernel" if stack.geom.d_model == 2048 else "stack_wide_kernel"
    else:
        per_launch = stack.k * sum(c.nbytes for c in stack.geom.components
                                   if c.name.startswith(("gate_proj", "up_proj")))
        avg_ms, med_ms, n = time_dominant_kernel(stack, xs, min(args.profile_tokens, args.tokens))
        kname = "ffn_gate_up_kernel"
    achieved = per_launch / (avg_ms * 1e-3) / 1e9
    traffic, traffic_src = measured_traffic(args.workload, mode)
    roof = {"bound": "hbm", "kernel": kname, "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic, "traffic_source": traffic_src, "bytes_per_launch": per_launch,
            "avg_us": round(avg_ms * 1e3, 3), "median_us": round(med_ms * 1e3, 3),
            "launches": n}
    block_bytes = stack.expert_bytes_per_token()
    metric = ("MoE decode tok/s (bs=1, 48 layers) + gather_qmm achieved HBM GB/s vs peak"
              if args.workload == "qwen3-48l" else
              "MoE decode tok/s (bs=1, 36 layers, gpt-oss-120b shape) + achieved HBM GB/s vs peak")
    out = {"metric": metric,
           "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "bf16", "data": "synthetic",
           "config": cfg, "roofline": roof,
           "expert_bytes_per_token": block_bytes,
           "stack_expert_GBs": round(block_bytes * tok_s / 1e9, 1),
           "wall_s": round(wall, 3)}
    if not args.no_cpu:
        gs = torch.cuda.current_stream()

        def gpu_token(t):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(gs)
            if mode == "persistent":
                stack.token_persistent(xs[t], ordinary=ordinary)
            else:
                stack.run_token(xs[t], mode == "graph")
            b.record(gs)
            b.synchronize()
            return a.elapsed_time(b) * 1e3
        out["cpu_baseline"] = cpu_baseline(stack, xs, args.cpu_repeats, gpu_token)
        if mode == "persistent":
            stack.check_persistent()
    return out


def _sub_args(args, **kw):
    a = argparse.Namespace(**vars(args))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


# the other benchmark configurations, measured after the headline in the
# default run: (key, function, arguments); short step counts, bounded CPU samples
SECONDARY = (
    ("qwen3_layer", single_layer, dict(steps=4, warmup=1, cpu_repeats=60)),
    ("gptoss_36l", decode, dict(workload="gptoss-36l", mode="auto", tokens=16, steps=2,
                                warmup=1, cpu_repeats=24)),
    ("qwen3_prefill_512", prefill, dict(workload="qwen3-prefill", tokens=512, steps=2,
                                        warmup=1, cpu_layers=2)),
    ("qwen3_verify_8", verify, dict(workload="qwen3-verify", tokens=8, steps=4, warmup=1,
                                    verify_block="auto", cpu_layers=8)),
    ("qwen3_stream_256", stream, dict(workload="qwen3-stream", tokens=256, warmup=2,
                                      engine="native", pool_layout="records", depths="1",
                                      cpu_repeats=48)),
)


def secondaries(args):
    """Every other benchmark configuration, each with its roofline and a CPU
    baseline of the same configuration; a failure is reported in its entry."""
    import gc
    import torch
    res = {}
    for key, fn, kw in SECONDARY:
        t0 = time.perf_counter()
        print(f"[bench] {key} ...", file=sys.stderr, flush=True)
        try:
            r = fn(_sub_args(args, **kw))
        except Exception as e:          # report, keep the headline line
            r = {"error": f"{type(e).__name__}: {e}"}
        r["driver_s"] = round(time.perf_counter() - t0, 1)
        res[key] = r
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build runs the expert path on one GPU "
              "(a bs=1 decode stack is one independent replica per GPU); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    fn = {"qwen3-prefill": prefill, "qwen3-stream": stream, "hbm-copy": hbm_copy,
          "qwen3-verify": verify, "qwen3-layer": single_layer}.get(args.workload, decode)
    out = fn(args)
    if args.workload == "qwen3-48l" and not args.no_secondary:
        import gc
        import torch
        gc.collect()
        torch.cuda.empty_cache()
        out["secondary"] = secondaries(args)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
