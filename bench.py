#!/usr/bin/env python3
"""Bench: MoE-layer us/token and HBM GB/s, Qwen3-30B-A3B-shaped Q4_K/Q6_K decode.

One step = one decode token through all 48 stacked MoE layers (router tail,
grouped expert FFN, combine into the residual, and rms_norm between layers),
every layer with its own synthetic weights resident in HBM (18.8 GB), the
activation chain never leaving the device.  Inputs are resident before the
timed region starts.

Prints ONE JSON line (rank 0).  `value` is microseconds per MoE layer per token
(lower is better); `step_layer_us` gives p10 / p50 / p90 of single steps
(an event pair around each), per layer; `drop_in_layer_us` is the same layer
through hoard_moe_layer (one launch per layer, the entry point an engine calls
when attention runs between MoE layers); `roofline` covers the dominant
kernel, timed with a HIP event pair around each of its launches on the stream
it runs on;
`cpu_baseline` is the C restatement of ggml-CPU's algorithm for the same stage
on this host's cores.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
TYPE_NAMES = {11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}
MODEL_NAMES = {"qwen3_30b": "Qwen3-30B-A3B", "qwen3_next": "Qwen3-Next-80B-A3B", "olmoe": "OLMoE-1B-7B",
               "qwen35": "Qwen3.5-35B-A3B", "olmoe_q3": "OLMoE-1B-7B (Q3_K_M)"}
CPU_THREADS_MAX = 16  # the host-core share of one GPU on the measurement boxes


def metric_label(shape) -> str:
    """The headline metric's wording for the shape measured."""
    gu = TYPE_NAMES[shape.gate_type]
    return f"MoE-layer us/token + HBM GB/s (% of peak), {MODEL_NAMES[shape.name]}-shape {gu} decode"


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--shape", default="qwen3_30b", choices=["qwen3_30b", "qwen3_next", "olmoe", "qwen35", "olmoe_q3"])
    ap.add_argument("--layers", type=int, default=None, help="stacked layers (default: the shape's)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--decode-kernel", default="auto", choices=["auto", "xcd", "spread", "launches"],
                    help="one-launch decode kernel: expert-per-XCD, rows spread over all CUs, or auto; "
                         "'launches' runs the per-layer kernels (hoard_moe_layer's path) instead")
    ap.add_argument("--decode-launch", default="plain", choices=["cooperative", "plain"],
                    help="how the one-launch decode is launched: plain (HOARD_OPT_DECODE_LAUNCH 1) for a "
                         "caller that owns the device, as this benchmark does; cooperative (the library's "
                         "default) has the runtime guarantee co-residency and costs about 18 us more a launch")
    ap.add_argument("--phases", action="store_true", help="trace one-launch decode phases of one token")
    ap.add_argument("--pool", type=int, default=0, metavar="K",
                    help="slot-pool workload: K HBM slots per layer, all experts in pinned host memory, "
                         "routing from the seeded 512-token Zipf(0.8)+reuse trace")
    ap.add_argument("--pool-mode", default="both", choices=["both", "demand", "trace"],
                    help="demand: each layer's uploads are issued after its router has run and its selection "
                         "was read back (the engine's situation); trace: every layer's uploads are enqueued "
                         "ahead from the known trace, overlapping the previous layer's FFN; both: the two in "
                         "turn, `value` being the on-demand rate")
    ap.add_argument("--store", action="store_true",
                    help="with --pool: experts streamed from a GGUF file on local disk through the storage tier "
                         "(RAM tier of --ram experts, --readers parallel O_DIRECT reads) instead of pinned masters")
    ap.add_argument("--ram", type=int, default=256, help="storage tier: RAM-tier capacity in experts")
    ap.add_argument("--readers", type=int, default=8, help="storage tier: reads in flight")
    ap.add_argument("--store-dir", default="/tmp", help="storage tier: directory for the model file")
    ap.add_argument("--batch", type=int, default=0, metavar="M",
                    help="batched workload: M tokens per step (1..512), routed independently, grouped by expert; "
                         "up to 16 the verify-sized kernels, above that the prefill-sized sorted-pair units, "
                         "all on int8 MFMA")
    ap.add_argument("--batch-same", action="store_true",
                    help="with --batch: the M tokens of a step share one hidden, so every expert group holds "
                         "M tokens and runs on MFMA (the skewed end of the verify workload)")
    ap.add_argument("--no-extra", action="store_true",
                    help="headline run only: skip the other workloads carried on its line (Qwen3-Next decode, "
                         "16-token verify batch, 512-token prefill)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 5 device-to-device copies of BYTES (HBM counter calibration) and exit")
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_bytes(shape, kind: int, n_layer: int) -> int:
    """Algorithmic HBM bytes of one launch of each kernel for one token."""
    from hoard_amd import KERNEL_DECODE, KERNEL_DOWN, KERNEL_GATEUP, KERNEL_LAYER, KERNEL_ROUTER, expert_bytes
    s = shape
    n = s.n_embd
    if kind == KERNEL_DECODE:  # one launch runs every layer of the token
        return n_layer * s.bytes_per_token_layer()
    if kind == KERNEL_LAYER:  # one launch runs one layer
        return s.bytes_per_token_layer()
    if kind == KERNEL_ROUTER:
        return 4 * s.n_expert * n + 4 * n + 4 * n  # W, x in, fx out
    sh = bool(s.n_ff_shexp)
    if kind == KERNEL_GATEUP:
        b = s.n_used * (expert_bytes(s.gate_type, s.n_ff, n) + expert_bytes(s.up_type, s.n_ff, n))
        if sh:
            b += expert_bytes(s.sh_gate_type, s.n_ff_shexp, n) + expert_bytes(s.sh_up_type, s.n_ff_shexp, n)
            b += 4 * n  # shared gate row
        return b + 4 * n + 4 * (s.n_used * s.n_ff + s.n_ff_shexp)  # fx in, h out
    if kind == KERNEL_DOWN:
        b = s.n_used * expert_bytes(s.down_type, n, s.n_ff)
        if sh:
            b += expert_bytes(s.sh_down_type, n, s.n_ff_shexp)
        return b + 4 * (s.n_used * s.n_ff + s.n_ff_shexp) + 8 * n  # h in, res in, out
    raise ValueError(kind)


PHASES = ["layer_start", "x_gathered", "router_rows_q8x", "router_rows_q8x_", "logits_gathered_topk",
          "loads_issued", "gateup_rows_landed", "h_published", "h_gathered_q8h", "down_y_published",
          "y_gathered_x_published", "y_gathered_x_published_"]
# the rows-spread kernel's stamps (decode_spread.hip), in time order
PHASES_SPREAD = ["layer_start", "x_gathered", "logits_gathered", "softmax_summed", "wave_candidates",
                 "topk", "gateup_rows_landed", "wave0_gateup_done", "h_gathered", "q8h", "down_done",
                 "combined_x_published"]


def phase_breakdown(lib, h, step, H, names=PHASES):
    """Per-phase time of the one-launch decode: for each boundary, when the slowest
    workgroup reached it, relative to the previous boundary (median over layers)."""
    H.check(lib.hoard_moe_phase_trace(h, 1))
    step()
    buf = np.zeros(512 * 256 * H.TRACE_PHASES, dtype=np.uint64)
    nl = ctypes.c_int()
    H.check(lib.hoard_moe_phase_trace_read(h, ctypes.c_void_p(buf.ctypes.data), buf.size, ctypes.byref(nl)))
    H.check(lib.hoard_moe_phase_trace(h, 0))
    if nl.value == 0:
        return None
    t = buf[: nl.value * 256 * H.TRACE_PHASES].reshape(nl.value, 256, H.TRACE_PHASES).astype(np.int64)
    reach = t.max(axis=1)                      # [layer, phase]: slowest workgroup
    reach[:, 0] = t[:, :, 0].min(axis=1)       # layer start: first workgroup
    # phases 7..9 are skipped by workgroups without an expert; they hold 0 then
    d = np.diff(reach, axis=1) * 10e-3         # 100 MHz ticks -> us
    med = np.median(d[1:] if nl.value > 1 else d, axis=0)
    out = {f"{names[i]}->{names[i + 1]}": round(float(med[i]), 3) for i in range(len(names) - 1)}
    out["layer_total"] = round(float(np.median((reach[1:, -1] - reach[1:, 0]) * 10e-3)) if nl.value > 1 else 0.0, 3)
    return out


def copy_probe(nbytes: int):
    """A plain copy kernel of known size, for scaling the FETCH_SIZE / WRITE_SIZE
    counters of the decode kernel to bytes."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": nbytes, "copies": 5}), flush=True)


def h2d_probe_gbps(nbytes: int = 1 << 30) -> float:
    """Pinned host -> HBM copy bandwidth (the link that bounds the slot pool)."""
    import torch
    src = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nbytes, dtype=torch.uint8, device="cuda:0")
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        dst.copy_(src, non_blocking=True)
    e1.record()
    torch.cuda.synchronize()
    return 3 * nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9


def run_pool(args, shape, n_layer):
    """Slot-pool workload: one token = every layer's pool step (LRU bookkeeping,
    uploads of the misses on side streams) and expert FFN + combine, with the
    selection taken from the seeded synthetic trace.  Two ways to fetch:
    * on demand, as in the engine, where layer l's experts are known only once
      its router has run (notes/MEMORY-FLOW.md:58-64 of the reference): the
      router runs, its selection is read back (a synchronisation), then the
      misses are uploaded and the FFN waits for them;
    * trace-known prefetch: the host enqueues every layer's pool step ahead of
      the device, so the uploads of layer l+1 overlap the FFN of layer l, and
      each FFN waits only for its own layer's uploads.
    Both start from an empty pool and see the same hits and misses."""
    import torch

    import hoard_amd as H
    from hoard_amd import workloads as W
    lib = H.load_library()
    K = args.pool
    t0 = time.perf_counter()
    cfg = shape.cfg(n_layer, K, 1)
    h = ctypes.c_void_p()
    H.check(lib.hoard_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
    store = path = None
    if args.store:
        import tempfile

        sys.path.insert(0, str(ROOT / "tests"))
        from gguf_writer import write_stage_streaming

        from hoard_amd.gguf import GGUFWeights
        from hoard_amd.store import ExpertStore
        tmpdir = tempfile.mkdtemp(prefix="hoard_store_", dir=args.store_dir)
        path = Path(tmpdir) / f"{shape.name}_{n_layer}l.gguf"
        hl = W.make_layer(shape, args.seed, 0)
        write_stage_streaming(path, shape, n_layer, lambda l: W.fill_layer(hl, args.seed, l) if l else hl,
                              "qwen3moe" if shape.renorm else "olmoe")
        del hl
        log(f"[bench] wrote {path} ({path.stat().st_size / 1e9:.1f} GB, fsynced) in {time.perf_counter() - t0:.1f} s")
        store = ExpertStore.from_gguf(path, readers=args.readers, ram_experts=args.ram, direct=True, pinned=True)
        H.check(lib.hoard_moe_attach_store(h, store.h))
        with GGUFWeights(path) as g:
            for l in range(n_layer):
                H.check(lib.hoard_moe_set_layer_weights(h, l, ctypes.byref(g.layer_weights(l))))
        where = f"streamed from {path} through a RAM tier of {store.stats().ram_experts} experts"
    else:
        hl = W.make_layer(shape, args.seed, 0)
        for l in range(n_layer):
            if l:
                W.fill_layer(hl, args.seed, l)
            H.check(lib.hoard_moe_set_layer_weights(h, l, ctypes.byref(hl.weights())))
        del hl
        where = "in pinned host memory"
    log(f"[bench] pool K={K}: {n_layer} layers of {shape.name} {where} "
        f"({n_layer * shape.n_expert * shape.expert_bytes() / 1e9:.1f} GB), "
        f"{n_layer * K * shape.expert_bytes() / 1e9:.2f} GB of HBM slots, in {time.perf_counter() - t0:.1f} s")
    trace = W.routing_trace(shape, args.seed, tokens=512, n_layer=n_layer)
    T = trace.sel.shape[0]
    warm = min(args.warmup, T - 1)
    steps = min(args.steps, T - warm)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    copy_stream = torch.cuda.Stream()
    sp, cp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p(copy_stream.cuda_stream)
    n_tok = 16
    hid = [W.make_hidden(shape, args.seed, 0, t) for t in range(n_tok)]
    fx_d = torch.stack([torch.from_numpy(f) for f, _ in hid]).to(dev)
    x_d = torch.stack([torch.from_numpy(r) for _, r in hid]).to(dev)
    w_d = torch.from_numpy(trace.w).to(dev)
    slots_d = torch.empty((n_layer, shape.n_used), dtype=torch.int32, device=dev)
    sel_h = np.ascontiguousarray(trace.sel)

    sel_scratch = torch.empty(shape.n_used, dtype=torch.int32, device=dev)
    w_scratch = torch.empty(shape.n_used, dtype=torch.float32, device=dev)

    def token(t, on_demand):
        x = x_d[t % n_tok]
        fx = ctypes.c_void_p(fx_d[t % n_tok].data_ptr())
        for l in range(n_layer):
            if on_demand:
                # the layer's router runs and its selection is read back before the
                # fetch can start (the reference's D2H of sel, src/run_moe_stream.cpp:367);
                # the selection used is the trace's
                H.check(lib.hoard_moe_route(h, l, fx, ctypes.c_void_p(sel_scratch.data_ptr()),
                                            ctypes.c_void_p(w_scratch.data_ptr()), sp))
                stream.synchronize()
            H.check(lib.hoard_moe_pool_ensure(h, l, ctypes.c_void_p(sel_h[t, l].ctypes.data), None,
                                              ctypes.c_void_p(slots_d[l].data_ptr()), sp, cp))
            H.check(lib.hoard_moe_ffn_combine(h, l, fx, ctypes.c_void_p(slots_d[l].data_ptr()),
                                              ctypes.c_void_p(w_d[t, l].data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                              ctypes.c_void_p(x.data_ptr()), sp))

    def timed(on_demand):
        """Warm-up tokens, then the timed ones, from an empty pool; (ms per token, stats)."""
        H.check(lib.hoard_moe_set_option(h, H.OPT_POOL_NAIVE, 1))  # toggling naive mode empties every layer's slots
        H.check(lib.hoard_moe_set_option(h, H.OPT_POOL_NAIVE, 0))
        for t in range(warm):
            token(t, on_demand)
        torch.cuda.synchronize()
        H.check(lib.hoard_moe_reset_stats(h))
        if store is not None:
            store.reset_stats()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for t in range(warm, warm + steps):
            token(t, on_demand)
        e1.record(stream)
        torch.cuda.synchronize()
        st = H.MoeStats()
        H.check(lib.hoard_moe_get_stats(h, ctypes.byref(st)))
        # the events span the device's whole timeline, the idle gaps of the on-demand
        # read-backs included
        return e0.elapsed_time(e1) / steps, st

    modes = {"both": [False, True], "trace": [False], "demand": [True]}[args.pool_mode]
    runs = {}
    for on_demand in modes:
        runs[on_demand] = timed(on_demand)
        sst_mode = store.stats() if store is not None else None
        runs[on_demand] += (sst_mode,)
    lib.hoard_moe_destroy(h)
    if store is not None:
        store.close()
        import shutil
        shutil.rmtree(path.parent, ignore_errors=True)
    probe = h2d_probe_gbps()

    def summary(ms, st, sst):
        bytes_tok = st.bytes_h2d / steps
        out = {"tokens_per_s": round(1000.0 / ms, 3), "ms_per_token": round(ms, 4),
               "hit_rate": round(st.hits / max(1, st.reqs), 4), "requests": int(st.reqs), "misses": int(st.misses),
               "h2d_bytes_per_token": int(bytes_tok), "h2d_gbps": round(bytes_tok / (ms * 1e-3) / 1e9, 2),
               "link_frac": round(bytes_tok / (ms * 1e-3) / 1e9 / probe, 4)}
        if sst is not None:
            out["store"] = {
                "requests": int(sst.requests), "ram_hits": int(sst.ram_hits), "file_reads": int(sst.file_reads),
                "ram_hit_rate": round(sst.ram_hits / max(1, sst.requests), 4),
                "read_gbps": round(sst.bytes_read / max(1, sst.read_ns), 3),
                "read_ms_per_token": round(sst.read_ns / 1e6 / steps, 3),
                "direct": int(sst.direct),
            }
        return out

    main_mode = True if True in runs else False
    ms, st, sst = runs[main_mode]
    head = summary(ms, st, sst)
    result = {
        "metric": "slot-pool decode tokens/s, Qwen3-30B-A3B-shape Q4_K, K-slot HBM LRU over pinned host experts",
        "value": head["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": head["ms_per_token"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K/q6_K weights x q8_K activations (int8 dot), f32 router/accumulate",
        "data": "synthetic weights; routing from a seeded 512-token trace: Zipf(0.8) popularity per layer, "
                "40% reuse of the previous 4 tokens' experts",
        "config": {"workload": f"{shape.name}: {n_layer} layers, K={K} slots per layer, "
                               f"all {shape.n_expert} experts per layer in pinned host memory",
                   "pool_k": K, "layers": n_layer,
                   "fetch": "on demand: each layer's uploads issued after its router ran and the selection was "
                            "read back" if main_mode else
                            "trace-known prefetch: every layer's uploads enqueued ahead from the trace"},
        "h2d_probe_gbps": round(probe, 2),
    }
    result.update({k: v for k, v in head.items() if k not in ("tokens_per_s", "ms_per_token")})
    if main_mode and False in runs:
        result["trace_known_prefetch"] = summary(*runs[False])
    if store is not None:
        result["metric"] = ("slot-pool decode tokens/s, Qwen3-30B-A3B-shape Q4_K, K-slot HBM LRU over a RAM tier "
                            "streamed from the model file")
        result["config"]["workload"] = (f"{shape.name}: {n_layer} layers, K={K} slots per layer, RAM tier of "
                                        f"{sst.ram_experts} experts, the rest read from a GGUF on local disk")
        result["config"].update(ram_experts=int(sst.ram_experts), readers=args.readers)
    print(json.dumps(result), flush=True)


MFMA_MIN_TOKENS = 12  # smallest expert group the batched kernels run on MFMA (kMfmaMinTokens)
MFMA_INT8_PEAK = 5.0e15  # MI355X dense int8 MFMA ops/s


def load_layers(lib, h, shape, n_layer, seed):
    """Every layer's synthetic weights into the handle (one host layer regenerated in place)."""
    import hoard_amd as H
    from hoard_amd import workloads as W
    hl = W.make_layer(shape, seed, 0)
    for l in range(n_layer):
        if l:
            W.fill_layer(hl, seed, l)
        H.check(lib.hoard_moe_set_layer_weights(h, l, ctypes.byref(hl.weights())))
    del hl


def run_batched(args, shape, n_layer):
    """Batched workload on a handle of its own (see batched_measure)."""
    import hoard_amd as H
    lib = H.load_library()
    M = args.batch
    cfg = shape.cfg(n_layer, 0, M)
    h = ctypes.c_void_p()
    H.check(lib.hoard_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
    load_layers(lib, h, shape, n_layer, args.seed)
    result = batched_measure(lib, h, shape, n_layer, M, args.steps, args.warmup, args.seed, args.batch_same)
    lib.hoard_moe_destroy(h)
    print(json.dumps(result), flush=True)


def batched_measure(lib, h, shape, n_layer, M, steps, warm, seed, same=False):
    """Batched workload: one step = M tokens through every layer, each layer one
    hoard_moe_forward_batched (router for M tokens, grouping by expert, gate/up
    and down per expert group, ordered combine).  Each token keeps its own
    normalised hidden as the layer input (fx); the residual chain is in place.
    The handle holds n_layer layers of `shape` and takes M tokens."""
    import torch

    import hoard_amd as H
    from hoard_amd import workloads as W
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    n_groups = 8
    toks = [[W.make_hidden(shape, seed, 0, g * M + (0 if same else t)) for t in range(M)]
            for g in range(n_groups)]
    fx_d = torch.stack([torch.stack([torch.from_numpy(f) for f, _ in grp]) for grp in toks]).to(dev)
    x_d = torch.stack([torch.stack([torch.from_numpy(r) for _, r in grp]) for grp in toks]).to(dev)
    sel_d = torch.empty((n_layer, M, shape.n_used), dtype=torch.int32, device=dev)

    def step(i):
        g = i % n_groups
        fx, x = ctypes.c_void_p(fx_d[g].data_ptr()), ctypes.c_void_p(x_d[g].data_ptr())
        for l in range(n_layer):
            H.check(lib.hoard_moe_forward_batched(h, l, M, fx, x, x, ctypes.c_void_p(sel_d[l].data_ptr()),
                                                  None, sp))

    for i in range(warm):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(warm, warm + steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    us_layer = ms * 1000.0 / n_layer
    # unique experts per layer of the last step, from its routing
    sel = sel_d.cpu().numpy()
    uniq = np.array([len(np.unique(sel[l])) for l in range(n_layer)])
    hist = np.concatenate([np.bincount(sel[l].ravel(), minlength=shape.n_expert) for l in range(n_layer)])
    H.check(lib.hoard_moe_profile(h, 1))
    step(warm + steps)
    kt = H.KernelTimes()
    H.check(lib.hoard_moe_profile_read(h, ctypes.byref(kt)))
    H.check(lib.hoard_moe_profile(h, 0))
    # a shared expert (and its gate row) is read once per layer and taken by every token
    eb, sb = shape.expert_bytes(), shape.shared_bytes() + (4 * shape.n_embd if shape.n_ff_shexp else 0)
    layer_bytes = float(uniq.mean()) * eb + sb + 4 * shape.n_expert * shape.n_embd + M * 4 * shape.n_embd * 2
    kb = H.KERNEL_BATCHED
    bat_us = kt.total_ms[kb] / max(1, kt.launches[kb]) * 1000.0
    bat_bytes = float(uniq.mean()) * eb + sb + M * 4 * shape.n_embd * 2
    gbps = bat_bytes / bat_us / 1e3
    macs_per_pair = 3 * shape.n_ff * shape.n_embd
    sh_pairs = M * n_layer if shape.n_ff_shexp else 0  # the shared expert's group: all M tokens
    int8_ops = 2 * macs_per_pair * (int(hist.sum()) + sh_pairs)
    # verify-sized batches run groups of MFMA_MIN_TOKENS or more on MFMA; prefill-sized
    # ones (more than 32 tokens) run every group on MFMA
    mfma_groups = hist >= (MFMA_MIN_TOKENS if M <= 32 else 1)
    sh_mfma = sh_pairs if (M > 32 or M >= MFMA_MIN_TOKENS) else 0
    mfma_ops = 2 * macs_per_pair * (int(hist[mfma_groups].sum()) + sh_mfma)
    result = {
        "metric": f"batched MoE-layer us per step of {M} tokens + HBM GB/s, "
                  f"{MODEL_NAMES[shape.name]}-shape {TYPE_NAMES[shape.gate_type]}",
        "value": round(us_layer, 3), "unit": "us/layer", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K/q6_K weights x q8_K activations (int8 dot / MFMA), f32 router/accumulate",
        "data": "synthetic weights and N(0,1) hiddens, every token routed independently",
        "config": {"workload": f"{shape.name}: {n_layer} layers, {M} tokens per step, all experts resident",
                   "tokens_per_step": M, "layers": n_layer,
                   "path": "verify-sized: expert groups of 32 token places" if M <= 32 else
                           "prefill-sized: pairs sorted by expert, 64-pair units on MFMA"},
        "tokens_per_s": round(M * 1000.0 / ms, 2),
        "unique_experts_per_layer": round(float(uniq.mean()), 2),
        "tokens_per_expert_max": int(hist.max()),
        "expert_token_histogram": {str(c): int((hist == c).sum()) for c in range(1, int(hist.max()) + 1)},
        "layer_bytes": int(layer_bytes),
        "layer_hbm_gbps": round(layer_bytes / (us_layer * 1e3), 1),
        "roofline": {"bound": "hbm", "kernel": "batched_experts", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": None, "avg_us": round(bat_us, 3)},
        # expert groups of 12 or more tokens run on int8 MFMA, smaller ones on
        # the per-token int8 dot (MFMA_MIN_TOKENS in the batched kernels)
        "expert_groups": {"per_token_dot": int(((hist > 0) & ~mfma_groups).sum()),
                          "mfma": int(((hist > 0) & mfma_groups).sum())},
        # int8 operations of the expert products (2 per multiply-add: gate, up and
        # down of every (token, expert) pair), the MFMA share of them, and that
        # share's rate against MI355X's dense int8 peak of 5.0 POP/s
        "mfma": {"int8_ops_per_step": int(int8_ops), "mfma_ops_per_step": int(mfma_ops),
                 "mfma_tops": round(mfma_ops / (ms * 1e-3) / 1e12, 2),
                 "utilization": round(mfma_ops / (ms * 1e-3) / MFMA_INT8_PEAK, 5), "peak_tops": MFMA_INT8_PEAK / 1e12},
    }
    if same:
        result["data"] = "synthetic weights; the M tokens of a step share one N(0,1) hidden (every group M tokens)"
        result["config"]["workload"] += ", tokens sharing one hidden"
    return result




def decode_measure(lib, h, shape, n_layer, steps, warm, seed):
    """One-launch decode of one token through n_layer layers (plain launch),
    timed as the headline: an event pair around `steps` steps, and an event pair
    around each launch for the kernel's own duration."""
    import torch

    import hoard_amd as H
    from hoard_amd import workloads as W
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    eps = ctypes.c_float(W.RMS_EPS)
    H.check(lib.hoard_moe_set_option(h, H.OPT_DECODE_LAUNCH, 1))
    xs = torch.stack([torch.from_numpy(W.make_hidden(shape, seed, 0, t)[1]) for t in range(steps + warm)]).to(dev)

    def step(i):
        H.check(lib.hoard_moe_decode(h, 0, n_layer, ctypes.c_void_p(xs[i].data_ptr()), eps, sp))

    for i in range(warm):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(warm, warm + steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    assert torch.isfinite(xs).all().item(), f"non-finite {shape.name} decode output"
    H.check(lib.hoard_moe_profile(h, 1))
    for i in range(warm, warm + steps):
        step(i)
    kt = H.KernelTimes()
    H.check(lib.hoard_moe_profile_read(h, ctypes.byref(kt)))
    H.check(lib.hoard_moe_profile(h, 0))
    kd = H.KERNEL_DECODE
    us = ms * 1000.0 / n_layer
    lb = shape.bytes_per_token_layer()
    out = {"us_per_layer": round(us, 3), "tokens_per_s": round(1000.0 / ms, 2), "layer_bytes": lb,
           "layer_hbm_gbps": round(lb / (us * 1e3), 1), "layer_hbm_frac": round(lb / (us * 1e3) / HBM_PEAK_GBPS, 4)}
    if kt.launches[kd]:
        kus = kt.total_ms[kd] / kt.launches[kd] * 1000.0
        out["kernel"] = {"name": "decode_persistent", "avg_us_per_launch": round(kus, 3),
                         "us_per_layer": round(kus / n_layer, 3),
                         "gbps": round(n_layer * lb / kus / 1e3, 1),
                         "frac": round(n_layer * lb / kus / 1e3 / HBM_PEAK_GBPS, 4)}
    del xs
    return out


def extra_summary(r):
    """The keys of a batched_measure result carried on the headline line."""
    return {"us_per_layer": r["value"], "tokens_per_step": r["config"]["tokens_per_step"],
            "tokens_per_s": r["tokens_per_s"], "layer_hbm_gbps": r["layer_hbm_gbps"],
            "layer_hbm_frac": round(r["layer_hbm_gbps"] / HBM_PEAK_GBPS, 4),
            "batched_call_hbm_frac": r["roofline"]["frac"],
            "unique_experts_per_layer": r["unique_experts_per_layer"], "tokens_per_expert_max": r["tokens_per_expert_max"],
            "expert_groups": r["expert_groups"], "mfma_utilization": r["mfma"]["utilization"],
            "mfma_tops": r["mfma"]["mfma_tops"], "path": r["config"]["path"]}


def measured_traffic(shape, kernel: str, n_layer: int):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-probe factor), or
    None when no summary covers this kernel and workload."""
    f = ROOT / "profiles" / f"traffic_{kernel}_{shape.name}.json"
    if not f.exists():
        return None
    t = json.loads(f.read_text())
    if t.get("kernel") != kernel or t.get("layers") != n_layer:
        return None
    return int(t["hbm_bytes_per_launch"])


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(shape, seed: int, budget_s: float, n_layer: int):
    """The oracle (C restatement of ggml-CPU's algorithm: f32 router, Q8_K of the
    activations, integer super-block dots, OpenMP over rows) on host cores.  The
    sample cycles through every layer of the stack, each with its own weights and
    4 hiddens, so the weights stream from DRAM (only the experts those hiddens
    select are generated: several GB, far above the last-level cache)."""
    import oracle
    from hoard_amd import workloads as W
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(avail, CPU_THREADS_MAX))
    n_hid = 4
    layers, toks, touched = [], [], 0
    for l in range(n_layer):
        hid = [W.make_hidden(shape, seed, 1000 + l, t) for t in range(n_hid)]
        router = W.make_router(shape, seed, l)
        need = set()
        for fx, _ in hid:
            need |= set(oracle.route(router, fx, shape.n_expert, shape.n_used, shape.renorm)[0].tolist())
        layers.append(W.make_layer(shape, seed, l, experts=sorted(need)))
        toks.append(hid)
        touched += len(need) * shape.expert_bytes() + router.nbytes
    lib = oracle.lib()

    def run(nthreads, budget):
        lib.orc_set_num_threads(nthreads)
        oracle.moe_layer(layers[0], *toks[0][0])  # warm
        done, t0 = 0, time.perf_counter()
        while True:
            l = done % n_layer
            oracle.moe_layer(layers[l], *toks[l][(done // n_layer) % n_hid])
            done += 1
            el = time.perf_counter() - t0
            if el >= budget and done >= n_layer:
                return el / done * 1e6, done, el

    us, done, el = run(threads, budget_s)
    us1, done1, el1 = run(1, budget_s / 3)
    lb = shape.bytes_per_token_layer()
    return {
        "value": round(us, 2), "unit": "us/layer", "cores": threads, "kind": "port",
        "sample": f"{done} token-layers cycling the {n_layer} layers of {shape.name} (4 hiddens each, "
                  f"{touched / 1e9:.1f} GB of weights touched), OpenMP over rows, {el:.1f} s",
        "cpu_model": cpu_model(), "cores_available": avail,
        "tokens_per_s": round(1e6 / (us * n_layer), 3),
        "dram_gbps": round(lb / us / 1e3, 2),
        "one_thread": {"value": round(us1, 2), "unit": "us/layer", "sample": f"{done1} token-layers, {el1:.1f} s",
                       "tokens_per_s": round(1e6 / (us1 * n_layer), 3)},
        "what": "ggml-algorithm restatement (ggml itself is not available offline)",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the MoE stage would shard by expert id; see the design notes)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_probe:
        copy_probe(args.copy_probe)
        return

    import hoard_amd as H
    from hoard_amd import workloads as W

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    lib = H.load_library()
    shape = W.SHAPES[args.shape]
    n_layer = args.layers or shape.n_layer
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pool:
        run_pool(args, shape, n_layer)
        return
    if args.batch:
        run_batched(args, shape, n_layer)
        return

    # ---- resident weights: 48 independent synthetic layers -------------------
    t0 = time.perf_counter()
    # the default run also measures the batched workloads on the same weights
    extras = not args.no_extra and args.shape == "qwen3_30b" and args.layers is None and args.decode_kernel == "auto"
    cfg = shape.cfg(n_layer, 0, 512 if extras else 1)
    h = ctypes.c_void_p()
    H.check(lib.hoard_moe_create(ctypes.byref(cfg), ctypes.byref(h)))
    if args.decode_kernel == "launches":
        dk_opt = H.DECODE_AUTO
        H.check(lib.hoard_moe_set_option(h, H.OPT_PERSISTENT_DECODE, 0))
    else:
        dk_opt = {"auto": H.DECODE_AUTO, "xcd": H.DECODE_XCD, "spread": H.DECODE_SPREAD}[args.decode_kernel]
        H.check(lib.hoard_moe_set_option(h, H.OPT_DECODE_KERNEL, dk_opt))
    H.check(lib.hoard_moe_set_option(h, H.OPT_DECODE_LAUNCH, 1 if args.decode_launch == "plain" else 0))
    hl = W.make_layer(shape, args.seed, 0)
    for l in range(n_layer):
        if l:
            W.fill_layer(hl, args.seed, l)
        w = hl.weights()
        H.check(lib.hoard_moe_set_layer_weights(h, l, ctypes.byref(w)))
    del hl
    log(f"[bench] {n_layer} layers of {shape.name} resident ({n_layer * shape.n_expert * shape.expert_bytes() / 1e9:.1f} GB "
        f"experts) in {time.perf_counter() - t0:.1f} s")

    # ---- one input token per step, already on device --------------------------
    steps, warm = args.steps, args.warmup
    xs = torch.stack([torch.from_numpy(W.make_hidden(shape, args.seed, 0, t)[1]) for t in range(steps + warm)]).to(dev)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    eps = ctypes.c_float(W.RMS_EPS)

    def step(i):
        H.check(lib.hoard_moe_decode(h, 0, n_layer, ctypes.c_void_p(xs[i].data_ptr()), eps, sp))

    for i in range(warm):
        step(i)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(warm, warm + steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = ev0.elapsed_time(ev1) / steps
    us_layer = ms_per_step * 1000.0 / n_layer
    assert torch.isfinite(xs).all().item(), "non-finite decode output"

    # ---- the drop-in path: hoard_moe_layer per layer (fx given, residual chained) --
    fxs = torch.stack([torch.from_numpy(W.make_hidden(shape, args.seed, 0, t)[0]) for t in range(8)]).to(dev)
    xl = xs[:8].clone()

    def layer_step(i):
        x = xl[i % 8]
        fx = ctypes.c_void_p(fxs[i % 8].data_ptr())
        for l in range(n_layer):
            H.check(lib.hoard_moe_layer(h, l, fx, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(x.data_ptr()),
                                        None, None, sp))

    for i in range(warm):
        layer_step(i)
    torch.cuda.synchronize()
    ev0.record(stream)
    for i in range(steps):
        layer_step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    drop_in_us = ev0.elapsed_time(ev1) * 1000.0 / (steps * n_layer)
    assert torch.isfinite(xl).all().item(), "non-finite hoard_moe_layer output"

    # ---- the spread of single steps: an event pair around each of `steps` steps --
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i, (e0, e1) in enumerate(evs):
        e0.record(stream)
        step(warm + i)
        e1.record(stream)
    torch.cuda.synchronize()
    step_us = np.array([e0.elapsed_time(e1) * 1000.0 for e0, e1 in evs])
    step_pct = {f"p{q}": round(float(np.percentile(step_us, q)) / n_layer, 3) for q in (10, 50, 90)}

    # ---- per-kernel durations: a HIP event pair around every launch, on its stream --
    H.check(lib.hoard_moe_profile(h, 1))
    for i in range(warm, warm + steps):
        step(i)
    kt = H.KernelTimes()
    H.check(lib.hoard_moe_profile_read(h, ctypes.byref(kt)))
    H.check(lib.hoard_moe_profile(h, 0))
    kernels = {}
    for kind, name in H.KERNEL_NAMES.items():
        n = kt.launches[kind]
        if n:
            avg_us = kt.total_ms[kind] / n * 1000.0
            b = kernel_bytes(shape, kind, n_layer)
            kernels[name] = {"launches": int(n), "avg_us": round(avg_us, 3), "bytes": b,
                             "gbps": round(b / avg_us / 1e3, 1)}
    dom = max(kernels, key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    dk = kernels[dom]

    layer_bytes = shape.bytes_per_token_layer()
    layer_gbps = layer_bytes / (us_layer * 1e3)
    wtypes = "/".join(dict.fromkeys(TYPE_NAMES[t] for t in (shape.gate_type, shape.up_type, shape.down_type)))
    result = {
        "metric": metric_label(shape),
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{wtypes.replace('Q', 'q')} weights x q8_K activations (int8 dot), f32 router/accumulate",
        "data": f"synthetic (seeded random {wtypes} super-blocks, f32 router, N(0,1) hidden)",
        "config": {"workload": f"{shape.name}: {n_layer} stacked MoE layers, batch-1 decode, "
                               f"hidden {shape.n_embd}, {shape.n_expert} experts top-{shape.n_used}, "
                               f"ff {shape.n_ff}, all experts resident in HBM",
                   "tokens_per_step": 1, "layers": n_layer},
        "tokens_per_s": round(1000.0 / ms_per_step, 2),
        "step_layer_us": step_pct,
        "layer_hbm_gbps": round(layer_gbps, 1),
        "layer_hbm_frac": round(layer_gbps / HBM_PEAK_GBPS, 4),
        "layer_bytes": layer_bytes,
        "drop_in_layer_us": round(drop_in_us, 3),
        "drop_in_layer_hbm_frac": round(layer_bytes / (drop_in_us * 1e3) / HBM_PEAK_GBPS, 4),
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": dk["gbps"], "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(dk["gbps"] / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(shape, dom, n_layer),
                     "algorithmic_bytes": dk["bytes"],
                     "basis": "algorithmic bytes per launch / mean duration of a hipEvent pair recorded around "
                              "each launch on its stream (launch gaps included)"},
    }
    persistent = ctypes.c_int()
    H.check(lib.hoard_moe_get_option(h, H.OPT_PERSISTENT_AVAILABLE, ctypes.byref(persistent)))
    avail = ctypes.c_int()
    H.check(lib.hoard_moe_get_option(h, H.OPT_DECODE_KERNELS_AVAILABLE, ctypes.byref(avail)))
    spread = dk_opt == H.DECODE_SPREAD or (dk_opt == H.DECODE_AUTO and not avail.value & 1)
    result["config"]["decode_path"] = (
        (f"one {args.decode_launch} launch per token, " + ("expert rows spread over all CUs" if spread
                                                           else "one expert per XCD"))
        if "decode_persistent" in kernels else
        "one launch per layer (router, gate/up and down workgroups in ticket order)" if "layer_fused" in kernels else
        "router, gate/up and down+combine launches per layer")
    if args.phases:
        ph = phase_breakdown(lib, h, lambda: step(warm), H, PHASES_SPREAD if spread else PHASES)
        if ph:
            result["phases_us"] = ph
            for k_, v_ in ph.items():
                log(f"[phase] {k_:40s} {v_:8.3f} us")
    if extras:
        # the verify-sized batch (16 tokens) and a prompt-sized one (512 tokens) on
        # the same 48 resident layers, each token routed independently
        xsteps, xwarm = max(1, min(steps, 20)), min(warm, 5)
        for M, key in ((16, "batched_m16"), (512, "prefill_m512")):
            r = batched_measure(lib, h, shape, n_layer, M, xsteps, xwarm, args.seed)
            result[key] = extra_summary(r)
            log(f"[bench] {key}: {r['value']:.2f} us/layer, {r['layer_hbm_gbps'] / 1e3:.2f} TB/s, "
                f"{r['unique_experts_per_layer']:.1f} unique experts")
    # release every device object before the next handle and the CPU leg: the
    # handle, then torch's tensors
    lib.hoard_moe_destroy(h)
    del xs, xl, fxs
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if extras:
        # the Qwen3-Next-shaped decode: 48 layers of 512 experts, top-10 and a
        # shared expert (50 GB resident), one plain launch of the rows-spread kernel
        nx = W.QWEN3_NEXT
        t1 = time.perf_counter()
        cfg2 = nx.cfg(nx.n_layer)
        h2 = ctypes.c_void_p()
        H.check(lib.hoard_moe_create(ctypes.byref(cfg2), ctypes.byref(h2)))
        load_layers(lib, h2, nx, nx.n_layer, args.seed)
        log(f"[bench] {nx.n_layer} layers of {nx.name} resident in {time.perf_counter() - t1:.1f} s")
        r2 = decode_measure(lib, h2, nx, nx.n_layer, max(1, min(steps, 20)), min(warm, 5), args.seed)
        lib.hoard_moe_destroy(h2)
        r2["workload"] = (f"{nx.name}: {nx.n_layer} stacked MoE layers, batch-1 decode, {nx.n_expert} experts "
                          f"top-{nx.n_used} + a shared expert, ff {nx.n_ff}, all resident")
        r2["decode_path"] = "one plain launch per token, expert rows spread over all CUs"
        result["qwen3_next_decode"] = r2
        log(f"[bench] qwen3_next_decode: {r2['us_per_layer']:.2f} us/layer ({r2['layer_hbm_frac']:.3f} of peak)")
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(shape, args.seed, args.cpu_seconds, n_layer)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
