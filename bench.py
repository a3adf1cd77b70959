#!/usr/bin/env python3
"""Benchmark of the candle-moe hot path on one MI355X.

Metric: fused-MoE µs & TFLOP/s (Qwen3 h4096 E8 k2 bf16);
topk-softmax µs. One step = one MoE layer over one batch of synthetic
tokens already resident in HBM: topk-softmax over the router logits
[T, E], then FusedMoE::forward (zeroed output, grouping, gate/up GEMM with
SwiGLU, down GEMM with the weighted combine). Default workload: Qwen3
T=32768, H=4096, I=1536, E=8, k=2, bf16 (BASELINE config 4 at its largest T).

Prints ONE JSON line. `value` is TFLOP/s of the whole step (algorithmic
MoE FLOPs = T*k*6*H*I for Qwen3, T*k*4*H*I for Nomic). `roofline` is for the
dominant kernel (the gate/up GEMM), timed with HIP events on the stream it
runs on (candle_moe_profile_begin_slots: only that launch is bracketed in the
timed region; the per-kernel breakdown comes from a separate untimed pass). `cpu_baseline` times the CPU oracle (the
candle-native per-expert loop, a port) on a bounded token sample.

    python bench.py [--steps K] [--warmup W] [--workload qwen3|nomic|q30b|router|fp8]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "candle-moe_amd"))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/f16 MFMA
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0

WORKLOADS = {
    # BASELINE config 4 (headline): Qwen3 SwiGLU
    "qwen3": dict(T=32768, H=4096, I=1536, E=8, k=2, moe_type=0, act="silu", dtype="bf16", zipf=0.0),
    # Nomic fc1 -> GELU -> fc2
    "nomic": dict(T=32768, H=768, I=3072, E=8, k=2, moe_type=1, act="gelu", dtype="bf16", zipf=0.0),
    # Qwen3-30B-A3B-shaped, Zipf-skewed routing
    "q30b": dict(T=4096, H=2048, I=768, E=128, k=8, moe_type=0, act="silu", dtype="bf16", zipf=1.1),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="qwen3", choices=sorted(WORKLOADS) + ["router", "fp8"],
                    help="MoE layer (qwen3 headline, nomic, q30b), router alone, or fp8: bf16 against fp8 "
                         "expert weights only (the decode GEMMs, and whole prefill calls with their GEMMs)")
    ap.add_argument("--tokens", type=int, default=0, help="override T")
    ap.add_argument("--fp8-shape", default="", choices=["", "qwen3_T16", "qwen3_T64", "q30b_T1", "q30b_T16", "nomic_T16"],
                    help="fp8 workload: this decode shape only (no prefill calls), e.g. for a per-shape kernel trace")
    ap.add_argument("--dtype", default="", choices=["", "bf16", "f16", "f32"])
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-sample", type=int, default=32768,
                    help="tokens in the CPU-baseline sample (0 = skip; default: the whole batch)")
    ap.add_argument("--tile", type=int, default=0, choices=[0, 1, 5, 7, 12, 14, 15, 16, 17, 18],
                    help="GEMM kernel: 0 auto, 1 register-staged 128x128, 5 LDS-DMA 128x128, 7 LDS-DMA 256x256 "
                         "8 waves, 12 32-row (decode), 14 128x256 two workgroups per CU, 15/16 f32 32-row / 128-row, "
                         "17 fp8 register-operand decode kernel (--workload fp8), 18 16-bit decode kernels")
    ap.add_argument("--combine", type=int, default=0, choices=[0, 1, 2], help="0 auto, 1 pairs, 2 expert sets")
    ap.add_argument("--graph", action="store_true",
                    help="also time the step captured once in a CUDA (HIP) graph and replayed (graph_ms_per_step)")
    ap.add_argument("--no-router-shapes", dest="router_shapes", action="store_false",
                    help="skip the topk-softmax config-2 shapes reported next to the MoE step")
    ap.add_argument("--no-packed", dest="packed", action="store_false",
                    help="skip the step on pre-packed (K-contiguous) weights reported next to the headline")
    ap.add_argument("--no-decode", dest="decode", action="store_false",
                    help="skip the decode steps (router + forward at small T, graph-replayed) reported next to the "
                         "headline step")
    ap.add_argument("--no-fp8-decode", dest="fp8_decode", action="store_false",
                    help="skip the decode GEMM timings with bf16 against fp8 expert weights")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="before the warmup, run 3 plain copy kernels of MIB MiB (read MIB, write MIB; "
                         "the reference point that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


def copy_calibration(torch, dev, mib):
    """A plain streaming kernel of known traffic: b = -a over `mib` MiB of f32
    (reads exactly mib MiB, writes exactly mib MiB)."""
    n = (mib << 20) // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(a, out=b)
    torch.cuda.synchronize()
    del a, b


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the hot path is a single-device kernel "
                                   "set; run with --gpus 1 (sharding design: DESIGN.md)"}))
        sys.exit(2)

    import torch

    import candle_moe as cm

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = cm.lib()
    cm.set_tile_policy(args.tile)
    cm.set_combine_policy(args.combine)

    if args.workload == "router":
        return bench_router_only(args, torch, cm, dev)
    if args.workload == "fp8":
        res = bench_fp8_decode(torch, cm, dev, args)
        pre = None if args.fp8_shape else bench_fp8_prefill(torch, cm, dev, args)
        gu = [v["bf16"]["gemm_gate_up"] / v["fp8"]["gemm_gate_up"] for v in res.values()]
        print(json.dumps({"metric": "decode GEMM time, bf16 over fp8 e4m3 expert weights", "value": round(min(gu), 3),
                          "unit": "x (gate/up GEMM, worst shape)", "n_gpus": 1, "higher_is_better": True,
                          "data": "synthetic", "config": {"workload": "fp8 decode GEMMs"}, "fp8_decode": res,
                          "fp8_prefill": pre}))
        return None

    wl = dict(WORKLOADS[args.workload])
    if args.tokens:
        wl["T"] = args.tokens
    if args.dtype:
        wl["dtype"] = args.dtype
    T, H, I, E, k = wl["T"], wl["H"], wl["I"], wl["E"], wl["k"]
    qwen3 = wl["moe_type"] == 0
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[wl["dtype"]]
    act = {"silu": cm.Activation.Silu, "gelu": cm.Activation.Gelu, "relu": cm.Activation.Relu}[wl["act"]]

    # synthetic inputs (torch's seeded GPU generator), weights N(0, 0.02) in the API layout
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    x = torch.randn((T, H), generator=g, device=dev).to(tdt)
    gate = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(tdt)
    up = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(tdt)
    down = (torch.randn((E, I, H), generator=g, device=dev) * 0.02).to(tdt) if qwen3 else None
    logits = torch.randn((T, E), generator=g, device=dev)
    if wl["zipf"]:
        ranks = torch.randperm(E, generator=torch.Generator().manual_seed(args.seed)).double() + 1
        p = ranks ** (-wl["zipf"])
        logits += torch.log(p / p.sum()).float().to(dev)[None, :]
    topk_w = torch.empty((T, k), dtype=torch.float32, device=dev)
    topk_i = torch.empty((T, k), dtype=torch.int32, device=dev)
    tok_ei = torch.empty((T, k), dtype=torch.int32, device=dev)
    moe = cm.FusedMoE.new(E, k, act)
    torch.cuda.synchronize()
    if args.copy_calibration:
        copy_calibration(torch, dev, args.copy_calibration)

    def step():
        cm.apply_topk_softmax_inplace(logits, topk_w, topk_i, tok_ei)
        return moe.forward(x, gate, up, down, topk_w, topk_i, wl["moe_type"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    L.candle_moe_profile_slot_name.restype = ctypes.c_char_p

    def slot_times(nslots):
        ms = (ctypes.c_double * nslots)()
        cnt = (ctypes.c_int * nslots)()
        cm.check(L.candle_moe_profile_end(ms, cnt, nslots))
        return {L.candle_moe_profile_slot_name(s).decode(): round(1000.0 * ms[s] / cnt[s], 3)
                for s in range(nslots) if cnt[s]}

    # timed region: HIP events around the dominant kernel only (the gate/up
    # GEMM), so that event records do not sit between the other launches
    nslots = L.candle_moe_profile_begin()
    cm.check(L.candle_moe_profile_end(None, None, 0))
    g1_slot = [L.candle_moe_profile_slot_name(s).decode() for s in range(nslots)].index("gemm_gate_up")
    L.candle_moe_profile_begin_slots(1 << g1_slot)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    timed = slot_times(nslots)
    # per-kernel breakdown: a separate, untimed pass with events around every launch
    L.candle_moe_profile_begin()
    for _ in range(min(args.steps, 10)):
        out = step()
    torch.cuda.synchronize()
    kernels = slot_times(nslots)
    kernels["gemm_gate_up"] = timed.get("gemm_gate_up", kernels.get("gemm_gate_up", 0.0))

    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    graph_ms = None
    if args.graph:
        # capture stream warmed first (the library's workspace is per stream);
        # the last replay is checked against an eager step
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            gout = step()
        for _ in range(args.warmup):
            graph.replay()
        torch.cuda.synchronize()
        g0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        graph_ms = (time.perf_counter() - g0) * 1000.0 / args.steps
        ref = step().float()
        torch.cuda.synchronize()
        rms = float(ref.pow(2).mean().sqrt())
        if not torch.allclose(gout.float(), ref, rtol=2e-2, atol=2e-2 * rms):
            graph_ms = None
    # the drop-in path: what the reference's Rust caller runs per call
    # (Tensor::zeros of the output, /root/reference/src/lib.rs:296, then the
    # fused_moe symbol adding into it, ffi.rs:35), timed the same way
    dropin = bench_dropin(torch, L, x, gate, up, down, topk_w, topk_i, wl, act, args)
    router = bench_router_shapes(torch, cm, dev, args) if args.router_shapes else None
    decode = bench_decode(torch, cm, dev, args) if args.decode else None
    packed = (bench_packed(torch, cm, dev, args, x, gate, up, down, logits, topk_w, topk_i, tok_ei, wl)
              if args.packed and wl["dtype"] in ("bf16", "f16") else None)
    fp8 = bench_fp8_decode(torch, cm, dev, args) if args.fp8_decode else None

    c = 6 if qwen3 else 4
    flops = float(T) * k * c * H * I
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_F32_TFLOPS if wl["dtype"] == "f32" else PEAK_BF16_TFLOPS

    # dominant kernel: gate/up (Qwen3: x.[G|U], 2*P*H*2I flops) or fc1 (Nomic: 2*P*H*I)
    g1_us = kernels.get("gemm_gate_up", 0.0)
    g1_flops = float(T) * k * (4 if qwen3 else 2) * H * I
    g1_achieved = g1_flops / (g1_us * 1e-6) / 1e12 if g1_us else 0.0
    topk_us = kernels.get("topk_softmax", 0.0)
    topk_bytes = T * E * 4 + T * k * 12
    traffic = load_traffic(args.workload, wl, args.tile)

    cpu = None
    if args.cpu_sample > 0:
        cpu = cpu_baseline(torch, x, gate, up, down, topk_w, topk_i, wl, min(args.cpu_sample, T))

    line = {
        "metric": "fused-MoE µs & TFLOP/s (Qwen3 h4096 E8 k2 bf16); topk-softmax µs",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": "synthetic (torch seeded GPU RNG: x ~ N(0,1), weights ~ N(0,0.02), logits ~ N(0,1))",
        "config": {
            "workload": f"{args.workload}-moe layer: topk-softmax [{T},{E}] k={k} + fused MoE T={T} H={H} I={I} "
                        f"E={E} k={k} {'SwiGLU' if qwen3 else 'fc1-' + wl['act'] + '-fc2'} {wl['dtype']}",
            "tokens": T, "hidden": H, "intermediate": I, "experts": E, "top_k": k,
            "moe_type": wl["moe_type"], "activation": wl["act"], "zipf_bias": wl["zipf"], "seed": args.seed,
            "parallelism": "single GPU",
        },
        "fused_moe_us": round(1000.0 * ms_per_step - topk_us, 1),
        "topk_softmax_us": topk_us,
        "topk_softmax_gbs": round(topk_bytes / (topk_us * 1e-6) / 1e9, 1) if topk_us else None,
        "kernels_us": kernels,
        "graph_ms_per_step": round(graph_ms, 4) if graph_ms else None,
        "dropin_fused_moe": dropin,
        "topk_softmax_config2": router,
        "decode": decode,
        "packed_weights": packed,
        "fp8_decode": fp8,
        "kernels_note": "HIP-event averages per launch: gemm_gate_up from the timed steps (the only kernel "
                        "bracketed there), the others from an untimed pass of up to 10 steps with every "
                        "launch bracketed",
        "roofline": {
            "kernel": "gemm_gate_up" if qwen3 else "gemm_fc1",
            "bound": "mfma",
            "achieved": round(g1_achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(g1_achieved / peak, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    del out


def load_traffic(workload, wl, tile):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 --pmc measurement (profiles/traffic.json: FETCH_SIZE and
    WRITE_SIZE scaled by a plain 1 GiB copy), or None when the workload,
    token count or GEMM kernel differs from the measured one."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        rec = d.get(workload)
        if rec and rec.get("tokens") == wl["T"] and wl["dtype"] == "bf16" and tile == 0:
            return rec.get("bytes_per_launch")
    except (OSError, ValueError):
        pass
    return None


def cpu_baseline(torch, x, gate, up, down, topk_w, topk_i, wl, S):
    """CPU oracle (candle-native per-expert loop, bf16 per-op rounding, f32
    matmul accumulation) on the first S tokens with all weights."""
    import numpy as np

    import oracle as O

    dt = {"bf16": O.BF16, "f16": O.F16, "f32": O.F32}[wl["dtype"]]

    def host(t):
        if t is None:
            return None
        t = t.contiguous().cpu()
        if t.dtype in (torch.bfloat16, torch.float16):
            return t.view(torch.int16).numpy().view(np.uint16)
        return t.numpy()

    xs = host(x[:S])
    G, U, D = host(gate), host(up), host(down)
    w = topk_w[:S].cpu().numpy()
    idx = topk_i[:S].cpu().numpy().astype(np.uint32)
    host_cpus = len(os.sched_getaffinity(0))
    # every CPU this process may run on, unless the environment limits the
    # OpenMP threads (the GPU boxes set OMP_NUM_THREADS to their per-GPU share)
    threads = min(host_cpus, int(os.environ.get("OMP_NUM_THREADS", "0")) or host_cpus)
    act = {"silu": O.SILU, "gelu": O.GELU, "relu": O.RELU}[wl["act"]]
    t0 = time.perf_counter()
    O.fused_moe(xs, G, U, D, w, idx, E=wl["E"], k=wl["k"], act=act, moe_type=wl["moe_type"], dtype=dt,
                mode=O.MODE_CANDLE, nthreads=threads)
    dt_s = time.perf_counter() - t0
    c = 6 if wl["moe_type"] == 0 else 4
    flops = float(S) * wl["k"] * c * wl["H"] * wl["I"]
    return {
        "value": round(flops / dt_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "host_cpus": host_cpus,
        "host_cpus_online": os.cpu_count(),
        "cpu_model": cpu_model(),
        "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
        "kind": "port",
        "sample": f"{'all' if S == wl['T'] else 'first'} {S} of {wl['T']} tokens with all {wl['E']} experts' "
                  f"weights; candle-native per-expert loop (oracle/oracle.c, per-op {wl['dtype']} rounding); "
                  f"{dt_s:.2f} s wall on {threads} OpenMP threads (one per CPU of this process's affinity set "
                  f"of {host_cpus}, capped by OMP_NUM_THREADS)",
    }


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def bench_dropin(torch, L, x, gate, up, down, topk_w, topk_i, wl, act, args):
    """ms per call of the reference caller's sequence: a zeroed [T, H] output
    (torch.zeros, a fill kernel) then the raw fused_moe symbol, which adds into
    it; warm library workspace, same inputs as the step."""
    T, H = x.shape
    I = gate.shape[2]
    dt = {"f16": 0, "bf16": 1, "f32": 2}[wl["dtype"]]
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call():
        out = torch.zeros((T, H), dtype=x.dtype, device=x.device)
        L.fused_moe(p(x), p(gate), p(up), p(down), p(topk_w), p(topk_i), p(out), T, H, I, wl["E"], wl["k"],
                    int(act), wl["moe_type"], dt, stream)
        return out

    for _ in range(max(2, args.warmup)):
        call()
    torch.cuda.synchronize()
    n = max(5, args.steps // 2)
    t0 = time.perf_counter()
    for _ in range(n):
        call()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / n
    return {"ms_per_call": round(ms, 4),
            "note": "torch.zeros([T,H]) + the raw fused_moe symbol accumulating into it (the reference caller's "
                    "per-call work); the step above uses FusedMoE::forward, whose last kernel writes every output "
                    "element instead"}


def bench_router_shapes(torch, cm, dev, args):
    """topk-softmax at BASELINE config 2 (f32 logits N(0,1); [32768,8] k2,
    [32768,64] k6, [32768,128] k8 and the skewed [32768,8] k2 with a per-expert
    N(0, 2) bias): GPU µs per call from 50 calls captured in one graph and
    replayed, rotating over logits buffers that exceed the 256 MB last-level
    cache (cold), and the achieved GB/s of T*E*4 + T*k*12 bytes."""
    res = {}
    for name, T, E, k, skew in [("32768x8k2", 32768, 8, 2, 0.0), ("32768x64k6", 32768, 64, 6, 0.0),
                                ("32768x128k8", 32768, 128, 8, 0.0), ("32768x8k2_skewed", 32768, 8, 2, 2.0)]:
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + E)
        nbuf = max(1, (512 << 20) // (T * E * 4))
        bias = torch.randn((E,), generator=g, device=dev) * skew
        logits = [torch.randn((T, E), generator=g, device=dev) + bias[None, :] for _ in range(nbuf)]
        w = torch.empty((T, k), device=dev)
        i = torch.empty((T, k), dtype=torch.int32, device=dev)
        ei = torch.empty((T, k), dtype=torch.int32, device=dev)
        for _ in range(3):
            cm.apply_topk_softmax_inplace(logits[0], w, i, ei)
        torch.cuda.synchronize()
        cm.apply_topk_softmax_inplace(logits[49 % nbuf], w, i, ei)
        ref = (w.clone(), i.clone(), ei.clone())
        gus = graph_us(torch, lambda: [cm.apply_topk_softmax_inplace(logits[s % nbuf], w, i, ei) for s in range(50)],
                       50, 20, lambda: torch.equal(w, ref[0]) and torch.equal(i, ref[1]) and torch.equal(ei, ref[2]))
        nbytes = T * E * 4 + T * k * 12
        res[name] = {"us": round(gus, 2) if gus else None,
                     "gbs": round(nbytes / (gus * 1e-6) / 1e9, 1) if gus else None,
                     "hbm_frac": round(nbytes / (gus * 1e-6) / 1e9 / PEAK_HBM_GBS, 4) if gus else None}
        del logits
    return res


def bench_packed(torch, cm, dev, args, x, gate, up, down, logits, topk_w, topk_i, tok_ei, wl):
    """The step on pre-packed weights (the opt-in K-contiguous format,
    candle_moe_fused_moe_packed; never the headline, which runs the drop-in
    layout) next to the same step on the API layout through the drop-in
    fused_moe symbol: topk-softmax, a zeroed output (both add into it) and
    the call. ms per step, the kernels' µs per launch (HIP events around
    every launch, a separate pass) and the gate/up GEMM's TFLOP/s for each
    layout. hipblaslt_nk: the gate/up-sized dense GEMM [T*k, H] x [H, 2I]
    through torch.matmul (hipBLASLt) with the weight K-contiguous ([2I, H],
    x @ W^T), the library's figure for the packed layout on this GPU."""
    L = cm.lib()
    T, H, I, E, k = wl["T"], wl["H"], wl["I"], wl["E"], wl["k"]
    qwen3 = wl["moe_type"] == 0
    act = {"silu": 0, "gelu": 1, "relu": 2}[wl["act"]]
    dt = {"f16": 0, "bf16": 1}[wl["dtype"]]
    gp = cm.pack_weights(gate)
    upk = cm.pack_weights(up) if qwen3 else up
    dp = cm.pack_weights(down) if qwen3 else None
    out = torch.zeros((T, H), dtype=x.dtype, device=dev)
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    g1_flops = float(T) * k * (4 if qwen3 else 2) * H * I

    def measure(call):
        def step():
            cm.apply_topk_softmax_inplace(logits, topk_w, topk_i, tok_ei)
            out.zero_()
            call()

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1000.0 / args.steps
        nslots = L.candle_moe_profile_begin()
        for _ in range(min(args.steps, 10)):
            step()
        torch.cuda.synchronize()
        msv = (ctypes.c_double * nslots)()
        cnt = (ctypes.c_int * nslots)()
        cm.check(L.candle_moe_profile_end(msv, cnt, nslots))
        kern = {L.candle_moe_profile_slot_name(s_).decode(): round(1000.0 * msv[s_] / cnt[s_], 3)
                for s_ in range(nslots) if cnt[s_]}
        return {"ms_per_step": round(ms, 4), "kernels_us": kern,
                "gate_up_tflops": round(g1_flops / (kern["gemm_gate_up"] * 1e-6) / 1e12, 1)}

    res = {"note": "steps include out.zero_(): both calls add into their output",
           "packed": measure(lambda: cm.fused_moe_packed(x, gp, upk, dp, topk_w, topk_i, out, E, k, act,
                                                         wl["moe_type"])),
           "api_layout": measure(lambda: L.fused_moe(p(x), p(gate), p(up), p(down), p(topk_w), p(topk_i), p(out),
                                                     T, H, I, E, k, act, wl["moe_type"], dt, stream))}
    del gp, upk, dp, out
    torch.cuda.empty_cache()
    # hipBLASLt reference: [T*k, H] x [H, 2I] with the weight stored [2I, H]
    a = torch.randn((T * k, H), device=dev).to(torch.bfloat16)
    w = (torch.randn((2 * I if qwen3 else I, H), device=dev) * 0.02).to(torch.bfloat16)
    for _ in range(3):
        c = a @ w.t()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(10):
        c = a @ w.t()
    ev[1].record()
    torch.cuda.synchronize()
    us = 1000.0 * ev[0].elapsed_time(ev[1]) / 10
    res["hipblaslt_nk"] = {"us": round(us, 1), "tflops": round(g1_flops / (us * 1e-6) / 1e12, 1),
                           "shape": f"[{T * k},{H}] x [{H},{w.shape[0]}] (weight [{w.shape[0]},{H}])"}
    del a, w, c
    torch.cuda.empty_cache()
    return res


def bench_decode(torch, cm, dev, args):
    """Decode steps at BASELINE's small batches: topk-softmax over [T, E]
    logits then FusedMoE::forward, as the headline step, 20 steps in a row
    rotating over bf16 weight copies that exceed the 256 MB last-level cache
    (cold weights). `graph_us`: per step, the 20 steps captured once in a HIP
    graph and replayed (every replay's outputs checked against the eager
    ones); `eager_us`: per step between two events around the 20 launches
    from the host. `weight_frac`: the touched experts' weight bytes at 8 TB/s
    over graph_us (the roofline of a decode step: every touched expert's
    weights streamed once)."""
    res = {}
    for wname, T in [("qwen3", 8), ("qwen3", 64), ("q30b", 1), ("q30b", 16), ("nomic", 16)]:
        wl = WORKLOADS[wname]
        H, I, E, k = wl["H"], wl["I"], wl["E"], wl["k"]
        qwen3 = wl["moe_type"] == 0
        act = {"silu": cm.Activation.Silu, "gelu": cm.Activation.Gelu, "relu": cm.Activation.Relu}[wl["act"]]
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + 100 + T)
        nw = 3 if qwen3 else 2
        ncopy = max(2, -(-(1024 << 20) // (nw * E * H * I * 2)))
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn((T, E), generator=g, device=dev)
        if wl["zipf"]:
            ranks = torch.randperm(E, generator=torch.Generator().manual_seed(args.seed)).double() + 1
            pz = ranks ** (-wl["zipf"])
            logits += torch.log(pz / pz.sum()).float().to(dev)[None, :]
        ws = []
        for _ in range(ncopy):
            gw = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            uw = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
            dw = (torch.randn((E, I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16) if qwen3 else None
            ws.append((gw, uw, dw))
        tw = torch.empty((T, k), device=dev)
        ti = torch.empty((T, k), dtype=torch.int32, device=dev)
        tei = torch.empty((T, k), dtype=torch.int32, device=dev)
        moe = cm.FusedMoE.new(E, k, act)
        nsteps = 20

        def steps():
            outs = []
            for s_ in range(nsteps):
                cm.apply_topk_softmax_inplace(logits, tw, ti, tei)
                gw, uw, dw = ws[s_ % ncopy]
                outs.append(moe.forward(x, gw, uw, dw, tw, ti, wl["moe_type"]))
            return outs

        ref = steps()
        torch.cuda.synchronize()
        touched = int(torch.unique(ti).numel())
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        steps()
        ev[1].record()
        torch.cuda.synchronize()
        eager_us = 1000.0 * ev[0].elapsed_time(ev[1]) / nsteps
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            steps()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):  # the stream whose library workspace is warm
            gouts = steps()
        graph.replay()
        torch.cuda.synchronize()
        reps = 10
        ev[0].record()
        for _ in range(reps):
            graph.replay()
        ev[1].record()
        torch.cuda.synchronize()
        graph_us = 1000.0 * ev[0].elapsed_time(ev[1]) / (reps * nsteps)
        ok = all(torch.equal(a, b) for a, b in zip(gouts, ref))
        wbytes = touched * nw * H * I * 2
        res[f"{wname}_T{T}"] = {
            "tokens": T, "touched_experts": touched, "weight_mb": round(wbytes / 1e6, 1),
            "graph_us": round(graph_us, 2) if ok else None, "eager_us": round(eager_us, 2),
            "weight_frac": round(wbytes / (PEAK_HBM_GBS * 1e9) / (graph_us * 1e-6), 4) if ok else None,
            "kernel": cm.fused_moe_kernel(T, H, I, E, k, 1, wl["moe_type"]),
        }
        del ws, graph, gouts, ref
    return res


def bench_fp8_decode(torch, cm, dev, args):
    """Decode GEMMs with bf16 against fp8 e4m3 expert weights
    (candle_moe_fused_moe_status against candle_moe_fused_moe_fp8, the same
    inputs and routing): µs per launch of the gate/up and down GEMMs from HIP
    events around every launch, over 60 calls rotating across weight copies
    whose total exceeds the 256 MB last-level cache twice (cold weights),
    and the weight bytes each GEMM streams (touched experts x 2HI or HI x bytes
    per weight) over its time. `gemm_speedup`: bf16 over fp8 time of the two
    GEMMs; `launch_speedup`: the same over every launch of the forward
    (grouping where the path has one, GEMMs, finishing launches)."""
    L = cm.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nslots = L.candle_moe_profile_begin()
    cm.check(L.candle_moe_profile_end(None, None, 0))
    names = [L.candle_moe_profile_slot_name(s).decode() for s in range(nslots)]
    res = {}
    for wname, T in [("qwen3", 16), ("qwen3", 64), ("q30b", 1), ("q30b", 16), ("nomic", 16)]:
        if getattr(args, "fp8_shape", "") and args.fp8_shape != f"{wname}_T{T}":
            continue
        wl = WORKLOADS[wname]
        H, I, E, k = wl["H"], wl["I"], wl["E"], wl["k"]
        qwen3 = wl["moe_type"] == 0
        act = {"silu": 0, "gelu": 1, "relu": 2}[wl["act"]]
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + T)
        ncopy = max(2, -(-(1024 << 20) // (3 * E * H * I)))  # fp8 bytes of all copies >= 1 GiB
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        logits = torch.randn((T, E), generator=g, device=dev)
        if wl["zipf"]:
            ranks = torch.randperm(E, generator=torch.Generator().manual_seed(args.seed)).double() + 1
            pz = ranks ** (-wl["zipf"])
            logits += torch.log(pz / pz.sum()).float().to(dev)[None, :]
        tw = torch.empty((T, k), device=dev)
        ti = torch.empty((T, k), dtype=torch.int32, device=dev)
        tei = torch.empty((T, k), dtype=torch.int32, device=dev)
        cm.apply_topk_softmax_inplace(logits, tw, ti, tei)
        touched = int(torch.unique(ti).numel())
        bf, f8 = [], []
        for _ in range(ncopy):
            # Qwen3: gate/up [E,H,I], down [E,I,H]; Nomic: fc1 [E,H,I], fc2 [E,H,I] (already [N,K])
            shapes = ((E, H, I), (E, H, I), (E, I, H)) if qwen3 else ((E, H, I), (E, H, I))
            w3 = [(torch.randn(shape, generator=g, device=dev) * 0.02).to(torch.bfloat16) for shape in shapes]
            if not qwen3:
                w3.append(None)
            bf.append(w3)
            f8.append([cm.quantize_fp8(w, input_kn=(qwen3 or j == 0)) if w is not None else (None, None)
                       for j, w in enumerate(w3)])
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)

        def run(fp8, c):
            if fp8:
                (gq, gs), (uq, us_), (dq, ds) = f8[c]
                return L.candle_moe_fused_moe_fp8(p(x), p(gq), p(uq), p(dq), p(gs), p(us_), p(ds), p(tw), p(ti),
                                                  p(out), T, H, I, E, k, act, wl["moe_type"], 1, stream)
            gw, uw, dw = bf[c]
            return L.candle_moe_fused_moe_status(p(x), p(gw), p(uw), p(dw), p(tw), p(ti), p(out), T, H, I, E, k, act,
                                                 wl["moe_type"], 1, stream)

        entry = {"tokens": T, "touched_experts": touched, "weight_copies": ncopy}
        for label, fp8 in (("bf16", False), ("fp8", True)):
            for c in range(ncopy):
                cm.check(run(fp8, c))
            torch.cuda.synchronize()
            L.candle_moe_profile_begin()
            for s in range(60):
                cm.check(run(fp8, s % ncopy))
            torch.cuda.synchronize()
            ms = (ctypes.c_double * nslots)()
            cnt = (ctypes.c_int * nslots)()
            cm.check(L.candle_moe_profile_end(ms, cnt, nslots))
            us = {names[s]: round(1000.0 * ms[s] / cnt[s], 2) for s in range(nslots) if cnt[s]}
            bpe = 1 if fp8 else 2
            g1b, g2b = touched * (2 if qwen3 else 1) * H * I * bpe, touched * H * I * bpe
            us["gate_up_gbs"] = round(g1b / (us["gemm_gate_up"] * 1e-6) / 1e9, 1)
            us["down_gbs"] = round(g2b / (us["gemm_down"] * 1e-6) / 1e9, 1)
            entry[label] = us
        b, f = entry["bf16"], entry["fp8"]
        entry["gemm_speedup"] = round((b["gemm_gate_up"] + b["gemm_down"]) / (f["gemm_gate_up"] + f["gemm_down"]), 3)
        launches = lambda d: sum(v for k_, v in d.items() if k_ in names)  # noqa: E731
        entry["launch_speedup"] = round(launches(b) / launches(f), 3)
        res[f"{wname}_T{T}"] = entry
        del bf, f8
    return res


def bench_fp8_prefill(torch, cm, dev, args):
    """Prefill with bf16 against fp8 e4m3 expert weights (Qwen3 T=4096 and
    T=32768, Nomic T=32768): µs per call over 10 calls between two events —
    bf16 the host FusedMoE::forward (router outputs given), fp8 the zeroing of
    the output plus candle_moe_fused_moe_fp8 adding into it (its drop-in
    form) — and each GEMM's µs per launch from a separate pass with HIP events
    around every launch; rel_rms = RMS(fp8 output - bf16 output) / RMS(bf16
    output), the weight quantization's effect on the layer."""
    L = cm.lib()
    nslots = L.candle_moe_profile_begin()
    cm.check(L.candle_moe_profile_end(None, None, 0))
    names = [L.candle_moe_profile_slot_name(s).decode() for s in range(nslots)]
    res = {}
    for wname, T in (("qwen3", 4096), ("qwen3", 32768), ("nomic", 32768)):
        wl = WORKLOADS[wname]
        H, I, E, k = wl["H"], wl["I"], wl["E"], wl["k"]
        qwen3 = wl["moe_type"] == 0
        act = {"silu": cm.Activation.Silu, "gelu": cm.Activation.Gelu, "relu": cm.Activation.Relu}[wl["act"]]
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed + T)
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        gate = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        up = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        down = (torch.randn((E, I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16) if qwen3 else None
        logits = torch.randn((T, E), generator=g, device=dev)
        tw = torch.empty((T, k), device=dev)
        ti = torch.empty((T, k), dtype=torch.int32, device=dev)
        tei = torch.empty((T, k), dtype=torch.int32, device=dev)
        cm.apply_topk_softmax_inplace(logits, tw, ti, tei)
        gq, gs = cm.quantize_fp8(gate, input_kn=True)
        uq, us_ = cm.quantize_fp8(up, input_kn=qwen3)  # Nomic fc2 [E, H, I] is already [N, K]
        dq, ds = cm.quantize_fp8(down, input_kn=True) if qwen3 else (None, None)
        moe = cm.FusedMoE.new(E, k, act)
        out8 = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)

        def run_bf16():
            return moe.forward(x, gate, up, down, tw, ti, wl["moe_type"])

        def run_fp8():
            out8.zero_()
            cm.fused_moe_fp8(x, gq, uq, dq, gs, us_, ds, tw, ti, out8, E, k, int(act), wl["moe_type"])
            return out8

        entry = {"tokens": T}
        outs = {}
        for label, fn in (("bf16", run_bf16), ("fp8", run_fp8)):
            for _ in range(3):
                outs[label] = fn()
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                fn()
            e1.record()
            e1.synchronize()
            call_us = e0.elapsed_time(e1) / 10 * 1e3
            L.candle_moe_profile_begin()
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            ms = (ctypes.c_double * nslots)()
            cnt = (ctypes.c_int * nslots)()
            cm.check(L.candle_moe_profile_end(ms, cnt, nslots))
            us = {names[s]: round(1000.0 * ms[s] / cnt[s], 1) for s in range(nslots) if cnt[s] and "gemm" in names[s]}
            entry[label] = {"call_us": round(call_us, 1), **us}
        ref = outs["bf16"].float()
        entry["rel_rms"] = round(float((outs["fp8"].float() - ref).pow(2).mean().sqrt() / ref.pow(2).mean().sqrt()), 4)
        res[f"{wname}_T{T}"] = entry
        del x, gate, up, down, gq, uq, dq, out8, outs, ref
    return res


def graph_us(torch, calls, ncalls, reps, check):
    """Per-call GPU time of `calls` (ncalls launches) captured once in a
    torch CUDA graph and replayed `reps` times between two events: no host
    launch cost and no per-launch events. `check()` compares the outputs of
    the last replay with the eager ones (False: the number is not used)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        calls()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):  # the stream whose library workspace is warm
        calls()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    ev[0].record()
    for _ in range(reps):
        graph.replay()
    ev[1].record()
    torch.cuda.synchronize()
    us = 1000.0 * ev[0].elapsed_time(ev[1]) / (reps * ncalls)
    return us if check() else None


def bench_router_only(args, torch, cm, dev):
    """topk-softmax alone over BASELINE config 2 shapes (µs and GB/s), and the
    router GEMM fused with it. `us`: per call with HIP events around every
    launch (eager); `graph_us`: per call from a captured sequence of 50 calls
    replayed (GPU time only), the headline `value`."""
    L = cm.lib()
    res = {}
    for (T, E, k) in [(32768, 8, 2), (32768, 64, 6), (32768, 128, 8)]:
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed)
        # rotate over enough logits buffers to exceed the 256 MB last-level cache
        nbuf = max(1, (512 << 20) // (T * E * 4))
        logits = [torch.randn((T, E), generator=g, device=dev) for _ in range(nbuf)]
        w = torch.empty((T, k), device=dev)
        i = torch.empty((T, k), dtype=torch.int32, device=dev)
        ei = torch.empty((T, k), dtype=torch.int32, device=dev)
        for _ in range(args.warmup):
            cm.apply_topk_softmax_inplace(logits[0], w, i, ei)
        torch.cuda.synchronize()
        n = L.candle_moe_profile_begin()
        for s in range(max(args.steps, 50)):
            cm.apply_topk_softmax_inplace(logits[s % nbuf], w, i, ei)
        torch.cuda.synchronize()
        ms = (ctypes.c_double * n)()
        cnt = (ctypes.c_int * n)()
        cm.check(L.candle_moe_profile_end(ms, cnt, n))
        us = 1000.0 * ms[0] / cnt[0]
        nbytes = T * E * 4 + T * k * 12
        last = (logits[49 % nbuf], w.clone(), i.clone(), ei.clone())
        cm.apply_topk_softmax_inplace(last[0], w, i, ei)
        ref = (w.clone(), i.clone(), ei.clone())
        gus = graph_us(torch, lambda: [cm.apply_topk_softmax_inplace(logits[s % nbuf], w, i, ei) for s in range(50)],
                       50, 20, lambda: torch.equal(w, ref[0]) and torch.equal(i, ref[1]) and torch.equal(ei, ref[2]))
        res[f"{T}x{E}k{k}"] = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                               "graph_us": round(gus, 2) if gus else None,
                               "graph_gbs": round(nbytes / (gus * 1e-6) / 1e9, 1) if gus else None}
    # router GEMM fused with topk-softmax (hidden [T,H] bf16, Linear weight
    # [E,H]): bytes = hidden + weight + outputs; HBM-bound on hidden
    fused = {}
    for (name, T, H, E, k) in [("qwen3", 32768, 4096, 8, 2), ("nomic", 32768, 768, 8, 2),
                               ("q30b", 32768, 2048, 128, 8), ("q30b", 4096, 2048, 128, 8),
                               ("q30b", 128, 2048, 128, 8), ("q30b", 16, 2048, 128, 8)]:
        g = torch.Generator(device=dev)
        g.manual_seed(args.seed)
        nbuf = min(64, max(1, (512 << 20) // (T * H * 2)))
        xs = [torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16) for _ in range(nbuf)]
        wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
        w = torch.empty((T, k), device=dev)
        i = torch.empty((T, k), dtype=torch.int32, device=dev)
        ei = torch.empty((T, k), dtype=torch.int32, device=dev)
        for _ in range(args.warmup):
            cm.router_topk(xs[0], wr, w, i, ei)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        nrep = max(args.steps, 50)
        ev[0].record()
        for s in range(nrep):
            cm.router_topk(xs[s % nbuf], wr, w, i, ei)
        ev[1].record()
        torch.cuda.synchronize()
        us = 1000.0 * ev[0].elapsed_time(ev[1]) / nrep
        nbytes = T * H * 2 + E * H * 2 + T * k * 12
        cm.router_topk(xs[49 % nbuf], wr, w, i, ei)
        ref = (w.clone(), i.clone(), ei.clone())
        gus = graph_us(torch, lambda: [cm.router_topk(xs[s % nbuf], wr, w, i, ei) for s in range(50)], 50, 20,
                       lambda: torch.equal(w, ref[0]) and torch.equal(i, ref[1]) and torch.equal(ei, ref[2]))
        fused[f"{name} T={T} H={H} E={E} k={k}"] = {
            "us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "graph_us": round(gus, 2) if gus else None,
            "graph_gbs": round(nbytes / (gus * 1e-6) / 1e9, 1) if gus else None}
    head = res["32768x8k2"]
    hus = head["graph_us"] or head["us"]
    hgbs = head["graph_gbs"] or head["gbs"]
    print(json.dumps({
        "metric": "topk-softmax µs", "value": hus, "unit": "us", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": hus / 1000.0, "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic N(0,1) logits, cold buffers",
        "config": {"workload": "topk-softmax [32768,E] (config 2)",
                   "timing": "graph_us: 50 calls captured in one graph, replayed (GPU time per call); "
                             "us: HIP events around every launch"},
        "shapes": res, "router_gemm_topk_bf16": fused,
        "roofline": {"bound": "hbm", "achieved": hgbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(hgbs / PEAK_HBM_GBS, 4), "traffic": None},
        "cpu_baseline": None,
    }))


if __name__ == "__main__":
    main()
