#!/usr/bin/env python3
"""W4A16 QuantLinear on one MI355X: decode GB/s (headline), prefill TFLOP/s (sweep).

One step = one Llama-3-8B decoder layer's four quantized projections at batch 1
(decode): qkv (K 4096, N 6144), o (4096, 4096), gate_up (4096, 28672) and down
(14336, 4096), 4-bit asymmetric round-to-nearest with group 128 (the reference's
packed layout), bf16 activations ~N(0, 1), weights ~N(0, 0.02). Steps cycle through
several distinct layer copies (at least 512 MB of packed weights) so the 256 MB
Infinity Cache cannot hold them: every step streams its weights from HBM, like a real
decode walking through a model's layers. Inputs are resident in HBM before timing.

value       = algorithmic bytes of all timed steps / timed seconds
              bytes per call = N*K/2 + 4*N*G*2 + 2*M*K + 2*M*N  (G = K/128)
roofline    = the dominant kernel (gate_up decode GEMV): its algorithmic bytes per
              launch / its mean launch time from HIP events on the launch stream
cpu_baseline= the reference's host sequence (dequantize once, cache, F.linear in bf16)
              timed on this host's cores for a bounded sample of the same steps

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO / "quantized-llm-inference-engine-_amd"), str(REPO)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W4A16 QuantLinear GB/s & %HBM peak (decode); TFLOP/s & %MFMA peak (prefill)"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PROJECTIONS = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
GROUP = 128
MIN_ROTATION_BYTES = 512 * 2**20


def algorithmic_bytes(m: int, n: int, k: int, bits: int = 4, group: int = GROUP, asym: bool = True) -> int:
    codes = n * k // 2 if bits < 8 else n * k
    meta = 4 * n * (k // group) * (2 if asym else 1)
    return codes + meta + 2 * m * k + 2 * m * n


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--m", type=int, default=1, help="tokens per decode step")
    p.add_argument("--kernel-launches", type=int, default=100, help="timed launches of the dominant kernel")
    p.add_argument("--sweep", action="store_true", help="also time every projection at M in {1,8,32,64,256,2048,8192}")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    return p.parse_args()


def build_layers(torch, count: int, m: int):
    """`count` distinct copies of the four quantized projections plus their inputs/outputs."""
    from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    base = {}
    for name, n, k in PROJECTIONS:
        w = torch.randn(n, k, generator=gen, device=dev) * 0.02
        base[name] = RoundToNearestQuantizer(4, GROUP, symmetric=False).quantize(w)
        del w
    layers = []
    for _ in range(count):
        layer = {}
        for name, n, k in PROJECTIONS:
            qt = base[name]
            layer[name] = QuantizedTensor(
                qt.qweight.clone(), qt.scales.clone(), qt.zeros.clone(), 4, GROUP, False, qt.shape
            )
        layers.append(layer)
    xs = {name: torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16) for name, _, k in PROJECTIONS}
    return base, layers, xs


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (the kernels run on one "
            "device; see DESIGN.md for how the projections would shard). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    import torch

    from llmopt.kernels import _lib, ops

    _lib.load_library()
    torch.cuda.set_device(0)
    bf16 = torch.bfloat16

    layer_bytes = sum(algorithmic_bytes(0, n, k) for _, n, k in PROJECTIONS)
    copies = max(2, -(-MIN_ROTATION_BYTES // layer_bytes))
    base, layers, xs = build_layers(torch, copies, args.m)
    outs = {name: torch.empty(args.m, n, dtype=bf16, device="cuda:0") for name, n, _ in PROJECTIONS}
    step_bytes = sum(algorithmic_bytes(args.m, n, k) for _, n, k in PROJECTIONS)

    # One HIP graph per layer copy: the four launches of a step, replayed back to back.
    stream = torch.cuda.Stream()
    graphs = []
    with torch.cuda.stream(stream):
        for layer in layers:  # eager warm-up before capture
            for name, _, _ in PROJECTIONS:
                ops.quant_linear(xs[name], layer[name], None, bf16)
        torch.cuda.synchronize()
        for layer in layers:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for name, _, _ in PROJECTIONS:
                    outs[name] = ops.quant_linear(xs[name], layer[name], None, bf16)
            graphs.append(g)
    torch.cuda.synchronize()

    print(f"# decode step: 4 projections, M={args.m}, {copies} layer copies "
          f"({copies * layer_bytes / 2**20:.0f} MiB packed)", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    cur = torch.cuda.current_stream()
    start.record(cur)
    for i in range(args.steps):
        graphs[i % copies].replay()
    end.record(cur)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    value = step_bytes * args.steps / (total_ms * 1e-3) / 1e9

    # Dominant kernel: gate_up at M, one event pair per launch, rotating over the copies.
    name, n, k = PROJECTIONS[2]
    x = xs[name]
    times = []
    for i in range(args.kernel_launches + 10):
        s_ev = torch.cuda.Event(enable_timing=True)
        e_ev = torch.cuda.Event(enable_timing=True)
        s_ev.record(cur)
        ops.quant_linear(x, layers[i % copies][name], None, bf16)
        e_ev.record(cur)
        if i >= 10:
            times.append((s_ev, e_ev))
    torch.cuda.synchronize()
    kernel_us = statistics.mean(s.elapsed_time(e) * 1e3 for s, e in times)
    kernel_bytes = algorithmic_bytes(args.m, n, k)
    achieved = kernel_bytes / (kernel_us * 1e-6) / 1e9
    roofline = {
        "bound": "hbm",
        "kernel": f"qlinear_decode gate_up M={args.m} (K 4096, N 28672)",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": _measured_traffic(f"gate_up_m{args.m}"),
        "algorithmic_bytes": kernel_bytes,
        "mean_launch_us": round(kernel_us, 3),
    }

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b decoder-layer projections (qkv, o, gate_up, down), W4A16 decode",
            "M": args.m,
            "bits": 4,
            "group": GROUP,
            "symmetric": False,
            "layer_copies": copies,
            "bytes_per_step": step_bytes,
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
    }
    if args.sweep:
        result["sweep"] = sweep(torch, ops, layers, copies)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, base, args.m, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def _measured_traffic(key: str):
    """HBM bytes per launch measured with rocprofv3 counters, if recorded in profiles/."""
    path = REPO / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key)
    except (OSError, ValueError):
        return None


def sweep(torch, ops, layers, copies):
    """Per-projection kernel times (HIP events) for decode and prefill batch sizes."""
    bf16 = torch.bfloat16
    cur = torch.cuda.current_stream()
    rows = []
    for m in (1, 8, 32, 64, 256, 2048, 8192):
        for name, n, k in PROJECTIONS:
            x = torch.randn(m, k, device="cuda:0").to(bf16)
            reps = 20 if m <= 2048 else 5
            for i in range(3):
                ops.quant_linear(x, layers[i % copies][name], None, bf16)
            pairs = []
            for i in range(reps):
                s_ev = torch.cuda.Event(enable_timing=True)
                e_ev = torch.cuda.Event(enable_timing=True)
                s_ev.record(cur)
                ops.quant_linear(x, layers[i % copies][name], None, bf16)
                e_ev.record(cur)
                pairs.append((s_ev, e_ev))
            torch.cuda.synchronize()
            us = statistics.median(s.elapsed_time(e) * 1e3 for s, e in pairs)
            gbs = algorithmic_bytes(m, n, k) / (us * 1e-6) / 1e9
            tflops = 2 * m * n * k / (us * 1e-6) / 1e12
            rows.append({
                "proj": name, "M": m, "us": round(us, 2), "GB/s": round(gbs, 1),
                "hbm_frac": round(gbs / HBM_PEAK_GBS, 3), "TFLOP/s": round(tflops, 2),
                "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
            })
            print(f"# sweep {name:8s} M={m:5d} {us:9.2f} us {gbs:8.1f} GB/s {tflops:8.2f} TFLOP/s",
                  file=sys.stderr, flush=True)
            del x
    return rows


def cpu_baseline(torch, base, m: int, seconds: float):
    """The reference's host sequence on this machine's cores, on a bounded sample."""
    from oracle.cpu_reference import ReferenceLinear

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(1)
    mods = {}
    for name, n, k in PROJECTIONS:
        qt = base[name]
        mods[name] = ReferenceLinear(
            qt.qweight.cpu(), qt.scales.cpu(), qt.zeros.cpu(), 4, GROUP, False, qt.shape, torch.bfloat16
        )
    xs = {name: torch.randn(m, k, generator=gen).to(torch.bfloat16) for name, _, k in PROJECTIONS}
    step_bytes = sum(algorithmic_bytes(m, n, k) for _, n, k in PROJECTIONS)

    # Cold: one full step that dequantizes every weight (the reference's first call).
    t0 = time.perf_counter()
    for name, _, _ in PROJECTIONS:
        mods[name](xs[name])
    cold_s = time.perf_counter() - t0
    # Warm: the reference's steady state (cached dense bf16 weight, F.linear only).
    steps = 0
    t0 = time.perf_counter()
    while True:
        for name, _, _ in PROJECTIONS:
            mods[name](xs[name])
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds or steps >= 10000:
            break
    warm = step_bytes * steps / elapsed / 1e9
    return {
        "value": round(warm, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} warm decode steps (4 projections, M={m}, bf16, dense weight cached) "
                  f"in {elapsed:.1f} s; cold first step (dequantize + F.linear) {cold_s:.2f} s "
                  f"= {step_bytes / cold_s / 1e9:.3f} GB/s",
        "cold_value": round(step_bytes / cold_s / 1e9, 3),
        "torch": torch.__version__,
    }


if __name__ == "__main__":
    raise SystemExit(main())
