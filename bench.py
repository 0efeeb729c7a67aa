#!/usr/bin/env python3
"""W4A16 QuantLinear on one MI355X: decode GB/s (headline) and prefill TFLOP/s.

Workload (one step): one Llama-3-8B decoder layer's four quantized projections at batch 1
(decode) -- qkv (K 4096, N 6144), o (4096, 4096), gate_up (4096, 28672), down (14336, 4096) --
with 4-bit asymmetric round-to-nearest weights, group 128, in the reference's packed layout
(two codes per byte, fp32 scales and zeros per group); bf16 activations ~N(0, 1), weights
~N(0, 0.02), all synthetic and seeded. Steps cycle through enough distinct layer copies
(>= 512 MiB of packed weights) that the 256 MB Infinity Cache cannot hold them: every step
streams its weights from HBM, like a decode walking through a model's layers. Inputs are
resident in HBM before timing; the layer copies' steps (four launches each) are one HIP graph,
replayed as a whole, as a decode step of a model runs its layers from one graph.

value          algorithmic bytes of all timed steps / timed seconds, where one call moves
               N*K/2 (codes) + 4*N*G*2 (scales, zeros; G = K/128) + 2*M*K + 2*M*N bytes
roofline       the dominant kernel (gate_up): its algorithmic bytes / its mean time per launch,
               from HIP events around replays of a graph of back-to-back launches (rotating
               over >= 512 MiB of gate_up copies) on the replay stream -- so it includes the
               inter-kernel gap;
               `traffic` = HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (each
               scaled by what it reads for a plain copy of known size), when recorded
prefill        gate_up at M = 8192 as QuantLinear runs it (from 1024 tokens: the weight
               dequantized into the workspace, then hipBLASLt), TFLOP/s vs dense bf16 peak; and
               the fused register-dequant MFMA GEMM on the same shape (`fused_gemm`)
dense_comparator  (in roofline and prefill) torch's dense bf16 F.linear on the dequantized
               weight at the same shape: hipBLASLt's figure for the unquantized layer
dequant, quantize, attention  the device dequantize and RTN quantizer on gate_up, and the
               decode-step paged attention / KV write / last-token vocabulary projection of the
               end-to-end Llama-3-8B workload (32 sequences, 512-token prompts)
e2e            that workload end to end (config 5): the Llama-3-8B model, every decoder linear
               W4 g128 asymmetric, 32 prompts of 512 tokens, one prefill forward, then 128
               greedy decode steps through the paged cache, each step one HIP-graph replay;
               decode and prefill tokens/s (reported, not a roofline figure)
shapes         every projection (qkv, o, gate_up, down) at M in {1, 8, 32, 64} (decode: GB/s and
               fraction of HBM) and {256, 2048, 8192} (prefill: TFLOP/s and fraction of the dense
               bf16 MFMA peak), W4 g128 asymmetric, bf16
bits_sweep     the down projection at 8-bit, 4-bit and 2-bit RTN and 4-bit GPTQ (asymmetric and
               symmetric; calibrated on 128 seeded embedding rows), M in {1, 32, 2048}
cpu_baseline   the reference's host sequence (dequantize once, cache the dense weight, F.linear)
               on this host's cores: `value` is the decode step at M = 1 (bf16, warm); `configs`
               holds a bounded sample of the reference's CPU configurations -- one fp32 linear
               (K = N = 4096, M = 1), the four projections at M in {1, 8, 32, 64, 256, 2048}, the
               bit-width sweep -- warm (dense weight cached) and cold (dequantize + F.linear)

Every single-projection timing (roofline, prefill, shapes, bits_sweep) rotates over at least
512 MiB of that projection's own weight copies.

Modes: default prints the JSON line. `--e2e-only` runs only the end-to-end generation (for a
kernel trace of it). `--pmc-workload` runs only the dominant kernel and a
256 MiB copy (for `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`); `--traffic-from DIR`
turns two such rocprofv3 CSV outputs into profiles/traffic_decode_gate_up_m1.json;
`--trace-runs CSV` prints a rocprofv3 kernel trace of this script per timed block (run),
`--trace-kernels CSV` per kernel and grid.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-shapes] [--no-cpu]
       [--no-prefill] [--no-e2e] [--e2e-only]
"""

from __future__ import annotations

import argparse
import csv
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
REPLAYS = 50  # timed graph replays per figure (each of several back-to-back launches); median
TRAFFIC_FILE = REPO / "profiles" / "traffic_decode_gate_up_m1.json"
COPY_BYTES = 256 * 2**20


def algorithmic_bytes(m: int, n: int, k: int, bits: int = 4, group: int = GROUP, asym: bool = True) -> int:
    codes = n * k // 2 if bits < 8 else n * k
    meta = 4 * n * (k // group) * (2 if asym else 1)
    return codes + meta + 2 * m * k + 2 * m * n


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--m", type=int, default=1, help="tokens per decode step")
    p.add_argument("--kernel-launches", type=int, default=60, help="timed launches of the dominant kernel")
    p.add_argument("--no-shapes", action="store_true",
                   help="skip the per-shape block and the bit-width sweep")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-prefill", action="store_true", help="skip the prefill measurement")
    p.add_argument("--no-e2e", action="store_true", help="skip the end-to-end Llama-3-8B generation")
    p.add_argument("--e2e-only", action="store_true", help="only the end-to-end generation (for profiling)")
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--pmc-workload", action="store_true", help="only the dominant kernel + a copy")
    p.add_argument("--pmc-prefill", action="store_true",
                   help="only gate_up at M = 8192, two-pass and fused GEMM, three calls each (for --pmc)")
    p.add_argument("--pmc-decode", action="store_true",
                   help="only qkv and o at M = 32 and 64, five calls each, and a copy (for --pmc)")
    p.add_argument("--counters-from", type=str, default=None,
                   help="rocprofv3 --pmc output dir: print each counter's mean per dispatch, per kernel and grid")
    p.add_argument("--roofline-only", action="store_true",
                   help="only the roofline block (graph replays of the dominant kernel), for rocprofv3 --stats")
    p.add_argument("--traffic-from", type=str, default=None, help="rocprofv3 --pmc output dir")
    p.add_argument("--trace-runs", type=str, default=None,
                   help="rocprofv3 --kernel-trace CSV: print this library's kernels per run of dispatches")
    p.add_argument("--trace-kernels", type=str, default=None,
                   help="rocprofv3 --kernel-trace CSV: print every kernel's count and durations per grid")
    return p.parse_args()


def build_layers(torch, count: int, m: int):
    """`count` distinct copies of the four quantized projections plus their inputs."""
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


def build_rotations(layers, min_bytes: int = MIN_ROTATION_BYTES):
    """Per projection, distinct weight copies totalling at least `min_bytes`: the layer copies,
    plus clones of them. Timing one projection alone over fewer bytes than the 256 MB Infinity
    Cache would let repeats hit that cache."""
    from llmopt.quantization import QuantizedTensor

    rot = {}
    for name, n, k in PROJECTIONS:
        copies = [layer[name] for layer in layers]
        need = max(2, -(-min_bytes // algorithmic_bytes(0, n, k)))
        while len(copies) < need:
            qt = copies[len(copies) % len(layers)]
            copies.append(QuantizedTensor(qt.qweight.clone(), qt.scales.clone(), qt.zeros.clone(), qt.bits,
                                          qt.group_size, qt.symmetric, qt.shape))
        rot[name] = copies
    return rot


def kernel_launch_times(torch, launch, count: int, replays: int = REPLAYS) -> list[float]:
    """Per-launch times (us) of `count` back-to-back launches captured in one HIP graph and
    replayed `replays` times (after one untimed replay), each replay bracketed by HIP events on
    the replay stream. The figure includes the few-microsecond gap the GPU leaves between two
    dependent kernels. Callers report the median over the replays."""
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        launch(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            for i in range(count):
                launch(i)
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    g.replay()
    torch.cuda.synchronize()
    out = []
    for _ in range(replays):
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(cur)
        g.replay()
        e.record(cur)
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) * 1e3 / count)
    return out


def main() -> int:
    args = parse_args()
    if args.traffic_from:
        return traffic_summary(Path(args.traffic_from))
    if args.trace_runs:
        return trace_runs(Path(args.trace_runs))
    if args.trace_kernels:
        return trace_kernels(Path(args.trace_kernels))
    if args.counters_from:
        return counters_summary(Path(args.counters_from))
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: the quantized-linear kernels run on one device and there "
            "is no multi-GPU path (tensor parallelism would split qkv / gate_up along N and o / down "
            "along K on group boundaries, with one all-reduce per row-parallel projection). "
            "Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    import torch

    from llmopt.kernels import _lib, ops

    _lib.load_library()
    torch.cuda.set_device(0)
    bf16 = torch.bfloat16
    if args.e2e_only:
        print(json.dumps({"e2e": end_to_end(torch)}), flush=True)
        return 0
    if args.pmc_prefill or args.pmc_decode:
        return pmc_blocks(torch, ops, args.pmc_prefill)

    layer_bytes = sum(algorithmic_bytes(0, n, k) for _, n, k in PROJECTIONS)
    copies = max(2, -(-MIN_ROTATION_BYTES // layer_bytes))
    base, layers, xs = build_layers(torch, copies, args.m)
    flush_src = torch.empty(COPY_BYTES // 2, dtype=bf16, device="cuda:0")
    flush_dst = torch.empty_like(flush_src)

    def flush():
        flush_dst.copy_(flush_src)

    rotations = build_rotations(layers)
    name, n, k = PROJECTIONS[2]  # gate_up: the dominant kernel
    gate_up_copies = rotations[name]

    def launch_gate_up(i):
        ops.quant_linear(xs[name], gate_up_copies[i % len(gate_up_copies)], None, bf16)

    if args.pmc_workload:
        for i in range(3):
            launch_gate_up(i)
            flush()
        torch.cuda.synchronize()
        for i in range(args.kernel_launches):
            flush()
            launch_gate_up(i)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_workload": "gate_up decode", "M": args.m, "launches": args.kernel_launches,
                          "copy_bytes": COPY_BYTES, "algorithmic_bytes": algorithmic_bytes(args.m, n, k)}))
        return 0

    if args.roofline_only:
        times = kernel_launch_times(torch, launch_gate_up, 3 * len(gate_up_copies))
        kernel_us = statistics.mean(times)
        print(json.dumps({"roofline_only": "gate_up decode", "M": args.m, "mean_launch_us": round(kernel_us, 3),
                          "median_launch_us": round(statistics.median(times), 3),
                          "GB/s": round(algorithmic_bytes(args.m, n, k) / (kernel_us * 1e-6) / 1e9, 1)}))
        return 0

    outs = {p: torch.empty(args.m, pn, dtype=bf16, device="cuda:0") for p, pn, _ in PROJECTIONS}
    step_bytes = sum(algorithmic_bytes(args.m, pn, pk) for _, pn, pk in PROJECTIONS)

    # The layer copies in one HIP graph, as a decode step of a model walks through its layers:
    # `copies` steps (four launches each) per replay. Steps that do not fill a whole replay run
    # from one-layer graphs of the same launches.
    stream = torch.cuda.Stream()
    graphs = []
    with torch.cuda.stream(stream):
        for layer in layers:  # eager warm-up before capture
            for p, _, _ in PROJECTIONS:
                ops.quant_linear(xs[p], layer[p], None, bf16)
        torch.cuda.synchronize()
        for layer in layers:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for p, _, _ in PROJECTIONS:
                    outs[p] = ops.quant_linear(xs[p], layer[p], None, bf16)
            graphs.append(g)
        model_graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(model_graph, stream=stream):
            for layer in layers:
                for p, _, _ in PROJECTIONS:
                    outs[p] = ops.quant_linear(xs[p], layer[p], None, bf16)
    torch.cuda.synchronize()

    def run_steps(count):
        for _ in range(count // copies):
            model_graph.replay()
        for i in range(count % copies):
            graphs[i].replay()

    print(f"# decode step: 4 projections, M={args.m}, {copies} layer copies "
          f"({copies * layer_bytes / 2**20:.0f} MiB packed), {copies} steps per graph replay",
          file=sys.stderr, flush=True)
    run_steps(args.warmup)
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(cur)
    run_steps(args.steps)
    end.record(cur)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    value = step_bytes * args.steps / (total_ms * 1e-3) / 1e9
    print(f"# timed {args.steps} steps: {ms_per_step * 1e3:.2f} us/step, {value:.0f} GB/s",
          file=sys.stderr, flush=True)

    times = kernel_launch_times(torch, launch_gate_up, 3 * len(gate_up_copies))
    kernel_us = statistics.mean(times)
    kernel_bytes = algorithmic_bytes(args.m, n, k)
    achieved = kernel_bytes / (kernel_us * 1e-6) / 1e9
    traffic, traffic_note = _measured_traffic(args.m)
    roofline = {
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "traffic_source": traffic_note,
        "kernel": f"quantized-linear decode, gate_up M={args.m} (K 4096, N 28672, W4 g128 asym)",
        "algorithmic_bytes": kernel_bytes,
        "mean_launch_us": round(kernel_us, 3),
        "median_launch_us": round(statistics.median(times), 3),
        "weight_copies": len(gate_up_copies),
        "dense_comparator": dense_comparator(torch, base[name], args.m),
    }
    print(f"# gate_up kernel: mean {kernel_us:.2f} us, {achieved:.0f} GB/s", file=sys.stderr, flush=True)

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
            "steps_per_graph_replay": copies,
            "bytes_per_step": step_bytes,
            "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": roofline,
    }
    result["dequant"] = dequant_rate(torch, ops, rotations)
    result["quantize"] = quantize_rate(torch, ops)
    result["attention"] = attention_rates(torch)
    if not args.no_e2e:
        result["e2e"] = end_to_end(torch)
    if not args.no_prefill:
        result["prefill"] = prefill(torch, ops, rotations)
    gptq = None
    if not args.no_shapes:
        result["shapes"] = shapes(torch, ops, rotations)
        result["bits_sweep"], gptq = bits_sweep(torch, ops)
        result["engine_config"] = engine_config(torch, ops)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, base, args.m, args.cpu_seconds, gptq)
    print(json.dumps(result), flush=True)
    return 0


def _code_only(text: str) -> str:
    """A C++ source without its comments and blank-line or indentation differences: what the
    compiler sees (no kernel source here has comment markers inside string literals)."""
    import re

    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return "\n".join(" ".join(line.split()) for line in text.splitlines() if line.strip())


def source_digest() -> str:
    """sha256 (16 hex digits) of the code of the kernel sources the library is built from, comments
    and layout left out: names the build a counter measurement belongs to, so that a change to a
    comment does not orphan a measurement and a change to the code does."""
    import hashlib

    h = hashlib.sha256()
    csrc = REPO / "quantized-llm-inference-engine-_amd" / "csrc"
    for path in sorted(list(csrc.glob("*.hip")) + list(csrc.glob("*.hpp"))):
        h.update(path.name.encode())
        h.update(_code_only(path.read_text()).encode())
    return h.hexdigest()[:16]


def _measured_traffic(m: int):
    """HBM bytes per launch of the dominant kernel, from rocprofv3 counters, when they were
    measured on the current kernel sources (same digest); otherwise None and a note naming the
    sources they came from."""
    if not TRAFFIC_FILE.exists() or m != 1:
        return None, "no counter measurement recorded for this workload"
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None, "unreadable counter record"
    if rec.get("build") != source_digest():
        return None, (f"counters were measured on kernel sources {rec.get('build')}, not on the current ones "
                      f"({source_digest()}): {rec.get('hbm_bytes_per_launch')} B per launch then")
    return rec.get("hbm_bytes_per_launch"), (f"rocprofv3 FETCH_SIZE + WRITE_SIZE on the current kernel sources "
                                              f"({rec.get('build')})")


def prefill(torch, ops, rotations):
    """gate_up at M = 8192, per-call time of back-to-back calls: the automatic choice (the
    two-pass path: device dequantize into the workspace, then hipBLASLt) and the fused
    register-dequant GEMM (LLMOPT_ALGO_PREFILL) on the same shape."""
    from llmopt.kernels._lib import ALGO_AUTO, ALGO_PREFILL

    name, n, k = PROJECTIONS[2]
    m = 8192
    qts = rotations[name]
    x = torch.randn(m, k, device="cuda:0").to(torch.bfloat16)
    out = {}
    for label, algo in (("auto", ALGO_AUTO), ("fused_gemm", ALGO_PREFILL)):
        ops.quant_linear(x, qts[0], None, torch.bfloat16, algo=algo)
        times = kernel_launch_times(
            torch, lambda i: ops.quant_linear(x, qts[i % len(qts)], None, torch.bfloat16, algo=algo), len(qts)
        )
        us = statistics.median(times)
        out[label] = (us, 2 * m * n * k / (us * 1e-6) / 1e12)
        print(f"# prefill gate_up M={m} ({label}): {us:.1f} us, {out[label][1]:.1f} TFLOP/s", file=sys.stderr,
              flush=True)
    us, tflops = out["auto"]
    dense = dense_comparator(torch, qts[0], m)
    return {"kernel": f"quantized-linear prefill, gate_up M={m} (K 4096, N 28672): device dequantize into the "
                      f"workspace, then hipBLASLt", "mean_launch_us": round(us, 2),
            "achieved": round(tflops, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / BF16_PEAK_TFLOPS, 4), "bound": "mfma",
            "fused_gemm": {"mean_launch_us": round(out["fused_gemm"][0], 2),
                           "achieved": round(out["fused_gemm"][1], 1),
                           "frac": round(out["fused_gemm"][1] / BF16_PEAK_TFLOPS, 4)},
            "dense_comparator": dense}


def end_to_end(torch, seqs: int = 32, prompt_len: int = 512, steps: int = 128, ref_steps: int = 16):
    """Llama-3-8B (random init, every decoder linear W4 g128 asymmetric RTN, fused q/k/v and
    gate/up), 32 seeded prompts of 512 tokens, then 128 greedy steps through the paged cache
    (block 16). Prefill: one forward over all prompts (the reference's torch sequence for the
    prefill attention). Decode: each step one HIP-graph replay; tokens/s over steps 2..127.
    Beside it, the reference's way on the same GPU (`reference_twin`: dense bf16 linears holding
    the dequantized weights, torch norms / rotary / attention over the gathered cache, eager
    steps as the reference's engine runs them) for `ref_steps` steps."""
    from llmopt.model import GreedyGenerator, ModelConfig, fuse_projections_, random_quantized_model, reference_twin

    cfg = ModelConfig.llama3_8b()
    t0 = time.perf_counter()
    model = random_quantized_model(cfg, device="cuda:0", dtype=torch.bfloat16, seed=0, fuse=False)
    ref = reference_twin(model)
    fuse_projections_(model)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - t0
    prompts = torch.randint(0, cfg.vocab_size, (seqs, prompt_len), generator=torch.Generator().manual_seed(1))
    gen = GreedyGenerator(model, block_size=16)
    gen.generate(prompts[:, :32], 4)  # warm-up: first calls, graph machinery
    res = gen.generate(prompts, steps)
    step_ms = res.decode_seconds / (steps - 2) * 1e3
    packed = sum(b.numel() * b.element_size() for n, b in model.named_buffers() if "rotary" not in n)
    ref_gen = GreedyGenerator(ref, block_size=16, use_graph=False)
    ref_gen.generate(prompts[:, :32], 4)
    ref_res = ref_gen.generate(prompts, ref_steps)
    # Random-init weights give nearly flat logits, so greedy tokens part ways on rounding noise;
    # the logits themselves are what to compare.
    def rel(a, b):
        a, b = a.double(), b.double()
        return float((a - b).abs().max() / b.abs().max())

    diff = rel(res.prefill_logits, ref_res.prefill_logits)
    # The same reference computation in float32 (the dequantized bf16 weights, every activation in
    # fp32): how far each bf16 computation -- the HIP path's and the reference's -- drifts from it.
    ref32 = ref.float()
    exact = GreedyGenerator(ref32, block_size=16, use_graph=False).generate(prompts, 2).prefill_logits
    del ref32, ref
    torch.cuda.empty_cache()
    e_hip, e_ref = rel(res.prefill_logits, exact), rel(ref_res.prefill_logits, exact)
    out = {
        "workload": f"llama3-8b, {seqs} prompts x {prompt_len} tokens, then {steps} greedy steps, W4 g128 asym "
                    "RTN linears (fused qkv and gate_up), bf16, paged KV block 16",
        "decode_tokens_per_s": round(res.decode_tokens_per_second, 1),
        "decode_step_ms": round(step_ms, 3),
        "prefill_tokens_per_s": round(seqs * prompt_len / res.prefill_seconds, 1),
        "prefill_ms": round(res.prefill_seconds * 1e3, 1),
        "packed_linear_bytes": packed,
        "model_build_s": round(build_s, 2),
        "reference_way": {
            "how": "dense bf16 F.linear on the dequantized weights, torch norms/rotary/attention over the "
                   f"gathered cache, eager steps; {ref_steps} steps",
            "decode_tokens_per_s": round(ref_res.decode_tokens_per_second, 1),
            "decode_step_ms": round(ref_res.decode_seconds / (ref_steps - 2) * 1e3, 3),
            "prefill_tokens_per_s": round(seqs * prompt_len / ref_res.prefill_seconds, 1),
            "prefill_logits_max_abs_rel_diff": round(diff, 5),
        },
        "drift_vs_fp32": {
            "how": "prefill last-position logits against the reference computation run in float32 "
                   "(max|a - b| / max|b|)",
            "hip_path_bf16": round(e_hip, 5),
            "reference_way_bf16": round(e_ref, 5),
            # The bound the deep-model parity test holds the HIP path to: no more than twice the
            # reference's own bf16 drift.
            "within_bound": bool(e_hip <= 2 * e_ref + 2e-3),
        },
    }
    print(f"# e2e llama3-8b: prefill {out['prefill_ms']} ms ({out['prefill_tokens_per_s']:.0f} tok/s), decode "
          f"{step_ms:.2f} ms/step ({out['decode_tokens_per_s']:.0f} tok/s); the reference's way: decode "
          f"{out['reference_way']['decode_step_ms']:.2f} ms/step, prefill "
          f"{out['reference_way']['prefill_tokens_per_s']:.0f} tok/s", file=sys.stderr, flush=True)
    print(f"# e2e drift from the fp32 reference: HIP path {e_hip:.4f}, the reference's bf16 way {e_ref:.4f}",
          file=sys.stderr, flush=True)
    del model, gen, ref_gen, res, ref_res
    torch.cuda.empty_cache()
    return out


def dequant_rate(torch, ops, rotations):
    """The device dequantize (QuantizedTensor -> dense bf16, bit-exact with the reference) of
    gate_up: packed codes, scales and zeros read once, the dense weight written once."""
    name, n, k = PROJECTIONS[2]
    qts = rotations[name]
    count = min(len(qts), 8)
    times = kernel_launch_times(torch, lambda i: ops.dequantize(qts[i % count], torch.bfloat16), count)
    us = statistics.median(times)
    moved = algorithmic_bytes(0, n, k) + 2 * n * k
    gbs = moved / (us * 1e-6) / 1e9
    print(f"# dequantize gate_up -> bf16: {us:.1f} us, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    return {"kernel": f"dequantize gate_up (N {n}, K {k}) W4 g128 -> bf16", "us": round(us, 2),
            "bytes": moved, "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}


def quantize_rate(torch, ops):
    """The on-device round-to-nearest quantizer on gate_up (bf16 [28672, 4096] -> W4 g128 asym),
    beside the reference's torch sequence (choose_qparams, quantize_to_codes, pack_int4) run by
    torch on the same GPU. Both are bit-exact with the reference; `GB/s` counts the weight read
    once and codes, scales and zeros written once."""
    from llmopt.quantization.quantizers import choose_qparams, pack_int4, quantize_to_codes

    name, n, k = PROJECTIONS[2]
    gen = torch.Generator(device="cuda:0").manual_seed(5)
    copies = max(2, -(-MIN_ROTATION_BYTES // (2 * n * k)))
    ws = [(torch.randn(n, k, generator=gen, device="cuda:0") * 0.02).to(torch.bfloat16) for _ in range(copies)]
    times = kernel_launch_times(torch, lambda i: ops.quantize_rtn(ws[i % copies], 4, GROUP, False), 2 * copies)
    us = statistics.median(times)
    moved = 2 * n * k + algorithmic_bytes(0, n, k)
    gbs = moved / (us * 1e-6) / 1e9

    def torch_sequence(w):
        scales, zeros = choose_qparams(w, 4, GROUP, False)
        return pack_int4(quantize_to_codes(w, scales, zeros, 4, GROUP, False)), scales, zeros

    torch_sequence(ws[0])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(copies):
        torch_sequence(ws[i])
    torch.cuda.synchronize()
    torch_us = (time.perf_counter() - t0) * 1e6 / copies
    print(f"# quantize gate_up bf16 -> W4 g128: {us:.1f} us, {gbs:.0f} GB/s; torch sequence {torch_us:.0f} us",
          file=sys.stderr, flush=True)
    del ws
    return {"kernel": f"round-to-nearest quantize gate_up bf16 (N {n}, K {k}) -> W4 g128 asym", "us": round(us, 2),
            "bytes": moved, "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "torch_sequence_us": round(torch_us, 1)}


def attention_rates(torch):
    """Decode-step attention of the Llama-3-8B end-to-end workload: 32 sequences with 512-640
    cached tokens (512-token prompts, then up to 128 decoded), 32 query / 8 KV heads of 128,
    block 16, bf16 cache; one layer per call, rotating over 8 layers' caches (> 512 MiB) as a
    decode step walks the layers. Also: this step's KV write, the decode step as the model runs
    it (rotary step, cache write and attention in one launch), the reference's torch sequence for
    the same attention (gather, matmul, softmax, matmul) on the same GPU, the prefill attention of
    32 x 512-token prompts (kernel and torch sequence), and the vocabulary projection of a
    32 x 512-token prefill chunk for all positions vs the last ones only."""
    from llmopt.attention import PagedAttention, PagedAttentionConfig
    from llmopt.cache import PagedKVCache
    from llmopt.kernels import ops
    from llmopt.logits import last_token_logits

    seqs, heads, kv_heads, head_dim, bs, layers = 32, 32, 8, 128, 16, 8
    dev = torch.device("cuda:0")
    gen = torch.Generator().manual_seed(6)
    ctx = torch.randint(512, 641, (seqs,), generator=gen)
    width = 41
    blocks = seqs * width
    cache = PagedKVCache(layers, blocks, bs, kv_heads, head_dim, dtype=torch.bfloat16, device=dev)
    cache.key_cache.normal_()
    cache.value_cache.normal_()
    table = torch.randperm(blocks, generator=gen).view(seqs, width).to(torch.int32).to(dev)
    lens = ctx.to(torch.int32).to(dev)
    q = torch.randn(seqs, heads, 1, head_dim, device=dev).to(torch.bfloat16)
    attn = PagedAttention(heads, kv_heads, head_dim, config=PagedAttentionConfig(block_size=bs))
    times = kernel_launch_times(torch, lambda i: attn.forward(q, cache, i % layers, table, lens), 2 * layers)
    us = statistics.median(times)
    moved = int(ctx.sum()) * kv_heads * head_dim * 2 * 2 + 2 * q.numel() * 2 + table.numel() * 4
    gbs = moved / (us * 1e-6) / 1e9
    torch_attn = PagedAttention(heads, kv_heads, head_dim, config=PagedAttentionConfig(block_size=bs), backend="sdpa")
    torch_attn.forward(q, cache, 0, table, lens)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(layers):
        torch_attn.forward(q, cache, i % layers, table, lens)
    torch.cuda.synchronize()
    torch_us = (time.perf_counter() - t0) * 1e6 / layers
    new_k = torch.randn(seqs, kv_heads, head_dim, device=dev).to(torch.bfloat16)
    offsets = (lens - 1).to(torch.int64)
    w_times = kernel_launch_times(torch, lambda i: cache.write_decode(i % layers, table, offsets, new_k, new_k),
                                  2 * layers)
    # The decode step as the model runs it: rotary step, cache write and attention in one launch,
    # on the raw q / k / v rows of the fused projection's output.
    from llmopt.model import RotaryEmbedding

    rot = RotaryEmbedding(head_dim, 8192, base=500000.0).to(dev)
    qkv = torch.randn(seqs, (heads + 2 * kv_heads) * head_dim, device=dev).to(torch.bfloat16)
    rq = qkv[:, : heads * head_dim].view(seqs, heads, head_dim)
    rk = qkv[:, heads * head_dim : (heads + kv_heads) * head_dim].view(seqs, kv_heads, head_dim)
    rv = qkv[:, (heads + kv_heads) * head_dim :].view(seqs, kv_heads, head_dim)
    step_times = kernel_launch_times(
        torch, lambda i: ops.paged_decode_attention_rope(
            rq, rk, rv, offsets, rot.cos_cached, rot.sin_cached, cache.key_cache[i % layers],
            cache.value_cache[i % layers], table, lens, offsets.to(torch.int32), head_dim**-0.5), 2 * layers)
    step_us = statistics.median(step_times)
    print(f"# paged decode attention (32 seqs x 512-640 tokens, 32/8 heads): {us:.1f} us, {gbs:.0f} GB/s; "
          f"torch sequence {torch_us:.0f} us; KV write {statistics.median(w_times):.1f} us; with the rotary "
          f"step and the cache write in the same launch {step_us:.1f} us", file=sys.stderr, flush=True)
    del cache

    # Prefill attention: 32 prompts of 512 tokens, no prefix, causal.
    p_len, p_blocks = 512, 32
    pcache = PagedKVCache(1, seqs * p_blocks, bs, kv_heads, head_dim, dtype=torch.bfloat16, device=dev)
    pcache.key_cache.normal_()
    pcache.value_cache.normal_()
    ptable = torch.arange(seqs * p_blocks, dtype=torch.int32, device=dev).view(seqs, p_blocks)
    plens = torch.full((seqs,), p_len, dtype=torch.int32, device=dev)
    pq = torch.randn(seqs, p_len, heads, head_dim, device=dev).to(torch.bfloat16).permute(0, 2, 1, 3)
    pre_times = kernel_launch_times(
        torch, lambda i: attn.forward(pq, pcache, 0, ptable, plens), 8)
    pre_us = statistics.median(pre_times)
    pre_flop = seqs * heads * (p_len * (p_len + 1) / 2) * head_dim * 4
    torch_pre = PagedAttention(heads, kv_heads, head_dim, config=PagedAttentionConfig(block_size=bs), backend="sdpa")
    torch_pre.forward(pq, pcache, 0, ptable, plens)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        torch_pre.forward(pq, pcache, 0, ptable, plens)
    torch.cuda.synchronize()
    torch_pre_us = (time.perf_counter() - t0) * 1e6 / 3
    print(f"# paged prefill attention (32 x 512-token prompts, 32/8 heads, causal): {pre_us:.1f} us, "
          f"{pre_flop / pre_us / 1e6:.1f} TFLOP/s; torch sequence {torch_pre_us:.0f} us", file=sys.stderr, flush=True)
    del pcache

    # Vocabulary projection of one prefill chunk: every position vs the last ones.
    hidden_size, vocab, q_len = 4096, 128256, 512
    head = torch.nn.Linear(hidden_size, vocab, bias=False, device=dev, dtype=torch.bfloat16)
    hidden = torch.randn(seqs * q_len, hidden_size, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        full = kernel_launch_times(torch, lambda i: head(hidden), 2, 10)
        last = kernel_launch_times(torch, lambda i: last_token_logits(hidden, head, q_len), 8)
    full_us, last_us = statistics.median(full), statistics.median(last)
    print(f"# lm_head over a 32 x 512 prefill chunk: all positions {full_us:.0f} us, last positions {last_us:.0f} us",
          file=sys.stderr, flush=True)
    del head, hidden
    return {
        "decode_attention": {
            "workload": "32 seqs x 512-640 cached tokens, 32 query / 8 KV heads x 128, block 16, bf16 cache, "
                        "one layer per call over 8 layers",
            "us": round(us, 2), "bytes": moved, "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "torch_sequence_us": round(torch_us, 1),
        },
        "kv_write_decode_us": round(statistics.median(w_times), 2),
        "decode_step_rope_write_attention_us": round(step_us, 2),
        "prefill_attention": {
            "workload": "32 prompts x 512 tokens, 32 query / 8 KV heads x 128, causal, block 16, bf16 cache",
            "us": round(pre_us, 1), "TFLOP/s": round(pre_flop / pre_us / 1e6, 1),
            "torch_sequence_us": round(torch_pre_us, 1),
        },
        "lm_head_prefill_chunk": {"tokens": seqs * q_len, "all_positions_us": round(full_us, 1),
                                  "last_positions_us": round(last_us, 1)},
    }


def dense_comparator(torch, qt, m: int):
    """torch's dense bf16 F.linear (hipBLASLt) on the dequantized weight at the same shape: a
    comparator, not the reference. Rotates over enough weight copies to exceed the 256 MB
    Infinity Cache (a dense bf16 weight is four times the packed bytes)."""
    from llmopt.quantization import dequantize

    n, k = qt.shape
    w = dequantize(qt, torch.bfloat16)
    copies = max(2, -(-MIN_ROTATION_BYTES // (2 * n * k)))
    ws = [w] + [w.clone() for _ in range(copies - 1)]
    x = torch.randn(m, k, device="cuda:0").to(torch.bfloat16)
    f = torch.nn.functional.linear
    times = kernel_launch_times(torch, lambda i: f(x, ws[i % copies]), 2 * copies if m <= 64 else copies)
    us = statistics.median(times)
    dense_bytes = 2 * n * k + 2 * m * k + 2 * m * n
    out = {"op": f"F.linear bf16 [{m}, {k}] x [{n}, {k}]^T", "us": round(us, 2),
           "GB/s": round(dense_bytes / (us * 1e-6) / 1e9, 1),
           "TFLOP/s": round(2 * m * n * k / (us * 1e-6) / 1e12, 1), "weight_copies": copies}
    print(f"# dense comparator M={m}: {us:.1f} us, {out['GB/s']:.0f} GB/s, {out['TFLOP/s']:.1f} TFLOP/s",
          file=sys.stderr, flush=True)
    del ws, w
    return out


def gptq_down(torch, symmetric: bool):
    """The down projection (K 14336, N 4096) quantized by GPTQQuantizer(4 bits, group 128, damping
    0.01, activation order) on the GPU, calibrated on H = (2/128) X^T X of 128 rows gathered from a
    seeded N(0, 1) token-embedding table of width 14336 (seed 2) at seeded random ids (seed 3);
    weights 0.02 N(0, 1), seed 0."""
    from llmopt.quantization import GPTQQuantizer

    name, n, k = PROJECTIONS[3]
    dev = torch.device("cuda:0")
    table = torch.randn(1024, k, generator=torch.Generator().manual_seed(2))
    ids = torch.randint(0, 1024, (128,), generator=torch.Generator().manual_seed(3))
    x_cal = table[ids].to(dev)
    hessian = (2.0 / 128) * (x_cal.t() @ x_cal)
    w = (torch.randn(n, k, generator=torch.Generator().manual_seed(0)) * 0.02).to(dev)
    return GPTQQuantizer(bits=4, group_size=GROUP, symmetric=symmetric).quantize(w, hessian)


def bits_sweep(torch, ops):
    """The bit-width sweep on the down projection (K 14336, N 4096): RTN at 8 bits (one code per
    byte), 4 and 2 bits (two codes per byte), asymmetric, group 128; and 4-bit GPTQ (asymmetric
    and symmetric), which has the 4-bit layout. M in {1, 32, 2048}. Returns the rows and the
    asymmetric GPTQ weight (for the CPU baseline)."""
    from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer

    name, n, k = PROJECTIONS[3]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(4)
    weights = []
    for bits in (8, 4, 2):
        w = torch.randn(n, k, generator=gen, device=dev) * 0.02
        weights.append((f"rtn{bits}", RoundToNearestQuantizer(bits, GROUP, symmetric=False).quantize(w)))
        del w
    t0 = time.perf_counter()
    gptq_asym = gptq_down(torch, False)
    weights.append(("gptq4", gptq_asym))
    weights.append(("gptq4_sym", gptq_down(torch, True)))
    torch.cuda.synchronize()
    print(f"# GPTQ quantization of down (asymmetric and symmetric) on the GPU: {time.perf_counter() - t0:.1f} s",
          file=sys.stderr, flush=True)
    rows = []
    for label, qt in weights:
        bits = qt.bits
        copies = max(2, -(-MIN_ROTATION_BYTES // qt.qweight.numel()))
        qts = [QuantizedTensor(qt.qweight.clone(), qt.scales.clone(), qt.zeros.clone(), bits, GROUP, qt.symmetric,
                               qt.shape) for _ in range(copies)]
        for m in (1, 32, 2048):
            x = torch.randn(m, k, generator=gen, device=dev).to(torch.bfloat16)
            ops.quant_linear(x, qts[0], None, torch.bfloat16)
            times = kernel_launch_times(
                torch, lambda i: ops.quant_linear(x, qts[i % copies], None, torch.bfloat16), 2 * copies
            )
            us = statistics.median(times)
            gbs = algorithmic_bytes(m, n, k, bits=bits, asym=not qt.symmetric) / (us * 1e-6) / 1e9
            tflops = 2 * m * n * k / (us * 1e-6) / 1e12
            rows.append({"proj": name, "weights": label, "bits": bits, "symmetric": qt.symmetric, "M": m,
                         "us": round(us, 2), "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                         "TFLOP/s": round(tflops, 2), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4)})
            print(f"# bits {name} {label:9s} M={m:5d} {us:9.2f} us {gbs:8.1f} GB/s {tflops:8.2f} TFLOP/s",
                  file=sys.stderr, flush=True)
            del x
        del qts
    return rows, gptq_asym


def engine_config(torch, ops):
    """The reference engine's own quantized configuration: ``LLMEngine.from_pretrained(quantize=
    True)`` quantizes a float32 model with ``quantize_model_(model, bits=4, group_size=64)``
    (symmetric), and each QuantLinear computes in float32 (src/llmopt/engine/llm_engine.py:258-264,
    quantization/quant_linear.py:199-201, model/modeling.py:57-58). Per projection and M in
    {1, 32, 2048}: the fp32 path (three exact bf16 pieces per activation on the decode kernels,
    fp32 sums), bf16 activations on the same packed weight, and the reference's way in fp32 on the
    same GPU (F.linear on the dequantized fp32 weight, dense and cached), each rotating over at
    least 512 MiB of weight copies. GB/s counts the fp32 (or bf16) activations and outputs."""
    from llmopt.quantization import QuantizedTensor, RoundToNearestQuantizer, dequantize

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(6)
    group = 64
    rows = []
    f = torch.nn.functional.linear
    for name, n, k in PROJECTIONS:
        w = torch.randn(n, k, generator=gen, device=dev) * 0.02
        qt = RoundToNearestQuantizer(4, group, symmetric=True).quantize(w)
        del w
        packed = algorithmic_bytes(0, n, k, group=group, asym=False)
        copies = max(2, -(-MIN_ROTATION_BYTES // packed))
        qts = [qt] + [QuantizedTensor(qt.qweight.clone(), qt.scales.clone(), qt.zeros.clone(), 4, group, True,
                                      qt.shape) for _ in range(copies - 1)]
        dense = dequantize(qt, torch.float32)
        dcopies = max(2, -(-MIN_ROTATION_BYTES // (4 * n * k)))
        dws = [dense] + [dense.clone() for _ in range(dcopies - 1)]
        for m in (1, 32, 2048):
            reps = 2 * copies if m <= 64 else copies
            row = {"proj": name, "N": n, "K": k, "M": m, "bits": 4, "group": group, "symmetric": True}
            for label, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
                x = torch.randn(m, k, generator=gen, device=dev).to(dt)
                ops.quant_linear(x, qts[0], None, dt)
                us = statistics.median(
                    kernel_launch_times(torch, lambda i: ops.quant_linear(x, qts[i % copies], None, dt), reps))
                es = 4 if dt == torch.float32 else 2
                nbytes = packed + es * m * k + es * m * n
                row[f"{label}_us"] = round(us, 2)
                row[f"{label}_GB/s"] = round(nbytes / (us * 1e-6) / 1e9, 1)
                row[f"{label}_TFLOP/s"] = round(2 * m * n * k / (us * 1e-6) / 1e12, 2)
                if dt == torch.float32:
                    xr = x
            ref_us = statistics.median(kernel_launch_times(
                torch, lambda i: f(xr, dws[i % dcopies]), 2 * dcopies if m <= 64 else dcopies, 20))
            row["reference_fp32_us"] = round(ref_us, 2)
            row["fp32_vs_bf16"] = round(row["fp32_us"] / row["bf16_us"], 3)
            row["reference_fp32_vs_fp32"] = round(ref_us / row["fp32_us"], 3)
            rows.append(row)
            print(f"# engine config {name:8s} M={m:5d} fp32 {row['fp32_us']:9.2f} us ({row['fp32_GB/s']:7.1f} GB/s) "
                  f"bf16 {row['bf16_us']:8.2f} us  reference fp32 way {ref_us:9.2f} us", file=sys.stderr, flush=True)
            del x, xr
        del qts, dws, dense
    return rows


def shapes(torch, ops, rotations):
    """Per-projection kernel times at the decode (M <= 64: HBM-bound, GB/s) and prefill
    (M >= 256: MFMA-bound, TFLOP/s) batch sizes, each rotating over at least 512 MiB of that
    projection's weight copies; per-launch medians of graph replays of back-to-back launches."""
    bf16 = torch.bfloat16
    rows = []
    for m in (1, 2, 4, 8, 32, 64, 256, 2048, 8192):
        for name, n, k in PROJECTIONS:
            qts = rotations[name]
            x = torch.randn(m, k, device="cuda:0").to(bf16)
            ops.quant_linear(x, qts[0], None, bf16)
            reps = 2 * len(qts) if m <= 2048 else min(len(qts), 16)
            times = kernel_launch_times(
                torch, lambda i: ops.quant_linear(x, qts[i % len(qts)], None, bf16), reps
            )
            us = statistics.median(times)
            gbs = algorithmic_bytes(m, n, k) / (us * 1e-6) / 1e9
            tflops = 2 * m * n * k / (us * 1e-6) / 1e12
            decode = m <= 64
            rows.append({
                "proj": name, "N": n, "K": k, "M": m, "us": round(us, 2), "bound": "hbm" if decode else "mfma",
                "GB/s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 3),
                "TFLOP/s": round(tflops, 2), "mfma_frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                "frac": round(gbs / HBM_PEAK_GBS if decode else tflops / BF16_PEAK_TFLOPS, 4),
            })
            print(f"# shape {name:8s} M={m:5d} {us:9.2f} us {gbs:8.1f} GB/s ({gbs / HBM_PEAK_GBS:6.1%}) "
                  f"{tflops:8.2f} TFLOP/s ({tflops / BF16_PEAK_TFLOPS:6.1%})", file=sys.stderr, flush=True)
            del x
    return rows


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(torch, base, m: int, seconds: float, gptq=None):
    """The reference's host sequence on this machine's cores (`oracle.cpu_reference`, a
    restatement of QuantLinear.forward: dequantize once, cache, F.linear), on a bounded
    sample. `value`: the decode step (4 projections, M = `m`, bf16, dense weight cached) for
    `seconds`. `configs`: the reference's CPU configurations, warm (cached weight, median of a
    few calls) and cold (dequantize + F.linear, once per weight; M does not change its cost)."""
    from llmopt.quantization import RoundToNearestQuantizer
    from oracle.cpu_reference import ReferenceLinear

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(1)
    bf16 = torch.bfloat16

    def module(qt, dtype):
        return ReferenceLinear(qt.qweight.cpu(), qt.scales.cpu(), qt.zeros.cpu(), qt.bits, qt.group_size,
                               qt.symmetric, qt.shape, dtype)

    def timed(fn, reps):
        out = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            out.append(time.perf_counter() - t0)
        return statistics.median(out)

    rows = []

    def record(config, label, n, k, mm, bits, asym, warm_s, cold_s, dtype):
        es = 4 if dtype == torch.float32 else 2
        nbytes = algorithmic_bytes(mm, n, k, bits=bits, asym=asym) + (es - 2) * (mm * k + mm * n)
        row = {"config": config, "weights": label, "N": n, "K": k, "M": mm, "dtype": str(dtype).split(".")[-1],
               "warm_ms": round(warm_s * 1e3, 3), "warm_GB/s": round(nbytes / warm_s / 1e9, 2),
               "warm_TFLOP/s": round(2 * mm * n * k / warm_s / 1e12, 4)}
        if cold_s is not None:
            row["cold_ms"] = round(cold_s * 1e3, 2)
            row["cold_GB/s"] = round(nbytes / cold_s / 1e9, 3)
        rows.append(row)

    def run_weight(config, label, qt, ms, dtype):
        mod = module(qt, dtype)
        n, k = qt.shape
        x1 = torch.randn(1, k, generator=gen).to(dtype)
        t0 = time.perf_counter()
        mod(x1)  # cold: the first call dequantizes, then multiplies
        cold = time.perf_counter() - t0
        for i, mm in enumerate(ms):
            x = torch.randn(mm, k, generator=gen).to(dtype)
            reps = 10 if mm <= 64 else 3
            mod(x)
            record(config, label, n, k, mm, qt.bits, not qt.symmetric, timed(lambda: mod(x), reps),
                   cold if i == 0 else None, dtype)
        del mod

    t_start = time.perf_counter()
    # Config 1: one fp32 QuantLinear, K = N = 4096, M = 1, RTN b4 asymmetric g128 (weights seed 0).
    w1 = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(0)) * 0.02
    run_weight("1: fp32 linear", "rtn4", RoundToNearestQuantizer(4, GROUP, symmetric=False).quantize(w1), [1],
               torch.float32)
    # Configs 2 and 3: the four projections, decode and prefill batch sizes (M = 8192 skipped:
    # one such call is ~1 TFLOP of dense bf16 on the host).
    for name, n, k in PROJECTIONS:
        run_weight("2+3: projection", name, base[name], [1, 8, 32, 64, 256, 2048], bf16)
    # Config 4: the bit-width sweep on down.
    dn, dk = PROJECTIONS[3][1], PROJECTIONS[3][2]
    gen_w = torch.Generator().manual_seed(4)
    for bits in (8, 2):
        w = torch.randn(dn, dk, generator=gen_w) * 0.02
        run_weight("4: bit width", f"rtn{bits}", RoundToNearestQuantizer(bits, GROUP, symmetric=False).quantize(w),
                   [1, 32, 2048], bf16)
    if gptq is not None:
        run_weight("4: bit width", "gptq4", gptq, [1, 32, 2048], bf16)
    configs_s = time.perf_counter() - t_start

    # The headline-shaped sample: warm decode steps over the four projections.
    mods = {name: module(base[name], bf16) for name, _, _ in PROJECTIONS}
    xs = {name: torch.randn(m, k, generator=gen).to(bf16) for name, _, k in PROJECTIONS}
    step_bytes = sum(algorithmic_bytes(m, n, k) for _, n, k in PROJECTIONS)
    for name, _, _ in PROJECTIONS:
        mods[name](xs[name])
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
    print(f"# cpu baseline: {warm:.1f} GB/s warm decode step on {threads} threads ({_cpu_model()}); "
          f"{len(rows)} config rows in {configs_s:.1f} s", file=sys.stderr, flush=True)
    return {
        "value": round(warm, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{steps} warm decode steps (4 projections, M={m}, bf16, dense weight cached) in {elapsed:.1f} s; "
                  f"plus {len(rows)} configuration rows in {configs_s:.1f} s",
        "cpu_model": _cpu_model(),
        "torch": torch.__version__,
        "configs": rows,
    }


def _counter_per_dispatch(csv_path: Path, counter: str):
    """Mean value of `counter` per dispatch for the gate_up decode kernel and for the copy."""
    kern, copy = [], []
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            name = row["Kernel_Name"]
            value = float(row["Counter_Value"])
            grid = int(row["Grid_Size"])
            if "llmopt" in name and "decode_" in name:
                kern.append(value)
            elif "copy" in name.lower() and grid > 0:
                copy.append(value)
    # Keep the flush copies (COPY_BYTES, one before every launch; the counter may see half of
    # them), not the smaller copies that set up the weight copies.
    flushes = [v for v in copy if v * 1024 >= COPY_BYTES / 4]
    return kern, flushes


def pmc_blocks(torch, ops, prefill_block: bool) -> int:
    """Workloads for counter runs: gate_up at M = 8192 through the two-pass path and through the
    fused GEMM (one warm call, three counted calls each), or qkv and o at M = 32 and 64 (five
    calls each from two weight copies, a 256 MiB copy between calls so no call finds the
    previous one's weights in the caches; the copy also scales FETCH_SIZE / WRITE_SIZE)."""
    from llmopt.kernels._lib import ALGO_AUTO, ALGO_PREFILL

    base, layers, _ = build_layers(torch, 2, 1)
    bf16 = torch.bfloat16
    src = torch.empty(COPY_BYTES // 2, dtype=bf16, device="cuda:0")
    dst = torch.empty_like(src)
    if prefill_block:
        name, n, k = PROJECTIONS[2]
        x = torch.randn(8192, k, device="cuda:0").to(bf16)
        for algo in (ALGO_AUTO, ALGO_PREFILL):
            ops.quant_linear(x, base[name], None, bf16, algo=algo)
            torch.cuda.synchronize()
            for i in range(3):
                dst.copy_(src)
                ops.quant_linear(x, layers[i % 2][name], None, bf16, algo=algo)
            torch.cuda.synchronize()
        print(json.dumps({"pmc_prefill": "gate_up", "M": 8192, "calls": {"two-pass": 3, "fused_gemm": 3}}))
        return 0
    for name, n, k in PROJECTIONS[:2]:
        for m in (32, 64):
            x = torch.randn(m, k, device="cuda:0").to(bf16)
            ops.quant_linear(x, base[name], None, bf16)
            for i in range(5):
                dst.copy_(src)
                ops.quant_linear(x, layers[i % 2][name], None, bf16)
            torch.cuda.synchronize()
    print(json.dumps({"pmc_decode": ["qkv", "o"], "M": [32, 64], "calls": 5, "copy_bytes": COPY_BYTES}))
    return 0


def counters_summary(pmc_dir: Path) -> int:
    """Each counter's mean value per dispatch, per kernel and grid size, over every
    *counter_collection.csv under `pmc_dir` (one rocprofv3 --pmc pass each). Where the runs
    hold the 256 MiB flush copies, FETCH_SIZE and WRITE_SIZE (KiB) are also given in bytes,
    each scaled by what it reads for those copies, and TCP_TCC_READ_REQ_sum (L1 -> L2 read
    requests) in bytes at the copy's bytes per request."""
    table: dict[tuple[str, int], dict[str, list[float]]] = {}
    flush: dict[str, list[float]] = {}
    for path in sorted(pmc_dir.glob("**/*counter_collection.csv")):
        with open(path) as f:
            for row in csv.DictReader(f):
                name, cname, value = row["Kernel_Name"], row["Counter_Name"], float(row["Counter_Value"])
                key = (_kernel_short_name(name), int(row["Grid_Size"]))
                table.setdefault(key, {}).setdefault(cname, []).append(value)
                if "copy" in name.lower():
                    flush.setdefault(cname, []).append(value)
    # The flush copies are the largest copies of the runs (the others set up weight copies).
    flush = {c: [v for v in vals if v >= 0.25 * max(vals)] for c, vals in flush.items() if max(vals) > 0}
    scale = {}
    if "FETCH_SIZE" in flush:
        scale["FETCH_SIZE"] = COPY_BYTES / (statistics.median(flush["FETCH_SIZE"]) * 1024)
    if "WRITE_SIZE" in flush:
        scale["WRITE_SIZE"] = COPY_BYTES / (statistics.median(flush["WRITE_SIZE"]) * 1024)
    per_req = COPY_BYTES / statistics.median(flush["TCP_TCC_READ_REQ_sum"]) if "TCP_TCC_READ_REQ_sum" in flush else 0
    notes = [f"{c} scale {v:.4f}" for c, v in sorted(scale.items())]
    if per_req:
        notes.append(f"{per_req:.1f} bytes per TCP_TCC_READ_REQ")
    if notes:
        print("# 256 MiB flush copies: " + ", ".join(notes))
    for (kname, grid), counters in sorted(table.items()):
        calls = max(len(v) for v in counters.values())
        print(f"{kname}  grid {grid}  dispatches {calls}")
        for cname, vals in sorted(counters.items()):
            mean = statistics.mean(vals)
            extra = ""
            if cname in scale:
                extra = f"   = {mean * 1024 * scale[cname] / 1e6:10.2f} MB"
            elif cname == "TCP_TCC_READ_REQ_sum" and per_req:
                extra = f"   = {mean * per_req / 1e6:10.2f} MB read from L2"
            print(f"    {cname:32s} {mean:16.1f}{extra}")
    return 0


def _kernel_short_name(name: str) -> str:
    import re

    name = name.replace("void llmopt::(anonymous namespace)::", "").replace("llmopt::", "")
    return name.split(">(")[0] + ">" if ">(" in name else re.sub(r"\(.*$", "", name)[:100]


def trace_kernels(trace_csv: Path) -> int:
    """Summarise a rocprofv3 kernel trace per (kernel, grid, workgroup), every kernel of the run:
    count, mean, median, min and max kernel-only duration in microseconds, VGPR / AGPR counts and
    LDS bytes, sorted by total time."""
    stats: dict[tuple, list[float]] = {}
    regs: dict[tuple, tuple] = {}
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            block = int(r["Workgroup_Size_X"])
            key = (_kernel_short_name(r["Kernel_Name"]), int(r["Grid_Size_X"]) // block, block)
            stats.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
            regs[key] = (r.get("VGPR_Count", ""), r.get("Accum_VGPR_Count", ""), r.get("LDS_Block_Size", ""))
    print("count\tmean\tmedian\tmin\tmax\tgrid x workgroup\tVGPR/AGPR\tLDS\tkernel")
    for key, v in sorted(stats.items(), key=lambda kv: -sum(kv[1])):
        vg, ag, lds = regs[key]
        print(f"{len(v)}\t{statistics.mean(v):.2f}\t{statistics.median(v):.2f}\t{min(v):.2f}\t{max(v):.2f}\t"
              f"{key[1]}x{key[2]}\t{vg}/{ag}\t{lds}\t{key[0]}")
    return 0


def trace_runs(trace_csv: Path, min_launches: int = 8) -> int:
    """Summarise a rocprofv3 kernel trace of this script by runs: consecutive dispatches of
    this library's kernels (and of hipBLASLt's, which its two-pass path and torch's dense
    comparator launch) with the same main kernel (name, grid, workgroup) form one run -- one
    timed block, e.g. one (projection, M) of the per-shape sweep. The split-K reductions that
    follow a kernel and the dequantization that precedes a hipBLASLt GEMM are counted with it.
    Prints one line per run of at least `min_launches` main-kernel dispatches: kernel, grid x
    workgroup, count, median and mean kernel-only duration in microseconds."""
    short = _kernel_short_name
    with open(trace_csv, newline="") as f:
        rows = sorted((r for r in csv.DictReader(f) if "llmopt" in r["Kernel_Name"] or "Cijk" in r["Kernel_Name"]),
                      key=lambda r: int(r["Start_Timestamp"]))
    runs: list[tuple[tuple, dict]] = []
    ahead: list[tuple[tuple, float]] = []  # a dequantization waiting for the GEMM after it
    for i, r in enumerate(rows):
        block = int(r["Workgroup_Size_X"])
        key = (short(r["Kernel_Name"])[:90], int(r["Grid_Size_X"]) // block, block)
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        nxt = rows[i + 1]["Kernel_Name"] if i + 1 < len(rows) else ""
        if key[0].startswith("dequant_") and "Cijk" in nxt:
            ahead.append((key, dur))
            continue
        if not key[0].startswith("splitk_reduce") and (not runs or runs[-1][0] != key):
            runs.append((key, {}))
        if runs:
            runs[-1][1].setdefault(key, []).append(dur)
            for k, d in ahead:
                runs[-1][1].setdefault(k, []).append(d)
            ahead.clear()
    for i, (main_key, kernels) in enumerate(runs):
        if len(kernels[main_key]) < min_launches:
            continue
        parts = [f"{k[0]} {k[1]}x{k[2]} n={len(v)} median={statistics.median(v):.2f} mean={statistics.mean(v):.2f}"
                 for k, v in kernels.items()]
        print(f"run {i}: " + " | ".join(parts))
    return 0


def traffic_summary(pmc_dir: Path) -> int:
    """HBM bytes per launch of the dominant kernel from FETCH_SIZE and WRITE_SIZE runs."""
    fetch_csv = next(pmc_dir.glob("**/fetch*counter_collection.csv"))
    write_csv = next(pmc_dir.glob("**/write*counter_collection.csv"))
    kf, cf = _counter_per_dispatch(fetch_csv, "FETCH_SIZE")
    kw, cw = _counter_per_dispatch(write_csv, "WRITE_SIZE")
    # The copy moves COPY_BYTES in and COPY_BYTES out: its counters (KiB) give the scale factor.
    copy_fetch = statistics.median(cf) * 1024
    copy_write = statistics.median(cw) * 1024
    f_scale = COPY_BYTES / copy_fetch
    w_scale = COPY_BYTES / copy_write
    kfetch = statistics.median(kf) * 1024 * f_scale
    kwrite = statistics.median(kw) * 1024 * w_scale
    out = {
        "kernel": "quantized-linear decode, gate_up M=1",
        "fetch_bytes_per_launch": round(kfetch),
        "write_bytes_per_launch": round(kwrite),
        "hbm_bytes_per_launch": round(kfetch + kwrite),
        "algorithmic_bytes": algorithmic_bytes(1, 28672, 4096),
        "fetch_scale": round(f_scale, 4),
        "write_scale": round(w_scale, 4),
        "copy_bytes": COPY_BYTES,
        "samples": {"kernel_fetch": len(kf), "kernel_write": len(kw), "copy_fetch": len(cf), "copy_write": len(cw)},
        "build": source_digest(),
    }
    TRAFFIC_FILE.parent.mkdir(exist_ok=True)
    TRAFFIC_FILE.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
