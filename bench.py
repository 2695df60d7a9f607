"""Benchmark of the hot path on one MI355X.

Workloads (synthetic seeded inputs, random-init weights of the named shapes):
  * ResNet-50 v1.5, FP32 NCHW, batch 32: one step = one inference of the
    batch through BuildEngine/ExecutionContext (53 fused conv nodes, MaxPool,
    GAP, Flatten view, Gemm), replayed as one hipGraph. `value` is img/s.
    Batch 64 (the top of the reference's dynamic-batch profile) on its own
    engine is reported beside it.
  * FP16 FFN block M=4096, H=1024, I=4096 (GemmGelu -> Gemm -> SkipLayerNorm):
    reported as TFLOP/s of its two GEMMs beside the main line.
  * FP16 Softmax over attention scores [16*16*1024, 1024] and a standalone
    FP16 LayerNorm of the same shape: reported as GB/s (HBM-bound) beside the
    main line.
  * Fused FP16 attention [8, 16, 2048, 128], full and causal: TFLOP/s.

Timing: the first run tunes every op (TuneOnMiss, cache in a temporary
directory). Then W untimed warm-up steps and K timed steps bracketed by
torch.cuda.synchronize(), on an engine built from that cache with profiling
off; each step is RunAsync on the measured stream + Synchronize, as in the
reference harness (benchmarks/resnet50_native.cpp:281-291). A second set of K
steps on a profiled engine (per-op HIP event pairs recorded inside the graph)
gives each kernel's duration; the dominant kernel family (the FP32
implicit-GEMM convolutions) is priced against the FP32 MFMA peak from those
durations.

The CPU baseline is the reference's CPU path (the same graph in PyTorch-CPU
FP32, oracle/torch_cpu.py) on a bounded sample, timed on this host.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ResNet-50 fp32 img/s @bs32 (% FP32 MFMA peak); FFN fp16 TFLOP/s @M=4096"
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2516.6
KERNEL_TIMING_LAUNCHES = 20
CONV_OPS = ("FusedConvBatchNormRelu", "FusedConvBatchNorm", "FusedConvBatchNormAddRelu", "Conv")


def log(*args) -> None:
    print(*args, file=sys.stderr, flush=True)


def _context(graph, feeds, cache_dir: str, profiling: bool, tuning_mode: str):
    import numpy as np
    import torch

    from cutriton_amd import engine, workloads

    opts = engine.CompileOptions(tuning_mode=tuning_mode, tuning_cache_dir=cache_dir,
                                 enable_profiling=profiling, enable_cuda_graph=True,
                                 tuning_warmup_iterations=3, tuning_measurement_iterations=10)
    eng = engine.build_engine(workloads.to_model(graph), opts)
    ctx = eng.create_execution_context()
    inputs = {n: torch.from_numpy(np.ascontiguousarray(v)).to("cuda:0") for n, v in feeds.items()}
    for name, t in inputs.items():
        ctx.bind_input(name, t, layout=graph.inputs[name][2])
    outputs = {}
    for name in graph.outputs:
        shape, dtype = eng.value_desc(name)
        outputs[name] = torch.empty(shape, dtype=getattr(torch, dtype), device="cuda:0")
        ctx.bind_output(name, outputs[name], layout=eng.value_layout(name))
    return eng, ctx, (inputs, outputs)


def run_workload(graph, feeds, steps: int, warmup: int, cache_dir: str):
    """Tunes `graph` (TuneOnMiss), then:
      1. a profiled engine replays `steps` steps and sums each op's HIP-event
         duration (kernel time, read from the event nodes inside the graph);
      2. an unprofiled engine built from the tuning cache (UseCache) replays
         `steps` steps bracketed by device synchronisation: the wall time of
         these is the step time.
      3. each op's selected kernels are timed over back-to-back launches on
         the measured stream (ExecutionContext::TimeOp).
    Returns (ms per step, per-op kernel ms, per-op graph-event ms per step,
    plan ops, selected candidate per op)."""
    import torch

    stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    eng, ctx, keep = _context(graph, feeds, cache_dir, True, "tune_on_miss")
    t0 = time.perf_counter()
    ctx.run_async(handle)  # first run: tuning, module loads, graph capture
    ctx.synchronize()
    log(f"  first run (tuning + capture) {time.perf_counter() - t0:.1f} s")
    for _ in range(warmup):
        ctx.run_async(handle)
        ctx.synchronize()
    ops = eng.ops()
    op_ms = [0.0] * len(ops)
    for _ in range(steps):
        ctx.run_async(handle)
        ctx.synchronize()
        for i, (_, ms) in enumerate(ctx.profile_events()):
            op_ms[i] += ms
    selected = [op.candidates[s] for op, s in zip(ops, ctx.selected_candidates(len(ops)))]
    del ctx, eng, keep

    eng, ctx, keep = _context(graph, feeds, cache_dir, False, "use_cache")
    ctx.run_async(handle)
    ctx.synchronize()
    plain = [op.candidates[s] for op, s in zip(eng.ops(), ctx.selected_candidates(len(ops)))]
    if plain != selected:
        raise RuntimeError("the tuning cache did not reproduce the tuned plan")
    for _ in range(warmup):
        ctx.run_async(handle)
        ctx.synchronize()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for _ in range(steps):
        ctx.run_async(handle)
        ctx.synchronize()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - wall0) * 1e3 / steps
    # Kernel time per op on the same stream: back-to-back launches between
    # one event pair, free of the event nodes' dispatch gaps.
    kernel_ms = [ctx.time_op(i, KERNEL_TIMING_LAUNCHES, handle) for i in range(len(ops))]
    graph_event_ms = [v / steps for v in op_ms]
    return ms_per_step, kernel_ms, graph_event_ms, ops, selected


TRAFFIC_SUMMARY = ROOT / "profiles" / "resnet50_bs32_fp32_hbm_traffic.md"


def measured_traffic() -> int | None:
    """HBM bytes per conv-family launch from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter
    on a copy of known size). Counters need rocprofv3 around the process, so
    the figure is read from that summary, not measured in this run."""
    try:
        for line in TRAFFIC_SUMMARY.read_text().splitlines():
            if line.startswith("conv_family_hbm_bytes_per_launch ="):
                return int(line.split("=", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def bench_resnet(args, cache_dir: str, batch: int = 32) -> dict:
    from cutriton_amd import workloads

    graph = workloads.resnet50(batch)
    x = workloads.resnet50_input(batch)
    ms_per_step, kernel_ms, event_ms, ops, selected = run_workload(graph, {"input": x}, args.steps, args.warmup,
                                                                   cache_dir)
    flops = workloads.node_flops(graph)
    conv_flops = sum(v for k, v in flops.items() if k != "classifier")
    total_flops = sum(flops.values())
    img_s = batch * 1e3 / ms_per_step
    conv_idx = [i for i, op in enumerate(ops) if op.op_type in CONV_OPS]
    conv_ms = sum(kernel_ms[i] for i in conv_idx)
    launches = len(conv_idx)
    achieved = conv_flops / (conv_ms * 1e-3) / 1e12

    def op_flops(name: str) -> int:
        keys = [k for k in flops if name.startswith(k)]
        return flops[max(keys, key=len)] if keys else 0

    per_op = sorted(((kernel_ms[i], ops[i].node_name, selected[i].split(":", 1)[-1], op_flops(ops[i].node_name))
                     for i in range(len(ops))), reverse=True)
    log(f"  resnet50 bs{batch}: {ms_per_step:.3f} ms/step, {img_s:.1f} img/s; kernel time per step: conv "
        f"{conv_ms:.3f} ms, all {sum(kernel_ms):.3f} ms (profiled graph events {sum(event_ms):.3f} ms)")
    for ms, name, var, fl in per_op:
        rate = f"{fl / (ms * 1e-3) / 1e12:6.1f} TF/s" if fl and ms > 0 else " " * 11
        log(f"    {ms * 1e3:8.1f} us {rate}  {name}  [{var}]")
    return {
        "ms_per_step": ms_per_step,
        "img_s": img_s,
        "tflops": total_flops / (ms_per_step * 1e-3) / 1e12,
        "pct_fp32_mfma_peak": 100.0 * total_flops / (ms_per_step * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
        "roofline": {
            "kernel": "conv_bn[_add]_relu_fp32 implicit-GEMM family (53 launches/step)",
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": f"{TRAFFIC_SUMMARY.relative_to(ROOT)} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)",
            "flop_per_launch": conv_flops / launches,
            "launches_per_step": launches,
            "avg_launch_us": conv_ms * 1e3 / launches,
            "timing": f"ExecutionContext::TimeOp, {KERNEL_TIMING_LAUNCHES} back-to-back launches per op, HIP events",
        },
        "selected": selected,
    }


def bench_ffn(args, cache_dir: str) -> dict:
    from cutriton_amd import workloads

    m, h, i = 4096, 1024, 4096
    graph, x = workloads.ffn(m, h, i)
    ms_per_step, kernel_ms, _, ops, selected = run_workload(graph, {"x": x}, args.steps, args.warmup, cache_dir)
    gemm_flops = 2 * m * h * i
    per_op = {op.op_type: kernel_ms[j] for j, op in enumerate(ops)}
    out = {
        "workload": f"ffn_fp16_m{m}_h{h}_i{i}",
        "ms_per_step": ms_per_step,
        "tflops_block": 2 * gemm_flops / (ms_per_step * 1e-3) / 1e12,
        "gemm_gelu_us": per_op["GemmGelu"] * 1e3,
        "gemm_us": per_op["Gemm"] * 1e3,
        "skip_layer_norm_us": per_op["SkipLayerNormalization"] * 1e3,
        "gemm_gelu_tflops": gemm_flops / (per_op["GemmGelu"] * 1e-3) / 1e12,
        "gemm_tflops": gemm_flops / (per_op["Gemm"] * 1e-3) / 1e12,
        "skip_layer_norm_gbps": 3 * m * h * 2 / (per_op["SkipLayerNormalization"] * 1e-3) / 1e9,
        "selected": selected,
    }
    out["pct_fp16_mfma_peak_gemms"] = 100.0 * (2 * gemm_flops) / ((per_op["GemmGelu"] + per_op["Gemm"]) * 1e-3) \
        / 1e12 / FP16_MFMA_PEAK_TFLOPS
    log(f"  ffn: {ms_per_step * 1e3:.1f} us/step; GemmGelu {out['gemm_gelu_us']:.1f} us "
        f"({out['gemm_gelu_tflops']:.0f} TF), Gemm {out['gemm_us']:.1f} us ({out['gemm_tflops']:.0f} TF), "
        f"SkipLN {out['skip_layer_norm_us']:.1f} us; selected {[s.rsplit(':', 1)[1] for s in selected]}")
    return out


def bench_norms(args, cache_dir: str) -> dict:
    """Softmax over attention scores (16 sequences x 16 heads x 1024 queries,
    1024 keys) and a standalone LayerNorm of the same [262144, 1024] shape,
    FP16: each reads and writes 512 MiB once (the LayerNorm's scale and bias
    add 4 KiB). 512 MiB exceeds the 256 MB Infinity Cache, so back-to-back
    launches stream from HBM."""
    import numpy as np

    from cutriton_amd import workloads

    rows, columns = 16 * 16 * 1024, 1024
    rng = np.random.default_rng(workloads.SEED)
    x = (rng.standard_normal((rows, columns), dtype=np.float32) * 4).astype(np.float16)
    out: dict = {"softmax_shape": [rows, columns], "layer_norm_shape": [rows, columns]}
    moved = 2 * rows * columns * 2
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, columns), "float16", "")
    g.add("softmax", "Softmax", ["x"], ["y"], axis=-1)
    g.outputs.append("y")
    _, kernel_ms, _, _, selected = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir)
    out.update(softmax_us=kernel_ms[0] * 1e3, softmax_gbps=moved / (kernel_ms[0] * 1e-3) / 1e9,
               softmax_variant=selected[0].rsplit(":", 1)[1])
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, columns), "float16", "")
    gamma = g.constant("gamma", rng.uniform(0.5, 1.5, columns).astype(np.float16))
    beta = g.constant("beta", rng.normal(0.0, 0.1, columns).astype(np.float16))
    g.add("ln", "LayerNormalization", ["x", gamma, beta], ["y"], axis=-1, epsilon=1e-5)
    g.outputs.append("y")
    _, kernel_ms, _, _, _ = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir)
    out.update(layer_norm_us=kernel_ms[0] * 1e3, layer_norm_gbps=(moved + 4 * columns) / (kernel_ms[0] * 1e-3) / 1e9)
    log(f"  softmax: {out['softmax_us']:.1f} us ({out['softmax_gbps']:.0f} GB/s, {out['softmax_variant']}); "
        f"layer norm: {out['layer_norm_us']:.1f} us ({out['layer_norm_gbps']:.0f} GB/s)")
    return out


def bench_attention(args, cache_dir: str) -> dict:
    """Fused attention, FP16 [batch 8, heads 16, sequence 2048, head dim 128],
    without and with the causal mask. FLOPs: 4 B H Sq Sk D for the two
    products (the causal mask needs about half, counted as the exact number
    of unmasked query-key pairs)."""
    import numpy as np

    from cutriton_amd import workloads

    b, h, s, d = 8, 16, 2048, 128
    rng = np.random.default_rng(workloads.SEED)
    feeds = {n: rng.standard_normal((b, h, s, d), dtype=np.float32).astype(np.float16) for n in ("q", "k", "v")}
    out: dict = {"shape": [b, h, s, d]}
    for causal in (False, True):
        g = workloads.GraphSpec()
        for n in feeds:
            g.inputs[n] = ((b, h, s, d), "float16", "")
        g.add("attention", "Attention", ["q", "k", "v"], ["o"], is_causal=int(causal))
        g.outputs.append("o")
        _, kernel_ms, _, _, _ = run_workload(g, feeds, args.steps, args.warmup, cache_dir)
        pairs = s * (s + 1) // 2 if causal else s * s
        flops = 4 * b * h * pairs * d
        key = "causal" if causal else "full"
        out[f"{key}_us"] = kernel_ms[0] * 1e3
        out[f"{key}_tflops"] = flops / (kernel_ms[0] * 1e-3) / 1e12
    log(f"  attention {b}x{h}x{s}x{d}: {out['full_us']:.1f} us ({out['full_tflops']:.0f} TF), "
        f"causal {out['causal_us']:.1f} us ({out['causal_tflops']:.0f} TF)")
    return out


def bench_copy(args, cache_dir: str) -> dict:
    """One Relu over 64 Mi non-negative floats: the relu_fp32 kernel reads and
    writes exactly 256 MiB each. Its GB/s is the streaming reference for the
    bandwidth kernels, and its FETCH_SIZE / WRITE_SIZE counters calibrate the
    HBM traffic figures of the other kernels."""
    import numpy as np

    from cutriton_amd import workloads

    count = 64 << 20
    g = workloads.GraphSpec()
    g.inputs["x"] = ((count,), "float32", "")
    g.add("copy", "Relu", ["x"], ["y"])
    g.outputs.append("y")
    x = np.abs(np.random.default_rng(workloads.SEED).standard_normal(count, dtype=np.float32))
    ms_per_step, op_kernel_ms, _, ops, _ = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir)
    kernel_ms = op_kernel_ms[0]
    out = {"workload": "relu_fp32_64Mi", "bytes": 2 * 4 * count, "kernel_us": kernel_ms * 1e3,
           "gbps": 2 * 4 * count / (kernel_ms * 1e-3) / 1e9, "ms_per_step": ms_per_step}
    log(f"  copy: {out['kernel_us']:.1f} us, {out['gbps']:.0f} GB/s")
    return out


def cpu_baseline(budget_s: float) -> dict:
    """The same ResNet-50 bs32 graph in PyTorch-CPU FP32, timed for about
    `budget_s` seconds after one warm-up batch."""
    import torch

    from cutriton_amd import workloads
    from oracle import torch_cpu

    cores = os.cpu_count() or 1
    # The host share of one GPU is capped by OMP_NUM_THREADS where it is set.
    torch.set_num_threads(min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    batch = 32
    graph = workloads.resnet50(batch)
    consts = torch_cpu.prepare(graph)
    x = torch.from_numpy(workloads.resnet50_input(batch))
    torch_cpu.run(graph, consts, {"input": x})
    times = []
    t_start = time.perf_counter()
    while not times or (time.perf_counter() - t_start < budget_s and len(times) < 10):
        t0 = time.perf_counter()
        torch_cpu.run(graph, consts, {"input": x})
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    cpu_model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(batch / med, 2),
        "unit": "img/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"ResNet-50 bs32 FP32 PyTorch-CPU restatement of the same graph, {len(times)} batches after 1 "
                  f"warm-up, median {med:.2f} s/batch; host {cpu_model} ({cores} logical CPUs)",
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=30)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=("all", "resnet50", "ffn", "norms", "attention", "copy"), default="all")
    parser.add_argument("--tuning-cache", default="",
                        help="tuning cache folder to reuse (default: a fresh temporary folder, so every op is tuned)")
    parser.add_argument("--cpu-baseline-seconds", type=float, default=15.0,
                        help="bounded CPU sample; 0 skips the CPU baseline")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (cuda:0)", file=sys.stderr)
        return 2
    log(f"device: {torch.cuda.get_device_name(0)}")
    cache_dir = args.tuning_cache or tempfile.mkdtemp(prefix="cutriton-tuning-")
    os.makedirs(cache_dir, exist_ok=True)
    result = {
        "metric": METRIC, "value": None, "unit": "img/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic (seeded N(0,1) inputs, random-init weights)",
        "config": {"workload": "resnet50_v1.5_fp32_nchw_bs32", "global_batch": 32, "image": [3, 224, 224],
                   "parallelism": "single-gpu"},
    }
    if args.workload in ("all", "resnet50"):
        r = bench_resnet(args, cache_dir)
        result.update(value=round(r["img_s"], 2), ms_per_step=round(r["ms_per_step"], 4),
                      pct_fp32_mfma_peak=round(r["pct_fp32_mfma_peak"], 2), roofline=r["roofline"])
        result["resnet50_tflops"] = round(r["tflops"], 3)
        # The profile-max batch of the same graph, on its own tuned engine.
        r64 = bench_resnet(args, cache_dir, batch=64)
        result["resnet50_bs64"] = {"img_s": round(r64["img_s"], 2), "ms_per_step": round(r64["ms_per_step"], 4),
                                   "pct_fp32_mfma_peak": round(r64["pct_fp32_mfma_peak"], 2),
                                   "conv_tflops": r64["roofline"]["achieved"]}
    if args.workload in ("all", "ffn"):
        f = bench_ffn(args, cache_dir)
        f.pop("selected", None)
        result["ffn"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in f.items()}
        if args.workload == "ffn":
            result.update(value=round(f["tflops_block"], 3), unit="TFLOP/s", ms_per_step=round(f["ms_per_step"], 4),
                          dtype="fp16", config={"workload": f["workload"], "parallelism": "single-gpu"})
    if args.workload in ("all", "norms"):
        n = bench_norms(args, cache_dir)
        result["norms"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in n.items()}
        if args.workload == "norms":
            result.update(value=round(n["softmax_gbps"], 1), unit="GB/s", dtype="fp16",
                          ms_per_step=round(n["softmax_us"] * 1e-3, 4),
                          config={"workload": "softmax_fp16_262144x1024", "parallelism": "single-gpu"})
    if args.workload in ("all", "attention"):
        a = bench_attention(args, cache_dir)
        result["attention"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in a.items()}
        if args.workload == "attention":
            result.update(value=round(a["full_tflops"], 3), unit="TFLOP/s", dtype="fp16",
                          ms_per_step=round(a["full_us"] * 1e-3, 4),
                          config={"workload": "attention_fp16_b8_h16_s2048_d128", "parallelism": "single-gpu"})
    if args.workload == "copy":
        c = bench_copy(args, cache_dir)
        result.update(value=round(c["gbps"], 1), unit="GB/s", ms_per_step=round(c["ms_per_step"], 4),
                      config={"workload": c["workload"], "parallelism": "single-gpu"}, copy=c)
    if args.cpu_baseline_seconds > 0 and args.workload in ("all", "resnet50"):
        result["cpu_baseline"] = cpu_baseline(args.cpu_baseline_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
