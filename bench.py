"""Benchmark of the hot path on one MI355X.

Workloads (synthetic seeded inputs, random-init weights of the named shapes):
  * ResNet-50 v1.5, FP32 NCHW, on one engine built with the dynamic batch
    profile min1/opt32/max64 (workspace planned at the profile max, one
    hipGraph per shape), run at batch 32 and 64: one step = one inference of
    the batch through BuildEngine/ExecutionContext (53 fused conv nodes,
    MaxPool, GAP, Flatten view, Gemm). `value` is img/s at batch 32.
  * ResNet-50 at batch 1 on a static engine, and the single
    FusedConvBatchNormRelu node x[1,64,56,56] * W[64,64,3,3].
  * FP16 FFN block GemmGelu -> Gemm -> SkipLayerNorm at M=4096, H=1024,
    I=4096 on the dynamic M profile min128/opt4096/max8192, and at M=512,
    H=768, I=3072 on a static engine: TFLOP/s of the two GEMMs.
  * FP16 Softmax over attention scores [16*16*1024, 1024] and a standalone
    FP16 LayerNorm of the same shape: GB/s (HBM-bound).
  * Fused FP16 attention [8, 16, 2048, 128], full and causal: TFLOP/s.

Timing: the first run tunes every op (TuneOnMiss, cache in a temporary
directory). Then W untimed warm-up steps and K timed steps bracketed by
torch.cuda.synchronize(), on an engine built from that cache with profiling
off; each step is RunAsync on the measured stream + Synchronize, as in the
reference harness (benchmarks/resnet50_native.cpp:281-291,
benchmarks/transformer_ffn_native.cpp:188-218). Each op's kernels are then
timed over back-to-back launches between HIP events on the same stream
(ExecutionContext::TimeOp); the roofline blocks divide algorithmic FLOPs by
those durations.

HBM traffic: two child processes rerun the ResNet bs32 and FFN M=4096 engines
from the tuning cache under `rocprofv3 --pmc FETCH_SIZE` and `--pmc
WRITE_SIZE`, together with a Relu over 64 Mi floats whose known 256 MiB read
and 256 MiB write calibrate both counters. The calibrated bytes per launch of
the conv family and of the FFN GEMMs are the roofline blocks' `traffic`.

The CPU baseline is the reference's CPU path (the same graphs in PyTorch-CPU
FP32, oracle/torch_cpu.py), timed on this host: 3 warm-ups, then at least 10
timed iterations, median reported.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import csv
import dataclasses
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time
from collections import defaultdict
from pathlib import Path
from typing import Any, NamedTuple

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ResNet-50 fp32 img/s @bs32 (% FP32 MFMA peak); FFN fp16 TFLOP/s @M=4096"
FP32_MFMA_PEAK_TFLOPS = 157.3
FP16_MFMA_PEAK_TFLOPS = 2516.6
KERNEL_TIMING_LAUNCHES = 20
CONV_OPS = ("FusedConvBatchNormRelu", "FusedConvBatchNorm", "FusedConvBatchNormAddRelu", "Conv")
RESNET_PROFILE = {"batch": {"input": ((1, 3, 224, 224), (32, 3, 224, 224), (64, 3, 224, 224))}}
FFN_SHAPE = (4096, 1024, 4096)
FFN_PROFILE = {"tokens": {"x": ((128, 1024), (4096, 1024), (8192, 1024))}}
FFN_SMALL_SHAPE = (512, 768, 3072)
COPY_FLOATS = 64 << 20
CPU_WARMUPS = 3
CPU_MIN_ITERATIONS = 10


def log(*args) -> None:
    print(*args, file=sys.stderr, flush=True)


def _context(graph, feeds, cache_dir: str, profiling: bool, tuning_mode: str, profiles=None):
    """An engine and execution context for `graph` with `feeds` bound. With
    `profiles` ({name: {input: (min, opt, max)}}) the engine is built for
    that shape profile and the context runs at the feeds' shapes."""
    import numpy as np
    import torch

    from cutriton_amd import engine, workloads

    opts = engine.CompileOptions(tuning_mode=tuning_mode, tuning_cache_dir=cache_dir,
                                 enable_profiling=profiling, enable_cuda_graph=True,
                                 tuning_warmup_iterations=3, tuning_measurement_iterations=10,
                                 shape_profiles=dict(profiles or {}))
    eng = engine.build_engine(workloads.to_model(graph), opts)
    ctx = eng.create_execution_context()
    inputs = {n: torch.from_numpy(np.ascontiguousarray(v)).to("cuda:0") for n, v in feeds.items()}
    if profiles:
        ctx.select_shape_profile(next(iter(profiles)))
        for name, t in inputs.items():
            ctx.set_input_shape(name, tuple(t.shape))
        ctx.resolve_shapes()
    for name, t in inputs.items():
        ctx.bind_input(name, t, layout=graph.inputs[name][2])
    outputs = {}
    for name in graph.outputs:
        if profiles:
            shape, dtype, layout = ctx.resolved_desc(name)
        else:
            (shape, dtype), layout = eng.value_desc(name), eng.value_layout(name)
        outputs[name] = torch.empty(shape, dtype=getattr(torch, dtype), device="cuda:0")
        ctx.bind_output(name, outputs[name], layout=layout)
    return eng, ctx, (inputs, outputs)


class Run(NamedTuple):
    ms_per_step: float          # wall time per step over the timed steps
    median_event_ms: float      # median of per-step HIP event pairs
    kernel_ms: list[float]      # per op: TimeOp kernel duration
    graph_event_ms: list[float]  # per op: profiled-graph event duration per step
    ops: list[Any]
    selected: list[str]         # per op: the tuned candidate


def run_workload(graph, feeds, steps: int, warmup: int, cache_dir: str, profiles=None, warm_ms: float = 0.0) -> Run:
    """Tunes `graph` (TuneOnMiss), then:
      1. a profiled engine replays `steps` steps and sums each op's HIP-event
         duration (kernel time, read from the event nodes inside the graph);
      2. an unprofiled engine built from the tuning cache (UseCache) replays
         `steps` steps bracketed by device synchronisation: the wall time of
         these is the step time.
      3. the same engine's steps are timed again one by one between HIP
         events on that stream (the reference harness's figure), median kept;
      4. each op's selected kernels are timed over back-to-back launches on
         the measured stream (ExecutionContext::TimeOp)."""
    import torch

    # A stream of the caller's own (default priority), as the reference
    # harness creates one: RunAsync enqueues the graph on it, so events
    # recorded on it bracket the step.
    stream = torch.cuda.Stream()
    handle = stream.cuda_stream
    torch.cuda.synchronize()
    eng, ctx, keep = _context(graph, feeds, cache_dir, True, "tune_on_miss", profiles)
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

    eng, ctx, keep = _context(graph, feeds, cache_dir, False, "use_cache", profiles)
    ctx.run_async(handle)
    ctx.synchronize()
    plain = [op.candidates[s] for op, s in zip(eng.ops(), ctx.selected_candidates(len(ops)))]
    if plain != selected:
        raise RuntimeError("the tuning cache did not reproduce the tuned plan")
    for _ in range(warmup):
        ctx.run_async(handle)
        ctx.synchronize()
    # Steps of about 0.1 ms leave the GPU below its steady clocks after a few
    # warm-up steps (measured: 113 us per FFN step after 5, 105 us after 200),
    # so a workload may ask for warm-up by time as well.
    warm0 = time.perf_counter()
    while (time.perf_counter() - warm0) * 1e3 < warm_ms:
        ctx.run_async(handle)
        ctx.synchronize()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for _ in range(steps):
        ctx.run_async(handle)
        ctx.synchronize()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - wall0) * 1e3 / steps
    # The reference harness's figure: event pair around each RunAsync,
    # median over the steps (resnet50_native.cpp:281-291).
    latencies = []
    for _ in range(steps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        ctx.run_async(handle)
        end.record(stream)
        ctx.synchronize()
        latencies.append(start.elapsed_time(end))
    median_ms = sorted(latencies)[len(latencies) // 2]
    # Kernel time per op on the same stream: back-to-back launches between
    # one event pair, free of the event nodes' dispatch gaps.
    kernel_ms = [ctx.time_op(i, KERNEL_TIMING_LAUNCHES, handle) for i in range(len(ops))]
    graph_event_ms = [v / steps for v in op_ms]
    return Run(ms_per_step, median_ms, kernel_ms, graph_event_ms, ops, selected)


# --- algorithmic work --------------------------------------------------------


def conv_family_bytes(graph) -> tuple[int, int]:
    """(algorithmic HBM bytes, launches) of one step's fused conv nodes:
    each reads its input and weights once and writes its output once (FP32),
    and each residual join also reads its residual once."""
    from cutriton_amd import workloads

    shapes = workloads.value_shapes(graph)

    def size(name: str) -> int:
        n = 1
        for d in shapes[name]:
            n *= d
        return 4 * n

    total = launches = 0
    for node in graph.nodes:
        if node.op_type == "Conv":
            total += size(node.inputs[0]) + size(node.inputs[1]) + size(node.outputs[0])
            launches += 1
        elif node.op_type == "Add":
            total += size(node.inputs[1])
    return total, launches


def ffn_gemm_bytes(m: int, h: int, i: int) -> tuple[int, int]:
    """Algorithmic FP16 bytes of GemmGelu (X, W1, b1 in; [m, i] out) and of
    Gemm ([m, i], W2, b2 in; [m, h] out)."""
    return 2 * (m * h + h * i + i + m * i), 2 * (m * i + i * h + h + m * h)


# --- workloads -----------------------------------------------------------------


def bench_resnet(args, cache_dir: str, batch: int, profile: bool) -> dict:
    from cutriton_amd import workloads

    graph = workloads.resnet50(1 if profile else batch)
    x = workloads.resnet50_input(batch)
    # The headline batch (32) warms up by the --warmup steps alone; the other
    # legs also by time, like the FFN's.
    run = run_workload(graph, {"input": x}, args.steps, args.warmup, cache_dir, RESNET_PROFILE if profile else None,
                       warm_ms=0.0 if batch == 32 else 100.0)
    ms_per_step, kernel_ms, event_ms, ops, selected = (run.ms_per_step, run.kernel_ms, run.graph_event_ms, run.ops,
                                                       run.selected)
    # The profile engine's graph is declared at batch 1; FLOPs and bytes
    # are those of the batch it runs.
    at_batch = dataclasses.replace(graph, inputs={"input": ((batch, 3, 224, 224), "float32", "NCHW")})
    flops = workloads.node_flops(at_batch)
    conv_flops = sum(v for k, v in flops.items() if k != "classifier")
    total_flops = sum(flops.values())
    img_s = batch * 1e3 / ms_per_step
    conv_idx = [i for i, op in enumerate(ops) if op.op_type in CONV_OPS]
    conv_ms = sum(kernel_ms[i] for i in conv_idx)
    launches = len(conv_idx)
    achieved = conv_flops / (conv_ms * 1e-3) / 1e12
    step_bytes, conv_nodes = conv_family_bytes(at_batch)
    if conv_nodes != launches:
        raise RuntimeError(f"{launches} conv launches for {conv_nodes} conv nodes")

    def op_flops(name: str) -> int:
        keys = [k for k in flops if name.startswith(k)]
        return flops[max(keys, key=len)] if keys else 0

    per_op = sorted(((kernel_ms[i], ops[i].node_name, selected[i].split(":", 1)[-1], op_flops(ops[i].node_name))
                     for i in range(len(ops))), reverse=True)
    engine_kind = "profile min1/opt32/max64" if profile else "static"
    log(f"  resnet50 bs{batch} ({engine_kind} engine): {ms_per_step:.3f} ms/step, {img_s:.1f} img/s; kernel time "
        f"per step: conv {conv_ms:.3f} ms, all {sum(kernel_ms):.3f} ms (profiled graph events {sum(event_ms):.3f} ms)")
    for ms, name, var, fl in per_op:
        rate = f"{fl / (ms * 1e-3) / 1e12:6.1f} TF/s" if fl and ms > 0 else " " * 11
        log(f"    {ms * 1e3:8.1f} us {rate}  {name}  [{var}]")
    return {
        "engine": engine_kind,
        "ms_per_step": ms_per_step,
        "median_event_ms": run.median_event_ms,
        "img_s": img_s,
        "tflops": total_flops / (ms_per_step * 1e-3) / 1e12,
        "pct_fp32_mfma_peak": 100.0 * total_flops / (ms_per_step * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS,
        "kernel_us": {name: round(ms * 1e3, 2) for ms, name, _, _ in per_op},
        "roofline": {
            "kernel": f"conv_bn[_add]_relu_fp32 implicit-GEMM family ({launches} launches/step)",
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": FP32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": step_bytes // launches,
            "flop_per_launch": conv_flops / launches,
            "launches_per_step": launches,
            "avg_launch_us": conv_ms * 1e3 / launches,
            "timing": f"ExecutionContext::TimeOp, {KERNEL_TIMING_LAUNCHES} back-to-back launches per op, HIP events",
        },
        "selected": selected,
    }


def bench_single_node(args, cache_dir: str) -> dict:
    """The single FusedConvBatchNormRelu node: x[1,64,56,56], W[64,64,3,3],
    stride 1, pad 1 (231.2 MFLOP)."""
    from cutriton_amd import workloads

    graph, x = workloads.conv_bn_relu()
    run = run_workload(graph, {"x": x}, args.steps, args.warmup, cache_dir, warm_ms=100.0)
    ms_per_step, kernel_ms, selected = run.ms_per_step, run.kernel_ms, run.selected
    flops = sum(workloads.node_flops(graph).values())
    out = {
        "workload": "conv_bn_relu_fp32_1x64x56x56_k3s1p1",
        "ms_per_step": ms_per_step,
        "kernel_us": kernel_ms[0] * 1e3,
        "tflops": flops / (kernel_ms[0] * 1e-3) / 1e12,
        "variant": selected[0].rsplit(":", 1)[1],
    }
    log(f"  single conv node: {out['kernel_us']:.1f} us kernel ({out['tflops']:.1f} TF), "
        f"{ms_per_step * 1e3:.1f} us/step, {out['variant']}")
    return out


def bench_ffn(args, cache_dir: str, shape: tuple[int, int, int], profile: bool) -> dict:
    from cutriton_amd import workloads

    m, h, i = shape
    if profile:
        template, x = workloads.ffn(FFN_PROFILE["tokens"]["x"][2][0], h, i)
        x = x[:m]
    else:
        template, x = workloads.ffn(m, h, i)
    run = run_workload(template, {"x": x}, args.steps, args.warmup, cache_dir, FFN_PROFILE if profile else None,
                       warm_ms=100.0)
    ms_per_step, kernel_ms, ops, selected = run.ms_per_step, run.kernel_ms, run.ops, run.selected
    gemm_flops = 2 * m * h * i
    per_op = {op.op_type: kernel_ms[j] for j, op in enumerate(ops)}
    gemm_ms = per_op["GemmGelu"] + per_op["Gemm"]
    achieved = 2 * gemm_flops / (gemm_ms * 1e-3) / 1e12
    gelu_bytes, gemm_bytes = ffn_gemm_bytes(m, h, i)
    out = {
        "workload": f"ffn_fp16_m{m}_h{h}_i{i}",
        "engine": "profile min128/opt4096/max8192" if profile else "static",
        "ms_per_step": ms_per_step,
        "median_event_ms": run.median_event_ms,
        "tflops_block": 2 * gemm_flops / (ms_per_step * 1e-3) / 1e12,
        "gemm_gelu_us": per_op["GemmGelu"] * 1e3,
        "gemm_us": per_op["Gemm"] * 1e3,
        "skip_layer_norm_us": per_op["SkipLayerNormalization"] * 1e3,
        "gemm_gelu_tflops": gemm_flops / (per_op["GemmGelu"] * 1e-3) / 1e12,
        "gemm_tflops": gemm_flops / (per_op["Gemm"] * 1e-3) / 1e12,
        "skip_layer_norm_gbps": 3 * m * h * 2 / (per_op["SkipLayerNormalization"] * 1e-3) / 1e9,
        "pct_fp16_mfma_peak_gemms": 100.0 * achieved / FP16_MFMA_PEAK_TFLOPS,
        "roofline": {
            "kernel": "FP16 GEMMs: GemmGelu + Gemm (2 launches/step)",
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": FP16_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / FP16_MFMA_PEAK_TFLOPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": (gelu_bytes + gemm_bytes) // 2,
            "flop_per_launch": gemm_flops,
            "avg_launch_us": gemm_ms * 1e3 / 2,
            "timing": f"ExecutionContext::TimeOp, {KERNEL_TIMING_LAUNCHES} back-to-back launches per op, HIP events",
        },
        "selected": [s.rsplit(":", 1)[1] for s in selected],
    }
    log(f"  ffn M={m} H={h} I={i} ({out['engine']} engine): {ms_per_step * 1e3:.1f} us/step; GemmGelu "
        f"{out['gemm_gelu_us']:.1f} us ({out['gemm_gelu_tflops']:.0f} TF), Gemm {out['gemm_us']:.1f} us "
        f"({out['gemm_tflops']:.0f} TF), SkipLN {out['skip_layer_norm_us']:.1f} us; selected {out['selected']}")
    return out


def vendor_ffn_gemms(m: int, h: int, i: int) -> dict:
    """The FFN's two products through torch on the same GPU (hipBLASLt), as a
    library reference beside the block's own kernels: X[m,h] @ W1[h,i] + b1,
    the erf GELU as a kernel of its own, and H[m,i] @ W2[i,h] + b2, FP16
    with FP32 accumulation. Each is timed over 50 back-to-back calls between
    events on the current stream, after 10 warm-up calls."""
    import torch

    gen = torch.Generator().manual_seed(0)
    dev = "cuda:0"
    x = torch.randn(m, h, generator=gen).half().to(dev)
    w1 = (torch.randn(h, i, generator=gen) * 0.02).half().to(dev)
    w2 = (torch.randn(i, h, generator=gen) * 0.02).half().to(dev)
    b1 = torch.zeros(i, dtype=torch.float16, device=dev)
    b2 = torch.zeros(h, dtype=torch.float16, device=dev)
    # The weights also as [N][K] (the layout of torch.nn.Linear and of this
    # block's own kernels): F.linear multiplies by their transpose.
    w1t, w2t = w1.t().contiguous(), w2.t().contiguous()
    mid = torch.addmm(b1, x, w1)
    linear = torch.nn.functional.linear

    def per_call_us(fn) -> float:
        for _ in range(10):
            fn()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(50):
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) * 1e3 / 50

    out = {
        "gemm_bias_h_to_i_us": per_call_us(lambda: torch.addmm(b1, x, w1)),
        "gemm_bias_h_to_i_nk_us": per_call_us(lambda: linear(x, w1t, b1)),
        "gelu_us": per_call_us(lambda: torch.nn.functional.gelu(mid)),
        "gemm_bias_i_to_h_us": per_call_us(lambda: torch.addmm(b2, mid, w2)),
        "gemm_bias_i_to_h_nk_us": per_call_us(lambda: linear(mid, w2t, b2)),
        "gemm_h_to_i_us": per_call_us(lambda: torch.matmul(x, w1)),
        "gemm_h_to_i_nk_us": per_call_us(lambda: linear(x, w1t)),
        "gemm_i_to_h_us": per_call_us(lambda: torch.matmul(mid, w2)),
        "gemm_i_to_h_nk_us": per_call_us(lambda: linear(mid, w2t)),
    }
    out = {k: round(v, 2) for k, v in out.items()}
    out["timing"] = ("torch.addmm / torch.matmul ([K][N] weight), torch.nn.functional.linear ([N][K] weight, "
                     "_nk), torch.nn.functional.gelu; 50 calls between events")
    log(f"  torch (hipBLASLt) M={m} H={h} I={i}: GEMM+bias {out['gemm_bias_h_to_i_us']:.1f} / "
        f"{out['gemm_bias_h_to_i_nk_us']:.1f} us ([K][N] / [N][K] weight) + GELU {out['gelu_us']:.1f} us; "
        f"GEMM+bias {out['gemm_bias_i_to_h_us']:.1f} / {out['gemm_bias_i_to_h_nk_us']:.1f} us; no bias "
        f"{out['gemm_h_to_i_us']:.1f} / {out['gemm_h_to_i_nk_us']:.1f} and {out['gemm_i_to_h_us']:.1f} / "
        f"{out['gemm_i_to_h_nk_us']:.1f} us")
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
    run = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir)
    kernel_ms, selected = run.kernel_ms, run.selected
    out.update(softmax_us=kernel_ms[0] * 1e3, softmax_gbps=moved / (kernel_ms[0] * 1e-3) / 1e9,
               softmax_variant=selected[0].rsplit(":", 1)[1])
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, columns), "float16", "")
    gamma = g.constant("gamma", rng.uniform(0.5, 1.5, columns).astype(np.float16))
    beta = g.constant("beta", rng.normal(0.0, 0.1, columns).astype(np.float16))
    g.add("ln", "LayerNormalization", ["x", gamma, beta], ["y"], axis=-1, epsilon=1e-5)
    g.outputs.append("y")
    kernel_ms = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir).kernel_ms
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
        kernel_ms = run_workload(g, feeds, args.steps, args.warmup, cache_dir).kernel_ms
        pairs = s * (s + 1) // 2 if causal else s * s
        flops = 4 * b * h * pairs * d
        key = "causal" if causal else "full"
        out[f"{key}_us"] = kernel_ms[0] * 1e3
        out[f"{key}_tflops"] = flops / (kernel_ms[0] * 1e-3) / 1e12
    log(f"  attention {b}x{h}x{s}x{d}: {out['full_us']:.1f} us ({out['full_tflops']:.0f} TF), "
        f"causal {out['causal_us']:.1f} us ({out['causal_tflops']:.0f} TF)")
    return out


def copy_graph():
    """One Relu over 64 Mi non-negative floats: the relu_fp32 kernel reads and
    writes exactly 256 MiB each."""
    import numpy as np

    from cutriton_amd import workloads

    g = workloads.GraphSpec()
    g.inputs["x"] = ((COPY_FLOATS,), "float32", "")
    g.add("copy", "Relu", ["x"], ["y"])
    g.outputs.append("y")
    x = np.abs(np.random.default_rng(workloads.SEED).standard_normal(COPY_FLOATS, dtype=np.float32))
    return g, x


def bench_copy(args, cache_dir: str) -> dict:
    """The Relu copy's GB/s: the streaming reference for the bandwidth
    kernels."""
    g, x = copy_graph()
    run = run_workload(g, {"x": x}, args.steps, args.warmup, cache_dir)
    ms_per_step, kernel_ms = run.ms_per_step, run.kernel_ms[0]
    out = {"workload": "relu_fp32_64Mi", "bytes": 2 * 4 * COPY_FLOATS, "kernel_us": kernel_ms * 1e3,
           "gbps": 2 * 4 * COPY_FLOATS / (kernel_ms * 1e-3) / 1e9, "ms_per_step": ms_per_step}
    log(f"  copy: {out['kernel_us']:.1f} us, {out['gbps']:.0f} GB/s")
    return out


# --- HBM traffic from rocprofv3 counter passes -------------------------------


def counter_pass(cache_dir: str) -> None:
    """The workload of one counter pass (run under rocprofv3 by
    measure_traffic): the Relu copy, ResNet-50 bs32 and the FFN at M=4096 on
    the engines the timed run used, three steps each, tuned choices read from
    the cache."""
    import torch

    from cutriton_amd import workloads

    handle = torch.cuda.current_stream().cuda_stream
    g, x = copy_graph()
    template, fx = workloads.ffn(FFN_PROFILE["tokens"]["x"][2][0], FFN_SHAPE[1], FFN_SHAPE[2])
    cases = (
        (g, {"x": x}, None),
        (workloads.resnet50(1), {"input": workloads.resnet50_input(32)}, RESNET_PROFILE),
        (template, {"x": fx[:FFN_SHAPE[0]]}, FFN_PROFILE),
    )
    for graph, feeds, profiles in cases:
        eng, ctx, keep = _context(graph, feeds, cache_dir, False, "use_cache", profiles)
        for _ in range(3):
            ctx.run_async(handle)
            ctx.synchronize()
        del ctx, eng, keep
        torch.cuda.synchronize()


def _read_counter(path: str) -> dict[str, list[float]]:
    """Per kernel name, the counter's value of each dispatch (summed over the
    instances rocprofv3 reports for one dispatch)."""
    per: dict[str, dict[str, float]] = defaultdict(lambda: defaultdict(float))
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            per[row["Kernel_Name"]][row["Dispatch_Id"]] += float(row["Counter_Value"])
    return {name: list(values.values()) for name, values in per.items()}


def measure_traffic(cache_dir: str) -> dict:
    """Calibrated HBM bytes per launch of the conv family (ResNet-50 bs32) and
    of the FFN GEMMs (M=4096), from one FETCH_SIZE and one WRITE_SIZE pass.
    FETCH_SIZE and WRITE_SIZE count KiB at the L2's memory side; each is
    scaled by the factor that maps the Relu copy's reading to its known
    256 MiB."""
    tool = shutil.which("rocprofv3")
    if tool is None:
        return {"error": "rocprofv3 not found"}
    families = {
        "conv": lambda k: k.startswith("conv_"),
        "ffn_gemms": lambda k: k.startswith("gemm") and "fp16" in k,
    }
    known_kib = 4 * COPY_FLOATS / 1024
    result: dict = {"calibration": {}, "kib_per_launch": {f: {} for f in families}}
    env = dict(os.environ, TMPDIR="/tmp")
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out_dir = tempfile.mkdtemp(prefix=f"cutriton-{counter.lower()}-")
        cmd = ["timeout", "-s", "KILL", "300", tool, "--pmc", counter, "--output-format", "csv", "-d", out_dir,
               "-o", "run", "--", sys.executable, "-u", str(ROOT / "bench.py"), "--counter-pass",
               "--tuning-cache", cache_dir]
        log(f"  counter pass {counter} ...")
        t0 = time.perf_counter()
        with open(os.path.join(out_dir, "rocprofv3.log"), "w") as logf:
            rc = subprocess.run(cmd, stdout=logf, stderr=subprocess.STDOUT, cwd="/tmp", env=env).returncode
        files = glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True)
        log(f"  counter pass {counter}: exit {rc}, {time.perf_counter() - t0:.1f} s")
        if not files:
            return {"error": f"rocprofv3 --pmc {counter} exited {rc} without a counter file"}
        values = _read_counter(files[0])
        copy = values.get("relu_fp32")
        if not copy:
            return {"error": f"no relu_fp32 dispatch in the {counter} pass"}
        scale = known_kib / (sum(copy) / len(copy))
        result["calibration"][counter] = round(scale, 4)
        for family, match in families.items():
            samples = [v for name, vs in values.items() if match(name) for v in vs]
            if not samples:
                return {"error": f"no {family} dispatch in the {counter} pass"}
            result["kib_per_launch"][family][counter] = sum(samples) / len(samples) * scale
        shutil.rmtree(out_dir, ignore_errors=True)
    result["bytes_per_launch"] = {f: int(round(1024 * sum(v.values()))) for f, v in result["kib_per_launch"].items()}
    return result


# --- CPU baseline ------------------------------------------------------------------


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baselines(budget_s: float) -> dict:
    """The reference's CPU path on this host: each graph in PyTorch-CPU FP32
    (FP16 constants and inputs widened), 3 warm-ups, then timed iterations
    until at least 10 are done and `budget_s` seconds have passed (at most
    30), median reported."""
    import numpy as np
    import torch

    from cutriton_amd import workloads
    from oracle import torch_cpu

    cores = os.cpu_count() or 1
    # The host share of one GPU is capped by OMP_NUM_THREADS where it is set.
    torch.set_num_threads(min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    host = f"{_cpu_model()} ({cores} logical CPUs)"

    def timed(graph, feeds) -> tuple[float, int]:
        consts = torch_cpu.prepare(graph)
        tensors = {k: torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32)) for k, v in feeds.items()}
        for _ in range(CPU_WARMUPS):
            torch_cpu.run(graph, consts, tensors)
        times = []
        start = time.perf_counter()
        while len(times) < CPU_MIN_ITERATIONS or (time.perf_counter() - start < budget_s and len(times) < 30):
            t0 = time.perf_counter()
            torch_cpu.run(graph, consts, tensors)
            times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2], len(times)

    out: dict = {}
    for batch in (32, 1, 64):
        graph = workloads.resnet50(batch)
        med, n = timed(graph, {"input": workloads.resnet50_input(batch)})
        out[f"resnet50_bs{batch}"] = {
            "value": round(batch / med, 2), "unit": "img/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"ResNet-50 bs{batch} FP32, PyTorch-CPU restatement of the same graph, {CPU_WARMUPS} warm-ups "
                      f"+ {n} timed batches, median {med * 1e3:.1f} ms/batch; host {host}"}
        log(f"  cpu resnet50 bs{batch}: {med * 1e3:.1f} ms/batch over {n}")
    for m, h, i in (FFN_SHAPE, FFN_SMALL_SHAPE):
        graph, x = workloads.ffn(m, h, i)
        med, n = timed(graph, {"x": x})
        out[f"ffn_m{m}_h{h}_i{i}"] = {
            "value": round(2 * 2 * m * h * i / med / 1e12, 4), "unit": "TFLOP/s (two GEMMs)",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"FFN M={m} H={h} I={i} in FP32 (FP16 weights and input widened), {CPU_WARMUPS} warm-ups + {n} "
                      f"timed steps, median {med * 1e3:.2f} ms/step; host {host}"}
        log(f"  cpu ffn M={m}: {med * 1e3:.2f} ms/step over {n}")
    graph, x = workloads.conv_bn_relu()
    med, n = timed(graph, {"x": x})
    flops = sum(workloads.node_flops(graph).values())
    out["conv_bn_relu_1x64x56x56"] = {
        "value": round(flops / med / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
        "sample": f"Conv 3x3 + BatchNorm + Relu x[1,64,56,56] FP32, {CPU_WARMUPS} warm-ups + {n} timed runs, median "
                  f"{med * 1e3:.3f} ms; host {host}"}
    log(f"  cpu single conv node: {med * 1e3:.3f} ms over {n}")
    return out


def _rounded(d: dict) -> dict:
    return {k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=30)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--workload", choices=("all", "resnet50", "resnet50_bs32", "ffn", "norms", "attention", "copy"),
                        default="all", help="resnet50_bs32: only the batch-32 leg of resnet50")
    parser.add_argument("--tuning-cache", default="",
                        help="tuning cache folder to reuse (default: a fresh temporary folder, so every op is tuned)")
    parser.add_argument("--cpu-baseline-seconds", type=float, default=5.0,
                        help="time budget per CPU baseline case beyond its 3 warm-ups and 10 iterations; "
                             "0 skips the CPU baselines")
    parser.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    parser.add_argument("--counter-pass", action="store_true", help=argparse.SUPPRESS)
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (cuda:0)", file=sys.stderr)
        return 2
    if args.counter_pass:
        counter_pass(args.tuning_cache)
        return 0
    log(f"device: {torch.cuda.get_device_name(0)}")
    cache_dir = args.tuning_cache or tempfile.mkdtemp(prefix="cutriton-tuning-")
    os.makedirs(cache_dir, exist_ok=True)
    result = {
        "metric": METRIC, "value": None, "unit": "img/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic (seeded N(0,1) inputs, random-init weights)",
        "config": {"workload": "resnet50_v1.5_fp32_nchw_bs32", "global_batch": 32, "image": [3, 224, 224],
                   "engine": "dynamic batch profile min1/opt32/max64, hipGraph replay",
                   "parallelism": "single-gpu"},
    }
    if args.workload in ("all", "resnet50", "resnet50_bs32"):
        r = bench_resnet(args, cache_dir, 32, profile=True)
        result.update(value=round(r["img_s"], 2), ms_per_step=round(r["ms_per_step"], 4),
                      median_event_ms=round(r["median_event_ms"], 4),
                      pct_fp32_mfma_peak=round(r["pct_fp32_mfma_peak"], 2), roofline=r["roofline"])
        result["resnet50_tflops"] = round(r["tflops"], 3)
    if args.workload in ("all", "resnet50"):
        r64 = bench_resnet(args, cache_dir, 64, profile=True)
        result["resnet50_bs64"] = {"engine": r64["engine"], "img_s": round(r64["img_s"], 2),
                                   "ms_per_step": round(r64["ms_per_step"], 4),
                                   "pct_fp32_mfma_peak": round(r64["pct_fp32_mfma_peak"], 2),
                                   "conv_tflops": r64["roofline"]["achieved"]}
        r1 = bench_resnet(args, cache_dir, 1, profile=False)
        result["resnet50_bs1"] = {"engine": r1["engine"], "img_s": round(r1["img_s"], 2),
                                  "ms_per_step": round(r1["ms_per_step"], 4),
                                  "pct_fp32_mfma_peak": round(r1["pct_fp32_mfma_peak"], 2),
                                  "conv_tflops": r1["roofline"]["achieved"]}
        result["conv_bn_relu_node"] = _rounded(bench_single_node(args, cache_dir))
    if args.workload in ("all", "ffn"):
        f = bench_ffn(args, cache_dir, FFN_SHAPE, profile=True)
        result["ffn"] = _rounded(f)
        result["ffn"]["torch_hipblaslt"] = vendor_ffn_gemms(*FFN_SHAPE)
        if args.workload == "ffn":
            result.update(value=round(f["tflops_block"], 3), unit="TFLOP/s", ms_per_step=round(f["ms_per_step"], 4),
                          dtype="fp16", config={"workload": f["workload"], "engine": f["engine"],
                                                "parallelism": "single-gpu"})
        result["ffn_m512"] = _rounded(bench_ffn(args, cache_dir, FFN_SMALL_SHAPE, profile=False))
        result["ffn_m512"].pop("roofline", None)
    if args.workload in ("all", "norms"):
        n = bench_norms(args, cache_dir)
        result["norms"] = _rounded(n)
        if args.workload == "norms":
            result.update(value=round(n["softmax_gbps"], 1), unit="GB/s", dtype="fp16",
                          ms_per_step=round(n["softmax_us"] * 1e-3, 4),
                          config={"workload": "softmax_fp16_262144x1024", "parallelism": "single-gpu"})
    if args.workload in ("all", "attention"):
        a = bench_attention(args, cache_dir)
        result["attention"] = _rounded(a)
        if args.workload == "attention":
            result.update(value=round(a["full_tflops"], 3), unit="TFLOP/s", dtype="fp16",
                          ms_per_step=round(a["full_us"] * 1e-3, 4),
                          config={"workload": "attention_fp16_b8_h16_s2048_d128", "parallelism": "single-gpu"})
    if args.workload == "copy":
        c = bench_copy(args, cache_dir)
        result.update(value=round(c["gbps"], 1), unit="GB/s", ms_per_step=round(c["ms_per_step"], 4),
                      config={"workload": c["workload"], "parallelism": "single-gpu"}, copy=c)
    if args.workload == "all" and not args.no_traffic:
        traffic = measure_traffic(cache_dir)
        result["traffic"] = traffic
        if "bytes_per_launch" in traffic:
            for key, family in (("roofline", "conv"), ("ffn", "ffn_gemms")):
                block = result[key] if key == "roofline" else result[key]["roofline"]
                block["traffic"] = traffic["bytes_per_launch"][family]
                block["traffic_vs_algorithmic"] = round(block["traffic"] / block["algorithmic_bytes_per_launch"], 3)
                block["traffic_source"] = "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE child passes of this run, " \
                                          "scaled by a 256 MiB copy"
        else:
            log(f"  traffic not measured: {traffic.get('error')}")
    if args.cpu_baseline_seconds > 0 and args.workload in ("all", "resnet50"):
        cpu = cpu_baselines(args.cpu_baseline_seconds)
        result["cpu_baseline"] = cpu["resnet50_bs32"]
        result["cpu_baselines"] = cpu
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
