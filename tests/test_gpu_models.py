"""Whole-graph parity on the GPU: ResNet-50 and the FP16 FFN through the
engine (fused plan, hipGraph replay) against the FP64 oracle, plus the stem
known-answer test of the reference (tests/cpp/test_cuda.cpp:444-479).

Tolerances: ResNet-50 logits 1e-3 relative (norm-wise, and per element with
a 1e-3*RMS floor); FFN outputs 1e-2 absolute; the stem KAT 1e-4 + 1e-4|e|
as in the reference (test_cuda.cpp:168-180).
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from oracle import oracle
from tests.helpers import assert_close_fp32, run_graph

pytestmark = pytest.mark.gpu


def test_stem_known_answer():
    g, x, expected = workloads.stem_kat()
    opts = engine.CompileOptions(tuning_mode="disabled", enable_profiling=True)
    out, eng, ctx = run_graph(g, {"input": x}, opts, repeats=2)
    got = out["output"].astype(np.float64)
    assert np.all(np.abs(got - expected) <= 1e-4 + 1e-4 * np.abs(expected))
    assert [op.op_type for op in eng.ops()] == ["FusedConvBatchNormRelu", "GlobalAveragePool", "Flatten", "Gemm"]
    events = ctx.profile_events()
    assert len(events) == 4 and events[2][1] == 0.0  # Flatten is a view and is not timed
    assert ctx.cached_cuda_graph_count() == 1


def test_conv_bn_relu_single_node():
    g, x = workloads.conv_bn_relu()
    out, eng, _ = run_graph(g, {"x": x})
    assert [op.op_type for op in eng.ops()] == ["FusedConvBatchNormRelu"]
    assert_close_fp32(out[g.outputs[0]], oracle.evaluate(g, {"x": x})[g.outputs[0]], what="conv_bn_relu cfg0")


def check_logits(got: np.ndarray, want: np.ndarray) -> None:
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-3, f"norm-wise relative error {rel:.3e}"
    assert_close_fp32(got, want, rtol=1e-3, what="resnet50 logits")


def test_resnet50_batch1():
    g = workloads.resnet50(1)
    x = workloads.resnet50_input(1)
    out, eng, ctx = run_graph(g, {"input": x}, repeats=2)
    ops = eng.ops()
    assert len(ops) == 57
    want = oracle.evaluate(g, {"input": x})["output"]
    check_logits(out["output"].astype(np.float64), want)
    assert ctx.cached_cuda_graph_count() == 1


def test_resnet50_batch32_matches_single_images():
    """Batch invariance at the measured size: image i of a batch-32 run equals
    the batch-1 run of that image (same kernels, same per-column arithmetic),
    and images 0 and 31 also match the FP64 oracle."""
    g32 = workloads.resnet50(32)
    x = workloads.resnet50_input(32)
    out32, _, _ = run_graph(g32, {"input": x}, repeats=2)
    g1 = workloads.resnet50(1)
    for i in (0, 31):
        out1, _, _ = run_graph(g1, {"input": x[i:i + 1]})
        assert_close_fp32(out32["output"][i:i + 1], out1["output"], rtol=1e-4, what=f"image {i}")
        want = oracle.evaluate(g1, {"input": x[i:i + 1]})["output"]
        check_logits(out32["output"][i:i + 1].astype(np.float64), want)


def test_ffn_config_m512():
    g, x = workloads.ffn(512, 768, 3072)
    out, eng, _ = run_graph(g, {"x": x})
    assert [op.op_type for op in eng.ops()] == ["GemmGelu", "Gemm", "SkipLayerNormalization"]
    err = np.abs(out["y"].astype(np.float64) - oracle.evaluate(g, {"x": x})["y"])
    assert err.max() <= 1e-2, err.max()


def test_ffn_config_m4096():
    g, x = workloads.ffn(4096, 1024, 4096)
    out, _, _ = run_graph(g, {"x": x})
    err = np.abs(out["y"].astype(np.float64) - oracle.evaluate(g, {"x": x})["y"])
    assert err.max() <= 1e-2, err.max()


@pytest.mark.parametrize("tuning", ["disabled", "tune_on_miss"])
def test_ffn_integer_pattern(tuning, tmp_path):
    """The reference's FP16 transformer test inputs (tokens 17, hidden 128,
    intermediate 512; tests/cpp/test_cuda.cpp:336-393): Gemm -> Gelu ->
    Add(residual) -> LayerNormalization fuses to GemmGelu +
    SkipLayerNormalization and matches the FP64 oracle within 1e-2."""
    g, feeds = workloads.ffn_pattern()
    opts = engine.CompileOptions(tuning_mode=tuning, tuning_cache_dir=str(tmp_path), enable_profiling=True)
    out, eng, ctx = run_graph(g, feeds, opts, repeats=2)
    assert [op.op_type for op in eng.ops()] == ["GemmGelu", "SkipLayerNormalization"]
    err = np.abs(out["output"].astype(np.float64) - oracle.evaluate(g, feeds)["output"])
    assert err.max() <= 1e-2, err.max()
    assert len(ctx.profile_events()) == 2


def test_time_op_reports_kernel_time():
    """ExecutionContext::TimeOp: positive per-launch kernel time for ops with
    kernels, 0 for the Flatten view, an error before the first run."""
    g, x, _ = workloads.stem_kat()
    eng = engine.build_engine(workloads.to_model(g), engine.CompileOptions(tuning_mode="disabled"))
    ctx = eng.create_execution_context()
    import torch

    xi = torch.from_numpy(x).to("cuda:0")
    shape, _ = eng.value_desc("output")
    y = torch.empty(shape, device="cuda:0")
    ctx.bind_input("input", xi)
    ctx.bind_output("output", y)
    with pytest.raises(engine.CutritonError):
        ctx.time_op(0, 5)
    ctx.run()
    before = y.cpu().numpy().copy()
    times = [ctx.time_op(i, 5) for i in range(len(eng.ops()))]
    assert times[0] > 0 and times[2] == 0.0 and times[3] > 0
    ctx.run()
    assert np.array_equal(before, y.cpu().numpy())


def _profile_context(graph, opts):
    eng = engine.build_engine(workloads.to_model(graph), opts)
    return eng, eng.create_execution_context()


def _run_shape(ctx, eng, feeds: dict[str, np.ndarray], out_name: str, layout: str):
    import torch

    for name, value in feeds.items():
        ctx.set_input_shape(name, value.shape)
    ctx.resolve_shapes()
    keep = []
    for name, value in feeds.items():
        t = torch.from_numpy(np.ascontiguousarray(value)).to("cuda:0")
        keep.append(t)
        ctx.bind_input(name, t, layout=layout)
    shape, dtype, _ = ctx.resolved_desc(out_name)
    out = torch.empty(shape, dtype=getattr(torch, dtype), device="cuda:0")
    ctx.bind_output(out_name, out, layout="")
    ctx.run()
    ctx.run()  # graph replay
    return out.cpu().numpy()


def test_resnet50_dynamic_batch_profile_32_and_64(tmp_path):
    """Profile min1/opt32/max64, workspace planned at the profile max, run at
    batch 32 then 64 on one context (a hipGraph per shape). Images are
    checked against the FP64 oracle, one per batch end."""
    g = workloads.resnet50(1)
    opts = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(tmp_path), shape_profiles={
        "batch": {"input": ((1, 3, 224, 224), (32, 3, 224, 224), (64, 3, 224, 224))}})
    eng, ctx = _profile_context(g, opts)
    ctx.select_shape_profile("batch")
    x64 = workloads.resnet50_input(64)
    for batch in (32, 64):
        out = _run_shape(ctx, eng, {"input": x64[:batch]}, "output", "NCHW")
        assert out.shape == (batch, 1000)
        for i in (0, batch - 1):
            want = oracle.evaluate(g, {"input": x64[i:i + 1]})["output"]
            check_logits(out[i:i + 1].astype(np.float64), want)
    assert ctx.cached_cuda_graph_count() == 2


def test_ffn_dynamic_m_profile(tmp_path):
    """FFN with the M profile min128/opt4096/max8192 and tuned variants, run
    at M = 128, 4096 and 8192. Rows are independent (GEMM rows, per-row
    LayerNorm), so the FP64 check evaluates the first and last 64 rows."""
    g, x = workloads.ffn(8192, 1024, 4096)
    opts = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(tmp_path), shape_profiles={
        "tokens": {"x": ((128, 1024), (4096, 1024), (8192, 1024))}})
    eng, ctx = _profile_context(g, opts)
    ctx.select_shape_profile("tokens")
    for m in (128, 4096, 8192):
        out = _run_shape(ctx, eng, {"x": x[:m]}, "y", "")
        assert out.shape == (m, 1024)
        for rows in (slice(0, 64), slice(m - 64, m)):
            want = oracle.evaluate(g, {"x": x[rows]})["y"]
            err = np.abs(out[rows].astype(np.float64) - want).max()
            assert err <= 1e-2, (m, rows, err)
