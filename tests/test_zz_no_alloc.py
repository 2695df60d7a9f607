"""ct_context_run_async_no_alloc against ct_context_run_async, through the C-ABI.

The graph is one FP32 Gemm, [M, 2048] x [2048, 1000] (the ResNet-50
classifier), with an M profile 1..64 (opt 32) on a pack holding only the
split-K Gemm entries, so the kernel that runs uses the runtime scratch: tile
counters and partial sums. The allocation-free call binds that scratch to the
library's static device array; the ordinary call to the context's own buffer.

Two allocation-free calls in a row on one context, the second with a smaller
input (M = 32, then M = 7), are each compared with an ordinary run of the
same shape on another context: bit for bit (the same kernel sums its shares
in split order, so the result cannot depend on where the scratch lives), and
with the FP64 oracle at the FP32 bound.
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from oracle import oracle
from tests.helpers import assert_close_fp32, filtered_pack

pytestmark = pytest.mark.gpu

K, N = 2048, 1000


def classifier_graph() -> tuple[workloads.GraphSpec, np.ndarray]:
    rng = np.random.default_rng(workloads.SEED)
    g = workloads.GraphSpec()
    g.inputs["x"] = ((32, K), "float32", "")
    w = g.constant("w", rng.normal(0.0, 0.01, (K, N)).astype(np.float32))
    g.add("classifier", "Gemm", ["x", w], ["y"])
    g.outputs.append("y")
    return g, rng.standard_normal((64, K), dtype=np.float32)


def test_no_alloc_run_matches_the_ordinary_run(tmp_path):
    import torch

    graph, x_all = classifier_graph()
    pack = filtered_pack(tmp_path / "pack", lambda e: e["op_type"] == "Gemm" and e["kernel_id"] == "gemm.fp32.splitk")
    opts = engine.CompileOptions(tuning_mode="disabled", kernel_artifact_dir=pack,
                                 shape_profiles={"rows": {"x": ((1, K), (32, K), (64, K))}})
    eng = engine.build_engine(workloads.to_model(graph), opts)
    (op,) = eng.ops()
    assert all(".splitk:" in c for c in op.candidates if not c.startswith("unfused:")), op.candidates

    stream = torch.cuda.Stream()
    keep = []

    def bind(ctx, rows: int) -> torch.Tensor:
        ctx.set_input_shape("x", (rows, K))
        ctx.resolve_shapes()
        x = torch.from_numpy(np.ascontiguousarray(x_all[:rows])).to("cuda:0")
        y = torch.full((rows, N), float("nan"), dtype=torch.float32, device="cuda:0")
        keep.extend((x, y))
        ctx.bind_input("x", x, layout="")
        ctx.bind_output("y", y, layout="")
        return y

    def ordinary(rows: int) -> np.ndarray:
        ctx = eng.create_execution_context()
        ctx.select_shape_profile("rows")
        y = bind(ctx, rows)
        ctx.run()
        assert ".splitk:" in op.candidates[ctx.selected_candidates(1)[0]]
        return y.cpu().numpy()

    # The context runs once the ordinary way (any shape of the profile): that
    # uploads the constants, sizes its workspace for the profile and loads
    # the code objects. The allocation-free calls then need nothing new.
    ctx = eng.create_execution_context()
    ctx.select_shape_profile("rows")
    bind(ctx, 64)
    ctx.run()

    results = {}
    for rows in (32, 7):  # two calls in a row, the second with a smaller input
        y = bind(ctx, rows)
        ctx.run_async_no_alloc(stream.cuda_stream)
        ctx.synchronize()
        results[rows] = y.cpu().numpy()
        assert ".splitk:" in op.candidates[ctx.selected_candidates(1)[0]]

    for rows, got in results.items():
        want = ordinary(rows)
        assert np.array_equal(got, want), f"M={rows}: max |difference| {np.nanmax(np.abs(got - want)):.3e}"
        exact = oracle.evaluate(graph_with_rows(graph, rows), {"x": x_all[:rows]})["y"]
        assert_close_fp32(got, exact, what=f"split-K Gemm M={rows} (static scratch)")


def graph_with_rows(graph: workloads.GraphSpec, rows: int) -> workloads.GraphSpec:
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, K), "float32", "")
    g.constants.update(graph.constants)
    g.nodes.extend(graph.nodes)
    g.outputs.extend(graph.outputs)
    return g


def test_no_alloc_run_refuses_an_unprepared_context(tmp_path):
    """A context that never ran has no workspace, constants or code objects
    on the device: the allocation-free call reports that and enqueues nothing."""
    import torch

    graph, x_all = classifier_graph()
    eng = engine.build_engine(workloads.to_model(graph), engine.CompileOptions(tuning_mode="disabled"))
    ctx = eng.create_execution_context()
    x = torch.from_numpy(np.ascontiguousarray(x_all[:32])).to("cuda:0")
    y = torch.zeros((32, N), dtype=torch.float32, device="cuda:0")
    ctx.bind_input("x", x, layout="")
    ctx.bind_output("y", y, layout="")
    stream = torch.cuda.Stream()
    with pytest.raises(engine.CutritonError) as refused:
        ctx.run_async_no_alloc(stream.cuda_stream)
    assert "RunAsync first" in str(refused.value)
    ctx.synchronize()
    assert not y.any().item()
