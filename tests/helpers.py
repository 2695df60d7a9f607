"""Helpers shared by the GPU tests: running graphs through the engine,
filtered packs, and the tolerance checks."""

from __future__ import annotations

import json
import os
from pathlib import Path
from typing import Any, Iterable

import numpy as np

from cutriton_amd import engine, workloads
from cutriton_amd.native import PACK_DIR


def run_model(model: engine.Model, feeds: dict[str, np.ndarray], outputs: Iterable[str],
              input_layouts: dict[str, str], options: engine.CompileOptions | None = None,
              repeats: int = 1) -> tuple[dict[str, np.ndarray], engine.Engine, engine.ExecutionContext]:
    """Builds `model`, binds device copies of `feeds` and runs; returns host
    outputs (each bound in the layout the plan gives it), the engine and the
    context."""
    import torch

    eng = engine.build_engine(model, options or engine.CompileOptions(tuning_mode="disabled"))
    ctx = eng.create_execution_context()
    keep = []
    for name, value in feeds.items():
        t = torch.from_numpy(np.ascontiguousarray(value)).to("cuda:0")
        keep.append(t)
        ctx.bind_input(name, t, layout=input_layouts[name])
    outs = {}
    for name in outputs:
        shape, dtype = eng.value_desc(name)
        t = torch.empty(shape, dtype=getattr(torch, dtype), device="cuda:0")
        outs[name] = t
        ctx.bind_output(name, t, layout=eng.value_layout(name))
    for _ in range(repeats):
        ctx.run()
    return {k: v.cpu().numpy() for k, v in outs.items()}, eng, ctx


def run_graph(graph: workloads.GraphSpec, feeds: dict[str, np.ndarray], options: engine.CompileOptions | None = None,
              repeats: int = 1) -> tuple[dict[str, np.ndarray], engine.Engine, engine.ExecutionContext]:
    """Builds, binds (device copies of `feeds`) and runs `graph`; returns host outputs."""
    layouts = {name: graph.inputs[name][2] for name in feeds}
    return run_model(workloads.to_model(graph), feeds, graph.outputs, layouts, options, repeats)


def filtered_pack(tmp: Path, keep: Any) -> str:
    """A pack holding the entries of the built pack for which keep(entry) is
    true; if a kept op/dtype loses its default, its first kept entry becomes
    the default. Binaries are shared through a symlink."""
    pack = json.loads((PACK_DIR / "pack.json").read_text())
    kept = [e for e in pack["kernels"] if keep(e)]
    by_key: dict[tuple[str, str, str], list[dict]] = {}
    for e in kept:
        by_key.setdefault((e["op_type"], e["dtype"], e["kernel_id"]), []).append(e)
    for entries in by_key.values():
        if not any(e["default"] for e in entries):
            entries[0]["default"] = True
    pack["kernels"] = kept
    tmp.mkdir(parents=True, exist_ok=True)
    (tmp / "pack.json").write_text(json.dumps(pack))
    link = tmp / "kernels"
    if not link.exists():
        os.symlink(PACK_DIR / "kernels", link)
    return str(tmp)


def only_variant(kernel_id: str, variant_id: str):
    def keep(e: dict) -> bool:
        return e["kernel_id"] != kernel_id or e["variant_id"] == variant_id
    return keep


def only_kernel_variant(kernel_id: str, variant_id: str, family_prefix: str):
    """Keeps only `variant_id` of `kernel_id` among the kernels whose id starts
    with `family_prefix` (the sibling implementations of the same op)."""
    def keep(e: dict) -> bool:
        if not e["kernel_id"].startswith(family_prefix + "."):
            return True
        return e["kernel_id"] == kernel_id and e["variant_id"] == variant_id
    return keep


def without_kernels(kernel_ids: Iterable[str]):
    ids = set(kernel_ids)
    return lambda e: e["kernel_id"] not in ids


def assert_close_fp32(got: np.ndarray, want: np.ndarray, rtol: float = 1e-4, what: str = "") -> float:
    """Per-element |got - want| <= rtol*|want| + rtol*max(1, rms(want)).

    The absolute floor is the relative tolerance scaled by the output's RMS:
    elements near zero are judged against the size of the whole output,
    which is what an FP32 sum of many terms can guarantee."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    scale = max(1.0, float(np.sqrt(np.mean(want ** 2)))) if want.size else 1.0
    err = np.abs(got - want)
    bound = rtol * np.abs(want) + rtol * scale
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - bound, -np.inf)), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {err.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]!r} want {want[i]!r} (err {err[i]:.3e}, bound {bound[i]:.3e})")
    return float(err.max()) if err.size else 0.0
