"""Offline pre-tuning: point expansion and the CLI on the CPU; on the GPU a
small FFN profile is pre-tuned, checked by fresh TuneOnMiss and UseCache
engines, and a point inside the profile that was not pre-tuned runs from
the profile-opt choice with FFN parity (1e-2 absolute against the FP64
oracle)."""

from __future__ import annotations

import subprocess
import sys

import numpy as np
import pytest

from cutriton_amd import pretune
from tests.conftest import ROOT

RANGES = {"x": ((64, 256), (256, 256), (512, 256))}


def test_points_are_min_opt_max_then_extra_without_duplicates():
    points = pretune.expand_points(RANGES, [{"x": (128, 256)}, {"x": (256, 256)}])
    assert points == [{"x": (64, 256)}, {"x": (256, 256)}, {"x": (512, 256)}, {"x": (128, 256)}]


@pytest.mark.parametrize("point", [{"x": (32, 256)}, {"x": (1024, 256)}, {"x": (128, 128)}, {"x": (128,)}])
def test_points_outside_the_profile_are_rejected(point):
    with pytest.raises(ValueError, match="outside the profile"):
        pretune.expand_points(RANGES, [point])


def test_points_must_name_every_profiled_input():
    with pytest.raises(ValueError, match="every profiled input"):
        pretune.expand_points(RANGES, [{"y": (128, 256)}])


def test_cli_help_runs_without_a_device():
    out = subprocess.run([sys.executable, "-m", "cutriton_amd.pretune", "--help"], cwd=ROOT, capture_output=True,
                         text=True, timeout=120, check=True).stdout
    assert "--workload" in out and "--verify" in out


@pytest.mark.gpu
def test_pretuned_ffn_profile_resolves_from_the_cache(tmp_path):
    from cutriton_amd import engine, workloads
    from oracle import oracle
    import torch

    spec, x = workloads.ffn(512, 256, 1024)
    report = pretune.pretune(spec, RANGES, tmp_path, [{"x": (128, 256)}], verify=True, log=lambda _: None)
    assert report.verified and len(report.points) == 4
    assert report.points[0].written > 0
    files = sorted(p.name for p in tmp_path.glob("*.json"))
    assert len(files) == sum(p.written for p in report.points)

    # M = 200 was not pre-tuned: UseCache resolves it to the profile-opt
    # (M = 256) choice, writes nothing, and the result matches the oracle.
    opts = engine.CompileOptions(tuning_mode="use_cache", tuning_cache_dir=str(tmp_path),
                                 shape_profiles={"p": RANGES})
    eng = engine.build_engine(workloads.to_model(spec), opts)
    ctx = eng.create_execution_context()
    ctx.select_shape_profile("p")
    m = 200
    ctx.set_input_shape("x", (m, 256))
    ctx.resolve_shapes()
    xt = torch.from_numpy(np.ascontiguousarray(x[:m])).to("cuda:0")
    ctx.bind_input("x", xt, layout="")
    out = torch.empty((m, 256), dtype=torch.float16, device="cuda:0")
    ctx.bind_output("y", out, layout="")
    ctx.run()
    ops = eng.ops()
    selected = [ops[i].candidates[s] for i, s in enumerate(ctx.selected_candidates(len(ops)))]
    assert selected == report.points[1].selected
    assert sorted(p.name for p in tmp_path.glob("*.json")) == files
    got = out.cpu().numpy().astype(np.float64)
    want = oracle.evaluate(spec, {"x": x[:m]})["y"]
    assert np.abs(got - want).max() <= 1e-2
