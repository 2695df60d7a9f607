"""Offline pre-tuning across shape-profile points.

The reference's tuner (``src/runtime/engine.cpp:725-891``) times candidates
on the first run of every new shape (TuneOnMiss) or reads a cache
(UseCache, ``engine.cpp:750-788``); an offline pre-tuning tool is listed as
unfinished there (``docs/development.md:84-88``, ``README.md:337``). This
module is that tool for the gfx950 engine:

1. build the model with TuneOnMiss and one shape profile (min/opt/max per
   input);
2. for every profile point (min, opt, max and any extra points) bind seeded
   synthetic inputs of that shape and run once: every op with more than one
   candidate is timed at that shape and its choice written to the tuning
   cache, one JSON file per TuningKey (the reference's cache format,
   ``engine.cpp:311-335``);
3. optionally verify, with two fresh engines on the same folder: one in
   TuneOnMiss mode, which writes a cache file for any op whose key is
   missing, must write none and select the pre-tuned candidates at every
   point; one in UseCache mode must select the same candidates.

Points between the profile's min and max that were not pre-tuned resolve to
the profile-opt key under UseCache (``engine.cpp:750-788``).

Usage::

    python -m cutriton_amd.pretune --workload resnet50 --cache DIR --verify
    python -m cutriton_amd.pretune --workload ffn --cache DIR --points 1024,2048
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Sequence

import numpy as np

from . import engine, workloads

Shape = tuple[int, ...]
Ranges = dict[str, tuple[Sequence[int], Sequence[int], Sequence[int]]]


def expand_points(ranges: Ranges, extra: Sequence[dict[str, Sequence[int]]] = ()) -> list[dict[str, Shape]]:
    """The profile's min, opt and max points, then `extra` points, without
    duplicates, each checked to lie inside [min, max] on every axis."""
    points: list[dict[str, Shape]] = []
    for which in range(3):
        points.append({name: tuple(int(d) for d in r[which]) for name, r in ranges.items()})
    for point in extra:
        if set(point) != set(ranges):
            raise ValueError(f"a point must give every profiled input: {sorted(ranges)}")
        points.append({name: tuple(int(d) for d in shape) for name, shape in point.items()})
    unique: list[dict[str, Shape]] = []
    for point in points:
        for name, shape in point.items():
            lo, _, hi = ranges[name]
            if len(shape) != len(lo) or any(d < a or d > b for d, a, b in zip(shape, lo, hi)):
                raise ValueError(f"point {name}={shape} is outside the profile [{tuple(lo)}, {tuple(hi)}]")
        if point not in unique:
            unique.append(point)
    return unique


@dataclass
class PointReport:
    shapes: dict[str, Shape]
    seconds: float
    selected: list[str]
    written: int = 0


@dataclass
class Report:
    cache_dir: str
    points: list[PointReport] = field(default_factory=list)
    verified: bool = False

    def to_json(self) -> str:
        return json.dumps({
            "cache_dir": self.cache_dir, "verified": self.verified,
            "points": [{"shapes": {k: list(v) for k, v in p.shapes.items()}, "seconds": round(p.seconds, 3),
                        "cache_files_written": p.written, "selected": p.selected} for p in self.points],
        }, indent=1)


def _cache_files(cache_dir: Path) -> set[str]:
    return {p.name for p in cache_dir.glob("*.json")}


def _run_point(ctx: engine.ExecutionContext, eng: engine.Engine, spec: workloads.GraphSpec,
               shapes: dict[str, Shape], seed: int) -> list[int]:
    import torch

    rng = np.random.default_rng(seed)
    keep = []
    for name, shape in shapes.items():
        ctx.set_input_shape(name, list(shape))
    ctx.resolve_shapes()
    for name, shape in shapes.items():
        _, dtype, layout = spec.inputs[name]
        t = torch.from_numpy(rng.standard_normal(shape).astype(np.dtype(dtype))).to("cuda:0")
        keep.append(t)
        ctx.bind_input(name, t, layout=layout)
    for name in spec.outputs:
        out_shape, out_dtype, out_layout = ctx.resolved_desc(name)
        t = torch.empty(out_shape, dtype=getattr(torch, out_dtype), device="cuda:0")
        keep.append(t)
        ctx.bind_output(name, t, layout=out_layout)
    ctx.run()
    torch.cuda.synchronize()
    return ctx.selected_candidates(len(eng.ops()))


def pretune(spec: workloads.GraphSpec, ranges: Ranges, cache_dir: str | Path,
            extra_points: Sequence[dict[str, Sequence[int]]] = (), verify: bool = False, seed: int = workloads.SEED,
            log=print) -> Report:
    """Tunes `spec` at every point of the profile `ranges` into `cache_dir`."""
    cache = Path(cache_dir)
    cache.mkdir(parents=True, exist_ok=True)
    points = expand_points(ranges, extra_points)
    profile = {"pretune": ranges}
    report = Report(str(cache))
    options = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(cache), shape_profiles=profile,
                                    enable_profiling=False)
    eng = engine.build_engine(workloads.to_model(spec), options)
    ops = eng.ops()
    ctx = eng.create_execution_context()
    ctx.select_shape_profile("pretune")
    chosen: list[list[int]] = []
    for i, shapes in enumerate(points):
        before = _cache_files(cache)
        t0 = time.perf_counter()
        selected = _run_point(ctx, eng, spec, shapes, seed + i)
        seconds = time.perf_counter() - t0
        written = len(_cache_files(cache) - before)
        chosen.append(selected)
        report.points.append(PointReport(shapes, seconds, [ops[j].candidates[s] for j, s in enumerate(selected)],
                                         written))
        log(f"pretune {shapes}: {seconds:.1f} s, {written} cache files written")
    del ctx, eng
    if verify:
        for mode in ("tune_on_miss", "use_cache"):
            options = engine.CompileOptions(tuning_mode=mode, tuning_cache_dir=str(cache), shape_profiles=profile,
                                            enable_profiling=False)
            eng = engine.build_engine(workloads.to_model(spec), options)
            ctx = eng.create_execution_context()
            ctx.select_shape_profile("pretune")
            before = _cache_files(cache)
            for i, shapes in enumerate(points):
                selected = _run_point(ctx, eng, spec, shapes, seed + 1000 + i)
                if selected != chosen[i]:
                    raise RuntimeError(f"{mode}: other candidates selected at {shapes} than were pre-tuned")
            if _cache_files(cache) != before:
                raise RuntimeError(f"{mode}: tuning-cache files were written, so some key was not pre-tuned")
            del ctx, eng
        report.verified = True
        log(f"verified: the cache resolves every op at all {len(points)} points")
    return report


def _workload(name: str) -> tuple[workloads.GraphSpec, Ranges, str]:
    if name == "resnet50":
        return (workloads.resnet50(1),
                {"input": ((1, 3, 224, 224), (32, 3, 224, 224), (64, 3, 224, 224))}, "input")
    if name == "ffn":
        spec, _ = workloads.ffn(8192, 1024, 4096)
        return spec, {"x": ((128, 1024), (4096, 1024), (8192, 1024))}, "x"
    raise ValueError(f"unknown workload {name}")


def main(argv: Sequence[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--workload", choices=("resnet50", "ffn"), required=True)
    parser.add_argument("--cache", required=True, help="tuning-cache folder to fill")
    parser.add_argument("--points", default="",
                        help="extra leading-dimension sizes to tune besides the profile's min/opt/max, e.g. 8,16")
    parser.add_argument("--verify", action="store_true", help="check UseCache reproduces every pre-tuned choice")
    parser.add_argument("--report", default="", help="write a JSON report here")
    args = parser.parse_args(argv)
    spec, ranges, name = _workload(args.workload)
    lo = ranges[name][0]
    extra = [{name: (int(p),) + tuple(lo[1:])} for p in args.points.split(",") if p.strip()]
    report = pretune(spec, ranges, args.cache, extra, verify=args.verify,
                     log=lambda msg: print(msg, file=sys.stderr, flush=True))
    if args.report:
        Path(args.report).write_text(report.to_json())
    print(report.to_json())
    return 0


if __name__ == "__main__":
    sys.exit(main())
