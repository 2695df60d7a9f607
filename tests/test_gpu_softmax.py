"""Softmax over the last axis (softmax.fp16.last_axis) on the GPU against the
FP64 oracle (python/cutriton/triton_kernels/transformer.py:180-190 restated).

Bound: |y - e| <= 2^-10 |e| + 2^-24. The output is FP16: rounding costs half
an ulp (2^-11 relative, 2^-25 absolute among subnormals), and the FP32
arithmetic (exp on the max-shifted value, a sum over at most a few hundred
terms per lane, the reciprocal) stays below 1e-4 relative, which can move the
rounding by at most one more half ulp. Rows whose entries are all -inf give
NaN, as in the reference.
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from cutriton_amd.kernel_specs.transformer import SOFTMAX_VARIANTS
from oracle import oracle
from tests.helpers import filtered_pack, only_variant, run_graph

pytestmark = pytest.mark.gpu

KERNEL = "softmax.fp16.last_axis"

# Cached rows for each variant's limit (128 ... 4096 columns), rows that are
# not a multiple of a workgroup's rows, rows past every limit (aligned online
# pass), and column counts that are not a multiple of 8 (element-wise pass).
SHAPES = [(1, 1), (1, 8), (7, 128), (33, 256), (19, 512), (9, 1024), (5, 2048), (3, 4096), (4, 4104),
          (2, 20000), (3, 37), (65, 1001)]


def softmax_graph(rows: int, columns: int) -> workloads.GraphSpec:
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, columns), "float16", "")
    g.add("softmax", "Softmax", ["x"], ["y"], axis=-1)
    g.outputs.append("y")
    return g


def softmax_input(rng: np.random.Generator, rows: int, columns: int) -> np.ndarray:
    x = rng.standard_normal((rows, columns)) * 4
    if rows > 2 and columns > 1:
        x[1, rng.random(columns) < 0.5] = -np.inf          # masked entries (attention masks)
        x[1, 0] = 0.0
        x[2] = rng.uniform(60000.0, 65000.0, columns)       # exp alone would overflow
    return x.astype(np.float16)


def check(got: np.ndarray, x: np.ndarray, what: str) -> None:
    want = oracle.softmax(x.astype(np.float64))
    got = got.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(want)), what
    ok = ~np.isnan(want)
    err = np.abs(got[ok] - want[ok])
    bound = 2.0**-10 * np.abs(want[ok]) + 2.0**-24
    assert np.all(err <= bound), f"{what}: max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"


@pytest.mark.parametrize("variant", [name for name, _ in SOFTMAX_VARIANTS])
def test_softmax_variants(tmp_path, variant):
    rng = np.random.default_rng(41)
    pack = filtered_pack(tmp_path / "pack", only_variant(KERNEL, variant))
    opts = engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled")
    for rows, columns in SHAPES:
        x = softmax_input(rng, rows, columns)
        out, eng, _ = run_graph(softmax_graph(rows, columns), {"x": x}, opts)
        ops = eng.ops()
        assert len(ops) == 1 and ops[0].candidates[ops[0].selected_candidate].endswith(f"{KERNEL}:{variant}")
        check(out["y"], x, f"{variant} {rows}x{columns}")


def test_softmax_row_of_minus_infinity_is_nan_as_in_the_reference():
    x = np.full((4, 64), -np.inf, np.float16)
    x[0, :3] = (0.0, 1.0, 2.0)
    x[2, 5] = -3.0
    out, _, _ = run_graph(softmax_graph(4, 64), {"x": x})
    y = out["y"].astype(np.float64)
    assert np.isnan(y[1]).all() and np.isnan(y[3]).all()
    assert y[2, 5] == 1.0 and np.count_nonzero(y[2]) == 1
    check(out["y"], x, "masked rows")


def test_softmax_tuned_attention_scores(tmp_path):
    """Attention-score shape [batch*heads*queries, keys] with every variant a
    candidate; the tuner's pick must meet the same bound."""
    rng = np.random.default_rng(43)
    rows, columns = 4 * 16 * 128, 512
    x = softmax_input(rng, rows, columns)
    opts = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(tmp_path))
    out, eng, _ = run_graph(softmax_graph(rows, columns), {"x": x}, opts, repeats=2)
    ops = eng.ops()
    assert len(ops) == 1 and len(ops[0].candidates) == len(SOFTMAX_VARIANTS)
    check(out["y"], x, "tuned")
