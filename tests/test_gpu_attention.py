"""Fused attention (attention.fp16.*) on the GPU against the FP64 oracle.

Bound per element: |o - e| <= (2^-11 + 2e-4) max|V| + 2^-10 |e|, max|V| over
the (batch, head). P enters the second product rounded to FP16 (relative
2^-11 per weight) while the normaliser sums the unrounded weights, which
moves an output by at most 2^-11 of the largest |V| it averages; the FP32
logits, exp2 and sums add below 2e-4 of it; the FP16 output rounding is
half an ulp.
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from cutriton_amd.kernel_specs.transformer import ATTENTION_VARIANTS
from oracle import oracle
from tests.helpers import filtered_pack, run_graph

pytestmark = pytest.mark.gpu

# (batch, heads, queries, keys, head dimension, causal)
SHAPES = [
    (1, 1, 1, 1, 64, False),
    (2, 3, 17, 33, 64, True),
    (2, 3, 17, 33, 64, False),
    (1, 2, 128, 128, 64, True),
    (1, 1, 300, 5, 64, True),       # more queries than keys
    (1, 2, 130, 200, 40, False),    # head dimension below the variant's
    (1, 1, 19, 23, 36, True),       # head dimension not a multiple of 8
    (2, 2, 257, 257, 128, True),
    (1, 2, 64, 300, 96, False),
    (1, 1, 1000, 1000, 128, True),
]


def attention_graph(b, h, s_q, s_k, d, causal, scale=None):
    g = workloads.GraphSpec()
    for name, s in (("q", s_q), ("k", s_k), ("v", s_k)):
        g.inputs[name] = ((b, h, s, d), "float16", "")
    attrs = {"is_causal": int(causal)}
    if scale is not None:
        attrs["scale"] = scale
    g.add("attention", "Attention", ["q", "k", "v"], ["o"], **attrs)
    g.outputs.append("o")
    return g


def check(got: np.ndarray, feeds: dict, causal: bool, scale, what: str) -> None:
    want = oracle.attention(feeds["q"], feeds["k"], feeds["v"], scale, causal)
    vmax = np.abs(feeds["v"].astype(np.float64)).max(axis=(2, 3), keepdims=True)
    err = np.abs(got.astype(np.float64) - want)
    bound = (2.0**-11 + 2e-4) * vmax + 2.0**-10 * np.abs(want)
    assert np.all(err <= bound), f"{what}: max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"


@pytest.mark.parametrize("variant,dmax", ATTENTION_VARIANTS)
def test_attention_variants(tmp_path, variant, dmax):
    rng = np.random.default_rng(51)
    kid = f"attention.fp16.{variant}"
    pack = filtered_pack(tmp_path / "pack", lambda e: e["op_type"] != "Attention" or e["kernel_id"] == kid)
    opts = engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled")
    for b, h, s_q, s_k, d, causal in SHAPES:
        if d > dmax:
            continue
        feeds = {n: rng.standard_normal((b, h, s, d)).astype(np.float16)
                 for n, s in (("q", s_q), ("k", s_k), ("v", s_k))}
        out, eng, _ = run_graph(attention_graph(b, h, s_q, s_k, d, causal), feeds, opts)
        op = eng.ops()[0]
        assert op.candidates[op.selected_candidate].endswith(f"{kid}:w4")
        check(out["o"], feeds, causal, None, f"{variant} {(b, h, s_q, s_k, d, causal)}")


def test_attention_explicit_scale_and_large_logits():
    """An explicit scale, and logits of several hundred where exp would
    overflow without the running maximum."""
    rng = np.random.default_rng(53)
    feeds = {n: (rng.standard_normal((1, 2, 96, 64)) * 4).astype(np.float16) for n in ("q", "k", "v")}
    out, _, _ = run_graph(attention_graph(1, 2, 96, 96, 64, False, scale=2.0), feeds)
    check(out["o"], feeds, False, 2.0, "scale 2")


def test_attention_tuned(tmp_path):
    rng = np.random.default_rng(55)
    feeds = {n: rng.standard_normal((2, 4, 256, 64)).astype(np.float16) for n in ("q", "k", "v")}
    opts = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(tmp_path))
    out, eng, _ = run_graph(attention_graph(2, 4, 256, 256, 64, True), feeds, opts, repeats=2)
    assert len(eng.ops()[0].candidates) == 2
    check(out["o"], feeds, True, None, "tuned")
