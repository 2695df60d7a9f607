"""Kernel-family parity on the GPU: every pack variant against the FP64 oracle.

Each case builds a small graph, lowers it through the engine (a filtered
pack pins the variant under test), runs it on cuda:0 through the C ABI and
compares with oracle.evaluate on the same inputs.
Tolerances: FP32 ops 1e-4 relative with a 1e-4*RMS floor; MaxPool and the
Flatten view bit-exact; FP16 outputs 1e-2 absolute against FP64.
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from cutriton_amd.kernel_specs.resnet import CONV_TILES, DIRECT_TILES, SPLIT_TILES
from cutriton_amd.kernel_specs.transformer import GEMM_NT_SPLIT_TILES, GEMM_NT_TILES, ROW_VARIANTS
from oracle import oracle
from tests.helpers import (assert_close_fp32, filtered_pack, only_kernel_variant, only_variant, run_graph,
                           without_kernels)

pytestmark = pytest.mark.gpu

# Every conv tile the pack builds: LDS-staged, split-K and register-direct.
CONV_VARIANTS = tuple(f"mfma:{v[0]}" for v in CONV_TILES) + tuple(f"splitk:{v[0]}" for v in SPLIT_TILES) + \
    tuple(f"direct:{v[0]}" for v in DIRECT_TILES)
# (kernel-id suffix, variant): "" reads the constant B from its [N][K] copy,
# "_kn" reads B as it is.
GEMM16_VARIANTS = tuple(("", v[0]) for v in GEMM_NT_TILES + GEMM_NT_SPLIT_TILES) + \
    tuple(("_kn", v) for v in ("m64n64k64", "m128n128k64", "m256n128k64", "m256n256k64"))


def conv_graph(rng, n, c, h, w, k, r, stride, pad, dil, tail: str):
    """Conv -> BatchNormalization [-> Relu | -> Add(residual) -> Relu]."""
    g = workloads.GraphSpec()
    g.inputs["x"] = ((n, c, h, w), "float32", "NCHW")
    wt = rng.normal(0, np.sqrt(2.0 / (c * r * r)), (k, c, r, r)).astype(np.float32)
    g.constant("w", wt, "OIHW")
    names = []
    for nm, arr in (("scale", rng.uniform(0.5, 1.5, k)), ("bias", rng.normal(0, 0.1, k)),
                    ("mean", rng.normal(0, 0.1, k)), ("var", rng.uniform(0.5, 1.5, k))):
        names.append(g.constant(nm, arr.astype(np.float32)))
    y = g.add("conv", "Conv", ["x", "w"], ["conv_y"], strides=[stride, stride], pads=[pad] * 4,
              dilations=[dil, dil])
    feeds = {"x": rng.standard_normal((n, c, h, w), dtype=np.float32)}
    if tail == "conv":
        g.outputs.append(y)
        return g, feeds
    y = g.add("bn", "BatchNormalization", [y, *names], ["bn_y"], epsilon=1e-5)
    if tail == "relu":
        y = g.add("relu", "Relu", [y], ["out"])
    elif tail == "add_relu":
        oh = (h + 2 * pad - dil * (r - 1) - 1) // stride + 1
        ow = (w + 2 * pad - dil * (r - 1) - 1) // stride + 1
        g.inputs["res"] = ((n, k, oh, ow), "float32", "NCHW")
        feeds["res"] = rng.standard_normal(g.inputs["res"][0], dtype=np.float32)
        y = g.add("add", "Add", [y, "res"], ["sum"])
        y = g.add("relu", "Relu", [y], ["out"])
    g.outputs.append(y)
    return g, feeds


CONV_SHAPES = [
    # n, c, h, w, k, r, stride, pad, dil
    (1, 64, 56, 56, 64, 3, 1, 1, 1),     # the single-node configuration
    (2, 36, 15, 13, 40, 3, 2, 1, 1),     # ragged tiles, stride 2, non-square
    (2, 20, 7, 7, 72, 1, 1, 0, 1),       # 1x1, P*Q = 49 straddles tile columns
    (1, 3, 31, 29, 16, 7, 2, 3, 1),      # stem-like: C*R*S = 147 (scalar weight loads)
    (1, 8, 12, 12, 24, 3, 1, 2, 2),      # dilation 2
    # C a multiple of the depth tile: the channel-run loader
    (2, 64, 9, 11, 40, 3, 2, 1, 1),      # stride 2, ragged tiles
    (1, 64, 12, 12, 24, 3, 1, 2, 2),     # dilation 2, padding 2
    (2, 64, 14, 14, 72, 1, 2, 0, 1),     # strided 1x1 (downsample)
    (1, 48, 10, 10, 20, 3, 1, 1, 1),     # C = 48: channel runs only for 16-deep tiles
]


CONV_TAILS = {"relu": "conv_bn_relu.fp32.nchw", "bn": "conv_bn.fp32.nchw",
              "add_relu": "conv_bn_add_relu.fp32.nchw", "conv": "conv.fp32.nchw"}
# Every tile variant runs the residual-join epilogue (BN + residual + ReLU,
# the one that reads the most); every epilogue runs on one variant of each
# family. The epilogue code is shared by all tiles of a family.
CONV_CASES = [(fv, "add_relu") for fv in CONV_VARIANTS] + [
    (fv, tail) for fv in ("mfma:m64n64", "splitk:m64n64s4", "direct:d64n64") for tail in ("relu", "bn", "conv")]


@pytest.mark.parametrize("family_variant,tail", CONV_CASES)
def test_conv_family_variants(tmp_path, family_variant, tail):
    kernel_base = CONV_TAILS[tail]
    rng = np.random.default_rng(7)
    family, variant = family_variant.split(":")
    kernel_id = f"{kernel_base}.{family}"
    pack = filtered_pack(tmp_path / "pack", only_kernel_variant(kernel_id, variant, kernel_base))
    for shape in CONV_SHAPES:
        g, feeds = conv_graph(rng, *shape, tail=tail)
        opts = engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled")
        out, eng, _ = run_graph(g, feeds, opts)
        ops = eng.ops()
        assert len(ops) == 1 and ops[0].candidates[ops[0].selected_candidate].endswith(f"{kernel_id}:{variant}"), ops
        want = oracle.evaluate(g, feeds)[g.outputs[0]]
        assert_close_fp32(out[g.outputs[0]], want, what=f"{kernel_id}:{variant} {shape}")


SMALLC_SHAPES = [
    # n, c, h, w, k, r, stride, pad, dil
    (2, 3, 33, 29, 16, 7, 2, 3, 1),     # stem-like, P = 17 and Q = 15: ragged rows and columns
    (1, 3, 64, 240, 64, 7, 2, 3, 1),    # Q = 120: two column chunks
    (2, 4, 9, 11, 40, 3, 1, 1, 1),      # 3x3, K = 40: a partial channel block
    (1, 1, 12, 12, 8, 1, 1, 0, 1),      # 1x1, one channel
    (1, 4, 40, 60, 8, 7, 1, 3, 6),      # dilation 6: the patch exceeds LDS (global path)
]


@pytest.mark.parametrize("tail,kernel_base", [
    ("relu", "conv_bn_relu.fp32.nchw"),
    ("bn", "conv_bn.fp32.nchw"),
    ("add_relu", "conv_bn_add_relu.fp32.nchw"),
    ("conv", "conv.fp32.nchw"),
])
def test_small_channel_conv(tmp_path, tail, kernel_base):
    rng = np.random.default_rng(41)
    kernel_id = f"{kernel_base}.smallc"
    pack = filtered_pack(tmp_path / "pack", only_kernel_variant(kernel_id, "r2c64", kernel_base))
    for shape in SMALLC_SHAPES:
        g, feeds = conv_graph(rng, *shape, tail=tail)
        out, eng, _ = run_graph(g, feeds, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
        ops = eng.ops()
        assert len(ops) == 1 and ops[0].candidates[ops[0].selected_candidate].endswith(f"{kernel_id}:r2c64"), ops
        assert_close_fp32(out[g.outputs[0]], oracle.evaluate(g, feeds)[g.outputs[0]], what=f"{kernel_id} {shape}")


def test_small_channel_conv_does_not_match_wide_inputs():
    """dim_le keeps the few-channel kernel off a convolution with C = 8."""
    rng = np.random.default_rng(43)
    g, _ = conv_graph(rng, 1, 8, 12, 12, 16, 3, 1, 1, 1, tail="relu")
    ops = engine.build_engine(workloads.to_model(g), engine.CompileOptions(tuning_mode="disabled")).ops()
    assert not any(".smallc:" in cand for cand in ops[0].candidates), ops[0].candidates


@pytest.mark.parametrize("channels,variant", [(8, "m64n64s5"), (32, "m64n64s6")])
def test_split_k_with_empty_shares(tmp_path, channels, variant):
    """Splits whose depth range is empty add zero: 8 channels x 3 x 3 = 3 depth
    tiles of 32 over 5 splits (general gather), and 32 channels x 3 x 3 = 9
    tiles over 6 splits of 2 (channel-run gather, the last split starts past
    the last tap)."""
    rng = np.random.default_rng(29)
    kernel_id = "conv_bn_relu.fp32.nchw.splitk"
    pack = filtered_pack(tmp_path / "pack", only_kernel_variant(kernel_id, variant, "conv_bn_relu.fp32.nchw"))
    g, feeds = conv_graph(rng, 2, channels, 10, 10, 16, 3, 1, 1, 1, tail="relu")
    out, eng, _ = run_graph(g, feeds, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
    assert eng.ops()[0].candidates[eng.ops()[0].selected_candidate].endswith(f"{kernel_id}:{variant}")
    assert_close_fp32(out[g.outputs[0]], oracle.evaluate(g, feeds)[g.outputs[0]], what=f"{variant}, C={channels}")


@pytest.mark.parametrize("variant", ["m128n128s2", "m128n128s8", "m64n64s4", "m64n64s5"])
def test_split_k_shares_follow_the_inputs(tmp_path, variant):
    """Split-K partial sums travel through the runtime scratch and the tile
    counters reset themselves: consecutive launches on one context with
    different inputs each match the oracle (a stale share or counter from the
    previous launch would not), also under hipGraph replay."""
    import torch

    rng = np.random.default_rng(23)
    kernel_id = "conv_bn_relu.fp32.nchw.splitk"
    pack = filtered_pack(tmp_path / "pack", only_kernel_variant(kernel_id, variant, "conv_bn_relu.fp32.nchw"))
    g, feeds_a = conv_graph(rng, 2, 256, 14, 14, 256, 3, 1, 1, 1, tail="relu")
    feeds_b = {"x": rng.standard_normal(feeds_a["x"].shape, dtype=np.float32) * 3.0}
    eng = engine.build_engine(workloads.to_model(g), engine.CompileOptions(kernel_artifact_dir=pack,
                                                                           tuning_mode="disabled"))
    assert eng.ops()[0].candidates[eng.ops()[0].selected_candidate].endswith(f"{kernel_id}:{variant}")
    ctx = eng.create_execution_context()
    x = torch.empty(feeds_a["x"].shape, device="cuda:0")
    shape, _ = eng.value_desc(g.outputs[0])
    y = torch.empty(shape, device="cuda:0")
    ctx.bind_input("x", x)
    ctx.bind_output(g.outputs[0], y, layout="NCHW")
    want = {"a": oracle.evaluate(g, feeds_a)[g.outputs[0]], "b": oracle.evaluate(g, feeds_b)[g.outputs[0]]}
    for which in ("a", "b", "b", "a", "b"):
        x.copy_(torch.from_numpy((feeds_a if which == "a" else feeds_b)["x"]))
        ctx.run()
        assert_close_fp32(y.cpu().numpy(), want[which], what=f"{variant} input {which}")


@pytest.mark.parametrize("op", ["BatchNormalization", "Relu", "Add", "AddRelu"])
@pytest.mark.parametrize("shape", [(2, 24, 9, 11), (1, 3, 5, 5), (32, 64, 56, 56)])
def test_fp32_elementwise_kernels(op, shape):
    """The unfused decomposition kernels (fusion.cpp:44-55 alternatives) as
    single-op graphs; Add -> Relu fuses to AddRelu."""
    rng = np.random.default_rng(11)
    g = workloads.GraphSpec()
    g.inputs["a"] = (shape, "float32", "NCHW")
    feeds = {"a": rng.standard_normal(shape, dtype=np.float32)}
    if op == "BatchNormalization":
        c = shape[1]
        names = [g.constant(nm, arr.astype(np.float32)) for nm, arr in (
            ("scale", rng.uniform(0.5, 1.5, c)), ("bias", rng.normal(0, 0.1, c)),
            ("mean", rng.normal(0, 0.1, c)), ("var", rng.uniform(0.5, 1.5, c)))]
        g.add("bn", "BatchNormalization", ["a", *names], ["y"], epsilon=1e-5)
    elif op == "Relu":
        g.add("relu", "Relu", ["a"], ["y"])
    else:
        g.inputs["b"] = (shape, "float32", "NCHW")
        feeds["b"] = rng.standard_normal(shape, dtype=np.float32)
        y = g.add("add", "Add", ["a", "b"], ["s" if op == "AddRelu" else "y"])
        if op == "AddRelu":
            g.add("relu", "Relu", [y], ["y"])
    g.outputs.append("y")
    out, eng, _ = run_graph(g, feeds)
    assert [o.op_type for o in eng.ops()] == [op]
    assert_close_fp32(out["y"], oracle.evaluate(g, feeds)["y"], what=f"{op} {shape}")


def test_tuner_runs_every_candidate(tmp_path):
    """TuneOnMiss times every candidate of each op (fused variants and the
    unfused decomposition) after checking it against candidate 0, writes one
    cache file per op, and a second build reads the cache without rewriting."""
    rng = np.random.default_rng(23)
    g, feeds = conv_graph(rng, 2, 32, 14, 14, 64, 3, 1, 1, 1, tail="add_relu")
    cache = tmp_path / "tuning"
    opts = engine.CompileOptions(tuning_mode="tune_on_miss", tuning_cache_dir=str(cache),
                                 tuning_warmup_iterations=1, tuning_measurement_iterations=3)
    out, eng, ctx = run_graph(g, feeds, opts)
    assert_close_fp32(out[g.outputs[0]], oracle.evaluate(g, feeds)[g.outputs[0]], what="tuned conv")
    files = sorted(cache.glob("*.json"))
    assert len(files) == 1
    chosen = files[0].read_text()
    assert any(c in chosen for c in eng.ops()[0].candidates)
    stamp = files[0].stat().st_mtime_ns
    out2, _, _ = run_graph(g, feeds, opts)
    assert files[0].stat().st_mtime_ns == stamp
    assert np.array_equal(out[g.outputs[0]], out2[g.outputs[0]])


@pytest.mark.parametrize("family,variant", (("mfma", "m64n64"), ("mfma", "m128n128"), ("splitk", "m64n64s8"),
                                            ("splitk", "m64n64s16")))
@pytest.mark.parametrize("m,k,n,bias", [(32, 2048, 1000, False), (5, 37, 29, True), (130, 64, 70, False),
                                         (3, 2048, 1000, True)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_gemm_fp32(tmp_path, family, variant, m, k, n, bias, trans_b):
    """transB = 1 (B stored [N][K], as an exported Linear layer has it) runs
    the "_tb" entries, which read B's transposed copy."""
    rng = np.random.default_rng(3)
    base = "gemm_bias.fp32" if bias else "gemm.fp32"
    suffix = "_tb" if trans_b else ""
    kid = f"{base}.{family}{suffix}"
    sibling = f"{base}.{'splitk' if family == 'mfma' else 'mfma'}{suffix}"

    def keep(e: dict) -> bool:
        return e["kernel_id"] != sibling and (e["kernel_id"] != kid or e["variant_id"] == variant)

    pack = filtered_pack(tmp_path / "pack", keep)
    g = workloads.GraphSpec()
    g.inputs["a"] = ((m, k), "float32", "")
    g.constant("b", rng.normal(0, 0.05, (n, k) if trans_b else (k, n)).astype(np.float32))
    ins = ["a", "b"]
    if bias:
        ins.append(g.constant("bias", rng.normal(0, 0.1, n).astype(np.float32)))
    g.add("gemm", "Gemm", ins, ["y"], **({"transB": 1} if trans_b else {}))
    g.outputs.append("y")
    feeds = {"a": rng.standard_normal((m, k), dtype=np.float32)}
    out, eng, _ = run_graph(g, feeds, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
    op = eng.ops()[0]
    assert op.candidates[op.selected_candidate].endswith(f"{kid}:{variant}")
    assert_close_fp32(out["y"], oracle.evaluate(g, feeds)["y"], what=f"gemm fp32 {variant} {m}x{k}x{n}")


@pytest.mark.parametrize("shape,kernel,stride,pad", [
    ((2, 64, 112, 112), 3, 2, 1),   # ResNet stem pool
    ((1, 5, 17, 14), 3, 2, 1),      # ragged
    ((2, 3, 9, 9), 2, 2, 0),        # no padding, even window
    ((1, 2, 8, 3000), 3, 1, 1),     # band too wide for LDS: global reads
    ((3, 4, 30, 7), 3, 1, 0),       # stride 1, bands with a ragged last one
])
def test_max_pool_bit_exact(shape, kernel, stride, pad):
    rng = np.random.default_rng(5)
    g = workloads.GraphSpec()
    g.inputs["x"] = (shape, "float32", "NCHW")
    g.add("pool", "MaxPool", ["x"], ["y"], kernel_shape=[kernel, kernel], strides=[stride, stride],
          pads=[pad] * 4, dilations=[1, 1])
    g.outputs.append("y")
    feeds = {"x": rng.standard_normal(shape, dtype=np.float32)}
    out, _, _ = run_graph(g, feeds)
    want = oracle.evaluate(g, feeds)["y"].astype(np.float32)
    assert np.array_equal(out["y"].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("variant", ["w4", "b16g4", "d8"])
@pytest.mark.parametrize("shape,kernel,stride,pad", [
    ((2, 8, 112, 112), 3, 2, 1),    # stem pool: even/odd split rows
    ((1, 3, 20, 24), 3, 1, 1),      # stride 1: plain staged rows
    ((1, 2, 17, 14), 3, 2, 1),      # rows not whole float4s: global reads
    ((1, 2, 9, 16), 2, 2, 0),       # even window, no padding, split rows
    ((1, 3, 15, 16), 3, 2, 1),      # odd height: the last window hangs below the image
])
def test_max_pool_special_values(tmp_path, variant, shape, kernel, stride, pad):
    """Bit-exact against the oracle on inputs full of NaN, +-inf and +-0:
    NaN never wins (an all-NaN window gives -inf), +0 beats -0."""
    rng = np.random.default_rng(17)
    specials = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.5, -2.0], dtype=np.float32)
    x = rng.standard_normal(shape, dtype=np.float32)
    mask = rng.random(shape) < 0.6
    x[mask] = rng.choice(specials, size=int(mask.sum()))
    x[0, 0, :4, :4] = np.nan                    # all-NaN windows
    x[0, -1, -4:, -4:] = -0.0                   # windows of -0 only
    x[0, -1, -4:, -2] = 0.0                     # and with a +0 among them
    g = workloads.GraphSpec()
    g.inputs["x"] = (shape, "float32", "NCHW")
    g.add("pool", "MaxPool", ["x"], ["y"], kernel_shape=[kernel, kernel], strides=[stride, stride],
          pads=[pad] * 4, dilations=[1, 1])
    g.outputs.append("y")
    kid = "max_pool.fp32.nchw"
    pack = filtered_pack(tmp_path / "pack", lambda e: e["kernel_id"] != kid or e["variant_id"] == variant)
    out, eng, _ = run_graph(g, {"x": x}, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
    op = eng.ops()[0]
    assert op.candidates[op.selected_candidate].endswith(f"{kid}:{variant}"), op
    want = oracle.evaluate(g, {"x": x})["y"].astype(np.float32)
    assert not np.isnan(want).any()
    assert np.array_equal(out["y"].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("shape", [(2, 2048, 7, 7), (3, 5, 1, 1), (1, 3, 60, 61), (1, 300, 8, 8), (1, 70, 7, 7)])
@pytest.mark.parametrize("variant", ["w4", "p16"])
def test_global_average_pool(tmp_path, shape, variant):
    rng = np.random.default_rng(9)
    g = workloads.GraphSpec()
    g.inputs["x"] = (shape, "float32", "NCHW")
    g.add("gap", "GlobalAveragePool", ["x"], ["y"])
    g.outputs.append("y")
    feeds = {"x": rng.standard_normal(shape, dtype=np.float32)}
    kid = "global_average_pool.fp32.nchw"
    pack = filtered_pack(tmp_path / "pack", lambda e: e["kernel_id"] != kid or e["variant_id"] == variant)
    out, eng, _ = run_graph(g, feeds, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
    op = eng.ops()[0]
    assert op.candidates[op.selected_candidate].endswith(f"{kid}:{variant}"), op
    assert_close_fp32(out["y"], oracle.evaluate(g, feeds)["y"], what=f"gap {shape}")


def gemm16_graph(rng, m, k, n, gelu, bias, trans_b=False):
    g = workloads.GraphSpec()
    g.inputs["a"] = ((m, k), "float16", "")
    g.constant("b", rng.normal(0, 0.05, (n, k) if trans_b else (k, n)).astype(np.float16))
    ins = ["a", "b"]
    if bias:
        ins.append(g.constant("bias", rng.normal(0, 0.1, n).astype(np.float16)))
    y = g.add("gemm", "Gemm", ins, ["h"], **({"transB": 1} if trans_b else {}))
    if gelu:
        y = g.add("gelu", "Gelu", [y], ["y"])
    g.outputs.append(y)
    return g, {"a": rng.standard_normal((m, k)).astype(np.float16)}


# Every tile variant runs the bias + GELU epilogue; every epilogue runs on
# one variant of each family.
# "_tb" (transB = 1, B stored [N][K]) runs the NT tiles on B as it is.
GEMM16_CASES = [(f, v, True, True) for f, v in GEMM16_VARIANTS] + [
    ("_tb", v, True, True) for f, v in GEMM16_VARIANTS if f == ""] + [
    (f, v, gelu, bias) for f, v in (("", "m128n128w4"), ("_kn", "m128n128k64"), ("_tb", "m128n128w4"))
    for gelu, bias in ((False, False), (True, False), (False, True))]


@pytest.mark.parametrize("family,variant,gelu,bias", GEMM16_CASES)
def test_gemm_fp16_variants(tmp_path, family, variant, gelu, bias):
    rng = np.random.default_rng(13)
    base = {(False, False): "gemm.fp16.mfma", (True, False): "gemm_gelu.fp16.mfma",
            (False, True): "gemm_bias.fp16.mfma", (True, True): "gemm_gelu_bias.fp16.mfma"}[(gelu, bias)]
    kid = base + family
    # The other family serving the same transB; none serves transB = 1.
    sibling = {"": base + "_kn", "_kn": base, "_tb": None}[family]
    trans_b = family == "_tb"

    def keep(e: dict) -> bool:
        if e["kernel_id"] == sibling:
            return False
        return e["kernel_id"] != kid or e["variant_id"] == variant

    pack = filtered_pack(tmp_path / "pack", keep)
    # Full and ragged tiles, N not a multiple of 4, depth not a multiple of 8
    # (the element-wise loader) and of the 64-deep tile.
    for m, k, n in ((512, 768, 3072), (17, 128, 40), (70, 72, 37), (300, 200, 264), (33, 100, 50), (1, 8, 4),
                    (260, 96, 520)):
        g, feeds = gemm16_graph(rng, m, k, n, gelu, bias, trans_b)
        out, eng, _ = run_graph(g, feeds, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
        ops = eng.ops()
        assert len(ops) == 1 and ops[0].candidates[ops[0].selected_candidate].endswith(f"{kid}:{variant}"), ops
        want = oracle.evaluate(g, feeds)[g.outputs[0]]
        err = np.abs(out[g.outputs[0]].astype(np.float64) - want)
        assert err.max() <= 1e-2, f"{kid}:{variant} {(m, k, n)} max abs err {err.max():.3e}"


@pytest.mark.parametrize("variant", [v[0] for v in GEMM_NT_SPLIT_TILES])
def test_gemm_fp16_split_k_shares_follow_the_inputs(tmp_path, variant):
    """FP16 split-K: consecutive launches on one context with different
    inputs each match the oracle (a stale share or counter from the previous
    launch would not), also under hipGraph replay; the last share of the
    (1, 8, 4) product is empty (one depth tile for up to four shares)."""
    import torch

    rng = np.random.default_rng(29)
    kid = "gemm_gelu_bias.fp16.mfma"
    pack = filtered_pack(tmp_path / "pack", lambda e: e["kernel_id"] not in (kid, kid + "_kn") or
                         (e["kernel_id"] == kid and e["variant_id"] == variant))
    for m, k, n in ((512, 3072, 768), (1, 8, 4)):
        g, feeds_a = gemm16_graph(rng, m, k, n, True, True)
        feeds_b = {"a": (rng.standard_normal((m, k)) * 2).astype(np.float16)}
        eng = engine.build_engine(workloads.to_model(g), engine.CompileOptions(kernel_artifact_dir=pack,
                                                                               tuning_mode="disabled"))
        assert eng.ops()[0].candidates[eng.ops()[0].selected_candidate].endswith(f"{kid}:{variant}")
        ctx = eng.create_execution_context()
        a = torch.empty((m, k), dtype=torch.float16, device="cuda:0")
        y = torch.empty((m, n), dtype=torch.float16, device="cuda:0")
        ctx.bind_input("a", a, layout="")
        ctx.bind_output(g.outputs[0], y, layout="")
        want = {"a": oracle.evaluate(g, feeds_a)[g.outputs[0]], "b": oracle.evaluate(g, feeds_b)[g.outputs[0]]}
        for which in ("a", "b", "b", "a", "b"):
            a.copy_(torch.from_numpy((feeds_a if which == "a" else feeds_b)["a"]))
            ctx.run()
            err = np.abs(y.cpu().numpy().astype(np.float64) - want[which]).max()
            assert err <= 1e-2, f"{variant} {(m, k, n)} input {which}: max abs err {err:.3e}"


@pytest.mark.parametrize("family", ["", "_kn"])
def test_gemm_gelu_epilogue_over_the_activation_range(tmp_path, family):
    """The fused erf-GELU epilogue on exactly known pre-activations: a one-hot
    product passes a[i, 0] + bias[j] through unchanged, for a[i, 0] over
    [-12, 12] and the special values 0 and +-1e-6, so each output is within
    one FP16 rounding (plus the erfc evaluation's 1e-6) of GELU(a + bias)
    evaluated in float64."""
    from scipy.special import erf

    m, k, n = 520, 16, 64
    vals = np.concatenate([np.linspace(-12.0, 12.0, m - 8), [0.0, 1e-6, -1e-6, 0.5, -0.5, 3.0, -3.0, 8.0]])
    a = np.zeros((m, k), np.float16)
    a[:, 0] = vals.astype(np.float16)
    b = np.zeros((k, n), np.float16)
    b[0, :] = 1.0
    bias = np.zeros(n, np.float16)
    bias[n // 2:] = np.linspace(-0.25, 0.25, n - n // 2).astype(np.float16)
    g = workloads.GraphSpec()
    g.inputs["a"] = ((m, k), "float16", "")
    g.constant("b", b)
    g.constant("bias", bias)
    y = g.add("gemm", "Gemm", ["a", "b", "bias"], ["h"])
    g.add("gelu", "Gelu", [y], ["y"])
    g.outputs.append("y")
    base = "gemm_gelu_bias.fp16.mfma"
    kid, sibling = base + family, base + ("_kn" if family == "" else "")
    pack = filtered_pack(tmp_path / "pack", lambda e: e["kernel_id"] != sibling)
    out, eng, _ = run_graph(g, {"a": a}, engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled"))
    assert kid + ":" in eng.ops()[0].candidates[eng.ops()[0].selected_candidate]
    pre = a[:, :1].astype(np.float64) + bias[None, :].astype(np.float64)
    want = 0.5 * pre * (1.0 + erf(pre / np.sqrt(2.0)))
    # One FP16 rounding (2^-11 relative, doubled) plus the absolute error of
    # the FP32 erfc evaluation (below 1e-6, doubled): the floor matters only
    # in the negative tail, where GELU is a few 1e-6.
    err = np.abs(out["y"].astype(np.float64) - want)
    bound = 2.0 ** -10 * np.abs(want) + 2e-6
    assert np.all(err <= bound), (err.max(), pre.ravel()[np.argmax(err - bound)])


def test_gemm_fp16_activation_operand_uses_b_as_is():
    """With B an activation there is no transposed copy to read: only the
    kernels that read B as it is lower, and they compute the product."""
    rng = np.random.default_rng(31)
    m, k, n = 96, 200, 72
    g = workloads.GraphSpec()
    g.inputs["a"] = ((m, k), "float16", "")
    g.inputs["b"] = ((k, n), "float16", "")
    g.add("gemm", "Gemm", ["a", "b"], ["y"])
    g.outputs.append("y")
    feeds = {"a": rng.standard_normal((m, k)).astype(np.float16),
             "b": rng.normal(0, 0.05, (k, n)).astype(np.float16)}
    out, eng, _ = run_graph(g, feeds)
    candidates = eng.ops()[0].candidates
    assert candidates and all(".fp16.mfma_kn:" in c for c in candidates), candidates
    err = np.abs(out["y"].astype(np.float64) - oracle.evaluate(g, feeds)["y"])
    assert err.max() <= 1e-2, err.max()


def layer_norm_graph(rng, rows, cols, skip):
    g = workloads.GraphSpec()
    g.inputs["x"] = ((rows, cols), "float16", "")
    feeds = {"x": rng.standard_normal((rows, cols)).astype(np.float16)}
    gamma = g.constant("gamma", rng.uniform(0.5, 1.5, cols).astype(np.float16))
    beta = g.constant("beta", rng.normal(0, 0.1, cols).astype(np.float16))
    y = "x"
    if skip:
        g.inputs["r"] = ((rows, cols), "float16", "")
        feeds["r"] = rng.standard_normal((rows, cols)).astype(np.float16)
        y = g.add("add", "Add", ["x", "r"], ["s"])
    g.add("ln", "LayerNormalization", [y, gamma, beta], ["y"], axis=-1, epsilon=1e-5)
    g.outputs.append("y")
    return g, feeds


@pytest.mark.parametrize("variant", [name for name, _ in ROW_VARIANTS])
@pytest.mark.parametrize("skip", [False, True])
def test_layer_norm_fp16(tmp_path, variant, skip):
    """Every row-group variant over rows at each variant's register limit,
    ragged row counts, rows past every limit and unaligned column counts."""
    rng = np.random.default_rng(17)
    kid = "skip_layer_norm.fp16.last_axis" if skip else "layer_norm.fp16.last_axis"
    pack = filtered_pack(tmp_path / "pack", only_variant(kid, variant))
    opts = engine.CompileOptions(kernel_artifact_dir=pack, tuning_mode="disabled")
    for rows, cols in ((512, 768), (17, 100), (4, 5000), (64, 1024), (33, 128), (9, 256), (3, 4096), (5, 40)):
        g, feeds = layer_norm_graph(rng, rows, cols, skip)
        out, eng, _ = run_graph(g, feeds, opts)
        ops = eng.ops()
        assert [op.op_type for op in ops] == (["SkipLayerNormalization"] if skip else ["LayerNormalization"])
        assert ops[0].candidates[ops[0].selected_candidate].endswith(f"{kid}:{variant}")
        err = np.abs(out["y"].astype(np.float64) - oracle.evaluate(g, feeds)["y"])
        assert err.max() <= 1e-2, f"{kid}:{variant} {rows}x{cols}: {err.max():.3e}"


@pytest.mark.parametrize("skip", [False, True])
def test_layer_norm_long_rows_with_a_large_mean(skip):
    """Rows past every register limit (the one-pass merged statistics) with a
    mean far from zero, where a sum-of-squares variance would lose digits."""
    rng = np.random.default_rng(19)
    for rows, cols in ((3, 12288), (5, 4104)):
        g, feeds = layer_norm_graph(rng, rows, cols, skip)
        feeds["x"] = (feeds["x"].astype(np.float32) * 3 + 40).astype(np.float16)
        out, _, _ = run_graph(g, feeds)
        err = np.abs(out["y"].astype(np.float64) - oracle.evaluate(g, feeds)["y"])
        assert err.max() <= 1e-2, f"{rows}x{cols} skip={skip}: {err.max():.3e}"


@pytest.mark.parametrize("op", ["Gelu", "Add"])
@pytest.mark.parametrize("count", [(512, 3072), (3, 37)])
def test_fp16_elementwise_kernels(op, count):
    rng = np.random.default_rng(29)
    g = workloads.GraphSpec()
    g.inputs["a"] = (count, "float16", "")
    feeds = {"a": (rng.standard_normal(count) * 2).astype(np.float16)}
    if op == "Gelu":
        g.add("gelu", "Gelu", ["a"], ["y"])
    else:
        g.inputs["b"] = (count, "float16", "")
        feeds["b"] = rng.standard_normal(count).astype(np.float16)
        g.add("add", "Add", ["a", "b"], ["y"])
    g.outputs.append("y")
    out, eng, _ = run_graph(g, feeds)
    assert [o.op_type for o in eng.ops()] == [op]
    want = oracle.evaluate(g, feeds)["y"]
    # One FP16 rounding of an exact (Add) or FP32-accurate (Gelu) value.
    err = np.abs(out["y"].astype(np.float64) - want)
    assert np.all(err <= 2.0 ** -10 * np.abs(want) + 1e-6), err.max()
