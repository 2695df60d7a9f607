"""Engine library on the CPU: exports, the C++ API, and planning for gfx950
without a device (CUTRITON_TARGET_ARCH=gfx950 stands in for the device query).

Plan expectations follow the reference's fusion and candidate tests
(tests/cpp/test_core.cpp:215-233, 333-353; tests/cpp/test_cuda.cpp:395-406):
ResNet-50 lowers to 57 ops (53 fused convolutions), the FFN block to
GemmGelu + Gemm + SkipLayerNormalization, and every fused op also carries
its FusionRegistry decomposition as a candidate.
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
from collections import Counter
from pathlib import Path

import pytest

from cutriton_amd import engine, native, workloads
from cutriton_amd.kernel_specs.transformer import GEMM_NT_SPLIT_TILES, GEMM_NT_TILES

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not native.LIBRARY_PATH.exists():
        native.build_engine_library()
    return ctypes.CDLL(str(native.LIBRARY_PATH))


@pytest.fixture
def gfx950(monkeypatch):
    monkeypatch.setenv("CUTRITON_TARGET_ARCH", "gfx950")
    if not (native.PACK_DIR / "pack.json").exists():
        native.build_kernel_pack()


def declared_functions(header: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b((?:ct|cth)_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", ["cutriton_engine.h", "cutriton_hip_runtime.h"])
def test_library_exports_every_declared_function(lib, header):
    names = declared_functions(ROOT / "include" / header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_channel(lib):
    lib.ct_version.restype = ctypes.c_char_p
    assert b"cutriton-amd" in lib.ct_version()
    model = engine.Model()
    with pytest.raises(engine.CutritonError) as err:
        model.add_output("never_defined_value_that_has_no_producer")
        engine.build_engine(model, engine.CompileOptions(target="no_such_backend"))
    assert err.value.kind in ("NotFound", "InvalidArgument", "Unsupported")


def test_cpp_api_suite(lib, tmp_path):
    """tests/cpp/test_api.cc against the built library (mock host backend)."""
    exe = tmp_path / "test_api"
    cmd = ["g++", "-std=c++17", "-O1", "-I", str(ROOT / "include"), str(ROOT / "tests/cpp/test_api.cc"),
           "-L", str(native.LIBRARY_PATH.parent), "-lcutriton_gfx950", f"-Wl,-rpath,{native.LIBRARY_PATH.parent}",
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    env = {k: v for k, v in os.environ.items() if k != "CUTRITON_TARGET_ARCH"}
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.count("ok ") == 10, run.stdout


def test_resnet50_plan(gfx950):
    eng = engine.build_engine(workloads.to_model(workloads.resnet50(1)), engine.CompileOptions())
    ops = eng.ops()
    counts = Counter(op.op_type for op in ops)
    assert len(ops) == 57
    assert counts == {"FusedConvBatchNormRelu": 33, "FusedConvBatchNormAddRelu": 16, "FusedConvBatchNorm": 4,
                      "MaxPool": 1, "GlobalAveragePool": 1, "Flatten": 1, "Gemm": 1}
    stem = ops[0]
    assert stem.op_type == "FusedConvBatchNormRelu"
    kernels = [c for c in stem.candidates if not c.startswith("unfused:")]
    assert len(kernels) >= 2 and any(".mfma:" in c for c in kernels)
    assert sum(c.startswith("unfused:") for c in stem.candidates) == 1
    add_relu = next(op for op in ops if op.op_type == "FusedConvBatchNormAddRelu")
    assert any(c.startswith("unfused:") for c in add_relu.candidates)
    flatten = next(op for op in ops if op.op_type == "Flatten")
    assert len(flatten.candidates) == 1
    assert eng.value_desc("output") == ([1, 1000], "float32")
    assert eng.workspace_bytes() > 0 and eng.workspace_bytes() % 256 == 0


def test_residual_epilogue_fusion_can_be_disabled(gfx950):
    opts = engine.CompileOptions(enable_residual_epilogue_fusion=False)
    ops = engine.build_engine(workloads.to_model(workloads.resnet50(1)), opts).ops()
    counts = Counter(op.op_type for op in ops)
    assert counts["FusedConvBatchNormAddRelu"] == 0
    assert counts["AddRelu"] == 16 and counts["FusedConvBatchNorm"] == 20


def test_ffn_plan_and_candidates(gfx950):
    graph, _ = workloads.ffn(512, 768, 3072)
    ops = engine.build_engine(workloads.to_model(graph), engine.CompileOptions()).ops()
    assert [op.op_type for op in ops] == ["GemmGelu", "Gemm", "SkipLayerNormalization"]
    for op in ops:
        assert sum(c.startswith("unfused:") for c in op.candidates) == (0 if op.op_type == "Gemm" else 1)
    # every weight-transposed tile (whole depth and split-K), four B-as-is
    # tiles, then Gemm,Gelu
    assert len(ops[0].candidates) == len(GEMM_NT_TILES) + len(GEMM_NT_SPLIT_TILES) + 5
    assert ops[0].candidates[ops[0].selected_candidate].endswith("gemm_gelu_bias.fp16.mfma:m128n128w4")
    assert ops[0].candidates[-1] == "unfused:gemm_gelu"


def test_ffn_pattern_plan(gfx950):
    graph, _ = workloads.ffn_pattern()
    ops = engine.build_engine(workloads.to_model(graph), engine.CompileOptions()).ops()
    assert [op.op_type for op in ops] == ["GemmGelu", "SkipLayerNormalization"]


def softmax_model(axis: int):
    g = workloads.GraphSpec()
    g.inputs["x"] = ((2048, 512), "float16", "")
    g.add("softmax", "Softmax", ["x"], ["y"], axis=axis)
    g.outputs.append("y")
    return workloads.to_model(g)


def test_softmax_plan(gfx950):
    from cutriton_amd.kernel_specs.transformer import SOFTMAX_DEFAULT, SOFTMAX_VARIANTS

    ops = engine.build_engine(softmax_model(-1), engine.CompileOptions()).ops()
    assert [op.op_type for op in ops] == ["Softmax"]
    assert [c.rsplit(":", 1)[1] for c in ops[0].candidates] == [name for name, _ in SOFTMAX_VARIANTS]
    assert ops[0].candidates[ops[0].selected_candidate].endswith("softmax.fp16.last_axis:" + SOFTMAX_DEFAULT)
    assert len(engine.build_engine(softmax_model(1), engine.CompileOptions()).ops()) == 1


def test_softmax_over_another_axis_is_refused(gfx950):
    # The reference's kernel would compute the last-axis softmax here.
    with pytest.raises(engine.CutritonError) as err:
        engine.build_engine(softmax_model(0), engine.CompileOptions())
    assert err.value.kind == "Unsupported"


def attention_model(shapes, **attrs):
    g = workloads.GraphSpec()
    for name, shape in zip(("q", "k", "v", "mask"), shapes):
        g.inputs[name] = (shape, "float16", "")
    g.add("attention", "Attention", list(g.inputs), ["o"], **attrs)
    g.outputs.append("o")
    return workloads.to_model(g)


def test_attention_plan(gfx950):
    eng = engine.build_engine(attention_model([(2, 4, 100, 64), (2, 4, 70, 64), (2, 4, 70, 64)]),
                              engine.CompileOptions())
    assert eng.value_desc("o") == ([2, 4, 100, 64], "float16") and eng.value_layout("o") == ""
    ops = eng.ops()
    assert [op.op_type for op in ops] == ["Attention"]
    assert [c.split(":")[1] for c in ops[0].candidates] == ["attention.fp16.d064", "attention.fp16.d128"]
    assert ops[0].selected_candidate == 0
    ops = engine.build_engine(attention_model([(1, 2, 8, 128)] * 3, is_causal=1), engine.CompileOptions()).ops()
    assert [c.split(":")[1] for c in ops[0].candidates] == ["attention.fp16.d128"]


@pytest.mark.parametrize("shapes,attrs,kind", [
    ([(2, 8, 64)] * 3, {}, "ShapeError"),                                          # 3-D inputs
    ([(1, 2, 8, 64), (1, 2, 8, 64), (1, 2, 8, 32)], {}, "Unsupported"),            # value head dimension
    ([(1, 2, 8, 64), (1, 3, 8, 64), (1, 2, 8, 64)], {}, "ShapeError"),             # heads disagree
    ([(1, 2, 8, 64)] * 3, {"softcap": 30.0}, "Unsupported"),
    ([(1, 2, 8, 256)] * 3, {}, "Unsupported"),                                     # no kernel for D = 256
])
def test_attention_refusals(gfx950, shapes, attrs, kind):
    with pytest.raises(engine.CutritonError) as err:
        engine.build_engine(attention_model(shapes, **attrs), engine.CompileOptions())
    assert err.value.kind == kind


def test_shape_profiles_resolve_on_cpu(gfx950):
    graph = workloads.resnet50(1)
    opts = engine.CompileOptions(shape_profiles={"batch": {"input": ((1, 3, 224, 224), (32, 3, 224, 224),
                                                                      (64, 3, 224, 224))}})
    eng = engine.build_engine(workloads.to_model(graph), opts)
    ctx = eng.create_execution_context()
    ctx.select_shape_profile("batch")
    ctx.set_input_shape("input", (48, 3, 224, 224))
    ctx.resolve_shapes()
    assert ctx.resolved_desc("output")[0] == [48, 1000]
    with pytest.raises(engine.CutritonError) as err:
        ctx.set_input_shape("input", (65, 3, 224, 224))
    assert err.value.kind == "ShapeError"


def test_missing_pack_is_an_error(gfx950, tmp_path):
    opts = engine.CompileOptions(kernel_artifact_dir=str(tmp_path / "absent"))
    with pytest.raises(engine.CutritonError):
        engine.build_engine(workloads.to_model(workloads.conv_bn_relu()[0]), opts)


def test_wrong_architecture_pack_is_unsupported(monkeypatch):
    monkeypatch.setenv("CUTRITON_TARGET_ARCH", "gfx942")
    with pytest.raises(engine.CutritonError) as err:
        engine.build_engine(workloads.to_model(workloads.conv_bn_relu()[0]), engine.CompileOptions())
    assert err.value.kind == "Unsupported"


def test_buffer_resource_kernels_refuse_two_gibibyte_tensors(gfx950):
    """Kernels that address tensors through 32-bit buffer resources declare
    tensor_bytes_le 2^31 - 1. A ResNet-50 profile whose max batch (1024)
    makes the stem's output 3.3 GB leaves the stem convolution without a
    kernel at that corner: the build fails and names the tensor, instead of
    planning a run whose padded reads would wrap (the reference's i32
    narrowing checks play this part, src/backend/cuda_launcher.cpp:140-192)."""
    graph = workloads.resnet50(1)
    opts = engine.CompileOptions(shape_profiles={"batch": {"input": ((1, 3, 224, 224), (32, 3, 224, 224),
                                                                     (1024, 3, 224, 224))}})
    with pytest.raises(engine.CutritonError) as refused:
        engine.build_engine(workloads.to_model(graph), opts)
    assert refused.value.kind == "Unsupported", refused.value
    assert "2147483647" in str(refused.value) and "stem" in str(refused.value)
    # The same profile up to batch 64 plans (every tensor stays below 2 GiB).
    ok = engine.CompileOptions(shape_profiles={"batch": {"input": ((1, 3, 224, 224), (32, 3, 224, 224),
                                                                   (64, 3, 224, 224))}})
    assert len(engine.build_engine(workloads.to_model(graph), ok).ops()) == 57
    # A static graph of batch 1024 is refused at lowering already.
    with pytest.raises(engine.CutritonError) as static:
        engine.build_engine(workloads.to_model(workloads.resnet50(1024)), engine.CompileOptions())
    assert static.value.kind == "Unsupported"


def test_tensor_bytes_constraint_is_declared_by_every_buffer_resource_kernel():
    """Every pack entry whose source builds 32-bit buffer resources carries
    the byte limit."""
    import json

    from cutriton_amd.kernel_sdk.builder import KERNEL_SOURCE_DIR

    manifest = json.loads((native.PACK_DIR / "pack.json").read_text())
    uses_resources = {p.stem for p in KERNEL_SOURCE_DIR.glob("*.hip") if "make_buffer_rsrc" in p.read_text()}
    assert uses_resources >= {"conv_fp32", "gemm_fp16_nt", "attention_fp16"}
    for entry in manifest["kernels"]:
        if Path(entry["binary"]).stem in uses_resources:
            limits = [c for c in entry["constraints"] if c["kind"] == "tensor_bytes_le"]
            assert limits == [{"kind": "tensor_bytes_le", "value": 2**31 - 1}], entry["kernel_id"]
