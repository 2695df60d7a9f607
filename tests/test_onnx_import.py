"""Native ONNX import (include/cutriton/ir/onnx_import.h).

The files come from two writers that share no code with the reader:
  * tests/golden/onnx/*.onnx, written by the ONNX serializer compiled into
    libtorch (tests/golden/make_onnx_fixtures.py), with torch float64
    outputs beside them;
  * tests/onnx_proto.py, google.protobuf over a schema declared with the
    field numbers of onnx/onnx.proto, for graphs built here.
A hand-assembled wire-format model pins that schema's encoding. The CPU tests
plan for gfx950 without a device; the GPU tests run the imported models
against torch's float64 results and against directly built engines.
"""

from __future__ import annotations

import numpy as np
import pytest

from cutriton_amd import engine, workloads
from tests.conftest import ROOT
from tests.onnx_proto import ONNX, attribute, tensor, to_onnx, value_info

GOLDEN = ROOT / "tests" / "golden" / "onnx"
CNN_FIXTURES = ("tiny_resnet_folded", "tiny_resnet_batchnorm")


@pytest.fixture
def gfx950(monkeypatch):
    monkeypatch.setenv("CUTRITON_TARGET_ARCH", "gfx950")


def plan(model) -> list[tuple[str, str]]:
    ops = engine.build_engine(model, engine.CompileOptions()).ops()
    return [(op.op_type, op.candidates[op.selected_candidate].split(":", 1)[1]) for op in ops]


# ---- wire format ---------------------------------------------------------------

def varint(v: int) -> bytes:
    out = bytearray()
    while True:
        byte, v = v & 0x7F, v >> 7
        out.append(byte | (0x80 if v else 0))
        if not v:
            return bytes(out)


def field(number: int, payload: bytes | int) -> bytes:
    if isinstance(payload, int):
        return varint(number << 3) + varint(payload)
    return varint(number << 3 | 2) + varint(len(payload)) + payload


def relu_model_bytes() -> bytes:
    """ModelProto{ir_version 8, graph{node Relu(x) -> y, input x: FLOAT[2,3],
    output y}, opset_import{version 17}} assembled field by field."""
    dims = field(1, field(1, 2)) + field(1, field(1, 3))
    x_type = field(1, field(1, 1) + field(2, dims))
    graph = (field(1, field(1, b"x") + field(2, b"y") + field(4, b"Relu"))
             + field(11, field(1, b"x") + field(2, x_type))
             + field(12, field(1, b"y")))
    return field(1, 8) + field(7, graph) + field(8, field(2, 17))


def test_hand_assembled_model_matches_the_schema_encoder(gfx950):
    m = ONNX["ModelProto"](ir_version=8)
    n = m.graph.node.add(op_type="Relu")
    n.input.append("x")
    n.output.append("y")
    m.graph.input.append(value_info(ONNX, "x", (2, 3), "float32"))
    m.graph.output.append(value_info(ONNX, "y"))
    m.opset_import.add(version=17)
    assert m.SerializeToString() == relu_model_bytes()
    model = engine.Model.from_onnx(relu_model_bytes())
    assert model.op_types() == ["Relu"]
    assert plan(model) == [("Relu", "relu.fp32.contiguous:w4")]


# ---- files written by libtorch --------------------------------------------------

# Nodes keep the exporter's order where dependencies allow; the shortcut
# convolution comes last in the block, so it takes the residual join.
FUSED_CNN_PLAN = ["FusedConvBatchNormRelu", "MaxPool", "FusedConvBatchNormRelu", "FusedConvBatchNormRelu",
                  "FusedConvBatchNorm", "FusedConvBatchNormAddRelu", "GlobalAveragePool", "Flatten", "Gemm"]


@pytest.mark.parametrize("name", CNN_FIXTURES)
def test_torch_exported_cnn_plans_to_fused_kernels(gfx950, name):
    """Both exports (BatchNorm folded into a Conv bias, or kept) give the
    fused plan; Linear is Gemm with transB = 1."""
    model = engine.Model.from_onnx(GOLDEN / f"{name}.onnx", {"batch": 2})
    ops = plan(model)
    assert [op for op, _ in ops] == FUSED_CNN_PLAN
    assert ops[-1][1].startswith("gemm_bias.fp32.mfma_tb:")


def test_torch_exported_ffn_plans_to_fused_kernels(gfx950):
    ops = plan(engine.Model.from_onnx((GOLDEN / "tiny_ffn_fp16.onnx").read_bytes()))
    assert [op for op, _ in ops] == ["GemmGelu", "Gemm", "SkipLayerNormalization"]
    assert ops[0][1].startswith("gemm_gelu_bias.fp16.mfma_tb:") and ops[1][1].startswith("gemm_bias.fp16.mfma_tb:")


def test_symbolic_dimensions_take_the_given_sizes(gfx950):
    path = GOLDEN / "tiny_resnet_folded.onnx"
    with pytest.raises(engine.CutritonError) as err:
        engine.Model.from_onnx(path)
    assert err.value.kind == "InvalidArgument" and "'batch'" in str(err.value)
    eng = engine.build_engine(engine.Model.from_onnx(path, {"batch": 5}), engine.CompileOptions())
    assert eng.value_desc("output") == ([5, 10], "float32")


# ---- graphs built here -------------------------------------------------------------

@pytest.mark.parametrize("raw,packed", [(True, False), (False, False), (False, True)])
def test_resnet50_plans_like_the_direct_build(gfx950, raw, packed):
    """Initializers as raw_data or typed fields, repeated fields packed or not."""
    spec = workloads.resnet50(1)
    direct = engine.build_engine(workloads.to_model(spec), engine.CompileOptions()).ops()
    imported = engine.build_engine(engine.Model.from_onnx(to_onnx(spec, raw=raw, packed=packed)),
                                   engine.CompileOptions()).ops()
    assert [(o.op_type, o.candidates) for o in imported] == [(o.op_type, o.candidates) for o in direct]


def test_file_path_and_missing_file(tmp_path, gfx950):
    path = tmp_path / "relu.onnx"
    path.write_bytes(relu_model_bytes())
    assert engine.Model.from_onnx(path).op_types() == ["Relu"]
    with pytest.raises(engine.CutritonError) as err:
        engine.Model.from_onnx(tmp_path / "absent.onnx")
    assert err.value.kind == "NotFound"


def _refused(mutate) -> str:
    spec, _ = workloads.conv_bn_relu(channels=8, size=8)
    m = ONNX["ModelProto"]()
    m.ParseFromString(to_onnx(spec))
    mutate(m)
    with pytest.raises(engine.CutritonError) as err:
        engine.Model.from_onnx(m.SerializeToString())
    return err.value.kind


def _node(m, op_type):
    return next(n for n in m.graph.node if n.op_type == op_type)


@pytest.mark.parametrize("what,mutate", [
    ("grouped conv", lambda m: _node(m, "Conv").attribute.append(attribute(ONNX, "group", 2))),
    ("auto_pad", lambda m: _node(m, "Conv").attribute.append(attribute(ONNX, "auto_pad", "SAME_UPPER"))),
    ("other domain", lambda m: setattr(_node(m, "Relu"), "domain", "com.example")),
    ("graph attribute", lambda m: _node(m, "Relu").attribute.add(name="body", type=5)),
    ("external data", lambda m: setattr(m.graph.initializer[0], "data_location", 1)),
    ("sparse initializer", lambda m: m.graph.sparse_initializer.add(name="s", data_type=1)),
    ("double tensor", lambda m: m.graph.initializer.append(tensor(ONNX, "d", np.zeros(2)))),
])
def test_unsupported_constructs_are_refused(what, mutate):
    assert _refused(mutate) == "Unsupported", what


def test_values_the_engine_would_drop_are_refused():
    g = workloads.GraphSpec()
    g.inputs["x"] = ((2, 8, 8, 8), "float32", "NCHW")
    g.add("pool", "MaxPool", ["x"], ["y"], kernel_shape=[3, 3], strides=[2, 2], ceil_mode=1)
    g.outputs.append("y")
    with pytest.raises(engine.CutritonError) as err:
        engine.Model.from_onnx(to_onnx(g))
    assert err.value.kind == "Unsupported"
    f = workloads.GraphSpec()
    f.inputs["a"] = ((4, 8), "float32", "")
    f.constant("b", np.ones((8, 3), np.float32))
    f.add("gemm", "Gemm", ["a", "b"], ["y"], alpha=2.0)
    f.outputs.append("y")
    h = workloads.GraphSpec()
    h.inputs["a"] = ((4, 8), "float16", "")
    h.add("gelu", "Gelu", ["a"], ["y"], approximate="tanh")
    h.outputs.append("y")
    for spec in (f, h):
        with pytest.raises(engine.CutritonError) as err:
            engine.Model.from_onnx(to_onnx(spec, opset=20))
        assert err.value.kind == "Unsupported"


def test_malformed_bytes_are_errors_not_crashes():
    """Every proper prefix of a model and 400 seeded single-byte corruptions:
    each either imports or returns an error."""
    spec, _ = workloads.conv_bn_relu(channels=8, size=8)
    data = to_onnx(spec)
    for cut in range(0, len(data) - 1, 7):
        try:
            engine.Model.from_onnx(data[:cut])
        except engine.CutritonError as err:
            assert err.kind in ("InvalidArgument", "Unsupported", "NotFound", "AlreadyExists", "ShapeError")
    rng = np.random.default_rng(9)
    for _ in range(400):
        corrupt = bytearray(data)
        corrupt[rng.integers(len(corrupt))] = int(rng.integers(256))
        try:
            engine.Model.from_onnx(bytes(corrupt))
        except engine.CutritonError:
            pass
    # dims that claim more elements than the data holds
    m = ONNX["ModelProto"]()
    m.ParseFromString(data)
    m.graph.initializer[0].dims[0] = 1 << 40
    with pytest.raises(engine.CutritonError) as err:
        engine.Model.from_onnx(m.SerializeToString())
    assert err.value.kind == "InvalidArgument"


# ---- GPU: imported models against torch float64 and the direct build ------------------

@pytest.mark.gpu
@pytest.mark.parametrize("name", CNN_FIXTURES)
def test_torch_exported_cnn_matches_torch_float64(name):
    from tests.helpers import assert_close_fp32, run_model

    golden = np.load(GOLDEN / f"{name}.npz")
    model = engine.Model.from_onnx(GOLDEN / f"{name}.onnx", {"batch": 2})
    out, _, _ = run_model(model, {"input": golden["input"]}, ["output"], {"input": "NCHW"})
    assert_close_fp32(out["output"], golden["output"], what=name)


@pytest.mark.gpu
def test_torch_exported_ffn_matches_torch_float64():
    from tests.helpers import run_model

    golden = np.load(GOLDEN / "tiny_ffn_fp16.npz")
    model = engine.Model.from_onnx(GOLDEN / "tiny_ffn_fp16.onnx")
    out, _, _ = run_model(model, {"x": golden["input"]}, ["y"], {"x": ""})
    err = np.abs(out["y"].astype(np.float64) - golden["output"]).max()
    assert err <= 1e-2, err


@pytest.mark.gpu
@pytest.mark.parametrize("raw,packed", [(True, False), (False, True)])
def test_imported_resnet50_matches_the_direct_build(raw, packed):
    """Same kernels, same weights: the outputs agree to FP32 rounding (the
    ONNX BatchNorm epsilon is the float32 nearest 1e-5)."""
    from oracle import oracle
    from tests.helpers import run_graph, run_model
    from tests.test_gpu_models import check_logits

    spec = workloads.resnet50(1)
    x = workloads.resnet50_input(1)
    direct, _, _ = run_graph(spec, {"input": x})
    out, _, _ = run_model(engine.Model.from_onnx(to_onnx(spec, raw=raw, packed=packed)), {"input": x},
                          ["output"], {"input": "NCHW"})
    got = out["output"].astype(np.float64)
    want = direct["output"].astype(np.float64)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    check_logits(got, oracle.evaluate(spec, {"input": x})["output"])
