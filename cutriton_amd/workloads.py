"""Graphs of the measured workloads, with seeded synthetic weights and inputs.

A :class:`GraphSpec` is plain data (nodes, constants, inputs, outputs) that
``to_model`` turns into an engine :class:`~cutriton_amd.engine.Model`. The
graphs are written unfused, the way the reference harness builds them; the
compiler's passes do the fusion.

* ``resnet50`` follows the reference builder
  ``benchmarks/resnet50_native.cpp:61-193``: ResNet-50 v1.5 (stride on the
  3x3 of each bottleneck), a downsample branch when the stride or the channel
  count changes, head GAP -> Flatten -> Gemm(2048 -> 1000) without bias.
* ``ffn`` is the two-GEMM block Y = SkipLayerNorm(Gemm(GemmGelu(X, W1, b1),
  W2, b2) + X), written as Gemm -> Gelu -> Gemm -> Add -> LayerNormalization
  like ``benchmarks/transformer_ffn_native.cpp:112-140``.
* ``conv_bn_relu`` is the single fused node.
* ``stem_kat`` is the known-answer graph of ``tests/cpp/test_cuda.cpp:133-165,
  444-479`` (one-hot 7x7 weights, identity BatchNorm) with its closed form.

Weights use the distributions of the measured configurations (Kaiming-normal
convolutions, BatchNorm gamma~U(0.5,1.5), beta~N(0,0.1), mean~N(0,0.1),
var~U(0.5,1.5), FC W~N(0,0.01); FFN X~N(0,1), W~N(0,0.02), zero biases,
gamma 1, beta 0), drawn from numpy's PCG64 with one seed, in graph order.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import numpy as np

SEED = 20260811


@dataclass
class NodeSpec:
    name: str
    op_type: str
    inputs: list[str]
    outputs: list[str]
    attributes: dict[str, Any] = field(default_factory=dict)


@dataclass
class GraphSpec:
    inputs: dict[str, tuple[tuple[int, ...], str, str]] = field(default_factory=dict)  # name -> (shape, dtype, layout)
    outputs: list[str] = field(default_factory=list)
    constants: dict[str, tuple[np.ndarray, str]] = field(default_factory=dict)  # name -> (array, layout)
    nodes: list[NodeSpec] = field(default_factory=list)

    def add(self, name: str, op_type: str, inputs: list[str], outputs: list[str], **attributes: Any) -> str:
        self.nodes.append(NodeSpec(name, op_type, list(inputs), list(outputs), dict(attributes)))
        return outputs[0]

    def constant(self, name: str, array: np.ndarray, layout: str = "") -> str:
        self.constants[name] = (array, layout)
        return name


def to_model(spec: GraphSpec) -> Any:
    from .engine import Model

    model = Model()
    for name, (shape, dtype, layout) in spec.inputs.items():
        model.add_input(name, shape, dtype, layout)
    for name, (array, layout) in spec.constants.items():
        model.add_constant(name, array, layout)
    for node in spec.nodes:
        model.add_node(node.name, node.op_type, node.inputs, node.outputs, **node.attributes)
    for name in spec.outputs:
        model.add_output(name)
    return model


def _bn_params(rng: np.random.Generator, channels: int) -> tuple[np.ndarray, ...]:
    gamma = rng.uniform(0.5, 1.5, channels).astype(np.float32)
    beta = rng.normal(0.0, 0.1, channels).astype(np.float32)
    mean = rng.normal(0.0, 0.1, channels).astype(np.float32)
    var = rng.uniform(0.5, 1.5, channels).astype(np.float32)
    return gamma, beta, mean, var


def _kaiming(rng: np.random.Generator, shape: tuple[int, ...]) -> np.ndarray:
    fan_in = int(np.prod(shape[1:]))
    return rng.normal(0.0, np.sqrt(2.0 / fan_in), shape).astype(np.float32)


def conv_bn(g: GraphSpec, rng: np.random.Generator, x: str, cin: int, cout: int, kernel: int, stride: int,
            pad: int, relu: bool, prefix: str) -> str:
    w = g.constant(prefix + "_weight", _kaiming(rng, (cout, cin, kernel, kernel)), "OIHW")
    gamma, beta, mean, var = _bn_params(rng, cout)
    names = [g.constant(prefix + s, a) for s, a in
             (("_scale", gamma), ("_bias", beta), ("_mean", mean), ("_variance", var))]
    y = g.add(prefix + "_conv_node", "Conv", [x, w], [prefix + "_conv"], strides=[stride, stride],
              pads=[pad, pad, pad, pad], dilations=[1, 1])
    y = g.add(prefix + "_bn_node", "BatchNormalization", [y, *names], [prefix + "_bn"], epsilon=1e-5)
    if relu:
        y = g.add(prefix + "_relu_node", "Relu", [y], [prefix + "_relu"])
    return y


def resnet50(batch: int, seed: int = SEED) -> GraphSpec:
    rng = np.random.default_rng(seed)
    g = GraphSpec()
    g.inputs["input"] = ((batch, 3, 224, 224), "float32", "NCHW")
    y = conv_bn(g, rng, "input", 3, 64, 7, 2, 3, True, "stem")
    y = g.add("stem_maxpool", "MaxPool", [y], ["stem_pool"], kernel_shape=[3, 3], strides=[2, 2],
              pads=[1, 1, 1, 1], dilations=[1, 1])
    channels = 64
    for stage, (blocks, planes) in enumerate(zip((3, 4, 6, 3), (64, 128, 256, 512))):
        for block in range(blocks):
            stride = 2 if stage != 0 and block == 0 else 1
            prefix = f"layer{stage + 1}_block{block + 1}"
            branch = conv_bn(g, rng, y, channels, planes, 1, 1, 0, True, prefix + "_conv1")
            branch = conv_bn(g, rng, branch, planes, planes, 3, stride, 1, True, prefix + "_conv2")
            branch = conv_bn(g, rng, branch, planes, planes * 4, 1, 1, 0, False, prefix + "_conv3")
            identity = y
            if stride != 1 or channels != planes * 4:
                identity = conv_bn(g, rng, y, channels, planes * 4, 1, stride, 0, False, prefix + "_downsample")
            s = g.add(prefix + "_add", "Add", [branch, identity], [prefix + "_sum"])
            y = g.add(prefix + "_relu", "Relu", [s], [prefix + "_output"])
            channels = planes * 4
    y = g.add("global_average_pool", "GlobalAveragePool", [y], ["gap"])
    y = g.add("flatten", "Flatten", [y], ["flattened"])
    fc = g.constant("fc_weight", rng.normal(0.0, 0.01, (2048, 1000)).astype(np.float32))
    g.add("classifier", "Gemm", [y, fc], ["output"])
    g.outputs.append("output")
    return g


def resnet50_input(batch: int, seed: int = SEED + 1) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal((batch, 3, 224, 224), dtype=np.float32)


def conv_bn_relu(seed: int = SEED, batch: int = 1, channels: int = 64, size: int = 56) -> tuple[GraphSpec, np.ndarray]:
    """One Conv(3x3, s1, p1) -> BatchNormalization -> Relu; fuses to FusedConvBatchNormRelu."""
    rng = np.random.default_rng(seed)
    g = GraphSpec()
    g.inputs["x"] = ((batch, channels, size, size), "float32", "NCHW")
    y = conv_bn(g, rng, "x", channels, channels, 3, 1, 1, True, "node")
    g.outputs.append(y)
    x = rng.standard_normal((batch, channels, size, size), dtype=np.float32)
    return g, x


def ffn(tokens: int, hidden: int, intermediate: int, seed: int = SEED) -> tuple[GraphSpec, np.ndarray]:
    rng = np.random.default_rng(seed)
    g = GraphSpec()
    g.inputs["x"] = ((tokens, hidden), "float16", "")
    x = rng.standard_normal((tokens, hidden)).astype(np.float16)
    w1 = g.constant("w1", rng.normal(0.0, 0.02, (hidden, intermediate)).astype(np.float16))
    b1 = g.constant("b1", np.zeros(intermediate, np.float16))
    w2 = g.constant("w2", rng.normal(0.0, 0.02, (intermediate, hidden)).astype(np.float16))
    b2 = g.constant("b2", np.zeros(hidden, np.float16))
    gamma = g.constant("gamma", np.ones(hidden, np.float16))
    beta = g.constant("beta", np.zeros(hidden, np.float16))
    h = g.add("fc1", "Gemm", ["x", w1, b1], ["fc1_out"])
    h = g.add("act", "Gelu", [h], ["act_out"])
    h = g.add("fc2", "Gemm", [h, w2, b2], ["fc2_out"])
    h = g.add("residual_add", "Add", [h, "x"], ["sum"])
    g.add("norm", "LayerNormalization", [h, gamma, beta], ["y"], axis=-1, epsilon=1e-5)
    g.outputs.append("y")
    return g, x


def ffn_pattern(tokens: int = 17, hidden: int = 128, intermediate: int = 512) -> tuple[GraphSpec, dict[str, np.ndarray]]:
    """FP16 Gemm -> Gelu -> Add(residual) -> LayerNormalization with the
    integer-pattern inputs of the reference's transformer test
    (tests/cpp/test_cuda.cpp:336-358, graph 300-333): x[t*H+i] = ((i%23)-11)/37,
    residual ((i%17)-8)/53, W ((i%19)-9)/181, scale 0.9+0.001*(c%13),
    bias ((c%7)-3)/100, epsilon 1e-5. Returns (graph, feeds)."""
    f16 = np.float16
    x = ((np.arange(tokens * hidden) % 23 - 11) / 37.0).astype(f16).reshape(tokens, hidden)
    residual = ((np.arange(tokens * intermediate) % 17 - 8) / 53.0).astype(f16).reshape(tokens, intermediate)
    w = ((np.arange(hidden * intermediate) % 19 - 9) / 181.0).astype(f16).reshape(hidden, intermediate)
    c = np.arange(intermediate)
    scale = (0.9 + 0.001 * (c % 13)).astype(f16)
    bias = (((c % 7) - 3) / 100.0).astype(f16)
    g = GraphSpec()
    g.inputs["x"] = ((tokens, hidden), "float16", "")
    g.inputs["residual"] = ((tokens, intermediate), "float16", "")
    g.constant("weight", w)
    g.constant("scale", scale)
    g.constant("bias", bias)
    g.add("projection", "Gemm", ["x", "weight"], ["projected"])
    g.add("activation", "Gelu", ["projected"], ["activated"])
    g.add("residual_add", "Add", ["activated", "residual"], ["sum"])
    g.add("output_norm", "LayerNormalization", ["sum", "scale", "bias"], ["output"], axis=-1, epsilon=1e-5)
    g.outputs.append("output")
    return g, {"x": x, "residual": residual}


def stem_kat(batch_shape: tuple[int, ...] = (1, 3, 224, 224)) -> tuple[GraphSpec, np.ndarray, np.ndarray]:
    """Known-answer stem: returns (graph, input, expected logits).

    The 7x7 stride-2 weights are one-hot at the window centre of input
    channel oc % 3 with value 0.05 * (1 + oc % 5); BatchNorm is the identity
    up to var + eps = 1. Conv output (oc, oh, ow) is therefore
    w_oc * x[oc % 3, 2 oh, 2 ow], and the logits follow in closed form.
    """
    g = GraphSpec()
    g.inputs["input"] = (tuple(batch_shape), "float32", "NCHW")
    count = int(np.prod(batch_shape))
    x = ((np.arange(count) % 29) - 14).astype(np.float32).reshape(batch_shape) / np.float32(29.0)
    conv_w = np.zeros((64, 3, 7, 7), np.float32)
    tap = np.float32(0.05) * (1 + np.arange(64) % 5).astype(np.float32)
    conv_w[np.arange(64), np.arange(64) % 3, 3, 3] = tap
    fc_w = (((np.arange(64 * 1000) % 11) - 5).astype(np.float32) / np.float32(101.0)).reshape(64, 1000)
    g.constant("conv_w", conv_w, "OIHW")
    g.constant("bn_scale", np.ones(64, np.float32))
    g.constant("bn_bias", np.zeros(64, np.float32))
    g.constant("bn_mean", np.zeros(64, np.float32))
    g.constant("bn_var", np.full(64, 0.99999, np.float32))
    g.constant("fc_w", fc_w)
    g.add("conv", "Conv", ["input", "conv_w"], ["conv_y"], pads=[3, 3, 3, 3], strides=[2, 2], dilations=[1, 1])
    g.add("bn", "BatchNormalization", ["conv_y", "bn_scale", "bn_bias", "bn_mean", "bn_var"], ["bn_y"],
          epsilon=1e-5)
    g.add("relu", "Relu", ["bn_y"], ["relu_y"])
    g.add("gap", "GlobalAveragePool", ["relu_y"], ["gap_y"])
    g.add("flatten", "Flatten", ["gap_y"], ["flat_y"])
    g.add("gemm", "Gemm", ["flat_y", "fc_w"], ["output"])
    g.outputs.append("output")
    n, _, h, w = batch_shape
    oh, ow = (h + 6 - 7) // 2 + 1, (w + 6 - 7) // 2 + 1
    sampled = x[:, :, 0:2 * oh:2, 0:2 * ow:2].astype(np.float64)  # [n, 3, oh, ow]
    conv = sampled[:, np.arange(64) % 3] * tap.astype(np.float64)[None, :, None, None]
    pooled = np.maximum(conv, 0.0).mean(axis=(2, 3))
    expected = pooled @ fc_w.astype(np.float64)
    return g, x, expected


def value_shapes(spec: GraphSpec) -> dict[str, tuple[int, ...]]:
    """The shape of every value of `spec` (inputs, constants and node
    outputs), by name, for the node types the workloads use."""
    shapes = {name: tuple(shape) for name, (shape, _, _) in spec.inputs.items()}
    shapes.update({name: tuple(arr.shape) for name, (arr, _) in spec.constants.items()})
    for node in spec.nodes:
        a, ins = node.attributes, [shapes[i] for i in node.inputs]
        if node.op_type == "Conv":
            (n, c, h, w), (k, _, r, s) = ins[0], ins[1]
            st, pd, dl = a.get("strides", [1, 1]), a.get("pads", [0, 0, 0, 0]), a.get("dilations", [1, 1])
            p = (h + pd[0] + pd[2] - dl[0] * (r - 1) - 1) // st[0] + 1
            q = (w + pd[1] + pd[3] - dl[1] * (s - 1) - 1) // st[1] + 1
            out = (n, k, p, q)
        elif node.op_type == "MaxPool":
            (n, c, h, w), ker = ins[0], a["kernel_shape"]
            st, pd = a.get("strides", ker), a.get("pads", [0, 0, 0, 0])
            out = (n, c, (h + pd[0] + pd[2] - ker[0]) // st[0] + 1, (w + pd[1] + pd[3] - ker[1]) // st[1] + 1)
        elif node.op_type == "GlobalAveragePool":
            out = ins[0][:2] + (1, 1)
        elif node.op_type == "Flatten":
            out = (ins[0][0], int(np.prod(ins[0][1:])))
        elif node.op_type == "Gemm":
            out = (ins[0][0], ins[1][1])
        else:
            out = ins[0]
        shapes[node.outputs[0]] = out
    return shapes


def node_flops(spec: GraphSpec) -> dict[str, int]:
    """Algorithmic FLOPs (2 x multiply-accumulates) of every Conv and Gemm node,
    by name; BatchNorm, activations, pooling and adds count zero."""
    shapes = value_shapes(spec)
    flops: dict[str, int] = {}
    for node in spec.nodes:
        if node.op_type == "Conv":
            (_, c, _, _), (_, _, r, s) = shapes[node.inputs[0]], shapes[node.inputs[1]]
            n, k, p, q = shapes[node.outputs[0]]
            flops[node.name] = 2 * n * k * c * r * s * p * q
        elif node.op_type == "Gemm":
            (m, k), (_, n) = shapes[node.inputs[0]], shapes[node.inputs[1]]
            flops[node.name] = 2 * m * n * k
    return flops
