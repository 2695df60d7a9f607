"""The reference's CPU path: the same graph in PyTorch-CPU FP32.

TEST INFRASTRUCTURE / CPU BASELINE ONLY (bench.py's cpu_baseline leg).
The reference has no native CPU kernels (its ``cpu_reference`` backend
returns Unsupported, src/backend/backend.cpp:22-35); its CPU numbers come
from the compare scripts that rebuild the graph with torch
(benchmarks/resnet50_compare.py:36-141, benchmarks/transformer_ffn_compare.py:52-60).
This module restates that: it walks a graph description node by node with
torch.nn.functional in FP32 under inference mode.
"""

from __future__ import annotations

from typing import Any, Mapping

import numpy as np
import torch
import torch.nn.functional as F


def _pads(attrs: Mapping[str, Any]) -> list[int]:
    return list(attrs.get("pads", [0, 0, 0, 0]))


def prepare(graph: Any, dtype: torch.dtype = torch.float32) -> dict[str, torch.Tensor]:
    np_dtype = np.float64 if dtype == torch.float64 else np.float32
    return {name: torch.from_numpy(np.ascontiguousarray(arr, dtype=np_dtype))
            for name, (arr, _) in graph.constants.items()}


@torch.inference_mode()
def run(graph: Any, constants: dict[str, torch.Tensor], feeds: Mapping[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    env = dict(constants)
    env.update(feeds)
    for node in graph.nodes:
        a, x = node.attributes, [env[i] for i in node.inputs]
        op = node.op_type
        if op == "Conv":
            top, left, bottom, right = _pads(a)
            inp = x[0]
            if (top, left) != (bottom, right):
                inp = F.pad(inp, (left, right, top, bottom))
                top = left = 0
            y = F.conv2d(inp, x[1], stride=tuple(a.get("strides", [1, 1])), padding=(top, left),
                         dilation=tuple(a.get("dilations", [1, 1])))
        elif op == "BatchNormalization":
            y = F.batch_norm(x[0], x[3], x[4], x[1], x[2], training=False, eps=a.get("epsilon", 1e-5))
        elif op == "Relu":
            y = F.relu(x[0])
        elif op == "Add":
            y = x[0] + x[1]
        elif op == "MaxPool":
            p = _pads(a)
            y = F.max_pool2d(x[0], tuple(a["kernel_shape"]), tuple(a.get("strides", a["kernel_shape"])),
                             padding=(p[0], p[1]), dilation=tuple(a.get("dilations", [1, 1])))
        elif op == "GlobalAveragePool":
            y = x[0].mean(dim=(2, 3), keepdim=True)
        elif op == "Flatten":
            y = torch.flatten(x[0], 1)
        elif op == "Gemm":
            y = x[0] @ x[1] + (x[2] if len(x) > 2 else 0)
        elif op == "Gelu":
            y = F.gelu(x[0])
        elif op == "LayerNormalization":
            y = F.layer_norm(x[0], (x[0].shape[-1],), x[1], x[2], eps=a.get("epsilon", 1e-5))
        else:
            raise NotImplementedError(op)
        env[node.outputs[0]] = y
    return {name: env[name] for name in graph.outputs}
