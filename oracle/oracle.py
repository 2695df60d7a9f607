"""FP64 CPU oracle: the reference's op semantics, evaluated in double.

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and
bench.py's CPU-baseline leg as the checker; never by the product. The
arithmetic lives in oracle.c (one function per reference kernel, each citing
the reference file:line it restates); this module loads it, wraps each
function for numpy arrays, and evaluates whole graphs node by node.

``evaluate(graph, feeds)`` walks a graph description (any object with
``nodes`` (name, op_type, inputs, outputs, attributes), ``constants``
(name -> (array, layout)) and ``outputs``) in list order and returns every
value as float64. Attribute defaults and shape rules are the reference's
(src/ir/pass.cpp:45-238): strides default to 1 for Conv and to the kernel
for MaxPool, pads are [top, left, bottom, right], Flatten splits at axis 1.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Any, Mapping

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = ORACLE_DIR / "liboracle.so"

_LIB: ctypes.CDLL | None = None


def build() -> Path:
    """gcc -O2 -fopenmp of oracle.c into liboracle.so (beside this file)."""
    staging = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-Wall", "-Wextra", str(ORACLE_DIR / "oracle.c"),
           "-o", str(staging), "-lm"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{result.stderr}")
    staging.replace(LIBRARY_PATH)
    return LIBRARY_PATH


def _lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIBRARY_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY_PATH))
        D, I, L = ctypes.POINTER(ctypes.c_double), ctypes.c_int, ctypes.c_long
        lib.ct_oracle_conv2d.argtypes = [D, I, I, I, I, D, I, I, I, I, I, I, I, I, I, I, I, D]
        lib.ct_oracle_batch_norm.argtypes = [D, I, I, L, D, D, D, D, ctypes.c_double, D]
        lib.ct_oracle_max_pool.argtypes = [D, I, I, I, I, I, I, I, I, I, I, I, I, I, I, D]
        lib.ct_oracle_global_avg_pool.argtypes = [D, L, L, D]
        lib.ct_oracle_gemm.argtypes = [D, D, D, I, I, I, D]
        lib.ct_oracle_gelu.argtypes = [D, L, D]
        lib.ct_oracle_layer_norm.argtypes = [D, D, L, L, D, D, ctypes.c_double, D]
        lib.ct_oracle_softmax.argtypes = [D, L, L, D]
        lib.ct_oracle_attention.argtypes = [D, D, D, L, L, L, L, ctypes.c_double, ctypes.c_int, D]
        for fn in ("ct_oracle_conv2d", "ct_oracle_batch_norm", "ct_oracle_max_pool", "ct_oracle_global_avg_pool",
                   "ct_oracle_gemm", "ct_oracle_gelu", "ct_oracle_layer_norm", "ct_oracle_softmax",
                   "ct_oracle_attention"):
            getattr(lib, fn).restype = None
        _LIB = lib
    return _LIB


def _d(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a: np.ndarray | None) -> Any:
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def conv2d(x: np.ndarray, w: np.ndarray, strides=(1, 1), pads=(0, 0, 0, 0), dilations=(1, 1)) -> np.ndarray:
    x, w = _d(x), _d(w)
    n, c, h, wd = x.shape
    k, c2, r, s = w.shape
    assert c == c2, "channel mismatch"
    out_h = (h + pads[0] + pads[2] - dilations[0] * (r - 1) - 1) // strides[0] + 1
    out_w = (wd + pads[1] + pads[3] - dilations[1] * (s - 1) - 1) // strides[1] + 1
    out = np.empty((n, k, out_h, out_w))
    _lib().ct_oracle_conv2d(_p(x), n, c, h, wd, _p(w), k, r, s, strides[0], strides[1], pads[0], pads[1],
                            dilations[0], dilations[1], out_h, out_w, _p(out))
    return out


def batch_norm(x: np.ndarray, scale, bias, mean, var, eps: float) -> np.ndarray:
    x = _d(x)
    n, c = x.shape[:2]
    spatial = int(np.prod(x.shape[2:])) if x.ndim > 2 else 1
    out = np.empty_like(x)
    args = [_d(v) for v in (scale, bias, mean, var)]
    _lib().ct_oracle_batch_norm(_p(x), n, c, spatial, *map(_p, args), eps, _p(out))
    return out


def max_pool(x: np.ndarray, kernel, strides=None, pads=(0, 0, 0, 0), dilations=(1, 1)) -> np.ndarray:
    x = _d(x)
    strides = strides or kernel
    n, c, h, w = x.shape
    out_h = (h + pads[0] + pads[2] - (dilations[0] * (kernel[0] - 1) + 1)) // strides[0] + 1
    out_w = (w + pads[1] + pads[3] - (dilations[1] * (kernel[1] - 1) + 1)) // strides[1] + 1
    out = np.empty((n, c, out_h, out_w))
    _lib().ct_oracle_max_pool(_p(x), n, c, h, w, kernel[0], kernel[1], strides[0], strides[1], pads[0], pads[1],
                              dilations[0], dilations[1], out_h, out_w, _p(out))
    return out


def global_average_pool(x: np.ndarray) -> np.ndarray:
    x = _d(x)
    n, c = x.shape[:2]
    spatial = int(np.prod(x.shape[2:]))
    out = np.empty((n, c) + (1,) * (x.ndim - 2))
    _lib().ct_oracle_global_avg_pool(_p(x), n * c, spatial, _p(out))
    return out


def gemm(a: np.ndarray, b: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    a, b = _d(a), _d(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2, "inner dimensions differ"
    if bias is not None:
        bias = _d(bias)
        if bias.shape != (n,):
            # [M, N] bias: add after the product.
            return gemm(a, b) + bias
    out = np.empty((m, n))
    _lib().ct_oracle_gemm(_p(a), _p(b), _p(bias), m, n, k, _p(out))
    return out


def gelu(x: np.ndarray) -> np.ndarray:
    x = _d(x)
    out = np.empty_like(x)
    _lib().ct_oracle_gelu(_p(x), x.size, _p(out))
    return out


def layer_norm(x: np.ndarray, gamma, beta, eps: float, residual: np.ndarray | None = None) -> np.ndarray:
    x = _d(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty_like(x)
    res = None if residual is None else _d(residual)
    _lib().ct_oracle_layer_norm(_p(x), _p(res), rows, cols, _p(_d(gamma)), _p(_d(beta)), eps, _p(out))
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    """Softmax over the last axis."""
    x = _d(x)
    cols = x.shape[-1]
    out = np.empty_like(x)
    _lib().ct_oracle_softmax(_p(x), x.size // cols if cols else 0, cols, _p(out))
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
              causal: bool = False) -> np.ndarray:
    """Attention over [..., S, D] inputs; scale defaults to 1 / sqrt(D)."""
    q, k, v = _d(q), _d(k), _d(v)
    s_q, d = q.shape[-2:]
    s_k = k.shape[-2]
    heads = q.size // (s_q * d) if s_q * d else 0
    out = np.empty(q.shape[:-1] + (v.shape[-1],))
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    _lib().ct_oracle_attention(_p(q), _p(k), _p(v), heads, s_q, s_k, d, scale, int(causal), _p(out))
    return out


def _ints(attrs: Mapping[str, Any], key: str, default):
    value = attrs.get(key, default)
    return list(value) if isinstance(value, (list, tuple)) else value


def evaluate(graph: Any, feeds: Mapping[str, np.ndarray]) -> dict[str, np.ndarray]:
    """Evaluates every node of `graph` in FP64; returns all values."""
    env: dict[str, np.ndarray] = {name: _d(arr) for name, (arr, _) in graph.constants.items()}
    env.update({name: _d(v) for name, v in feeds.items()})
    for node in graph.nodes:
        op, a, ins = node.op_type, node.attributes, [env[i] for i in node.inputs]
        if op in ("Conv", "FusedConvBatchNorm", "FusedConvBatchNormRelu", "FusedConvBatchNormAddRelu"):
            y = conv2d(ins[0], ins[1], _ints(a, "strides", [1, 1]), _ints(a, "pads", [0, 0, 0, 0]),
                       _ints(a, "dilations", [1, 1]))
            if op != "Conv":
                eps = a.get("batchnorm_epsilon", a.get("epsilon", 1e-5))
                y = batch_norm(y, ins[2], ins[3], ins[4], ins[5], eps)
                if op == "FusedConvBatchNormAddRelu":
                    y = y + ins[6]
                if op != "FusedConvBatchNorm":
                    y = np.maximum(y, 0.0)
        elif op == "BatchNormalization":
            y = batch_norm(ins[0], ins[1], ins[2], ins[3], ins[4], a.get("epsilon", 1e-5))
        elif op == "Relu":
            y = np.maximum(ins[0], 0.0)
        elif op == "Add":
            y = ins[0] + ins[1]
        elif op == "AddRelu":
            y = np.maximum(ins[0] + ins[1], 0.0)
        elif op == "MaxPool":
            kernel = _ints(a, "kernel_shape", [1, 1])
            y = max_pool(ins[0], kernel, _ints(a, "strides", kernel), _ints(a, "pads", [0, 0, 0, 0]),
                         _ints(a, "dilations", [1, 1]))
        elif op == "GlobalAveragePool":
            y = global_average_pool(ins[0])
        elif op == "Flatten":
            axis = a.get("axis", 1)
            shape = ins[0].shape
            y = ins[0].reshape(int(np.prod(shape[:axis])), int(np.prod(shape[axis:])))
        elif op in ("Gemm", "GemmGelu"):
            lhs = ins[0].T if a.get("transA", 0) else ins[0]
            rhs = ins[1].T if a.get("transB", 0) else ins[1]
            y = gemm(lhs, rhs, ins[2] if len(ins) > 2 else None)
            if op == "GemmGelu":
                y = gelu(y)
        elif op == "Gelu":
            y = gelu(ins[0])
        elif op == "LayerNormalization":
            y = layer_norm(ins[0], ins[1], ins[2], a.get("epsilon", 1e-5))
        elif op == "SkipLayerNormalization":
            y = layer_norm(ins[0], ins[2], ins[3], a.get("epsilon", 1e-5), residual=ins[1])
        elif op == "Attention":
            y = attention(ins[0], ins[1], ins[2], a.get("scale"), bool(a.get("is_causal", 0)))
        elif op == "Softmax":
            if a.get("axis", -1) not in (-1, ins[0].ndim - 1):
                raise NotImplementedError("the oracle's Softmax is over the last axis")
            y = softmax(ins[0])
        else:
            raise NotImplementedError(f"oracle has no rule for {op}")
        env[node.outputs[0]] = y
    return env
