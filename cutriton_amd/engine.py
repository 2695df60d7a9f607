"""Python host interface over the engine's C ABI (``include/cutriton_engine.h``).

It mirrors the C++ API of the reference engine one call for one call:
``Model`` (graph IR + constants, ``include/cutriton/ir/graph.h:22-161``),
``CompileOptions`` / ``build_engine`` (``include/cutriton/compiler/compiler.h``)
and ``ExecutionContext`` (``include/cutriton/runtime/engine.h:34-93``).
Every call goes through ``libcutriton_gfx950.so``; an error code becomes a
``CutritonError`` carrying ``Status::ToString()``.

Device memory handed to ``bind_input`` / ``bind_output`` is any HIP device
allocation; torch tensors on ``cuda`` are accepted directly.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from .native import PACK_DIR, library

c_int64_p = ctypes.POINTER(ctypes.c_int64)

ERROR_CODES = {
    1: "InvalidArgument", 2: "NotFound", 3: "AlreadyExists", 4: "Unsupported",
    5: "ShapeError", 6: "RuntimeError", 7: "Internal",
}
DTYPE_CODES = {"float32": 1, "float16": 2, "int32": 3, "int64": 4}
DTYPE_NAMES = {v: k for k, v in DTYPE_CODES.items()}
NUMPY_DTYPES = {"float32": np.float32, "float16": np.float16, "int32": np.int32, "int64": np.int64}
TUNING_MODES = {"disabled": 0, "use_cache": 1, "tune_on_miss": 2, "force_retune": 3}


class CutritonError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{ERROR_CODES.get(code, code)}] {message}")
        self.code = code
        self.kind = ERROR_CODES.get(code, str(code))


_CONFIGURED = False


def _lib() -> ctypes.CDLL:
    global _CONFIGURED
    lib = library()
    if _CONFIGURED:
        return lib
    P, I, S, D, C = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_double, ctypes.c_char_p
    sigs: dict[str, tuple[Any, list[Any]]] = {
        "ct_last_error": (C, []),
        "ct_version": (C, []),
        "ct_model_create": (P, []),
        "ct_model_destroy": (None, [P]),
        "ct_model_add_input": (I, [P, C, c_int64_p, I, I, C]),
        "ct_model_add_output": (I, [P, C]),
        "ct_model_add_constant": (I, [P, C, c_int64_p, I, I, C, P, S]),
        "ct_model_add_node": (I, [P, C, C, ctypes.POINTER(C), I, ctypes.POINTER(C), I]),
        "ct_model_set_attr_int": (I, [P, C, C, ctypes.c_int64]),
        "ct_model_set_attr_ints": (I, [P, C, C, c_int64_p, I]),
        "ct_model_set_attr_float": (I, [P, C, C, D]),
        "ct_model_set_attr_floats": (I, [P, C, C, ctypes.POINTER(D), I]),
        "ct_model_set_attr_bool": (I, [P, C, C, I]),
        "ct_model_set_attr_string": (I, [P, C, C, C]),
        "ct_model_run_default_passes": (I, [P, I, I]),
        "ct_model_import_onnx": (I, [C, ctypes.POINTER(C), c_int64_p, I, ctypes.POINTER(P)]),
        "ct_model_import_onnx_buffer": (I, [P, S, ctypes.POINTER(C), c_int64_p, I, ctypes.POINTER(P)]),
        "ct_model_node_count": (I, [P]),
        "ct_model_node_op_type": (I, [P, I, C, S]),
        "ct_options_create": (P, []),
        "ct_options_destroy": (None, [P]),
        "ct_options_set_string": (I, [P, C, C]),
        "ct_options_set_int": (I, [P, C, ctypes.c_int64]),
        "ct_options_add_profile_range": (I, [P, C, C, c_int64_p, c_int64_p, c_int64_p, I]),
        "ct_build_engine": (I, [P, P, ctypes.POINTER(P)]),
        "ct_engine_destroy": (None, [P]),
        "ct_engine_op_count": (I, [P]),
        "ct_engine_op_info": (I, [P, I, C, S, C, S, ctypes.POINTER(I), ctypes.POINTER(I)]),
        "ct_engine_candidate_id": (I, [P, I, I, C, S]),
        "ct_engine_value_desc": (I, [P, C, c_int64_p, ctypes.POINTER(I), ctypes.POINTER(I)]),
        "ct_engine_value_layout": (I, [P, C, C, S]),
        "ct_engine_workspace_bytes": (S, [P]),
        "ct_engine_create_context": (I, [P, ctypes.POINTER(P)]),
        "ct_context_destroy": (None, [P]),
        "ct_context_bind_input": (I, [P, C, P, S, S, c_int64_p, I, I, C, I]),
        "ct_context_bind_output": (I, [P, C, P, S, S, c_int64_p, I, I, C, I]),
        "ct_context_select_profile": (I, [P, C]),
        "ct_context_set_input_shape": (I, [P, C, c_int64_p, I]),
        "ct_context_resolve_shapes": (I, [P]),
        "ct_context_resolved_desc": (I, [P, C, c_int64_p, ctypes.POINTER(I), ctypes.POINTER(I), C, S]),
        "ct_context_run": (I, [P]),
        "ct_context_run_async": (I, [P, P]),
        "ct_context_run_async_no_alloc": (I, [P, P]),
        "ct_context_synchronize": (I, [P]),
        "ct_context_profile_event_count": (I, [P]),
        "ct_context_profile_event": (I, [P, I, C, S, ctypes.POINTER(D)]),
        "ct_context_graph_count": (S, [P]),
        "ct_context_module_count": (S, [P]),
        "ct_context_time_op": (I, [P, I, I, P, ctypes.POINTER(D)]),
        "ct_context_selected_candidate": (I, [P, I]),
    }
    for name, (restype, argtypes) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _CONFIGURED = True
    return lib


def _check(code: int) -> None:
    if code != 0:
        raise CutritonError(code, _lib().ct_last_error().decode(errors="replace"))


def _shape(dims: Sequence[int]) -> tuple[Any, int]:
    arr = (ctypes.c_int64 * max(1, len(dims)))(*dims)
    return arr, len(dims)


def _b(text: str) -> bytes:
    return text.encode()


def version() -> str:
    return _lib().ct_version().decode()


class Model:
    """Graph IR plus host constants (reference ``cutriton::Model``)."""

    def __init__(self) -> None:
        self._lib = _lib()
        self.handle = self._lib.ct_model_create()

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self._lib.ct_model_destroy(self.handle)
            self.handle = None

    @classmethod
    def from_onnx(cls, source: str | bytes | Path, dim_values: dict[str, int] | None = None) -> "Model":
        """Imports an ONNX model (a file path or the serialized bytes);
        `dim_values` sizes the symbolic input dimensions by name."""
        lib = _lib()
        names = list((dim_values or {}).keys())
        c_names = (ctypes.c_char_p * max(1, len(names)))(*[_b(n) for n in names])
        c_values = (ctypes.c_int64 * max(1, len(names)))(*[int((dim_values or {})[n]) for n in names])
        handle = ctypes.c_void_p()
        if isinstance(source, (bytes, bytearray)):
            data = bytes(source)
            _check(lib.ct_model_import_onnx_buffer(data, len(data), c_names, c_values, len(names),
                                                   ctypes.byref(handle)))
        else:
            _check(lib.ct_model_import_onnx(_b(str(source)), c_names, c_values, len(names), ctypes.byref(handle)))
        model = cls.__new__(cls)
        model._lib = lib
        model.handle = handle.value
        return model

    def add_input(self, name: str, shape: Sequence[int], dtype: str = "float32", layout: str = "NCHW") -> None:
        dims, rank = _shape(shape)
        _check(self._lib.ct_model_add_input(self.handle, _b(name), dims, rank, DTYPE_CODES[dtype], _b(layout)))

    def add_output(self, name: str) -> None:
        _check(self._lib.ct_model_add_output(self.handle, _b(name)))

    def add_constant(self, name: str, array: np.ndarray, layout: str = "") -> None:
        dtype = {np.dtype(np.float32): "float32", np.dtype(np.float16): "float16"}[array.dtype]
        data = np.ascontiguousarray(array)
        dims, rank = _shape(data.shape)
        _check(self._lib.ct_model_add_constant(
            self.handle, _b(name), dims, rank, DTYPE_CODES[dtype], _b(layout),
            data.ctypes.data_as(ctypes.c_void_p), data.nbytes))

    def add_node(self, name: str, op_type: str, inputs: Sequence[str], outputs: Sequence[str],
                 **attributes: Any) -> None:
        ins = (ctypes.c_char_p * max(1, len(inputs)))(*map(_b, inputs))
        outs = (ctypes.c_char_p * max(1, len(outputs)))(*map(_b, outputs))
        _check(self._lib.ct_model_add_node(self.handle, _b(name), _b(op_type), ins, len(inputs), outs,
                                           len(outputs)))
        for key, value in attributes.items():
            self.set_attribute(name, key, value)

    def set_attribute(self, node: str, key: str, value: Any) -> None:
        lib, h = self._lib, self.handle
        if isinstance(value, bool):
            _check(lib.ct_model_set_attr_bool(h, _b(node), _b(key), int(value)))
        elif isinstance(value, int):
            _check(lib.ct_model_set_attr_int(h, _b(node), _b(key), value))
        elif isinstance(value, float):
            _check(lib.ct_model_set_attr_float(h, _b(node), _b(key), value))
        elif isinstance(value, str):
            _check(lib.ct_model_set_attr_string(h, _b(node), _b(key), _b(value)))
        elif isinstance(value, (list, tuple)) and all(isinstance(v, int) for v in value):
            arr = (ctypes.c_int64 * max(1, len(value)))(*value)
            _check(lib.ct_model_set_attr_ints(h, _b(node), _b(key), arr, len(value)))
        elif isinstance(value, (list, tuple)):
            arr = (ctypes.c_double * max(1, len(value)))(*map(float, value))
            _check(lib.ct_model_set_attr_floats(h, _b(node), _b(key), arr, len(value)))
        else:
            raise TypeError(f"unsupported attribute type for {key}: {type(value)}")

    def run_default_passes(self, transformer_fusions: bool = True, residual_epilogue_fusion: bool = True) -> None:
        _check(self._lib.ct_model_run_default_passes(self.handle, int(transformer_fusions),
                                                     int(residual_epilogue_fusion)))

    def op_types(self) -> list[str]:
        out = []
        buf = ctypes.create_string_buffer(128)
        for i in range(self._lib.ct_model_node_count(self.handle)):
            _check(self._lib.ct_model_node_op_type(self.handle, i, buf, 128))
            out.append(buf.value.decode())
        return out


@dataclass
class CompileOptions:
    """Reference ``cutriton::CompileOptions``; graph capture is a hipGraph."""

    target: str = "hip_gfx950"
    kernel_artifact_dir: str = str(PACK_DIR)
    kernel_artifact_paths: list[str] = field(default_factory=list)
    tuning_cache_dir: str = ""
    enable_cuda_graph: bool = True
    enable_profiling: bool = True
    enable_transformer_fusions: bool = True
    enable_residual_epilogue_fusion: bool = True
    allow_cpu_fallback: bool = False
    device_id: int = 0
    tuning_mode: str = "use_cache"
    cuda_graph_cache_capacity: int = 4
    tuning_warmup_iterations: int = 5
    tuning_measurement_iterations: int = 20
    # name -> {input: (min, opt, max)}
    shape_profiles: dict[str, dict[str, tuple[Sequence[int], Sequence[int], Sequence[int]]]] = field(
        default_factory=dict)

    def _handle(self, lib: ctypes.CDLL) -> Any:
        h = lib.ct_options_create()
        try:
            for key in ("target", "kernel_artifact_dir", "tuning_cache_dir"):
                value = getattr(self, key)
                if value:
                    _check(lib.ct_options_set_string(h, _b(key), _b(value)))
            for path in self.kernel_artifact_paths:
                _check(lib.ct_options_set_string(h, b"kernel_artifact_path", _b(path)))
            for key in ("enable_cuda_graph", "enable_profiling", "enable_transformer_fusions",
                        "enable_residual_epilogue_fusion", "allow_cpu_fallback", "device_id",
                        "cuda_graph_cache_capacity", "tuning_warmup_iterations", "tuning_measurement_iterations"):
                _check(lib.ct_options_set_int(h, _b(key), int(getattr(self, key))))
            _check(lib.ct_options_set_int(h, b"tuning_mode", TUNING_MODES[self.tuning_mode]))
            for profile, inputs in self.shape_profiles.items():
                for name, (lo, opt, hi) in inputs.items():
                    a, rank = _shape(lo)
                    b, _ = _shape(opt)
                    c, _ = _shape(hi)
                    _check(lib.ct_options_add_profile_range(h, _b(profile), _b(name), a, b, c, rank))
        except Exception:
            lib.ct_options_destroy(h)
            raise
        return h


@dataclass
class PlanOp:
    op_type: str
    node_name: str
    candidates: list[str]
    selected_candidate: int


class Engine:
    def __init__(self, handle: Any) -> None:
        self._lib = _lib()
        self.handle = handle

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self._lib.ct_engine_destroy(self.handle)
            self.handle = None

    def ops(self) -> list[PlanOp]:
        lib, out = self._lib, []
        op_type, node = ctypes.create_string_buffer(128), ctypes.create_string_buffer(256)
        count, selected = ctypes.c_int(), ctypes.c_int()
        cand = ctypes.create_string_buffer(256)
        for i in range(lib.ct_engine_op_count(self.handle)):
            _check(lib.ct_engine_op_info(self.handle, i, op_type, 128, node, 256, ctypes.byref(count),
                                         ctypes.byref(selected)))
            ids = []
            for c in range(count.value):
                _check(lib.ct_engine_candidate_id(self.handle, i, c, cand, 256))
                ids.append(cand.value.decode())
            out.append(PlanOp(op_type.value.decode(), node.value.decode(), ids, selected.value))
        return out

    def value_desc(self, name: str) -> tuple[list[int], str]:
        dims = (ctypes.c_int64 * 8)()
        rank, dtype = ctypes.c_int(8), ctypes.c_int()
        _check(self._lib.ct_engine_value_desc(self.handle, _b(name), dims, ctypes.byref(rank), ctypes.byref(dtype)))
        return list(dims[: rank.value]), DTYPE_NAMES[dtype.value]

    def value_layout(self, name: str) -> str:
        """The layout a binding of value `name` must carry."""
        buf = ctypes.create_string_buffer(32)
        _check(self._lib.ct_engine_value_layout(self.handle, _b(name), buf, 32))
        return buf.value.decode()

    def workspace_bytes(self) -> int:
        return self._lib.ct_engine_workspace_bytes(self.handle)

    def create_execution_context(self) -> "ExecutionContext":
        h = ctypes.c_void_p()
        _check(self._lib.ct_engine_create_context(self.handle, ctypes.byref(h)))
        return ExecutionContext(h.value, self)


def build_engine(model: Model, options: CompileOptions | None = None) -> Engine:
    lib = _lib()
    opts = (options or CompileOptions())._handle(lib)
    try:
        h = ctypes.c_void_p()
        _check(lib.ct_build_engine(model.handle, opts, ctypes.byref(h)))
    finally:
        lib.ct_options_destroy(opts)
    return Engine(h.value)


def _tensor_view(tensor: Any) -> tuple[int, int, list[int], str, int]:
    """(pointer, buffer bytes, shape, dtype, device code) of a torch tensor."""
    import torch

    if not tensor.is_contiguous():
        raise ValueError("bound tensors must be contiguous")
    dtype = {torch.float32: "float32", torch.float16: "float16"}[tensor.dtype]
    device = 1 if tensor.is_cuda else 0
    return tensor.data_ptr(), tensor.numel() * tensor.element_size(), list(tensor.shape), dtype, device


class ExecutionContext:
    def __init__(self, handle: Any, engine: Engine) -> None:
        self._lib = _lib()
        self.handle = handle
        self._engine = engine  # keeps the plan alive for the Python side
        self._bound: dict[str, Any] = {}

    def __del__(self) -> None:
        if getattr(self, "handle", None):
            self._lib.ct_context_destroy(self.handle)
            self.handle = None

    def _bind(self, fn: Any, name: str, tensor: Any, layout: str) -> None:
        ptr, nbytes, shape, dtype, device = _tensor_view(tensor)
        dims, rank = _shape(shape)
        _check(fn(self.handle, _b(name), ctypes.c_void_p(ptr), nbytes, 0, dims, rank, DTYPE_CODES[dtype],
                  _b(layout), device))
        self._bound[name] = tensor

    def bind_input(self, name: str, tensor: Any, layout: str = "NCHW") -> None:
        self._bind(self._lib.ct_context_bind_input, name, tensor, layout)

    def bind_output(self, name: str, tensor: Any, layout: str = "") -> None:
        self._bind(self._lib.ct_context_bind_output, name, tensor, layout)

    def bind_raw(self, output: bool, name: str, pointer: int, buffer_bytes: int, byte_offset: int,
                 shape: Sequence[int], dtype: str, layout: str, device: int = 1) -> None:
        fn = self._lib.ct_context_bind_output if output else self._lib.ct_context_bind_input
        dims, rank = _shape(shape)
        _check(fn(self.handle, _b(name), ctypes.c_void_p(pointer), buffer_bytes, byte_offset, dims, rank,
                  DTYPE_CODES[dtype], _b(layout), device))

    def select_shape_profile(self, name: str) -> None:
        _check(self._lib.ct_context_select_profile(self.handle, _b(name)))

    def set_input_shape(self, name: str, shape: Sequence[int]) -> None:
        dims, rank = _shape(shape)
        _check(self._lib.ct_context_set_input_shape(self.handle, _b(name), dims, rank))

    def resolve_shapes(self) -> None:
        _check(self._lib.ct_context_resolve_shapes(self.handle))

    def resolved_desc(self, name: str) -> tuple[list[int], str, str]:
        dims = (ctypes.c_int64 * 8)()
        rank, dtype = ctypes.c_int(8), ctypes.c_int()
        layout = ctypes.create_string_buffer(32)
        _check(self._lib.ct_context_resolved_desc(self.handle, _b(name), dims, ctypes.byref(rank),
                                                  ctypes.byref(dtype), layout, 32))
        return list(dims[: rank.value]), DTYPE_NAMES[dtype.value], layout.value.decode()

    def run(self) -> None:
        _check(self._lib.ct_context_run(self.handle))

    def run_async(self, stream: int | None = None) -> None:
        _check(self._lib.ct_context_run_async(self.handle, ctypes.c_void_p(stream or 0)))

    def run_async_no_alloc(self, stream: int) -> None:
        """ct_context_run_async_no_alloc: the run that allocates no device
        memory (the kernels' scratch is the library's static array)."""
        _check(self._lib.ct_context_run_async_no_alloc(self.handle, ctypes.c_void_p(stream)))

    def synchronize(self) -> None:
        _check(self._lib.ct_context_synchronize(self.handle))

    def profile_events(self) -> list[tuple[str, float]]:
        out = []
        name = ctypes.create_string_buffer(256)
        ms = ctypes.c_double()
        for i in range(self._lib.ct_context_profile_event_count(self.handle)):
            _check(self._lib.ct_context_profile_event(self.handle, i, name, 256, ctypes.byref(ms)))
            out.append((name.value.decode(), ms.value))
        return out

    def cached_cuda_graph_count(self) -> int:
        return self._lib.ct_context_graph_count(self.handle)

    def loaded_cuda_module_count(self) -> int:
        return self._lib.ct_context_module_count(self.handle)

    def time_op(self, op_index: int, iterations: int = 20, stream: int | None = None) -> float:
        """Milliseconds per launch of plan op `op_index`'s selected kernels,
        timed over `iterations` back-to-back launches (needs a completed run)."""
        ms = ctypes.c_double()
        _check(self._lib.ct_context_time_op(self.handle, op_index, iterations, stream, ctypes.byref(ms)))
        return ms.value

    def selected_candidates(self, count: int) -> list[int]:
        return [self._lib.ct_context_selected_candidate(self.handle, i) for i in range(count)]

