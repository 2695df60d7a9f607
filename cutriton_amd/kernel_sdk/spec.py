"""Declarative Kernel Pack ABI for the gfx950 kernels.

A :class:`KernelSpec` names one pack ``kernel_id`` for one ``op_type``: the
HIP source that holds its entry points, the ordered launch arguments and
where the runtime binds each one from, the launch grid as a bounded
expression tree, the constraints a node must meet, and the tile variants
(one ``extern "C"`` symbol each). Nothing in a spec is executable: the
runtime accepts only the argument sources, grid nodes and constraint kinds
listed here, which is what lets a pack be loaded without trusting it.

The vocabulary (argument sources, grid AST, constraints, two trailing
``runtime_reserved`` arguments, exactly one default variant) is the one of
the reference SDK, ``python/cutriton/kernel_sdk/spec.py:7-187``; the
differences are the gfx950 ones: a variant names its compiled symbol, and
``num_warps`` counts 64-lane wavefronts.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

# An input may ask for another layout of a constant of the same logical shape:
# OHWI stores an OIHW convolution weight as [out][kh][kw][in]; NK stores a
# [K, N] matrix transposed, as [N][K].
INPUT_LAYOUTS = frozenset({"OHWI", "NK", "T"})

ARGUMENT_SOURCES: dict[str, frozenset[str]] = {
    "input": frozenset({"kind", "index", "layout"}),
    "output": frozenset({"kind", "index"}),
    "input_dim": frozenset({"kind", "index", "axis"}),
    "input_dim_product": frozenset({"kind", "index", "begin_axis"}),
    "output_dim": frozenset({"kind", "index", "axis"}),
    "output_numel": frozenset({"kind", "index"}),
    "attribute_i64": frozenset({"kind", "name", "alternate_name", "index", "default"}),
    "attribute_f64": frozenset({"kind", "name", "alternate_name", "index", "default"}),
    "literal_i32": frozenset({"kind", "default"}),
    "runtime_reserved": frozenset({"kind"}),
}

GRID_LEAVES: dict[str, frozenset[str]] = {
    "literal": frozenset({"kind", "value"}),
    "input_dim": frozenset({"kind", "index", "axis"}),
    "output_dim": frozenset({"kind", "index", "axis"}),
    "input_numel": frozenset({"kind", "index"}),
    "output_numel": frozenset({"kind", "index"}),
    "meta": frozenset({"kind", "name"}),
}
GRID_OPERATORS = frozenset({"ceil_div", "mul"})
MAX_GRID_DEPTH = 8

CONSTRAINTS: dict[str, frozenset[str]] = {
    "attribute_i64_eq": frozenset({"kind", "name", "value", "default"}),
    "input_count_eq": frozenset({"kind", "value"}),
    "tensor_rank_eq": frozenset({"kind", "source", "index", "value"}),
    # shape[axis] of an input/output is at most value
    "dim_le": frozenset({"kind", "source", "index", "axis", "value"}),
    # every input and output tensor bound by the kernel holds at most value bytes
    "tensor_bytes_le": frozenset({"kind", "value"}),
}

# Constraint of every kernel that addresses its tensors through 32-bit buffer
# resources (__builtin_amdgcn_make_buffer_rsrc with a byte count of type int):
# no tensor it binds may reach 2 GiB.
BUFFER_RESOURCE_LIMIT: dict[str, Any] = {"kind": "tensor_bytes_le", "value": 2**31 - 1}

ARGUMENT_TYPES = frozenset({"*fp32", "*fp16", "*i8", "i32", "fp32"})


@dataclass(frozen=True)
class ArgumentSpec:
    """One ordered kernel argument and the runtime source it is bound from."""

    name: str
    type: str
    source: dict[str, Any]


@dataclass(frozen=True)
class KernelVariant:
    """One compiled tile configuration: an entry point of the spec's source."""

    variant_id: str
    symbol: str
    num_warps: int = 4
    num_stages: int = 1
    meta: dict[str, int] = field(default_factory=dict)
    default: bool = False
    # Bytes of zero-initialised device scratch bound to the first
    # runtime_reserved argument (0: that argument stays null).
    scratch_bytes: int = 0


@dataclass(frozen=True)
class KernelSpec:
    kernel_id: str
    op_type: str
    version: int
    source: str
    arguments: tuple[ArgumentSpec, ...]
    grid: tuple[dict[str, Any], ...]
    variants: tuple[KernelVariant, ...]
    dtype: str = "float32"
    layout: str = ""
    min_compute_capability: int = 950
    target_arch: str = "gfx950"
    constraints: tuple[dict[str, Any], ...] = ()

    def validate(self) -> None:
        if not self.kernel_id or not self.op_type or self.version <= 0 or not self.source:
            raise ValueError("KernelSpec identity is incomplete")
        if self.dtype not in {"float32", "float16"}:
            raise ValueError(f"{self.kernel_id}: unsupported dtype {self.dtype}")
        if not self.variants or sum(1 for v in self.variants if v.default) != 1:
            raise ValueError(f"{self.kernel_id}: exactly one default variant is required")
        if len({v.variant_id for v in self.variants}) != len(self.variants):
            raise ValueError(f"{self.kernel_id}: duplicate variant id")
        for variant in self.variants:
            if not variant.symbol.isidentifier():
                raise ValueError(f"{self.kernel_id}: variant symbol is not a C identifier")
            if not 1 <= variant.num_warps <= 16:
                raise ValueError(f"{self.kernel_id}: num_warps must be 1..16 wavefronts")
            if not isinstance(variant.scratch_bytes, int) or variant.scratch_bytes < 0:
                raise ValueError(f"{self.kernel_id}: scratch_bytes must be a non-negative integer")
            if any(not name or not isinstance(value, int) or value <= 0 for name, value in variant.meta.items()):
                raise ValueError(f"{self.kernel_id}: variant meta must be positive integers")
        names = [argument.name for argument in self.arguments]
        if len(set(names)) != len(names):
            raise ValueError(f"{self.kernel_id}: duplicate argument name")
        for argument in self.arguments:
            kind = argument.source.get("kind")
            if kind not in ARGUMENT_SOURCES:
                raise ValueError(f"{self.kernel_id}: unsafe source for {argument.name}")
            unknown = set(argument.source) - ARGUMENT_SOURCES[kind]
            if unknown:
                raise ValueError(
                    f"{self.kernel_id}: unknown source field for {argument.name}: {sorted(unknown)}"
                )
            if argument.type not in ARGUMENT_TYPES:
                raise ValueError(f"{self.kernel_id}: unsupported argument type {argument.type}")
            if "layout" in argument.source and argument.source["layout"] not in INPUT_LAYOUTS:
                raise ValueError(f"{self.kernel_id}: unknown input layout for {argument.name}")
        reserved = [i for i, a in enumerate(self.arguments) if a.source.get("kind") == "runtime_reserved"]
        if reserved != [len(self.arguments) - 2, len(self.arguments) - 1]:
            raise ValueError(f"{self.kernel_id}: the ABI requires two trailing runtime_reserved arguments")
        _validate_grid(self.kernel_id, self.grid, self.variants)
        for constraint in self.constraints:
            kind = constraint.get("kind")
            if kind not in CONSTRAINTS or set(constraint) - CONSTRAINTS[kind]:
                raise ValueError(f"{self.kernel_id}: unsafe constraint")
            if kind in {"tensor_rank_eq", "dim_le"} and constraint.get("source") not in {"input", "output"}:
                raise ValueError(f"{self.kernel_id}: invalid tensor constraint source")
            if kind == "dim_le" and (not isinstance(constraint.get("axis"), int) or constraint["axis"] < 0):
                raise ValueError(f"{self.kernel_id}: dim_le needs a non-negative axis")
            if kind == "tensor_bytes_le" and (not isinstance(constraint.get("value"), int) or constraint["value"] <= 0):
                raise ValueError(f"{self.kernel_id}: tensor_bytes_le needs a positive byte count")


def _validate_grid(kernel_id: str, grid: Any, variants: tuple[KernelVariant, ...]) -> None:
    if not isinstance(grid, tuple) or not 1 <= len(grid) <= 3:
        raise ValueError(f"{kernel_id}: grid must contain one to three axes")
    # Every variant must define every meta name the grid reads.
    meta_sets = [set(v.meta) for v in variants]

    def check(expression: Any, depth: int) -> None:
        if depth > MAX_GRID_DEPTH or not isinstance(expression, dict):
            raise ValueError(f"{kernel_id}: invalid grid expression")
        kind = expression.get("kind")
        if kind in GRID_LEAVES:
            if set(expression) != GRID_LEAVES[kind]:
                raise ValueError(f"{kernel_id}: invalid {kind} grid leaf")
            if kind == "literal" and (not isinstance(expression["value"], int) or expression["value"] <= 0):
                raise ValueError(f"{kernel_id}: grid literals must be positive")
            if kind in {"input_dim", "output_dim"} and not (
                isinstance(expression["index"], int) and isinstance(expression["axis"], int)
            ):
                raise ValueError(f"{kernel_id}: grid tensor coordinates must be integers")
            if kind in {"input_numel", "output_numel"} and not isinstance(expression["index"], int):
                raise ValueError(f"{kernel_id}: grid tensor index must be an integer")
            if kind == "meta" and any(expression["name"] not in names for names in meta_sets):
                raise ValueError(f"{kernel_id}: grid references unknown variant meta")
            return
        if kind not in GRID_OPERATORS or set(expression) != {"kind", "args"}:
            raise ValueError(f"{kernel_id}: unsafe grid expression")
        args = expression["args"]
        if not isinstance(args, list) or len(args) != 2:
            raise ValueError(f"{kernel_id}: {kind} requires two operands")
        for operand in args:
            check(operand, depth + 1)

    for axis in grid:
        check(axis, 0)


_REGISTRY: list[KernelSpec] = []


def register(spec: KernelSpec) -> KernelSpec:
    spec.validate()
    if any(item.kernel_id == spec.kernel_id for item in _REGISTRY):
        raise ValueError(f"duplicate kernel id: {spec.kernel_id}")
    _REGISTRY.append(spec)
    return spec


def registered_specs() -> tuple[KernelSpec, ...]:
    return tuple(_REGISTRY)


def clear_registry() -> None:
    _REGISTRY.clear()


# ---- small constructors shared by the spec modules ----

def arg(argument_name: str, type_name: str, kind: str, **source: Any) -> ArgumentSpec:
    return ArgumentSpec(argument_name, type_name, {"kind": kind, **source})


def reserved() -> tuple[ArgumentSpec, ArgumentSpec]:
    return (
        arg("runtime_scratch", "*i8", "runtime_reserved"),
        arg("profile_scratch", "*i8", "runtime_reserved"),
    )


def literal(value: int) -> dict[str, Any]:
    return {"kind": "literal", "value": value}


def output_dim(axis: int, index: int = 0) -> dict[str, Any]:
    return {"kind": "output_dim", "index": index, "axis": axis}


def meta(name: str) -> dict[str, Any]:
    return {"kind": "meta", "name": name}


def ceil_div(a: dict[str, Any], b: dict[str, Any]) -> dict[str, Any]:
    return {"kind": "ceil_div", "args": [a, b]}


def mul(a: dict[str, Any], b: dict[str, Any]) -> dict[str, Any]:
    return {"kind": "mul", "args": [a, b]}


def numel_grid(per_workgroup: int) -> tuple[dict[str, Any], ...]:
    return (ceil_div({"kind": "output_numel", "index": 0}, literal(per_workgroup)),)
