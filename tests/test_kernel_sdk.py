"""Kernel SDK and pack producer (CPU only).

Spec validation follows the reference's SDK tests
(tests/python/test_kernel_sdk.py:39-107): the same rejections with the same
messages. The pack checks read the built pack.json and verify what the loader
relies on: every binary's SHA-256, every variant symbol present as a function
of its code object, one default variant per kernel id, the ABI tail.
"""

from __future__ import annotations

import hashlib
import json

import pytest

from cutriton_amd import native
from cutriton_amd.kernel_sdk import builder
from cutriton_amd.kernel_sdk.spec import (
    ArgumentSpec,
    KernelSpec,
    KernelVariant,
    clear_registry,
    register,
    registered_specs,
)


def _spec(source_kind: str = "input", variants=None, **overrides) -> KernelSpec:
    fields = dict(
        kernel_id="unit.relu.fp32",
        op_type="Relu",
        version=1,
        source="elementwise.hip",
        arguments=(
            ArgumentSpec("x", "*fp32", {"kind": source_kind, "index": 0}),
            ArgumentSpec("output", "*fp32", {"kind": "output", "index": 0}),
            ArgumentSpec("runtime_scratch", "*i8", {"kind": "runtime_reserved"}),
            ArgumentSpec("profile_scratch", "*i8", {"kind": "runtime_reserved"}),
        ),
        grid=({"kind": "ceil_div", "args": [{"kind": "output_numel", "index": 0}, {"kind": "literal", "value": 256}]},),
        variants=variants or (KernelVariant("default", "relu_fp32", default=True),),
    )
    fields.update(overrides)
    return KernelSpec(**fields)


@pytest.fixture
def registry():
    saved = registered_specs()
    clear_registry()
    yield
    clear_registry()
    for spec in saved:
        register(spec)


def test_valid_spec_round_trips(registry):
    spec = _spec()
    register(spec)
    assert registered_specs() == (spec,)
    assert registered_specs()[0].arguments[0].source["kind"] == "input"


def test_rejects_unsafe_argument_source():
    with pytest.raises(ValueError, match="unsafe source"):
        _spec(source_kind="python_callable").validate()


def test_rejects_duplicate_kernel_id(registry):
    register(_spec())
    with pytest.raises(ValueError, match="duplicate kernel id"):
        register(_spec())


def test_requires_two_trailing_reserved_arguments():
    spec = _spec()
    with pytest.raises(ValueError, match="two trailing"):
        _spec(arguments=spec.arguments[:-1]).validate()
    reordered = (spec.arguments[2], spec.arguments[0], spec.arguments[1], spec.arguments[3])
    with pytest.raises(ValueError, match="two trailing"):
        _spec(arguments=reordered).validate()


def test_requires_exactly_one_default_variant():
    both = (KernelVariant("a", "relu_fp32", default=True), KernelVariant("b", "relu_fp32", default=True))
    with pytest.raises(ValueError, match="exactly one default"):
        _spec(variants=both).validate()
    with pytest.raises(ValueError, match="exactly one default"):
        _spec(variants=(KernelVariant("a", "relu_fp32"),)).validate()


def test_rejects_arbitrary_grid_and_constraint_expressions():
    with pytest.raises(ValueError, match="grid"):
        _spec(grid=({"kind": "python", "callable": "evil"},)).validate()
    with pytest.raises(ValueError, match="unsafe constraint"):
        _spec(constraints=({"kind": "python", "expression": "x"},)).validate()


def test_dim_le_constraint_is_checked():
    ok = {"kind": "dim_le", "source": "input", "index": 1, "axis": 1, "value": 4}
    _spec(constraints=(ok,)).validate()
    with pytest.raises(ValueError, match="source"):
        _spec(constraints=({**ok, "source": "attribute"},)).validate()
    with pytest.raises(ValueError, match="axis"):
        _spec(constraints=({**ok, "axis": -1},)).validate()
    with pytest.raises(ValueError, match="unsafe constraint"):
        _spec(constraints=({**ok, "expression": "x"},)).validate()


def test_input_layout_nk_is_accepted():
    spec = _spec()
    laid_out = (ArgumentSpec("x", "*fp32", {"kind": "input", "index": 0, "layout": "NK"}),) + spec.arguments[1:]
    _spec(arguments=laid_out).validate()


def test_accepts_safe_multidimensional_grid():
    _spec(
        variants=(KernelVariant("tiled", "relu_fp32", meta={"BLOCK": 64}, default=True),),
        grid=(
            {"kind": "ceil_div", "args": [{"kind": "output_dim", "index": 0, "axis": 0}, {"kind": "meta", "name": "BLOCK"}]},
            {"kind": "literal", "value": 2},
        ),
    ).validate()


def test_rejects_unknown_grid_meta_and_deep_trees():
    with pytest.raises(ValueError, match="unknown variant meta"):
        _spec(grid=({"kind": "meta", "name": "UNDECLARED"},)).validate()
    deep = {"kind": "literal", "value": 1}
    for _ in range(9):
        deep = {"kind": "mul", "args": [deep, {"kind": "literal", "value": 1}]}
    with pytest.raises(ValueError):
        _spec(grid=(deep,)).validate()


def test_rejects_non_identifier_symbols_and_bad_wave_counts():
    with pytest.raises(ValueError, match="C identifier"):
        _spec(variants=(KernelVariant("v", "relu fp32", default=True),)).validate()
    with pytest.raises(ValueError, match="num_warps"):
        _spec(variants=(KernelVariant("v", "relu_fp32", num_warps=32, default=True),)).validate()


def test_input_layout_is_checked():
    spec = _spec()
    laid_out = (ArgumentSpec("x", "*fp32", {"kind": "input", "index": 0, "layout": "OHWI"}),) + spec.arguments[1:]
    _spec(arguments=laid_out).validate()
    bad = (ArgumentSpec("x", "*fp32", {"kind": "input", "index": 0, "layout": "NHWC"}),) + spec.arguments[1:]
    with pytest.raises(ValueError, match="layout"):
        _spec(arguments=bad).validate()
    on_output = spec.arguments[:1] + (ArgumentSpec("output", "*fp32", {"kind": "output", "index": 0,
                                                                       "layout": "OHWI"}),) + spec.arguments[2:]
    with pytest.raises(ValueError, match="unknown source field"):
        _spec(arguments=on_output).validate()


def test_elf_symbol_reader_rejects_non_elf():
    with pytest.raises(ValueError):
        builder.elf_function_symbols(b"// ptx\n")


@pytest.fixture(scope="module")
def pack() -> dict:
    path = native.PACK_DIR / "pack.json"
    if not path.exists():
        native.build_kernel_pack()
    return json.loads(path.read_text())


def test_pack_manifest_binaries_and_symbols(pack):
    assert pack["schema_version"] == 2 and pack["abi_schema_version"] == 2
    digests: dict[str, str] = {}
    symbols: dict[str, set[str]] = {}
    for entry in pack["kernels"]:
        binary = entry["binary"]
        assert not binary.startswith("/") and ".." not in binary.split("/")
        assert entry["binary_format"] == "hsaco" and entry["target_arch"] == "gfx950"
        if binary not in digests:
            image = (native.PACK_DIR / binary).read_bytes()
            digests[binary] = hashlib.sha256(image).hexdigest()
            symbols[binary] = builder.elf_function_symbols(image)
        assert entry["sha256"] == digests[binary], entry["kernel_id"]
        assert entry["symbol"] in symbols[binary], entry["symbol"]
        args = entry["arguments"]
        assert [a["source"]["kind"] for a in args[-2:]] == ["runtime_reserved"] * 2
        assert all(a["source"]["kind"] != "runtime_reserved" for a in args[:-2])


def test_pack_has_one_default_per_kernel_and_covers_the_hot_path(pack):
    defaults: dict[str, int] = {}
    for entry in pack["kernels"]:
        defaults[entry["kernel_id"]] = defaults.get(entry["kernel_id"], 0) + int(entry["default"])
    assert all(v == 1 for v in defaults.values()), defaults
    ops = {entry["op_type"] for entry in pack["kernels"]}
    for op in ("FusedConvBatchNormRelu", "FusedConvBatchNorm", "FusedConvBatchNormAddRelu", "Conv", "MaxPool",
               "GlobalAveragePool", "Gemm", "GemmGelu", "SkipLayerNormalization", "BatchNormalization", "Relu",
               "Add", "AddRelu", "Gelu", "LayerNormalization"):
        assert op in ops, op
