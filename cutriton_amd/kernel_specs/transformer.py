"""Pack entries of the FP16 FFN kernels (gemm_fp16.hip, gemm_fp16_nt.hip,
layer_norm_fp16.hip, elementwise.hip).

Argument order and sources follow the reference pack
(``python/cutriton/triton_kernels/transformer.py:193-371``): Gemm/GemmGelu
take ``a, b, output, m, n, k`` with m and n read from the output. The
3-input (bias) Gemm/GemmGelu entries are additions of this backend: they
insert ``bias`` (input 2) after ``b``.
"""

from __future__ import annotations

from cutriton_amd.kernel_sdk.spec import (
    BUFFER_RESOURCE_LIMIT,
    KernelSpec,
    KernelVariant,
    arg,
    ceil_div,
    literal,
    meta,
    mul,
    numel_grid,
    output_dim,
    register,
    reserved,
)

GEMM_SOURCE = "gemm_fp16.hip"

# (variant id, BLOCK_M, BLOCK_N, BLOCK_K, wavefronts)
GEMM_TILES = (
    ("m64n64k64", 64, 64, 64, 2),
    ("m128n128k64", 128, 128, 64, 4),
    ("m256n128k64", 256, 128, 64, 4),
    ("m256n256k64", 256, 256, 64, 8),
)
GEMM_DEFAULT = "m128n128k64"

# One workgroup per output tile: ceil(M / BLOCK_M) * ceil(N / BLOCK_N).
GEMM_GRID = (mul(ceil_div(output_dim(0), meta("BLOCK_M")), ceil_div(output_dim(1), meta("BLOCK_N"))),)

GEMM_DIMS = (
    arg("m", "i32", "output_dim", index=0, axis=0),
    arg("n", "i32", "output_dim", index=0, axis=1),
    arg("k", "i32", "input_dim", index=0, axis=1),
)

def gemm_constraints(trans_b: int) -> tuple[dict, ...]:
    return (
        {"kind": "attribute_i64_eq", "name": "transA", "value": 0, "default": 0},
        {"kind": "attribute_i64_eq", "name": "transB", "value": trans_b, "default": 0},
        {"kind": "tensor_rank_eq", "source": "input", "index": 0, "value": 2},
        {"kind": "tensor_rank_eq", "source": "input", "index": 1, "value": 2},
    )


# Weight-transposed kernels (gemm_fp16_nt.hip): `b` is bound to the [N][K]
# copy of a constant B (input layout NK). (variant id, BLOCK_M, BLOCK_N,
# BLOCK_K, wavefronts)
GEMM_NT_SOURCE = "gemm_fp16_nt.hip"
GEMM_NT_TILES = (
    ("m256n256w4", 256, 256, 64, 4),
    ("m256n256w8", 256, 256, 64, 8),
    ("m256n128w4", 256, 128, 64, 4),
    ("m128n256w4", 128, 256, 64, 4),
    ("m128n128w4", 128, 128, 64, 4),
    ("m128n128k128w4", 128, 128, 128, 4),
    ("m64n128w4", 64, 128, 64, 4),
    ("m64n64w4", 64, 64, 64, 4),
    ("m256n128w8", 256, 128, 64, 8),
    ("m128n256w8", 128, 256, 64, 8),
    ("m128n128w8", 128, 128, 64, 8),
    ("m128n128k128w8", 128, 128, 128, 8),
    ("m128n64w8", 128, 64, 64, 8),
    # 2 x 2 wavefront tiles times 2 depth groups that split each 128-deep stage
    ("m128n128k128w2x2k2", 128, 128, 128, 8),
)
GEMM_NT_DEFAULT = "m128n128w4"


def gemm_variants(prefix: str) -> tuple[KernelVariant, ...]:
    return tuple(
        KernelVariant(
            name, f"{prefix}_{name}", num_warps=waves,
            meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk}, default=name == GEMM_DEFAULT,
        )
        for name, bm, bn, bk, waves in GEMM_TILES
    )


# Split-K weight-transposed tiles: SPLIT workgroups per output tile, each on
# an equal share of the depth, with FP32 shares and per-tile counters in the
# runtime scratch (16384 counters, then at most 128 MiB of shares). (variant
# id, BLOCK_M, BLOCK_N, BLOCK_K, wavefronts, SPLIT)
GEMM_NT_SPLIT_TILES = (
    ("m64n64s2", 64, 64, 64, 4, 2),
    ("m64n64s4", 64, 64, 64, 4, 4),
    ("m128n64s4", 128, 64, 64, 8, 4),
    ("m128n128s2", 128, 128, 64, 8, 2),
)
GEMM_SPLIT_SCRATCH_BYTES = 16384 * 4 + (128 << 20)
# ceil(M / BLOCK_M) * ceil(N / BLOCK_N) tiles, SPLIT workgroups each.
GEMM_NT_GRID = (mul(GEMM_GRID[0], meta("SPLIT")),)


def gemm_nt_variants(prefix: str) -> tuple[KernelVariant, ...]:
    whole = tuple(
        KernelVariant(
            name, f"{prefix}_{name}", num_warps=waves,
            meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk, "SPLIT": 1}, default=name == GEMM_NT_DEFAULT,
        )
        for name, bm, bn, bk, waves in GEMM_NT_TILES
    )
    split = tuple(
        KernelVariant(
            name, f"{prefix}_{name}", num_warps=waves,
            meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk, "SPLIT": sp}, scratch_bytes=GEMM_SPLIT_SCRATCH_BYTES,
        )
        for name, bm, bn, bk, waves, sp in GEMM_NT_SPLIT_TILES
    )
    return whole + split


def register_gemms() -> None:
    for kernel_id, op_type, prefix, bias in (
        ("gemm.fp16.mfma", "Gemm", "gemm_fp16", False),
        ("gemm_gelu.fp16.mfma", "GemmGelu", "gemm_gelu_fp16", False),
        ("gemm_bias.fp16.mfma", "Gemm", "gemm_bias_fp16", True),
        ("gemm_gelu_bias.fp16.mfma", "GemmGelu", "gemm_gelu_bias_fp16", True),
    ):
        inputs = ("a", "b", "bias") if bias else ("a", "b")
        # The weight-transposed family comes first in the pack (kernel ids sort
        # that way), so its default is the untuned choice whenever B is a
        # constant; "_kn" kernels read B as it is and serve every other Gemm.
        # With transB = 1 (an exported Linear layer) B is [N][K] already and
        # the "_tb" entries pass it to the same NT kernels as it is.
        nt_variants = gemm_nt_variants(prefix.replace("_fp16", "_nt_fp16"))
        for suffix, source, variants, b_source, trans_b in (
            ("", GEMM_NT_SOURCE, nt_variants, {"layout": "NK"}, 0),
            ("_kn", GEMM_SOURCE, gemm_variants(prefix), {}, 0),
            ("_tb", GEMM_NT_SOURCE, nt_variants, {}, 1),
        ):
            constraints = ({"kind": "input_count_eq", "value": len(inputs)},) + gemm_constraints(trans_b)
            if source == GEMM_NT_SOURCE:  # 32-bit buffer resources over A and B
                constraints += (BUFFER_RESOURCE_LIMIT,)
            if bias:
                constraints += ({"kind": "tensor_rank_eq", "source": "input", "index": 2, "value": 1},)
            arguments = tuple(
                arg(name, "*fp16", "input", index=i, **(b_source if name == "b" else {}))
                for i, name in enumerate(inputs)
            ) + (arg("output", "*fp16", "output", index=0),) + GEMM_DIMS + reserved()
            register(KernelSpec(
                kernel_id + suffix, op_type, 1, source, arguments,
                GEMM_NT_GRID if source == GEMM_NT_SOURCE else GEMM_GRID, variants,
                dtype="float16", constraints=constraints,
            ))


def register_elementwise() -> None:
    # 8 halves per thread, 256 threads per workgroup.
    for kernel_id, op_type, symbol, inputs in (
        ("gelu.fp16.contiguous", "Gelu", "gelu_fp16", ("x",)),
        ("add.fp16.contiguous", "Add", "add_fp16", ("a", "b")),
    ):
        arguments = tuple(arg(name, "*fp16", "input", index=i) for i, name in enumerate(inputs)) + (
            arg("output", "*fp16", "output", index=0),
            arg("total", "i32", "output_numel", index=0),
        ) + reserved()
        register(KernelSpec(
            kernel_id, op_type, 1, "elementwise.hip", arguments, numel_grid(2048),
            (KernelVariant("w4", symbol, num_warps=4, default=True),), dtype="float16",
            constraints=({"kind": "input_count_eq", "value": len(inputs)},),
        ))


# Row-kernel variants of LayerNorm, SkipLayerNorm and Softmax: (name, rows
# per 256-thread workgroup). gNcM: N lanes per row, M 16-byte chunks per lane;
# rows of up to N * 8 * M columns stay in registers, longer rows re-read.
ROW_VARIANTS = (
    ("g16c1", 16), ("g32c1", 8), ("g64c1", 4), ("g64c2", 4), ("g64c4", 4), ("g64c8", 4),
)
ROW_DEFAULT = "g64c8"
SOFTMAX_VARIANTS = ROW_VARIANTS
SOFTMAX_DEFAULT = ROW_DEFAULT


def register_norms() -> None:
    for kernel_id, op_type, symbol, inputs in (
        ("layer_norm.fp16.last_axis", "LayerNormalization", "layer_norm_fp16", ("x", "scale", "bias")),
        ("skip_layer_norm.fp16.last_axis", "SkipLayerNormalization", "skip_layer_norm_fp16",
         ("x", "residual", "scale", "bias")),
    ):
        arguments = tuple(arg(name, "*fp16", "input", index=i) for i, name in enumerate(inputs)) + (
            arg("output", "*fp16", "output", index=0),
            arg("rows", "i32", "input_dim", index=0, axis=0),
            arg("columns", "i32", "input_dim", index=0, axis=1),
            arg("epsilon", "fp32", "attribute_f64", name="epsilon", default=1e-5),
        ) + reserved()
        register(KernelSpec(
            kernel_id, op_type, 1, "layer_norm_fp16.hip", arguments,
            (ceil_div(output_dim(0), meta("ROWS")),),
            tuple(KernelVariant(name, f"{symbol}_{name}", num_warps=4, meta={"ROWS": rows},
                                default=name == ROW_DEFAULT) for name, rows in ROW_VARIANTS),
            dtype="float16",
            constraints=(
                {"kind": "input_count_eq", "value": len(inputs)},
                {"kind": "tensor_rank_eq", "source": "input", "index": 0, "value": 2},
            ),
        ))




def register_softmax() -> None:
    arguments = (
        arg("x", "*fp16", "input", index=0),
        arg("output", "*fp16", "output", index=0),
        arg("rows", "i32", "input_dim", index=0, axis=0),
        arg("columns", "i32", "input_dim", index=0, axis=1),
    ) + reserved()
    register(KernelSpec(
        "softmax.fp16.last_axis", "Softmax", 1, "softmax_fp16.hip", arguments,
        (ceil_div(output_dim(0), meta("ROWS")),),
        tuple(KernelVariant(name, f"softmax_fp16_{name}", num_warps=4, meta={"ROWS": rows},
                            default=name == SOFTMAX_DEFAULT) for name, rows in SOFTMAX_VARIANTS),
        dtype="float16",
        constraints=(
            {"kind": "input_count_eq", "value": 1},
            {"kind": "tensor_rank_eq", "source": "input", "index": 0, "value": 2},
        ),
    ))


# Attention variants by the largest head dimension they serve. The ids sort
# so that the 64-wide kernel is the untuned choice whenever it applies.
ATTENTION_VARIANTS = (("d064", 64), ("d128", 128))
ATTENTION_QUERIES_PER_WORKGROUP = 128


def register_attention() -> None:
    arguments = (
        arg("q", "*fp16", "input", index=0),
        arg("k", "*fp16", "input", index=1),
        arg("v", "*fp16", "input", index=2),
        arg("output", "*fp16", "output", index=0),
        arg("batch", "i32", "input_dim", index=0, axis=0),
        arg("heads", "i32", "input_dim", index=0, axis=1),
        arg("sq", "i32", "input_dim", index=0, axis=2),
        arg("sk", "i32", "input_dim", index=1, axis=2),
        arg("d", "i32", "input_dim", index=0, axis=3),
        arg("scale", "fp32", "attribute_f64", name="scale", default=1.0),
        arg("causal", "i32", "attribute_i64", name="is_causal", default=0),
    ) + reserved()
    grid = (ceil_div(output_dim(2), literal(ATTENTION_QUERIES_PER_WORKGROUP)), mul(output_dim(0), output_dim(1)))
    for name, dmax in ATTENTION_VARIANTS:
        register(KernelSpec(
            f"attention.fp16.{name}", "Attention", 1, "attention_fp16.hip", arguments, grid,
            (KernelVariant("w4", f"attention_fp16_d{dmax}", num_warps=4, default=True),),
            dtype="float16",
            constraints=(
                {"kind": "input_count_eq", "value": 3},
                {"kind": "tensor_rank_eq", "source": "input", "index": 0, "value": 4},
                {"kind": "tensor_rank_eq", "source": "input", "index": 1, "value": 4},
                {"kind": "tensor_rank_eq", "source": "input", "index": 2, "value": 4},
                {"kind": "dim_le", "source": "input", "index": 0, "axis": 3, "value": dmax},
                BUFFER_RESOURCE_LIMIT,  # K is read through a 32-bit buffer resource
            ),
        ))


register_gemms()
register_elementwise()
register_norms()
register_softmax()
register_attention()
