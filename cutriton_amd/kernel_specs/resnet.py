"""Pack entries of the FP32 CNN kernels (conv_fp32.hip, pool_fp32.hip,
elementwise.hip).

Argument order and sources are those of the reference pack
(``python/cutriton/triton_kernels/resnet.py:216-400``), so a node binds the
same values in the same order; the grids and variants are this backend's.
``FusedConvBatchNormAddRelu`` and the 3-input FP32 Gemm have no reference
kernel: they take the reference convolution / Gemm ABI with one more input.
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

CONV_SOURCE = "conv_fp32.hip"

# (variant id, BLOCK_M, BLOCK_N, BLOCK_K); BLOCK_M tiles output channels and
# BLOCK_N tiles (image, output pixel) columns.
CONV_TILES = (
    ("m128n128", 128, 128, 32),
    ("m64n256", 64, 256, 16),
    ("m64n128", 64, 128, 32),
    ("m128n64", 128, 64, 32),
    ("m64n64", 64, 64, 32),
    ("m64n64k16", 64, 64, 16),
    ("m64n128k16", 64, 128, 16),
    ("m128n64k16", 128, 64, 16),
    ("m64n64k64", 64, 64, 64),
    ("m32n128", 32, 128, 32),
    ("m128n128k16", 128, 128, 16),
)
CONV_DEFAULT = "m64n64"

CONV_DIMENSIONS = (
    arg("n", "i32", "input_dim", index=0, axis=0),
    arg("c", "i32", "input_dim", index=0, axis=1),
    arg("h", "i32", "input_dim", index=0, axis=2),
    arg("w", "i32", "input_dim", index=0, axis=3),
    arg("k", "i32", "input_dim", index=1, axis=0),
    arg("r", "i32", "input_dim", index=1, axis=2),
    arg("s", "i32", "input_dim", index=1, axis=3),
    arg("out_h", "i32", "output_dim", index=0, axis=2),
    arg("out_w", "i32", "output_dim", index=0, axis=3),
    arg("stride_h", "i32", "attribute_i64", name="strides", index=0, default=1),
    arg("stride_w", "i32", "attribute_i64", name="strides", index=1, default=1),
    arg("pad_h", "i32", "attribute_i64", name="pads", index=0, default=0),
    arg("pad_w", "i32", "attribute_i64", name="pads", index=1, default=0),
    arg("dilation_h", "i32", "attribute_i64", name="dilations", index=0, default=1),
    arg("dilation_w", "i32", "attribute_i64", name="dilations", index=1, default=1),
)

# x: ceil(N*P*Q / BLOCK_N), y: ceil(K_out / BLOCK_M).
CONV_GRID = (
    ceil_div(mul(mul(output_dim(0), output_dim(2)), output_dim(3)), meta("BLOCK_N")),
    ceil_div(output_dim(1), meta("BLOCK_M")),
)


def conv_variants(prefix: str) -> tuple[KernelVariant, ...]:
    return tuple(
        KernelVariant(
            name,
            f"{prefix}_{name}",
            num_warps=4,
            meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk},
            default=name == CONV_DEFAULT,
        )
        for name, bm, bn, bk in CONV_TILES
    )


# Split-K variants (conv_fp32.hip): (variant id, BLOCK_M, BLOCK_N, BLOCK_K, SPLIT). SPLIT
# workgroups share one output tile's depth; they need runtime scratch for the
# per-tile counters (16384 x 4 bytes) and the partial sums (128 MiB).
SPLIT_TILES = (
    ("m128n128s2", 128, 128, 32, 2),
    ("m128n128s4", 128, 128, 32, 4),
    ("m128n128s8", 128, 128, 32, 8),
    ("m64n64s2", 64, 64, 32, 2),
    ("m64n64s4", 64, 64, 32, 4),
    ("m64n64s3", 64, 64, 32, 3),
    ("m64n64s5", 64, 64, 32, 5),
    ("m64n64s6", 64, 64, 32, 6),
    ("m64n64k64s2", 64, 64, 64, 2),
    ("m64n64k16s2", 64, 64, 16, 2),
    ("m64n64k16s3", 64, 64, 16, 3),
    ("m64n64k16s5", 64, 64, 16, 5),
    ("m64n64k16s8", 64, 64, 16, 8),
    ("m64n64k16s16", 64, 64, 16, 16),
)
SPLIT_DEFAULT = "m128n128s4"
SPLIT_SCRATCH_BYTES = 16384 * 4 + (128 << 20)
# x: ceil(N*P*Q / BLOCK_N), y: ceil(K_out / BLOCK_M), z: SPLIT.
SPLIT_GRID = CONV_GRID + (meta("SPLIT"),)


def split_variants(prefix: str) -> tuple[KernelVariant, ...]:
    return tuple(
        KernelVariant(name, f"{prefix}_{name}", num_warps=4,
                      meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk, "SPLIT": split},
                      default=name == SPLIT_DEFAULT, scratch_bytes=SPLIT_SCRATCH_BYTES)
        for name, bm, bn, bk, split in SPLIT_TILES
    )


# Register-direct variants (conv_direct_fp32.hip): (variant id, BLOCK_M, BLOCK_N).
DIRECT_SOURCE = "conv_direct_fp32.hip"
DIRECT_TILES = (
    ("d64n256", 64, 256),
    ("d64n64", 64, 64),
    ("d32n64", 32, 64),
)
DIRECT_DEFAULT = "d64n64"

def direct_variants(prefix: str) -> tuple[KernelVariant, ...]:
    return tuple(
        KernelVariant(name, f"{prefix}_{name}", num_warps=4, meta={"BLOCK_M": bm, "BLOCK_N": bn},
                      default=name == DIRECT_DEFAULT)
        for name, bm, bn in DIRECT_TILES
    )


# Few-channel variant (conv_small_c_fp32.hip): C <= 4 and kernels up to 7x7
# (the stem). x: images * ceil(P / 2) * ceil(Q / 112), y: ceil(K / 64).
SMALLC_SOURCE = "conv_small_c_fp32.hip"
SMALLC_GRID = (
    mul(mul(output_dim(0), ceil_div(output_dim(2), literal(2))), ceil_div(output_dim(3), literal(112))),
    ceil_div(output_dim(1), literal(64)),
)
SMALLC_CONSTRAINTS = tuple(
    {"kind": "dim_le", "source": "input", "index": 1, "axis": axis, "value": bound}
    for axis, bound in ((1, 4), (2, 7), (3, 7))
)


def smallc_variants(prefix: str) -> tuple[KernelVariant, ...]:
    return (KernelVariant("r2c64", f"{prefix}_smallc", num_warps=4, default=True),)


def register_conv_family() -> None:
    # conv_fp32.hip reads the weight as OHWI (a channel run of one tap is
    # contiguous); conv_direct_fp32.hip reads OIHW.
    def bn_inputs_for(weight_layout: str | None) -> tuple:
        return tuple(
            arg(name, "*fp32", "input", index=i, **({"layout": weight_layout} if i == 1 and weight_layout else {}))
            for i, name in enumerate(("x", "weight", "scale", "bias", "mean", "variance"))
        )
    epsilon = arg("epsilon", "fp32", "attribute_f64", name="batchnorm_epsilon", default=1e-5)
    # Every family addresses x, the weight, the residual and y through 32-bit
    # buffer resources.
    limit = (BUFFER_RESOURCE_LIMIT,)
    families = ((CONV_SOURCE, "mfma", conv_variants, CONV_GRID, "OHWI", limit),
                (CONV_SOURCE, "splitk", split_variants, SPLIT_GRID, "OHWI", limit),
                (DIRECT_SOURCE, "direct", direct_variants, CONV_GRID, None, limit),
                (SMALLC_SOURCE, "smallc", smallc_variants, SMALLC_GRID, None, SMALLC_CONSTRAINTS + limit))
    residual = (arg("residual", "*fp32", "input", index=6),)
    for op_type, kernel_id, prefix, extra in (
        ("FusedConvBatchNormRelu", "conv_bn_relu.fp32.nchw", "conv_bn_relu_fp32", ()),
        ("FusedConvBatchNorm", "conv_bn.fp32.nchw", "conv_bn_fp32", ()),
        ("FusedConvBatchNormAddRelu", "conv_bn_add_relu.fp32.nchw", "conv_bn_add_relu_fp32", residual),
    ):
        for source, suffix, variants, grid, weight_layout, more in families:
            inputs = bn_inputs_for(weight_layout) + extra
            arguments = inputs + (arg("output", "*fp32", "output", index=0),) + CONV_DIMENSIONS + (epsilon,) + reserved()
            register(KernelSpec(
                f"{kernel_id}.{suffix}", op_type, 1, source, arguments, grid, variants(prefix),
                layout="NCHW", constraints=({"kind": "input_count_eq", "value": len(inputs)},) + more,
            ))
    for source, suffix, variants, grid, weight_layout, more in families:
        conv_arguments = (
            arg("x", "*fp32", "input", index=0),
            arg("weight", "*fp32", "input", index=1, **({"layout": weight_layout} if weight_layout else {})),
            arg("output", "*fp32", "output", index=0),
        ) + CONV_DIMENSIONS + reserved()
        register(KernelSpec(
            f"conv.fp32.nchw.{suffix}", "Conv", 1, source, conv_arguments, grid, variants("conv_fp32"),
            layout="NCHW", constraints=({"kind": "input_count_eq", "value": 2},) + more,
        ))


def register_gemm() -> None:
    # C[M,N] = A[M,K] B[K,N]: x = ceil(N / BLOCK_N), y = ceil(M / BLOCK_M).
    grid = (ceil_div(output_dim(1), meta("BLOCK_N")), ceil_div(output_dim(0), meta("BLOCK_M")))
    tiles = (("m64n64", 64, 64, 32), ("m128n128", 128, 128, 32))
    # Split-K: z = SPLIT workgroups per output tile, runtime scratch as for
    # the split-K convolutions.
    split_tiles = (("m64n64s8", 64, 64, 32, 8), ("m64n64s16", 64, 64, 32, 16))
    split_grid = grid + (meta("SPLIT"),)
    # transB = 1 (e.g. an exported Linear layer: B is [N][K]): the kernels
    # read B's transposed copy ("T" layout, made at constant upload), which
    # is the [K][N] order they take for transB = 0.
    for trans_b, suffix in ((0, ""), (1, "_tb")):
        common = (
            {"kind": "attribute_i64_eq", "name": "transA", "value": 0, "default": 0},
            {"kind": "attribute_i64_eq", "name": "transB", "value": trans_b, "default": 0},
            {"kind": "tensor_rank_eq", "source": "input", "index": 0, "value": 2},
            {"kind": "tensor_rank_eq", "source": "input", "index": 1, "value": 2},
            BUFFER_RESOURCE_LIMIT,  # the conv core's 32-bit buffer resources
        )
        dims = (
            arg("m", "i32", "input_dim", index=0, axis=0),
            arg("n", "i32", "input_dim", index=1, axis=trans_b ^ 1),
            arg("k", "i32", "input_dim", index=0, axis=1),
        )
        register_gemm_family(suffix, {"layout": "T"} if trans_b else {}, common, dims, grid, tiles, split_tiles,
                             split_grid)


def register_gemm_family(suffix, b_source, common, dims, grid, tiles, split_tiles, split_grid) -> None:
    for kernel_id, prefix, inputs, extra in (
        ("gemm.fp32.mfma", "gemm_fp32", ("a", "b"), ()),
        ("gemm_bias.fp32.mfma", "gemm_bias_fp32", ("a", "b", "bias"),
         ({"kind": "tensor_rank_eq", "source": "input", "index": 2, "value": 1},)),
    ):
        arguments = tuple(arg(name, "*fp32", "input", index=i, **(b_source if name == "b" else {}))
                          for i, name in enumerate(inputs)) + (
            arg("output", "*fp32", "output", index=0),
        ) + dims + reserved()
        variants = tuple(
            KernelVariant(name, f"{prefix}_{name}", num_warps=4,
                          meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk}, default=name == "m64n64")
            for name, bm, bn, bk in tiles
        )
        register(KernelSpec(
            kernel_id + suffix, "Gemm", 1, CONV_SOURCE, arguments, grid, variants,
            constraints=({"kind": "input_count_eq", "value": len(inputs)},) + common + extra,
        ))
        split_variants_ = tuple(
            KernelVariant(name, f"{prefix}_{name}", num_warps=4,
                          meta={"BLOCK_M": bm, "BLOCK_N": bn, "BLOCK_K": bk, "SPLIT": split},
                          default=name == "m64n64s8", scratch_bytes=SPLIT_SCRATCH_BYTES)
            for name, bm, bn, bk, split in split_tiles
        )
        register(KernelSpec(
            kernel_id.replace(".mfma", ".splitk") + suffix, "Gemm", 1, CONV_SOURCE, arguments, split_grid,
            split_variants_,
            constraints=({"kind": "input_count_eq", "value": len(inputs)},) + common + extra,
        ))


def register_bandwidth_kernels() -> None:
    def variants(symbol: str) -> tuple[KernelVariant, ...]:
        return (KernelVariant("w4", symbol, num_warps=4, default=True),)

    # Elementwise: 4 elements per thread, 256 threads per workgroup.
    for kernel_id, op_type, symbol, inputs in (
        ("relu.fp32.contiguous", "Relu", "relu_fp32", ("x",)),
        ("add.fp32.contiguous", "Add", "add_fp32", ("a", "b")),
        ("add_relu.fp32.contiguous", "AddRelu", "add_relu_fp32", ("a", "b")),
    ):
        arguments = tuple(arg(name, "*fp32", "input", index=i) for i, name in enumerate(inputs)) + (
            arg("output", "*fp32", "output", index=0),
            arg("total", "i32", "output_numel", index=0),
        ) + reserved()
        register(KernelSpec(
            kernel_id, op_type, 1, "elementwise.hip", arguments, numel_grid(1024), variants(symbol),
            constraints=({"kind": "input_count_eq", "value": len(inputs)},),
        ))

    bn_arguments = (
        arg("x", "*fp32", "input", index=0),
        arg("scale", "*fp32", "input", index=1),
        arg("bias", "*fp32", "input", index=2),
        arg("mean", "*fp32", "input", index=3),
        arg("variance", "*fp32", "input", index=4),
        arg("output", "*fp32", "output", index=0),
        arg("total", "i32", "output_numel", index=0),
        arg("channels", "i32", "input_dim", index=0, axis=1),
        arg("spatial", "i32", "input_dim_product", index=0, begin_axis=2),
        arg("epsilon", "fp32", "attribute_f64", name="epsilon", alternate_name="batchnorm_epsilon", default=1e-5),
    ) + reserved()
    register(KernelSpec(
        "batch_norm.fp32.nchw", "BatchNormalization", 1, "elementwise.hip", bn_arguments, numel_grid(1024),
        variants("batch_norm_fp32_nchw"), layout="NCHW",
    ))

    pool_arguments = (
        arg("x", "*fp32", "input", index=0),
        arg("output", "*fp32", "output", index=0),
        arg("n", "i32", "input_dim", index=0, axis=0),
        arg("c", "i32", "input_dim", index=0, axis=1),
        arg("h", "i32", "input_dim", index=0, axis=2),
        arg("w", "i32", "input_dim", index=0, axis=3),
        arg("out_h", "i32", "output_dim", index=0, axis=2),
        arg("out_w", "i32", "output_dim", index=0, axis=3),
        arg("kernel_h", "i32", "attribute_i64", name="kernel_shape", index=0, default=1),
        arg("kernel_w", "i32", "attribute_i64", name="kernel_shape", index=1, default=1),
        arg("stride_h", "i32", "attribute_i64", name="strides", index=0, default=1),
        arg("stride_w", "i32", "attribute_i64", name="strides", index=1, default=1),
        arg("pad_h", "i32", "attribute_i64", name="pads", index=0, default=0),
        arg("pad_w", "i32", "attribute_i64", name="pads", index=1, default=0),
        arg("dilation_h", "i32", "attribute_i64", name="dilations", index=0, default=1),
        arg("dilation_w", "i32", "attribute_i64", name="dilations", index=1, default=1),
    ) + reserved()
    register(KernelSpec(
        "max_pool.fp32.nchw", "MaxPool", 1, "pool_fp32.hip", pool_arguments,
        # One workgroup per GROUP_BANDS bands of BAND output rows of one
        # (image, channel) plane.
        (ceil_div(mul(mul(output_dim(0), output_dim(1)), ceil_div(output_dim(2), meta("BAND"))),
                  meta("GROUP_BANDS")),),
        tuple(KernelVariant(name, symbol, num_warps=4, meta={"BAND": band, "GROUP_BANDS": group},
                            default=name == "w4")
              for name, symbol, band, group in (
                  ("w4", "max_pool_fp32_nchw", 8, 1),
                  ("b16g4", "max_pool_fp32_nchw_b16g4", 16, 4),
                  # 3 x 3 / 2 windows without LDS; other shapes as bands of 8
                  ("d8", "max_pool_fp32_nchw_d8", 8, 8))),
        layout="NCHW",
    ))

    gap_arguments = (
        arg("x", "*fp32", "input", index=0),
        arg("output", "*fp32", "output", index=0),
        arg("n", "i32", "input_dim", index=0, axis=0),
        arg("c", "i32", "input_dim", index=0, axis=1),
        arg("h", "i32", "input_dim", index=0, axis=2),
        arg("w", "i32", "input_dim", index=0, axis=3),
    ) + reserved()
    # One wavefront per PLANES (image, channel) pairs, 4 per workgroup.
    register(KernelSpec(
        "global_average_pool.fp32.nchw", "GlobalAveragePool", 1, "pool_fp32.hip", gap_arguments,
        (ceil_div(mul(output_dim(0), output_dim(1)), meta("PLANES_PER_GROUP")),),
        (KernelVariant("w4", "global_average_pool_fp32_nchw", num_warps=4, meta={"PLANES_PER_GROUP": 256},
                       default=True),
         KernelVariant("p16", "global_average_pool_fp32_nchw_p16", num_warps=4, meta={"PLANES_PER_GROUP": 64})),
        layout="NCHW",
    ))


register_conv_family()
register_gemm()
register_bandwidth_kernels()
