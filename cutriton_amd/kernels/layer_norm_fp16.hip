// LayerNormalization and SkipLayerNormalization over the last axis, FP16 in
// and out, FP32 statistics; one wavefront per row.
//
// Semantics follow python/cutriton/triton_kernels/transformer.py:
//   layer_norm_fp16 (128-149) and skip_layer_norm_fp16 (152-177):
//   v = x (+ residual), widened to FP32; mean = sum(v) / cols;
//   var = sum((v - mean)^2) / cols (two passes over the row);
//   y = fp16((v - mean) * rsqrt(var + eps) * gamma + beta).
// Unlike the reference (one 1024-wide block per row) any column count works:
// rows of up to kCachedColumns stay in registers between the passes, longer
// rows are re-read. Argument order is the pack ABI of transformer.py:323-371.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr int kChunk = 8;                                   // halves per lane per 16-byte access
constexpr int kCachedChunks = 8;                            // 16-byte chunks per lane kept in registers
constexpr int kCachedColumns = 64 * kChunk * kCachedChunks;  // 4096

template <bool SKIP>
__device__ __forceinline__ void LayerNormRow(const _Float16* __restrict__ x, const _Float16* __restrict__ residual,
                                             const _Float16* __restrict__ gamma, const _Float16* __restrict__ beta,
                                             _Float16* __restrict__ output, int rows, int columns, float epsilon) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const size_t offset = static_cast<size_t>(row) * columns;
  const _Float16* xr = x + offset;
  const _Float16* rr = SKIP ? residual + offset : nullptr;
  _Float16* yr = output + offset;
  const float inv_columns = 1.0f / static_cast<float>(columns);
  const bool vec = (columns % kChunk) == 0 && columns <= kCachedColumns &&
                   ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(output) |
                     reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta) |
                     (SKIP ? reinterpret_cast<uintptr_t>(residual) : 0)) & 15) == 0;

  if (vec) {
    float v[kCachedChunks][kChunk];
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < kCachedChunks; ++c) {
      const int col = (c * 64 + lane) * kChunk;
      if (col < columns) {
        const ct::f16x8 a = *reinterpret_cast<const ct::f16x8*>(xr + col);
        ct::f16x8 b;
        if (SKIP) b = *reinterpret_cast<const ct::f16x8*>(rr + col);
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          v[c][e] = static_cast<float>(a[e]) + (SKIP ? static_cast<float>(b[e]) : 0.0f);
          sum += v[c][e];
        }
      }
    }
    const float mean = ct::WaveSum(sum) * inv_columns;
    float sq = 0.0f;
#pragma unroll
    for (int c = 0; c < kCachedChunks; ++c) {
      const int col = (c * 64 + lane) * kChunk;
      if (col < columns) {
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          v[c][e] -= mean;
          sq += v[c][e] * v[c][e];
        }
      }
    }
    const float rstd = rsqrtf(ct::WaveSum(sq) * inv_columns + epsilon);
#pragma unroll
    for (int c = 0; c < kCachedChunks; ++c) {
      const int col = (c * 64 + lane) * kChunk;
      if (col < columns) {
        const ct::f16x8 g = *reinterpret_cast<const ct::f16x8*>(gamma + col);
        const ct::f16x8 bt = *reinterpret_cast<const ct::f16x8*>(beta + col);
        ct::f16x8 y;
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          y[e] = static_cast<_Float16>(v[c][e] * rstd * static_cast<float>(g[e]) + static_cast<float>(bt[e]));
        }
        *reinterpret_cast<ct::f16x8*>(yr + col) = y;
      }
    }
    return;
  }

  // General path: element-strided, three passes over global memory.
  auto value = [&](int col) {
    return static_cast<float>(xr[col]) + (SKIP ? static_cast<float>(rr[col]) : 0.0f);
  };
  float sum = 0.0f;
  for (int col = lane; col < columns; col += 64) sum += value(col);
  const float mean = ct::WaveSum(sum) * inv_columns;
  float sq = 0.0f;
  for (int col = lane; col < columns; col += 64) {
    const float d = value(col) - mean;
    sq += d * d;
  }
  const float rstd = rsqrtf(ct::WaveSum(sq) * inv_columns + epsilon);
  for (int col = lane; col < columns; col += 64) {
    yr[col] = static_cast<_Float16>((value(col) - mean) * rstd * static_cast<float>(gamma[col]) +
                                    static_cast<float>(beta[col]));
  }
}

}  // namespace

CT_KERNEL void __launch_bounds__(kThreads)
    layer_norm_fp16(const _Float16* x, const _Float16* scale, const _Float16* bias, _Float16* output, int rows,
                    int columns, float epsilon, void*, void*) {
  LayerNormRow<false>(x, nullptr, scale, bias, output, rows, columns, epsilon);
}

CT_KERNEL void __launch_bounds__(kThreads)
    skip_layer_norm_fp16(const _Float16* x, const _Float16* residual, const _Float16* scale, const _Float16* bias,
                         _Float16* output, int rows, int columns, float epsilon, void*, void*) {
  LayerNormRow<true>(x, residual, scale, bias, output, rows, columns, epsilon);
}
