// LayerNormalization and SkipLayerNormalization over the last axis, FP16 in
// and out, FP32 statistics.
//
// Semantics follow python/cutriton/triton_kernels/transformer.py:
//   layer_norm_fp16 (128-149) and skip_layer_norm_fp16 (152-177):
//   v = x (+ residual), widened to FP32; mean = sum(v) / cols;
//   var = sum((v - mean)^2) / cols (two passes over the row);
//   y = fp16((v - mean) * rsqrt(var + eps) * gamma + beta).
// Unlike the reference (one 1024-wide block per row) any column count works.
// A group of GROUP lanes owns one row (64 / GROUP rows per wavefront); each
// lane keeps CHUNKS 16-byte chunks of the row in registers between the two
// passes, so x (and the residual) are read once. Longer aligned rows take
// one statistics pass that merges per-chunk (count, mean, M2) triples
// (Chan et al.'s pairwise variance update, as stable as two passes) and a
// second pass that writes; unaligned rows take three element-wise passes.
// Variants differ only in GROUP and CHUNKS: fewer chunks use fewer
// registers and keep more rows in flight. Argument order is the pack ABI of
// transformer.py:323-371.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 8;  // halves per 16-byte access

template <int GROUP>
__device__ __forceinline__ float GroupSum(float v) {
#pragma unroll
  for (int offset = GROUP / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

// Running statistics of a set of values: count, mean, sum of squared
// deviations from the mean.
struct Moments {
  float n, mean, m2;
};

// Chan, Golub and LeVeque's update for the union of two disjoint sets.
__device__ __forceinline__ Moments Merge(Moments a, Moments b) {
  const float n = a.n + b.n;
  if (n == 0.0f) return a;
  const float delta = b.mean - a.mean;
  const float wb = b.n / n;
  return {n, a.mean + delta * wb, a.m2 + b.m2 + delta * delta * a.n * wb};
}

template <int GROUP>
__device__ __forceinline__ Moments GroupMerge(Moments v) {
#pragma unroll
  for (int offset = GROUP / 2; offset > 0; offset >>= 1) {
    const Moments other{__shfl_xor(v.n, offset, 64), __shfl_xor(v.mean, offset, 64), __shfl_xor(v.m2, offset, 64)};
    v = Merge(v, other);
  }
  return v;
}

template <int GROUP, int CHUNKS, bool SKIP>
__device__ __forceinline__ void LayerNormRow(const _Float16* __restrict__ x, const _Float16* __restrict__ residual,
                                             const _Float16* __restrict__ gamma, const _Float16* __restrict__ beta,
                                             _Float16* __restrict__ output, int rows, int columns, float epsilon) {
  static_assert(GROUP == 16 || GROUP == 32 || GROUP == 64, "a row group is 16, 32 or 64 lanes");
  constexpr int kRowsPerWave = 64 / GROUP;
  constexpr int kRowsPerBlock = (kThreads / 64) * kRowsPerWave;
  constexpr int kCachedColumns = GROUP * kChunk * CHUNKS;
  const int lane = threadIdx.x & 63;
  const int sub = lane % GROUP;
  const int row = blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6) * kRowsPerWave + lane / GROUP;
  // Whole groups leave together; the shuffles below stay inside a group.
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
    float v[CHUNKS][kChunk];
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
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
    const float mean = GroupSum<GROUP>(sum) * inv_columns;
    float sq = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
      if (col < columns) {
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          v[c][e] -= mean;
          sq += v[c][e] * v[c][e];
        }
      }
    }
    const float rstd = rsqrtf(GroupSum<GROUP>(sq) * inv_columns + epsilon);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
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

  const bool aligned = (columns % kChunk) == 0 &&
                       ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(output) |
                         reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta) |
                         (SKIP ? reinterpret_cast<uintptr_t>(residual) : 0)) & 15) == 0;
  auto load = [&](int col, float (&v)[kChunk]) {
    const ct::f16x8 a = *reinterpret_cast<const ct::f16x8*>(xr + col);
    ct::f16x8 b;
    if (SKIP) b = *reinterpret_cast<const ct::f16x8*>(rr + col);
#pragma unroll
    for (int e = 0; e < kChunk; ++e) v[e] = static_cast<float>(a[e]) + (SKIP ? static_cast<float>(b[e]) : 0.0f);
  };
  if (aligned) {
    // Long rows: statistics in one pass over 16-byte chunks, then the write.
    Moments acc{0.0f, 0.0f, 0.0f};
    for (int col = sub * kChunk; col < columns; col += GROUP * kChunk) {
      float v[kChunk];
      load(col, v);
      float chunk_sum = 0.0f;
#pragma unroll
      for (int e = 0; e < kChunk; ++e) chunk_sum += v[e];
      const float chunk_mean = chunk_sum * (1.0f / kChunk);
      float chunk_m2 = 0.0f;
#pragma unroll
      for (int e = 0; e < kChunk; ++e) chunk_m2 += (v[e] - chunk_mean) * (v[e] - chunk_mean);
      acc = Merge(acc, Moments{static_cast<float>(kChunk), chunk_mean, chunk_m2});
    }
    const Moments row_moments = GroupMerge<GROUP>(acc);
    const float mean = row_moments.mean;
    const float rstd = rsqrtf(row_moments.m2 * inv_columns + epsilon);
    for (int col = sub * kChunk; col < columns; col += GROUP * kChunk) {
      float v[kChunk];
      load(col, v);
      const ct::f16x8 g = *reinterpret_cast<const ct::f16x8*>(gamma + col);
      const ct::f16x8 bt = *reinterpret_cast<const ct::f16x8*>(beta + col);
      ct::f16x8 y;
#pragma unroll
      for (int e = 0; e < kChunk; ++e) {
        y[e] = static_cast<_Float16>((v[e] - mean) * rstd * static_cast<float>(g[e]) + static_cast<float>(bt[e]));
      }
      *reinterpret_cast<ct::f16x8*>(yr + col) = y;
    }
    return;
  }

  // Unaligned rows: element-strided, three passes over global memory.
  auto value = [&](int col) {
    return static_cast<float>(xr[col]) + (SKIP ? static_cast<float>(rr[col]) : 0.0f);
  };
  float sum = 0.0f;
  for (int col = sub; col < columns; col += GROUP) sum += value(col);
  const float mean = GroupSum<GROUP>(sum) * inv_columns;
  float sq = 0.0f;
  for (int col = sub; col < columns; col += GROUP) {
    const float d = value(col) - mean;
    sq += d * d;
  }
  const float rstd = rsqrtf(GroupSum<GROUP>(sq) * inv_columns + epsilon);
  for (int col = sub; col < columns; col += GROUP) {
    yr[col] = static_cast<_Float16>((value(col) - mean) * rstd * static_cast<float>(gamma[col]) +
                                    static_cast<float>(beta[col]));
  }
}

}  // namespace

#define CT_DEFINE_LAYER_NORM(NAME, GROUP, CHUNKS)                                                                   \
  CT_KERNEL void __launch_bounds__(kThreads)                                                                       \
      layer_norm_fp16_##NAME(const _Float16* x, const _Float16* scale, const _Float16* bias, _Float16* output,      \
                             int rows, int columns, float epsilon, void*, void*) {                                 \
    LayerNormRow<GROUP, CHUNKS, false>(x, nullptr, scale, bias, output, rows, columns, epsilon);                    \
  }                                                                                                                \
  CT_KERNEL void __launch_bounds__(kThreads)                                                                       \
      skip_layer_norm_fp16_##NAME(const _Float16* x, const _Float16* residual, const _Float16* scale,              \
                                  const _Float16* bias, _Float16* output, int rows, int columns, float epsilon,    \
                                  void*, void*) {                                                                  \
    LayerNormRow<GROUP, CHUNKS, true>(x, residual, scale, bias, output, rows, columns, epsilon);                   \
  }

// NAME: lanes per row (g) and 16-byte chunks per lane (c); rows of up to
// g * 8 * c columns stay in registers.
CT_DEFINE_LAYER_NORM(g16c1, 16, 1)
CT_DEFINE_LAYER_NORM(g32c1, 32, 1)
CT_DEFINE_LAYER_NORM(g64c1, 64, 1)
CT_DEFINE_LAYER_NORM(g64c2, 64, 2)
CT_DEFINE_LAYER_NORM(g64c4, 64, 4)
CT_DEFINE_LAYER_NORM(g64c8, 64, 8)
