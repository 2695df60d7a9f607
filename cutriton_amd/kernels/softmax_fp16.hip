// Softmax over the last axis of a [rows, columns] tensor, FP16 in and out,
// FP32 arithmetic.
//
// Semantics follow python/cutriton/triton_kernels/transformer.py:180-190
// (softmax_fp16): v = fp32(x); v -= max(v); e = exp(v); y = fp16(e / sum(e)).
// A row whose entries are all -inf gives NaN, as there (-inf - -inf).
// Unlike the reference (one 1024-wide block per row, so columns <= 1024 is
// silently required) any column count works:
//   * a group of GROUP lanes owns one row (64 / GROUP rows per wavefront,
//     so short attention rows still fill the wavefront); each lane holds
//     CHUNKS 16-byte chunks of the row in registers: one read of x, one
//     write of y, two group reductions (max, then sum);
//   * rows longer than GROUP * 8 * CHUNKS columns, or not 16-byte aligned,
//     take an online pass (running max and rescaled sum per lane, merged
//     across the group) and a second pass that writes y.
// Argument order is the pack ABI of transformer.py:374-396.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kChunk = 8;  // halves per 16-byte access

template <int GROUP>
__device__ __forceinline__ float GroupMax(float v) {
#pragma unroll
  for (int offset = GROUP / 2; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
  return v;
}

template <int GROUP>
__device__ __forceinline__ float GroupSum(float v) {
#pragma unroll
  for (int offset = GROUP / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

// Adds x to a running (max m, sum s of exp(. - m)); -inf entries add 0.
__device__ __forceinline__ void OnlineAdd(float x, float& m, float& s) {
  if (x > m) {
    s = s * __expf(m - x) + 1.0f;
    m = x;
  } else {
    s += x == -INFINITY ? 0.0f : __expf(x - m);
  }
}

template <int GROUP, int CHUNKS>
__device__ __forceinline__ void SoftmaxRow(const _Float16* __restrict__ x, _Float16* __restrict__ y, int rows,
                                           int columns) {
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
  _Float16* yr = y + offset;
  const bool aligned = (columns % kChunk) == 0 &&
                       ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0;

  if (aligned && columns <= kCachedColumns) {
    float v[CHUNKS][kChunk];
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
      if (col < columns) {
        const ct::f16x8 a = *reinterpret_cast<const ct::f16x8*>(xr + col);
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          v[c][e] = static_cast<float>(a[e]);
          m = fmaxf(m, v[c][e]);
        }
      }
    }
    m = GroupMax<GROUP>(m);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
      if (col < columns) {
#pragma unroll
        for (int e = 0; e < kChunk; ++e) {
          v[c][e] = __expf(v[c][e] - m);
          s += v[c][e];
        }
      }
    }
    const float inv = 1.0f / GroupSum<GROUP>(s);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      const int col = (c * GROUP + sub) * kChunk;
      if (col < columns) {
        ct::f16x8 out;
#pragma unroll
        for (int e = 0; e < kChunk; ++e) out[e] = static_cast<_Float16>(v[c][e] * inv);
        *reinterpret_cast<ct::f16x8*>(yr + col) = out;
      }
    }
    return;
  }

  // Long or unaligned rows: online max/sum, then a second pass.
  float m = -INFINITY;
  float s = 0.0f;
  if (aligned) {
    for (int col = sub * kChunk; col < columns; col += GROUP * kChunk) {
      const ct::f16x8 a = *reinterpret_cast<const ct::f16x8*>(xr + col);
#pragma unroll
      for (int e = 0; e < kChunk; ++e) OnlineAdd(static_cast<float>(a[e]), m, s);
    }
  } else {
    for (int col = sub; col < columns; col += GROUP) OnlineAdd(static_cast<float>(xr[col]), m, s);
  }
  const float row_max = GroupMax<GROUP>(m);
  const float inv = 1.0f / GroupSum<GROUP>(m == -INFINITY ? 0.0f : s * __expf(m - row_max));
  if (aligned) {
    for (int col = sub * kChunk; col < columns; col += GROUP * kChunk) {
      const ct::f16x8 a = *reinterpret_cast<const ct::f16x8*>(xr + col);
      ct::f16x8 out;
#pragma unroll
      for (int e = 0; e < kChunk; ++e) out[e] = static_cast<_Float16>(__expf(static_cast<float>(a[e]) - row_max) * inv);
      *reinterpret_cast<ct::f16x8*>(yr + col) = out;
    }
  } else {
    for (int col = sub; col < columns; col += GROUP) {
      yr[col] = static_cast<_Float16>(__expf(static_cast<float>(xr[col]) - row_max) * inv);
    }
  }
}

}  // namespace

#define CT_DEFINE_SOFTMAX(NAME, GROUP, CHUNKS)                                                      \
  CT_KERNEL void __launch_bounds__(kThreads)                                                       \
      softmax_fp16_##NAME(const _Float16* x, _Float16* output, int rows, int columns, void*, void*) { \
    SoftmaxRow<GROUP, CHUNKS>(x, output, rows, columns);                                           \
  }

// NAME: lanes per row (g) and 16-byte chunks per lane (c); rows of up to
// g * 8 * c columns stay in registers.
CT_DEFINE_SOFTMAX(g16c1, 16, 1)
CT_DEFINE_SOFTMAX(g32c1, 32, 1)
CT_DEFINE_SOFTMAX(g64c1, 64, 1)
CT_DEFINE_SOFTMAX(g64c2, 64, 2)
CT_DEFINE_SOFTMAX(g64c4, 64, 4)
CT_DEFINE_SOFTMAX(g64c8, 64, 8)
