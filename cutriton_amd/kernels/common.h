// Shared device helpers for the gfx950 kernel families.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CT_KERNEL extern "C" __global__

namespace ct {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Number of XCDs on MI355X. Workgroups are dispatched round-robin over the
// XCDs, each of which owns a private L2.
constexpr int kXcdCount = 8;

// Maps the hardware dispatch index to a tile index such that the workgroups
// resident on one XCD receive a contiguous range of tiles (neighbouring tiles
// share operand rows/columns, which then stay in that XCD's L2). A bijection
// on [0, total) for every total.
__device__ __forceinline__ int XcdContiguousIndex(int linear, int total) {
  const int per = total / kXcdCount;
  const int extra = total % kXcdCount;
  const int xcd = linear % kXcdCount;
  const int slot = linear / kXcdCount;
  return xcd * per + (xcd < extra ? xcd : extra) + slot;
}

__device__ __forceinline__ float WaveSum(float v) {
  // Butterfly over the 64 lanes of a wavefront.
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

__device__ __forceinline__ float WaveMax(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
  return v;
}

// erf-GELU in FP32: 0.5 * a * (1 + erf(a / sqrt(2))), with ROCm's erff.
__device__ __forceinline__ float GeluErf(float a) {
  return 0.5f * a * (1.0f + erff(a * 0.7071067811865476f));
}

}  // namespace ct
