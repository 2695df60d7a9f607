// Elementwise bandwidth kernels: the unfused decomposition steps of the fused
// ops (FP32 BatchNormalization, Relu, Add, AddRelu; FP16 Gelu, Add).
//
// Semantics follow the reference kernels:
//   resnet.py:117-130 batch_norm: channel = (i / spatial) % channels,
//     y = (x - mean[ch]) * rsqrt(var[ch] + eps) * scale[ch] + bias[ch];
//   resnet.py:133-156 relu, add, add_relu;
//   transformer.py:110-116 gelu_fp16 (FP32 erf-GELU of the widened input,
//     rounded to FP16); transformer.py:119-125 add_fp16 (FP16 add).
// Argument order is the pack ABI of resnet.py:279-338 and
// transformer.py:295-320, with two trailing reserved pointers.
//
// Each thread handles kVec consecutive elements with one 16-byte access
// when the pointers allow it, so a launch covers ceil(total / (256*kVec))
// workgroups.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kVecF32 = 4;
constexpr int kVecF16 = 8;

__device__ __forceinline__ bool Aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename Op>
__device__ __forceinline__ void MapF32(const float* __restrict__ a, const float* __restrict__ b,
                                       float* __restrict__ out, int total, Op op) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kVecF32;
  if (base >= total) return;
  const bool vec = base + kVecF32 <= total && Aligned16(a + base) && Aligned16(out + base) &&
                   (b == nullptr || Aligned16(b + base));
  if (vec) {
    const ct::f32x4 va = *reinterpret_cast<const ct::f32x4*>(a + base);
    ct::f32x4 vb = {0.0f, 0.0f, 0.0f, 0.0f};
    if (b != nullptr) vb = *reinterpret_cast<const ct::f32x4*>(b + base);
    ct::f32x4 r;
#pragma unroll
    for (int e = 0; e < kVecF32; ++e) r[e] = op(va[e], vb[e], base + e);
    *reinterpret_cast<ct::f32x4*>(out + base) = r;
  } else {
    for (int64_t i = base; i < total && i < base + kVecF32; ++i) out[i] = op(a[i], b == nullptr ? 0.0f : b[i], i);
  }
}

}  // namespace

CT_KERNEL void __launch_bounds__(kThreads)
    relu_fp32(const float* x, float* output, int total, void*, void*) {
  MapF32(x, nullptr, output, total, [](float v, float, int64_t) { return fmaxf(v, 0.0f); });
}

CT_KERNEL void __launch_bounds__(kThreads)
    add_fp32(const float* a, const float* b, float* output, int total, void*, void*) {
  MapF32(a, b, output, total, [](float u, float v, int64_t) { return u + v; });
}

CT_KERNEL void __launch_bounds__(kThreads)
    add_relu_fp32(const float* a, const float* b, float* output, int total, void*, void*) {
  MapF32(a, b, output, total, [](float u, float v, int64_t) { return fmaxf(u + v, 0.0f); });
}

CT_KERNEL void __launch_bounds__(kThreads)
    batch_norm_fp32_nchw(const float* x, const float* scale, const float* bias, const float* mean,
                         const float* variance, float* output, int total, int channels, int spatial, float epsilon,
                         void*, void*) {
  MapF32(x, nullptr, output, total, [=](float v, float, int64_t i) {
    const int ch = static_cast<int>((i / spatial) % channels);
    return (v - mean[ch]) * rsqrtf(variance[ch] + epsilon) * scale[ch] + bias[ch];
  });
}

CT_KERNEL void __launch_bounds__(kThreads)
    gelu_fp16(const _Float16* x, _Float16* output, int total, void*, void*) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kVecF16;
  if (base >= total) return;
  if (base + kVecF16 <= total && Aligned16(x + base) && Aligned16(output + base)) {
    const ct::f16x8 v = *reinterpret_cast<const ct::f16x8*>(x + base);
    ct::f16x8 r;
#pragma unroll
    for (int e = 0; e < kVecF16; ++e) r[e] = static_cast<_Float16>(ct::GeluErf(static_cast<float>(v[e])));
    *reinterpret_cast<ct::f16x8*>(output + base) = r;
  } else {
    for (int64_t i = base; i < total && i < base + kVecF16; ++i) {
      output[i] = static_cast<_Float16>(ct::GeluErf(static_cast<float>(x[i])));
    }
  }
}

CT_KERNEL void __launch_bounds__(kThreads)
    add_fp16(const _Float16* a, const _Float16* b, _Float16* output, int total, void*, void*) {
  const int64_t base = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * kVecF16;
  if (base >= total) return;
  if (base + kVecF16 <= total && Aligned16(a + base) && Aligned16(b + base) && Aligned16(output + base)) {
    const ct::f16x8 u = *reinterpret_cast<const ct::f16x8*>(a + base);
    const ct::f16x8 v = *reinterpret_cast<const ct::f16x8*>(b + base);
    *reinterpret_cast<ct::f16x8*>(output + base) = u + v;
  } else {
    for (int64_t i = base; i < total && i < base + kVecF16; ++i) output[i] = a[i] + b[i];
  }
}
