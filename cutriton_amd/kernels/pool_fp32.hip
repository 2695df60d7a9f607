// MaxPool and GlobalAveragePool (FP32, NCHW): bandwidth kernels.
//
// Semantics follow python/cutriton/triton_kernels/resnet.py:
//   max_pool (159-182): max over the dilated window; positions outside the
//     image read as -inf (so padding never wins);
//   global_average_pool (185-198): sum over H*W in increasing spatial order,
//     then divide by H*W.
// Argument order is the pack ABI of resnet.py:341-379 with two trailing
// reserved pointers.
#include "common.h"

namespace {

constexpr int kThreads = 256;

}  // namespace

// One thread per output element, in output order: neighbouring lanes take
// neighbouring output columns, so each window row is a short strided run that
// the wave reads from a few cache lines.
CT_KERNEL void __launch_bounds__(kThreads)
    max_pool_fp32_nchw(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h, int w,
                       int out_h, int out_w, int kernel_h, int kernel_w, int stride_h, int stride_w, int pad_h,
                       int pad_w, int dilation_h, int dilation_w, void*, void*) {
  const int64_t total = static_cast<int64_t>(n) * c * out_h * out_w;
  const int64_t index = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (index >= total) return;
  const int ow = static_cast<int>(index % out_w);
  const int64_t rest = index / out_w;
  const int oh = static_cast<int>(rest % out_h);
  const int64_t plane = rest / out_h;  // image * C + channel
  const float* src = x + plane * h * w;
  float best = -__builtin_huge_valf();
  for (int kh = 0; kh < kernel_h; ++kh) {
    const int ih = oh * stride_h - pad_h + kh * dilation_h;
    if (static_cast<unsigned>(ih) >= static_cast<unsigned>(h)) continue;
    const float* line = src + static_cast<int64_t>(ih) * w;
    for (int kw = 0; kw < kernel_w; ++kw) {
      const int iw = ow * stride_w - pad_w + kw * dilation_w;
      if (static_cast<unsigned>(iw) < static_cast<unsigned>(w)) best = fmaxf(best, line[iw]);
    }
  }
  output[index] = best;
}

// One wavefront reduces 64 consecutive (image, channel) planes. When a plane
// holds at most 64 pixels the wave's 64 planes are one contiguous span: it is
// copied coalesced into LDS and each lane then sums its own plane in
// increasing pixel order. Larger planes are summed by one lane directly.
CT_KERNEL void __launch_bounds__(kThreads)
    global_average_pool_fp32_nchw(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h,
                                  int w, void*, void*) {
  constexpr int kPlanes = 64;
  constexpr int kMaxSpan = 64;
  __shared__ float span[kThreads / 64][kPlanes * kMaxSpan];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t planes = static_cast<int64_t>(n) * c;
  const int spatial = h * w;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * kPlanes;
  const int count = first >= planes ? 0 : static_cast<int>(planes - first < kPlanes ? planes - first : kPlanes);
  const bool staged = spatial <= kMaxSpan;
  if (staged) {
    const float* src = x + first * spatial;
    const int total = count * spatial;
    for (int i = lane; i < total; i += 64) span[wave][i] = src[i];
  }
  __syncthreads();
  if (lane < count) {
    const float* mine = staged ? &span[wave][lane * spatial] : x + (first + lane) * spatial;
    float sum = 0.0f;
    for (int i = 0; i < spatial; ++i) sum += mine[i];
    output[first + lane] = sum / static_cast<float>(spatial);
  }
}
