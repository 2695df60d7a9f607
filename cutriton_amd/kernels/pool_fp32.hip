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

// A workgroup takes one (image, channel) plane and a band of BAND output
// rows. The input rows the band's windows read are copied once into LDS (one
// contiguous span, 16 bytes per lane), rows outside the image as -inf; each
// output is then the max over its window read from LDS, kernel row outer,
// kernel column inner, skipping columns outside the image. Grid:
// planes * ceil(out_h / BAND). A band too tall for LDS (large strides or
// dilations) reads its windows from global memory instead. (Bands of 16 and
// 28 rows were measured on the ResNet-50 stem pool and were no faster.)
namespace {

template <int BAND, int LDS_FLOATS>
__device__ __forceinline__ void MaxPoolBand(const float* __restrict__ x, float* __restrict__ output, int n, int c,
                                            int h, int w, int out_h, int out_w, int kernel_h, int kernel_w,
                                            int stride_h, int stride_w, int pad_h, int pad_w, int dilation_h,
                                            int dilation_w) {
  constexpr int kBand = BAND;
  constexpr int kPoolLds = LDS_FLOATS;
  __shared__ __attribute__((aligned(16))) float tile[kPoolLds];
  const int bands = (out_h + kBand - 1) / kBand;
  const int plane = blockIdx.x / bands;
  const int band = blockIdx.x - plane * bands;
  if (plane >= n * c) return;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int oh0 = band * kBand;
  const int rows_out = min(kBand, out_h - oh0);
  const int ih0 = oh0 * stride_h - pad_h;
  const int rows_in = (rows_out - 1) * stride_h + (kernel_h - 1) * dilation_h + 1;
  const bool staged = rows_in * w <= kPoolLds;
  const float* src = x + static_cast<int64_t>(plane) * h * w;
  float* dst = output + static_cast<int64_t>(plane) * out_h * out_w;
  const float neg_inf = -__builtin_huge_valf();
  if (staged) {
    // The band's rows inside the image are one contiguous span of the
    // plane: copied flat, 16 bytes per lane when rows are whole float4s.
    const int first = max(ih0, 0);
    const int last = min(ih0 + rows_in, h);  // exclusive
    const int span = max(last - first, 0) * w;
    float* to = tile + (first - ih0) * w;
    const float* from = src + static_cast<int64_t>(first) * w;
    if ((w & 3) == 0) {
      const int span4 = span >> 2;
      for (int i = threadIdx.x; i < span4; i += kThreads) {
        reinterpret_cast<ct::f32x4*>(to)[i] = reinterpret_cast<const ct::f32x4*>(from)[i];
      }
    } else {
      for (int i = threadIdx.x; i < span; i += kThreads) to[i] = from[i];
    }
    // Rows above or below the image read as -inf.
    for (int r = wave; r < rows_in; r += kThreads / 64) {
      const int ih = ih0 + r;
      if (static_cast<unsigned>(ih) < static_cast<unsigned>(h)) continue;
      for (int col = lane; col < w; col += 64) tile[r * w + col] = neg_inf;
    }
    __syncthreads();
  }
  // The two sources are separate instantiations: behind one pointer that may
  // be either, the staged reads would compile to generic (FLAT) loads
  // instead of LDS reads.
  auto pool_rows = [&](auto input_row) {
    for (int r = wave; r < rows_out; r += kThreads / 64) {
      const int oh = oh0 + r;
      for (int ow = lane; ow < out_w; ow += 64) {
        float best = neg_inf;
        for (int kh = 0; kh < kernel_h; ++kh) {
          const int ih = oh * stride_h - pad_h + kh * dilation_h;
          if (static_cast<unsigned>(ih) >= static_cast<unsigned>(h)) continue;
          const float* line = input_row(ih);
          for (int kw = 0; kw < kernel_w; ++kw) {
            const int iw = ow * stride_w - pad_w + kw * dilation_w;
            if (static_cast<unsigned>(iw) < static_cast<unsigned>(w)) best = fmaxf(best, line[iw]);
          }
        }
        dst[static_cast<int64_t>(oh) * out_w + ow] = best;
      }
    }
  };
  if (staged) {
    pool_rows([&](int ih) { return tile + (ih - ih0) * w; });
  } else {
    pool_rows([&](int ih) { return src + static_cast<int64_t>(ih) * w; });
  }
}

}  // namespace

#define CT_DEFINE_MAX_POOL(NAME, BAND, LDS_FLOATS)                                                          \
  CT_KERNEL void __launch_bounds__(kThreads)                                                                \
      NAME(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h, int w, int out_h,   \
           int out_w, int kernel_h, int kernel_w, int stride_h, int stride_w, int pad_h, int pad_w,          \
           int dilation_h, int dilation_w, void*, void*) {                                                  \
    MaxPoolBand<BAND, LDS_FLOATS>(x, output, n, c, h, w, out_h, out_w, kernel_h, kernel_w, stride_h,        \
                                  stride_w, pad_h, pad_w, dilation_h, dilation_w);                          \
  }

// symbol, output rows per workgroup, LDS floats
CT_DEFINE_MAX_POOL(max_pool_fp32_nchw, 8, 4096)

// One wavefront reduces PLANES consecutive (image, channel) planes. When a
// plane holds at most 64 pixels the wave's planes are one contiguous span: it
// is copied coalesced into LDS and each lane then sums its own plane in
// increasing pixel order. Larger planes are summed by one lane directly.
// Fewer planes per wavefront give more wavefronts for the same tensor (the
// 7x7 planes of ResNet-50: 1024 wavefronts at 64 planes, one per SIMD).
namespace {

template <int PLANES>
__device__ __forceinline__ void GlobalAveragePoolPlanes(const float* __restrict__ x, float* __restrict__ output,
                                                        int n, int c, int h, int w) {
  constexpr int kPlanes = PLANES;
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

}  // namespace

#define CT_DEFINE_GAP(NAME, PLANES)                                                                      \
  CT_KERNEL void __launch_bounds__(kThreads)                                                             \
      NAME(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h, int w, void*,     \
           void*) {                                                                                      \
    GlobalAveragePoolPlanes<PLANES>(x, output, n, c, h, w);                                              \
  }

// symbol, planes per wavefront
CT_DEFINE_GAP(global_average_pool_fp32_nchw, 64)
CT_DEFINE_GAP(global_average_pool_fp32_nchw_p16, 16)
