// MaxPool and GlobalAveragePool (FP32, NCHW): bandwidth kernels.
//
// Semantics follow python/cutriton/triton_kernels/resnet.py:
//   max_pool (159-182): max over the dilated window; positions outside the
//     image read as -inf (so padding never wins);
//   global_average_pool (185-198): sum over H*W in increasing spatial order,
//     then divide by H*W.
// Argument order is the pack ABI of resnet.py:341-379 with two trailing
// reserved pointers.
#include <type_traits>

#include "common.h"

namespace {

constexpr int kThreads = 256;

}  // namespace

// Window maximum as the reference's tl.maximum(accumulator, value) with an
// accumulator that starts at -inf: a NaN value never wins (maxNum), so a
// window of NaNs gives -inf, and of two zeros +0 is the larger (IEEE 754-2019
// maximumNumber; the reference leaves the sign of that tie unspecified).
// gfx950's v_max_f32 gives exactly that for a non-NaN accumulator: quiet and
// signalling NaN operands lose to any number, and max(-0, +0) = +0 in either
// operand order.
__device__ __forceinline__ float MaxNumber(float best, float v) { return __builtin_fmaxf(best, v); }

// The output is cut into bands: BAND output rows of one (image, channel)
// plane, numbered plane-major. A workgroup pools GROUP_BANDS consecutive
// bands. The input rows a band's windows read are one contiguous span of its
// plane: every thread issues all its 16-byte loads of the next band's span
// before it pools the current band from LDS, so the loads stream while the
// workgroup computes. Rows outside the image are stored as -inf. For a
// horizontal stride of 2 each LDS row holds the odd input columns, then the
// even ones, so neighbouring lanes (neighbouring outputs) read neighbouring
// words for every kernel column. A band's outputs are one contiguous span of
// the output plane. Grid: ceil(planes * ceil(out_h / BAND) / GROUP_BANDS).
// Bands too tall for LDS (large strides or dilations), or whose rows are not
// whole 16-byte chunks, read their windows from global memory instead.
namespace {

template <int BAND, int LDS_FLOATS, int GROUP_BANDS>
__device__ __forceinline__ void MaxPoolBands(const float* __restrict__ x, float* __restrict__ output, int n, int c,
                                             int h, int w, int out_h, int out_w, int kernel_h, int kernel_w,
                                             int stride_h, int stride_w, int pad_h, int pad_w, int dilation_h,
                                             int dilation_w) {
  constexpr int kChunksPerThread = LDS_FLOATS / 4 / kThreads;  // 16-byte loads per thread, at most
  static_assert(kChunksPerThread * 4 * kThreads == LDS_FLOATS, "whole rounds of 16-byte loads");
  __shared__ __attribute__((aligned(16))) float tile[LDS_FLOATS];
  const int bands_per_plane = (out_h + BAND - 1) / BAND;
  const int64_t bands = static_cast<int64_t>(n) * c * bands_per_plane;
  const int64_t band_begin = static_cast<int64_t>(blockIdx.x) * GROUP_BANDS;
  const int count = static_cast<int>(min(static_cast<int64_t>(GROUP_BANDS), bands - band_begin));
  if (count <= 0) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const float neg_inf = -__builtin_huge_valf();
  const int half = w >> 1;
  // LDS row: 4 floats of lead, then the row's w values, then 4 floats; the
  // words just before and just after the values hold -inf, so a window
  // column one step outside the image (iw = -1 or iw = w) reads -inf.
  const int rs = w + 8;
  const int full_rows_in = (BAND - 1) * stride_h + (kernel_h - 1) * dilation_h + 1;
  const bool staged = (w & 3) == 0 && full_rows_in * rs <= LDS_FLOATS;
  const bool split = staged && stride_w == 2;
  const bool guarded = pad_w <= 1 && (out_w - 1) * stride_w - pad_w + (kernel_w - 1) * dilation_w <= w;

  struct Band {
    const float* src;  // the plane's input
    float* dst;        // the band's first output
    int rows_out, ih0, rows_in, first, chunks;
  };
  auto band_at = [&](int k) {
    const int64_t b = band_begin + k;
    const int64_t plane = b / bands_per_plane;
    const int oh0 = static_cast<int>(b - plane * bands_per_plane) * BAND;
    Band g;
    g.src = x + plane * h * w;
    g.dst = output + (plane * out_h + oh0) * out_w;
    g.rows_out = min(BAND, out_h - oh0);
    g.ih0 = oh0 * stride_h - pad_h;
    g.rows_in = (g.rows_out - 1) * stride_h + (kernel_h - 1) * dilation_h + 1;
    g.first = max(g.ih0, 0);
    const int last = min(g.ih0 + g.rows_in, h);  // exclusive
    g.chunks = max(last - g.first, 0) * (w >> 2);
    return g;
  };
  // Unconditional loads (a thread past the span re-reads its last chunk), so
  // that all of them are in flight before the first wait.
  ct::f32x4 v[kChunksPerThread];
  auto issue_loads = [&](const Band& g) {
    const ct::f32x4* from = reinterpret_cast<const ct::f32x4*>(g.src + static_cast<int64_t>(g.first) * w);
    const int last_chunk = max(g.chunks - 1, 0);
#pragma unroll
    for (int k = 0; g.chunks > 0 && k < kChunksPerThread; ++k) v[k] = from[min(tid + k * kThreads, last_chunk)];
  };
  auto fill_tile = [&](const Band& g) {
    const int row0 = g.first - g.ih0;  // tile row of the span's first row
#pragma unroll
    for (int k = 0; k < kChunksPerThread; ++k) {
      const int i = tid + k * kThreads;
      if (i >= g.chunks) continue;
      const int at = 4 * i;  // float offset in the span; chunks never straddle rows
      const int r = row0 + at / w;
      const int col = at - (at / w) * w;
      float* row = tile + r * rs + 4;
      if (split) {  // odd columns first, then even ones
        *reinterpret_cast<ct::f32x2*>(row + (col >> 1)) = {v[k][1], v[k][3]};
        *reinterpret_cast<ct::f32x2*>(row + half + (col >> 1)) = {v[k][0], v[k][2]};
      } else {
        *reinterpret_cast<ct::f32x4*>(row + col) = v[k];
      }
    }
    // The guard words of every row, and whole rows above or below the image,
    // read as -inf.
    for (int r = tid; r < g.rows_in; r += kThreads) {
      tile[r * rs + 3] = neg_inf;
      tile[r * rs + 4 + w] = neg_inf;
    }
    for (int r = 0; r < g.rows_in; ++r) {
      const int ih = g.ih0 + r;
      if (static_cast<unsigned>(ih) < static_cast<unsigned>(h)) continue;
      for (int col = tid; col < w; col += kThreads) tile[r * rs + 4 + col] = neg_inf;
    }
  };
  // Staged windows: every window row is a tile row (rows outside the image
  // hold -inf). When no window column lies more than one step outside the
  // image, the guard words stand in for the outside columns; otherwise an
  // outside column is replaced by -inf after an in-bounds read. A wavefront
  // takes whole output rows, lanes along the row; with the 3 x 3 window
  // (compile-time bounds) the nine reads of an output are issued together.
  // Each source is its own instantiation: behind one pointer that may be
  // either, the LDS reads would compile to generic (FLAT) loads.
  auto pool_staged = [&](const Band& g, auto kh_count, auto kw_count, auto tile_index, auto guard) {
    for (int r = wave; r < g.rows_out; r += kThreads / 64) {
      for (int ow = lane; ow < out_w; ow += 64) {
        float best = neg_inf;
#pragma unroll
        for (int kh = 0; kh < kh_count; ++kh) {
          const float* row = tile + (r * stride_h + kh * dilation_h) * rs + 4;
#pragma unroll
          for (int kw = 0; kw < kw_count; ++kw) {
            const int iw = ow * stride_w - pad_w + kw * dilation_w;
            if constexpr (decltype(guard)::value) {
              best = MaxNumber(best, row[tile_index(iw)]);
            } else {
              const bool inside = static_cast<unsigned>(iw) < static_cast<unsigned>(w);
              const float value = row[tile_index(inside ? iw : 0)];
              best = MaxNumber(best, inside ? value : neg_inf);
            }
          }
        }
        g.dst[r * out_w + ow] = best;
      }
    }
  };
  auto pool_tile = [&](const Band& g, auto tile_index) {
    if (kernel_h == 3 && kernel_w == 3 && guarded) {
      pool_staged(g, std::integral_constant<int, 3>(), std::integral_constant<int, 3>(), tile_index,
                  std::true_type());
    } else {
      pool_staged(g, kernel_h, kernel_w, tile_index, std::false_type());
    }
  };
  auto pool_global = [&](const Band& g) {
    const int total = g.rows_out * out_w;
    for (int idx = tid; idx < total; idx += kThreads) {
      const int r = idx / out_w;
      const int ow = idx - r * out_w;
      float best = neg_inf;
      for (int kh = 0; kh < kernel_h; ++kh) {
        const int ih = g.ih0 + r * stride_h + kh * dilation_h;
        if (static_cast<unsigned>(ih) >= static_cast<unsigned>(h)) continue;
        for (int kw = 0; kw < kernel_w; ++kw) {
          const int iw = ow * stride_w - pad_w + kw * dilation_w;
          if (static_cast<unsigned>(iw) < static_cast<unsigned>(w)) {
            best = MaxNumber(best, g.src[static_cast<int64_t>(ih) * w + iw]);
          }
        }
      }
      g.dst[idx] = best;
    }
  };

  if (!staged) {
    for (int k = 0; k < count; ++k) pool_global(band_at(k));
    return;
  }
  Band cur = band_at(0);
  issue_loads(cur);
  for (int k = 0; k < count; ++k) {
    fill_tile(cur);  // waits for this band's loads
    __syncthreads();
    const Band next = k + 1 < count ? band_at(k + 1) : cur;
    if (k + 1 < count) issue_loads(next);
    if (split) {
      // Odd column iw at (iw >> 1), even column at half + (iw >> 1): iw = -1
      // lands on the guard before the row, iw = w on the guard after it.
      pool_tile(cur, [&](int iw) { return ((iw & 1) ? 0 : half) + (iw >> 1); });
    } else {
      pool_tile(cur, [&](int iw) { return iw; });
    }
    __syncthreads();  // the tile is free for the next band
    cur = next;
  }
}

}  // namespace

// Direct 3 x 3, stride-2 pooling with one pixel of padding on the top and
// left (the ResNet-50 stem pool), rows of w = 4k <= 128 floats and
// out_w = w / 2: no LDS and no barrier. A half-wavefront (32 lanes) pools one
// band of 8 output rows of one plane; lane j reads input columns 4j..4j+3 of
// the band's 17 input rows (one 16-byte load each, all issued before the
// first use) and writes outputs 2j and 2j + 1 of every row. Column 4j - 1
// comes from lane j - 1 (-inf for j = 0); rows outside the image are -inf.
// Each row's two column maxima serve the two output rows that read it. The
// maximum of a set does not depend on the order it is taken in (v_max_f32:
// NaN never wins against a number, +0 above -0); the final max with -inf
// turns an all-NaN window into -inf, as the reference's -inf accumulator
// does. Returns false, doing nothing, when the shape is not of this form.
namespace {

constexpr int kDirectBand = 8;
constexpr int kDirectRows = 2 * kDirectBand + 1;

template <int GROUP_BANDS>
__device__ __forceinline__ bool MaxPoolDirect3x3s2(const float* __restrict__ x, float* __restrict__ output, int n,
                                                   int c, int h, int w, int out_h, int out_w, int kernel_h,
                                                   int kernel_w, int stride_h, int stride_w, int pad_h, int pad_w,
                                                   int dilation_h, int dilation_w) {
  static_assert(GROUP_BANDS == 2 * kThreads / 64, "one band per half-wavefront");
  if (kernel_h != 3 || kernel_w != 3 || stride_h != 2 || stride_w != 2 || pad_h != 1 || pad_w != 1 ||
      dilation_h != 1 || dilation_w != 1 || (w & 3) != 0 || w > 128 || out_w * 2 != w) {
    return false;
  }
  const int tid = threadIdx.x;
  const int j = tid & 31;  // lane in the half-wavefront
  const int bands_per_plane = (out_h + kDirectBand - 1) / kDirectBand;
  const int64_t band = static_cast<int64_t>(blockIdx.x) * GROUP_BANDS + (tid >> 5);
  if (band >= static_cast<int64_t>(n) * c * bands_per_plane) return true;
  const int64_t plane = band / bands_per_plane;
  const int oh0 = static_cast<int>(band - plane * bands_per_plane) * kDirectBand;
  const int ih0 = 2 * oh0 - 1;
  const bool lane_on = j < (w >> 2);
  const float* src = x + plane * h * w + 4 * min(j, (w >> 2) - 1);
  const float neg_inf = -__builtin_huge_valf();
  ct::f32x4 row[kDirectRows];
#pragma unroll
  for (int r = 0; r < kDirectRows; ++r) {
    const int ih = min(max(ih0 + r, 0), h - 1);  // in bounds; rows outside are replaced below
    row[r] = *reinterpret_cast<const ct::f32x4*>(src + static_cast<int64_t>(ih) * w);
  }
  float left[kDirectRows];  // max over columns 4j-1, 4j, 4j+1
  float right[kDirectRows]; // max over columns 4j+1, 4j+2, 4j+3
#pragma unroll
  for (int r = 0; r < kDirectRows; ++r) {
    const bool inside = static_cast<unsigned>(ih0 + r) < static_cast<unsigned>(h);
    const float before = __shfl_up(row[r][3], 1, 32);
    const float col_m1 = (j == 0 || !inside) ? neg_inf : before;
    const float a = inside ? row[r][0] : neg_inf;
    const float b = inside ? row[r][1] : neg_inf;
    const float cc = inside ? row[r][2] : neg_inf;
    const float d = inside ? row[r][3] : neg_inf;
    left[r] = __builtin_fmaxf(__builtin_fmaxf(col_m1, a), b);
    right[r] = __builtin_fmaxf(__builtin_fmaxf(b, cc), d);
  }
  if (!lane_on) return true;
  float* dst = output + (plane * out_h + oh0) * out_w + 2 * j;
  const int rows_out = min(kDirectBand, out_h - oh0);
#pragma unroll
  for (int i = 0; i < kDirectBand; ++i) {
    if (i >= rows_out) break;
    const float o0 = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(left[2 * i], left[2 * i + 1]), left[2 * i + 2]),
                                     neg_inf);
    const float o1 = __builtin_fmaxf(
        __builtin_fmaxf(__builtin_fmaxf(right[2 * i], right[2 * i + 1]), right[2 * i + 2]), neg_inf);
    *reinterpret_cast<ct::f32x2*>(dst + static_cast<int64_t>(i) * out_w) = {o0, o1};
  }
  return true;
}

}  // namespace

// The direct path where the shape allows it, else bands of 8 rows, 8 bands per
// workgroup (the same grid).
CT_KERNEL void __launch_bounds__(kThreads)
    max_pool_fp32_nchw_d8(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h, int w,
                          int out_h, int out_w, int kernel_h, int kernel_w, int stride_h, int stride_w, int pad_h,
                          int pad_w, int dilation_h, int dilation_w, void*, void*) {
  if (MaxPoolDirect3x3s2<8>(x, output, n, c, h, w, out_h, out_w, kernel_h, kernel_w, stride_h, stride_w, pad_h,
                            pad_w, dilation_h, dilation_w)) {
    return;
  }
  MaxPoolBands<kDirectBand, 4096, 8>(x, output, n, c, h, w, out_h, out_w, kernel_h, kernel_w, stride_h, stride_w,
                                     pad_h, pad_w, dilation_h, dilation_w);
}

#define CT_DEFINE_MAX_POOL(NAME, BAND, LDS_FLOATS, GROUP_BANDS)                                            \
  CT_KERNEL void __launch_bounds__(kThreads)                                                                  \
      NAME(const float* __restrict__ x, float* __restrict__ output, int n, int c, int h, int w, int out_h,     \
           int out_w, int kernel_h, int kernel_w, int stride_h, int stride_w, int pad_h, int pad_w,            \
           int dilation_h, int dilation_w, void*, void*) {                                                    \
    MaxPoolBands<BAND, LDS_FLOATS, GROUP_BANDS>(x, output, n, c, h, w, out_h, out_w, kernel_h, kernel_w,      \
                                                stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w);    \
  }

// symbol, output rows per band, LDS floats, bands per workgroup
CT_DEFINE_MAX_POOL(max_pool_fp32_nchw, 8, 4096, 1)
CT_DEFINE_MAX_POOL(max_pool_fp32_nchw_b16g4, 16, 4096, 4)

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
  if (staged && count > 0) {
    // All of a lane's loads are issued before its first LDS store (a lane
    // past the span re-reads the span's last element), so the span costs
    // one memory latency.
    const float* src = x + first * spatial;
    const int total = count * spatial;
    constexpr int kPerLane = kPlanes * kMaxSpan / 64;
    float v[kPerLane];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) v[j] = src[min(lane + 64 * j, max(total - 1, 0))];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j)
      if (lane + 64 * j < total) span[wave][lane + 64 * j] = v[j];
  }
  __syncthreads();
  // Unrolled so that eight reads are in flight; the adds stay in increasing
  // spatial order. The LDS and global sources are separate loops: behind
  // one pointer that may be either, the LDS reads compile to generic (FLAT)
  // loads.
  auto plane_sum = [&](const auto* mine) {
    float sum = 0.0f;
#pragma unroll 8
    for (int i = 0; i < spatial; ++i) sum += mine[i];
    return sum;
  };
  if (lane < count) {
    const float sum = staged ? plane_sum(&span[wave][lane * spatial]) : plane_sum(x + (first + lane) * spatial);
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
