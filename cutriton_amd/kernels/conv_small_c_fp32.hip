// FP32 convolution with the BatchNorm / ReLU / residual-AddRelu epilogue for
// convolutions with few input channels and small kernels (C <= 4, R, S <= 7,
// so C*R*S <= 196), such as the ResNet-50 stem (C = 3, 7x7, stride 2).
//
// Semantics follow python/cutriton/triton_kernels/resnet.py:
//   fused_conv_batch_norm_relu (12-47), fused_conv_batch_norm (50-85),
//   conv (88-114); the residual-join entry applies add_relu (150-156) in the
//   epilogue. Argument order is the pack ABI of resnet.py:242-300 (the
//   residual-join entry inserts the residual after the BN vectors), with two
//   trailing reserved pointers. The weight is read as OIHW.
//
// With C*R*S this small, the implicit GEMM's depth is too shallow to tile
// like the channel-rich layers, and an im2col gather per element would cost
// more index arithmetic than MFMA work. Instead:
//   - a workgroup (4 wavefronts) computes 64 output channels of two output
//     rows of 112 output columns; wavefront w owns channels 16w..16w+15;
//   - each wavefront keeps its weights in registers for the whole kernel:
//     depth order (c, r, s), which is the OIHW row, zero-padded to a
//     multiple of 16 depths, at most 52 floats per lane;
//   - the workgroup stages the input patch of its two output rows once,
//     [C][rows_in][cols_in], zero where the window leaves the image, plus a
//     table of each depth's offset inside the patch;
// so an MFMA's weight operand is a register and its input operand one 4-byte
// LDS read per depth and 16-pixel block.
//
// MFMA: v_mfma_f32_16x16x4_f32, weights as the row operand (16 output
// channels), pixels as the column operand (16 output columns). Step e of
// depth group g gives lane quarter q depth 16g + 4q + e. Lane l ends with
// output column l % 16 and channels 4 * (l / 16) + 0..3.
//
// A patch larger than the LDS stage (large strides or dilations) is read
// from global memory instead, element by element, with the same results.
// Grid: x = images * ceil(P / 2) * ceil(Q / 112), y = ceil(K / 64).
#include "common.h"

namespace {

using ct::f32x4;

enum Epilogue : int { kPlain = 0, kBatchNorm = 1, kBatchNormRelu = 2, kBatchNormAddRelu = 3 };

constexpr int kDepthMax = 208;       // C*R*S (<= 196) rounded up to 16
constexpr int kGroupsMax = kDepthMax / 16;
#ifndef CT_SMALLC_ROWS
#define CT_SMALLC_ROWS 2
#endif
constexpr int kRows = CT_SMALLC_ROWS;  // output rows per workgroup
constexpr int kBlocks = 7;           // 16-column blocks per output row
constexpr int kCols = kBlocks * 16;  // output columns per workgroup
constexpr int kChannels = 64;        // output channels per workgroup (16 per wavefront)
constexpr int kPatchMax = 9216;      // floats of staged input
constexpr int kThreads = 256;

constexpr int kBufferFlags = 0x00020000;  // gfx9-family raw 32-bit buffer
constexpr int kNoRead = 0x80000000;       // past every resource's range: reads 0
typedef int i32x4 __attribute__((ext_vector_type(4)));


template <int EPI>
__device__ __forceinline__ void SmallCConv(const float* __restrict__ x, const float* __restrict__ weight,
                                           const float* __restrict__ scale, const float* __restrict__ bias,
                                           const float* __restrict__ mean, const float* __restrict__ variance,
                                           const float* __restrict__ residual, float* __restrict__ output,
                                           int n_imgs, int c, int h, int w, int k, int r, int s, int p, int q,
                                           int sh, int sw, int ph, int pw, int dh, int dw, float epsilon) {
  __shared__ __attribute__((aligned(16))) float patch[kPatchMax];
  __shared__ __attribute__((aligned(16))) int offsets[kDepthMax];
  __shared__ float epi_mul[kChannels];
  __shared__ float epi_add[kChannels];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int lane16 = lane & 15;
  const int quarter = lane >> 4;
  const int col_chunks = (q + kCols - 1) / kCols;
  const int row_pairs = (p + kRows - 1) / kRows;
  int linear = blockIdx.x;
  const int chunk = linear % col_chunks;
  linear /= col_chunks;
  const int pair = linear % row_pairs;
  const int img = linear / row_pairs;
  if (img >= n_imgs) return;
  const int oh0 = pair * kRows;
  const int ow0 = chunk * kCols;
  const int k0 = blockIdx.y * kChannels;

  const int rs = r * s;
  const int depth = c * rs;
  const int groups = (depth + 15) / 16;
  const int rows_in = (kRows - 1) * sh + (r - 1) * dh + 1;
  const int cols_in = (kCols - 1) * sw + (s - 1) * dw + 1;
  const int plane_in = rows_in * cols_in;
  const bool staged = c * plane_in <= kPatchMax;
  const int ih0 = oh0 * sh - ph;
  const int iw0 = ow0 * sw - pw;
  const float* x_img = x + static_cast<size_t>(img) * c * h * w;

  // ---- Weights of this lane's MFMA row (channel k0 + 16 wv + lane16) into
  // registers: element 4g + e holds depth 16g + 4q + e.
  // Raw buffer loads: an offset past the weight reads 0 (padding depths and
  // channels past k), so the 52 loads issue back to back without branches.
  const int my_k = k0 + 16 * wv + lane16;
  const __amdgpu_buffer_rsrc_t w_res =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(weight), 0, k * depth * 4, kBufferFlags);
  float wreg[4 * kGroupsMax];
#pragma unroll
  for (int g = 0; g < kGroupsMax; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d = 16 * g + 4 * quarter + e;
      const int offset = (my_k < k && d < depth) ? (my_k * depth + d) * 4 : kNoRead;
      wreg[4 * g + e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(w_res, offset, 0, 0));
    }

  // ---- Staging: depth offsets, the input patch (one patch row per
  // wavefront pass, a lane per column), the folded BatchNorm.
  for (int d = tid; d < groups * 16; d += kThreads) {
    const int ci = d / rs;
    const int rem = d - ci * rs;
    const int kr = rem / s;
    const int ks = rem - kr * s;
    // Staged: offset inside the patch. Otherwise (c, r, s) packed in bytes;
    // padding depths (zero weights) point at element 0 / carry -1.
    if (staged) {
      offsets[d] = d < depth ? ci * plane_in + kr * dh * cols_in + ks * dw : 0;
    } else {
      offsets[d] = d < depth ? (ci << 16) | (kr << 8) | ks : -1;
    }
  }
  if (staged) {
    // Patch rows (c, kernel row) go to the wavefronts in turn, a lane per
    // column. Each wavefront issues the loads of kBatchRows of its rows
    // before it stores any (raw buffer loads: a position outside the image
    // reads 0), so a batch costs one memory latency instead of one per row.
    constexpr int kBatchRows = 4;
    constexpr int kColSteps = 4;  // columns lane + 64 j, j < kColSteps
    const __amdgpu_buffer_rsrc_t x_res = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x_img), 0, c * h * w * 4, kBufferFlags);
    const int rows_total = c * rows_in;
    for (int col0 = 0; col0 < cols_in; col0 += 64 * kColSteps) {
      for (int row0 = wv; row0 < rows_total; row0 += (kThreads / 64) * kBatchRows) {
        float v[kBatchRows][kColSteps];
#pragma unroll
        for (int b = 0; b < kBatchRows; ++b) {
          const int row = row0 + b * (kThreads / 64);
          const int ci = row / rows_in;
          const int ih = ih0 + row - ci * rows_in;
          const bool row_ok = row < rows_total && static_cast<unsigned>(ih) < static_cast<unsigned>(h);
#pragma unroll
          for (int j = 0; j < kColSteps; ++j) {
            const int iw = iw0 + col0 + lane + 64 * j;
            const bool ok = row_ok && static_cast<unsigned>(iw) < static_cast<unsigned>(w);
            v[b][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                    x_res, ok ? ((ci * h + ih) * w + iw) * 4 : kNoRead, 0, 0));
          }
        }
#pragma unroll
        for (int b = 0; b < kBatchRows; ++b) {
          const int row = row0 + b * (kThreads / 64);
#pragma unroll
          for (int j = 0; j < kColSteps; ++j) {
            const int cc = col0 + lane + 64 * j;
            if (row < rows_total && cc < cols_in) patch[row * cols_in + cc] = v[b][j];
          }
        }
      }
    }
  }
  if (tid < kChannels) {
    const int kk = k0 + tid;
    if (EPI == kPlain) {
      epi_mul[tid] = 1.0f;
      epi_add[tid] = 0.0f;
    } else {
      const bool ok = kk < k;
      const float mul = ok ? scale[kk] * rsqrtf(variance[kk] + epsilon) : 0.0f;
      epi_mul[tid] = mul;
      epi_add[tid] = ok ? bias[kk] - mean[kk] * mul : 0.0f;
    }
  }
  __syncthreads();

  // ---- MFMAs: both output rows, all column blocks, this wavefront's 16
  // channels.
  f32x4 acc[kRows][kBlocks];
#pragma unroll
  for (int rb = 0; rb < kRows; ++rb)
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) acc[rb][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // Input of depth entry `off` at output row oh0 + rb, local column px.
  auto fetch_global = [&](int off, int rb, int px) -> float {
    if (off < 0) return 0.0f;
    const int ci = off >> 16;
    const int kr = (off >> 8) & 0xff;
    const int ks = off & 0xff;
    const int ih = (oh0 + rb) * sh - ph + kr * dh;
    const int iw = (ow0 + px) * sw - pw + ks * dw;
    const bool inside = static_cast<unsigned>(ih) < static_cast<unsigned>(h) &&
                        static_cast<unsigned>(iw) < static_cast<unsigned>(w);
    return inside ? x_img[(static_cast<size_t>(ci) * h + ih) * w + iw] : 0.0f;
  };

  // One pass over the depth groups; `read(off, rb, px)` gives the input.
  auto multiply = [&](auto read) {
#pragma unroll
    for (int g = 0; g < kGroupsMax; ++g) {
      if (g < groups) {
        const i32x4 off = *reinterpret_cast<const i32x4*>(offsets + 16 * g + 4 * quarter);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
          for (int rb = 0; rb < kRows; ++rb)
#pragma unroll
            for (int b = 0; b < kBlocks; ++b) {
              const float bv = read(off[e], rb, b * 16 + lane16);
              acc[rb][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(wreg[4 * g + e], bv, acc[rb][b], 0, 0, 0);
            }
        }
      }
    }
  };
  if (staged) {
    multiply([&](int off, int rb, int px) { return patch[off + rb * sh * cols_in + px * sw]; });
  } else {
    multiply(fetch_global);
  }

  // ---- Epilogue.
  // When Q % 4 == 0 each output row goes through LDS (the patch is free
  // once every wavefront has finished its MFMAs), so that a lane stores 16
  // bytes of four consecutive pixels of one channel and a wavefront writes
  // whole 448-byte row runs, instead of four 4-byte values of four channels.
  constexpr int kStageRow = kCols + 4;  // one channel's staged row, padded
  constexpr int kGroups4 = kCols / 4;   // 16-byte groups per channel row
  constexpr int kItems = kChannels * kGroups4 / kThreads;
  static_assert(kChannels * kStageRow <= kPatchMax && kItems * kThreads == kChannels * kGroups4, "stage");
  if ((q & 3) == 0) {
    float* stage = patch;
#pragma unroll
    for (int rb = 0; rb < kRows; ++rb) {
      const int oh = oh0 + rb;
      __syncthreads();  // the patch (first row) or the previous row's stage is no longer read
#pragma unroll
      for (int b = 0; b < kBlocks; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) stage[(16 * wv + 4 * quarter + e) * kStageRow + b * 16 + lane16] = acc[rb][b][e];
      __syncthreads();
#pragma unroll
      for (int it = 0; it < kItems; ++it) {
        const int item = tid + it * kThreads;
        const int local = item / kGroups4;
        const int g4 = item - local * kGroups4;
        const int kk = k0 + local;
        const int ow = ow0 + 4 * g4;
        if (oh >= p || kk >= k || ow >= q) continue;  // Q % 4 == 0: a group is whole or outside
        const size_t at = ((static_cast<size_t>(img) * k + kk) * p + oh) * q + ow;
        f32x4 v = *reinterpret_cast<const f32x4*>(stage + local * kStageRow + 4 * g4);
        f32x4 res = {0.0f, 0.0f, 0.0f, 0.0f};
        if (EPI == kBatchNormAddRelu) res = *reinterpret_cast<const f32x4*>(residual + at);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (EPI != kPlain) v[e] = fmaf(v[e], epi_mul[local], epi_add[local]);
          if (EPI == kBatchNormAddRelu) v[e] += res[e];
          if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v[e] = fmaxf(v[e], 0.0f);
        }
        *reinterpret_cast<f32x4*>(output + at) = v;
      }
    }
    return;
  }
#pragma unroll
  for (int rb = 0; rb < kRows; ++rb) {
    const int oh = oh0 + rb;
    if (oh >= p) break;
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      const int ow = ow0 + b * 16 + lane16;
      if (ow >= q) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int local = 16 * wv + 4 * quarter + e;
        const int kk = k0 + local;
        if (kk >= k) continue;
        const size_t at = ((static_cast<size_t>(img) * k + kk) * p + oh) * q + ow;
        float v = acc[rb][b][e];
        if (EPI != kPlain) v = fmaf(v, epi_mul[local], epi_add[local]);
        if (EPI == kBatchNormAddRelu) v += residual[at];
        if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v = fmaxf(v, 0.0f);
        output[at] = v;
      }
    }
  }
}

}  // namespace

#define CT_SMALLC_DIMS                                                                                 \
  int n, int c, int h, int w, int k, int r, int s, int out_h, int out_w, int stride_h, int stride_w, \
      int pad_h, int pad_w, int dilation_h, int dilation_w
#define CT_SMALLC_ARGS n, c, h, w, k, r, s, out_h, out_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w

CT_KERNEL void __launch_bounds__(kThreads)
    conv_bn_relu_fp32_smallc(const float* x, const float* weight, const float* scale, const float* bias,
                             const float* mean, const float* variance, float* output, CT_SMALLC_DIMS, float epsilon,
                             void*, void*) {
  SmallCConv<kBatchNormRelu>(x, weight, scale, bias, mean, variance, nullptr, output, CT_SMALLC_ARGS, epsilon);
}

CT_KERNEL void __launch_bounds__(kThreads)
    conv_bn_fp32_smallc(const float* x, const float* weight, const float* scale, const float* bias, const float* mean,
                        const float* variance, float* output, CT_SMALLC_DIMS, float epsilon, void*, void*) {
  SmallCConv<kBatchNorm>(x, weight, scale, bias, mean, variance, nullptr, output, CT_SMALLC_ARGS, epsilon);
}

CT_KERNEL void __launch_bounds__(kThreads)
    conv_bn_add_relu_fp32_smallc(const float* x, const float* weight, const float* scale, const float* bias,
                                 const float* mean, const float* variance, const float* residual, float* output,
                                 CT_SMALLC_DIMS, float epsilon, void*, void*) {
  SmallCConv<kBatchNormAddRelu>(x, weight, scale, bias, mean, variance, residual, output, CT_SMALLC_ARGS, epsilon);
}

CT_KERNEL void __launch_bounds__(kThreads)
    conv_fp32_smallc(const float* x, const float* weight, float* output, CT_SMALLC_DIMS, void*, void*) {
  SmallCConv<kPlain>(x, weight, nullptr, nullptr, nullptr, nullptr, nullptr, output, CT_SMALLC_ARGS, 0.0f);
}
