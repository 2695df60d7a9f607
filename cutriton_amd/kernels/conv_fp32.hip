// FP32 implicit-GEMM convolution family on CDNA4 FP32 MFMA
// (v_mfma_f32_32x32x2_f32), with the BatchNorm / ReLU / residual-AddRelu
// epilogue fused, plus the FP32 Gemm that shares the same core.
//
// Semantics follow the reference kernels in
// python/cutriton/triton_kernels/resnet.py:
//   fused_conv_batch_norm_relu (12-47), fused_conv_batch_norm (50-85),
//   conv (88-114) and gemm (201-213);
// the residual-join variant applies add_relu (150-156) in the epilogue.
// Argument order per entry point is the pack ABI order of resnet.py:242-300
// and 382-400, with two trailing reserved pointers.
//
// GEMM view of a convolution (NCHW input, OIHW weights):
//   rows    m = output channel                        (K_out)
//   columns j = image * P*Q + output pixel            (N*P*Q)
//   depth   d = (input channel, kernel row, kernel column)   (C*R*S)
//   A[m][d] = W[m][c][r][s]  (OIHW is already row-major [K_out, C*R*S])
//   B[d][j] = X[n][c][oh*sh - ph + r*dh][ow*sw - pw + s*dw]   (zero padded)
// Workgroup = 4 wavefronts in a 2x2 grid; each wavefront owns a
// (BM/2) x (BN/2) accumulator block made of 32x32 MFMA tiles. Operand tiles
// are staged through LDS in depth-major order ([d][m] and [d][j]), double
// buffered, with the next tile's global loads in flight during the MFMAs.
#include "common.h"

namespace {

using ct::f32x16;
using ct::f32x4;

enum Epilogue : int {
  kPlain = 0,             // y = acc
  kBatchNorm = 1,         // y = (acc - mean) * rsqrt(var + eps) * scale + bias
  kBatchNormRelu = 2,     // max(BN, 0)
  kBatchNormAddRelu = 3,  // max(BN + residual, 0)
  kColumnBias = 4,        // y = acc + bias[column]   (Gemm with a bias vector)
};

struct ConvGeometry {
  int n, c, h, w, k, r, s, p, q;
  int stride_h, stride_w, pad_h, pad_w, dil_h, dil_w;
};

constexpr int kThreads = 256;

template <int BM, int BN, int BK, int EPI>
__device__ __forceinline__ void ConvCore(const float* __restrict__ x, const float* __restrict__ weight,
                                         const float* __restrict__ scale, const float* __restrict__ bias,
                                         const float* __restrict__ mean, const float* __restrict__ variance,
                                         const float* __restrict__ residual, float* __restrict__ output,
                                         const ConvGeometry g, const float epsilon) {
  // Vector weight loads need every weight row to start 16-byte aligned.
  const bool vec_a = ((g.c * g.r * g.s) & 3) == 0;
  constexpr int WM = BM / 2;
  constexpr int WN = BN / 2;
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  constexpr int A_PER = BM * BK / kThreads;  // A elements per thread per tile
  constexpr int B_PER = BK * BN / kThreads;  // B elements per thread per tile
  constexpr int A_STRIDE = BM + 4;           // padded row of the [d][m] tile
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 MFMA tile");
  static_assert(kThreads % BN == 0, "B columns must divide the workgroup");
  static_assert(A_PER % 4 == 0, "vector A loads need 4-element runs");

  __shared__ float a_tile[2][BK][A_STRIDE];
  __shared__ float b_tile[2][BK][BN];
  __shared__ float epi_mean[BM];
  __shared__ float epi_rstd[BM];
  __shared__ float epi_scale[BM];
  __shared__ float epi_bias[BM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int pq = g.p * g.q;
  const int hw = g.h * g.w;
  const int rs = g.r * g.s;
  const int depth = g.c * rs;
  const int columns = g.n * pq;

  const int tiles_n = (columns + BN - 1) / BN;
  const int tiles_m = (g.k + BM - 1) / BM;
  const int tile = ct::XcdContiguousIndex(blockIdx.x + blockIdx.y * gridDim.x, tiles_n * tiles_m);
  const int m0 = (tile % tiles_m) * BM;
  const int n0 = (tile / tiles_m) * BN;

  if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) {
    for (int i = tid; i < BM; i += kThreads) {
      const int m = m0 + i;
      const bool ok = m < g.k;
      epi_mean[i] = ok ? mean[m] : 0.0f;
      epi_rstd[i] = ok ? rsqrtf(variance[m] + epsilon) : 0.0f;
      epi_scale[i] = ok ? scale[m] : 0.0f;
      epi_bias[i] = ok ? bias[m] : 0.0f;
    }
  }

  // ---- B (im2col) loader state: one fixed column per thread.
  const int b_col = tid % BN;
  const int b_row0 = (tid / BN) * B_PER;
  const int j = n0 + b_col;
  const bool col_ok = j < columns;
  const int img = col_ok ? j / pq : 0;
  const int pix = col_ok ? j - img * pq : 0;
  const int oh = pix / g.q;
  const int ow = pix - oh * g.q;
  const int ih0 = oh * g.stride_h - g.pad_h;
  const int iw0 = ow * g.stride_w - g.pad_w;
  const float* x_img = x + static_cast<size_t>(img) * g.c * hw;

  float ra[A_PER];
  float rb[B_PER];

  auto load_tile = [&](int d0) {
    // A: weights [K_out][depth], row-major.
    if (vec_a) {
#pragma unroll
      for (int v = 0; v < A_PER / 4; ++v) {
        const int f = tid + kThreads * v;
        const int kq = f % (BK / 4);
        const int m = f / (BK / 4);
        const int d = d0 + kq * 4;
        f32x4 val = {0.0f, 0.0f, 0.0f, 0.0f};
        if (m0 + m < g.k && d < depth) {
          val = *reinterpret_cast<const f32x4*>(weight + static_cast<size_t>(m0 + m) * depth + d);
        }
        ra[v * 4 + 0] = val[0];
        ra[v * 4 + 1] = val[1];
        ra[v * 4 + 2] = val[2];
        ra[v * 4 + 3] = val[3];
      }
    } else {
#pragma unroll
      for (int e = 0; e < A_PER; ++e) {
        const int f = tid + kThreads * e;
        const int kk = f % BK;
        const int m = f / BK;
        const int d = d0 + kk;
        ra[e] = (m0 + m < g.k && d < depth) ? weight[static_cast<size_t>(m0 + m) * depth + d] : 0.0f;
      }
    }
    // B: gathered input pixels, zero outside the image and past the depth.
    int d = d0 + b_row0;
    int ci = d / rs;
    int rr = d - ci * rs;
    int kr = rr / g.s;
    int ks = rr - kr * g.s;
#pragma unroll
    for (int e = 0; e < B_PER; ++e) {
      const int ih = ih0 + kr * g.dil_h;
      const int iw = iw0 + ks * g.dil_w;
      const bool inside = col_ok && (d + e) < depth && static_cast<unsigned>(ih) < static_cast<unsigned>(g.h) &&
                          static_cast<unsigned>(iw) < static_cast<unsigned>(g.w);
      rb[e] = inside ? x_img[static_cast<size_t>(ci) * hw + ih * g.w + iw] : 0.0f;
      if (++ks == g.s) {
        ks = 0;
        if (++kr == g.r) {
          kr = 0;
          ++ci;
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    if (vec_a) {
#pragma unroll
      for (int v = 0; v < A_PER / 4; ++v) {
        const int f = tid + kThreads * v;
        const int kq = f % (BK / 4);
        const int m = f / (BK / 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) a_tile[buf][kq * 4 + e][m] = ra[v * 4 + e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < A_PER; ++e) {
        const int f = tid + kThreads * e;
        a_tile[buf][f % BK][f / BK] = ra[e];
      }
    }
#pragma unroll
    for (int e = 0; e < B_PER; ++e) b_tile[buf][b_row0 + e][b_col] = rb[e];
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][t][r] = 0.0f;

  const int wm = (wave >> 1) * WM;
  const int wn = (wave & 1) * WN;
  const int half = lane >> 5;  // which depth row of the MFMA k-pair
  const int lane32 = lane & 31;
  const int depth_tiles = (depth + BK - 1) / BK;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < depth_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < depth_tiles;
    if (more) load_tile((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float av[TM];
      float bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = a_tile[cur][kk + half][wm + i * 32 + lane32];
#pragma unroll
      for (int t = 0; t < TN; ++t) bv[t] = b_tile[cur][kk + half][wn + t * 32 + lane32];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i], bv[t], acc[i][t], 0, 0, 0);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // ---- Epilogue. Lane holds column (lane % 32) of each 32x32 tile and rows
  // 8*(r/4) + 4*(lane/32) + (r%4) for accumulator register r.
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = n0 + wn + t * 32 + lane32;
    if (col >= columns) continue;
    const int cimg = col / pq;
    const int cpix = col - cimg * pq;
    const size_t col_base = static_cast<size_t>(cimg) * g.k * pq + cpix;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int lrow = wm + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        const int row = m0 + lrow;
        if (row >= g.k) continue;
        float v = acc[i][t][r];
        const size_t at = col_base + static_cast<size_t>(row) * pq;
        if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) {
          v = (v - epi_mean[lrow]) * epi_rstd[lrow] * epi_scale[lrow] + epi_bias[lrow];
        }
        if (EPI == kBatchNormAddRelu) v += residual[at];
        if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v = fmaxf(v, 0.0f);
        if (EPI == kColumnBias) v += bias[col];
        output[at] = v;
      }
    }
  }
}

__device__ __forceinline__ ConvGeometry MakeGeometry(int n, int c, int h, int w, int k, int r, int s, int out_h,
                                                     int out_w, int stride_h, int stride_w, int pad_h, int pad_w,
                                                     int dilation_h, int dilation_w) {
  ConvGeometry g;
  g.n = n; g.c = c; g.h = h; g.w = w; g.k = k; g.r = r; g.s = s; g.p = out_h; g.q = out_w;
  g.stride_h = stride_h; g.stride_w = stride_w; g.pad_h = pad_h; g.pad_w = pad_w;
  g.dil_h = dilation_h; g.dil_w = dilation_w;
  return g;
}

}  // namespace

#define CT_CONV_DIMS                                                                                   \
  int n, int c, int h, int w, int k, int r, int s, int out_h, int out_w, int stride_h, int stride_w, \
      int pad_h, int pad_w, int dilation_h, int dilation_w
#define CT_CONV_GEOMETRY \
  MakeGeometry(n, c, h, w, k, r, s, out_h, out_w, stride_h, stride_w, pad_h, pad_w, dilation_h, dilation_w)

#define CT_DISPATCH_A(BM, BN, BK, EPI, ...) ConvCore<BM, BN, BK, EPI>(__VA_ARGS__);

#define CT_DEFINE_CONV_VARIANTS(NAME, BM, BN, BK)                                                        \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_relu_fp32_##NAME(                                  \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {                 \
    CT_DISPATCH_A(BM, BN, BK, kBatchNormRelu, x, weight, scale, bias, mean, variance, nullptr, output,  \
                  CT_CONV_GEOMETRY, epsilon)                                                             \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_fp32_##NAME(                                       \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {                 \
    CT_DISPATCH_A(BM, BN, BK, kBatchNorm, x, weight, scale, bias, mean, variance, nullptr, output,      \
                  CT_CONV_GEOMETRY, epsilon)                                                             \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_add_relu_fp32_##NAME(                              \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, const float* residual, float* output, CT_CONV_DIMS, float epsilon, void*,   \
      void*) {                                                                                           \
    CT_DISPATCH_A(BM, BN, BK, kBatchNormAddRelu, x, weight, scale, bias, mean, variance, residual,      \
                  output, CT_CONV_GEOMETRY, epsilon)                                                     \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(kThreads) conv_fp32_##NAME(const float* x, const float* weight,      \
                                                              float* output, CT_CONV_DIMS, void*, void*) { \
    CT_DISPATCH_A(BM, BN, BK, kPlain, x, weight, nullptr, nullptr, nullptr, nullptr, nullptr, output,   \
                  CT_CONV_GEOMETRY, 0.0f)                                                                \
  }

CT_DEFINE_CONV_VARIANTS(m128n128, 128, 128, 16)
CT_DEFINE_CONV_VARIANTS(m64n128, 64, 128, 32)
CT_DEFINE_CONV_VARIANTS(m128n64, 128, 64, 16)
CT_DEFINE_CONV_VARIANTS(m64n64, 64, 64, 32)

// C[m][n] = sum_k A[m][k] * B[k][n] (+ bias[n]) with A, B row-major: the
// depth-major core with rows = m, columns = n, depth = k (a 1x1 convolution
// of one 1 x n "image").
#define CT_DEFINE_GEMM_VARIANTS(NAME, BM, BN, BK)                                                         \
  CT_KERNEL void __launch_bounds__(kThreads) gemm_fp32_##NAME(const float* a, const float* b, float* output, \
                                                              int m, int n, int k, void*, void*) {        \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    ConvCore<BM, BN, BK, kPlain>(b, a, nullptr, nullptr, nullptr, nullptr, nullptr, output, g, 0.0f); \
  }                                                                                                       \
  CT_KERNEL void __launch_bounds__(kThreads) gemm_bias_fp32_##NAME(                                      \
      const float* a, const float* b, const float* bias, float* output, int m, int n, int k, void*, void*) { \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    ConvCore<BM, BN, BK, kColumnBias>(b, a, nullptr, bias, nullptr, nullptr, nullptr, output, g, 0.0f); \
  }

CT_DEFINE_GEMM_VARIANTS(m64n64, 64, 64, 32)
CT_DEFINE_GEMM_VARIANTS(m128n128, 128, 128, 16)
