// FP32 implicit-GEMM convolution, register-direct variant: every wavefront
// loads its own MFMA operand fragments straight from global memory (raw
// buffer loads, L1/L2-served re-reads) into registers, with no LDS staging
// and no barrier in the main loop. Same operation, arguments and epilogues as
// conv_fp32.hip (reference python/cutriton/triton_kernels/resnet.py:12-114,
// 150-156; pack ABI resnet.py:242-300).
//
// GEMM view: rows m = output channel, columns j = image*P*Q + pixel, depth
// d = (c, r, s); A = OIHW weights as [K_out][depth], B = the im2col gather.
// A wavefront owns (32*TM) x (32*TN) outputs (TM x TN accumulators of the
// 32x32x2 MFMA). The workgroup's 4 wavefronts form a WGM x WGN x WGK grid;
// WGK > 1 splits the depth range and the partial sums are added through LDS.
//
// Depth order inside an 8-deep group g: MFMA step 4g + e, lane half h uses
// depth 8g + 4h + e. A lane therefore reads 4 consecutive depths of its
// weight row with one 16-byte load; the gather for half h walks depths
// 8g + 4h .. 8g + 4h + 3.
#include "common.h"

namespace {

using ct::f32x16;
using ct::f32x4;

enum Epilogue : int { kPlain = 0, kBatchNorm = 1, kBatchNormRelu = 2, kBatchNormAddRelu = 3 };

struct Geometry {
  int n, c, h, w, k, r, s, p, q;
  int stride_h, stride_w, pad_h, pad_w, dil_h, dil_w;
};

constexpr int kThreads = 256;
constexpr int kBufferFlags = 0x00020000;  // gfx9-family raw 32-bit buffer
constexpr int kNoRead = 0x80000000;       // offset past every resource here: reads 0

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Resource(const float* base, long long elements) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(elements * 4),
                                           kBufferFlags);
}

template <int TM, int TN>
struct Fragment {
  f32x4 a[TM];
  float b[TN][4];
};

template <int TM, int TN, int WGM, int WGN, int WGK>
struct DirectLds {
  static constexpr int kBM = 32 * TM * WGM;
  static constexpr int kReduce = (WGK - 1) * WGM * WGN * TM * TN * 16 * 64;
  static constexpr int kFloats = kReduce + 2 * kBM;
};

template <int TM, int TN, int WGM, int WGN, int WGK, int EPI, bool POINTWISE>
__device__ __forceinline__ void DirectCore(float* __restrict__ smem, const float* __restrict__ x,
                                           const float* __restrict__ weight, const float* __restrict__ scale,
                                           const float* __restrict__ bias, const float* __restrict__ mean,
                                           const float* __restrict__ variance, const float* __restrict__ residual,
                                           float* __restrict__ output, const Geometry g, const float epsilon) {
  using L = DirectLds<TM, TN, WGM, WGN, WGK>;
  constexpr int BM = 32 * TM * WGM;
  constexpr int BN = 32 * TN * WGN;
  static_assert(WGM * WGN * WGK == kThreads / 64, "four wavefronts per workgroup");
  float* epi_mul = smem + L::kReduce;
  float* epi_add = epi_mul + BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int lane32 = lane & 31;
  const int pq = g.p * g.q;
  const int hw = g.h * g.w;
  const int rs = g.r * g.s;
  const int depth = g.c * rs;
  const int columns = g.n * pq;
  const bool vec_a = (depth & 3) == 0;

  const int tiles_n = (columns + BN - 1) / BN;
  const int tiles_m = (g.k + BM - 1) / BM;
  const int tile = ct::XcdContiguousIndex(blockIdx.x + blockIdx.y * gridDim.x, tiles_n * tiles_m);
  const int m0 = (tile % tiles_m) * BM;
  const int n0 = (tile / tiles_m) * BN;

  if (EPI != kPlain) {
    for (int i = tid; i < BM; i += kThreads) {
      const int m = m0 + i;
      const bool ok = m < g.k;
      const float mul = ok ? scale[m] * rsqrtf(variance[m] + epsilon) : 0.0f;
      epi_mul[i] = mul;
      epi_add[i] = ok ? bias[m] - mean[m] * mul : 0.0f;
    }
  }

  const int wk = wave / (WGM * WGN);
  const int wmn = wave % (WGM * WGN);
  const int wm = (wmn / WGN) * 32 * TM;
  const int wn = (wmn % WGN) * 32 * TN;

  const __amdgpu_buffer_rsrc_t x_res = Resource(x, static_cast<long long>(g.n) * g.c * hw);
  const __amdgpu_buffer_rsrc_t w_res = Resource(weight, static_cast<long long>(g.k) * depth);

  // Weight rows of this lane: element offset of (row, depth 4*half).
  int a_base[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = m0 + wm + i * 32 + lane32;
    a_base[i] = row < g.k ? row * depth + 4 * half : -1;
  }
  // Gather columns of this lane.
  int b_base[TN];   // element offset of (image, channel 0, ih0, iw0), or of the pointwise pixel
  int b_ih0[TN];
  int b_iw0[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int j = n0 + wn + t * 32 + lane32;
    const bool ok = j < columns;
    const int img = ok ? j / pq : 0;
    const int pix = ok ? j - img * pq : 0;
    const int oh = pix / g.q;
    const int ow = pix - oh * g.q;
    b_ih0[t] = oh * g.stride_h - g.pad_h;
    b_iw0[t] = ow * g.stride_w - g.pad_w;
    if (POINTWISE) {
      b_base[t] = ok ? img * g.c * hw + (oh * g.stride_h) * g.w + ow * g.stride_w + 4 * half * hw : -1;
    } else {
      b_base[t] = ok ? img * g.c * hw + b_ih0[t] * g.w + b_iw0[t] : -1;
      if (!ok) b_ih0[t] = -0x40000000;  // never inside
    }
  }

  // Depth range of this wavefront, in 8-deep groups.
  const int groups = (depth + 7) / 8;
  const int per_wave = (groups + WGK - 1) / WGK;
  const int g_begin = wk * per_wave;
  const int g_end = min(groups, g_begin + per_wave);

  auto load = [&](int gi, Fragment<TM, TN>& f) {
    const int d0 = gi * 8;  // uniform
    const bool full = d0 + 8 <= depth;
    const int dl = d0 + 4 * half;  // first depth of this lane's run
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if (vec_a) {
        const int off = (a_base[i] >= 0 && (full || dl < depth)) ? (a_base[i] + d0) * 4 : kNoRead;
        f.a[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(w_res, off, 0, 0));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int off = (a_base[i] >= 0 && dl + e < depth) ? (a_base[i] + d0 + e) * 4 : kNoRead;
          f.a[i][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(w_res, off, 0, 0));
        }
      }
    }
    if (POINTWISE) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool dok = full || dl + e < depth;
        const int soff = (d0 + e) * hw * 4;  // uniform
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const int off = (b_base[t] >= 0 && dok) ? b_base[t] * 4 : kNoRead;
          f.b[t][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_res, off, soff, 0));
        }
      }
    } else {
      // The two lane halves walk different depth runs: decompose both (scalar
      // work) and let each lane pick its own.
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int uo[2], ur[2], us[2];
        bool uv[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int d = d0 + 4 * hh + e;
          const int ci = d / rs;
          const int rr = d - ci * rs;
          const int kr = rr / g.s;
          const int ks = rr - kr * g.s;
          ur[hh] = kr * g.dil_h;
          us[hh] = ks * g.dil_w;
          uo[hh] = ci * hw + ur[hh] * g.w + us[hh];
          uv[hh] = d < depth;
        }
        const int o = half ? uo[1] : uo[0];
        const int dr = half ? ur[1] : ur[0];
        const int ds = half ? us[1] : us[0];
        const bool dv = half ? uv[1] : uv[0];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const bool inside = dv && static_cast<unsigned>(b_ih0[t] + dr) < static_cast<unsigned>(g.h) &&
                              static_cast<unsigned>(b_iw0[t] + ds) < static_cast<unsigned>(g.w);
          const int off = inside ? (b_base[t] + o) * 4 : kNoRead;
          f.b[t][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(x_res, off, 0, 0));
        }
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][t][r] = 0.0f;

  auto compute = [&](const Fragment<TM, TN>& f) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x2f32(f.a[i][e], f.b[t][e], acc[i][t], 0, 0, 0);
  };

  // Two fragments in flight: group gi+2 loads while gi computes.
  Fragment<TM, TN> f0, f1;
  if (g_begin < g_end) load(g_begin, f0);
  if (g_begin + 1 < g_end) load(g_begin + 1, f1);
  int gi = g_begin;
  for (; gi + 1 < g_end; gi += 2) {
    compute(f0);
    if (gi + 2 < g_end) load(gi + 2, f0);
    compute(f1);
    if (gi + 3 < g_end) load(gi + 3, f1);
  }
  if (gi < g_end) compute(f0);

  if (WGK > 1) {
    constexpr int REGS = TM * TN * 16;
    if (wk > 0) {
      float* mine = smem + ((wk - 1) * WGM * WGN + wmn) * REGS * 64;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) mine[((i * TN + t) * 16 + r) * 64 + lane] = acc[i][t][r];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll 1
    for (int sl = 1; sl < WGK; ++sl) {
      const float* theirs = smem + ((sl - 1) * WGM * WGN + wmn) * REGS * 64;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][t][r] += theirs[((i * TN + t) * 16 + r) * 64 + lane];
    }
  } else if (EPI != kPlain) {
    __syncthreads();  // BatchNorm parameters are in LDS
  }

  // Epilogue: lane holds column lane32 of each tile and rows
  // 8*(r/4) + 4*half + (r%4).
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
        if (EPI != kPlain) {
          const f32x4 mul = *reinterpret_cast<const f32x4*>(epi_mul + (lrow & ~3));
          const f32x4 add = *reinterpret_cast<const f32x4*>(epi_add + (lrow & ~3));
          v = fmaf(v, mul[r & 3], add[r & 3]);
        }
        if (EPI == kBatchNormAddRelu) v += residual[at];
        if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v = fmaxf(v, 0.0f);
        output[at] = v;
      }
    }
  }
}

__device__ __forceinline__ Geometry MakeGeometry(int n, int c, int h, int w, int k, int r, int s, int out_h,
                                                 int out_w, int stride_h, int stride_w, int pad_h, int pad_w,
                                                 int dilation_h, int dilation_w) {
  Geometry g;
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

#define CT_DISPATCH(TM, TN, WGM, WGN, WGK, EPI, ...)                                               \
  __shared__ __attribute__((aligned(16))) float smem[DirectLds<TM, TN, WGM, WGN, WGK>::kFloats];  \
  if (r == 1 && s == 1 && pad_h == 0 && pad_w == 0) {                                             \
    DirectCore<TM, TN, WGM, WGN, WGK, EPI, true>(smem, __VA_ARGS__);                              \
  } else {                                                                                        \
    DirectCore<TM, TN, WGM, WGN, WGK, EPI, false>(smem, __VA_ARGS__);                             \
  }

#define CT_DEFINE_DIRECT_VARIANTS(NAME, TM, TN, WGM, WGN, WGK)                                        \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_relu_fp32_##NAME(                               \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,  \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {              \
    CT_DISPATCH(TM, TN, WGM, WGN, WGK, kBatchNormRelu, x, weight, scale, bias, mean, variance,       \
                nullptr, output, CT_CONV_GEOMETRY, epsilon)                                           \
  }                                                                                                   \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_fp32_##NAME(                                    \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,  \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {              \
    CT_DISPATCH(TM, TN, WGM, WGN, WGK, kBatchNorm, x, weight, scale, bias, mean, variance, nullptr,  \
                output, CT_CONV_GEOMETRY, epsilon)                                                    \
  }                                                                                                   \
  CT_KERNEL void __launch_bounds__(kThreads) conv_bn_add_relu_fp32_##NAME(                           \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,  \
      const float* variance, const float* residual, float* output, CT_CONV_DIMS, float epsilon,       \
      void*, void*) {                                                                                 \
    CT_DISPATCH(TM, TN, WGM, WGN, WGK, kBatchNormAddRelu, x, weight, scale, bias, mean, variance,    \
                residual, output, CT_CONV_GEOMETRY, epsilon)                                          \
  }                                                                                                   \
  CT_KERNEL void __launch_bounds__(kThreads) conv_fp32_##NAME(const float* x, const float* weight,   \
                                                              float* output, CT_CONV_DIMS, void*,     \
                                                              void*) {                                \
    CT_DISPATCH(TM, TN, WGM, WGN, WGK, kPlain, x, weight, nullptr, nullptr, nullptr, nullptr,        \
                nullptr, output, CT_CONV_GEOMETRY, 0.0f)                                              \
  }

// name, TM, TN, WGM, WGN, WGK  (block tile = 32*TM*WGM x 32*TN*WGN)
CT_DEFINE_DIRECT_VARIANTS(d64n256, 2, 2, 1, 4, 1)
CT_DEFINE_DIRECT_VARIANTS(d64n64, 2, 2, 1, 1, 4)
CT_DEFINE_DIRECT_VARIANTS(d32n64, 1, 2, 1, 1, 4)
