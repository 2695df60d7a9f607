// FP16 Gemm and GemmGelu on CDNA4 FP16 MFMA (v_mfma_f32_32x32x16_f16) with
// FP32 accumulation, an optional bias vector and a fused erf-GELU epilogue.
//
// Semantics follow python/cutriton/triton_kernels/transformer.py:
//   gemm_fp16 (17-60): Y = fp16(sum_k A[m,k] * B[k,n]) with FP32 accumulation;
//   gemm_gelu_fp16 (63-107): Y = fp16(0.5 a (1 + erf(a / sqrt 2))), a the FP32 sum.
// The 3-input entry points add bias[n] (FP16, widened to FP32) to the FP32
// sum before the activation. Argument order is the pack ABI of
// transformer.py:256-271 (a, b, [bias,] output, m, n, k, two reserved).
//
// A is row-major [M, K] and B row-major [K, N]. The MFMA reads 8 consecutive
// depth values per lane for both operands, so the A tile is staged in LDS as
// [m][k] and the B tile is transposed on its way into LDS to [n][k]: each
// thread loads a 4 (depth) x 8 (column) block with four 16-byte loads and
// writes eight 8-byte [n][k..k+3] runs.
#include "common.h"

namespace {

using ct::f16x8;
using ct::f32x16;
using ct::u32x4;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool GELU, bool BIAS>
__device__ __forceinline__ void GemmF16Core(const _Float16* __restrict__ a, const _Float16* __restrict__ b,
                                            const _Float16* __restrict__ bias, _Float16* __restrict__ output,
                                            const int m, const int n, const int k) {
  constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int TM = WM / 32;
  constexpr int TN = WN / 32;
  constexpr int LDK = BK + 8;  // padded LDS row (halves); rows stay 16-byte aligned
  constexpr int A_CHUNKS = BM * BK / 8 / THREADS;         // 16-byte A chunks per thread
  constexpr int B_BLOCKS = (BK / 4) * (BN / 8) / THREADS;  // 4x8 B blocks per thread
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 MFMA tile");
  static_assert(A_CHUNKS >= 1 && A_CHUNKS * THREADS * 8 == BM * BK, "A tile split");
  static_assert(B_BLOCKS >= 1 && B_BLOCKS * THREADS * 32 == BK * BN, "B tile split");

  __shared__ __attribute__((aligned(16))) _Float16 a_tile[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) _Float16 b_tile[2][BN][LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Tile order: XCD-contiguous ranges, then groups of 8 row tiles walked
  // column by column so that concurrently running tiles share A and B panels.
  constexpr int GROUP_M = 8;
  const int tiles_m = (m + BM - 1) / BM;
  const int tiles_n = (n + BN - 1) / BN;
  const int tile = ct::XcdContiguousIndex(blockIdx.x, tiles_m * tiles_n);
  const int group_width = GROUP_M * tiles_n;
  const int group = tile / group_width;
  const int first_m = group * GROUP_M;
  const int group_rows = min(tiles_m - first_m, GROUP_M);
  const int within = tile - group * group_width;
  const int tile_m = first_m + within % group_rows;
  const int tile_n = within / group_rows;
  const int m0 = tile_m * BM;
  const int n0 = tile_n * BN;

  const bool vec_a = (k & 7) == 0;
  const bool vec_b = (n & 7) == 0;

  u32x4 ra[A_CHUNKS];
  u32x4 rb[B_BLOCKS][4];

  auto load_chunk = [](const _Float16* base, int row, int col, int rows, int cols, int ld, bool vec) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < rows) {
      const _Float16* p = base + static_cast<size_t>(row) * ld + col;
      if (vec && col + 8 <= cols) {
        v = *reinterpret_cast<const u32x4*>(p);
      } else {
        _Float16 h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (col + e < cols) ? p[e] : static_cast<_Float16>(0.0f);
        __builtin_memcpy(&v, h, 16);
      }
    }
    return v;
  };

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int chunk = tid + THREADS * i;
      const int row = chunk / (BK / 8);
      const int kc = (chunk % (BK / 8)) * 8;
      ra[i] = load_chunk(a, m0 + row, k0 + kc, m, k, k, vec_a);
    }
#pragma unroll
    for (int i = 0; i < B_BLOCKS; ++i) {
      const int block = tid + THREADS * i;
      const int nb = (block % (BN / 8)) * 8;
      const int kb = (block / (BN / 8)) * 4;
#pragma unroll
      for (int r = 0; r < 4; ++r) rb[i][r] = load_chunk(b, k0 + kb + r, n0 + nb, k, n, n, vec_b);
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int chunk = tid + THREADS * i;
      const int row = chunk / (BK / 8);
      const int kc = (chunk % (BK / 8)) * 8;
      *reinterpret_cast<u32x4*>(&a_tile[buf][row][kc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_BLOCKS; ++i) {
      const int block = tid + THREADS * i;
      const int nb = (block % (BN / 8)) * 8;
      const int kb = (block / (BN / 8)) * 4;
      // Row r holds columns nb..nb+7 as 4 dwords of 2 halves. Column c's
      // depth run (r = 0..3) becomes 2 dwords: (row0, row1), (row2, row3).
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int word = c >> 1;
        const bool high = c & 1;
        uint32_t h0 = rb[i][0][word], h1 = rb[i][1][word], h2 = rb[i][2][word], h3 = rb[i][3][word];
        if (high) {
          h0 >>= 16; h1 >>= 16; h2 >>= 16; h3 >>= 16;
        }
        u32x2 out;
        out[0] = (h0 & 0xffffu) | (h1 << 16);
        out[1] = (h2 & 0xffffu) | (h3 << 16);
        *reinterpret_cast<u32x2*>(&b_tile[buf][nb + c][kb]) = out;
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

  const int wm = (wave / WAVES_N) * WM;
  const int wn = (wave % WAVES_N) * WN;
  const int lane32 = lane & 31;
  const int koff = (lane >> 5) * 8;
  const int k_tiles = (k + BK - 1) / BK;

  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < k_tiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      f16x8 av[TM];
      f16x8 bv[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) av[i] = *reinterpret_cast<const f16x8*>(&a_tile[cur][wm + i * 32 + lane32][kk + koff]);
#pragma unroll
      for (int t = 0; t < TN; ++t) bv[t] = *reinterpret_cast<const f16x8*>(&b_tile[cur][wn + t * 32 + lane32][kk + koff]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[i], bv[t], acc[i][t], 0, 0, 0);
    }
    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Lane holds column (lane % 32) and rows 8*(r/4) + 4*(lane/32) + (r%4).
  const int half = lane >> 5;
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = n0 + wn + t * 32 + lane32;
    if (col >= n) continue;
    const float bias_value = BIAS ? static_cast<float>(bias[col]) : 0.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (row >= m) continue;
        float v = acc[i][t][r];
        if (BIAS) v += bias_value;
        if (GELU) v = ct::GeluErf(v);
        output[static_cast<size_t>(row) * n + col] = static_cast<_Float16>(v);
      }
    }
  }
}

}  // namespace

#define CT_DEFINE_GEMM_F16(NAME, BM, BN, BK, WM, WN)                                                        \
  CT_KERNEL void __launch_bounds__(64 * WM * WN)                                                           \
      gemm_fp16_##NAME(const _Float16* a, const _Float16* b, _Float16* output, int m, int n, int k, void*,  \
                       void*) {                                                                            \
    GemmF16Core<BM, BN, BK, WM, WN, false, false>(a, b, nullptr, output, m, n, k);                         \
  }                                                                                                        \
  CT_KERNEL void __launch_bounds__(64 * WM * WN)                                                           \
      gemm_gelu_fp16_##NAME(const _Float16* a, const _Float16* b, _Float16* output, int m, int n, int k,    \
                            void*, void*) {                                                                \
    GemmF16Core<BM, BN, BK, WM, WN, true, false>(a, b, nullptr, output, m, n, k);                          \
  }                                                                                                        \
  CT_KERNEL void __launch_bounds__(64 * WM * WN)                                                           \
      gemm_bias_fp16_##NAME(const _Float16* a, const _Float16* b, const _Float16* bias, _Float16* output,   \
                            int m, int n, int k, void*, void*) {                                           \
    GemmF16Core<BM, BN, BK, WM, WN, false, true>(a, b, bias, output, m, n, k);                             \
  }                                                                                                        \
  CT_KERNEL void __launch_bounds__(64 * WM * WN)                                                           \
      gemm_gelu_bias_fp16_##NAME(const _Float16* a, const _Float16* b, const _Float16* bias,                \
                                 _Float16* output, int m, int n, int k, void*, void*) {                    \
    GemmF16Core<BM, BN, BK, WM, WN, true, true>(a, b, bias, output, m, n, k);                              \
  }

CT_DEFINE_GEMM_F16(m64n64k64, 64, 64, 64, 2, 1)
CT_DEFINE_GEMM_F16(m128n128k64, 128, 128, 64, 2, 2)
CT_DEFINE_GEMM_F16(m256n128k64, 256, 128, 64, 2, 2)
CT_DEFINE_GEMM_F16(m256n256k64, 256, 256, 64, 4, 2)
