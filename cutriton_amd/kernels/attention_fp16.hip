// Fused scaled-dot-product attention, FP16 in and out, FP32 arithmetic, on
// CDNA4 FP16 MFMA (v_mfma_f32_16x16x32_f16):
//   O[b,h,i,:] = sum_j softmax_j(scale * Q[b,h,i,:] . K[b,h,j,:]) V[b,h,j,:]
// over j < Sk, and with is_causal only over j <= i (the upper-left aligned
// causal mask of the ONNX Attention operator). Inputs are [B, H, S, D]
// row-major; head dimensions up to the variant's DMAX (64 or 128) are
// served, shorter ones read as zero-padded.
//
// The reference has no attention operator; this is the block its FFN path
// leads to (Softmax, LayerNorm and the GEMMs are its parts).
//
// One workgroup of 4 wavefronts owns 128 queries of one (b, h); a wavefront
// owns 32 of them (two 16-query tiles) and walks the keys in blocks of 64
// with the online softmax: a running row maximum m and sum l per query, the
// output accumulator rescaled by exp2(m_old - m_new) when the maximum grows.
// Nothing of size Sq x Sk is ever stored.
//
// Layouts (no lane ever exchanges data with another to change layouts):
//   * S^T = K . Q^T: the key fragment is the MFMA's row operand, so a lane
//     ends with one query (lane % 16) and four consecutive keys
//     (4 (lane / 16) + 0..3) of each 16-key tile. Row statistics reduce
//     over the lane's 16 values, then over lanes xor 16 and xor 32.
//   * O^T = V^T . P^T: the contraction over keys may take the keys in any
//     order shared by both operands. The 32 keys of one step are ordered so
//     that lane group g supplies keys 4g..4g+3 of the first 16-key tile and
//     of the second: exactly the P values the lane already holds. The V
//     operand then needs, per lane, 4 consecutive keys at one column d, so V
//     is staged in LDS as [key / 4][d][4]: two 8-byte reads per fragment.
//     A lane ends with one query and four consecutive d: 8-byte stores.
//   * K is staged as [key][d] rows of 16-byte chunks, chunk c of row r at
//     c ^ f(r) (f as in the FP16 GEMMs), so the 16 lanes of an LDS read
//     phase hit distinct banks. V rows ([d][4] per key group) are padded by
//     128 bytes, which puts the two key groups of a read phase on opposite
//     halves of the 64 banks.
//
// Pipeline: K blocks go straight into LDS with buffer_load ... lds; V blocks
// go through registers (loaded before the block's MFMAs, transposed and
// written after them) into the other of two LDS stages.
#include "common.h"

namespace {

using ct::f16x8;
using ct::f32x4;
using ct::u32x4;

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kQueriesPerWave = 32;
constexpr int kQueriesPerBlock = 4 * kQueriesPerWave;
constexpr int kKeys = 64;  // keys per block
constexpr int kBufferFlags = 0x00020000;
constexpr int kNoRead = 0x80000000;  // beyond every resource's range: reads 0
constexpr float kLog2e = 1.4426950408889634f;

#define CT_LDS(p) ((__attribute__((address_space(3))) void*)(p))

template <int DMAX>
struct AttnShape {
  static constexpr int kChunks = DMAX / 8;                 // 16-byte chunks per K row
  static constexpr int kKChunks = kKeys * kChunks;         // u32x4 per K stage
  static constexpr int kVStride = DMAX + 16;               // 8-byte units per V key group (padded)
  static constexpr int kVUnits = (kKeys / 4) * kVStride;   // 8-byte units per V stage
  static constexpr int kStageBytes = kKChunks * 16 + kVUnits * 8;
};

__device__ __forceinline__ float GroupMax16(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

__device__ __forceinline__ float GroupSum16(float v) {
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

// Eight halves of `row`, depths [col, col + 8), zero outside rows x d.
__device__ __forceinline__ f16x8 LoadRow8(const _Float16* base, int row, int rows, int col, int d, bool vec) {
  if (vec) {
    if (row < rows && col < d) return *reinterpret_cast<const f16x8*>(base + static_cast<size_t>(row) * d + col);
    return f16x8{};
  }
  f16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v[e] = (row < rows && col + e < d) ? base[static_cast<size_t>(row) * d + col + e] : static_cast<_Float16>(0.0f);
  }
  return v;
}

// VEC: d is a multiple of 8 and the tensors are 16-byte aligned, so rows
// load as 16-byte chunks (K straight into LDS); otherwise element-wise.
template <int DMAX, bool VEC>
__device__ __forceinline__ void AttentionCore(uint8_t* __restrict__ lds, const _Float16* __restrict__ q,
                                              const _Float16* __restrict__ k, const _Float16* __restrict__ v,
                                              _Float16* __restrict__ out, const int sq, const int sk, const int d,
                                              const float scale, const int causal) {
  using S = AttnShape<DMAX>;
  constexpr int CH = S::kChunks;
  constexpr int STEPS = DMAX / 32;  // MFMA steps over the head dimension
  constexpr int DT = DMAX / 16;     // 16-wide d tiles of the output
  constexpr int RPL = 64 / CH;      // K rows one wavefront load fills
  constexpr int K_LOADS = kKeys / RPL / 4;  // K load instructions per wavefront and block
  constexpr int V_UNITS = (kKeys / 4) * (DMAX / 8);  // (4 keys x 8 d) units per block
  constexpr int V_PER_THREAD = (V_UNITS + kThreads - 1) / kThreads;
  static_assert(K_LOADS >= 1 && K_LOADS * RPL * 4 == kKeys, "K loads split evenly over the wavefronts");
  static_assert(V_PER_THREAD >= 1 && V_PER_THREAD <= 2, "V units per thread");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int lane16 = lane & 15;
  const int g = lane >> 4;
  // Without the mask, query blocks of one (b, h) run side by side and share
  // its K and V in L2. With the causal mask the last query blocks see the
  // most keys: the dispatch order is remapped (a bijection of the grid) so
  // that every (b, h)'s heaviest block starts first, then the next heaviest,
  // and the short ones fill in behind them.
  int q_index = blockIdx.x;
  size_t bh = blockIdx.y;
  if (causal) {
    const int linear = blockIdx.y * gridDim.x + blockIdx.x;
    q_index = gridDim.x - 1 - linear / gridDim.y;
    bh = linear % gridDim.y;
  }
  const int q_block = q_index * kQueriesPerBlock;
  const int q_wave = q_block + wave * kQueriesPerWave;

  const _Float16* qb = q + bh * static_cast<size_t>(sq) * d;
  const _Float16* kb_base = k + bh * static_cast<size_t>(sk) * d;
  const _Float16* vb = v + bh * static_cast<size_t>(sk) * d;
  _Float16* ob = out + bh * static_cast<size_t>(sq) * d;

  // Q fragments stay in registers: query tile qt, d-step s, depths 32 s + 8 g.
  f16x8 qf[2][STEPS];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int s = 0; s < STEPS; ++s) qf[qt][s] = LoadRow8(qb, q_wave + 16 * qt + lane16, sq, 32 * s + 8 * g, d, VEC);

  f32x4 o[DT][2];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) o[t][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.0f, 0.0f};
  const float scale_log2 = scale * kLog2e;

  // Keys this workgroup needs: all, or with the causal mask those up to its
  // last query.
  int key_blocks = (sk + kKeys - 1) / kKeys;
  if (causal) {
    const int last_query = min(q_block + kQueriesPerBlock, sq) - 1;
    key_blocks = min(key_blocks, last_query / kKeys + 1);
  }

  const __amdgpu_buffer_rsrc_t k_res =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(kb_base), 0, sk * d * 2, kBufferFlags);

  auto k_stage = [&](int stage) { return reinterpret_cast<u32x4*>(lds + stage * S::kStageBytes); };
  auto v_stage = [&](int stage) {
    return reinterpret_cast<uint64_t*>(lds + stage * S::kStageBytes + S::kKChunks * 16);
  };

  // K block kb -> stage: wavefront load j fills rows r0 .. r0 + RPL; lane i
  // lands at chunk i of that KiB: row r0 + i / CH, physical chunk i % CH,
  // holding logical chunk (i % CH) ^ f(row).
  auto load_k = [&](int stage, int kb) {
    u32x4* base = k_stage(stage);
#pragma unroll
    for (int j = 0; j < K_LOADS; ++j) {
      const int r0 = (j * 4 + wave) * RPL;
      const int row = r0 + lane / CH;
      const int logical = (lane % CH) ^ ((row / (16 / CH)) % CH);
      const int key = kb * kKeys + row;
      const int col = logical * 8;
      if (VEC) {
        const int offset = (key < sk && col < d) ? (key * d + col) * 2 : kNoRead;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(k_res, CT_LDS(base + r0 * CH), 16, offset, 0, 0, 0);
      } else {
        base[r0 * CH + lane] = __builtin_bit_cast(u32x4, LoadRow8(kb_base, key, sk, col, d, false));
      }
    }
  };

  // V block kb: unit u = (key group u / (DMAX / 8), d group u % (DMAX / 8))
  // covers keys 4 kg .. 4 kg + 3 and depths 8 dg .. 8 dg + 7; a thread
  // loads the unit's four rows, then writes its 8 columns of 4 keys.
  f16x8 vr[V_PER_THREAD][4];
  auto load_v = [&](int kb) {
#pragma unroll
    for (int i = 0; i < V_PER_THREAD; ++i) {
      const int u = tid + i * kThreads;
      if (V_UNITS % kThreads == 0 || u < V_UNITS) {
        const int kg = u / (DMAX / 8);
        const int dg = u % (DMAX / 8);
#pragma unroll
        for (int r = 0; r < 4; ++r) vr[i][r] = LoadRow8(vb, kb * kKeys + 4 * kg + r, sk, 8 * dg, d, VEC);
      }
    }
  };
  auto store_v = [&](int stage) {
    uint64_t* base = v_stage(stage);
#pragma unroll
    for (int i = 0; i < V_PER_THREAD; ++i) {
      const int u = tid + i * kThreads;
      if (V_UNITS % kThreads == 0 || u < V_UNITS) {
        const int kg = u / (DMAX / 8);
        const int dg = u % (DMAX / 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const f16x4 col = {vr[i][0][e], vr[i][1][e], vr[i][2][e], vr[i][3][e]};
          base[kg * S::kVStride + 8 * dg + e] = __builtin_bit_cast(uint64_t, col);
        }
      }
    }
  };

  if (key_blocks > 0) {
    load_k(0, 0);
    load_v(0);
    store_v(0);
  }
  const int swz = (lane16 / (16 / CH)) % CH;

  for (int kb = 0; kb < key_blocks; ++kb) {
    const int stage = kb & 1;
    if (VEC) __builtin_amdgcn_s_waitcnt(0x0070 | 0x0F00);  // vmcnt(0): this wavefront's K loads landed
    // Every wavefront's K and V of block kb are in LDS, and every wavefront
    // is done with block kb - 1, whose stage takes block kb + 1.
    __syncthreads();
    const bool more = kb + 1 < key_blocks;
    if (more) {
      load_k(stage ^ 1, kb + 1);
      load_v(kb + 1);
    }

    // S^T = K . Q^T for the 4 key tiles and 2 query tiles of this wavefront.
    const u32x4* kst = k_stage(stage);
    f32x4 s_acc[4][2];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) s_acc[t][qt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f16x8 kf = __builtin_bit_cast(f16x8, kst[(16 * t + lane16) * CH + ((4 * s + g) ^ swz)]);
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) s_acc[t][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[qt][s], s_acc[t][qt], 0, 0, 0);
      }
    }

    // Online softmax per query; P in FP16 as the MFMA operand. A block that
    // lies inside the keys and, with the causal mask, at or before this
    // wavefront's first query needs no mask (a wavefront-uniform test).
    const int last_key = (kb + 1) * kKeys - 1;
    const bool needs_mask = last_key >= sk || (causal && last_key > q_wave);
    f16x8 pf[2][2];  // [key step j][query tile]
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int query = q_wave + 16 * qt + lane16;
      float x[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) x[t][r] = s_acc[t][qt][r] * scale_log2;
      if (needs_mask) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kb * kKeys + 16 * t + 4 * g + r;
            if (key >= sk || (causal && key > query)) x[t][r] = -INFINITY;
          }
      }
      float row_max = -INFINITY;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) row_max = fmaxf(row_max, x[t][r]);
      const float m_new = fmaxf(m_run[qt], GroupMax16(row_max));
      // A row with no unmasked key yet keeps m = -inf: its P is 0 and its
      // (zero) accumulator needs no rescale.
      const bool empty = m_new == -INFINITY;
      const float alpha = empty ? 1.0f : __builtin_amdgcn_exp2f(m_run[qt] - m_new);
      float row_sum = 0.0f;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = empty ? 0.0f : __builtin_amdgcn_exp2f(x[t][r] - m_new);
          row_sum += p;
          pf[t >> 1][qt][4 * (t & 1) + r] = static_cast<_Float16>(p);
        }
      l_run[qt] = l_run[qt] * alpha + GroupSum16(row_sum);
      m_run[qt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt][qt] *= alpha;
    }

    // O^T += V^T . P^T over the two 32-key steps.
    const uint64_t* vst = v_stage(stage);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int dcol = 16 * dt + lane16;
        const uint64_t lo = vst[(8 * j + g) * S::kVStride + dcol];
        const uint64_t hi = vst[(8 * j + 4 + g) * S::kVStride + dcol];
        const f16x8 vf = __builtin_bit_cast(f16x8, (ct::u32x4){static_cast<uint32_t>(lo), static_cast<uint32_t>(lo >> 32),
                                                               static_cast<uint32_t>(hi), static_cast<uint32_t>(hi >> 32)});
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) o[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[j][qt], o[dt][qt], 0, 0, 0);
      }
    }

    if (more) store_v(stage ^ 1);
  }

  // Epilogue: lane holds query q_wave + 16 qt + lane16, depths 16 dt + 4 g + 0..3.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int query = q_wave + 16 * qt + lane16;
    if (query >= sq) continue;
    const float inv = l_run[qt] > 0.0f ? 1.0f / l_run[qt] : 0.0f;
    _Float16* orow = ob + static_cast<size_t>(query) * d;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = 16 * dt + 4 * g;
      if (col >= d) continue;
      f16x4 y;
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = static_cast<_Float16>(o[dt][qt][r] * inv);
      if (VEC && col + 4 <= d) {
        *reinterpret_cast<f16x4*>(orow + col) = y;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (col + r < d) orow[col + r] = y[r];
      }
    }
  }
}

}  // namespace

#define CT_DEFINE_ATTENTION(NAME, DMAX)                                                                       \
  CT_KERNEL void __launch_bounds__(kThreads, 2)                                                               \
      attention_fp16_##NAME(const _Float16* q, const _Float16* k, const _Float16* v, _Float16* output,        \
                            int batch, int heads, int sq, int sk, int d, float scale, int causal, void*, void*) { \
    (void)batch;                                                                                              \
    (void)heads;                                                                                              \
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * AttnShape<DMAX>::kStageBytes];                    \
    const bool vec = (d % 8) == 0 && ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |       \
                                       reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(output)) &  \
                                      15) == 0;                                                               \
    if (vec) {                                                                                                \
      AttentionCore<DMAX, true>(lds, q, k, v, output, sq, sk, d, scale, causal);                              \
    } else {                                                                                                  \
      AttentionCore<DMAX, false>(lds, q, k, v, output, sq, sk, d, scale, causal);                             \
    }                                                                                                         \
  }

// NAME: the largest head dimension the variant serves.
CT_DEFINE_ATTENTION(d64, 64)
CT_DEFINE_ATTENTION(d128, 128)
