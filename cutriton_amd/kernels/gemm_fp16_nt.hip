// FP16 Gemm / GemmGelu (+bias) on CDNA4 FP16 MFMA (v_mfma_f32_16x16x32_f16)
// with FP32 accumulation, reading the weight operand from its transposed
// copy.
//
// Semantics follow python/cutriton/triton_kernels/transformer.py:
//   gemm_fp16 (17-60): Y = fp16(sum_k A[m,k] * B[k,n]) with FP32 accumulation;
//   gemm_gelu_fp16 (63-107): Y = fp16(0.5 a (1 + erf(a / sqrt 2))), a the FP32 sum.
// The bias entry points add bias[n] (FP16 widened to FP32) to the FP32 sum
// before the activation. Argument order is the pack ABI of
// transformer.py:256-271 (a, b, [bias,] output, m, n, k, two reserved); the
// engine binds `b` to the [N][K] copy of the constant weight B[K][N], made
// once at constant upload.
//
// With both operands depth-contiguous ([M][K] and [N][K]) every global load
// is a 16-byte run of 8 depths, and so is every MFMA operand fragment: the
// tile goes from global memory to LDS and from LDS to the MFMA without any
// reordering.
//
// Pipeline. A workgroup owns a BM x BN output tile and walks the depth in
// BK-deep tiles through a ring of STAGES LDS stages, with STAGES - 1 tiles
// in flight (straight into LDS, with buffer_load ... lds) behind the MFMAs.
// One barrier per depth tile orders reuse of a stage; it sits in the middle
// of the tile's last MFMA step, so that the next tile's first fragment
// reads and the barrier wait overlap matrix work (measured 5% faster on the
// 4096 x 4096 x 1024 GemmGelu than a barrier between tiles).
//
// LDS layout. A stage holds BM A rows then BN B rows of BK halves, i.e.
// CH = BK / 8 chunks of 16 bytes per row. Chunk c of row r sits at chunk
// position c ^ f(r), f(r) = (r / (16 / CH)) % CH. An LDS read of 16 bytes per
// lane is served 16 lanes at a time over 64 banks (256 bytes); the 16 lanes
// of one phase read one logical chunk of 16 consecutive rows, and f makes
// their (row mod (16 / CH), position) pairs - hence their banks - distinct.
// (CH = 16: f(r) = r % 16, every row starts at bank 0.)
//
// MFMA. v_mfma_f32_16x16x32_f16 sustains a higher rate on gfx950 than the
// 32x32x16 form. A lane's operand fragment is 8 consecutive depths (one
// 16-byte chunk) of row lane % 16: depths 8 * (lane / 16) + 0..7 of the
// 32-deep step.
//
// Operand roles. The MFMA takes the weight fragment as its row operand and
// the activation fragment as its column operand, so it produces the
// transposed 16x16 tile: a lane holds one output row m (lane % 16) and the
// four consecutive columns n = 4 * (lane / 16) + 0..3 in its four registers.
// When n is a multiple of 8 the epilogue stages the FP16 tile in LDS and
// stores whole 16-byte row chunks; otherwise it stores the 8 contiguous bytes
// per lane and tile directly.
#include "common.h"

namespace {

using ct::f16x8;
using ct::f32x4;
using ct::u32x4;

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr int kBufferFlags = 0x00020000;  // gfx9-family raw 32-bit buffer
constexpr int kNoRead = 0x80000000;       // at or beyond every resource's range: reads 0

// Runtime scratch of the split-K variants: 16384 tile counters, then the
// FP32 shares (at most 128 MiB).
constexpr int kSplitMaxTiles = 16384;
constexpr long long kSplitCounterBytes = kSplitMaxTiles * 4LL;
constexpr long long kSplitShareBytes = 128LL << 20;

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

#define CT_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt immediate: vmcnt = n (6 bits, split over [3:0] and [15:14]),
// expcnt and lgkmcnt at their maximum (no wait on them).
template <int N>
__device__ __forceinline__ void WaitVmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070 | 0x0F00);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t HalfResource(const _Float16* base, long long elements) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(base), 0, static_cast<int>(elements * 2),
                                           kBufferFlags);
}

// Eight halves of row `row`, depths [col, col + 8), zero outside the matrix.
// `ld` is the row length (= depth k); used when k is not a multiple of 8.
__device__ __forceinline__ u32x4 LoadChunkScalar(const _Float16* base, int row, int rows, int col, int ld) {
  _Float16 h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    h[e] = (row < rows && col + e < ld) ? base[static_cast<size_t>(row) * ld + col + e] : static_cast<_Float16>(0.0f);
  }
  u32x4 v;
  __builtin_memcpy(&v, h, 16);
  return v;
}

// erf-GELU in FP32 without exp and without branches:
//   GELU(a) = a * Phi(a) = max(a, 0) - |a| * Q(|a|),  Q(x) = erfc(x / sqrt 2) / 2.
// erfc follows Abramowitz & Stegun, Handbook of Mathematical Functions,
// formula 7.1.28: erfc(z) = 1 / (1 + a1 z + ... + a6 z^6)^16 for z >= 0,
// absolute error at most 3e-7. The polynomial is evaluated in x = z * sqrt 2
// with every coefficient (the leading 1 too) scaled by 2^(1/16): its 16th
// power is then twice A&S's, and its reciprocal is Q itself, with no
// separate halving. Coefficient i is a_i / sqrt(2)^i * 2^(1/16). For large x
// the 16th power overflows to +inf and its reciprocal is 0, so GELU(a) =
// max(a, 0) there. FP32 evaluation keeps the total absolute error below 1e-6.
__device__ __forceinline__ float GeluErfAs(float a) {
  const float x = __builtin_fabsf(a);
  float p = 5.6212997e-06f;
  p = __builtin_fmaf(p, x, 5.1055209e-05f);
  p = __builtin_fmaf(p, x, 3.9686137e-05f);
  p = __builtin_fmaf(p, x, 3.4227392e-03f);
  p = __builtin_fmaf(p, x, 2.2076999e-02f);
  p = __builtin_fmaf(p, x, 5.2075163e-02f);
  p = __builtin_fmaf(p, x, 1.0442738f);  // 2^(1/16)
  p = p * p;
  p = p * p;
  p = p * p;
  p = p * p;
  const float q = __builtin_amdgcn_rcpf(p);  // Q(x)
  // x * Q(x) is below 1e-50 from x = 16 on; the clamp keeps +inf finite there
  // (inf * 0) so that GELU(+inf) = +inf.
  return __builtin_fmaf(__builtin_fminf(x, 16.0f), -q, __builtin_fmaxf(a, 0.0f));
}

template <int BM, int BN, int BK, int STAGES>
struct NtShape {
  static constexpr int kChunks = BK / 8;             // 16-byte chunks per row
  static constexpr int kRowsPerLoad = 64 / kChunks;  // rows one wavefront load fills
  static constexpr int kStageChunks = (BM + BN) * kChunks;
  static constexpr int kLdsChunks = STAGES * kStageChunks;
};

// VEC: k is a multiple of 8, so every 16-byte chunk is 8 depths of one row
// and the tiles load straight into LDS; otherwise chunks are assembled
// element by element through registers.
//
// WAVES_K > 1 splits each depth tile among WAVES_K groups of WAVES_M x
// WAVES_N wavefronts: group g multiplies steps [g, g + 1) * STEPS / WAVES_K
// of every stage for the whole output tile, so each wavefront's tile is
// WAVES_K times larger (fewer LDS fragment reads per MFMA), and the groups'
// partial sums are added through the idle LDS ring after the last stage.
//
// SPLIT > 1 gives SPLIT workgroups one output tile, each multiplying an
// equal share of the depth tiles. Each writes its FP32 share to the runtime
// scratch; the last to arrive adds the shares in split order (0, 1, ...:
// the result does not depend on arrival order) and runs the epilogue. The
// hand-off is the one of the split-K convolutions (conv_fp32.hip, where its
// ordering argument is written out): agent-scope atomic stores of the
// shares, a wait for their completion, a barrier, one agent-scope count.
template <int BM, int BN, int BK, int STAGES, int WAVES_M, int WAVES_N, bool GELU, bool BIAS, bool VEC, int WAVES_K = 1,
          int SPLIT = 1>
__device__ __forceinline__ void GemmNtCore(u32x4* __restrict__ lds, const _Float16* __restrict__ a,
                                           const _Float16* __restrict__ bt, const _Float16* __restrict__ bias,
                                           _Float16* __restrict__ output, const int m, const int n, const int k,
                                           void* __restrict__ scratch = nullptr) {
  using S = NtShape<BM, BN, BK, STAGES>;
  constexpr int CH = S::kChunks;
  constexpr int RPL = S::kRowsPerLoad;
  constexpr int TILE_WAVES = WAVES_M * WAVES_N;
  constexpr int WAVES = TILE_WAVES * WAVES_K;
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int TM = WM / 16;
  constexpr int TN = WN / 16;
  constexpr int STEPS = BK / 32;
  constexpr int GROUP_STEPS = STEPS / WAVES_K;  // MFMA steps per stage and wavefront
  static_assert(GROUP_STEPS * WAVES_K == STEPS, "the depth groups split a stage's steps evenly");
  constexpr int LOADS = (BM + BN) / RPL / WAVES;  // load instructions per wavefront and tile
  static_assert(BK == 64 || BK == 128, "depth tile of 2 or 4 MFMA steps");
  static_assert(STAGES >= 2 && STAGES <= 4, "ring of 2..4 stages");
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 16x16 MFMA tile");
  static_assert(LOADS * RPL * WAVES == BM + BN && BM % RPL == 0, "loads split evenly; none straddles A and B");
  static_assert((STAGES - 2) * LOADS < 64, "vmcnt range");
  static_assert(SPLIT == 1 || WAVES_K == 1, "split-K keeps each stage's depth in one workgroup");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Tile order: XCD-contiguous ranges, then groups of 8 row tiles walked
  // column by column so that concurrently running tiles share A and B panels.
  constexpr int GROUP_M = 8;
  const int tiles_m = (m + BM - 1) / BM;
  const int tiles_n = (n + BN - 1) / BN;
  // Split-K: the SPLIT shares of a tile take adjacent slots (one XCD).
  const int slot = ct::XcdContiguousIndex(blockIdx.x, tiles_m * tiles_n * SPLIT);
  const int tile = slot / SPLIT;
  const int split = slot - tile * SPLIT;
  const int group_width = GROUP_M * tiles_n;
  const int group = tile / group_width;
  const int first_m = group * GROUP_M;
  const int group_rows = min(tiles_m - first_m, GROUP_M);
  const int within = tile - group * group_width;
  const int m0 = (first_m + within % group_rows) * BM;
  const int n0 = (within / group_rows) * BN;

  const __amdgpu_buffer_rsrc_t a_res = HalfResource(a, static_cast<long long>(m) * k);
  const __amdgpu_buffer_rsrc_t b_res = HalfResource(bt, static_cast<long long>(n) * k);

  // Loader: wavefront load j of a tile fills rows [R0, R0 + RPL) with
  // R0 = (j * WAVES + wave) * RPL; the hardware puts lane i's 16 bytes at
  // chunk position i of that KiB, i.e. row R0 + i / CH, physical chunk
  // i % CH, which holds logical chunk (i % CH) ^ f(row).
  const int ld_row = lane / CH;
  const int ld_pos = lane % CH;

  auto load_tile = [&](int stage, int kt) {
    u32x4* base = lds + stage * S::kStageChunks;
    const int k0 = kt * BK;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int r0 = (j * WAVES + wave) * RPL;  // wave-uniform
      const int row = r0 + ld_row;
      const int col = k0 + (ld_pos ^ ((row / (16 / CH)) % CH)) * 8;
      const bool is_a = r0 < BM;
      const int gr = is_a ? m0 + row : n0 + row - BM;
      const int rows = is_a ? m : n;
      if (VEC) {
        const int offset = (col < k && gr < rows) ? (gr * k + col) * 2 : kNoRead;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? a_res : b_res, CT_LDS(base + r0 * CH), 16, offset, 0, 0, 0);
      } else {
        base[r0 * CH + lane] = LoadChunkScalar(is_a ? a : bt, gr, rows, col, k);
      }
    }
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[t][i][r] = 0.0f;

  const int wk = wave / TILE_WAVES;  // depth group
  const int wmn = wave % TILE_WAVES;
  const int wm = (wmn / WAVES_N) * WM;
  const int wn = (wmn % WAVES_N) * WN;
  const int lane16 = lane & 15;
  const int quarter = lane >> 4;
  // Fragment rows are lane16 plus a multiple of 16, so f(row) = f(lane16).
  const int a_row = (wm + lane16) * CH;
  const int b_row = (BM + wn + lane16) * CH;
  const int swz = (lane16 / (16 / CH)) % CH;

  // Waits until this wavefront's loads of tile kt have landed, `later` being
  // the number of tiles issued after it (LOADS instructions each).
  auto wait_tile = [&](int later) {
    if (!VEC) return;  // the element-wise path stored synchronously
    if (STAGES >= 4 && later >= 2) {
      WaitVmcnt<(STAGES >= 4 ? 2 : 0) * LOADS>();
    } else if (later >= 1) {
      WaitVmcnt<LOADS>();
    } else {
      WaitVmcnt<0>();
    }
  };

  // This workgroup's depth tiles [kb, ke): all of them, or its share. When
  // the shares would not fit the scratch, share 0 takes the whole depth and
  // the others leave.
  const int k_tiles_all = (k + BK - 1) / BK;
  const bool split_fits = SPLIT > 1 && tiles_m * tiles_n <= kSplitMaxTiles &&
                          static_cast<long long>(tiles_m) * tiles_n * SPLIT * BM * BN * 4 <= kSplitShareBytes;
  if (SPLIT > 1 && !split_fits && split != 0) return;
  const int per_split = split_fits ? (k_tiles_all + SPLIT - 1) / SPLIT : k_tiles_all;
  const int kb = min(k_tiles_all, split * per_split);
  const int ke = min(k_tiles_all, kb + per_split);
  const int k_tiles = ke - kb;

  // Fragments, double-buffered by MFMA step: a lane's 8 depths of one row
  // of A (af) or of B (bf) per 16-row block.
  const int first_step = wk * GROUP_STEPS;
  f16x8 af[2][TM];
  f16x8 bf[2][TN];
  auto read_frags = [&](int stage, int step, f16x8* fa, f16x8* fb) {
    const u32x4* tile_base = lds + stage * S::kStageChunks;
    const int chunk = (4 * (first_step + step) + quarter) ^ swz;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = __builtin_bit_cast(f16x8, tile_base[a_row + i * 16 * CH + chunk]);
#pragma unroll
    for (int t = 0; t < TN; ++t) fb[t] = __builtin_bit_cast(f16x8, tile_base[b_row + t * 16 * CH + chunk]);
  };
  // MFMAs [from, to) of one step, t-major.
  auto mfmas = [&](const f16x8* fa, const f16x8* fb, int from, int to) {
#pragma unroll
    for (int q = from; q < to; ++q)
      acc[q / TM][q % TM] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fb[q / TM], fa[q % TM], acc[q / TM][q % TM], 0, 0, 0);
  };
  constexpr int READS = TM + TN;
  constexpr int MFMAS = TM * TN;
  constexpr int HALF = MFMAS / 2;  // MFMAs of a stage's last step issued before its barrier
  constexpr int TAIL = MFMAS - HALF;
  constexpr int PAIRS = READS < MFMAS ? READS : MFMAS;
  constexpr int TAIL_PAIRS = READS < TAIL ? READS : TAIL;

  // Pipeline. Depth tile kt + 1 is ordered after tile kt by one barrier,
  // placed in the middle of tile kt's last MFMA step: the first HALF of that
  // step's MFMAs are issued, then this wavefront waits for its loads of tile
  // kt + 1, meets the others at the barrier (after which every load of tile
  // kt + 1 has landed and no wavefront reads tile kt's stage any more: the
  // last step's fragments are in registers), issues the loads of tile
  // kt + STAGES into that stage, and reads the first fragments of tile
  // kt + 1 while the other TAIL MFMAs run. The barrier wait and the first
  // read latency of each stage thus hide behind matrix work. Within a stage,
  // the fragments of step s + 1 are read while the MFMAs of step s run; the
  // scheduling groups fix that order (one LDS read after each MFMA).
  //
  // P is the fragment buffer of the stage's first step: with an odd number
  // of steps per stage it alternates from stage to stage.
  auto run_stage = [&](auto p_const, int kt) {
    constexpr int P = decltype(p_const)::value;
    const int stage = kt % STAGES;
#pragma unroll
    for (int step = 0; step + 1 < GROUP_STEPS; ++step) {
      const int cur = (P + step) & 1;
      read_frags(stage, step + 1, af[cur ^ 1], bf[cur ^ 1]);
      mfmas(af[cur], bf[cur], 0, MFMAS);
#pragma unroll
      for (int q = 0; q < PAIRS; ++q) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      if (READS > PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, READS - PAIRS, 0);
      if (MFMAS > PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedMfma, MFMAS - PAIRS, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    constexpr int LAST = (P + GROUP_STEPS - 1) & 1;
    mfmas(af[LAST], bf[LAST], 0, HALF);
    __builtin_amdgcn_sched_barrier(0);
    // After the last stage the wait, the barrier and the fragment reads
    // (of a stage that holds no further tile) are idle work, kept so that
    // the stage stays one straight block of register code.
    wait_tile(min(STAGES - 2, k_tiles - 2 - kt));
    __syncthreads();
    if (kt + STAGES < k_tiles) load_tile(stage, kb + kt + STAGES);
    __builtin_amdgcn_sched_barrier(0);
    read_frags((kt + 1) % STAGES, 0, af[LAST ^ 1], bf[LAST ^ 1]);
    mfmas(af[LAST], bf[LAST], HALF, MFMAS);
#pragma unroll
    for (int q = 0; q < TAIL_PAIRS; ++q) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
    if (READS > TAIL_PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, READS - TAIL_PAIRS, 0);
    if (TAIL > TAIL_PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedMfma, TAIL - TAIL_PAIRS, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: tiles 0 .. STAGES - 2 in flight, tile 0 landed everywhere,
  // tile STAGES - 1 issued, the first fragments read.
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < k_tiles) load_tile(s, kb + s);
  if (k_tiles > 0) {
    wait_tile(min(STAGES - 2, k_tiles - 1));
    __syncthreads();
    if (STAGES - 1 < k_tiles) load_tile(STAGES - 1, kb + STAGES - 1);
    read_frags(0, 0, af[0], bf[0]);
  }
  if constexpr (GROUP_STEPS % 2 == 0) {
    for (int kt = 0; kt < k_tiles; ++kt) run_stage(std::integral_constant<int, 0>(), kt);
  } else {
    for (int kt = 0; kt < k_tiles; kt += 2) {
      run_stage(std::integral_constant<int, 0>(), kt);
      if (kt + 1 < k_tiles) run_stage(std::integral_constant<int, 1>(), kt + 1);
    }
  }

  if (SPLIT > 1 && split_fits) {
    // Scratch: one counter per tile, then [tile][split][wave][register][lane]
    // FP32 shares.
    unsigned* counters = static_cast<unsigned*>(scratch);
    float* shares = reinterpret_cast<float*>(static_cast<char*>(scratch) + kSplitCounterBytes) +
                    static_cast<size_t>(tile) * SPLIT * BM * BN;
    constexpr int WAVE_REGS = TN * TM * 4 * 64;
    float* mine = shares + static_cast<size_t>(split) * BM * BN + wave * WAVE_REGS;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          __hip_atomic_store(mine + ((t * TM + i) * 4 + r) * 64 + lane, acc[t][i][r], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // every share store has completed; the LDS ring is idle
    unsigned* flag = reinterpret_cast<unsigned*>(lds);
    if (tid == 0) *flag = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (*flag != SPLIT - 1) return;
    if (tid == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float* base = shares + wave * WAVE_REGS + lane;
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const float* block = base + (t * TM + i) * 4 * 64;
        float sum[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sum[r] = __hip_atomic_load(const_cast<float*>(block + r * 64), __ATOMIC_RELAXED,
                                                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int sp = 1; sp < SPLIT; ++sp)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sum[r] += __hip_atomic_load(const_cast<float*>(block + static_cast<size_t>(sp) * BM * BN + r * 64),
                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][i][r] = sum[r];
      }
    __syncthreads();  // the flag word is read by every thread before the epilogue reuses the ring
  }

  // Depth groups: group 0 adds the partial sums of groups 1..WAVES_K-1,
  // one group at a time through the idle LDS ring ([wmn][register][lane]
  // floats, one wavefront's accumulators per 64-lane row).
  if constexpr (WAVES_K > 1) {
    constexpr int REGS = TM * TN * 4;
    static_assert(TILE_WAVES * REGS * 64 * 4 <= S::kLdsChunks * 16, "one group's partial sums fit the LDS ring");
    float* partial = reinterpret_cast<float*>(lds) + wmn * REGS * 64 + lane;
#pragma unroll 1
    for (int g = 1; g < WAVES_K; ++g) {
      __syncthreads();  // the ring (or the previous group's sums) is free
      if (wk == g) {
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) partial[((t * TM + i) * 4 + r) * 64] = acc[t][i][r];
      }
      __syncthreads();
      if (wk == 0) {
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[t][i][r] += partial[((t * TM + i) * 4 + r) * 64];
      }
    }
  }

  // Epilogue: lane holds row m = m0 + wm + 16 i + lane16 and columns
  // n = n0 + wn + 16 t + 4 quarter + 0..3.
  if ((n & 7) == 0) {
    // Rows of 16-byte chunks: the finished FP16 tile is staged in the LDS
    // ring (idle after the last depth tile; every load has landed) and
    // leaves as whole 16-byte chunks, consecutive lanes along a row. Stored
    // straight from the MFMA layout, each instruction would write 16 rows x
    // 32 bytes; this way each writes 1 KiB in runs of whole rows, about
    // twice the store rate for the 32 MiB output of a 4096 x 4096 tile grid.
    //
    // LDS tile: BM rows of CHN chunks; chunk c of row r sits at
    // c ^ ((r / RSW) % SWM). The 16 lanes of a quarter write one 8-byte
    // column half of 16 consecutive rows, and the swizzle spreads them over
    // 16 distinct 16-byte bank groups (RSW rows share one 256-byte bank line
    // when rows are shorter than 256 bytes).
    constexpr int CHN = BN / 8;
    constexpr int RSW = BN >= 128 ? 1 : 128 / BN;
    constexpr int SWM = CHN < 16 ? CHN : 16;
    constexpr int THREADS = 64 * WAVES;
    static_assert(BM * BN * 2 <= S::kLdsChunks * 16, "output tile fits the LDS ring");
    static_assert((BM * CHN) % THREADS == 0, "whole rounds of chunk stores");
    __syncthreads();  // every wavefront is done reading the last depth tile (or partial sums)
    _Float16* tile_h = reinterpret_cast<_Float16*>(lds);
    if (wk == 0) {  // depth groups 1.. handed their sums to group 0
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const int lc = wn + t * 16 + 4 * quarter;
        float bias4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (BIAS) {
#pragma unroll
          for (int e = 0; e < 4; ++e) bias4[e] = n0 + lc + e < n ? static_cast<float>(bias[n0 + lc + e]) : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int lr = wm + i * 16 + lane16;
          f16x4 out4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = acc[t][i][e];
            if (BIAS) v += bias4[e];
            if (GELU) v = GeluErfAs(v);
            out4[e] = static_cast<_Float16>(v);
          }
          const int pc = (lc >> 3) ^ ((lr / RSW) % SWM);
          *reinterpret_cast<f16x4*>(tile_h + lr * BN + pc * 8 + (lc & 7)) = out4;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < BM * CHN / THREADS; ++it) {
      const int idx = it * THREADS + tid;
      const int lr = idx / CHN;
      const int c = idx % CHN;
      const int row = m0 + lr;
      const int col = n0 + c * 8;
      const u32x4 v = lds[lr * CHN + (c ^ ((lr / RSW) % SWM))];
      if (row < m && col < n) *reinterpret_cast<u32x4*>(output + static_cast<size_t>(row) * n + col) = v;
    }
    return;
  }
  const bool vec_out = (n & 3) == 0;
  if (wk != 0) return;  // depth groups 1.. handed their sums to group 0
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = n0 + wn + t * 16 + 4 * quarter;
    if (col >= n) continue;
    float bias4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (BIAS) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bias4[e] = col + e < n ? static_cast<float>(bias[col + e]) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = m0 + wm + i * 16 + lane16;
      if (row >= m) continue;
      f16x4 out4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[t][i][e];
        if (BIAS) v += bias4[e];
        if (GELU) v = GeluErfAs(v);
        out4[e] = static_cast<_Float16>(v);
      }
      _Float16* dst = output + static_cast<size_t>(row) * n + col;
      if (vec_out && col + 4 <= n) {
        *reinterpret_cast<f16x4*>(dst) = out4;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (col + e < n) dst[e] = out4[e];
      }
    }
  }
}

}  // namespace

// Entry point body: one LDS allocation shared by the two loader paths.
#define CT_GEMM_NT_BODY(BM, BN, BK, ST, WM, WN, WK, SP, GELU, BIAS, BIAS_PTR)                                   \
  __shared__ u32x4 lds[NtShape<BM, BN, BK, ST>::kLdsChunks];                                                   \
  if ((k & 7) == 0) {                                                                                          \
    GemmNtCore<BM, BN, BK, ST, WM, WN, GELU, BIAS, true, WK, SP>(lds, a, bt, BIAS_PTR, output, m, n, k,       \
                                                                 scratch);                                     \
  } else {                                                                                                     \
    GemmNtCore<BM, BN, BK, ST, WM, WN, GELU, BIAS, false, WK, SP>(lds, a, bt, BIAS_PTR, output, m, n, k,      \
                                                                  scratch);                                    \
  }

// WK depth groups per stage, SP workgroups per output tile (split-K; the
// first reserved argument is then the runtime scratch).
#define CT_DEFINE_GEMM_NT_FULL(NAME, BM, BN, BK, ST, WM, WN, WK, SP)                                         \
  CT_KERNEL void __launch_bounds__(64 * WM * WN * WK)                                                          \
      gemm_nt_fp16_##NAME(const _Float16* a, const _Float16* bt, _Float16* output, int m, int n, int k,        \
                          void* scratch, void*) {                                                              \
    CT_GEMM_NT_BODY(BM, BN, BK, ST, WM, WN, WK, SP, false, false, nullptr)                                     \
  }                                                                                                            \
  CT_KERNEL void __launch_bounds__(64 * WM * WN * WK)                                                          \
      gemm_gelu_nt_fp16_##NAME(const _Float16* a, const _Float16* bt, _Float16* output, int m, int n, int k,   \
                               void* scratch, void*) {                                                         \
    CT_GEMM_NT_BODY(BM, BN, BK, ST, WM, WN, WK, SP, true, false, nullptr)                                      \
  }                                                                                                            \
  CT_KERNEL void __launch_bounds__(64 * WM * WN * WK)                                                          \
      gemm_bias_nt_fp16_##NAME(const _Float16* a, const _Float16* bt, const _Float16* bias,                    \
                               _Float16* output, int m, int n, int k, void* scratch, void*) {                  \
    CT_GEMM_NT_BODY(BM, BN, BK, ST, WM, WN, WK, SP, false, true, bias)                                         \
  }                                                                                                            \
  CT_KERNEL void __launch_bounds__(64 * WM * WN * WK)                                                          \
      gemm_gelu_bias_nt_fp16_##NAME(const _Float16* a, const _Float16* bt, const _Float16* bias,               \
                                    _Float16* output, int m, int n, int k, void* scratch, void*) {             \
    CT_GEMM_NT_BODY(BM, BN, BK, ST, WM, WN, WK, SP, true, true, bias)                                          \
  }

#define CT_DEFINE_GEMM_NT_GROUPS(NAME, BM, BN, BK, ST, WM, WN, WK) \
  CT_DEFINE_GEMM_NT_FULL(NAME, BM, BN, BK, ST, WM, WN, WK, 1)
#define CT_DEFINE_GEMM_NT(NAME, BM, BN, BK, ST, WM, WN) CT_DEFINE_GEMM_NT_GROUPS(NAME, BM, BN, BK, ST, WM, WN, 1)
#define CT_DEFINE_GEMM_NT_SPLIT(NAME, BM, BN, BK, ST, WM, WN, SP) \
  CT_DEFINE_GEMM_NT_FULL(NAME, BM, BN, BK, ST, WM, WN, 1, SP)

// name, BLOCK_M, BLOCK_N, BLOCK_K, stages, wavefronts along M, along N
CT_DEFINE_GEMM_NT(m256n256w4, 256, 256, 64, 2, 2, 2)
CT_DEFINE_GEMM_NT(m256n256w8, 256, 256, 64, 2, 2, 4)
CT_DEFINE_GEMM_NT(m256n128w4, 256, 128, 64, 2, 2, 2)
CT_DEFINE_GEMM_NT(m128n256w4, 128, 256, 64, 2, 2, 2)
CT_DEFINE_GEMM_NT(m128n128w4, 128, 128, 64, 2, 2, 2)
CT_DEFINE_GEMM_NT(m128n128k128w4, 128, 128, 128, 2, 2, 2)
CT_DEFINE_GEMM_NT(m64n128w4, 64, 128, 64, 2, 1, 4)
CT_DEFINE_GEMM_NT(m64n64w4, 64, 64, 64, 2, 2, 2)
CT_DEFINE_GEMM_NT(m256n128w8, 256, 128, 64, 2, 4, 2)
CT_DEFINE_GEMM_NT(m128n256w8, 128, 256, 64, 2, 2, 4)
CT_DEFINE_GEMM_NT(m128n128w8, 128, 128, 64, 2, 2, 4)
CT_DEFINE_GEMM_NT(m128n128k128w8, 128, 128, 128, 2, 2, 4)
CT_DEFINE_GEMM_NT(m128n64w8, 128, 64, 64, 2, 4, 2)
// name, BLOCK_M, BLOCK_N, BLOCK_K, stages, wavefronts along M, along N, depth groups
CT_DEFINE_GEMM_NT_GROUPS(m128n128k128w2x2k2, 128, 128, 128, 2, 2, 2, 2)
// name, BLOCK_M, BLOCK_N, BLOCK_K, stages, wavefronts along M, along N, workgroups per tile
CT_DEFINE_GEMM_NT_SPLIT(m64n64s2, 64, 64, 64, 2, 2, 2, 2)
CT_DEFINE_GEMM_NT_SPLIT(m64n64s4, 64, 64, 64, 2, 2, 2, 4)
CT_DEFINE_GEMM_NT_SPLIT(m128n64s4, 128, 64, 64, 2, 4, 2, 4)
CT_DEFINE_GEMM_NT_SPLIT(m128n128s2, 128, 128, 64, 2, 2, 4, 2)
