// FP32 implicit-GEMM convolution family on CDNA4 FP32 MFMA
// (v_mfma_f32_16x16x4_f32), with the BatchNorm / ReLU / residual-AddRelu
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
// GEMM view of a convolution (NCHW input; the OIHW weight is read as its OHWI copy):
//   rows    m = output channel                        (K_out)
//   columns j = image * P*Q + output pixel            (N*P*Q)
//   depth   d = (kernel row, kernel column, input channel)   (R*S*C)
//   A[m][d] = W[m][r][s][c]  (the weight arrives as OHWI, row-major
//                             [K_out, R*S*C]: d = (r*S + s)*C + c)
//   B[d][j] = X[n][c][oh*sh - ph + r*dh][ow*sw - pw + s*dw]   (zero padded)
//
// Tiling. A workgroup (4 wavefronts) computes a BM x BN output tile and
// walks the depth in BK-deep tiles, double buffered in LDS with the next
// tile's global loads in flight during the MFMAs; the one barrier per tile
// sits in the middle of its last MFMA group, so the next tile's first
// fragment reads overlap matrix work. The wavefronts form a
// WGM x WGN x WGK grid: each owns a (BM/WGM) x (BN/WGN) block of 16x16 MFMA
// accumulators over 1/WGK of every depth tile; WGK > 1 partial sums are added
// through LDS before the epilogue. The 16x16x4 form sustains a higher rate on
// gfx950 than the 32x32x2 one.
//
// Split-K (SPLIT > 1): the grid carries SPLIT workgroups per output tile,
// each accumulating an equal share of the depth tiles. Every share is written
// to the runtime scratch with agent-coherent stores; after the stores have
// completed, one atomic increment of the tile's counter tells the workgroup
// whether it is the last of the tile. The last one reads all shares back and
// adds them in split order (0, 1, ..., SPLIT-1: the result does not depend on
// arrival order), applies the epilogue and resets the counter to zero for the
// next launch. Nothing waits on another workgroup.
//
// LDS holds both operands depth-contiguous, A as [m][d] and B as [j][d]
// (rows padded by 4 floats; gfx950 serves these 16-byte reads at 256 B and
// the 16-byte writes at 128 B per LDS cycle, padded or not, with no
// bank-conflict cycles), so one 16-byte read gives a lane four depths. A 16x16x4
// MFMA takes depth slot q = lane / 16 from every lane; within a depth tile
// the steps take the depths in the order
//   step 4g + e, lane quarter q  ->  depth 16g + 4q + e
// which visits every depth once; the sum is the same set of products.

#include "common.h"

namespace {

using ct::f32x4;

enum Epilogue : int {
  kPlain = 0,             // y = acc
  kBatchNorm = 1,         // y = (acc - mean) * rsqrt(var + eps) * scale + bias, as one FMA
  kBatchNormRelu = 2,     // max(BN, 0)
  kBatchNormAddRelu = 3,  // max(BN + residual, 0)
  kColumnBias = 4,        // y = acc + bias[column]   (Gemm with a bias vector)
};

struct ConvGeometry {
  int n, c, h, w, k, r, s, p, q;
  int stride_h, stride_w, pad_h, pad_w, dil_h, dil_w;
};

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// Raw buffer loads: an offset at or beyond the resource's byte range reads 0,
// which is how zero padding and ragged tile edges are produced without
// per-element branches. kNoRead is such an offset for every resource here
// (tensors stay below 2 GiB).
constexpr int kBufferFlags = 0x00020000;  // gfx9-family raw 32-bit buffer
constexpr int kNoRead = 0x80000000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t Resource(const float* base, long long elements) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, static_cast<int>(elements * 4),
                                           kBufferFlags);
}

__device__ __forceinline__ float LoadF32(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, 0, 0));
}

// Per-lane byte offset plus a wave-uniform one (kept in a scalar register).
// With byte_offset = kNoRead the sum stays at or above 2^31 (the uniform part
// is below 2^31), so the element still reads 0.
__device__ __forceinline__ float LoadF32(__amdgpu_buffer_rsrc_t r, int byte_offset, int uniform_offset) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_offset, uniform_offset, 0));
}

__device__ __forceinline__ f32x4 LoadF32x4(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  typedef int i32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0));
}

// Runtime scratch of the split-K variants: one counter per output tile, then
// the shares, [tile][split][BM*BN] floats in accumulator-register order.
constexpr int kSplitMaxTiles = 16384;
constexpr long long kSplitCounterBytes = kSplitMaxTiles * 4LL;
constexpr long long kSplitShareBytes = 128LL << 20;

// Agent-coherent (sc1) 32-bit accesses for the split-K shares and counters.
__device__ __forceinline__ void StoreShared(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float LoadShared(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS layout of one ConvCore instantiation (in floats).
template <int BM, int BN, int BK, int WGM, int WGN, int WGK>
struct ConvLds {
  static constexpr int kRow = BK + 4;                      // padded depth row
  static constexpr int kA = BM * kRow;                     // one A buffer
  static constexpr int kB = BN * kRow;                     // one B buffer
  static constexpr int kTiles = 2 * (kA + kB);
  static constexpr int kAccRegs = (BM / WGM / 16) * (BN / WGN / 16) * 4;
  static constexpr int kReduce = (WGK - 1) * WGM * WGN * kAccRegs * 64;
  static constexpr int kEpi = 2 * BM;
  static constexpr int kFloats = (kTiles > kReduce ? kTiles : kReduce) + kEpi;
};

// POINTWISE: 1x1 kernel without padding, so every gathered pixel is inside
// the image and a depth row is one input channel.
template <int BM, int BN, int BK, int WGM, int WGN, int WGK, int EPI, bool POINTWISE, int SPLIT = 1,
          bool CHANNEL_RUN = false>
__device__ __forceinline__ void ConvCore(float* __restrict__ smem, const float* __restrict__ x,
                                         const float* __restrict__ weight, const float* __restrict__ scale,
                                         const float* __restrict__ bias, const float* __restrict__ mean,
                                         const float* __restrict__ variance, const float* __restrict__ residual,
                                         float* __restrict__ output, const ConvGeometry g, const float epsilon,
                                         void* __restrict__ scratch = nullptr) {
  using L = ConvLds<BM, BN, BK, WGM, WGN, WGK>;
  constexpr int WM = BM / WGM;
  constexpr int WN = BN / WGN;
  constexpr int TM = WM / 16;
  constexpr int TN = WN / 16;
  constexpr int ROW = L::kRow;
  constexpr int GROUPS = BK / 16;                // 16-depth groups per tile
  constexpr int WAVE_GROUPS = GROUPS / WGK;      // groups per wavefront
  constexpr int THREADS = 64 * WGM * WGN * WGK;     // one wavefront per wave-grid cell
  constexpr int A_CHUNKS = BM * BK / 4 / THREADS;   // float4 chunks per thread
  constexpr int B_RUN = BK * BN / THREADS;          // depths per thread (one column)
  static_assert(TM >= 1 && TN >= 1 && WAVE_GROUPS >= 1, "wave tile too small");
  static_assert(A_CHUNKS >= 1 && A_CHUNKS * THREADS * 4 == BM * BK, "A tile split");
  static_assert(THREADS % BN == 0 && B_RUN % 4 == 0, "B tile split");
  static_assert(SPLIT == 1 || WGK == 1, "split-K variants keep the depth whole inside a workgroup");

  float* a_tile = smem;                  // [2][BM][ROW]
  float* b_tile = smem + 2 * L::kA;      // [2][BN][ROW]
  constexpr int EPI_BASE = L::kTiles > L::kReduce ? L::kTiles : L::kReduce;
  // BatchNorm folded per output channel: y = acc * epi_mul + epi_add with
  // epi_mul = scale * rsqrt(var + eps), epi_add = bias - mean * epi_mul.
  float* epi_mul = smem + EPI_BASE;
  float* epi_add = epi_mul + BM;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int pq = g.p * g.q;
  const int hw = g.h * g.w;
  const int rs = g.r * g.s;
  const int depth = g.c * rs;
  const int columns = g.n * pq;
  // Vector weight loads need every weight row to start 16-byte aligned.
  const bool vec_a = (depth & 3) == 0;

  const int tiles_n = (columns + BN - 1) / BN;
  const int tiles_m = (g.k + BM - 1) / BM;
  const int tiles = tiles_n * tiles_m;
  const int depth_tiles = (depth + BK - 1) / BK;

  // ---- B (im2col) loader: one fixed column per thread, a run of B_RUN
  // consecutive depths. The run start is wave-uniform, so the (channel,
  // kernel row, kernel column) walk stays in scalar registers.
  const int b_col = tid % BN;
  const int b_run0 = __builtin_amdgcn_readfirstlane(tid / BN) * B_RUN;
  const __amdgpu_buffer_rsrc_t x_res = Resource(x, static_cast<long long>(g.n) * g.c * hw);
  const __amdgpu_buffer_rsrc_t w_res = Resource(weight, static_cast<long long>(g.k) * depth);
  int m0 = 0, n0 = 0;
  bool col_ok = false;
  int ih0 = 0, iw0 = 0;
  // Element offset of (image, channel 0, ih0, iw0) and of the pointwise
  // gather position; columns past the end read nothing.
  int lane_base = 0, pw_base = 0;

  // Selects output tile `t` (m-fastest order) and loads its per-channel
  // epilogue parameters into LDS (visible after the next barrier).
  auto setup_tile = [&](int t) {
    m0 = (t % tiles_m) * BM;
    n0 = (t / tiles_m) * BN;
    if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) {
      for (int i = tid; i < BM; i += THREADS) {
        const int m = m0 + i;
        const bool ok = m < g.k;
        const float mul = ok ? scale[m] * rsqrtf(variance[m] + epsilon) : 0.0f;
        epi_mul[i] = mul;
        epi_add[i] = ok ? bias[m] - mean[m] * mul : 0.0f;
      }
    }
    const int j = n0 + b_col;
    col_ok = j < columns;
    const int img = col_ok ? j / pq : 0;
    const int pix = col_ok ? j - img * pq : 0;
    const int oh = pix / g.q;
    const int ow = pix - oh * g.q;
    ih0 = oh * g.stride_h - g.pad_h;
    iw0 = ow * g.stride_w - g.pad_w;
    lane_base = img * g.c * hw + ih0 * g.w + iw0;
    pw_base = img * g.c * hw + (oh * g.stride_h) * g.w + ow * g.stride_w;
  };

  // Register staging of one depth tile between its global loads and its LDS
  // store (the next tile's loads are in flight during the current MFMAs).
  struct Stage {
    f32x4 a[A_CHUNKS];
    float b[B_RUN];
  };
  // Tiles of up to 32 depths keep two tiles' loads in flight (tile kt + 2
  // is loaded while tile kt + 1 waits in the other registers for its LDS
  // store): one such tile is too little MFMA work to cover a load's
  // latency. Only where the second set of staging registers is small.
  constexpr bool PREFETCH2 = WGK == 1 && BK <= 32 && A_CHUNKS * 4 + B_RUN <= 16;
  Stage st[PREFETCH2 ? 2 : 1];

  // Channel-run depth order (CHANNEL_RUN, C % BK == 0): depth tile t holds
  // channels [c0, c0 + BK) of one kernel tap (r, s); tiles take c fastest,
  // then s, then r. Inside a tile the tap is fixed, so a B element needs no
  // index arithmetic and the padding test is made once per tile. The loads
  // always come in increasing tile order, so the tap walks forward.
  int run_c0 = 0, run_r = 0, run_s = 0;  // next tile to load
  auto seek_run = [&](int kt) {
    const int per_tap = g.c / BK;
    const int tap = kt / per_tap;
    run_c0 = (kt - tap * per_tap) * BK;
    run_r = tap / g.s;
    run_s = tap - run_r * g.s;
  };
  auto load_run = [&](Stage& st) {
    f32x4* ra = st.a;
    float* rb = st.b;
    const int tap = run_r * g.s + run_s;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int chunk = tid + THREADS * i;
      const int m = m0 + chunk / (BK / 4);
      const int c = run_c0 + (chunk % (BK / 4)) * 4;
      // OHWI weight: the channels of one tap are contiguous.
      ra[i] = LoadF32x4(w_res, m < g.k ? (m * depth + tap * g.c + c) * 4 : kNoRead);
    }
    const int dh = run_r * g.dil_h;
    const int dw = run_s * g.dil_w;
    const bool inside = col_ok && static_cast<unsigned>(ih0 + dh) < static_cast<unsigned>(g.h) &&
                        static_cast<unsigned>(iw0 + dw) < static_cast<unsigned>(g.w);
    const int off = inside ? (lane_base + (run_c0 + b_run0) * hw + dh * g.w + dw) * 4 : kNoRead;
#pragma unroll
    for (int e = 0; e < B_RUN; ++e) rb[e] = LoadF32(x_res, off, e * hw * 4);
    run_c0 += BK;
    if (run_c0 == g.c) {
      run_c0 = 0;
      if (++run_s == g.s) {
        run_s = 0;
        ++run_r;
      }
    }
  };

  auto load_tile = [&](Stage& st, int d0) {
    if (CHANNEL_RUN) {
      load_run(st);
      return;
    }
    f32x4* ra = st.a;
    float* rb = st.b;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int chunk = tid + THREADS * i;
      const int m = m0 + chunk / (BK / 4);
      const int d = d0 + (chunk % (BK / 4)) * 4;
      const int base = m * depth + d;
      if (vec_a) {
        ra[i] = LoadF32x4(w_res, (m < g.k && d < depth) ? base * 4 : kNoRead);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[i][e] = LoadF32(w_res, (m < g.k && d + e < depth) ? (base + e) * 4 : kNoRead);
      }
    }
    const int d = d0 + b_run0;  // wave-uniform
    if (POINTWISE) {
#pragma unroll
      for (int e = 0; e < B_RUN; ++e) {
        rb[e] = LoadF32(x_res, (col_ok && d + e < depth) ? (pw_base + (d + e) * hw) * 4 : kNoRead);
      }
    } else {
      // Depth order of an OHWI weight row: d = (kr * S + ks) * C + ci.
      const int tap = d / g.c;
      int ci = d - tap * g.c;
      int kr = tap / g.s;
      int ks = tap - kr * g.s;
#pragma unroll
      for (int e = 0; e < B_RUN; ++e) {
        const int dh = kr * g.dil_h;
        const int dw = ks * g.dil_w;
        const bool inside = col_ok && (d + e) < depth &&
                            static_cast<unsigned>(ih0 + dh) < static_cast<unsigned>(g.h) &&
                            static_cast<unsigned>(iw0 + dw) < static_cast<unsigned>(g.w);
        rb[e] = LoadF32(x_res, inside ? (lane_base + ci * hw + dh * g.w + dw) * 4 : kNoRead);
        if (++ci == g.c) {
          ci = 0;
          if (++ks == g.s) {
            ks = 0;
            ++kr;
          }
        }
      }
    }
  };

  auto store_tile = [&](const Stage& st, int buf) {
    const f32x4* ra = st.a;
    const float* rb = st.b;
    float* at = a_tile + buf * L::kA;
    float* bt = b_tile + buf * L::kB;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int chunk = tid + THREADS * i;
      *reinterpret_cast<f32x4*>(at + (chunk / (BK / 4)) * ROW + (chunk % (BK / 4)) * 4) = ra[i];
    }
#pragma unroll
    for (int e = 0; e < B_RUN; e += 4) {
      const f32x4 v = {rb[e], rb[e + 1], rb[e + 2], rb[e + 3]};
      *reinterpret_cast<f32x4*>(bt + b_col * ROW + b_run0 + e) = v;
    }
  };

  f32x4 acc[TM][TN];

  const int wk = wave / (WGM * WGN);
  const int wmn = wave % (WGM * WGN);
  const int wm = (wmn / WGN) * WM;
  const int wn = (wmn % WGN) * WN;
  const int quarter = lane >> 4;
  const int lane16 = lane & 15;

  // Fragments, double-buffered by 16-depth group: a lane's four depths of
  // one row of A (av) or of B (bv) per 16-row block.
  f32x4 av[2][TM];
  f32x4 bv[2][TN];
  auto read_frags = [&](int buf, int gi, f32x4* fa, f32x4* fb) {
    const float* at = a_tile + buf * L::kA + (wm + lane16) * ROW + 4 * quarter;
    const float* bt = b_tile + buf * L::kB + (wn + lane16) * ROW + 4 * quarter;
    const int col = (wk * WAVE_GROUPS + gi) * 16;
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[i] = *reinterpret_cast<const f32x4*>(at + i * 16 * ROW + col);
#pragma unroll
    for (int t = 0; t < TN; ++t) fb[t] = *reinterpret_cast<const f32x4*>(bt + t * 16 * ROW + col);
  };
  // MFMAs [from, to) of one group, in (e, i, t) order.
  auto mfmas = [&](const f32x4* fa, const f32x4* fb, int from, int to) {
#pragma unroll
    for (int q = from; q < to; ++q) {
      const int e = q / (TM * TN);
      const int i = (q / TN) % TM;
      const int t = q % TN;
      acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i][e], fb[t][e], acc[i][t], 0, 0, 0);
    }
  };
  constexpr int READS = TM + TN;
  constexpr int MFMAS = 4 * TM * TN;
  constexpr int HALF = MFMAS / 2;  // MFMAs of a tile's last group issued before its barrier
  constexpr int TAIL = MFMAS - HALF;
  constexpr int PAIRS = READS < MFMAS ? READS : MFMAS;
  constexpr int TAIL_PAIRS = READS < TAIL ? READS : TAIL;

  // Residual of the lane's outputs (residual-join epilogue without split-K):
  // loaded before the last depth tile is multiplied, so its latency hides
  // behind those MFMAs instead of stalling the epilogue.
  // Staged epilogue: when an image's output plane is a whole number of
  // 16-byte groups (P*Q % 4 == 0), the finished tile goes through LDS so that
  // every lane reads its residual and writes its output as 16 bytes of four
  // consecutive pixels of one channel, a wavefront covering whole 256-byte
  // runs, instead of four 4-byte values of four channels.
  constexpr int SROW = BN + 4;  // staged row: BN outputs of one channel, padded
  constexpr int SGROUPS = BN / 4;
  constexpr int SITEMS = BM * SGROUPS / THREADS;  // 16-byte groups per thread
  constexpr bool kStagedEpilogue = WGK == 1 && BM * SROW <= L::kTiles && SITEMS * THREADS == BM * SGROUPS;
  const bool staged_epilogue = kStagedEpilogue && (pq & 3) == 0;

  constexpr bool PREFETCH_RESIDUAL = EPI == kBatchNormAddRelu && SPLIT == 1;
  float res_pre[PREFETCH_RESIDUAL ? TM : 1][PREFETCH_RESIDUAL ? TN : 1][4];
  auto prefetch_residual = [&]() {
    if (!PREFETCH_RESIDUAL || wk != 0 || staged_epilogue) return;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int col = n0 + wn + t * 16 + lane16;
      const bool col_ok = col < columns;
      const int cimg = col_ok ? col / pq : 0;
      const size_t col_base = static_cast<size_t>(cimg) * g.k * pq + (col - cimg * pq);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm + i * 16 + 4 * quarter + r;
          res_pre[PREFETCH_RESIDUAL ? i : 0][PREFETCH_RESIDUAL ? t : 0][r] =
              (col_ok && row < g.k) ? residual[col_base + static_cast<size_t>(row) * pq] : 0.0f;
        }
    }
  };

  // Accumulates depth tiles [kb, ke) of the current output tile into acc.
  // Ends with a barrier, after which the LDS tiles are free.
  //
  // Depth tile kt + 1 is ordered after tile kt by one barrier in the middle
  // of tile kt's last group of MFMAs: the first HALF of that group's MFMAs
  // are issued, the staged loads of tile kt + 1 are written to the other
  // LDS buffer, the barrier makes them visible (no wavefront reads tile
  // kt's buffer after it: the last group's fragments are in registers), and
  // the first fragments of tile kt + 1 are read while the other TAIL MFMAs
  // run, so the barrier wait and the first read latency of each tile hide
  // behind matrix work. Within a tile, the fragments of group g + 1 are read
  // while the MFMAs of group g run; the scheduling groups fix that order.
  //
  // Q is the tile's parity; P is the fragment buffer of the tile's first
  // group (with an odd number of groups per wavefront it alternates from
  // tile to tile, like Q); MORE says whether another tile follows. The last tile is peeled off the loop: it
  // loads nothing and prefetches the residual instead, so the loop body
  // holds no residual registers.
  auto depth_tile = [&](auto q_const, auto more_const, int kt, int cur) {
    constexpr int Q = decltype(q_const)::value;  // parity of the tile
    constexpr int P = WAVE_GROUPS % 2 ? Q : 0;
    constexpr bool MORE = decltype(more_const)::value;
    // PREFETCH2: tile kt + 1 is in st[Q ^ 1], tile kt + 2 goes to st[Q]
    // (stored one tile ago). A load past the last tile reads zeros or data
    // that is never stored.
    constexpr int LOAD = PREFETCH2 ? Q : 0;
    constexpr int STORE = PREFETCH2 ? Q ^ 1 : 0;
    if (MORE) {
      load_tile(st[LOAD], (kt + (PREFETCH2 ? 2 : 1)) * BK);
    } else {
      prefetch_residual();
    }
#pragma unroll
    for (int gi = 0; gi + 1 < WAVE_GROUPS; ++gi) {
      const int c = (P + gi) & 1;
      read_frags(cur, gi + 1, av[c ^ 1], bv[c ^ 1]);
      mfmas(av[c], bv[c], 0, MFMAS);
#pragma unroll
      for (int q = 0; q < PAIRS; ++q) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      if (READS > PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, READS - PAIRS, 0);
      if (MFMAS > PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedMfma, MFMAS - PAIRS, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    constexpr int LAST = (P + WAVE_GROUPS - 1) & 1;
    mfmas(av[LAST], bv[LAST], 0, HALF);
    __builtin_amdgcn_sched_barrier(0);
    if (MORE) store_tile(st[STORE], cur ^ 1);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    if (MORE) read_frags(cur ^ 1, 0, av[LAST ^ 1], bv[LAST ^ 1]);
    mfmas(av[LAST], bv[LAST], HALF, MFMAS);
    if (MORE) {
#pragma unroll
      for (int q = 0; q < TAIL_PAIRS; ++q) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
      if (READS > TAIL_PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, READS - TAIL_PAIRS, 0);
      if (TAIL > TAIL_PAIRS) __builtin_amdgcn_sched_group_barrier(kSchedMfma, TAIL - TAIL_PAIRS, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using More = std::integral_constant<bool, true>;
  using Last = std::integral_constant<bool, false>;
  auto run_depth = [&](int kb, int ke) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][t][r] = 0.0f;
    if (CHANNEL_RUN) seek_run(kb);
    load_tile(st[0], kb * BK);
    store_tile(st[0], 0);
    if (PREFETCH2) load_tile(st[PREFETCH2 ? 1 : 0], (kb + 1) * BK);
    __syncthreads();
    if (ke <= kb) return;
    read_frags(0, 0, av[0], bv[0]);
    // Tiles go in pairs so that the parity of a tile (its LDS buffer, its
    // staging registers, its first fragment buffer) is a constant.
    int kt = kb;
    for (; kt + 2 < ke; kt += 2) {
      depth_tile(P0(), More(), kt, 0);
      depth_tile(P1(), More(), kt + 1, 1);
    }
    if (kt + 1 < ke) {
      depth_tile(P0(), More(), kt, 0);
      depth_tile(P1(), Last(), kt + 1, 1);
    } else {
      depth_tile(P0(), Last(), kt, 0);
    }
  };

  // Epilogue of the current tile. Lane holds column (lane % 16) of each
  // 16x16 tile and rows 4*(lane/16) + r for register r: four consecutive
  // output channels of one pixel.
  auto from_acc = [&](int i, int t, int r) { return acc[i][t][r]; };
  auto store_output = [&](auto value) {
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int col = n0 + wn + t * 16 + lane16;
      if (col >= columns) continue;
      const int cimg = col / pq;
      const int cpix = col - cimg * pq;
      const size_t col_base = static_cast<size_t>(cimg) * g.k * pq + cpix;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int lrow0 = wm + i * 16 + 4 * quarter;
        f32x4 mul = {1.0f, 1.0f, 1.0f, 1.0f}, add = {0.0f, 0.0f, 0.0f, 0.0f};
        if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) {
          // The four rows are consecutive channels: one 16-byte read each.
          mul = *reinterpret_cast<const f32x4*>(epi_mul + lrow0);
          add = *reinterpret_cast<const f32x4*>(epi_add + lrow0);
        }
        float res[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (PREFETCH_RESIDUAL) {
#pragma unroll
          for (int r = 0; r < 4; ++r) res[r] = res_pre[PREFETCH_RESIDUAL ? i : 0][PREFETCH_RESIDUAL ? t : 0][r];
        } else if (EPI == kBatchNormAddRelu) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = m0 + lrow0 + r;
            if (row < g.k) res[r] = residual[col_base + static_cast<size_t>(row) * pq];
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + lrow0 + r;
          if (row >= g.k) continue;
          float v = value(i, t, r);
          const size_t at = col_base + static_cast<size_t>(row) * pq;
          if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v = fmaf(v, mul[r], add[r]);
          if (EPI == kBatchNormAddRelu) v += res[r];
          if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v = fmaxf(v, 0.0f);
          if (EPI == kColumnBias) v += bias[col];
          output[at] = v;
        }
      }
    }
  };

  if (SPLIT == 1) {
    setup_tile(ct::XcdContiguousIndex(blockIdx.x + blockIdx.y * gridDim.x, tiles));
    run_depth(0, depth_tiles);
  } else {
    // Grid (tiles_n, tiles_m, SPLIT); the shares of one tile get adjacent
    // slots, so they run on one XCD at about the same time.
    const int linear = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    const int slot = ct::XcdContiguousIndex(linear, tiles * SPLIT);
    const int tile = slot / SPLIT;
    const int split = slot - tile * SPLIT;
    const bool fits = tiles <= kSplitMaxTiles &&
                      static_cast<long long>(tiles) * SPLIT * BM * BN * 4 <= kSplitShareBytes;
    if (!fits) {
      // Scratch too small for this shape: share 0 computes the whole depth.
      if (split != 0) return;
      setup_tile(tile);
      run_depth(0, depth_tiles);
    } else {
      const int per = (depth_tiles + SPLIT - 1) / SPLIT;
      const int kb = min(depth_tiles, split * per);
      const int ke = min(depth_tiles, kb + per);
      setup_tile(tile);
      run_depth(kb, ke);
      unsigned* counters = static_cast<unsigned*>(scratch);
      float* shares = reinterpret_cast<float*>(static_cast<char*>(scratch) + kSplitCounterBytes) +
                      static_cast<size_t>(tile) * SPLIT * BM * BN;
      constexpr int WAVE_REGS = TM * TN * 4 * 64;  // one wavefront's accumulators
      float* mine = shares + static_cast<size_t>(split) * BM * BN + wave * WAVE_REGS;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) StoreShared(mine + ((i * TN + t) * 4 + r) * 64 + lane, acc[i][t][r]);
      // Ordering of the hand-off. The shares are stored and loaded with
      // agent-scope atomics, which gfx950 issues with the device-coherence
      // bit (sc1): a store is written through to the device's coherence
      // point, and its vmcnt decrement comes back once it is there; a load
      // is served at that point, never from a stale L1 or L2 line. The
      // count is an agent-scope read-modify-write: its updates form one
      // order for the whole device.
      //  1. Each wave waits (vmcnt 0) until its share stores are at the
      //     coherence point; the barrier then holds thread 0 until every wave
      //     has waited, so the whole share is visible before the count.
      //  2. The workgroup that reads SPLIT - 1 comes after every other
      //     share's count in that order, hence after its stores.
      //  3. Thread 0 waits for the count's return value before it writes the
      //     flag, and the second barrier orders the flag before every share
      //     load, so no share load is issued before the count has returned.
      //  4. The counter's relaxed reset is ordered for the next launch by the
      //     kernel boundary.
      // In the language memory model these relaxed atomics order nothing
      // across locations; a release on the count and an acquire fence in the
      // last workgroup would. On gfx950 those become a write-back and an
      // invalidate of the whole L2 per workgroup, which made the ResNet-50
      // step 5 % slower (the tuner then dropped split-K for most layers), so
      // the hand-off relies on the ordering above instead.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      unsigned* flag = reinterpret_cast<unsigned*>(smem);
      if (tid == 0) {
        const unsigned arrived = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
        *flag = arrived;
      }
      __syncthreads();
      const unsigned arrived = *flag;
      if (arrived != SPLIT - 1) return;
      if (tid == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // Sum all shares in split order from the scratch (this workgroup's own
      // share is there too, stored and completed above).
      // The loads of one accumulator block per share are issued together so
      // that their latencies overlap.
      const float* base = shares + wave * WAVE_REGS + lane;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          const float* block = base + (i * TN + t) * 4 * 64;
          float sum[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) sum[r] = LoadShared(block + r * 64);
#pragma unroll
          for (int sp = 1; sp < SPLIT; ++sp) {
            float part[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) part[r] = LoadShared(block + static_cast<size_t>(sp) * BM * BN + r * 64);
#pragma unroll
            for (int r = 0; r < 4; ++r) sum[r] += part[r];
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][t][r] = sum[r];
        }
    }
  }

  // ---- Depth-split partial sums: wavefronts wk > 0 add theirs to wk == 0
  // through LDS (register r of lane l lands at [slot][r][l]).
  if (WGK > 1) {
    constexpr int REGS = TM * TN * 4;
    float* red = smem;
    if (wk > 0) {
      float* mine = red + ((wk - 1) * WGM * WGN + wmn) * REGS * 64;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) mine[((i * TN + t) * 4 + r) * 64 + lane] = acc[i][t][r];
    }
    __syncthreads();
    if (wk > 0) return;
#pragma unroll 1
    for (int s = 1; s < WGK; ++s) {
      const float* theirs = red + ((s - 1) * WGM * WGN + wmn) * REGS * 64;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][t][r] += theirs[((i * TN + t) * 4 + r) * 64 + lane];
    }
  }

  if constexpr (kStagedEpilogue) {
    if (staged_epilogue) {
      // The residual loads go out first; their latency overlaps the LDS
      // transpose. Group item = row * SGROUPS + cg: channel m0 + row,
      // columns n0 + 4 cg .. + 3, all in one image (P*Q % 4 == 0); its
      // offset is recomputed after the transpose rather than kept live.
      auto group_at = [&](int item, bool& ok) -> size_t {
        const int row = item / SGROUPS;
        const int col = n0 + 4 * (item - row * SGROUPS);
        const int m = m0 + row;
        ok = m < g.k && col < columns;  // columns % 4 == 0: a group is whole or outside
        const int cimg = ok ? col / pq : 0;
        return ok ? (static_cast<size_t>(cimg) * g.k + m) * pq + (col - cimg * pq) : 0;
      };
      f32x4 res[EPI == kBatchNormAddRelu ? SITEMS : 1];
      if constexpr (EPI == kBatchNormAddRelu) {
#pragma unroll
        for (int it = 0; it < SITEMS; ++it) {
          bool ok;
          const size_t at = group_at(tid + it * THREADS, ok);
          res[it] = ok ? *reinterpret_cast<const f32x4*>(residual + at) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
      __syncthreads();  // the LDS tiles (and the split-K flag) are free
      float* stage = smem;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) stage[(wm + i * 16 + 4 * quarter + r) * SROW + wn + t * 16 + lane16] = acc[i][t][r];
      __syncthreads();
#pragma unroll
      for (int it = 0; it < SITEMS; ++it) {
        const int item = tid + it * THREADS;
        const int row = item / SGROUPS;
        const int cg = item - row * SGROUPS;
        bool ok;
        const size_t at = group_at(item, ok);
        f32x4 v = *reinterpret_cast<const f32x4*>(stage + row * SROW + 4 * cg);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (EPI == kBatchNorm || EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) {
            v[e] = fmaf(v[e], epi_mul[row], epi_add[row]);
          }
          if (EPI == kBatchNormAddRelu) v[e] += res[EPI == kBatchNormAddRelu ? it : 0][e];
          if (EPI == kBatchNormRelu || EPI == kBatchNormAddRelu) v[e] = fmaxf(v[e], 0.0f);
          if (EPI == kColumnBias) v[e] += bias[n0 + 4 * cg + e];
        }
        if (ok) *reinterpret_cast<f32x4*>(output + at) = v;
      }
      return;
    }
  }
  store_output(from_acc);
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

// One LDS buffer per kernel, shared by the pointwise and general paths.
// Loader choice: channel runs when C is a multiple of the depth tile, else
// the pointwise gather for unpadded 1x1, else the general (c, r, s) walk.
#define CT_DISPATCH(BM, BN, BK, WGM, WGN, WGK, EPI, ...)                                         \
  __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, WGK>::kFloats];  \
  if (c % BK == 0) {                                                                                \
    ConvCore<BM, BN, BK, WGM, WGN, WGK, EPI, false, 1, true>(smem, __VA_ARGS__);                \
  } else if (r == 1 && s == 1 && pad_h == 0 && pad_w == 0) {                                        \
    ConvCore<BM, BN, BK, WGM, WGN, WGK, EPI, true>(smem, __VA_ARGS__);                       \
  } else {                                                                                          \
    ConvCore<BM, BN, BK, WGM, WGN, WGK, EPI, false>(smem, __VA_ARGS__);                      \
  }

#define CT_DEFINE_CONV_VARIANTS(NAME, BM, BN, BK, WGM, WGN, WGK, MIN_GROUPS)                            \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK, MIN_GROUPS) conv_bn_relu_fp32_##NAME(          \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,    \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {                \
    CT_DISPATCH(BM, BN, BK, WGM, WGN, WGK, kBatchNormRelu, x, weight, scale, bias, mean, variance,      \
                nullptr, output, CT_CONV_GEOMETRY, epsilon)                                             \
  }                                                                                                     \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK, MIN_GROUPS) conv_bn_fp32_##NAME(               \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,    \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void*, void*) {                \
    CT_DISPATCH(BM, BN, BK, WGM, WGN, WGK, kBatchNorm, x, weight, scale, bias, mean, variance, nullptr, \
                output, CT_CONV_GEOMETRY, epsilon)                                                      \
  }                                                                                                     \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK, MIN_GROUPS) conv_bn_add_relu_fp32_##NAME(      \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,    \
      const float* variance, const float* residual, float* output, CT_CONV_DIMS, float epsilon, void*,  \
      void*) {                                                                                          \
    CT_DISPATCH(BM, BN, BK, WGM, WGN, WGK, kBatchNormAddRelu, x, weight, scale, bias, mean, variance,   \
                residual, output, CT_CONV_GEOMETRY, epsilon)                                            \
  }                                                                                                     \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK, MIN_GROUPS) conv_fp32_##NAME(const float* x,   \
                                                              const float* weight, float* output,       \
                                                              CT_CONV_DIMS, void*, void*) {             \
    CT_DISPATCH(BM, BN, BK, WGM, WGN, WGK, kPlain, x, weight, nullptr, nullptr, nullptr, nullptr,       \
                nullptr, output, CT_CONV_GEOMETRY, 0.0f)                                                \
  }

// name, BM, BN, BK, WGM, WGN, WGK, workgroups per CU the registers must allow
CT_DEFINE_CONV_VARIANTS(m128n128, 128, 128, 32, 2, 2, 1, 1)
CT_DEFINE_CONV_VARIANTS(m64n256, 64, 256, 16, 1, 4, 1, 1)
CT_DEFINE_CONV_VARIANTS(m64n128, 64, 128, 32, 1, 2, 2, 1)
CT_DEFINE_CONV_VARIANTS(m128n64, 128, 64, 32, 2, 1, 2, 1)
CT_DEFINE_CONV_VARIANTS(m64n64, 64, 64, 32, 2, 2, 1, 4)
CT_DEFINE_CONV_VARIANTS(m64n64k16, 64, 64, 16, 2, 2, 1, 5)
CT_DEFINE_CONV_VARIANTS(m64n128k16, 64, 128, 16, 2, 2, 1, 1)
CT_DEFINE_CONV_VARIANTS(m128n64k16, 128, 64, 16, 2, 2, 1, 1)
CT_DEFINE_CONV_VARIANTS(m64n64k64, 64, 64, 64, 2, 2, 1, 1)
CT_DEFINE_CONV_VARIANTS(m32n128, 32, 128, 32, 1, 4, 1, 1)
CT_DEFINE_CONV_VARIANTS(m128n128k16, 128, 128, 16, 2, 2, 1, 1)

// Split-K entry points: the first reserved argument is the runtime scratch
// (kSplitCounterBytes + kSplitShareBytes, zero-initialised by the engine).
#define CT_SPLIT_DISPATCH(BM, BN, BK, WGM, WGN, SPLIT, EPI, ...)                                 \
  __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, 1>::kFloats];    \
  if (c % BK == 0) {                                                                                \
    ConvCore<BM, BN, BK, WGM, WGN, 1, EPI, false, SPLIT, true>(smem, __VA_ARGS__);              \
  } else if (r == 1 && s == 1 && pad_h == 0 && pad_w == 0) {                                        \
    ConvCore<BM, BN, BK, WGM, WGN, 1, EPI, true, SPLIT>(smem, __VA_ARGS__);                     \
  } else {                                                                                          \
    ConvCore<BM, BN, BK, WGM, WGN, 1, EPI, false, SPLIT>(smem, __VA_ARGS__);                    \
  }

#define CT_DEFINE_SPLIT_VARIANTS(NAME, BM, BN, BK, WGM, WGN, SPLIT, MIN_GROUPS)                                 \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN, MIN_GROUPS) conv_bn_relu_fp32_##NAME(                                  \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void* scratch, void*) {         \
    CT_SPLIT_DISPATCH(BM, BN, BK, WGM, WGN, SPLIT, kBatchNormRelu, x, weight, scale, bias, mean,         \
                      variance, nullptr, output, CT_CONV_GEOMETRY, epsilon, scratch)                     \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN, MIN_GROUPS) conv_bn_fp32_##NAME(                                       \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, float* output, CT_CONV_DIMS, float epsilon, void* scratch, void*) {         \
    CT_SPLIT_DISPATCH(BM, BN, BK, WGM, WGN, SPLIT, kBatchNorm, x, weight, scale, bias, mean, variance,   \
                      nullptr, output, CT_CONV_GEOMETRY, epsilon, scratch)                               \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN, MIN_GROUPS) conv_bn_add_relu_fp32_##NAME(                              \
      const float* x, const float* weight, const float* scale, const float* bias, const float* mean,     \
      const float* variance, const float* residual, float* output, CT_CONV_DIMS, float epsilon,          \
      void* scratch, void*) {                                                                            \
    CT_SPLIT_DISPATCH(BM, BN, BK, WGM, WGN, SPLIT, kBatchNormAddRelu, x, weight, scale, bias, mean,      \
                      variance, residual, output, CT_CONV_GEOMETRY, epsilon, scratch)                    \
  }                                                                                                      \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN, MIN_GROUPS) conv_fp32_##NAME(const float* x, const float* weight,      \
                                                              float* output, CT_CONV_DIMS, void* scratch, \
                                                              void*) {                                   \
    CT_SPLIT_DISPATCH(BM, BN, BK, WGM, WGN, SPLIT, kPlain, x, weight, nullptr, nullptr, nullptr, nullptr, \
                      nullptr, output, CT_CONV_GEOMETRY, 0.0f, scratch)                                  \
  }

// name, BM, BN, BK, WGM, WGN, SPLIT, workgroups per CU the registers must allow
CT_DEFINE_SPLIT_VARIANTS(m128n128s2, 128, 128, 32, 2, 2, 2, 1)
CT_DEFINE_SPLIT_VARIANTS(m128n128s4, 128, 128, 32, 2, 2, 4, 1)
CT_DEFINE_SPLIT_VARIANTS(m128n128s8, 128, 128, 32, 2, 2, 8, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64s2, 64, 64, 32, 2, 2, 2, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64s4, 64, 64, 32, 2, 2, 4, 1)
// Split counts that are not powers of two fill the last round of
// workgroups better for some tile counts (e.g. 200 tiles x 5 = 1000).
CT_DEFINE_SPLIT_VARIANTS(m64n64s3, 64, 64, 32, 2, 2, 3, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64s5, 64, 64, 32, 2, 2, 5, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64s6, 64, 64, 32, 2, 2, 6, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64k64s2, 64, 64, 64, 2, 2, 2, 1)
CT_DEFINE_SPLIT_VARIANTS(m64n64k16s2, 64, 64, 16, 2, 2, 2, 5)
CT_DEFINE_SPLIT_VARIANTS(m64n64k16s3, 64, 64, 16, 2, 2, 3, 5)
CT_DEFINE_SPLIT_VARIANTS(m64n64k16s5, 64, 64, 16, 2, 2, 5, 5)
CT_DEFINE_SPLIT_VARIANTS(m64n64k16s8, 64, 64, 16, 2, 2, 8, 5)
CT_DEFINE_SPLIT_VARIANTS(m64n64k16s16, 64, 64, 16, 2, 2, 16, 5)

// C[m][n] = sum_k A[m][k] * B[k][n] (+ bias[n]) with A, B row-major: the
// core with rows = m, columns = n, depth = k (a 1x1 convolution of one
// 1 x n "image").
#define CT_DEFINE_GEMM_VARIANTS(NAME, BM, BN, BK, WGM, WGN, WGK)                                           \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK) gemm_fp32_##NAME(const float* a, const float* b, \
                                                              float* output, int m, int n, int k, void*, void*) {        \
    __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, WGK>::kFloats];      \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    if (k % BK == 0) {                                                                                    \
      ConvCore<BM, BN, BK, WGM, WGN, WGK, kPlain, false, 1, true>(smem, b, a, nullptr, nullptr, nullptr, \
                                                                     nullptr, nullptr, output, g, 0.0f);  \
    } else {                                                                                              \
      ConvCore<BM, BN, BK, WGM, WGN, WGK, kPlain, true>(smem, b, a, nullptr, nullptr, nullptr, nullptr,   \
                                                        nullptr, output, g, 0.0f);                        \
    }                                                                                                     \
  }                                                                                                       \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN * WGK) gemm_bias_fp32_##NAME(                         \
      const float* a, const float* b, const float* bias, float* output, int m, int n, int k, void*, void*) { \
    __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, WGK>::kFloats];      \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    if (k % BK == 0) {                                                                                    \
      ConvCore<BM, BN, BK, WGM, WGN, WGK, kColumnBias, false, 1, true>(smem, b, a, nullptr, bias,      \
                                                                          nullptr, nullptr, nullptr,      \
                                                                          output, g, 0.0f);               \
    } else {                                                                                              \
      ConvCore<BM, BN, BK, WGM, WGN, WGK, kColumnBias, true>(smem, b, a, nullptr, bias, nullptr, nullptr, \
                                                             nullptr, output, g, 0.0f);                   \
    }                                                                                                     \
  }

CT_DEFINE_GEMM_VARIANTS(m64n64, 64, 64, 32, 2, 2, 1)
CT_DEFINE_GEMM_VARIANTS(m128n128, 128, 128, 32, 2, 2, 1)

// Split-K Gemm entry points (grid z = SPLIT; the first reserved argument is
// the runtime scratch, as for the split-K convolutions): a short, wide
// product such as the classifier [N, 2048] x [2048, 1000] has few output
// tiles, so the depth is shared out to fill the chip.
#define CT_DEFINE_GEMM_SPLIT_VARIANTS(NAME, BM, BN, BK, WGM, WGN, SPLIT)                                  \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN) gemm_fp32_##NAME(const float* a, const float* b, float* output, \
                                                              int m, int n, int k, void* scratch, void*) { \
    __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, 1>::kFloats];        \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    if (k % BK == 0) {                                                                                    \
      ConvCore<BM, BN, BK, WGM, WGN, 1, kPlain, false, SPLIT, true>(smem, b, a, nullptr, nullptr, nullptr, \
                                                                       nullptr, nullptr, output, g, 0.0f, \
                                                                       scratch);                          \
    } else {                                                                                              \
      ConvCore<BM, BN, BK, WGM, WGN, 1, kPlain, true, SPLIT>(smem, b, a, nullptr, nullptr, nullptr,       \
                                                             nullptr, nullptr, output, g, 0.0f, scratch); \
    }                                                                                                     \
  }                                                                                                       \
  CT_KERNEL void __launch_bounds__(64 * WGM * WGN) gemm_bias_fp32_##NAME(                                      \
      const float* a, const float* b, const float* bias, float* output, int m, int n, int k, void* scratch, \
      void*) {                                                                                            \
    __shared__ __attribute__((aligned(16))) float smem[ConvLds<BM, BN, BK, WGM, WGN, 1>::kFloats];        \
    const ConvGeometry g = MakeGeometry(1, k, 1, n, m, 1, 1, 1, n, 1, 1, 0, 0, 1, 1);                    \
    if (k % BK == 0) {                                                                                    \
      ConvCore<BM, BN, BK, WGM, WGN, 1, kColumnBias, false, SPLIT, true>(smem, b, a, nullptr, bias,      \
                                                                            nullptr, nullptr, nullptr,    \
                                                                            output, g, 0.0f, scratch);    \
    } else {                                                                                              \
      ConvCore<BM, BN, BK, WGM, WGN, 1, kColumnBias, true, SPLIT>(smem, b, a, nullptr, bias, nullptr,    \
                                                                  nullptr, nullptr, output, g, 0.0f,      \
                                                                  scratch);                               \
    }                                                                                                     \
  }

CT_DEFINE_GEMM_SPLIT_VARIANTS(m64n64s8, 64, 64, 32, 2, 2, 8)
CT_DEFINE_GEMM_SPLIT_VARIANTS(m64n64s16, 64, 64, 32, 2, 2, 16)
