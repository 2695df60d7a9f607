// Engine-internal kernels that make the laid-out copies of constants on the
// device, once per engine, from the original already uploaded to HBM. The
// library embeds this code object; it is not part of any Kernel Pack.
//
// Both are permutations: every output element is one input element, moved
// as raw bits, so the copies are exact for every element type. One thread
// per output element keeps the stores coalesced; the loads are strided,
// which costs little for a one-time copy of at most a few hundred MB.
// Grid-stride loops with 64-bit indices: any element count fits any grid.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;

// OIHW [k][c][rs] -> OHWI [k][rs][c].
template <typename T>
__device__ void OihwToOhwi(const T* __restrict__ in, T* __restrict__ out, int64_t k, int64_t c, int64_t rs) {
  const int64_t total = k * c * rs;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total; i += step) {
    const int64_t channel = i % c;
    const int64_t rest = i / c;
    const int64_t tap = rest % rs;
    const int64_t filter = rest / rs;
    out[i] = in[(filter * c + channel) * rs + tap];
  }
}

// [k][n] -> [n][k].
template <typename T>
__device__ void KnToNk(const T* __restrict__ in, T* __restrict__ out, int64_t k, int64_t n) {
  const int64_t total = k * n;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total; i += step) {
    const int64_t row = i % k;
    const int64_t col = i / k;
    out[i] = in[row * n + col];
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(kThreads)
    relayout_oihw_to_ohwi_b32(const uint32_t* in, uint32_t* out, int64_t k, int64_t c, int64_t rs) {
  OihwToOhwi(in, out, k, c, rs);
}

extern "C" __global__ void __launch_bounds__(kThreads)
    relayout_kn_to_nk_b8(const uint8_t* in, uint8_t* out, int64_t k, int64_t n) {
  KnToNk(in, out, k, n);
}

extern "C" __global__ void __launch_bounds__(kThreads)
    relayout_kn_to_nk_b16(const uint16_t* in, uint16_t* out, int64_t k, int64_t n) {
  KnToNk(in, out, k, n);
}

extern "C" __global__ void __launch_bounds__(kThreads)
    relayout_kn_to_nk_b32(const uint32_t* in, uint32_t* out, int64_t k, int64_t n) {
  KnToNk(in, out, k, n);
}

extern "C" __global__ void __launch_bounds__(kThreads)
    relayout_kn_to_nk_b64(const uint64_t* in, uint64_t* out, int64_t k, int64_t n) {
  KnToNk(in, out, k, n);
}
