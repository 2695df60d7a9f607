// The library's static device scratch: the runtime scratch of the
// allocation-free run (ExecutionContext::RunAsyncWithoutAllocation,
// ct_context_run_async_no_alloc), for callers that cannot allocate device
// memory (code under stream capture, serving loops that forbid hipMalloc).
//
// `scratch` is a file-scope device array, so every GPU the library runs on
// holds its own copy for the life of the process. In host code the array's
// name is not a device address: its address on a device comes from
// hipGetSymbolAddress with that device current, taken once per device and
// kept; only that address is ever passed to kernels or copies.
//
// Layout (what the split-K kernels expect of a runtime scratch): 64 KiB of
// tile counters, which must be zero when a run starts, then 128 MiB of
// partial sums. Calls that overlap on one GPU share the array and race.
#include <hip/hip_runtime.h>

#include <array>
#include <cstddef>
#include <mutex>
#include <string>

#include "runtime/static_scratch.h"

namespace cutriton {
namespace {

static_assert(kStaticScratchBytes % 256 == 0, "whole 256-byte blocks");
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;

// Zeroes `words` 32-bit words from `base`.
__global__ void __launch_bounds__(256) ClearWords(unsigned* base, unsigned words) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i < words) base[i] = 0u;
}

struct Addresses {
  std::mutex mutex;
  std::array<void*, kMaxDevices> device{};
};

Addresses& Known() {
  static Addresses known;
  return known;
}

thread_local std::string g_error;

int Fail(hipError_t code, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorString(code);
  return static_cast<int>(code);
}

}  // namespace

int StaticScratchAddress(int device, void** address) {
  if (address == nullptr || device < 0 || device >= kMaxDevices) {
    g_error = "static scratch: no such device slot";
    return static_cast<int>(hipErrorInvalidValue);
  }
  Addresses& known = Known();
  std::lock_guard<std::mutex> lock(known.mutex);
  void*& slot = known.device[static_cast<std::size_t>(device)];
  if (slot == nullptr) {
    int current = 0;
    hipError_t code = hipGetDevice(&current);
    if (code != hipSuccess) return Fail(code, "hipGetDevice");
    if (current != device && (code = hipSetDevice(device)) != hipSuccess) return Fail(code, "hipSetDevice");
    void* found = nullptr;
    code = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
    const hipError_t restored = current != device ? hipSetDevice(current) : hipSuccess;
    if (code != hipSuccess) return Fail(code, "hipGetSymbolAddress(scratch)");
    if (restored != hipSuccess) return Fail(restored, "hipSetDevice");
    if (found == nullptr) {
      g_error = "hipGetSymbolAddress(scratch) returned null";
      return static_cast<int>(hipErrorInvalidSymbol);
    }
    slot = found;
  }
  *address = slot;
  return 0;
}

int ClearStaticScratchCounters(void* address, void* stream) {
  constexpr unsigned kWords = static_cast<unsigned>(kStaticScratchCounterBytes / 4);
  ClearWords<<<dim3((kWords + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<unsigned*>(address), kWords);
  const hipError_t code = hipGetLastError();
  return code == hipSuccess ? 0 : Fail(code, "clearing the static scratch counters");
}

const char* StaticScratchError() { return g_error.c_str(); }

}  // namespace cutriton
