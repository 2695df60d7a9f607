// The library's static device scratch (static_scratch.hip).
#pragma once

#include <cstddef>

namespace cutriton {

// 64 KiB of tile counters then 128 MiB of partial sums: the runtime scratch
// the split-K kernels declare (runtime_scratch_bytes of their pack entries).
constexpr std::size_t kStaticScratchCounterBytes = std::size_t{64} << 10;
constexpr std::size_t kStaticScratchBytes = kStaticScratchCounterBytes + (std::size_t{128} << 20);

// The device address of the array on `device`, found once per device (with
// that device current) and kept. 0 or a HIP error code.
int StaticScratchAddress(int device, void** address);
// Enqueues a kernel on `stream` that zeroes the counter region at `address`
// (no hipMemsetAsync, so the call may sit inside a caller's stream capture).
int ClearStaticScratchCounters(void* address, void* stream);
// Message of the calling thread's last failure of the two above.
const char* StaticScratchError();

}  // namespace cutriton
