// Device identity. Mirrors include/cutriton/core/device.h:9-25 of the
// reference with a HIP device in place of the CUDA one.
#pragma once

#include <cstddef>
#include <string>

#include "cutriton/core/tensor.h"

namespace cutriton {

struct Device {
  DeviceType type{DeviceType::kCPU};
  int id{0};
  std::string name{"cpu"};

  static Device CPU() { return Device{}; }
  static Device HIP(int device_id = 0) {
    return Device{DeviceType::kHIP, device_id, "hip:" + std::to_string(device_id)};
  }
};

struct DeviceProperties {
  Device device;
  // Compute units (CUs) of the HIP device; the reference's field name.
  int sm_count{0};
  std::size_t l2_cache_bytes{0};
  std::size_t global_memory_bytes{0};
};

}  // namespace cutriton
