// Loads the embedded re-layout code object (relayout.hip) once per device
// and launches its kernels.
#include "runtime/relayout.h"

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <unordered_map>

#include "cutriton_hip_runtime.h"

namespace cutriton {

// The gfx950 code object of relayout.hip, embedded at build time.
extern const unsigned char kRelayoutCodeObject[];
extern const std::size_t kRelayoutCodeObjectBytes;

namespace {

constexpr unsigned int kThreads = 256;     // relayout.hip's block size
constexpr int64_t kMaxBlocks = 8192;       // grid-stride beyond this

struct RelayoutKernels {
  cth_module module{nullptr};
  cth_function ohwi_b32{nullptr};
  cth_function nk[4]{};  // 1, 2, 4, 8-byte elements
};

Status Fail(const char* operation) { return Status::RuntimeError(std::string(operation) + ": " + cth_last_error()); }

// One module per device, kept until the process ends (unloading during
// runtime teardown is not safe).
Status Kernels(int device, const RelayoutKernels** out) {
  static std::mutex mutex;
  static std::unordered_map<int, RelayoutKernels> loaded;
  std::lock_guard<std::mutex> lock(mutex);
  auto it = loaded.find(device);
  if (it == loaded.end()) {
    RelayoutKernels k;
    if (cth_module_load_data(&k.module, kRelayoutCodeObject, kRelayoutCodeObjectBytes, device) != 0) {
      return Fail("loading the re-layout kernels");
    }
    const char* nk_names[4] = {"relayout_kn_to_nk_b8", "relayout_kn_to_nk_b16", "relayout_kn_to_nk_b32",
                               "relayout_kn_to_nk_b64"};
    if (cth_module_get_function(&k.ohwi_b32, k.module, "relayout_oihw_to_ohwi_b32") != 0) {
      return Fail("relayout_oihw_to_ohwi_b32");
    }
    for (int i = 0; i < 4; ++i) {
      if (cth_module_get_function(&k.nk[i], k.module, nk_names[i]) != 0) return Fail(nk_names[i]);
    }
    it = loaded.emplace(device, k).first;
  }
  *out = &it->second;
  return Status::OK();
}

Status Launch(cth_function function, int64_t elements, void** params) {
  if (elements == 0) return Status::OK();
  const int64_t blocks = std::min<int64_t>((elements + kThreads - 1) / kThreads, kMaxBlocks);
  const unsigned int grid[3] = {static_cast<unsigned int>(blocks), 1, 1};
  const unsigned int block[3] = {kThreads, 1, 1};
  if (cth_launch(function, grid, block, 0, nullptr, params) != 0) return Fail("re-layout launch");
  return Status::OK();
}

}  // namespace

Status RelayoutOnDevice(const std::string& layout, const TensorDesc& desc, const void* source, void* destination,
                        int device) {
  const RelayoutKernels* kernels = nullptr;
  CUTRITON_RETURN_IF_ERROR(Kernels(device, &kernels));
  for (const int64_t d : desc.shape) {
    if (d < 0) return Status::InvalidArgument("re-layout of a tensor with an unresolved dimension");
  }
  const void* in = source;
  void* out = destination;
  if (layout == "OHWI") {
    if (desc.shape.size() != 4 || ElementSize(desc.dtype) != 4) {
      return Status::InvalidArgument("OHWI needs a rank-4 tensor of 4-byte elements");
    }
    int64_t k = desc.shape[0], c = desc.shape[1], rs = desc.shape[2] * desc.shape[3];
    void* params[] = {&in, &out, &k, &c, &rs};
    return Launch(kernels->ohwi_b32, k * c * rs, params);
  }
  if (layout == "NK" || layout == "T") {
    if (desc.shape.size() != 2) return Status::InvalidArgument("NK needs a rank-2 tensor");
    int index = -1;
    switch (ElementSize(desc.dtype)) {
      case 1: index = 0; break;
      case 2: index = 1; break;
      case 4: index = 2; break;
      case 8: index = 3; break;
      default: return Status::InvalidArgument("NK needs 1, 2, 4 or 8-byte elements");
    }
    int64_t k = desc.shape[0], n = desc.shape[1];
    void* params[] = {&in, &out, &k, &n};
    return Launch(kernels->nk[index], k * n, params);
  }
  return Status::InvalidArgument("unknown constant layout " + layout);
}

}  // namespace cutriton
