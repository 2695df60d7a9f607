// Device-side re-layout of constants: the copies that kernels with an input
// "layout" read ("OHWI", "NK"), made on the GPU from the uploaded original.
#pragma once

#include <string>

#include "cutriton/core/status.h"
#include "cutriton/core/tensor.h"

namespace cutriton {

// Enqueues, on `device`'s null stream, the copy of the device tensor at
// `source` (logical shape `desc`, stored in its logical order) in `layout`
// to `destination` (desc.ByteSize() bytes). The caller synchronizes the
// device before reading `destination`.
//   "OHWI": rank-4 4-byte elements, [K][C][R][S] -> [K][R][S][C];
//   "NK", "T": rank-2 1/2/4/8-byte elements, [R][C] -> [C][R].
Status RelayoutOnDevice(const std::string& layout, const TensorDesc& desc, const void* source, void* destination,
                        int device);

}  // namespace cutriton
