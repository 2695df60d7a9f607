// Status names, tensor descriptions and buffers.
// Behaviour follows reference src/core/status.cpp:5-32,
// src/core/tensor.cpp:7-102 and src/core/buffer.cpp:47-176; device memory
// goes through the C-ABI runtime layer (hipMalloc / hipMemcpy).
#include <cstring>
#include <limits>
#include <string>

#include "cutriton/core/buffer.h"
#include "cutriton/core/status.h"
#include "cutriton/core/tensor.h"
#include "cutriton_hip_runtime.h"

namespace cutriton {

const char* ErrorCodeName(ErrorCode code) {
  switch (code) {
    case ErrorCode::kOk: return "OK";
    case ErrorCode::kInvalidArgument: return "InvalidArgument";
    case ErrorCode::kNotFound: return "NotFound";
    case ErrorCode::kAlreadyExists: return "AlreadyExists";
    case ErrorCode::kUnsupported: return "Unsupported";
    case ErrorCode::kShapeError: return "ShapeError";
    case ErrorCode::kRuntimeError: return "RuntimeError";
    case ErrorCode::kInternal: return "Internal";
  }
  return "Unknown";
}

std::string Status::ToString() const {
  return ok() ? std::string("OK") : std::string(ErrorCodeName(code_)) + ": " + message_;
}

const char* DataTypeName(DataType dtype) {
  switch (dtype) {
    case DataType::kFloat32: return "float32";
    case DataType::kFloat16: return "float16";
    case DataType::kInt32: return "int32";
    case DataType::kInt64: return "int64";
    case DataType::kUnknown: break;
  }
  return "unknown";
}

const char* DeviceTypeName(DeviceType device_type) {
  return device_type == DeviceType::kHIP ? "hip" : "cpu";
}

std::size_t ElementSize(DataType dtype) {
  switch (dtype) {
    case DataType::kFloat32:
    case DataType::kInt32: return 4;
    case DataType::kFloat16: return 2;
    case DataType::kInt64: return 8;
    case DataType::kUnknown: break;
  }
  return 0;
}

bool TensorDesc::IsStatic() const {
  if (shape.empty() || dtype == DataType::kUnknown) return false;
  for (const int64_t dim : shape) {
    if (dim <= 0) return false;
  }
  return true;
}

int64_t TensorDesc::NumElements() const {
  if (shape.empty()) return 0;
  int64_t count = 1;
  for (const int64_t dim : shape) {
    if (dim <= 0 || count > std::numeric_limits<int64_t>::max() / dim) return 0;
    count *= dim;
  }
  return count;
}

std::size_t TensorDesc::ByteSize() const {
  const std::size_t element = ElementSize(dtype);
  const int64_t count = NumElements();
  return element == 0 || count <= 0 ? 0 : static_cast<std::size_t>(count) * element;
}

Status TensorDesc::Validate() const {
  if (dtype == DataType::kUnknown) return Status::ShapeError("tensor dtype is unknown");
  if (shape.empty()) return Status::ShapeError("tensor shape is empty");
  for (const int64_t dim : shape) {
    if (dim <= 0) return Status::ShapeError("static tensor shape has a non-positive dimension");
  }
  if (ByteSize() == 0) return Status::ShapeError("tensor byte size is zero");
  return Status::OK();
}

namespace {

Status RuntimeStatus(int code, const char* operation) {
  if (code == 0) return Status::OK();
  return Status::RuntimeError(std::string(operation) + ": " + cth_last_error());
}

}  // namespace

std::shared_ptr<Buffer> Buffer::AllocateHost(std::size_t size_bytes) {
  if (size_bytes == 0) return std::make_shared<Buffer>();
  auto* raw = new std::uint8_t[size_bytes]();
  std::shared_ptr<void> owner(raw, [](void* p) { delete[] static_cast<std::uint8_t*>(p); });
  return std::shared_ptr<Buffer>(new Buffer(raw, size_bytes, DeviceType::kCPU, 0, owner));
}

Status Buffer::AllocateHip(std::size_t size_bytes, int device_id,
                           std::shared_ptr<Buffer>* buffer) {
  if (buffer == nullptr) return Status::InvalidArgument("Buffer output pointer is null");
  if (size_bytes == 0) {
    *buffer = std::make_shared<Buffer>();
    return Status::OK();
  }
  void* raw = nullptr;
  CUTRITON_RETURN_IF_ERROR(RuntimeStatus(cth_malloc(&raw, size_bytes, device_id), "hipMalloc"));
  std::shared_ptr<void> owner(raw, [device_id](void* p) { cth_free(p, device_id); });
  *buffer = std::shared_ptr<Buffer>(new Buffer(raw, size_bytes, DeviceType::kHIP, device_id, owner));
  return Status::OK();
}

std::shared_ptr<Buffer> Buffer::WrapExternal(void* data, std::size_t size_bytes,
                                             DeviceType device_type, int device_id) {
  return std::shared_ptr<Buffer>(new Buffer(data, size_bytes, device_type, device_id, nullptr));
}

Status Buffer::CopyFromHost(const void* source, std::size_t size_bytes,
                            std::size_t destination_offset) {
  if (source == nullptr && size_bytes != 0) return Status::InvalidArgument("host source is null");
  if (destination_offset > size_bytes_ || size_bytes > size_bytes_ - destination_offset) {
    return Status::InvalidArgument("copy exceeds the destination Buffer");
  }
  if (size_bytes == 0) return Status::OK();
  auto* destination = static_cast<std::uint8_t*>(data_) + destination_offset;
  if (device_type_ == DeviceType::kCPU) {
    std::memcpy(destination, source, size_bytes);
    return Status::OK();
  }
  return RuntimeStatus(cth_memcpy_htod(destination, source, size_bytes, device_id_),
                       "hipMemcpy(HostToDevice)");
}

Status Buffer::CopyToHost(void* destination, std::size_t size_bytes,
                          std::size_t source_offset) const {
  if (destination == nullptr && size_bytes != 0) {
    return Status::InvalidArgument("host destination is null");
  }
  if (source_offset > size_bytes_ || size_bytes > size_bytes_ - source_offset) {
    return Status::InvalidArgument("copy exceeds the source Buffer");
  }
  if (size_bytes == 0) return Status::OK();
  const auto* source = static_cast<const std::uint8_t*>(data_) + source_offset;
  if (device_type_ == DeviceType::kCPU) {
    std::memcpy(destination, source, size_bytes);
    return Status::OK();
  }
  return RuntimeStatus(cth_memcpy_dtoh(destination, source, size_bytes, device_id_),
                       "hipMemcpy(DeviceToHost)");
}

}  // namespace cutriton
