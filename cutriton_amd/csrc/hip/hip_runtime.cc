// Implementation of the thin C-ABI runtime layer (cutriton_hip_runtime.h)
// directly over the HIP runtime API.
#include "cutriton_hip_runtime.h"

#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <string>

namespace {

thread_local std::string g_last_error;

int Fail(hipError_t error, const char* operation) {
  if (error == hipSuccess) return 0;
  g_last_error = std::string(operation) + " failed: " + hipGetErrorName(error) +
                 " (" + hipGetErrorString(error) + ")";
  return static_cast<int>(error);
}

int FailMessage(const char* message) {
  g_last_error = message;
  return static_cast<int>(hipErrorInvalidValue);
}

#define CTH_CALL(expr)                                   \
  do {                                                   \
    hipError_t _cth_error = (expr);                      \
    if (_cth_error != hipSuccess) return Fail(_cth_error, #expr); \
  } while (false)

int ParseNumericArch(const char* name) {
  // "gfx950:sramecc+:xnack-" -> 950; hexadecimal stepping digits (gfx90a)
  // map to their hexadecimal value so ordering stays monotone.
  if (std::strncmp(name, "gfx", 3) != 0) return 0;
  int value = 0;
  for (const char* p = name + 3; *p != '\0' && *p != ':'; ++p) {
    int digit;
    if (*p >= '0' && *p <= '9') digit = *p - '0';
    else if (*p >= 'a' && *p <= 'f') digit = 10 + (*p - 'a');
    else break;
    value = value * (digit >= 10 ? 16 : 10) + digit;
  }
  return value;
}

}  // namespace

extern "C" {

const char* cth_last_error(void) { return g_last_error.c_str(); }

int cth_device_count(int* count) {
  if (count == nullptr) return FailMessage("cth_device_count: count is null");
  CTH_CALL(hipGetDeviceCount(count));
  return 0;
}

int cth_set_device(int device) {
  CTH_CALL(hipSetDevice(device));
  return 0;
}

int cth_device_query(int device, cth_device_info* info) {
  if (info == nullptr) return FailMessage("cth_device_query: info is null");
  hipDeviceProp_t props;
  CTH_CALL(hipGetDeviceProperties(&props, device));
  std::memset(info, 0, sizeof(*info));
  std::snprintf(info->arch_name, sizeof(info->arch_name), "%.63s", props.gcnArchName);
  info->numeric_arch = ParseNumericArch(props.gcnArchName);
  info->compute_units = props.multiProcessorCount;
  info->clock_khz = props.clockRate;
  info->memory_clock_khz = props.memoryClockRate;
  info->memory_bus_width_bits = props.memoryBusWidth;
  info->global_memory_bytes = props.totalGlobalMem;
  info->l2_cache_bytes = static_cast<size_t>(props.l2CacheSize);
  info->lds_per_workgroup_bytes = props.sharedMemPerBlock;
  CTH_CALL(hipDriverGetVersion(&info->driver_version));
  CTH_CALL(hipRuntimeGetVersion(&info->runtime_version));
  hipDevice_t handle;
  CTH_CALL(hipDeviceGet(&handle, device));
  hipUUID uuid;
  CTH_CALL(hipDeviceGetUuid(&uuid, handle));
  std::memcpy(info->uuid, uuid.bytes, sizeof(info->uuid));
  return 0;
}

int cth_malloc(void** pointer, size_t bytes, int device) {
  if (pointer == nullptr) return FailMessage("cth_malloc: pointer is null");
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipMalloc(pointer, bytes));
  return 0;
}

int cth_free(void* pointer, int device) {
  if (pointer == nullptr) return 0;
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipFree(pointer));
  return 0;
}

int cth_memcpy_htod(void* dst, const void* src, size_t bytes, int device) {
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return 0;
}

int cth_memcpy_dtoh(void* dst, const void* src, size_t bytes, int device) {
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return 0;
}

int cth_memcpy_dtod(void* dst, const void* src, size_t bytes, int device) {
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return 0;
}

int cth_memset(void* dst, int value, size_t bytes, int device) {
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipMemset(dst, value, bytes));
  return 0;
}

int cth_device_synchronize(int device) {
  CTH_CALL(hipSetDevice(device));
  CTH_CALL(hipDeviceSynchronize());
  return 0;
}

int cth_module_load_data(cth_module* module, const void* image, size_t bytes, int device) {
  if (module == nullptr || image == nullptr || bytes == 0) {
    return FailMessage("cth_module_load_data: invalid code object");
  }
  CTH_CALL(hipSetDevice(device));
  hipModule_t loaded = nullptr;
  CTH_CALL(hipModuleLoadData(&loaded, image));
  *module = loaded;
  return 0;
}

int cth_module_unload(cth_module module) {
  if (module == nullptr) return 0;
  CTH_CALL(hipModuleUnload(static_cast<hipModule_t>(module)));
  return 0;
}

int cth_module_get_function(cth_function* function, cth_module module, const char* symbol) {
  if (function == nullptr || module == nullptr || symbol == nullptr) {
    return FailMessage("cth_module_get_function: invalid argument");
  }
  hipFunction_t loaded = nullptr;
  CTH_CALL(hipModuleGetFunction(&loaded, static_cast<hipModule_t>(module), symbol));
  *function = loaded;
  return 0;
}

int cth_launch(cth_function function, const unsigned int grid[3], const unsigned int block[3],
               unsigned int lds_bytes, cth_stream stream, void** params) {
  if (function == nullptr || grid == nullptr || block == nullptr) {
    return FailMessage("cth_launch: invalid argument");
  }
  CTH_CALL(hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid[0], grid[1], grid[2],
                                 block[0], block[1], block[2], lds_bytes,
                                 static_cast<hipStream_t>(stream), params, nullptr));
  return 0;
}

int cth_stream_create(cth_stream* stream, int device) {
  if (stream == nullptr) return FailMessage("cth_stream_create: stream is null");
  CTH_CALL(hipSetDevice(device));
  hipStream_t created = nullptr;
  // Default priority: streams of different priorities are never mixed here.
  CTH_CALL(hipStreamCreateWithFlags(&created, hipStreamNonBlocking));
  *stream = created;
  return 0;
}

int cth_stream_destroy(cth_stream stream) {
  if (stream == nullptr) return 0;
  CTH_CALL(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return 0;
}

int cth_stream_synchronize(cth_stream stream) {
  CTH_CALL(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return 0;
}

int cth_event_create(cth_event* event) {
  if (event == nullptr) return FailMessage("cth_event_create: event is null");
  hipEvent_t created = nullptr;
  CTH_CALL(hipEventCreate(&created));
  *event = created;
  return 0;
}

int cth_event_destroy(cth_event event) {
  if (event == nullptr) return 0;
  CTH_CALL(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return 0;
}

int cth_event_record(cth_event event, cth_stream stream) {
  CTH_CALL(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
  return 0;
}

int cth_event_synchronize(cth_event event) {
  CTH_CALL(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return 0;
}

int cth_event_elapsed_ms(float* milliseconds, cth_event start, cth_event end) {
  if (milliseconds == nullptr) return FailMessage("cth_event_elapsed_ms: output is null");
  CTH_CALL(hipEventElapsedTime(milliseconds, static_cast<hipEvent_t>(start),
                               static_cast<hipEvent_t>(end)));
  return 0;
}

int cth_stream_begin_capture(cth_stream stream) {
  CTH_CALL(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeGlobal));
  return 0;
}

int cth_stream_end_capture(cth_stream stream, cth_graph* graph) {
  if (graph == nullptr) return FailMessage("cth_stream_end_capture: graph is null");
  *graph = nullptr;
  hipGraph_t captured = nullptr;
  CTH_CALL(hipStreamEndCapture(static_cast<hipStream_t>(stream), &captured));
  hipGraphExec_t exec = nullptr;
  hipError_t error = hipGraphInstantiate(&exec, captured, nullptr, nullptr, 0);
  // The executable graph holds everything it needs; the template is freed.
  (void)hipGraphDestroy(captured);
  if (error != hipSuccess) return Fail(error, "hipGraphInstantiate");
  *graph = exec;
  return 0;
}

int cth_stream_end_capture_template(cth_stream stream, cth_graph_template* graph) {
  if (graph == nullptr) return FailMessage("cth_stream_end_capture_template: graph is null");
  *graph = nullptr;
  hipGraph_t captured = nullptr;
  CTH_CALL(hipStreamEndCapture(static_cast<hipStream_t>(stream), &captured));
  *graph = captured;
  return 0;
}

int cth_graph_template_create(cth_graph_template* graph) {
  if (graph == nullptr) return FailMessage("cth_graph_template_create: graph is null");
  hipGraph_t created = nullptr;
  CTH_CALL(hipGraphCreate(&created, 0));
  *graph = created;
  return 0;
}

int cth_graph_template_destroy(cth_graph_template graph) {
  if (graph == nullptr) return 0;
  CTH_CALL(hipGraphDestroy(static_cast<hipGraph_t>(graph)));
  return 0;
}

int cth_graph_add_child(cth_graph_template parent, cth_graph_node dependency, cth_graph_template child,
                        cth_graph_node* node) {
  if (node == nullptr) return FailMessage("cth_graph_add_child: node is null");
  hipGraphNode_t created = nullptr;
  hipGraphNode_t dep = static_cast<hipGraphNode_t>(dependency);
  CTH_CALL(hipGraphAddChildGraphNode(&created, static_cast<hipGraph_t>(parent), dep ? &dep : nullptr,
                                     dep ? 1 : 0, static_cast<hipGraph_t>(child)));
  *node = created;
  return 0;
}

int cth_graph_add_event_record(cth_graph_template parent, cth_graph_node dependency, cth_event event,
                               cth_graph_node* node) {
  if (node == nullptr) return FailMessage("cth_graph_add_event_record: node is null");
  hipGraphNode_t created = nullptr;
  hipGraphNode_t dep = static_cast<hipGraphNode_t>(dependency);
  CTH_CALL(hipGraphAddEventRecordNode(&created, static_cast<hipGraph_t>(parent), dep ? &dep : nullptr,
                                      dep ? 1 : 0, static_cast<hipEvent_t>(event)));
  *node = created;
  return 0;
}

int cth_graph_instantiate(cth_graph_template graph, cth_graph* exec) {
  if (exec == nullptr) return FailMessage("cth_graph_instantiate: exec is null");
  *exec = nullptr;
  hipGraphExec_t created = nullptr;
  CTH_CALL(hipGraphInstantiate(&created, static_cast<hipGraph_t>(graph), nullptr, nullptr, 0));
  *exec = created;
  return 0;
}

int cth_graph_launch(cth_graph graph, cth_stream stream) {
  CTH_CALL(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), static_cast<hipStream_t>(stream)));
  return 0;
}

int cth_graph_destroy(cth_graph graph) {
  if (graph == nullptr) return 0;
  CTH_CALL(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
  return 0;
}

}  // extern "C"
