/* Thin C-ABI runtime layer over HIP for the gfx950 backend.
 *
 * Every call that the reference makes into the CUDA Driver API on the hot
 * path goes through one of these functions instead:
 *   device query        <- cuDeviceGetAttribute / cuDeviceGetUuid / cuDriverGetVersion
 *                          (reference src/backend/backend.cpp:86-100,
 *                           src/runtime/engine.cpp:277-290)
 *   memory              <- cuMemAlloc / cuMemFree / cuMemcpyHtoD / cuMemcpyDtoH
 *                          (reference src/core/buffer.cpp:58-176)
 *   modules             <- cuModuleLoadDataEx / cuModuleGetFunction / cuModuleUnload
 *                          (reference src/backend/cuda_launcher.cpp:47-118)
 *   launch              <- cuLaunchKernel (reference src/backend/cuda_launcher.cpp:415-422)
 *   streams and events  <- cuStreamCreate / cuEventRecord / cuEventElapsedTime
 *                          (reference src/runtime/engine.cpp:151-176, 971-997, 1081-1113)
 *   graphs              <- cuStreamBeginCapture / cuStreamEndCapture /
 *                          cuGraphInstantiate / cuGraphLaunch / cuGraphExecDestroy
 *                          (reference src/runtime/engine.cpp:1029-1069)
 *
 * Conventions: every function returns 0 on success or a non-zero HIP error
 * code; cth_last_error() returns the message of the calling thread's most
 * recent failure. Handles are opaque pointers; sizes are in bytes. No
 * function allocates host memory that the caller must free.
 */
#ifndef CUTRITON_HIP_RUNTIME_H_
#define CUTRITON_HIP_RUNTIME_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* cth_module;
typedef void* cth_function;
typedef void* cth_stream;
typedef void* cth_event;
typedef void* cth_graph;      /* an instantiated, launchable graph */
typedef void* cth_graph_template;  /* a graph under construction (hipGraph_t) */
typedef void* cth_graph_node;      /* a node of a graph template (hipGraphNode_t) */

typedef struct cth_device_info {
  char arch_name[64];          /* e.g. "gfx950:sramecc+:xnack-" */
  int numeric_arch;            /* 950 for gfx950 */
  int compute_units;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width_bits;
  size_t global_memory_bytes;
  size_t l2_cache_bytes;
  size_t lds_per_workgroup_bytes;
  int driver_version;
  int runtime_version;
  unsigned char uuid[16];
} cth_device_info;

const char* cth_last_error(void);

int cth_device_count(int* count);
int cth_set_device(int device);
int cth_device_query(int device, cth_device_info* info);

int cth_malloc(void** pointer, size_t bytes, int device);
int cth_free(void* pointer, int device);
int cth_memcpy_htod(void* device_dst, const void* host_src, size_t bytes, int device);
int cth_memcpy_dtoh(void* host_dst, const void* device_src, size_t bytes, int device);
int cth_memcpy_dtod(void* device_dst, const void* device_src, size_t bytes, int device);
int cth_memset(void* device_dst, int value, size_t bytes, int device);
int cth_device_synchronize(int device);

int cth_module_load_data(cth_module* module, const void* image, size_t bytes, int device);
int cth_module_unload(cth_module module);
int cth_module_get_function(cth_function* function, cth_module module, const char* symbol);
/* grid and block hold three dimensions each; params points at one pointer
 * per kernel argument, in declaration order. */
int cth_launch(cth_function function, const unsigned int grid[3],
               const unsigned int block[3], unsigned int lds_bytes,
               cth_stream stream, void** params);

int cth_stream_create(cth_stream* stream, int device);
int cth_stream_destroy(cth_stream stream);
int cth_stream_synchronize(cth_stream stream);

int cth_event_create(cth_event* event);
int cth_event_destroy(cth_event event);
int cth_event_record(cth_event event, cth_stream stream);
int cth_event_synchronize(cth_event event);
int cth_event_elapsed_ms(float* milliseconds, cth_event start, cth_event end);

int cth_stream_begin_capture(cth_stream stream);
/* Ends the capture and instantiates it; on failure *graph stays NULL. */
int cth_stream_end_capture(cth_stream stream, cth_graph* graph);
/* Explicit graph construction, used to place hipEvent record nodes between
 * captured op groups (hipEventRecordWithFlags(..., hipEventRecordExternal)
 * is refused inside stream capture by the HIP runtime):
 *   end_capture_template  <- hipStreamEndCapture (no instantiation)
 *   graph_template_create <- hipGraphCreate
 *   graph_add_child       <- hipGraphAddChildGraphNode (dependency may be NULL)
 *   graph_add_event_record<- hipGraphAddEventRecordNode
 *   graph_instantiate     <- hipGraphInstantiate
 * A child graph is copied into its parent; destroy templates after use. */
int cth_stream_end_capture_template(cth_stream stream, cth_graph_template* graph);
int cth_graph_template_create(cth_graph_template* graph);
int cth_graph_template_destroy(cth_graph_template graph);
int cth_graph_add_child(cth_graph_template parent, cth_graph_node dependency, cth_graph_template child,
                        cth_graph_node* node);
int cth_graph_add_event_record(cth_graph_template parent, cth_graph_node dependency, cth_event event,
                               cth_graph_node* node);
int cth_graph_instantiate(cth_graph_template graph, cth_graph* exec);
int cth_graph_launch(cth_graph graph, cth_stream stream);
int cth_graph_destroy(cth_graph graph);

#ifdef __cplusplus
}
#endif

#endif /* CUTRITON_HIP_RUNTIME_H_ */
