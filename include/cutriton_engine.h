/* C-ABI facade over the C++ engine API (Model/Graph IR, BuildEngine,
 * ExecutionContext), for FFI callers that cannot use C++ directly.
 *
 * Each entry point forwards to the C++ call named beside it; the reference
 * exposes only those C++ calls:
 *   ct_model_*            <- cutriton::Model / Graph / Node
 *                            (reference include/cutriton/ir/graph.h:22-161)
 *   ct_build_engine       <- cutriton::BuildEngine
 *                            (reference include/cutriton/compiler/compiler.h:44-46)
 *   ct_engine_*           <- cutriton::Engine / ExecutablePlan
 *                            (reference include/cutriton/runtime/engine.h:20-31,
 *                             include/cutriton/runtime/executable_plan.h:16-93)
 *   ct_context_*          <- cutriton::ExecutionContext
 *                            (reference include/cutriton/runtime/engine.h:34-93)
 *
 * Return values are cutriton::ErrorCode values (0 = OK); ct_last_error()
 * holds the calling thread's last Status::ToString(). Strings are UTF-8 and
 * NUL-terminated. Device pointers are HIP device addresses (see
 * cutriton_hip_runtime.h). Dtype codes: 1 float32, 2 float16, 3 int32,
 * 4 int64. Device codes: 0 host, 1 HIP device.
 */
#ifndef CUTRITON_ENGINE_H_
#define CUTRITON_ENGINE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ct_model ct_model;
typedef struct ct_options ct_options;
typedef struct ct_engine ct_engine;
typedef struct ct_context ct_context;

const char* ct_last_error(void);
const char* ct_version(void);

/* ---- model construction ---- */
ct_model* ct_model_create(void);
void ct_model_destroy(ct_model* model);
int ct_model_add_input(ct_model* model, const char* name, const int64_t* shape,
                       int rank, int dtype, const char* layout);
int ct_model_add_output(ct_model* model, const char* name);
/* Copies `bytes` of host data into a host constant. */
int ct_model_add_constant(ct_model* model, const char* name, const int64_t* shape,
                          int rank, int dtype, const char* layout,
                          const void* host_data, size_t bytes);
int ct_model_add_node(ct_model* model, const char* name, const char* op_type,
                      const char* const* inputs, int input_count,
                      const char* const* outputs, int output_count);
int ct_model_set_attr_int(ct_model* model, const char* node, const char* key, int64_t value);
int ct_model_set_attr_ints(ct_model* model, const char* node, const char* key,
                           const int64_t* values, int count);
int ct_model_set_attr_float(ct_model* model, const char* node, const char* key, double value);
int ct_model_set_attr_floats(ct_model* model, const char* node, const char* key,
                             const double* values, int count);
int ct_model_set_attr_bool(ct_model* model, const char* node, const char* key, int value);
int ct_model_set_attr_string(ct_model* model, const char* node, const char* key,
                             const char* value);
/* Runs the default pass pipeline in place (fusion tests, inspection). */
int ct_model_run_default_passes(ct_model* model, int transformer_fusions,
                                int residual_epilogue_fusion);
/* Reads an ONNX model into a new model (*model; free with
 * ct_model_destroy). Symbolic input dimensions take the `dim_count` sizes
 * named by `dim_names`. No counterpart in the reference, which has no
 * importer (python/cutriton/api.py:77-99 only lists a model's structure
 * through the onnx package); for callers that hold .onnx files. */
int ct_model_import_onnx(const char* path, const char* const* dim_names, const int64_t* dim_values,
                         int dim_count, ct_model** model);
/* As ct_model_import_onnx, from `bytes` of a serialized ModelProto. */
int ct_model_import_onnx_buffer(const void* data, size_t bytes, const char* const* dim_names,
                                const int64_t* dim_values, int dim_count, ct_model** model);
int ct_model_node_count(const ct_model* model);
/* Copies node `index`'s op_type into `buffer` (truncated to `length`). */
int ct_model_node_op_type(const ct_model* model, int index, char* buffer, size_t length);

/* ---- compile options ---- */
ct_options* ct_options_create(void);
void ct_options_destroy(ct_options* options);
/* Keys: "target", "kernel_artifact_dir", "kernel_artifact_path" (appends),
 * "tuning_cache_dir". */
int ct_options_set_string(ct_options* options, const char* key, const char* value);
/* Keys: "enable_cuda_graph", "enable_profiling", "enable_transformer_fusions",
 * "enable_residual_epilogue_fusion", "device_id", "tuning_mode"
 * (0 disabled, 1 use-cache, 2 tune-on-miss, 3 force-retune),
 * "cuda_graph_cache_capacity", "tuning_warmup_iterations",
 * "tuning_measurement_iterations", "allow_cpu_fallback". */
int ct_options_set_int(ct_options* options, const char* key, int64_t value);
/* Adds (or extends) shape profile `profile` with a range for `input`. */
int ct_options_add_profile_range(ct_options* options, const char* profile,
                                 const char* input, const int64_t* min_shape,
                                 const int64_t* opt_shape, const int64_t* max_shape,
                                 int rank);

/* ---- engine ---- */
int ct_build_engine(const ct_model* model, const ct_options* options, ct_engine** engine);
void ct_engine_destroy(ct_engine* engine);
int ct_engine_op_count(const ct_engine* engine);
int ct_engine_op_info(const ct_engine* engine, int index, char* op_type, size_t op_type_length,
                      char* node_name, size_t node_name_length, int* candidate_count,
                      int* selected_candidate);
int ct_engine_candidate_id(const ct_engine* engine, int op_index, int candidate_index,
                           char* buffer, size_t length);
/* Shape/dtype of a value in the compiled graph; *rank is in/out (capacity). */
int ct_engine_value_desc(const ct_engine* engine, const char* name, int64_t* shape,
                         int* rank, int* dtype);
/* Layout of a value in the compiled graph ("NCHW", "" ...), copied into
 * `buffer` (truncated to `length`): the layout a binding of it must carry. */
int ct_engine_value_layout(const ct_engine* engine, const char* name, char* buffer, size_t length);
size_t ct_engine_workspace_bytes(const ct_engine* engine);
int ct_engine_create_context(const ct_engine* engine, ct_context** context);

/* ---- execution context ---- */
void ct_context_destroy(ct_context* context);
/* Binds `buffer_bytes` of memory at `data` (device code `device`) viewed at
 * `byte_offset` as a tensor of the given shape and dtype. */
int ct_context_bind_input(ct_context* context, const char* name, void* data,
                          size_t buffer_bytes, size_t byte_offset, const int64_t* shape,
                          int rank, int dtype, const char* layout, int device);
int ct_context_bind_output(ct_context* context, const char* name, void* data,
                           size_t buffer_bytes, size_t byte_offset, const int64_t* shape,
                           int rank, int dtype, const char* layout, int device);
int ct_context_select_profile(ct_context* context, const char* name);
int ct_context_set_input_shape(ct_context* context, const char* name, const int64_t* shape,
                               int rank);
int ct_context_resolve_shapes(ct_context* context);
int ct_context_resolved_desc(const ct_context* context, const char* name, int64_t* shape,
                             int* rank, int* dtype, char* layout, size_t layout_length);
int ct_context_run(ct_context* context);
int ct_context_run_async(ct_context* context, void* stream);
/* Allocation-free variant of ct_context_run_async, for callers that cannot
 * allocate device memory: code under stream capture, serving loops that
 * forbid hipMalloc. No counterpart in the reference. It enqueues the op
 * sequence on `stream` (required) with no graph capture and no per-op events,
 * binding the kernels' runtime scratch (split-K partial sums and tile
 * counters) to the library's static device array of 64 KiB + 128 MiB, held by
 * every GPU the library runs on until the process ends; it calls no
 * hipMalloc/hipFree, loads no code object and times no candidate. The context
 * must already hold its constants, a workspace for its profile and the code
 * objects of its kernels (one ct_context_run_async of the context at any shape
 * of its profile provides them), and its tuning choices must resolve without
 * timing; otherwise it returns an error and enqueues nothing. Calls that
 * overlap on one GPU share the array and race. Complete with
 * ct_context_synchronize. Forwards to ExecutionContext::RunAsyncWithoutAllocation. */
int ct_context_run_async_no_alloc(ct_context* context, void* stream);
int ct_context_synchronize(ct_context* context);
int ct_context_profile_event_count(const ct_context* context);
int ct_context_profile_event(const ct_context* context, int index, char* name,
                             size_t name_length, double* duration_ms);
size_t ct_context_graph_count(const ct_context* context);
size_t ct_context_module_count(const ct_context* context);
int ct_context_selected_candidate(const ct_context* context, int op_index);
/* Kernel time per launch of plan op `op_index` (ExecutionContext::TimeOp):
 * `iterations` back-to-back launches between one event pair on `stream`. */
int ct_context_time_op(ct_context* context, int op_index, int iterations, void* stream,
                       double* ms_per_launch);

#ifdef __cplusplus
}
#endif

#endif /* CUTRITON_ENGINE_H_ */
