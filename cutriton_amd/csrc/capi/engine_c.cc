// C-ABI facade (cutriton_engine.h) over the C++ engine API.
#include "cutriton_engine.h"

#include <cstring>
#include <memory>
#include <string>

#include "cutriton/cutriton.h"

namespace {

using namespace cutriton;

thread_local std::string g_last_error;

int Report(const Status& status) {
  if (status.ok()) return 0;
  g_last_error = status.ToString();
  return static_cast<int>(status.code());
}

int Invalid(const char* message) { return Report(Status::InvalidArgument(message)); }

DataType DtypeFromCode(int code) {
  switch (code) {
    case 1: return DataType::kFloat32;
    case 2: return DataType::kFloat16;
    case 3: return DataType::kInt32;
    case 4: return DataType::kInt64;
    default: return DataType::kUnknown;
  }
}

int CodeFromDtype(DataType dtype) {
  switch (dtype) {
    case DataType::kFloat32: return 1;
    case DataType::kFloat16: return 2;
    case DataType::kInt32: return 3;
    case DataType::kInt64: return 4;
    case DataType::kUnknown: break;
  }
  return 0;
}

std::vector<int64_t> Shape(const int64_t* dims, int rank) {
  return dims == nullptr || rank <= 0 ? std::vector<int64_t>{} : std::vector<int64_t>(dims, dims + rank);
}

void CopyString(const std::string& text, char* buffer, std::size_t length) {
  if (buffer == nullptr || length == 0) return;
  const std::size_t n = std::min(text.size(), length - 1);
  std::memcpy(buffer, text.data(), n);
  buffer[n] = '\0';
}

int FillDesc(const TensorDesc& desc, int64_t* shape, int* rank, int* dtype) {
  if (rank == nullptr) return Invalid("rank pointer is null");
  const int capacity = *rank;
  *rank = static_cast<int>(desc.shape.size());
  if (shape != nullptr) {
    for (int i = 0; i < *rank && i < capacity; ++i) shape[i] = desc.shape[static_cast<std::size_t>(i)];
  }
  if (dtype != nullptr) *dtype = CodeFromDtype(desc.dtype);
  return capacity < *rank ? Invalid("shape capacity is too small") : 0;
}

}  // namespace

struct ct_model {
  Model model;
};
struct ct_options {
  CompileOptions options;
};
struct ct_engine {
  std::unique_ptr<Engine> engine;
};
struct ct_context {
  std::unique_ptr<ExecutionContext> context;
};

extern "C" {

const char* ct_last_error(void) { return g_last_error.c_str(); }
const char* ct_version(void) { return "cutriton-amd 0.1.0 (hip_gfx950)"; }

ct_model* ct_model_create(void) { return new ct_model(); }
void ct_model_destroy(ct_model* model) { delete model; }

static int ImportOnnx(const void* data, size_t bytes, const char* path, const char* const* dim_names,
                      const int64_t* dim_values, int dim_count, ct_model** model) {
  if (model == nullptr || dim_count < 0 || (dim_count > 0 && (dim_names == nullptr || dim_values == nullptr))) {
    return Invalid("ONNX import arguments are invalid");
  }
  *model = nullptr;
  OnnxDimValues dims;
  for (int i = 0; i < dim_count; ++i) {
    if (dim_names[i] == nullptr) return Invalid("symbolic dimension name is null");
    dims[dim_names[i]] = dim_values[i];
  }
  auto created = std::make_unique<ct_model>();
  const Status status = path != nullptr ? ImportOnnxFile(path, dims, &created->model)
                                        : ImportOnnxModel(data, bytes, dims, &created->model);
  if (!status.ok()) return Report(status);
  *model = created.release();
  return 0;
}

int ct_model_import_onnx(const char* path, const char* const* dim_names, const int64_t* dim_values,
                         int dim_count, ct_model** model) {
  if (path == nullptr) return Invalid("ONNX path is null");
  return ImportOnnx(nullptr, 0, path, dim_names, dim_values, dim_count, model);
}

int ct_model_import_onnx_buffer(const void* data, size_t bytes, const char* const* dim_names,
                                const int64_t* dim_values, int dim_count, ct_model** model) {
  if (data == nullptr && bytes != 0) return Invalid("ONNX buffer is null");
  return ImportOnnx(data, bytes, nullptr, dim_names, dim_values, dim_count, model);
}

int ct_model_add_input(ct_model* model, const char* name, const int64_t* shape, int rank, int dtype,
                       const char* layout) {
  if (model == nullptr || name == nullptr) return Invalid("model or name is null");
  return Report(model->model.graph().AddInput(
      name, TensorDesc(Shape(shape, rank), DtypeFromCode(dtype), DeviceType::kCPU, 0, layout ? layout : "")));
}

int ct_model_add_output(ct_model* model, const char* name) {
  if (model == nullptr || name == nullptr) return Invalid("model or name is null");
  return Report(model->model.graph().AddOutput(name));
}

int ct_model_add_constant(ct_model* model, const char* name, const int64_t* shape, int rank, int dtype,
                          const char* layout, const void* host_data, size_t bytes) {
  if (model == nullptr || name == nullptr) return Invalid("model or name is null");
  TensorDesc desc(Shape(shape, rank), DtypeFromCode(dtype), DeviceType::kCPU, 0, layout ? layout : "");
  if (desc.ByteSize() != bytes) return Invalid("constant byte count does not match its description");
  auto buffer = Buffer::AllocateHost(bytes);
  const Status copied = buffer->CopyFromHost(host_data, bytes);
  if (!copied.ok()) return Report(copied);
  return Report(model->model.AddConstant(name, Tensor(desc, buffer)));
}

int ct_model_add_node(ct_model* model, const char* name, const char* op_type, const char* const* inputs,
                      int input_count, const char* const* outputs, int output_count) {
  if (model == nullptr || name == nullptr || op_type == nullptr) return Invalid("node arguments are null");
  std::vector<std::string> in, out;
  for (int i = 0; i < input_count; ++i) in.emplace_back(inputs[i]);
  for (int i = 0; i < output_count; ++i) out.emplace_back(outputs[i]);
  return Report(model->model.graph().AddNode(Node(name, op_type, std::move(in), std::move(out))));
}

static Node* FindNode(ct_model* model, const char* node) {
  if (model == nullptr || node == nullptr) return nullptr;
  for (auto& n : model->model.graph().mutable_nodes()) {
    if (n.name() == node) return &n;
  }
  return nullptr;
}

int ct_model_set_attr_int(ct_model* model, const char* node, const char* key, int64_t value) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, value);
  return 0;
}

int ct_model_set_attr_ints(ct_model* model, const char* node, const char* key, const int64_t* values,
                           int count) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, std::vector<int64_t>(values, values + count));
  return 0;
}

int ct_model_set_attr_float(ct_model* model, const char* node, const char* key, double value) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, value);
  return 0;
}

int ct_model_set_attr_floats(ct_model* model, const char* node, const char* key, const double* values,
                             int count) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, std::vector<double>(values, values + count));
  return 0;
}

int ct_model_set_attr_bool(ct_model* model, const char* node, const char* key, int value) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, value != 0);
  return 0;
}

int ct_model_set_attr_string(ct_model* model, const char* node, const char* key, const char* value) {
  Node* n = FindNode(model, node);
  if (n == nullptr || key == nullptr || value == nullptr) return Report(Status::NotFound("node is not in the model"));
  n->SetAttribute(key, std::string(value));
  return 0;
}

int ct_model_run_default_passes(ct_model* model, int transformer_fusions, int residual_epilogue_fusion) {
  if (model == nullptr) return Invalid("model is null");
  return Report(CreateDefaultCompilePasses(transformer_fusions != 0, residual_epilogue_fusion != 0)
                    .Run(&model->model.graph()));
}

int ct_model_node_count(const ct_model* model) {
  return model == nullptr ? -1 : static_cast<int>(model->model.graph().nodes().size());
}

int ct_model_node_op_type(const ct_model* model, int index, char* buffer, size_t length) {
  if (model == nullptr || index < 0 || static_cast<std::size_t>(index) >= model->model.graph().nodes().size()) {
    return Invalid("node index is out of range");
  }
  CopyString(model->model.graph().nodes()[static_cast<std::size_t>(index)].op_type(), buffer, length);
  return 0;
}

ct_options* ct_options_create(void) { return new ct_options(); }
void ct_options_destroy(ct_options* options) { delete options; }

int ct_options_set_string(ct_options* options, const char* key, const char* value) {
  if (options == nullptr || key == nullptr || value == nullptr) return Invalid("option arguments are null");
  CompileOptions& o = options->options;
  const std::string k = key;
  if (k == "target") o.target = value;
  else if (k == "kernel_artifact_dir") o.kernel_artifact_dir = value;
  else if (k == "kernel_artifact_path") o.kernel_artifact_paths.emplace_back(value);
  else if (k == "tuning_cache_dir") o.tuning_cache_dir = value;
  else return Report(Status::NotFound("unknown string option: " + k));
  return 0;
}

int ct_options_set_int(ct_options* options, const char* key, int64_t value) {
  if (options == nullptr || key == nullptr) return Invalid("option arguments are null");
  CompileOptions& o = options->options;
  const std::string k = key;
  if (k == "enable_cuda_graph") o.enable_cuda_graph = value != 0;
  else if (k == "enable_profiling") o.enable_profiling = value != 0;
  else if (k == "enable_transformer_fusions") o.enable_transformer_fusions = value != 0;
  else if (k == "enable_residual_epilogue_fusion") o.enable_residual_epilogue_fusion = value != 0;
  else if (k == "allow_cpu_fallback") o.allow_cpu_fallback = value != 0;
  else if (k == "device_id") o.device_id = static_cast<int>(value);
  else if (k == "cuda_graph_cache_capacity") o.cuda_graph_cache_capacity = static_cast<std::size_t>(value);
  else if (k == "tuning_warmup_iterations") o.tuning_warmup_iterations = static_cast<int>(value);
  else if (k == "tuning_measurement_iterations") o.tuning_measurement_iterations = static_cast<int>(value);
  else if (k == "tuning_mode") {
    if (value < 0 || value > 3) return Invalid("tuning_mode must be 0..3");
    o.tuning_mode = static_cast<TuningMode>(value);
  } else {
    return Report(Status::NotFound("unknown integer option: " + k));
  }
  return 0;
}

int ct_options_add_profile_range(ct_options* options, const char* profile, const char* input,
                                 const int64_t* min_shape, const int64_t* opt_shape,
                                 const int64_t* max_shape, int rank) {
  if (options == nullptr || profile == nullptr || input == nullptr) return Invalid("profile arguments are null");
  auto& profiles = options->options.shape_profiles;
  auto it = std::find_if(profiles.begin(), profiles.end(), [&](const ShapeProfile& p) { return p.name == profile; });
  if (it == profiles.end()) {
    profiles.push_back(ShapeProfile{profile, {}});
    it = std::prev(profiles.end());
  }
  it->inputs[input] = ShapeRange{Shape(min_shape, rank), Shape(opt_shape, rank), Shape(max_shape, rank)};
  return 0;
}

int ct_build_engine(const ct_model* model, const ct_options* options, ct_engine** engine) {
  if (model == nullptr || options == nullptr || engine == nullptr) return Invalid("build arguments are null");
  auto built = std::make_unique<ct_engine>();
  const Status status = BuildEngine(model->model, options->options, &built->engine);
  if (!status.ok()) return Report(status);
  *engine = built.release();
  return 0;
}

void ct_engine_destroy(ct_engine* engine) { delete engine; }

int ct_engine_op_count(const ct_engine* engine) {
  return engine == nullptr ? -1 : static_cast<int>(engine->engine->plan().ops().size());
}

int ct_engine_op_info(const ct_engine* engine, int index, char* op_type, size_t op_type_length,
                      char* node_name, size_t node_name_length, int* candidate_count, int* selected_candidate) {
  if (engine == nullptr) return Invalid("engine is null");
  const auto& ops = engine->engine->plan().ops();
  if (index < 0 || static_cast<std::size_t>(index) >= ops.size()) return Invalid("op index is out of range");
  const PlanOp& op = ops[static_cast<std::size_t>(index)];
  CopyString(op.op_type, op_type, op_type_length);
  CopyString(op.node_name, node_name, node_name_length);
  if (candidate_count != nullptr) *candidate_count = static_cast<int>(op.candidates.size());
  if (selected_candidate != nullptr) *selected_candidate = static_cast<int>(op.selected_candidate);
  return 0;
}

int ct_engine_candidate_id(const ct_engine* engine, int op_index, int candidate_index, char* buffer,
                           size_t length) {
  if (engine == nullptr) return Invalid("engine is null");
  const auto& ops = engine->engine->plan().ops();
  if (op_index < 0 || static_cast<std::size_t>(op_index) >= ops.size()) return Invalid("op index is out of range");
  const auto& candidates = ops[static_cast<std::size_t>(op_index)].candidates;
  if (candidate_index < 0 || static_cast<std::size_t>(candidate_index) >= candidates.size()) {
    return Invalid("candidate index is out of range");
  }
  CopyString(candidates[static_cast<std::size_t>(candidate_index)].candidate_id, buffer, length);
  return 0;
}

int ct_engine_value_desc(const ct_engine* engine, const char* name, int64_t* shape, int* rank, int* dtype) {
  if (engine == nullptr || name == nullptr) return Invalid("engine or name is null");
  const ValueDesc* value = engine->engine->plan().graph().FindValue(name);
  if (value == nullptr) return Report(Status::NotFound(std::string("value is not in the plan: ") + name));
  return FillDesc(value->tensor, shape, rank, dtype);
}

int ct_engine_value_layout(const ct_engine* engine, const char* name, char* buffer, size_t length) {
  if (engine == nullptr || name == nullptr) return Invalid("engine or name is null");
  const ValueDesc* value = engine->engine->plan().graph().FindValue(name);
  if (value == nullptr) return Report(Status::NotFound(std::string("value is not in the plan: ") + name));
  CopyString(value->tensor.layout, buffer, length);
  return 0;
}

size_t ct_engine_workspace_bytes(const ct_engine* engine) {
  return engine == nullptr ? 0 : engine->engine->plan().memory_plan().workspace_size_bytes;
}

int ct_engine_create_context(const ct_engine* engine, ct_context** context) {
  if (engine == nullptr || context == nullptr) return Invalid("engine or context output is null");
  auto created = std::make_unique<ct_context>();
  created->context = engine->engine->CreateExecutionContext();
  *context = created.release();
  return 0;
}

void ct_context_destroy(ct_context* context) { delete context; }

static int Bind(ct_context* context, bool input, const char* name, void* data, size_t buffer_bytes,
                size_t byte_offset, const int64_t* shape, int rank, int dtype, const char* layout, int device) {
  if (context == nullptr || name == nullptr) return Invalid("bind arguments are null");
  const DeviceType type = device == 1 ? DeviceType::kHIP : DeviceType::kCPU;
  const int device_id = 0;
  TensorDesc desc(Shape(shape, rank), DtypeFromCode(dtype), type, device_id, layout ? layout : "");
  Tensor tensor(desc, Buffer::WrapExternal(data, buffer_bytes, type, device_id), byte_offset);
  return Report(input ? context->context->BindInput(name, tensor) : context->context->BindOutput(name, tensor));
}

int ct_context_bind_input(ct_context* context, const char* name, void* data, size_t buffer_bytes,
                          size_t byte_offset, const int64_t* shape, int rank, int dtype, const char* layout,
                          int device) {
  return Bind(context, true, name, data, buffer_bytes, byte_offset, shape, rank, dtype, layout, device);
}

int ct_context_bind_output(ct_context* context, const char* name, void* data, size_t buffer_bytes,
                           size_t byte_offset, const int64_t* shape, int rank, int dtype, const char* layout,
                           int device) {
  return Bind(context, false, name, data, buffer_bytes, byte_offset, shape, rank, dtype, layout, device);
}

int ct_context_select_profile(ct_context* context, const char* name) {
  if (context == nullptr || name == nullptr) return Invalid("context or name is null");
  return Report(context->context->SelectShapeProfile(name));
}

int ct_context_set_input_shape(ct_context* context, const char* name, const int64_t* shape, int rank) {
  if (context == nullptr || name == nullptr) return Invalid("context or name is null");
  return Report(context->context->SetInputShape(name, Shape(shape, rank)));
}

int ct_context_resolve_shapes(ct_context* context) {
  if (context == nullptr) return Invalid("context is null");
  return Report(context->context->ResolveShapes());
}

int ct_context_resolved_desc(const ct_context* context, const char* name, int64_t* shape, int* rank, int* dtype,
                             char* layout, size_t layout_length) {
  if (context == nullptr || name == nullptr) return Invalid("context or name is null");
  const TensorDesc* desc = context->context->GetResolvedTensorDesc(name);
  if (desc == nullptr) return Report(Status::NotFound(std::string("no resolved description for ") + name));
  CopyString(desc->layout, layout, layout_length);
  return FillDesc(*desc, shape, rank, dtype);
}

int ct_context_run(ct_context* context) {
  if (context == nullptr) return Invalid("context is null");
  return Report(context->context->Run());
}

int ct_context_run_async(ct_context* context, void* stream) {
  if (context == nullptr) return Invalid("context is null");
  return Report(context->context->RunAsync(stream));
}

int ct_context_run_async_no_alloc(ct_context* context, void* stream) {
  if (context == nullptr) return Invalid("context is null");
  return Report(context->context->RunAsyncWithoutAllocation(stream));
}

int ct_context_synchronize(ct_context* context) {
  if (context == nullptr) return Invalid("context is null");
  return Report(context->context->Synchronize());
}

int ct_context_profile_event_count(const ct_context* context) {
  return context == nullptr ? -1 : static_cast<int>(context->context->profiler().events().size());
}

int ct_context_profile_event(const ct_context* context, int index, char* name, size_t name_length,
                             double* duration_ms) {
  if (context == nullptr) return Invalid("context is null");
  const auto& events = context->context->profiler().events();
  if (index < 0 || static_cast<std::size_t>(index) >= events.size()) return Invalid("event index is out of range");
  CopyString(events[static_cast<std::size_t>(index)].name, name, name_length);
  if (duration_ms != nullptr) *duration_ms = events[static_cast<std::size_t>(index)].duration_ms;
  return 0;
}

size_t ct_context_graph_count(const ct_context* context) {
  return context == nullptr ? 0 : context->context->cached_cuda_graph_count();
}

size_t ct_context_module_count(const ct_context* context) {
  return context == nullptr ? 0 : context->context->loaded_cuda_module_count();
}

int ct_context_selected_candidate(const ct_context* context, int op_index) {
  if (context == nullptr) return -1;
  const auto& selected = context->context->selected_candidates();
  return op_index < 0 || static_cast<std::size_t>(op_index) >= selected.size()
             ? -1
             : static_cast<int>(selected[static_cast<std::size_t>(op_index)]);
}

int ct_context_time_op(ct_context* context, int op_index, int iterations, void* stream, double* ms_per_launch) {
  if (context == nullptr || op_index < 0) return Invalid("null context or negative op index");
  return Report(context->context->TimeOp(static_cast<std::size_t>(op_index), iterations, stream, ms_per_launch));
}

}  // extern "C"
