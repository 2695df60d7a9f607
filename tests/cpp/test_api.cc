// Host-side tests of the engine's C++ API (no GPU): the same public surface
// the reference's core tests exercise (tests/cpp/test_core.cpp:187-480),
// written against this library with a CPU mock backend.
//
// Build: g++ -std=c++17 -I include tests/cpp/test_api.cc -L cutriton_amd
//        -lcutriton_gfx950 -Wl,-rpath,<dir> -o test_api
// Usage: test_api [test-name ...]   (no argument: every test)
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "cutriton/backend/backend.h"
#include "cutriton/backend/kernel_artifact.h"
#include "cutriton/compiler/compiler.h"
#include "cutriton/core/buffer.h"
#include "cutriton/core/tensor.h"
#include "cutriton/ir/fusion.h"
#include "cutriton/ir/graph.h"
#include "cutriton/ir/op_schema.h"
#include "cutriton/ir/pass.h"
#include "cutriton/runtime/engine.h"
#include "cutriton/runtime/executable_plan.h"
#include "cutriton/runtime/memory_planner.h"
#include "cutriton/runtime/profiler.h"

using namespace cutriton;

namespace {

int g_failures = 0;

#define EXPECT(cond)                                                            \
  do {                                                                          \
    if (!(cond)) {                                                              \
      std::fprintf(stderr, "  %s:%d: expected %s\n", __FILE__, __LINE__, #cond); \
      ++g_failures;                                                             \
    }                                                                           \
  } while (0)

#define EXPECT_OK(expr)                                                                   \
  do {                                                                                    \
    const Status status_ = (expr);                                                        \
    if (!status_.ok()) {                                                                  \
      std::fprintf(stderr, "  %s:%d: %s -> %s\n", __FILE__, __LINE__, #expr,              \
                   status_.ToString().c_str());                                           \
      ++g_failures;                                                                       \
    }                                                                                     \
  } while (0)

// Host kernel of the mock backend: Relu computes, every other op is a no-op.
class HostKernel final : public OpKernel {
 public:
  explicit HostKernel(std::string op) : op_(std::move(op)) {}
  const char* backend_name() const override { return "mock"; }
  const char* op_type() const override { return op_.c_str(); }
  Status Compute(KernelContext* context) override {
    if (context == nullptr || context->node == nullptr || context->tensors == nullptr) {
      return Status::InvalidArgument("mock kernel called without a context");
    }
    ScopedCpuTimer timer(context->profiler, context->node->name(), "mock");
    if (op_ != "Relu") return Status::OK();
    const Tensor& in = context->tensors->at(context->node->inputs().front());
    Tensor& out = context->tensors->at(context->node->outputs().front());
    const auto* x = reinterpret_cast<const float*>(static_cast<const char*>(in.buffer()->data()) + in.byte_offset());
    auto* y = reinterpret_cast<float*>(static_cast<char*>(out.buffer()->data()) + out.byte_offset());
    const int64_t n = in.desc().NumElements();
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] > 0.0F ? x[i] : 0.0F;
    return Status::OK();
  }

 private:
  std::string op_;
};

class HostBackend final : public Backend {
 public:
  explicit HostBackend(std::string name = "mock") : name_(std::move(name)) {}
  const char* name() const override { return name_.c_str(); }
  Status CheckSupport(const Node&, const Graph&, const BackendOptions&) const override { return Status::OK(); }
  Status CreateKernel(const Node& node, const Graph&, const BackendOptions&,
                      std::unique_ptr<OpKernel>* kernel) const override {
    if (kernel == nullptr) return Status::InvalidArgument("null kernel slot");
    *kernel = std::make_unique<HostKernel>(node.op_type());
    return Status::OK();
  }

 private:
  std::string name_;
};

void UseHostBackend() {
  KernelRegistry::Global().ClearForTests();
  EXPECT_OK(KernelRegistry::Global().RegisterBackend(std::make_shared<HostBackend>()));
}

CompileOptions HostOptions() {
  CompileOptions options;
  options.target = "mock";
  options.enable_cuda_graph = false;
  return options;
}

Tensor HostTensor(std::vector<int64_t> shape, DataType dtype = DataType::kFloat32) {
  TensorDesc desc(std::move(shape), dtype);
  return Tensor(desc, Buffer::AllocateHost(desc.ByteSize()));
}

void Constant(Model* model, const std::string& name, std::vector<int64_t> shape,
              DataType dtype = DataType::kFloat32) {
  EXPECT_OK(model->AddConstant(name, HostTensor(std::move(shape), dtype)));
}

// Conv(7x7/2) -> BN(eps 1e-3) -> Relu -> GAP -> Flatten -> Gemm.
Model StemModel() {
  Model model;
  Graph& g = model.graph();
  EXPECT_OK(g.AddInput("input", TensorDesc({1, 3, 224, 224}, DataType::kFloat32)));
  Constant(&model, "w", {64, 3, 7, 7});
  for (const char* name : {"gamma", "beta", "mu", "var"}) Constant(&model, name, {64});
  Constant(&model, "fc", {64, 1000});
  Node conv("stem_conv", "Conv", {"input", "w"}, {"c"});
  conv.SetAttribute("pads", std::vector<int64_t>{3, 3, 3, 3});
  conv.SetAttribute("strides", std::vector<int64_t>{2, 2});
  conv.SetAttribute("dilations", std::vector<int64_t>{1, 1});
  EXPECT_OK(g.AddNode(std::move(conv)));
  Node bn("stem_bn", "BatchNormalization", {"c", "gamma", "beta", "mu", "var"}, {"b"});
  bn.SetAttribute("epsilon", 1e-3);
  EXPECT_OK(g.AddNode(std::move(bn)));
  EXPECT_OK(g.AddNode(Node("stem_relu", "Relu", {"b"}, {"r"})));
  EXPECT_OK(g.AddNode(Node("pool", "GlobalAveragePool", {"r"}, {"p"})));
  Node flatten("flat", "Flatten", {"p"}, {"f"});
  flatten.SetAttribute("axis", static_cast<int64_t>(1));
  EXPECT_OK(g.AddNode(std::move(flatten)));
  EXPECT_OK(g.AddNode(Node("head", "Gemm", {"f", "fc"}, {"logits"})));
  EXPECT_OK(g.AddOutput("logits"));
  return model;
}

Model ReluModel(int64_t n) {
  Model model;
  EXPECT_OK(model.graph().AddInput("x", TensorDesc({n}, DataType::kFloat32, DeviceType::kCPU)));
  EXPECT_OK(model.graph().AddNode(Node("relu", "Relu", {"x"}, {"y"})));
  EXPECT_OK(model.graph().AddOutput("y"));
  return model;
}

Model ReluChainModel() {
  Model model;
  EXPECT_OK(model.graph().AddInput("x", TensorDesc({17}, DataType::kFloat32, DeviceType::kCPU)));
  const char* chain[][3] = {{"n0", "x", "a"}, {"n1", "a", "b"}, {"n2", "b", "c"}, {"n3", "c", "y"}};
  for (const auto& link : chain) EXPECT_OK(model.graph().AddNode(Node(link[0], "Relu", {link[1]}, {link[2]})));
  EXPECT_OK(model.graph().AddOutput("y"));
  return model;
}

// Gemm -> Gelu -> Add(residual) -> LayerNormalization, FP16 [16,128]x[128,512].
Model TransformerModel(bool expose_gemm_output) {
  Model model;
  Graph& g = model.graph();
  EXPECT_OK(g.AddInput("x", TensorDesc({16, 128}, DataType::kFloat16, DeviceType::kCPU, 0, "")));
  EXPECT_OK(g.AddInput("skip", TensorDesc({16, 512}, DataType::kFloat16, DeviceType::kCPU, 0, "")));
  Constant(&model, "w", {128, 512}, DataType::kFloat16);
  Constant(&model, "gamma", {512}, DataType::kFloat16);
  Constant(&model, "beta", {512}, DataType::kFloat16);
  EXPECT_OK(g.AddNode(Node("fc", "Gemm", {"x", "w"}, {"h"})));
  EXPECT_OK(g.AddNode(Node("act", "Gelu", {"h"}, {"g"})));
  EXPECT_OK(g.AddNode(Node("join", "Add", {"g", "skip"}, {"s"})));
  Node ln("norm", "LayerNormalization", {"s", "gamma", "beta"}, {"out"});
  ln.SetAttribute("axis", static_cast<int64_t>(-1));
  ln.SetAttribute("epsilon", 1e-5);
  EXPECT_OK(g.AddNode(std::move(ln)));
  if (expose_gemm_output) EXPECT_OK(g.AddOutput("h"));
  EXPECT_OK(g.AddOutput("out"));
  return model;
}

// --- tests ------------------------------------------------------------------

void TensorsBuffersAndConstants() {
  EXPECT(TensorDesc({1, 3, 4, 5}, DataType::kFloat32).ByteSize() == 240);
  EXPECT(TensorDesc({3, 5, 7}, DataType::kFloat16).ByteSize() == 210);
  EXPECT(std::string(DataTypeName(DataType::kFloat16)) == "float16");
  EXPECT(std::string(DataTypeName(DataType::kFloat32)) == "float32");
  const TensorDesc desc({1, 3, 4, 5}, DataType::kFloat32);
  auto buffer = Buffer::AllocateHost(desc.ByteSize());
  EXPECT(buffer->owns_memory());
  Model model;
  EXPECT_OK(model.AddConstant("k", Tensor(desc, buffer)));
  EXPECT(model.constants().size() == 1);
  EXPECT(model.graph().FindValue("k") != nullptr && model.graph().FindValue("k")->is_constant);
  EXPECT(model.AddConstant("k", Tensor(desc, buffer)).code() == ErrorCode::kAlreadyExists);
  EXPECT(Model{}.AddConstant("small", Tensor(desc, Buffer::AllocateHost(4))).code() == ErrorCode::kInvalidArgument);
  // A constant added after the node that reads it still marks the value.
  Model late;
  EXPECT_OK(late.graph().AddNode(Node("add", "Add", {"x", "k2"}, {"y"})));
  EXPECT_OK(late.AddConstant("k2", Tensor(desc, buffer)));
  EXPECT(late.graph().FindValue("k2")->is_constant);
}

void CompilerPipeline() {
  UseHostBackend();
  ExecutablePlan plan;
  EXPECT_OK(Compiler{}.Compile(StemModel(), HostOptions(), &plan));
  EXPECT(plan.constants().size() == 6);
  EXPECT(plan.ops().size() == 4);
  if (plan.ops().size() == 4) {
    EXPECT(plan.ops()[0].op_type == "FusedConvBatchNormRelu");
    EXPECT(plan.ops()[1].op_type == "GlobalAveragePool");
    EXPECT(plan.ops()[2].op_type == "Flatten");
    EXPECT(plan.ops()[3].op_type == "Gemm");
  }
  const auto eps = plan.graph().nodes().front().GetAttribute<double>("batchnorm_epsilon");
  EXPECT(eps.has_value() && std::abs(*eps - 1e-3) < 1e-12);
  const ValueDesc* logits = plan.graph().FindValue("logits");
  EXPECT(logits != nullptr && (logits->tensor.shape == std::vector<int64_t>{1, 1000}));
  const ValueDesc* conv_out = plan.graph().FindValue(plan.graph().nodes().front().outputs().front());
  EXPECT(conv_out != nullptr && (conv_out->tensor.shape == std::vector<int64_t>{1, 64, 112, 112}));
  EXPECT(plan.memory_plan().workspace_size_bytes > 0);
}

void MemoryPlannerReuseAndAlias() {
  Graph g;
  EXPECT_OK(g.AddInput("in", TensorDesc({17}, DataType::kFloat32)));
  const char* chain[][3] = {{"n0", "in", "a"}, {"n1", "a", "b"}, {"n2", "b", "c"}, {"n3", "c", "out"}};
  for (const auto& link : chain) {
    EXPECT_OK(g.AddNode(Node(link[0], "Relu", {link[1]}, {link[2]})));
    EXPECT_OK(g.SetValueDesc(link[2], TensorDesc({17}, DataType::kFloat32)));
  }
  EXPECT_OK(g.AddOutput("out"));
  MemoryPlan plan;
  EXPECT_OK(MemoryPlanner{}.Plan(g, &plan));
  EXPECT(plan.workspace_size_bytes % 256 == 0);
  EXPECT(plan.allocations.size() == 3);
  if (plan.allocations.size() == 3) {
    // 68-byte intermediates: a at 0, b at 256 (a still live), c reuses a's slot.
    EXPECT(plan.allocations[0].value_name == "a" && plan.allocations[0].offset == 0);
    EXPECT(plan.allocations[1].value_name == "b" && plan.allocations[1].offset == 256);
    EXPECT(plan.allocations[2].value_name == "c" && plan.allocations[2].offset == 0);
    EXPECT(plan.allocations[2].reused);
    EXPECT(!plan.allocations[0].reused && !plan.allocations[1].reused);
  }
  EXPECT(plan.workspace_size_bytes == 512);

  Graph alias;
  EXPECT_OK(alias.AddInput("x", TensorDesc({1, 4}, DataType::kFloat32)));
  EXPECT_OK(alias.AddNode(Node("r0", "Relu", {"x"}, {"hidden"})));
  EXPECT_OK(alias.SetValueDesc("hidden", TensorDesc({1, 4}, DataType::kFloat32)));
  EXPECT_OK(alias.AddNode(Node("flat", "Flatten", {"hidden"}, {"view"})));
  EXPECT_OK(alias.SetValueDesc("view", TensorDesc({1, 4}, DataType::kFloat32, DeviceType::kCPU, 0, "")));
  EXPECT_OK(alias.AddNode(Node("r1", "Relu", {"view"}, {"y"})));
  EXPECT_OK(alias.SetValueDesc("y", TensorDesc({1, 4}, DataType::kFloat32)));
  EXPECT_OK(alias.AddOutput("y"));
  EXPECT_OK(MemoryPlanner{}.Plan(alias, &plan));
  EXPECT(plan.allocations.size() == 2);
  if (plan.allocations.size() == 2) {
    EXPECT(plan.allocations[1].value_name == "view");
    EXPECT(plan.allocations[1].alias_of == "hidden");
    EXPECT(plan.allocations[1].offset == plan.allocations[0].offset);
  }
}

void RegistryThreadSafety() {
  auto& registry = KernelRegistry::Global();
  registry.ClearForTests();
  std::vector<std::thread> threads;
  for (int i = 0; i < 8; ++i) {
    threads.emplace_back([i, &registry] {
      EXPECT_OK(registry.RegisterBackend(std::make_shared<HostBackend>("host_" + std::to_string(i))));
    });
  }
  for (auto& t : threads) t.join();
  EXPECT(registry.AvailableBackends().size() == 8);
  EXPECT(registry.RegisterBackend(std::make_shared<HostBackend>("host_3")).code() == ErrorCode::kAlreadyExists);
  EXPECT(registry.GetBackend("host_5") != nullptr);
}

void SchemasFusionsAndShapeProfiles() {
  OpSchemaRegistry::Global().ClearForTests();
  FusionRegistry::Global().ClearForTests();
  EXPECT_OK(RegisterBuiltinOpSchemas());
  EXPECT_OK(RegisterBuiltinFusionAlternatives());
  const auto relu = OpSchemaRegistry::Global().Find("Relu");
  EXPECT(relu != nullptr && relu->min_inputs == 1 && relu->outputs == 1);
  const auto conv_bn_relu = FusionRegistry::Global().Find("FusedConvBatchNormRelu");
  EXPECT(conv_bn_relu.size() == 1);
  if (!conv_bn_relu.empty()) {
    EXPECT((conv_bn_relu.front().decomposed_ops == std::vector<std::string>{"Conv", "BatchNormalization", "Relu"}));
  }
  const auto add_relu = FusionRegistry::Global().Find("FusedConvBatchNormAddRelu");
  EXPECT(add_relu.size() == 1);
  if (!add_relu.empty()) {
    EXPECT((add_relu.front().decomposed_ops == std::vector<std::string>{"FusedConvBatchNorm", "AddRelu"}));
  }
  EXPECT(FusionRegistry::Global().Find("GemmGelu").size() == 1);
  EXPECT(FusionRegistry::Global().Find("SkipLayerNormalization").size() == 1);
  const auto fused_schema = OpSchemaRegistry::Global().Find("FusedConvBatchNormAddRelu");
  EXPECT(fused_schema != nullptr && fused_schema->min_inputs == 7);

  UseHostBackend();
  CompileOptions options = HostOptions();
  ShapeProfile profile;
  profile.name = "batch";
  profile.inputs["x"] = ShapeRange{{2}, {4}, {8}};
  options.shape_profiles = {profile};
  std::unique_ptr<Engine> engine;
  EXPECT_OK(BuildEngine(ReluModel(4), options, &engine));
  if (!engine) return;
  EXPECT(engine->plan().profile_plans().size() == 1);
  EXPECT((engine->plan().profile_plans()[0].max_graph.FindValue("y")->tensor.shape == std::vector<int64_t>{8}));
  auto context = engine->CreateExecutionContext();
  EXPECT_OK(context->SetInputShape("x", {2}));
  EXPECT_OK(context->ResolveShapes());
  EXPECT((context->GetResolvedTensorDesc("y")->shape == std::vector<int64_t>{2}));
  EXPECT(context->SetInputShape("x", {9}).code() == ErrorCode::kShapeError);
  EXPECT(context->SelectShapeProfile("no_such_profile").code() == ErrorCode::kNotFound);
}

void TransformerFusionPasses() {
  Model model = TransformerModel(false);
  EXPECT_OK(CreateDefaultCompilePasses().Run(&model.graph()));
  const auto& nodes = model.graph().nodes();
  EXPECT(nodes.size() == 2);
  if (nodes.size() == 2) {
    EXPECT(nodes[0].op_type() == "GemmGelu");
    EXPECT(nodes[1].op_type() == "SkipLayerNormalization");
    EXPECT(nodes[1].GetAttribute<double>("epsilon").value_or(0.0) == 1e-5);
  }
  const ValueDesc* out = model.graph().FindValue("out");
  EXPECT(out != nullptr && out->tensor.dtype == DataType::kFloat16);
  EXPECT(out != nullptr && (out->tensor.shape == std::vector<int64_t>{16, 512}));

  // The GEMM output is a graph output: Gemm+Gelu must stay apart.
  Model observable = TransformerModel(true);
  EXPECT_OK(CreateDefaultCompilePasses().Run(&observable.graph()));
  EXPECT(observable.graph().nodes().size() >= 2);
  if (observable.graph().nodes().size() >= 2) {
    EXPECT(observable.graph().nodes()[0].op_type() == "Gemm");
    EXPECT(observable.graph().nodes()[1].op_type() == "Gelu");
  }
  // Transformer fusions off: the graph keeps its four nodes.
  Model unfused = TransformerModel(false);
  EXPECT_OK(CreateDefaultCompilePasses(false).Run(&unfused.graph()));
  EXPECT(unfused.graph().nodes().size() == 4);
}

std::filesystem::path ScratchDir(const char* tag) {
  const auto stamp = std::chrono::steady_clock::now().time_since_epoch().count();
  auto root = std::filesystem::temp_directory_path() / (std::string("cutriton-") + tag + "-" + std::to_string(stamp));
  std::filesystem::create_directories(root / "kernels");
  return root;
}

// SHA-256 of the 7 bytes "// ptx\n" (a known answer, checked with sha256sum).
constexpr const char* kDummySha = "f2ee4765bc61528cec8f6987ea5b1c2ea694169ea5ab848e2026139b285db499";

std::string PackText(int abi, const std::string& grid, const std::string& overrides = "") {
  std::map<std::string, std::string> f = {
      {"binary", "\"kernels/dummy.hsaco\""}, {"binary_format", "\"hsaco\""}, {"sha256", std::string("\"") + kDummySha + "\""},
      {"min_compute_capability", "950"}, {"schema_version", "2"}, {"default", "true"},
  };
  // overrides: "key=value;key=value"
  size_t pos = 0;
  while (pos < overrides.size()) {
    const size_t end = std::min(overrides.find(';', pos), overrides.size());
    const std::string item = overrides.substr(pos, end - pos);
    const size_t eq = item.find('=');
    f[item.substr(0, eq)] = item.substr(eq + 1);
    pos = end + 1;
  }
  return "{\n \"schema_version\": " + f["schema_version"] + ",\n \"abi_schema_version\": " + std::to_string(abi) +
         ",\n \"pack_name\": \"unit\", \"pack_version\": 1, \"generator_version\": \"unit\", \"triton_version\": \"unit\",\n"
         " \"kernels\": [{\n  \"kernel_id\": \"relu.unit\", \"op_type\": \"Relu\", \"kernel_version\": 1,\n"
         "  \"variant_id\": \"only\", \"default\": " + f["default"] + ", \"symbol\": \"relu\",\n"
         "  \"binary\": " + f["binary"] + ", \"binary_format\": " + f["binary_format"] + ", \"sha256\": " + f["sha256"] + ",\n"
         "  \"dtype\": \"float32\", \"layout\": \"\", \"min_compute_capability\": " + f["min_compute_capability"] + ",\n"
         "  \"target_arch\": \"gfx950\", \"num_warps\": 4, \"num_stages\": 1, \"shared_memory_bytes\": 0,\n"
         "  \"arguments\": [\n"
         "   {\"name\": \"x\", \"type\": \"*fp32\", \"source\": {\"kind\": \"input\", \"index\": 0}},\n"
         "   {\"name\": \"output\", \"type\": \"*fp32\", \"source\": {\"kind\": \"output\", \"index\": 0}},\n"
         "   {\"name\": \"runtime_scratch\", \"type\": \"*i8\", \"source\": {\"kind\": \"runtime_reserved\"}},\n"
         "   {\"name\": \"profile_scratch\", \"type\": \"*i8\", \"source\": {\"kind\": \"runtime_reserved\"}}],\n"
         "  \"constraints\": [], \"tuning\": {\"BLOCK\": 256},\n"
         "  \"grid\": " + grid + "\n }]\n}\n";
}

void KernelPackAbi() {
  const auto root = ScratchDir("pack");
  std::ofstream(root / "kernels" / "dummy.hsaco", std::ios::binary) << "// ptx\n";
  auto write = [&](const std::string& text) { std::ofstream(root / "pack.json") << text; };
  ArtifactRepository repo;
  const std::string v2_grid =
      R"([{"kind":"ceil_div","args":[{"kind":"output_numel","index":0},{"kind":"meta","name":"BLOCK"}]}])";

  // ABI v1 grid object: ceil(output_numel / divisor).
  write(PackText(1, R"({"op":"ceil_div","value":{"kind":"output_numel","index":0},"divisor":256})"));
  EXPECT_OK(repo.Load({root.string()}));
  if (!repo.artifacts().empty()) {
    EXPECT(repo.artifacts().front().abi_schema_version == 1);
    EXPECT(repo.artifacts().front().launch_grid[0].kind == GridExpressionKind::kCeilDiv);
    EXPECT(repo.artifacts().front().sha256 == kDummySha);
  }
  // ABI v2 grid AST with a meta lookup; the folder or the pack.json path.
  write(PackText(2, v2_grid));
  EXPECT_OK(repo.Load({root.string()}));
  if (!repo.artifacts().empty()) {
    EXPECT(repo.artifacts().front().abi_schema_version == 2);
    EXPECT(repo.artifacts().front().launch_meta.at("BLOCK") == 256);
    EXPECT(repo.artifacts().front().block_threads() == 256);
    EXPECT(repo.artifacts().front().identity() == "unit:relu.unit:only");
  }
  EXPECT_OK(repo.Load({(root / "pack.json").string()}));

  // Rejections (all InvalidArgument).
  const std::pair<std::string, std::string> bad[] = {
      {"expression grid", PackText(2, R"([{"kind":"python","expression":"unsafe"}])")},
      {"sha mismatch", PackText(2, v2_grid, "sha256=\"" + std::string(64, '0') + "\"")},
      {"absolute binary", PackText(2, v2_grid, "binary=\"/etc/passwd\"")},
      {"parent binary", PackText(2, v2_grid, "binary=\"../kernels/dummy.hsaco\"")},
      {"ptx format", PackText(2, v2_grid, "binary_format=\"ptx\"")},
      {"schema v1", PackText(2, v2_grid, "schema_version=1")},
      {"no default", PackText(2, v2_grid, "default=false")},
      {"abi v3", PackText(3, v2_grid)},
  };
  for (const auto& [what, text] : bad) {
    write(text);
    const Status s = repo.Load({root.string()});
    if (s.code() != ErrorCode::kInvalidArgument) {
      std::fprintf(stderr, "  pack case '%s' gave %s\n", what.c_str(), s.ToString().c_str());
      ++g_failures;
    }
  }
  // Two variants share one code object: the file is hashed once per load,
  // and each entry's sha256 is still checked against that digest.
  {
    const std::string text = PackText(2, v2_grid);
    const size_t begin = text.find("{\n  \"kernel_id\"");
    const size_t end = text.rfind("\n }") + 3;
    std::string second = text.substr(begin, end - begin);
    second.replace(second.find("\"only\""), 6, "\"second\"");
    second.replace(second.find("\"default\": true"), 15, "\"default\": false");
    write(text.substr(0, end) + ", " + second + text.substr(end));
    EXPECT_OK(repo.Load({root.string()}));
    EXPECT(repo.artifacts().size() == 2);
    second.replace(second.find(kDummySha), 64, std::string(64, '0'));
    write(text.substr(0, end) + ", " + second + text.substr(end));
    EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);
  }
  // Input layouts: OHWI on an input is accepted; any other layout, or a
  // layout on an output, is rejected.
  auto with_source = [&](const std::string& from, const std::string& to) {
    std::string text = PackText(2, v2_grid);
    text.replace(text.find(from), from.size(), to);
    return text;
  };
  const std::string x_source = R"("source": {"kind": "input", "index": 0})";
  const std::string y_source = R"("source": {"kind": "output", "index": 0})";
  write(with_source(x_source, R"("source": {"kind": "input", "index": 0, "layout": "OHWI"})"));
  EXPECT_OK(repo.Load({root.string()}));
  if (!repo.artifacts().empty()) EXPECT(repo.artifacts().front().arguments[0].source.layout == "OHWI");
  EXPECT(LaidOutConstantName("w", "OHWI") == "w#OHWI");
  write(with_source(x_source, R"("source": {"kind": "input", "index": 0, "layout": "NHWC"})"));
  EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);
  write(with_source(y_source, R"("source": {"kind": "output", "index": 0, "layout": "OHWI"})"));
  EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);
  write(with_source(x_source, R"("source": {"kind": "input", "index": 0, "layout": "NK"})"));
  EXPECT_OK(repo.Load({root.string()}));
  if (!repo.artifacts().empty()) EXPECT(repo.artifacts().front().arguments[0].source.layout == "NK");

  // dim_le constraints: parsed with their axis; a bad source or a missing
  // axis is rejected.
  auto with_constraints = [&](const std::string& list) {
    std::string text = PackText(2, v2_grid);
    const std::string from = "\"constraints\": []";
    text.replace(text.find(from), from.size(), "\"constraints\": " + list);
    return text;
  };
  write(with_constraints(R"([{"kind": "dim_le", "source": "input", "index": 0, "axis": 1, "value": 4}])"));
  EXPECT_OK(repo.Load({root.string()}));
  if (!repo.artifacts().empty() && !repo.artifacts().front().constraints.empty()) {
    const KernelConstraint& c = repo.artifacts().front().constraints.front();
    EXPECT(c.kind == KernelConstraintKind::kTensorDimAtMost && c.tensor_axis == 1 && c.expected == 4);
  }
  write(with_constraints(R"([{"kind": "dim_le", "source": "weights", "index": 0, "axis": 1, "value": 4}])"));
  EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);
  write(with_constraints(R"([{"kind": "dim_le", "source": "input", "index": 0, "value": 4}])"));
  EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);

  // Too deep a grid tree (depth 9).
  std::string deep = R"({"kind":"literal","value":1})";
  for (int i = 0; i < 9; ++i) deep = R"({"kind":"mul","args":[)" + deep + R"(,{"kind":"literal","value":1}]})";
  write(PackText(2, "[" + deep + "]"));
  EXPECT(repo.Load({root.string()}).code() == ErrorCode::kInvalidArgument);
  // A missing pack.
  EXPECT(repo.Load({(root / "absent").string()}).code() != ErrorCode::kOk);
  std::filesystem::remove_all(root);
}

void HostExecutionAndLifetime() {
  UseHostBackend();
  CompileOptions options = HostOptions();
  options.enable_profiling = true;
  std::unique_ptr<Engine> engine;
  EXPECT_OK(BuildEngine(ReluModel(4), options, &engine));
  if (!engine) return;
  auto context = engine->CreateExecutionContext();
  const TensorDesc in_desc = engine->plan().graph().FindValue("x")->tensor;
  const TensorDesc out_desc = engine->plan().graph().FindValue("y")->tensor;
  engine.reset();  // the context keeps the engine state alive

  Tensor input(in_desc, Buffer::AllocateHost(in_desc.ByteSize()));
  Tensor output(out_desc, Buffer::AllocateHost(out_desc.ByteSize()));
  const float values[4] = {-2.0F, -0.5F, 1.0F, 3.0F};
  EXPECT_OK(input.buffer()->CopyFromHost(values, sizeof(values)));
  EXPECT(context->BindInput("y", input).code() == ErrorCode::kNotFound);
  EXPECT(context->BindInput("x", HostTensor({5})).code() == ErrorCode::kInvalidArgument);
  EXPECT_OK(context->BindInput("x", input));
  EXPECT_OK(context->BindOutput("y", output));
  EXPECT_OK(context->RunAsync(nullptr));
  EXPECT(context->RunAsync(nullptr).code() == ErrorCode::kRuntimeError);  // one pending run at most
  EXPECT_OK(context->Synchronize());
  float result[4] = {9, 9, 9, 9};
  EXPECT_OK(output.buffer()->CopyToHost(result, sizeof(result)));
  EXPECT(result[0] == 0.0F && result[1] == 0.0F && result[2] == 1.0F && result[3] == 3.0F);
  EXPECT(context->profiler().events().size() == 1);

  options.enable_profiling = false;
  EXPECT_OK(BuildEngine(ReluModel(4), options, &engine));
  auto quiet = engine->CreateExecutionContext();
  EXPECT_OK(quiet->BindInput("x", input));
  EXPECT_OK(quiet->BindOutput("y", output));
  EXPECT_OK(quiet->Run());
  EXPECT(quiet->profiler().events().empty());
}

void WorkspaceBacksIntermediates() {
  UseHostBackend();
  std::unique_ptr<Engine> engine;
  EXPECT_OK(BuildEngine(ReluChainModel(), HostOptions(), &engine));
  if (!engine) return;
  auto context = engine->CreateExecutionContext();
  const auto in_desc = engine->plan().graph().FindValue("x")->tensor;
  const auto out_desc = engine->plan().graph().FindValue("y")->tensor;
  EXPECT_OK(context->BindInput("x", Tensor(in_desc, Buffer::AllocateHost(in_desc.ByteSize()))));
  EXPECT_OK(context->BindOutput("y", Tensor(out_desc, Buffer::AllocateHost(out_desc.ByteSize()))));
  EXPECT_OK(context->Run());
  const auto& t = context->tensors();
  EXPECT(t.at("a").buffer() == t.at("b").buffer());
  EXPECT(t.at("a").buffer() == t.at("c").buffer());
  EXPECT(t.at("a").byte_offset() == t.at("c").byte_offset());
  EXPECT(t.at("a").byte_offset() != t.at("b").byte_offset());
}

void CpuReferenceBackendIsUnsupported() {
  KernelRegistry::Global().ClearForTests();
  EXPECT_OK(RegisterBuiltinBackends());
  CompileOptions options;
  options.target = "cpu_reference";
  options.enable_cuda_graph = false;
  std::unique_ptr<Engine> engine;
  const Status s = BuildEngine(ReluModel(4), options, &engine);
  EXPECT(s.code() == ErrorCode::kUnsupported);
}

}  // namespace

int main(int argc, char** argv) {
  const std::vector<std::pair<const char*, std::function<void()>>> tests = {
      {"tensors_buffers_and_constants", TensorsBuffersAndConstants},
      {"compiler_pipeline", CompilerPipeline},
      {"memory_planner_reuse_and_alias", MemoryPlannerReuseAndAlias},
      {"registry_thread_safety", RegistryThreadSafety},
      {"schemas_fusions_and_shape_profiles", SchemasFusionsAndShapeProfiles},
      {"transformer_fusion_passes", TransformerFusionPasses},
      {"kernel_pack_abi", KernelPackAbi},
      {"host_execution_and_lifetime", HostExecutionAndLifetime},
      {"workspace_backs_intermediates", WorkspaceBacksIntermediates},
      {"cpu_reference_backend_is_unsupported", CpuReferenceBackendIsUnsupported},
  };
  int failed_tests = 0;
  for (const auto& [name, fn] : tests) {
    bool selected = argc <= 1;
    for (int i = 1; i < argc; ++i) selected |= std::strcmp(argv[i], name) == 0;
    if (!selected) continue;
    const int before = g_failures;
    fn();
    const bool ok = g_failures == before;
    failed_tests += ok ? 0 : 1;
    std::printf("%s %s\n", ok ? "ok" : "FAIL", name);
  }
  return failed_tests == 0 ? 0 : 1;
}
