// Contract test of tensorcx::hip::HipBackend::execute at the C++ backend ABI.
//
// The reference holds its CUDA backend to three properties
// (tests/cpp/test_cuda_backend_contract.cpp:416-443, 568-599, 604-625); this
// program checks the same three for the hip device, with its own requests:
//
//   1. A malformed request (wrong op class, launch metadata on a primitive,
//      wrong arity, a tensor that is not a contiguous device-0 hip tensor,
//      axes, shapes, dtypes or parameters the op's plan rejects) returns
//      kInvalidArgument before any allocation: the active pool's
//      allocation_calls do not move, and every output slot keeps exactly what
//      the caller put there.
//   2. The same requests are rejected on a machine without a device: they
//      never reach the device. Here the tensors' buffers come from a bounded
//      pool over a host allocator (the pool's injectable runtime), and the
//      program then exits 77, as the reference's test does without CUDA.
//   3. With a device: well-formed requests of every hot-path family run once
//      outside any pool and then twice inside a bounded pool, with
//      bit-identical results; known answers pin a few of them; the pool
//      reuses blocks, stays within its bounds and holds nothing after exit.
//
// Built by tensor.cx_amd/build.py (build_contract) into tests/cpp/_bin/.

#include <array>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <iostream>
#include <limits>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "tensorcx/backends/hip/hip_backend.h"
#include "tensorcx/core/backend.h"
#include "tensorcx_hip.h"

namespace {

using namespace tensorcx;

int failures = 0;

void expect(bool ok, const std::string& what) {
  if (!ok) {
    std::cerr << "FAIL: " << what << '\n';
    ++failures;
  }
}

const char* code_name(StatusCode code) {
  switch (code) {
    case StatusCode::kOk: return "ok";
    case StatusCode::kInvalidArgument: return "invalid_argument";
    case StatusCode::kUnavailable: return "unavailable";
    default: return "internal";
  }
}

// Storage that is not device memory.
class HostBytes final : public Buffer {
 public:
  explicit HostBytes(std::size_t n) : bytes_(n) {}
  std::size_t nbytes() const override { return bytes_.size(); }

 private:
  std::vector<unsigned char> bytes_;
};

// ---------------------------------------------------------------- pools
// Host allocator behind the pool's seam: lets HipBuffer::create hand out
// buffers without a device, so request validation is testable anywhere.
int host_allocate(void** ptr, std::size_t bytes) {
  *ptr = std::aligned_alloc(256, (bytes + 255) / 256 * 256);
  return *ptr ? TCX_OK : TCX_POOL_OOM;
}
int host_free(void* ptr) {
  std::free(ptr);
  return TCX_OK;
}
int host_clear() { return TCX_OK; }

struct Pool {
  tcx_hip_pool_t* pool{nullptr};
  Pool(std::size_t max_bytes, std::size_t max_blocks, const tcx_hip_pool_runtime_t* runtime) {
    if (tcx_hip_pool_create(max_bytes, max_blocks, runtime, &pool) != TCX_OK)
      throw std::runtime_error(std::string("pool create: ") + tcx_hip_last_error());
  }
  ~Pool() { tcx_hip_pool_destroy(pool); }
  tcx_hip_pool_stats_t stats() const {
    tcx_hip_pool_stats_t s{};
    tcx_hip_pool_stats(pool, &s);
    return s;
  }
  void enter() {
    if (tcx_hip_pool_enter(pool) != TCX_OK) throw std::runtime_error(std::string("pool enter: ") + tcx_hip_last_error());
  }
  bool exit() { return tcx_hip_pool_exit(pool) == TCX_OK; }
};

// ---------------------------------------------------------------- tensors
// An uninitialised contiguous hip tensor from whatever tcx_hip_allocate
// serves (the entered pool, else the device).
Tensor make(DType dtype, Shape shape) {
  const auto bytes = static_cast<std::size_t>(numel(shape)) * dtype_size(dtype);
  auto buffer = hip::HipBuffer::create(bytes);
  if (!buffer) throw std::runtime_error("buffer: " + buffer.status().message());
  Shape strides = contiguous_strides(shape);
  return Tensor{dtype, std::move(shape), std::move(strides), Device{"hip", 0},
                std::static_pointer_cast<Buffer>(buffer.move_value()), 0};
}

template <typename T>
Tensor upload(DType dtype, Shape shape, const std::vector<T>& values) {
  auto t = hip::from_host(values.data(), dtype, std::move(shape));
  if (!t) throw std::runtime_error("upload: " + t.status().message());
  return t.move_value();
}

std::vector<std::uint32_t> download_words(const Tensor& t) {
  std::vector<std::uint32_t> words((static_cast<std::size_t>(numel(t.shape)) * dtype_size(t.dtype) + 3) / 4);
  std::vector<unsigned char> bytes(static_cast<std::size_t>(numel(t.shape)) * dtype_size(t.dtype));
  const Status s = hip::to_host(t, bytes.data(), bytes.size());
  if (!s.ok()) throw std::runtime_error("download: " + s.message());
  if (!bytes.empty()) std::memcpy(words.data(), bytes.data(), bytes.size());
  return words;
}

std::vector<float> download_floats(const Tensor& t) {
  std::vector<float> v(static_cast<std::size_t>(numel(t.shape)));
  const Status s = hip::to_host(t, v.data(), v.size() * sizeof(float));
  if (!s.ok()) throw std::runtime_error("download: " + s.message());
  return v;
}

bool same_slot(const Tensor& a, const Tensor& b) {
  return a.dtype == b.dtype && a.shape == b.shape && a.strides == b.strides && a.device.type == b.device.type &&
         a.device.index == b.device.index && a.buffer == b.buffer && a.offset == b.offset;
}

// ---------------------------------------------------------------- requests
struct Request {
  std::string name;
  BackendOpClass op_class{BackendOpClass::kPrimitive};
  OpDesc op{};
  std::vector<Tensor> inputs;
  std::vector<Tensor> outputs;
  std::optional<LaunchConfig> launch;
  std::optional<CompilationTarget> target;
  std::vector<Tensor> argument_tensors;  // what tensor kernel arguments point at
  std::vector<KernelArgument> arguments;

  Status run() {
    for (std::size_t i = 0, t = 0; i < arguments.size(); ++i)
      if (arguments[i].kind == KernelArgumentKind::kTensor && t < argument_tensors.size())
        arguments[i].tensor = &argument_tensors[t++];
    BackendExecution e{op_class, op, inputs, outputs, launch, target, arguments};
    hip::HipBackend backend;
    return backend.execute(e);
  }
};

// Requests that must fail with kInvalidArgument. x and y are good float32 [3]
// hip tensors, xi a good int32 [3] one, empty a good float32 [0] one, and
// slot the tensor placed in output slots that must stay untouched.
std::vector<Request> malformed(const Tensor& x, const Tensor& y, const Tensor& xi, const Tensor& empty,
                               const Tensor& slot) {
  std::vector<Request> out;
  const Tensor descriptor{DType::kFloat32, {3}, {1}, {"hip", 0}, nullptr, 0};
  auto fill = [&](std::string name, std::function<void(Request&)> change) {
    Request r{std::move(name)};
    r.op = OpDesc{OpKind::kFill};
    r.op.scalar_value = 2.5;
    r.outputs = {descriptor};
    change(r);
    out.push_back(std::move(r));
  };
  fill("fill without an output slot", [](Request& r) { r.outputs.clear(); });
  fill("fill with launch metadata", [](Request& r) { r.launch = LaunchConfig{1, 1, 1, 1, 1, 1}; });
  fill("fill with a compilation target",
       [](Request& r) { r.target = CompilationTarget{KernelArtifactKind::kStaticLibrary, "tensorcx_hip", "bias_act"}; });
  fill("fill with kernel arguments", [](Request& r) { r.arguments = {KernelArgument{KernelArgumentKind::kUInt32, nullptr, 1}}; });
  fill("fill sent as a kernel", [](Request& r) { r.op_class = BackendOpClass::kKernel; });
  fill("fill descriptor on cpu", [](Request& r) { r.outputs[0].device.type = "cpu"; });
  fill("fill descriptor on device 1", [](Request& r) { r.outputs[0].device.index = 1; });
  fill("fill descriptor on device -1", [](Request& r) { r.outputs[0].device.index = -1; });
  fill("fill descriptor with an offset", [](Request& r) { r.outputs[0].offset = 1; });
  fill("fill descriptor with strides {2}", [](Request& r) { r.outputs[0].strides = {2}; });
  fill("fill descriptor of dtype 255", [](Request& r) { r.outputs[0].dtype = static_cast<DType>(255); });
  fill("fill descriptor carrying a buffer", [&](Request& r) { r.outputs[0].buffer = x.buffer; });
  fill("fill descriptor with extent -1", [](Request& r) {
    r.outputs[0].shape = {-1};
    r.outputs[0].strides = {1};
  });
  fill("fill descriptor past size_t bytes", [](Request& r) {
    r.outputs[0].shape = {std::numeric_limits<std::int64_t>::max() / 2 + 1};
  });
  fill("int32 fill of 0.5", [](Request& r) {
    r.outputs[0].dtype = DType::kInt32;
    r.op.scalar_value = 0.5;
  });

  auto add = [&](std::string name, std::function<void(Request&)> change) {
    Request r{std::move(name)};
    r.op = OpDesc{OpKind::kAdd};
    r.inputs = {x, y};
    r.outputs = {slot};
    change(r);
    out.push_back(std::move(r));
  };
  add("add with one input", [](Request& r) { r.inputs.pop_back(); });
  add("add with three inputs", [&](Request& r) { r.inputs.push_back(y); });
  add("add with two output slots", [&](Request& r) { r.outputs.push_back(slot); });
  add("add with launch metadata", [](Request& r) { r.launch = LaunchConfig{3, 1, 1, 64, 1, 1}; });
  add("add with an unknown op kind", [](Request& r) { r.op.kind = static_cast<OpKind>(250); });
  add("add of a cpu input", [](Request& r) { r.inputs[0].device.type = "cpu"; });
  add("add of a device-1 input", [](Request& r) { r.inputs[0].device.index = 1; });
  add("add of an offset input", [](Request& r) { r.inputs[0].offset = 1; });
  add("add of a strided input", [](Request& r) { r.inputs[0].strides = {2}; });
  add("add of an input without a buffer", [](Request& r) { r.inputs[0].buffer.reset(); });
  add("add of an input in host memory", [](Request& r) { r.inputs[0].buffer = std::make_shared<HostBytes>(12); });
  add("add of an input larger than its buffer", [](Request& r) {
    r.inputs[0].shape = {4};
    r.inputs[0].strides = {1};
  });
  add("add of mixed dtypes", [&](Request& r) { r.inputs[1] = xi; });
  add("add of bool inputs", [](Request& r) {
    r.inputs[0].dtype = DType::kBool;
    r.inputs[1].dtype = DType::kBool;
  });
  add("add of an input with extent -1", [](Request& r) { r.inputs[0].shape = {-1}; });
  add("add of broadcast-incompatible shapes", [&](Request& r) {
    r.inputs[1].shape = {2};
    r.inputs[1].strides = {1};
  });
  add("int32 division", [&](Request& r) {
    r.op.kind = OpKind::kDivide;
    r.inputs = {xi, xi};
  });

  auto unary = [&](std::string name, OpDesc op, Tensor input) {
    Request r{std::move(name)};
    r.op = op;
    r.inputs = {std::move(input)};
    r.outputs = {slot};
    out.push_back(std::move(r));
  };
  OpDesc sum_axis{OpKind::kSum};
  sum_axis.axis = 1;
  unary("sum over axis 1 of a rank-1 tensor", sum_axis, x);
  OpDesc repeated{OpKind::kSum};
  repeated.reduction_axes = Shape{0, 0};
  unary("sum over a repeated axis", repeated, x);
  OpDesc out_of_range{OpKind::kMean};
  out_of_range.reduction_axes = Shape{-2};
  unary("mean over axis -2 of a rank-1 tensor", out_of_range, x);
  unary("max over an empty axis", OpDesc{OpKind::kMax}, empty);
  unary("mean of int32", OpDesc{OpKind::kMean}, xi);
  OpDesc argmax_empty{OpKind::kArgmax};
  argmax_empty.reduction_axes = Shape{0};
  unary("argmax over an empty axis", argmax_empty, empty);
  unary("softmax of int32", OpDesc{OpKind::kSoftmax}, xi);
  OpDesc negative_eps{OpKind::kLayerNorm};
  negative_eps.epsilon = -1.0;
  unary("layernorm with a negative epsilon", negative_eps, x);
  OpDesc huge_eps{OpKind::kRmsNorm};
  huge_eps.epsilon = 1e300;
  unary("rmsnorm with an epsilon past float32", huge_eps, x);
  unary("exp of int32", OpDesc{OpKind::kExp}, xi);

  auto binary = [&](std::string name, OpKind kind, std::vector<Tensor> inputs) {
    Request r{std::move(name)};
    r.op = OpDesc{kind};
    r.inputs = std::move(inputs);
    r.outputs = {slot};
    out.push_back(std::move(r));
  };
  Tensor w23 = x;  // [3] storage viewed as [1, 3]: a (1, 3) weight
  w23.shape = {1, 3};
  w23.strides = {3, 1};
  Tensor m13 = w23;
  binary("matmul of int32", OpKind::kMatmul, {xi, xi});
  binary("matmul of mismatched inner sizes", OpKind::kMatmul, {m13, m13});
  binary("matmul of a scalar", OpKind::kMatmul, {[&] {
                                                   Tensor s = x;
                                                   s.shape = {};
                                                   s.strides = {};
                                                   return s;
                                                 }(),
                                                 x});
  Tensor w24 = x;
  w24.shape = {3, 1};
  w24.strides = {1, 1};
  binary("linear with a weight of the wrong width", OpKind::kLinear, {x, w24});
  binary("linear with a bias of the wrong size", OpKind::kLinear, {x, w23, x});
  binary("attention with mismatched features", OpKind::kAttention, {m13, w24, m13});

  auto kernel = [&](std::string name, CompilationTarget target, std::vector<Tensor> tensors) {
    Request r{std::move(name)};
    r.op_class = BackendOpClass::kKernel;
    r.launch = LaunchConfig{3, 1, 1, 64, 1, 1};
    r.target = std::move(target);
    r.outputs = {slot};
    r.argument_tensors = std::move(tensors);
    for (std::size_t i = 0; i < r.argument_tensors.size(); ++i)
      r.arguments.push_back(KernelArgument{KernelArgumentKind::kTensor, nullptr, 0});
    r.arguments.push_back(KernelArgument{KernelArgumentKind::kUInt32, nullptr, TCX_ACT_NONE});
    out.push_back(std::move(r));
  };
  kernel("kernel with an unknown artifact", CompilationTarget{KernelArtifactKind::kBinary, "unused", "entry"}, {x});
  kernel("kernel with an unknown entry point", CompilationTarget{KernelArtifactKind::kStaticLibrary, "tensorcx_hip", "nope"},
         {x, y});
  kernel("bias_act with a bias of the wrong size",
         CompilationTarget{KernelArtifactKind::kStaticLibrary, "tensorcx_hip", "bias_act"}, {x, w23});
  kernel("kernel without launch dimensions", CompilationTarget{KernelArtifactKind::kStaticLibrary, "tensorcx_hip", "bias_act"},
         {x, x});
  out.back().launch = LaunchConfig{0, 1, 1, 64, 1, 1};
  return out;
}

// Runs every malformed request; each must be kInvalidArgument with its
// output slots untouched and no allocation from `pool`.
void check_malformed(std::vector<Request> requests, const Pool& pool) {
  const auto before = pool.stats();
  for (Request& r : requests) {
    const std::vector<Tensor> slots = r.outputs;
    const Status status = r.run();
    expect(status.code() == StatusCode::kInvalidArgument,
           r.name + ": expected invalid_argument, got " + code_name(status.code()) + " (" + status.message() + ")");
    bool untouched = r.outputs.size() == slots.size();
    for (std::size_t i = 0; untouched && i < slots.size(); ++i) untouched = same_slot(r.outputs[i], slots[i]);
    expect(untouched, r.name + ": a failed request changed an output slot");
  }
  const auto after = pool.stats();
  expect(after.allocation_calls == before.allocation_calls && after.hits == before.hits,
         "malformed requests allocated from the pool (" + std::to_string(after.allocation_calls - before.allocation_calls) +
             " calls, " + std::to_string(after.hits - before.hits) + " cache hits)");
  std::cout << requests.size() << " malformed requests rejected before allocation\n";
}

// ---------------------------------------------------------------- device suite
struct Case {
  std::string name;
  std::function<Request()> build;
  std::vector<std::uint32_t> known;  // expected output words, when pinned
};

std::vector<float> ramp(std::size_t n, float scale, float offset = 0.F) {
  std::vector<float> v(n);
  for (std::size_t i = 0; i < n; ++i) v[i] = std::sin(0.37F * static_cast<float>(i) + offset) * scale;
  return v;
}

std::vector<std::uint32_t> words_of(const std::vector<float>& v) {
  std::vector<std::uint32_t> w(v.size());
  std::memcpy(w.data(), v.data(), v.size() * sizeof(float));
  return w;
}

std::vector<Case> suite() {
  std::vector<Case> cases;
  auto primitive = [](OpDesc op, std::vector<Tensor> inputs) {
    Request r{"", BackendOpClass::kPrimitive, op, std::move(inputs), {Tensor{}}};
    return r;
  };
  auto f32 = [](Shape shape, float scale, float offset = 0.F) {
    return upload(DType::kFloat32, shape, ramp(static_cast<std::size_t>(numel(shape)), scale, offset));
  };
  cases.push_back({"matmul 2x2 known answer", [=] {
                     return primitive(OpDesc{OpKind::kMatmul},
                                      {upload(DType::kFloat32, {2, 2}, std::vector<float>{1, 2, 3, 4}),
                                       upload(DType::kFloat32, {2, 2}, std::vector<float>{5, 6, 7, 8})});
                   },
                   words_of({19, 22, 43, 50})});
  cases.push_back({"row sums known answer", [=] {
                     OpDesc op{OpKind::kSum};
                     op.axis = 1;
                     return primitive(op, {upload(DType::kFloat32, {2, 3}, std::vector<float>{1, 2, 3, 4, 5, 6})});
                   },
                   words_of({6, 15})});
  std::vector<float> iota(24);
  for (int i = 0; i < 24; ++i) iota[static_cast<std::size_t>(i)] = static_cast<float>(i);
  const std::array<std::pair<OpKind, std::vector<float>>, 3> multi{
      {{OpKind::kSum, {60, 92, 124}}, {OpKind::kMax, {15, 19, 23}}, {OpKind::kMean, {7.5F, 11.5F, 15.5F}}}};
  for (const auto& [kind, expected] : multi)
    cases.push_back({"multi-axis (2, 0) known answer", [=, kind = kind] {
                       OpDesc op{kind};
                       op.reduction_axes = Shape{2, 0};
                       return primitive(op, {upload(DType::kFloat32, {2, 3, 4}, iota)});
                     },
                     words_of(expected)});
  cases.push_back({"fill float32", [] {
                     Request r{"", BackendOpClass::kPrimitive, OpDesc{OpKind::kFill}, {},
                               {Tensor{DType::kFloat32, {5, 7}, {7, 1}, {"hip", 0}, nullptr, 0}}};
                     r.op.scalar_value = -1.25;
                     return r;
                   },
                   std::vector<std::uint32_t>(35, 0xBFA00000U)});
  cases.push_back({"matmul 33x20x17", [=] { return primitive(OpDesc{OpKind::kMatmul}, {f32({33, 20}, 1.F), f32({20, 17}, 1.F, 1.F)}); }, {}});
  cases.push_back({"matmul 1000x1000x1000", [=] {
                     return primitive(OpDesc{OpKind::kMatmul}, {f32({1000, 1000}, 1.F), f32({1000, 1000}, 1.F, .5F)});
                   },
                   {}});
  cases.push_back({"batched matmul broadcast", [=] {
                     return primitive(OpDesc{OpKind::kMatmul}, {f32({2, 1, 8, 12}, 1.F), f32({3, 12, 5}, 1.F, 2.F)});
                   },
                   {}});
  cases.push_back({"linear with bias", [=] {
                     return primitive(OpDesc{OpKind::kLinear}, {f32({6, 16}, 1.F), f32({10, 16}, .5F, 1.F), f32({10}, .1F)});
                   },
                   {}});
  for (const OpKind kind : {OpKind::kSum, OpKind::kMax, OpKind::kMean, OpKind::kMin, OpKind::kArgmax})
    cases.push_back({"reduce rows", [=] {
                       OpDesc op{kind};
                       op.axis = -1;
                       if (kind == OpKind::kMin || kind == OpKind::kArgmax) op.reduction_axes = Shape{1};
                       return primitive(op, {f32({7, 3000}, 3.F)});
                     },
                     {}});
  cases.push_back({"full-tensor sum (one launch, static scratch)", [=] {
                     OpDesc op{OpKind::kSum};
                     op.reduction_axes = Shape{0, 1};
                     return primitive(op, {f32({4, 500000}, 1.F)});
                   },
                   {}});
  cases.push_back({"int32 row sums", [] {
                     std::vector<std::int32_t> v(4 * 1000);
                     for (std::size_t i = 0; i < v.size(); ++i) v[i] = static_cast<std::int32_t>(i * 2654435761U);
                     OpDesc op{OpKind::kSum};
                     op.axis = 1;
                     Request r{"", BackendOpClass::kPrimitive, op, {upload(DType::kInt32, {4, 1000}, v)}, {Tensor{}}};
                     return r;
                   },
                   {}});
  for (const OpKind kind : {OpKind::kSoftmax, OpKind::kRmsNorm, OpKind::kLayerNorm})
    cases.push_back({"row normalisation", [=] {
                       OpDesc op{kind};
                       op.axis = 1;
                       return primitive(op, {f32({5, 4096}, 3.F)});
                     },
                     {}});
  cases.push_back({"affine layernorm", [=] {
                     OpDesc op{OpKind::kAffineLayerNorm};
                     op.axis = -1;
                     op.has_weight = op.has_bias = true;
                     return primitive(op, {f32({3, 257}, 2.F), f32({257}, .5F, 1.F), f32({257}, .1F, 2.F)});
                   },
                   {}});
  for (const OpKind kind : {OpKind::kExp, OpKind::kGelu, OpKind::kSilu})
    cases.push_back({"elementwise", [=] { return primitive(OpDesc{kind}, {f32({300}, 4.F)}); }, {}});
  for (const OpKind kind : {OpKind::kAdd, OpKind::kSubtract, OpKind::kMultiply, OpKind::kDivide})
    cases.push_back({"broadcast arithmetic", [=] { return primitive(OpDesc{kind}, {f32({4, 1, 6}, 2.F), f32({5, 1}, 2.F, 1.F)}); },
                     {}});
  cases.push_back({"fused attention (causal)", [=] {
                     OpDesc op{OpKind::kAttention};
                     op.causal = true;
                     return primitive(op, {f32({2, 40, 64}, 1.F), f32({2, 70, 64}, 1.F, 1.F), f32({2, 70, 64}, 1.F, 2.F)});
                   },
                   {}});
  return cases;
}

void run_suite() {
  std::vector<Case> cases = suite();
  // Unpooled reference results.
  std::vector<std::vector<std::uint32_t>> expected;
  for (Case& c : cases) {
    Request r = c.build();
    const Status s = r.run();
    expect(s.ok(), c.name + ": " + s.message());
    expected.push_back(s.ok() ? download_words(r.outputs[0]) : std::vector<std::uint32_t>{});
    if (!c.known.empty()) expect(expected.back() == c.known, c.name + ": result differs from the known answer");
  }
  // The same requests twice inside a bounded pool: bit-identical results.
  constexpr std::size_t kMaxBytes = 64 << 20, kMaxBlocks = 64;
  Pool pool(kMaxBytes, kMaxBlocks, nullptr);
  pool.enter();
  for (int round = 0; round < 2; ++round) {
    for (std::size_t i = 0; i < cases.size(); ++i) {
      Request r = cases[i].build();
      const Status s = r.run();
      expect(s.ok(), cases[i].name + " (pooled): " + s.message());
      if (s.ok()) expect(download_words(r.outputs[0]) == expected[i], cases[i].name + ": pooled result differs");
    }
  }
  const auto stats = pool.stats();
  expect(stats.hits > 0, "the bounded pool reused no block");
  expect(stats.peak_cached_bytes <= kMaxBytes && stats.cached_blocks <= kMaxBlocks, "the pool exceeded its bounds");
  expect(pool.exit(), "pool exit failed");
  const auto closed = pool.stats();
  expect(closed.cached_bytes == 0 && closed.in_use_bytes == 0, "the pool held memory after exit");
  std::cout << cases.size() << " primitive requests matched inside a bounded pool (" << stats.hits << " hits, "
            << stats.misses << " misses)\n";
}

}  // namespace

int main() {
  try {
    const bool device = hip::available();
    if (!device) {
      // Buffers from a pool over host memory: validation never reaches a device.
      const tcx_hip_pool_runtime_t host{host_allocate, host_free, host_clear};
      Pool pool(1 << 20, 64, &host);
      pool.enter();
      {
        const Tensor x = make(DType::kFloat32, {3}), y = make(DType::kFloat32, {3});
        const Tensor xi = make(DType::kInt32, {3}), empty = make(DType::kFloat32, {0});
        const Tensor slot = make(DType::kFloat32, {3});
        check_malformed(malformed(x, y, xi, empty, slot), pool);
        // A well-formed request is only stopped by the missing device.
        Request good{"add", BackendOpClass::kPrimitive, OpDesc{OpKind::kAdd}, {x, y}, {slot}};
        const Status status = good.run();
        expect(status.code() == StatusCode::kUnavailable, std::string("well-formed add without a device: ") +
                                                                code_name(status.code()) + " " + status.message());
        expect(same_slot(good.outputs[0], slot), "a request without a device changed its output slot");
      }
      expect(pool.exit(), "host pool exit failed");
      if (failures) {
        std::cerr << failures << " contract failures\n";
        return 1;
      }
      if (std::getenv("TENSORCX_REQUIRE_HIP")) {
        std::cerr << "TENSORCX_REQUIRE_HIP is set but no HIP device is usable\n";
        return 1;
      }
      std::cout << "HIP device unavailable; metadata validation passed\n";
      return 77;
    }
    {
      // Device tensors, counted against a bounded pool with the HIP runtime.
      Pool pool(1 << 20, 64, nullptr);
      pool.enter();
      {
        const Tensor x = upload(DType::kFloat32, {3}, std::vector<float>{1, 2, 3});
        const Tensor y = upload(DType::kFloat32, {3}, std::vector<float>{10, 20, 30});
        const Tensor xi = upload(DType::kInt32, {3}, std::vector<std::int32_t>{1, 2, 3});
        const Tensor empty = make(DType::kFloat32, {0});
        const Tensor slot = upload(DType::kFloat32, {3}, std::vector<float>{-1, -1, -1});
        check_malformed(malformed(x, y, xi, empty, slot), pool);
        expect(download_floats(slot) == std::vector<float>({-1, -1, -1}), "a failed request wrote into the slot");
        Request good{"add", BackendOpClass::kPrimitive, OpDesc{OpKind::kAdd}, {x, y}, {slot}};
        const Status status = good.run();
        expect(status.ok(), "well-formed add: " + status.message());
        expect(status.ok() && good.outputs[0].buffer != slot.buffer &&
                   download_floats(good.outputs[0]) == std::vector<float>({11, 22, 33}),
               "well-formed add did not publish a fresh result");
      }
      expect(pool.exit(), "device pool exit failed");
    }
    run_suite();
  } catch (const std::exception& error) {
    std::cerr << "contract test error: " << error.what() << '\n';
    return 1;
  }
  if (failures) {
    std::cerr << failures << " contract failures\n";
    return 1;
  }
  std::cout << "HIP backend contract passed\n";
  return 0;
}
