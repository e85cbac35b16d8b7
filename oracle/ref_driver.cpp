// Test infrastructure only. A C entry point over the reference's own CPU
// backend (tensorcx::cpu::CpuBackend::execute, cpu_backend.cpp:246-366), built
// by oracle/Makefile from the reference sources where they lie under
// /root/reference into oracle/_ref/libtcxref.so. It is used to write golden
// vectors, to check the oracle restatement, and as the CPU baseline.
//
// Operation kinds and dtypes are passed as the reference's own enum values
// (core/operation.h:12-53, core/dtype.h:8-12).

#include <array>
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "tensorcx/backends/cpu/cpu_backend.h"
#include "tensorcx/core/backend.h"

namespace {

struct Result {
  int status{0};
  std::string message;
  tensorcx::Tensor tensor;
  std::vector<tensorcx::Tensor> extra;
};

thread_local Result last;

// Attributes beyond the common ones, set by tcxref_set_attributes for the next
// tcxref_execute call on this thread (core/operation.h OpDesc fields).
struct Attributes {
  bool set{false};
  bool causal{false};
  bool has_scale{false};
  double scale{1.0};
  tensorcx::Shape attention_shape{};
  std::int64_t k{0};
  bool largest{true};
  bool sorted{true};
  double scalar{0.0};
  bool layout{false};
  tensorcx::Shape axes{}, starts{}, steps{}, lengths{};
  int target_dtype{0};
  bool scalar_left{false};
};

thread_local Attributes pending;

tensorcx::cpu::CpuTensor make_input(int dtype, int rank, const std::int64_t* shape,
                                    const void* data) {
  tensorcx::Shape s(shape, shape + rank);
  const auto dt = static_cast<tensorcx::DType>(dtype);
  tensorcx::cpu::CpuTensor t(dt, s);
  const auto bytes = static_cast<std::size_t>(t.size()) * tensorcx::dtype_size(dt);
  if (bytes) std::memcpy(t.mutable_data(), data, bytes);
  return t;
}

}  // namespace

extern "C" {

// Runs one primitive. Input tensor i has dtype dtypes[i], rank ranks[i] and its
// shape at shapes[offset_i ...] where offset_i is the running sum of ranks.
// Returns the reference StatusCode value; the result stays available to
// tcxref_result_* until the next call on this thread.
int tcxref_execute(int kind, std::int64_t axis, double epsilon, int has_axes,
                   const std::int64_t* axes, int n_axes, int has_weight, int has_bias,
                   int n_inputs, const int* dtypes, const int* ranks, const std::int64_t* shapes,
                   const void* const* datas, int n_outputs) {
  last = Result{};
  try {
    std::vector<tensorcx::cpu::CpuTensor> inputs;
    std::vector<tensorcx::Tensor> core_inputs;
    int shape_offset = 0;
    for (int i = 0; i < n_inputs; ++i) {
      inputs.push_back(make_input(dtypes[i], ranks[i], shapes + shape_offset, datas[i]));
      shape_offset += ranks[i];
    }
    for (const auto& t : inputs) core_inputs.push_back(tensorcx::cpu::to_core_tensor(t));
    tensorcx::OpDesc op{static_cast<tensorcx::OpKind>(kind)};
    op.axis = axis;
    op.epsilon = epsilon;
    if (has_axes) op.reduction_axes = tensorcx::Shape(axes, axes + n_axes);
    op.has_weight = has_weight != 0;
    op.has_bias = has_bias != 0;
    if (pending.set) {
      op.causal = pending.causal;
      if (pending.has_scale) op.attention_scale = pending.scale;
      op.attention_shape = pending.attention_shape;
      op.k = pending.k;
      op.largest = pending.largest;
      op.sorted = pending.sorted;
      op.scalar_value = pending.scalar;
      if (pending.layout) {
        op.axes = pending.axes;
        op.slice_starts = pending.starts;
        op.slice_steps = pending.steps;
        op.slice_shape = pending.lengths;
        op.target_dtype = static_cast<tensorcx::DType>(pending.target_dtype);
        op.scalar_left = pending.scalar_left;
      }
      pending = Attributes{};
    }
    std::vector<tensorcx::Tensor> outputs(static_cast<std::size_t>(n_outputs));
    tensorcx::BackendExecution e{tensorcx::BackendOpClass::kPrimitive, op, core_inputs, outputs,
                                 std::nullopt, std::nullopt, {}};
    tensorcx::cpu::CpuBackend backend;
    const auto status = backend.execute(e);
    last.status = static_cast<int>(status.code());
    last.message = status.message();
    if (status.ok()) {
      last.tensor = outputs[0];
      for (std::size_t i = 1; i < outputs.size(); ++i) last.extra.push_back(outputs[i]);
    }
  } catch (const std::exception& error) {
    last.status = 3;
    last.message = error.what();
  }
  return last.status;
}

// Sets causal / attention_scale / attention_shape / k / largest / sorted /
// scalar_value for the next tcxref_execute on this thread.
void tcxref_set_attributes(int causal, int has_scale, double scale, int attention_rank,
                           const std::int64_t* attention_shape, std::int64_t k, int largest, int sorted,
                           double scalar) {
  pending = Attributes{};
  pending.set = true;
  pending.causal = causal != 0;
  pending.has_scale = has_scale != 0;
  pending.scale = scale;
  pending.attention_shape = tensorcx::Shape(attention_shape, attention_shape + attention_rank);
  pending.k = k;
  pending.largest = largest != 0;
  pending.sorted = sorted != 0;
  pending.scalar = scalar;
}

// Adds transpose axes, slice starts/steps/lengths (each `rank` long, the
// ones not used may be NULL), the cast target dtype and the scalar operand
// side to the attributes of the next tcxref_execute (call after
// tcxref_set_attributes).
void tcxref_set_layout(int axes_rank, const std::int64_t* axes, int slice_rank, const std::int64_t* starts,
                       const std::int64_t* steps, const std::int64_t* lengths, int target_dtype, int scalar_left) {
  pending.set = true;
  pending.layout = true;
  pending.axes = axes ? tensorcx::Shape(axes, axes + axes_rank) : tensorcx::Shape{};
  pending.starts = starts ? tensorcx::Shape(starts, starts + slice_rank) : tensorcx::Shape{};
  pending.steps = steps ? tensorcx::Shape(steps, steps + slice_rank) : tensorcx::Shape{};
  pending.lengths = lengths ? tensorcx::Shape(lengths, lengths + slice_rank) : tensorcx::Shape{};
  pending.target_dtype = target_dtype;
  pending.scalar_left = scalar_left != 0;
}

const char* tcxref_message() { return last.message.c_str(); }

// Output `index` (0 = first output): dtype, rank and up to 512 dims.
int tcxref_result_info(int index, int* dtype, int* rank, std::int64_t* shape) {
  const tensorcx::Tensor* t = index == 0 ? &last.tensor
                              : static_cast<std::size_t>(index) <= last.extra.size()
                                  ? &last.extra[static_cast<std::size_t>(index - 1)]
                                  : nullptr;
  if (!t || !t->buffer || t->shape.size() > 512) return -1;
  *dtype = static_cast<int>(t->dtype);
  *rank = static_cast<int>(t->shape.size());
  for (std::size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
  return 0;
}

int tcxref_result_copy(int index, void* dst, std::size_t bytes) {
  const tensorcx::Tensor* t = index == 0 ? &last.tensor
                              : static_cast<std::size_t>(index) <= last.extra.size()
                                  ? &last.extra[static_cast<std::size_t>(index - 1)]
                                  : nullptr;
  if (!t || !t->buffer) return -1;
  const auto cpu = tensorcx::cpu::from_core_tensor(*t);
  const auto nbytes = static_cast<std::size_t>(cpu.size()) * tensorcx::dtype_size(cpu.dtype());
  if (bytes != nbytes) return -2;
  if (nbytes) std::memcpy(dst, cpu.data(), nbytes);
  return 0;
}

// The reference matmul (cpu_backend.cpp:1251-1276) on contiguous row-major
// [m,k]x[k,n] float32, for timing the reference algorithm on a row slab: it
// runs the reference on rows [0, rows) only by passing an [rows, k] operand.
int tcxref_matmul_rows(const float* a, const float* b, float* out, std::int64_t rows,
                       std::int64_t n, std::int64_t k) {
  const std::array<std::int64_t, 4> shapes{rows, k, k, n};
  const std::array<int, 2> dtypes{0, 0}, ranks{2, 2};
  const std::array<const void*, 2> datas{a, b};
  const int status = tcxref_execute(3, 0, 1e-5, 0, nullptr, 0, 0, 0, 2, dtypes.data(),
                                    ranks.data(), shapes.data(), datas.data(), 1);
  if (status != 0) return status;
  return tcxref_result_copy(0, out, static_cast<std::size_t>(rows * n) * sizeof(float));
}

}  // extern "C"
