#include "tensorcx/core/shape.h"

#include <algorithm>
#include <limits>
#include <stdexcept>

namespace tensorcx {
namespace {

Dim checked_product(Dim a, Dim b, const char* what) {
  if (a != 0 && b > std::numeric_limits<Dim>::max() / a) throw std::invalid_argument(what);
  return a * b;
}

void require_non_negative(Dim d) {
  if (d < 0) throw std::invalid_argument("shape dimensions must be non-negative");
}

}  // namespace

std::int64_t numel(const Shape& shape) {
  Dim total = 1;
  for (const Dim d : shape) {
    require_non_negative(d);
    total = checked_product(total, d, "shape size overflow");
  }
  return total;
}

Shape contiguous_strides(const Shape& shape) {
  Shape strides(shape.size(), 1);
  Dim running = 1;
  for (std::size_t i = shape.size(); i-- > 0;) {
    require_non_negative(shape[i]);
    strides[i] = running;
    running = checked_product(running, shape[i], "shape stride overflow");
  }
  return strides;
}

BroadcastPlan make_broadcast_plan(const Shape& lhs, const Shape& rhs) {
  (void)numel(lhs);
  (void)numel(rhs);
  const Shape ls = contiguous_strides(lhs), rs = contiguous_strides(rhs);
  const std::size_t rank = std::max(lhs.size(), rhs.size());
  BroadcastPlan plan{Shape(rank), Shape(rank, 0), Shape(rank, 0)};
  for (std::size_t axis = 0; axis < rank; ++axis) {
    const bool has_l = axis + lhs.size() >= rank, has_r = axis + rhs.size() >= rank;
    const std::size_t li = axis + lhs.size() - rank, ri = axis + rhs.size() - rank;
    const Dim l = has_l ? lhs[li] : 1, r = has_r ? rhs[ri] : 1;
    if (l != r && l != 1 && r != 1)
      throw std::invalid_argument("shape mismatch: tensor shapes are not broadcastable");
    plan.output_shape[axis] = l == 1 ? r : l;  // a zero extent against 1 stays 0
    if (has_l && l != 1) plan.lhs_strides[axis] = ls[li];
    if (has_r && r != 1) plan.rhs_strides[axis] = rs[ri];
  }
  (void)numel(plan.output_shape);
  (void)contiguous_strides(plan.output_shape);
  return plan;
}

MatmulPlan make_matmul_plan(const Shape& lhs, const Shape& rhs) {
  if (lhs.empty() || rhs.empty()) throw std::invalid_argument("matmul requires rank >= 1 tensors");
  (void)numel(lhs);
  (void)numel(rhs);
  const Shape ls = contiguous_strides(lhs), rs = contiguous_strides(rhs);
  const bool lhs_vector = lhs.size() == 1, rhs_vector = rhs.size() == 1;
  const Dim m = lhs_vector ? 1 : lhs[lhs.size() - 2];
  const Dim k = lhs.back();
  const Dim rk = rhs_vector ? rhs[0] : rhs[rhs.size() - 2];
  const Dim n = rhs_vector ? 1 : rhs.back();
  if (k != rk) throw std::invalid_argument("matmul shape mismatch: contracting dimensions differ");
  const std::size_t lb = lhs_vector ? 0 : lhs.size() - 2, rb = rhs_vector ? 0 : rhs.size() - 2;
  const std::size_t rank = std::max(lb, rb);
  MatmulPlan plan{{}, Shape(rank, 1), Shape(rank, 0), Shape(rank, 0), m, k, n};
  for (std::size_t axis = 0; axis < rank; ++axis) {
    const bool has_l = axis + lb >= rank, has_r = axis + rb >= rank;
    const std::size_t li = axis + lb - rank, ri = axis + rb - rank;
    const Dim l = has_l ? lhs[li] : 1, r = has_r ? rhs[ri] : 1;
    if (l != r && l != 1 && r != 1) throw std::invalid_argument("matmul batch dimensions cannot broadcast");
    plan.batch_shape[axis] = l == 1 ? r : l;
    if (has_l && l != 1) plan.lhs_batch_strides[axis] = ls[li];
    if (has_r && r != 1) plan.rhs_batch_strides[axis] = rs[ri];
  }
  plan.output_shape = plan.batch_shape;
  if (!lhs_vector) plan.output_shape.push_back(m);
  if (!rhs_vector) plan.output_shape.push_back(n);
  (void)numel(plan.output_shape);
  (void)contiguous_strides(plan.output_shape);
  return plan;
}

Dim matmul_batch_offset(Dim batch, const Shape& shape, const Shape& strides) {
  Dim offset = 0;
  for (std::size_t axis = shape.size(); axis-- > 0;) {
    offset += (batch % shape[axis]) * strides[axis];
    batch /= shape[axis];
  }
  return offset;
}

ReductionPlan make_reduction_plan(const Shape& input, const Shape& axes) {
  (void)numel(input);
  const Shape strides = contiguous_strides(input);
  const Dim rank = static_cast<Dim>(input.size());
  std::vector<bool> selected(input.size(), false);
  for (Dim axis : axes) {
    if (axis < 0) axis += rank;
    if (axis < 0 || axis >= rank) throw std::invalid_argument("reduction axis is out of range");
    if (selected[static_cast<std::size_t>(axis)]) throw std::invalid_argument("reduction axes must not repeat");
    selected[static_cast<std::size_t>(axis)] = true;
  }
  ReductionPlan plan;
  Shape reduced;
  for (std::size_t axis = 0; axis < input.size(); ++axis) {
    if (selected[axis]) continue;
    plan.output_shape.push_back(input[axis]);
    plan.index_metadata.push_back(input[axis]);
    plan.index_metadata.push_back(strides[axis]);
  }
  for (std::size_t axis = 0; axis < input.size(); ++axis) {
    if (!selected[axis]) continue;
    reduced.push_back(input[axis]);
    plan.index_metadata.push_back(input[axis]);
    plan.index_metadata.push_back(strides[axis]);
  }
  const Dim outputs = numel(plan.output_shape);
  (void)contiguous_strides(plan.output_shape);
  // A zero reduced extent gives an empty reduction; with no outputs a
  // non-empty reduction keeps size 1 so nothing is ever multiplied out.
  if (std::find(reduced.begin(), reduced.end(), 0) != reduced.end())
    plan.reduction_size = 0;
  else if (outputs != 0)
    plan.reduction_size = numel(reduced);
  return plan;
}

TransposePlan make_transpose_plan(const Shape& input, const Shape& axes) {
  (void)numel(input);
  const Shape strides = contiguous_strides(input);
  if (axes.size() != input.size()) throw std::invalid_argument("transpose axes must be a full permutation");
  const Dim rank = static_cast<Dim>(input.size());
  std::vector<bool> used(input.size(), false);
  TransposePlan plan{Shape(input.size()), Shape(input.size()), 0};
  for (std::size_t i = 0; i < axes.size(); ++i) {
    const Dim axis = axes[i] < 0 ? axes[i] + rank : axes[i];
    if (axis < 0 || axis >= rank) throw std::invalid_argument("transpose axis is out of range");
    if (used[static_cast<std::size_t>(axis)]) throw std::invalid_argument("transpose axes must not repeat");
    used[static_cast<std::size_t>(axis)] = true;
    plan.output_shape[i] = input[static_cast<std::size_t>(axis)];
    plan.input_strides[i] = strides[static_cast<std::size_t>(axis)];
  }
  (void)numel(plan.output_shape);
  return plan;
}

TransposePlan make_slice_plan(const Shape& input, const Shape& starts, const Shape& steps, const Shape& lengths) {
  (void)numel(input);
  const Shape strides = contiguous_strides(input);
  if (starts.size() != input.size() || steps.size() != input.size() || lengths.size() != input.size())
    throw std::invalid_argument("slice metadata must match input rank");
  const Dim total = numel(lengths);
  TransposePlan plan{lengths, Shape(input.size(), 0), 0};
  for (std::size_t a = 0; a < input.size(); ++a) {
    const Dim start = starts[a], step = steps[a], length = lengths[a];
    if (step == 0) throw std::invalid_argument("slice step cannot be zero");
    if (length == 0) continue;
    if (start < 0 || start >= input[a]) throw std::invalid_argument("slice start is out of bounds");
    if (length > 1) {
      // The last index start + step * (length - 1) must stay in [0, extent);
      // compared by division so the product cannot overflow.
      const bool past_end = step > 0 && step > (input[a] - 1 - start) / (length - 1);
      const bool before_start = step < 0 && step < -(start / (length - 1));
      if (past_end || before_start) throw std::invalid_argument("slice endpoint is out of bounds");
      if (total != 0) plan.input_strides[a] = step * strides[a];
    }
    if (total != 0) plan.offset += start * strides[a];
  }
  return plan;
}

ConcatPlan make_concat_plan(const std::vector<Shape>& inputs, Dim axis) {
  if (inputs.empty()) throw std::invalid_argument("concat requires at least one tensor");
  const Dim rank = static_cast<Dim>(inputs[0].size());
  if (axis < 0) axis += rank;
  if (axis < 0 || axis >= rank) throw std::invalid_argument("concat axis is out of range");
  const auto ax = static_cast<std::size_t>(axis);
  Shape output = inputs[0];
  output[ax] = 0;
  for (const Shape& shape : inputs) {
    (void)numel(shape);
    if (shape.size() != output.size()) throw std::invalid_argument("concat ranks must match");
    for (std::size_t i = 0; i < shape.size(); ++i)
      if (i != ax && shape[i] != output[i]) throw std::invalid_argument("concat non-axis dimensions must match");
    if (shape[ax] > std::numeric_limits<Dim>::max() - output[ax]) throw std::invalid_argument("concat dimension overflow");
    output[ax] += shape[ax];
  }
  (void)numel(output);
  return {output, ax, contiguous_strides(output)[ax]};
}

}  // namespace tensorcx
