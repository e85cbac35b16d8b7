#include "tensorcx/core/backend.h"

#include <exception>
#include <string>

namespace tensorcx {
namespace {

Status invalid(std::string message) { return Status(StatusCode::kInvalidArgument, std::move(message)); }

// Concrete metadata: a device, offset 0, contiguous strides and a buffer.
Status check_concrete(const Tensor& t, const std::string& what) {
  if (t.device.type.empty()) return invalid(what + " requires a device type");
  if (t.device.index < 0) return invalid(what + " requires a non-negative device index");
  if (t.offset != 0) return invalid(what + " requires offset 0");
  try {
    (void)numel(t.shape);
    if (t.strides != contiguous_strides(t.shape)) return invalid(what + " must be contiguous");
  } catch (const std::exception& error) {
    return invalid(error.what());
  }
  if (!t.buffer) return invalid(what + " requires a buffer");
  return Status::Ok();
}

}  // namespace

Status validate_fill_output_descriptor(const Tensor& output, std::string_view expected_device_type) {
  if (expected_device_type.empty()) {
    if (output.device.type.empty()) return invalid("fill output descriptor requires a device type");
  } else if (output.device.type != expected_device_type) {
    return invalid("fill output descriptor device type does not match backend");
  }
  if (output.device.index < 0) return invalid("fill output descriptor requires a non-negative device index");
  if (output.offset != 0) return invalid("fill output descriptor requires offset 0");
  try {
    (void)numel(output.shape);
    if (output.strides != contiguous_strides(output.shape))
      return invalid("fill output descriptor must be contiguous");
  } catch (const std::exception& error) {
    return invalid(error.what());
  }
  if (output.buffer) return invalid("fill output descriptor must not include a buffer");
  return Status::Ok();
}

Status validate_primitive_execution_contract(const BackendExecution& e, std::string_view fill_device_type) {
  if (e.op_class != BackendOpClass::kPrimitive)
    return invalid("primitive backend execution requires primitive op class");
  if (e.launch || e.compilation_target)
    return invalid("primitive backend execution cannot include kernel launch metadata");
  if (!e.kernel_arguments.empty()) return invalid("primitive backend execution cannot include kernel arguments");
  const auto schema = primitive_op_schema(e.op.kind);
  if (!schema) return invalid("primitive operation is not expressible by BackendExecution");
  const bool count_ok = schema->variadic_inputs ? e.inputs.size() >= schema->input_count
                                                : e.inputs.size() == schema->input_count;
  if (!count_ok) return invalid("primitive backend execution input count mismatch");
  if (e.outputs.size() != schema->output_count) return invalid("primitive backend execution output count mismatch");
  if (e.op.kind == OpKind::kFill) return validate_fill_output_descriptor(e.outputs[0], fill_device_type);
  return Status::Ok();
}

Status validate_kernel_execution_contract(const BackendExecution& e) {
  if (e.op_class != BackendOpClass::kKernel) return invalid("kernel backend execution requires kernel op class");
  if (!e.inputs.empty()) return invalid("kernel backend execution uses kernel arguments instead of primitive inputs");
  if (e.outputs.empty()) return invalid("kernel backend execution requires output metadata");
  for (const Tensor& output : e.outputs)
    if (Status s = check_concrete(output, "kernel output metadata"); !s.ok()) return s;
  if (!e.launch) return invalid("kernel backend execution requires launch metadata");
  const LaunchConfig& l = *e.launch;
  if (!l.grid_x || !l.grid_y || !l.grid_z || !l.threads_per_group_x || !l.threads_per_group_y ||
      !l.threads_per_group_z)
    return invalid("kernel launch dimensions must be non-zero");
  if (!e.compilation_target) return invalid("kernel backend execution requires a compilation target");
  if (e.compilation_target->entry_point.empty()) return invalid("kernel compilation target requires an entry point");
  if (e.compilation_target->artifact_kind == KernelArtifactKind::kNone)
    return invalid("kernel compilation target requires an artifact kind");
  if (e.compilation_target->artifact.empty()) return invalid("kernel compilation target requires an artifact");
  for (const KernelArgument& argument : e.kernel_arguments) {
    if (argument.kind != KernelArgumentKind::kTensor) continue;
    if (!argument.tensor) return invalid("kernel tensor argument requires tensor metadata");
    if (Status s = check_concrete(*argument.tensor, "kernel tensor argument"); !s.ok()) return s;
  }
  return Status::Ok();
}

}  // namespace tensorcx
