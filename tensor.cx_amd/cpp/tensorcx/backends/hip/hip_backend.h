// The MI355X hip device behind tensor.cx's backend execution ABI.
//
// HipBackend fills the device slot the reference's CUDA prototype occupies
// (reference backends/cuda/cuda_backend.h:31-49): it implements
// Backend::execute(const BackendExecution&) (core/backend.h:67-73) with the
// same contract: validate before allocating, allocate fresh result buffers,
// complete synchronously, publish outputs only on success, never throw across
// the boundary. All device work goes through the C ABI in tensorcx_hip.h.
#pragma once

#include <cstddef>
#include <memory>
#include <string>

#include "tensorcx/core/backend.h"
#include "tensorcx/core/expected.h"
#include "tensorcx_hip.h"

namespace tensorcx::hip {

// Device memory owned by a hip tensor; returned to its pool (or freed) when
// the last tensor referring to it goes away.
class HipBuffer final : public Buffer {
 public:
  static Expected<std::shared_ptr<HipBuffer>> create(std::size_t bytes);
  ~HipBuffer() override;
  HipBuffer(const HipBuffer&) = delete;
  HipBuffer& operator=(const HipBuffer&) = delete;
  std::size_t nbytes() const override { return bytes_; }
  void* data() const { return data_; }

 private:
  HipBuffer() = default;
  void* data_{nullptr};
  std::size_t bytes_{0};
  tcx_hip_pool_t* owner_{nullptr};
};

class HipBackend final : public Backend {
 public:
  std::string name() const override { return "hip"; }
  Status execute(const BackendExecution& execution) override;
};

// Free functions mirroring the CUDA prototype's (cuda_backend.h:37-49).
bool available();
Expected<std::string> device_name();
struct DeviceInfo {
  std::string name, arch;
  int compute_units{0}, clock_khz{0}, memory_clock_khz{0}, memory_bus_width{0}, l2_bytes{0};
  int runtime_version{0}, driver_version{0};
  std::size_t free_bytes{0}, total_bytes{0};
};
Expected<DeviceInfo> device_info();
// Uninitialised contiguous device tensor {"hip", 0}.
Expected<Tensor> empty(Shape shape, DType dtype);
// Host <-> device placement (cuda::from_cpu / to_cpu, cuda_backend.cpp:215-264):
// `host` holds numel(shape) contiguous elements of `dtype`.
Expected<Tensor> from_host(const void* host, DType dtype, Shape shape);
Status to_host(const Tensor& tensor, void* host, std::size_t bytes);
// A new device tensor with the same contents (independent storage).
Expected<Tensor> clone(const Tensor& tensor);

// Built-in kernels reachable through BackendOpClass::kKernel with
// KernelArtifactKind::kStaticLibrary and artifact kStaticArtifact:
//   "linear_bias_act": kernel_arguments = x, weight, bias, uint32 activation;
//                      outputs[0] = preallocated act(x @ weight^T + bias)
//   "bias_act":        kernel_arguments = x, bias, uint32 activation;
//                      outputs[0] = preallocated act(x + bias)
inline constexpr const char* kStaticArtifact = "tensorcx_hip";

}  // namespace tensorcx::hip
