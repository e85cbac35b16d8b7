// The MI355X hip device behind tensor.cx's backend execution ABI.
//
// HipBackend fills the device slot the reference's CUDA prototype occupies
// (reference backends/cuda/cuda_backend.h:31-49): it implements
// Backend::execute(const BackendExecution&) (core/backend.h:67-73) with the
// same contract: validate before allocating, allocate fresh result buffers,
// complete synchronously, publish outputs only on success, never throw across
// the boundary. All device work goes through the C ABI in tensorcx_hip.h.
#pragma once

#include <atomic>
#include <cstddef>
#include <memory>
#include <string>

#include "tensorcx/core/backend.h"
#include "tensorcx/core/expected.h"
#include "tensorcx_hip.h"

namespace tensorcx::hip {

// Device memory of a hip tensor. Owned memory returns to its pool (or is
// freed) when the last tensor referring to it goes away; borrowed memory
// (another framework's, through DLPack) releases its external owner instead.
// Mirrors CudaBuffer (reference backends/cuda/cuda_buffer.h:22-42).
class HipBuffer final : public Buffer {
 public:
  static Expected<std::shared_ptr<HipBuffer>> create(std::size_t bytes);
  // Wraps `bytes` of device-0 memory at `data`, kept alive by `owner`, after
  // tcx_hip_borrow_check (CudaBuffer::borrow, cuda_backend.cpp:106-144).
  static Expected<std::shared_ptr<HipBuffer>> borrow(void* data, std::size_t bytes, std::shared_ptr<void> owner);
  ~HipBuffer() override;
  HipBuffer(const HipBuffer&) = delete;
  HipBuffer& operator=(const HipBuffer&) = delete;
  std::size_t nbytes() const override { return bytes_; }
  // Device memory is one address space: identity is the address range, so
  // independently wrapped views of the same memory relate as the reference's
  // CudaBuffer::storage_relation does (cuda_backend.cpp:87-98).
  StorageIdentity storage_identity() const override;
  void* data() const { return data_; }
  bool borrowed() const { return external_ != nullptr; }
  // Storage seen by another framework never returns to a pool cache.
  void mark_exported() { exported_.store(true, std::memory_order_relaxed); }

 private:
  HipBuffer() = default;
  void* data_{nullptr};
  std::size_t bytes_{0};
  tcx_hip_pool_t* owner_{nullptr};
  std::shared_ptr<void> external_;
  std::atomic<bool> exported_{false};
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
// A contiguous hip tensor over another framework's device-0 memory, kept
// alive by `owner` (the CUDA import of bindings/dlpack.cpp:142-153).
Expected<Tensor> borrow(void* data, DType dtype, Shape shape, std::shared_ptr<void> owner);
// The device address of a contiguous hip tensor handed to another framework;
// its storage is marked exported (bindings/dlpack.cpp:193-207).
Expected<void*> export_storage(const Tensor& tensor);

// Built-in kernels reachable through BackendOpClass::kKernel with
// KernelArtifactKind::kStaticLibrary and artifact kStaticArtifact:
//   "linear_bias_act": kernel_arguments = x, weight, bias, uint32 activation;
//                      outputs[0] = preallocated act(x @ weight^T + bias)
//   "bias_act":        kernel_arguments = x, bias, uint32 activation;
//                      outputs[0] = preallocated act(x + bias)
inline constexpr const char* kStaticArtifact = "tensorcx_hip";

}  // namespace tensorcx::hip
