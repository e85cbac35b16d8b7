// The DLPack exchange ABI, version 1.0: the C structs a DLPack capsule
// carries between frameworks. Declared here from the published DLPack
// specification (https://dmlc.github.io/dlpack/latest/c_api.html); member
// order, widths and enumerator values are fixed by that specification, since
// every producer and consumer reads the same memory. Only what this module
// uses is declared. (The reference vendors the upstream header,
// third_party/dlpack/dlpack.h.)
#pragma once

#include <cstdint>

namespace tcx_bind::dl {

struct PackVersion {
  std::uint32_t major;
  std::uint32_t minor;
};

// DLDeviceType values used here.
enum DeviceType : std::int32_t {
  kCPU = 1,
  kCUDA = 2,
  kROCM = 10,
};

struct Device {
  std::int32_t device_type;  // a DeviceType value
  std::int32_t device_id;
};

// DLDataTypeCode values used here.
enum TypeCode : std::uint8_t {
  kInt = 0,
  kFloat = 2,
  kBool = 6,
};

struct DataType {
  std::uint8_t code;
  std::uint8_t bits;
  std::uint16_t lanes;
};

struct Tensor {
  void* data;
  Device device;
  std::int32_t ndim;
  DataType dtype;
  std::int64_t* shape;
  std::int64_t* strides;  // in elements; may be null for a compact row-major tensor
  std::uint64_t byte_offset;
};

// The capsule payload named "dltensor" (no version, no flags).
struct ManagedTensor {
  Tensor dl_tensor;
  void* manager_ctx;
  void (*deleter)(ManagedTensor* self);
};

inline constexpr std::uint64_t kFlagReadOnly = 1ULL << 0;
inline constexpr std::uint64_t kFlagIsCopied = 1ULL << 1;

// The capsule payload named "dltensor_versioned". Only the prefix up to and
// including `deleter` is stable across major versions.
struct ManagedTensorVersioned {
  PackVersion version;
  void* manager_ctx;
  void (*deleter)(ManagedTensorVersioned* self);
  std::uint64_t flags;
  Tensor dl_tensor;
};

}  // namespace tcx_bind::dl
