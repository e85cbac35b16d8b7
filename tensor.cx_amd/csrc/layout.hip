// Data movement and conversion: strided gathers (kTranspose / kSlice), block
// copies (kConcat), kCast and the scalar arithmetic family (kNegate,
// k*Scalar). Semantics are the reference CPU backend's
// (backends/cpu/cpu_backend.cpp:801-930, plans in core/shape.cpp:87-200):
// movement is bit-preserving for 1- and 4-byte elements (NaN payloads and
// signed zeros included); float32 -> int32 truncates toward zero after every
// source was checked finite and inside [-2^31, 2^31); bool conversions test
// value != 0; float32 scalar arithmetic rounds the scalar to float32 once and
// each result once; int32 scalar arithmetic wraps in uint32.

#include "common.hpp"

namespace tcx {
namespace {

struct GatherMeta {
  std::int64_t shape[TCX_HIP_MAX_RANK];
  std::int64_t strides[TCX_HIP_MAX_RANK];
  std::int64_t offset;
  std::int32_t rank;
};

template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(const T* __restrict__ in, T* __restrict__ out, GatherMeta m,
                                                     std::int64_t n) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    std::int64_t rest = i, src = m.offset;
    for (int a = m.rank - 1; a >= 0; --a) {
      src += (rest % m.shape[a]) * m.strides[a];
      rest /= m.shape[a];
    }
    out[i] = in[src];
  }
}

template <typename T>
__global__ __launch_bounds__(256) void block_copy_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                         std::int64_t outer, std::int64_t block,
                                                         std::int64_t out_block, std::int64_t dst_offset) {
  const std::int64_t n = outer * block;
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[(i / block) * out_block + dst_offset + i % block] = in[i];
}

// float32 values a cast to int32 cannot represent: NaN, +-inf, outside
// [-2^31, 2^31) (cpu_backend.cpp:857-863).
__global__ __launch_bounds__(256) void cast_check_kernel(const float* __restrict__ in, std::int64_t n,
                                                         std::int32_t* __restrict__ flag) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = in[i];
    if (!__builtin_isfinite(v) || v < -2147483648.0F || v >= 2147483648.0F) *flag = 1;  // one value from all writers
  }
}

template <int kFrom, int kTo>
__global__ __launch_bounds__(256) void cast_kernel(const void* __restrict__ in, void* __restrict__ out,
                                                   std::int64_t n) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    if constexpr (kTo == TCX_BOOL || kFrom == TCX_BOOL) {
      bool v;
      if constexpr (kFrom == TCX_FLOAT32) v = static_cast<const float*>(in)[i] != 0.F;
      else if constexpr (kFrom == TCX_INT32) v = static_cast<const std::int32_t*>(in)[i] != 0;
      else v = static_cast<const std::uint8_t*>(in)[i] != 0;
      if constexpr (kTo == TCX_BOOL) static_cast<std::uint8_t*>(out)[i] = v ? 1 : 0;
      else if constexpr (kTo == TCX_FLOAT32) static_cast<float*>(out)[i] = v ? 1.F : 0.F;
      else static_cast<std::int32_t*>(out)[i] = v ? 1 : 0;
    } else if constexpr (kFrom == TCX_FLOAT32 && kTo == TCX_INT32) {
      static_cast<std::int32_t*>(out)[i] = static_cast<std::int32_t>(static_cast<const float*>(in)[i]);
    } else if constexpr (kFrom == TCX_INT32 && kTo == TCX_FLOAT32) {
      static_cast<float*>(out)[i] = static_cast<float>(static_cast<const std::int32_t*>(in)[i]);
    } else {  // same dtype: word copy
      static_cast<std::uint32_t*>(out)[i] = static_cast<const std::uint32_t*>(in)[i];
    }
  }
}

template <int kOp>
__global__ __launch_bounds__(256) void scalar_f32_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                         std::int64_t n, float scalar, int scalar_left) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = in[i];
    const float l = scalar_left ? scalar : v, r = scalar_left ? v : scalar;
    float y;
    if constexpr (kOp == TCX_SCALAR_NEGATE) y = -v;
    else if constexpr (kOp == TCX_SCALAR_ADD) y = l + r;
    else if constexpr (kOp == TCX_SCALAR_SUBTRACT) y = l - r;
    else if constexpr (kOp == TCX_SCALAR_MULTIPLY) y = l * r;
    else y = l / r;
    out[i] = y;
  }
}

template <int kOp>
__global__ __launch_bounds__(256) void scalar_i32_kernel(const std::uint32_t* __restrict__ in,
                                                         std::uint32_t* __restrict__ out, std::int64_t n,
                                                         std::uint32_t scalar, int scalar_left) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const std::uint32_t v = in[i];
    const std::uint32_t l = scalar_left ? scalar : v, r = scalar_left ? v : scalar;
    std::uint32_t y;
    if constexpr (kOp == TCX_SCALAR_NEGATE) y = 0U - v;
    else if constexpr (kOp == TCX_SCALAR_ADD) y = l + r;
    else if constexpr (kOp == TCX_SCALAR_SUBTRACT) y = l - r;
    else y = l * r;
    out[i] = y;
  }
}

dim3 grid_of(std::int64_t n) { return dim3(grid_for(n, 256, 256 * 32)); }

int check_bytes(int elem_bytes) {
  if (elem_bytes != 1 && elem_bytes != 4) return fail(TCX_INVALID_ARGUMENT, "element size must be 1 or 4 bytes");
  return TCX_OK;
}

template <int kFrom>
void launch_cast_from(int to, const void* in, void* out, std::int64_t n, hipStream_t s) {
  if (to == TCX_FLOAT32) hipLaunchKernelGGL((cast_kernel<kFrom, TCX_FLOAT32>), grid_of(n), dim3(256), 0, s, in, out, n);
  else if (to == TCX_INT32) hipLaunchKernelGGL((cast_kernel<kFrom, TCX_INT32>), grid_of(n), dim3(256), 0, s, in, out, n);
  else hipLaunchKernelGGL((cast_kernel<kFrom, TCX_BOOL>), grid_of(n), dim3(256), 0, s, in, out, n);
}

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_gather_strided(int elem_bytes, const void* in, void* out, int32_t rank, const int64_t* out_shape,
                           const int64_t* in_strides, int64_t offset, tcx_stream_t stream) {
  using namespace tcx;
  if (int rc = check_bytes(elem_bytes); rc != TCX_OK) return rc;
  if (rank < 0 || rank > TCX_HIP_MAX_RANK) return fail(TCX_INVALID_ARGUMENT, "gather rank must be in [0, 8]");
  if (rank > 0 && (out_shape == nullptr || in_strides == nullptr)) return fail(TCX_INVALID_ARGUMENT, "gather metadata is null");
  GatherMeta m{};
  m.rank = rank;
  m.offset = offset;
  std::int64_t n = 1;
  for (int a = 0; a < rank; ++a) {
    if (out_shape[a] < 0) return fail(TCX_INVALID_ARGUMENT, "gather extents must be non-negative");
    m.shape[a] = out_shape[a];
    m.strides[a] = in_strides[a];
    n *= out_shape[a];
  }
  if (n == 0) return TCX_OK;
  if (in == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "gather buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (elem_bytes == 4)
    hipLaunchKernelGGL((gather_kernel<std::uint32_t>), grid_of(n), dim3(256), 0, s,
                       static_cast<const std::uint32_t*>(in), static_cast<std::uint32_t*>(out), m, n);
  else
    hipLaunchKernelGGL((gather_kernel<std::uint8_t>), grid_of(n), dim3(256), 0, s,
                       static_cast<const std::uint8_t*>(in), static_cast<std::uint8_t*>(out), m, n);
  return check(hipGetLastError(), "gather launch");
}

int tcx_hip_copy_blocks(int elem_bytes, const void* in, void* out, int64_t outer, int64_t block, int64_t out_block,
                        int64_t dst_offset, tcx_stream_t stream) {
  using namespace tcx;
  if (int rc = check_bytes(elem_bytes); rc != TCX_OK) return rc;
  if (outer < 0 || block < 0 || dst_offset < 0 || out_block < dst_offset + block)
    return fail(TCX_INVALID_ARGUMENT, "block copy extents are inconsistent");
  if (outer == 0 || block == 0) return TCX_OK;
  if (in == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "block copy buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (elem_bytes == 4)
    hipLaunchKernelGGL((block_copy_kernel<std::uint32_t>), grid_of(outer * block), dim3(256), 0, s,
                       static_cast<const std::uint32_t*>(in), static_cast<std::uint32_t*>(out), outer, block,
                       out_block, dst_offset);
  else
    hipLaunchKernelGGL((block_copy_kernel<std::uint8_t>), grid_of(outer * block), dim3(256), 0, s,
                       static_cast<const std::uint8_t*>(in), static_cast<std::uint8_t*>(out), outer, block,
                       out_block, dst_offset);
  return check(hipGetLastError(), "block copy launch");
}

int tcx_hip_cast(int from, int to, const void* in, void* out, int64_t n, int32_t* flag, tcx_stream_t stream) {
  using namespace tcx;
  const auto valid = [](int d) { return d == TCX_FLOAT32 || d == TCX_INT32 || d == TCX_BOOL; };
  if (!valid(from) || !valid(to)) return fail(TCX_INVALID_ARGUMENT, "unsupported cast dtype");
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "cast extent must be non-negative");
  if (n == 0) return TCX_OK;
  if (in == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "cast buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (from == TCX_FLOAT32 && to == TCX_INT32) {
    // Every source is checked before any conversion result is used.
    if (flag == nullptr) return fail(TCX_INVALID_ARGUMENT, "float32 to int32 casts need a check flag");
    if (int rc = tcx_hip_fill(TCX_INT32, flag, 1, 0.0, stream); rc != TCX_OK) return rc;
    hipLaunchKernelGGL(cast_check_kernel, grid_of(n), dim3(256), 0, s, static_cast<const float*>(in), n, flag);
    if (int rc = check(hipGetLastError(), "cast check launch"); rc != TCX_OK) return rc;
    std::int32_t bad = 0;
    if (int rc = check(hipMemcpyAsync(&bad, flag, sizeof(bad), hipMemcpyDeviceToHost, s), "cast flag copy");
        rc != TCX_OK)
      return rc;
    if (int rc = check(hipStreamSynchronize(s), "cast synchronize"); rc != TCX_OK) return rc;
    if (bad) return fail(TCX_INVALID_ARGUMENT, "float32 value is out of range for int32 cast");
  }
  if (from == TCX_FLOAT32) launch_cast_from<TCX_FLOAT32>(to, in, out, n, s);
  else if (from == TCX_INT32) launch_cast_from<TCX_INT32>(to, in, out, n, s);
  else launch_cast_from<TCX_BOOL>(to, in, out, n, s);
  return check(hipGetLastError(), "cast launch");
}

int tcx_hip_scalar_op(int op, int dtype, const void* in, void* out, int64_t n, double scalar, int scalar_left,
                      tcx_stream_t stream) {
  using namespace tcx;
  if (op < TCX_SCALAR_NEGATE || op > TCX_SCALAR_DIVIDE) return fail(TCX_INVALID_ARGUMENT, "unknown scalar operation");
  if (dtype != TCX_FLOAT32 && dtype != TCX_INT32) return fail(TCX_INVALID_ARGUMENT, "numeric operations do not support bool");
  if (dtype == TCX_INT32 && op == TCX_SCALAR_DIVIDE) return fail(TCX_INVALID_ARGUMENT, "division only supports float32 tensors");
  if (dtype == TCX_INT32 && op != TCX_SCALAR_NEGATE &&
      !(scalar >= -2147483648.0 && scalar <= 2147483647.0 && scalar == static_cast<double>(static_cast<std::int64_t>(scalar))))
    return fail(TCX_INVALID_ARGUMENT, "arithmetic scalar must be an integer in int32 range");
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "extent must be non-negative");
  if (n == 0) return TCX_OK;
  if (in == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "scalar operation buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (dtype == TCX_FLOAT32) {
    const auto* x = static_cast<const float*>(in);
    auto* y = static_cast<float*>(out);
    const float v = static_cast<float>(scalar);
    switch (op) {
      case TCX_SCALAR_NEGATE: hipLaunchKernelGGL((scalar_f32_kernel<TCX_SCALAR_NEGATE>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      case TCX_SCALAR_ADD: hipLaunchKernelGGL((scalar_f32_kernel<TCX_SCALAR_ADD>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      case TCX_SCALAR_SUBTRACT: hipLaunchKernelGGL((scalar_f32_kernel<TCX_SCALAR_SUBTRACT>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      case TCX_SCALAR_MULTIPLY: hipLaunchKernelGGL((scalar_f32_kernel<TCX_SCALAR_MULTIPLY>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      default: hipLaunchKernelGGL((scalar_f32_kernel<TCX_SCALAR_DIVIDE>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
    }
  } else {
    const auto* x = static_cast<const std::uint32_t*>(in);
    auto* y = static_cast<std::uint32_t*>(out);
    const auto v = op == TCX_SCALAR_NEGATE ? 0U : static_cast<std::uint32_t>(static_cast<std::int32_t>(scalar));
    switch (op) {
      case TCX_SCALAR_NEGATE: hipLaunchKernelGGL((scalar_i32_kernel<TCX_SCALAR_NEGATE>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      case TCX_SCALAR_ADD: hipLaunchKernelGGL((scalar_i32_kernel<TCX_SCALAR_ADD>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      case TCX_SCALAR_SUBTRACT: hipLaunchKernelGGL((scalar_i32_kernel<TCX_SCALAR_SUBTRACT>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
      default: hipLaunchKernelGGL((scalar_i32_kernel<TCX_SCALAR_MULTIPLY>), grid_of(n), dim3(256), 0, s, x, y, n, v, scalar_left); break;
    }
  }
  return check(hipGetLastError(), "scalar operation launch");
}

}  // extern "C"
