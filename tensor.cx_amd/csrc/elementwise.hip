// Elementwise kernels: fused bias+activation, exp/gelu/silu, broadcast
// arithmetic and fill (reference cpu_backend.cpp:1000-1010, 1014-1097 and the
// fill of cpu_backend.cpp). All are HBM-bound streams with 16-byte accesses
// where the layout allows; each element is rounded exactly as the reference
// rounds it (one operation per step, -ffp-contract=off).

#include "common.hpp"

namespace tcx {
namespace {

__device__ __forceinline__ float act_apply(float v, int act) {
  if (act == TCX_ACT_SILU) return v / (1.0F + expf(-v));
  if (act == TCX_ACT_GELU) {
    const float cubic = 0.044715F * v * v * v;
    const float inner = 0.7978845608028654F * (v + cubic);
    return 0.5F * v * (1.0F + tanhf(inner));
  }
  return v;
}

// 16-byte rows: a block takes 256 consecutive float4 columns of a row and
// strides over rows (blockIdx.y), so a thread's bias float4 is loaded once and
// no column index is divided out; loads and stores are non-temporal (each
// element is touched once).
__global__ __launch_bounds__(256) void bias_act_vec_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ bias,
                                                           float* __restrict__ out, std::int64_t rows,
                                                           std::int64_t cols, int act) {
  const std::int64_t cq = cols / 4;
  const std::int64_t c = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= cq) return;
  float4_t b = {0.F, 0.F, 0.F, 0.F};
  if (bias) b = reinterpret_cast<const float4_t*>(bias)[c];
  for (std::int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    const std::int64_t i = r * cq + c;
    float4_t v = stream_load(reinterpret_cast<const float4_t*>(x) + i);
    if (bias) {
      v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
    }
    v.x = act_apply(v.x, act); v.y = act_apply(v.y, act);
    v.z = act_apply(v.z, act); v.w = act_apply(v.w, act);
    __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(out) + i);
  }
}

// Narrower 16-byte rows: one float4 per thread per step over the flat
// stream; the bias column advances by the grid stride modulo cols / 4, one
// compare per step instead of a 64-bit division.
__global__ __launch_bounds__(256) void bias_act_quad_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ out, std::int64_t rows,
                                                            std::int64_t cols, int act) {
  const std::int64_t quads = rows * cols / 4, cq = cols / 4;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  const std::int64_t start = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::int64_t col_step = step % cq;
  std::int64_t c = start % cq;
  for (std::int64_t i = start; i < quads; i += step) {
    float4_t v = stream_load(reinterpret_cast<const float4_t*>(x) + i);
    if (bias) {
      const float4_t b = reinterpret_cast<const float4_t*>(bias)[c];
      v.x = v.x + b.x; v.y = v.y + b.y; v.z = v.z + b.z; v.w = v.w + b.w;
    }
    v.x = act_apply(v.x, act); v.y = act_apply(v.y, act);
    v.z = act_apply(v.z, act); v.w = act_apply(v.w, act);
    __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(out) + i);
    c += col_step;
    if (c >= cq) c -= cq;
  }
}

// Any layout: one element per thread per step, the column stepped as above.
__global__ __launch_bounds__(256) void bias_act_kernel(const float* __restrict__ x, const float* __restrict__ bias,
                                                       float* __restrict__ out, std::int64_t rows,
                                                       std::int64_t cols, int act) {
  const std::int64_t n = rows * cols;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  const std::int64_t start = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const std::int64_t col_step = step % cols;
  std::int64_t c = start % cols;
  for (std::int64_t i = start; i < n; i += step) {
    float v = x[i];
    if (bias) v = v + bias[c];
    out[i] = act_apply(v, act);
    c += col_step;
    if (c >= cols) c -= cols;
  }
}

__device__ __forceinline__ float unary_apply(float v, int op) {
  return op == TCX_UNARY_EXP ? expf(v) : act_apply(v, op == TCX_UNARY_GELU ? TCX_ACT_GELU : TCX_ACT_SILU);
}

// n a multiple of 4 on 16-byte aligned buffers: one float4 per thread per
// step, non-temporal.
__global__ __launch_bounds__(256) void unary_vec_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                        std::int64_t quads, int op) {
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < quads;
       i += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
    float4_t v = stream_load(reinterpret_cast<const float4_t*>(x) + i);
    v.x = unary_apply(v.x, op); v.y = unary_apply(v.y, op);
    v.z = unary_apply(v.z, op); v.w = unary_apply(v.w, op);
    __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(out) + i);
  }
}

__global__ __launch_bounds__(256) void unary_kernel(const float* __restrict__ x, float* __restrict__ out,
                                                    std::int64_t n, int op) {
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
    const float v = x[i];
    out[i] = unary_apply(v, op);
  }
}

struct BroadcastMeta {
  std::int64_t shape[TCX_HIP_MAX_FOLDED_RANK];
  std::int64_t lhs[TCX_HIP_MAX_FOLDED_RANK];
  std::int64_t rhs[TCX_HIP_MAX_FOLDED_RANK];
  std::int32_t rank;
};

template <typename T>
__device__ __forceinline__ T binary_op(T a, T b, int op) {
  if constexpr (__is_same(T, float)) {
    switch (op) {
      case TCX_BINARY_ADD: return a + b;
      case TCX_BINARY_SUBTRACT: return a - b;
      case TCX_BINARY_MULTIPLY: return a * b;
      default: return a / b;
    }
  } else {
    switch (op) {
      case TCX_BINARY_ADD: return a + b;
      case TCX_BINARY_SUBTRACT: return a - b;
      default: return a * b;
    }
  }
}

template <typename T, typename U>
__global__ __launch_bounds__(256) void binary_kernel(const U* __restrict__ lhs, const U* __restrict__ rhs,
                                                     U* __restrict__ out, BroadcastMeta m, std::int64_t n,
                                                     int op) {
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
    std::int64_t index = i, l = 0, r = 0;
    for (int axis = m.rank - 1; axis >= 0; --axis) {
      const std::int64_t c = index % m.shape[axis];
      index /= m.shape[axis];
      l += c * m.lhs[axis];
      r += c * m.rhs[axis];
    }
    // int32 arithmetic runs in uint32 so overflow wraps (cpu_backend.cpp:1070-1093).
    out[i] = static_cast<U>(binary_op<T>(static_cast<T>(lhs[l]), static_cast<T>(rhs[r]), op));
  }
}

// Broadcasts of at most two folded axes, out [R, C] (a same-shape stream is
// [1, n]): a block strides over rows (blockIdx.y) and columns, so each
// element's operand offsets are a multiply-add, not a chain of 64-bit
// divisions. kVec: C a multiple of 4, inner strides 0 or 1, 16-byte aligned
// rows; a stride-0 operand is one word per row, splatted.
template <typename T, typename U, bool kVec>
__global__ __launch_bounds__(256) void binary_2d_kernel(const U* __restrict__ lhs, const U* __restrict__ rhs,
                                                        U* __restrict__ out, std::int64_t R, std::int64_t C,
                                                        std::int64_t l0, std::int64_t l1, std::int64_t r0,
                                                        std::int64_t r1, int op) {
  using V = U __attribute__((ext_vector_type(4)));
  const std::int64_t units = kVec ? C / 4 : C;
  const std::int64_t cstep = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t r = blockIdx.y; r < R; r += gridDim.y) {
    const U* __restrict__ lrow = lhs + r * l0;
    const U* __restrict__ rrow = rhs + r * r0;
    U* __restrict__ orow = out + r * C;
    for (std::int64_t c = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < units; c += cstep) {
      if constexpr (kVec) {
        V a, b;
        if (l1) a = stream_load(reinterpret_cast<const V*>(lrow) + c);
        else a = V{lrow[0], lrow[0], lrow[0], lrow[0]};
        if (r1) b = stream_load(reinterpret_cast<const V*>(rrow) + c);
        else b = V{rrow[0], rrow[0], rrow[0], rrow[0]};
        V o;
        o.x = static_cast<U>(binary_op<T>(static_cast<T>(a.x), static_cast<T>(b.x), op));
        o.y = static_cast<U>(binary_op<T>(static_cast<T>(a.y), static_cast<T>(b.y), op));
        o.z = static_cast<U>(binary_op<T>(static_cast<T>(a.z), static_cast<T>(b.z), op));
        o.w = static_cast<U>(binary_op<T>(static_cast<T>(a.w), static_cast<T>(b.w), op));
        __builtin_nontemporal_store(o, reinterpret_cast<V*>(orow) + c);
      } else {
        orow[c] = static_cast<U>(binary_op<T>(static_cast<T>(lrow[c * l1]), static_cast<T>(rrow[c * r1]), op));
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void fill_kernel(T* __restrict__ out, std::int64_t n, T value) {
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<std::int64_t>(gridDim.x) * blockDim.x)
    out[i] = value;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }
constexpr std::int64_t kMaxBlocks = 256 * 32;  // 32 blocks per CU for grid-stride loops
// The 16-byte streams: up to one float4 per thread (a 1 GiB copy probe ran
// best so, at 81 % of HBM peak), grid-stride beyond.
constexpr std::int64_t kVecBlocks = std::int64_t{1} << 18;

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_bias_act_f32(const float* x, const float* bias, float* out, int64_t rows, int64_t cols, int act,
                         tcx_stream_t stream) {
  using namespace tcx;
  if (rows < 0 || cols < 0) return fail(TCX_INVALID_ARGUMENT, "bias_act extents must be non-negative");
  if (act < TCX_ACT_NONE || act > TCX_ACT_GELU) return fail(TCX_INVALID_ARGUMENT, "unknown activation");
  if (rows == 0 || cols == 0) return TCX_OK;
  if (x == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "bias_act buffers are null");
  const int rc = ready();
  if (rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (cols % 4 == 0 && cols >= 1024 && aligned16(x) && aligned16(out) && (bias == nullptr || aligned16(bias))) {
    // Rows of at least 256 float4 (narrower rows would leave most of a
    // block's lanes idle and take the scalar kernel).
    const unsigned gx = grid_for(cols / 4, 256, kVecBlocks);
    const std::int64_t gy_max = kVecBlocks / gx < 65535 ? kVecBlocks / gx : 65535;
    const unsigned gy = static_cast<unsigned>(rows < gy_max ? rows : (gy_max > 0 ? gy_max : 1));
    hipLaunchKernelGGL(bias_act_vec_kernel, dim3(gx, gy), dim3(256), 0, s, x, bias, out, rows, cols, act);
  } else if (cols % 4 == 0 && aligned16(x) && aligned16(out) && (bias == nullptr || aligned16(bias))) {
    hipLaunchKernelGGL(bias_act_quad_kernel, dim3(grid_for(rows * cols / 4, 256, kVecBlocks)), dim3(256), 0, s,
                       x, bias, out, rows, cols, act);
  } else {
    hipLaunchKernelGGL(bias_act_kernel, dim3(grid_for(rows * cols, 256, kMaxBlocks)), dim3(256), 0, s, x, bias,
                       out, rows, cols, act);
  }
  return check(hipGetLastError(), "bias_act launch");
}

int tcx_hip_unary_f32(int op, const float* x, float* out, int64_t n, tcx_stream_t stream) {
  using namespace tcx;
  if (op < TCX_UNARY_EXP || op > TCX_UNARY_SILU) return fail(TCX_INVALID_ARGUMENT, "unknown unary op");
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "unary extent must be non-negative");
  if (n == 0) return TCX_OK;
  if (x == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "unary buffers are null");
  const int rc = ready();
  if (rc != TCX_OK) return rc;
  if (n % 4 == 0 && aligned16(x) && aligned16(out))
    hipLaunchKernelGGL(unary_vec_kernel, dim3(grid_for(n / 4, 256, kVecBlocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, out, n / 4, op);
  else
    hipLaunchKernelGGL(unary_kernel, dim3(grid_for(n, 256, kMaxBlocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, out, n, op);
  return check(hipGetLastError(), "unary launch");
}

int tcx_hip_binary(int op, int dtype, const void* lhs, const void* rhs, void* out, int32_t rank,
                   const int64_t* out_shape, const int64_t* lhs_strides, const int64_t* rhs_strides,
                   tcx_stream_t stream) {
  using namespace tcx;
  if (op < TCX_BINARY_ADD || op > TCX_BINARY_DIVIDE) return fail(TCX_INVALID_ARGUMENT, "unknown binary op");
  if (dtype != TCX_FLOAT32 && dtype != TCX_INT32)
    return fail(TCX_INVALID_ARGUMENT, "arithmetic requires float32 or int32 tensors");
  if (dtype == TCX_INT32 && op == TCX_BINARY_DIVIDE)
    return fail(TCX_INVALID_ARGUMENT, "division only supports float32 tensors");
  if (rank < 0 || rank > TCX_HIP_MAX_FOLDED_RANK)
    return fail(TCX_INVALID_ARGUMENT, "binary rank exceeds the supported maximum");
  BroadcastMeta m{};
  m.rank = rank;
  std::int64_t n = 1;
  for (int i = 0; i < rank; ++i) {
    if (out_shape[i] < 0) return fail(TCX_INVALID_ARGUMENT, "binary extents must be non-negative");
    m.shape[i] = out_shape[i];
    m.lhs[i] = lhs_strides[i];
    m.rhs[i] = rhs_strides[i];
    n *= out_shape[i];
  }
  if (n == 0) return TCX_OK;
  if (lhs == nullptr || rhs == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "binary buffers are null");
  const int rc = ready();
  if (rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (rank <= 2) {
    const std::int64_t R = rank == 2 ? m.shape[0] : 1, C = rank == 0 ? 1 : m.shape[rank - 1];
    const std::int64_t l0 = rank == 2 ? m.lhs[0] : 0, r0 = rank == 2 ? m.rhs[0] : 0;
    const std::int64_t l1 = rank == 0 ? 0 : m.lhs[rank - 1], r1 = rank == 0 ? 0 : m.rhs[rank - 1];
    const bool unit = (l1 == 0 || l1 == 1) && (r1 == 0 || r1 == 1);
    const bool vec = unit && C % 4 == 0 && aligned16(out) && (l1 == 0 || (aligned16(lhs) && l0 % 4 == 0)) &&
                     (r1 == 0 || (aligned16(rhs) && r0 % 4 == 0));
    const std::int64_t units = vec ? C / 4 : C;
    const unsigned gx = grid_for(units, 256, kVecBlocks);
    const std::int64_t gy_max = kVecBlocks / gx < 65535 ? kVecBlocks / gx : 65535;
    const dim3 grid2(gx, static_cast<unsigned>(R < gy_max ? R : (gy_max > 0 ? gy_max : 1)));
    auto launch2 = [&](auto kernel, auto p) {
      using P = decltype(p);
      hipLaunchKernelGGL(kernel, grid2, dim3(256), 0, s, static_cast<const P*>(lhs), static_cast<const P*>(rhs),
                         static_cast<P*>(out), R, C, l0, l1, r0, r1, op);
    };
    if (dtype == TCX_FLOAT32)
      vec ? launch2(binary_2d_kernel<float, float, true>, 0.F) : launch2(binary_2d_kernel<float, float, false>, 0.F);
    else
      vec ? launch2(binary_2d_kernel<std::uint32_t, std::uint32_t, true>, 0U)
          : launch2(binary_2d_kernel<std::uint32_t, std::uint32_t, false>, 0U);
    return check(hipGetLastError(), "binary launch");
  }
  const dim3 grid(grid_for(n, 256, kMaxBlocks));
  if (dtype == TCX_FLOAT32)
    hipLaunchKernelGGL((binary_kernel<float, float>), grid, dim3(256), 0, s, static_cast<const float*>(lhs),
                       static_cast<const float*>(rhs), static_cast<float*>(out), m, n, op);
  else
    hipLaunchKernelGGL((binary_kernel<std::uint32_t, std::uint32_t>), grid, dim3(256), 0, s,
                       static_cast<const std::uint32_t*>(lhs), static_cast<const std::uint32_t*>(rhs),
                       static_cast<std::uint32_t*>(out), m, n, op);
  return check(hipGetLastError(), "binary launch");
}

int tcx_hip_fill(int dtype, void* out, int64_t n, double value, tcx_stream_t stream) {
  using namespace tcx;
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "fill extent must be non-negative");
  if (n == 0) return TCX_OK;
  if (out == nullptr) return fail(TCX_INVALID_ARGUMENT, "fill output is null");
  const int rc = ready();
  if (rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n, 256, kMaxBlocks));
  if (dtype == TCX_FLOAT32)
    hipLaunchKernelGGL((fill_kernel<float>), grid, dim3(256), 0, s, static_cast<float*>(out), n,
                       static_cast<float>(value));
  else if (dtype == TCX_INT32)
    hipLaunchKernelGGL((fill_kernel<int>), grid, dim3(256), 0, s, static_cast<int*>(out), n,
                       static_cast<int>(value));
  else if (dtype == TCX_BOOL)
    hipLaunchKernelGGL((fill_kernel<std::uint8_t>), grid, dim3(256), 0, s, static_cast<std::uint8_t*>(out), n,
                       static_cast<std::uint8_t>(value != 0.0 ? 1 : 0));
  else
    return fail(TCX_INVALID_ARGUMENT, "fill requires float32, int32 or bool");
  return check(hipGetLastError(), "fill launch");
}

}  // extern "C"
