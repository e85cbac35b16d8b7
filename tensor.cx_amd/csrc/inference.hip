// Embedding gather and attention softmax: the native primitives under the
// reference's inference composites (backends/cpu/cpu_inference.cpp:10-47,
// plans in core/inference.cpp:47-84).
//
//   embedding_check_kernel  flags any index outside [0, vocabulary)
//   embedding_kernel        row gather, copied as 32-bit words (bits kept)
//   attention_softmax_kernel one wave per score row: masked / causal / scaled
//                           scores, NaN-first maximum, all-masked rows -> 0,
//                           exp(s - max) / sum (tree-order sum, expf)

#include "common.hpp"

namespace tcx {
namespace {

__global__ __launch_bounds__(256) void embedding_check_kernel(const std::int32_t* __restrict__ indices,
                                                              std::int64_t count, std::int64_t vocabulary,
                                                              std::int32_t* __restrict__ flag) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
    const std::int32_t id = indices[i];
    if (id < 0 || id >= vocabulary) *flag = 1;  // every writer stores the same value
  }
}

__global__ __launch_bounds__(256) void embedding_kernel(const std::int32_t* __restrict__ indices,
                                                        const std::uint32_t* __restrict__ weight,
                                                        std::uint32_t* __restrict__ out, std::int64_t count,
                                                        std::int64_t vocabulary, std::int64_t width) {
  const std::int64_t n = count * width;
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t e = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const std::int64_t i = e / width, c = e % width;
    const std::int32_t id = indices[i];
    // Out-of-range rows are never read; the check kernel reports them.
    out[e] = (id >= 0 && id < vocabulary) ? weight[static_cast<std::int64_t>(id) * width + c] : 0U;
  }
}

struct SoftmaxMeta {
  std::int64_t shape[TCX_HIP_MAX_RANK];
  std::int64_t s[TCX_HIP_MAX_RANK];
  std::int64_t m[TCX_HIP_MAX_RANK];
  std::int32_t rank;
  std::int32_t mask_kind;
  std::int32_t causal;
  float scale;
};

__device__ __forceinline__ float attention_score(const float* __restrict__ scores, const void* __restrict__ mask,
                                                 const SoftmaxMeta& d, std::int64_t sbase, std::int64_t mbase,
                                                 std::int64_t ss, std::int64_t ms, std::int64_t col,
                                                 std::int64_t query) {
  const float neg_inf = -__builtin_inff();
  if (d.causal && col > query) return neg_inf;
  if (d.mask_kind == TCX_MASK_BOOL && !static_cast<const std::uint8_t*>(mask)[mbase + col * ms]) return neg_inf;
  const float bias = d.mask_kind == TCX_MASK_ADDITIVE ? static_cast<const float*>(mask)[mbase + col * ms] : 0.F;
  if (bias == neg_inf) return bias;
  const float product = scores[sbase + col * ss] * d.scale;
  return product + bias;
}

__global__ __launch_bounds__(256) void attention_softmax_kernel(const float* __restrict__ scores,
                                                                const void* __restrict__ mask,
                                                                float* __restrict__ out, SoftmaxMeta d,
                                                                std::int64_t rows) {
  const int lane = threadIdx.x & 63;
  const int r = d.rank;
  const std::int64_t columns = d.shape[r - 1], queries = d.shape[r - 2];
  const std::int64_t ss = d.s[r - 1], ms = d.m[r - 1];
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
  for (std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < rows; row += step) {
    std::int64_t flat = row, sbase = 0, mbase = 0;
    for (int a = r - 2; a >= 0; --a) {
      const std::int64_t c = flat % d.shape[a];
      flat /= d.shape[a];
      sbase += c * d.s[a];
      mbase += c * d.m[a];
    }
    const std::int64_t query = row % queries;
    float m = -__builtin_inff();
    bool nan = false;
    for (std::int64_t col = lane; col < columns; col += 64) {
      const float v = attention_score(scores, mask, d, sbase, mbase, ss, ms, col, query);
      if (is_nan(v)) nan = true;
      else m = v > m ? v : m;
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) m = fmaxf(m, __shfl_xor(m, offset, kWave));
    if (__any(nan)) m = __builtin_nanf("");
    float* o = out + row * columns;
    if (m == -__builtin_inff()) {
      for (std::int64_t col = lane; col < columns; col += 64) o[col] = 0.F;
      continue;
    }
    float total = 0.F;
    for (std::int64_t col = lane; col < columns; col += 64)
      total += expf(attention_score(scores, mask, d, sbase, mbase, ss, ms, col, query) - m);
    total = wave_sum(total);
    for (std::int64_t col = lane; col < columns; col += 64)
      o[col] = expf(attention_score(scores, mask, d, sbase, mbase, ss, ms, col, query) - m) / total;
  }
}

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_embedding_f32(const int32_t* indices, const float* weight, float* out, int64_t count,
                          int64_t vocabulary, int64_t width, int32_t* flag, tcx_stream_t stream) {
  using namespace tcx;
  if (count < 0 || vocabulary < 0 || width < 0) return fail(TCX_INVALID_ARGUMENT, "embedding extents must be non-negative");
  if (count == 0) return TCX_OK;
  if (indices == nullptr || flag == nullptr) return fail(TCX_INVALID_ARGUMENT, "embedding buffers are null");
  if (width > 0 && (weight == nullptr || out == nullptr)) return fail(TCX_INVALID_ARGUMENT, "embedding buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (int rc = tcx_hip_fill(TCX_INT32, flag, 1, 0.0, stream); rc != TCX_OK) return rc;
  hipLaunchKernelGGL(embedding_check_kernel, dim3(grid_for(count, 256, 4096)), dim3(256), 0, s, indices, count,
                     vocabulary, flag);
  if (int rc = check(hipGetLastError(), "embedding check launch"); rc != TCX_OK) return rc;
  if (width > 0) {
    hipLaunchKernelGGL(embedding_kernel, dim3(grid_for(count * width, 256, 256 * 32)), dim3(256), 0, s, indices,
                       reinterpret_cast<const std::uint32_t*>(weight), reinterpret_cast<std::uint32_t*>(out), count,
                       vocabulary, width);
    if (int rc = check(hipGetLastError(), "embedding launch"); rc != TCX_OK) return rc;
  }
  std::int32_t host_flag = 0;
  if (int rc = check(hipMemcpyAsync(&host_flag, flag, sizeof(host_flag), hipMemcpyDeviceToHost, s),
                     "embedding flag copy");
      rc != TCX_OK)
    return rc;
  if (int rc = check(hipStreamSynchronize(s), "embedding synchronize"); rc != TCX_OK) return rc;
  if (host_flag != 0) return fail(TCX_INVALID_ARGUMENT, "embedding index out of range");
  return TCX_OK;
}

int tcx_hip_attention_softmax_f32(const float* scores, const void* mask, float* out,
                                  const tcx_hip_attention_softmax_desc_t* desc, tcx_stream_t stream) {
  using namespace tcx;
  if (desc == nullptr) return fail(TCX_INVALID_ARGUMENT, "attention softmax descriptor is null");
  const auto& in = *desc;
  if (in.rank < 2 || in.rank > TCX_HIP_MAX_RANK) return fail(TCX_INVALID_ARGUMENT, "attention softmax rank must be in [2, 8]");
  if (in.mask_kind < TCX_MASK_NONE || in.mask_kind > TCX_MASK_ADDITIVE)
    return fail(TCX_INVALID_ARGUMENT, "unknown attention mask kind");
  SoftmaxMeta d{};
  d.rank = in.rank;
  d.mask_kind = in.mask_kind;
  d.causal = in.causal != 0;
  d.scale = in.scale;
  std::int64_t count = 1;
  for (int i = 0; i < in.rank; ++i) {
    if (in.shape[i] < 0) return fail(TCX_INVALID_ARGUMENT, "attention softmax extents must be non-negative");
    d.shape[i] = in.shape[i];
    d.s[i] = in.score_strides[i];
    d.m[i] = in.mask_kind != TCX_MASK_NONE ? in.mask_strides[i] : 0;
    count *= in.shape[i];
  }
  if (count == 0) return TCX_OK;
  if (scores == nullptr || out == nullptr || (in.mask_kind != TCX_MASK_NONE && mask == nullptr))
    return fail(TCX_INVALID_ARGUMENT, "attention softmax buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const std::int64_t rows = count / in.shape[in.rank - 1];
  hipLaunchKernelGGL(attention_softmax_kernel, dim3(grid_for(rows, 4, 256 * 16)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), scores, mask, out, d, rows);
  return check(hipGetLastError(), "attention softmax launch");
}

}  // extern "C"
