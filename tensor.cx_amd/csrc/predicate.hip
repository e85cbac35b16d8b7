// Predicates and boolean reductions: comparisons, logical operations and
// where over a broadcast plan, any / all over reduction metadata, and
// masked_select (reference backends/cpu/cpu_predicate.cpp:9-98, plans in
// core/predicate.cpp:23-84). Comparisons use IEEE float32 / int32 / bool
// semantics (NaN compares unequal, +0 == -0); where copies the chosen branch's
// element bit for bit; masked_select keeps index order.
//
//   predicate_kernel     one output element per thread, three broadcast inputs
//   bool_reduce_kernel   one wave per output group, lanes stride the group
//   mask_count_kernel    true entries per 1024-entry chunk of the mask
//   mask_index_kernel    indices of true entries, in order, from chunk offsets
//   row_gather_kernel    out row r = in row index[r] (rows of `block` elements)

#include "common.hpp"

namespace tcx {
namespace {

constexpr int kChunk = 1024;  // mask entries per chunk (256 threads x 4)

struct PredicateMeta {
  std::int64_t shape[TCX_HIP_MAX_RANK];
  std::int64_t strides[3][TCX_HIP_MAX_RANK];
  std::int32_t rank;
};

template <typename T>
__device__ __forceinline__ bool compare(T a, T b, int op) {
  switch (op) {
    case TCX_PRED_EQUAL: return a == b;
    case TCX_PRED_NOT_EQUAL: return a != b;
    case TCX_PRED_LESS: return a < b;
    case TCX_PRED_LESS_EQUAL: return a <= b;
    case TCX_PRED_GREATER: return a > b;
    default: return a >= b;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void predicate_kernel(int op, const void* __restrict__ a_,
                                                        const void* __restrict__ b_, const void* __restrict__ c_,
                                                        void* __restrict__ out_, PredicateMeta m, std::int64_t n) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    std::int64_t rest = i, oa = 0, ob = 0, oc = 0;
    for (int d = m.rank - 1; d >= 0; --d) {
      const std::int64_t idx = rest % m.shape[d];
      rest /= m.shape[d];
      oa += idx * m.strides[0][d];
      ob += idx * m.strides[1][d];
      oc += idx * m.strides[2][d];
    }
    if (op == TCX_PRED_WHERE) {
      // T is the branch element type; the condition is bool.
      const bool cond = static_cast<const std::uint8_t*>(a_)[oa] != 0;
      static_cast<T*>(out_)[i] = cond ? static_cast<const T*>(b_)[ob] : static_cast<const T*>(c_)[oc];
    } else if (op >= TCX_PRED_LOGICAL_AND) {
      const bool l = static_cast<const std::uint8_t*>(a_)[oa] != 0;
      const bool r = op != TCX_PRED_LOGICAL_NOT && static_cast<const std::uint8_t*>(b_)[ob] != 0;
      bool y;
      if (op == TCX_PRED_LOGICAL_NOT) y = !l;
      else if (op == TCX_PRED_LOGICAL_AND) y = l && r;
      else if (op == TCX_PRED_LOGICAL_OR) y = l || r;
      else y = l != r;
      static_cast<std::uint8_t*>(out_)[i] = y ? 1 : 0;
    } else {
      bool y;
      if constexpr (sizeof(T) == 1) {
        y = compare<bool>(static_cast<const std::uint8_t*>(a_)[oa] != 0, static_cast<const std::uint8_t*>(b_)[ob] != 0, op);
      } else {
        y = compare<T>(static_cast<const T*>(a_)[oa], static_cast<const T*>(b_)[ob], op);
      }
      static_cast<std::uint8_t*>(out_)[i] = y ? 1 : 0;
    }
  }
}

struct ReduceMeta {
  std::int64_t pairs[2 * TCX_HIP_MAX_RANK];  // (extent, stride), kept axes then reduced axes
  std::int32_t rank;
};

__global__ __launch_bounds__(256) void bool_reduce_kernel(int all, const std::uint8_t* __restrict__ x,
                                                          std::uint8_t* __restrict__ out, ReduceMeta m,
                                                          std::int64_t groups, std::int64_t reduce) {
  const int lane = threadIdx.x & 63;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
  for (std::int64_t g = static_cast<std::int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); g < groups; g += step) {
    bool value = all != 0;
    for (std::int64_t j = lane; j < reduce; j += 64) {
      std::int64_t rest = g * reduce + j, src = 0;
      for (int a = m.rank - 1; a >= 0; --a) {
        src += (rest % m.pairs[2 * a]) * m.pairs[2 * a + 1];
        rest /= m.pairs[2 * a];
      }
      const bool v = x[src] != 0;
      value = all ? (value && v) : (value || v);
    }
    const bool result = all ? __all(value) : __any(value);
    if (lane == 0) out[g] = result ? 1 : 0;
  }
}

__global__ __launch_bounds__(256) void mask_count_kernel(const std::uint8_t* __restrict__ mask, std::int64_t n,
                                                         std::int64_t* __restrict__ counts) {
  __shared__ int wave_total[4];
  const std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kChunk;
  int c = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const std::int64_t i = base + threadIdx.x + 256 * e;
    if (i < n && mask[i] != 0) ++c;
  }
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) c += __shfl_xor(c, offset, kWave);
  if ((threadIdx.x & 63) == 0) wave_total[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[blockIdx.x] = wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
}

// Thread t of chunk c owns entries 4t .. 4t+3 of the chunk (in order), so the
// block-wide exclusive scan of per-thread counts gives each true entry its
// rank inside the chunk.
__global__ __launch_bounds__(256) void mask_index_kernel(const std::uint8_t* __restrict__ mask, std::int64_t n,
                                                         const std::int64_t* __restrict__ offsets,
                                                         std::int64_t* __restrict__ index, std::int64_t total) {
  __shared__ int scan[256];
  const std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kChunk + 4 * threadIdx.x;
  bool take[4];
  int c = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    take[e] = base + e < n && mask[base + e] != 0;
    c += take[e] ? 1 : 0;
  }
  scan[threadIdx.x] = c;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 256 per-thread counts.
  for (int d = 1; d < 256; d <<= 1) {
    const int add = threadIdx.x >= d ? scan[threadIdx.x - d] : 0;
    __syncthreads();
    scan[threadIdx.x] += add;
    __syncthreads();
  }
  std::int64_t pos = offsets[blockIdx.x] + scan[threadIdx.x] - c;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (take[e]) {
      if (pos < total) index[pos] = base + e;  // counts and indices come from the same mask
      ++pos;
    }
}

template <typename T>
__global__ __launch_bounds__(256) void row_gather_kernel(const T* __restrict__ in, const std::int64_t* __restrict__ index,
                                                         T* __restrict__ out, std::int64_t rows, std::int64_t block) {
  const std::int64_t n = rows * block;
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = in[index[i / block] * block + i % block];
}

dim3 grid_of(std::int64_t n) { return dim3(grid_for(n, 256, 256 * 32)); }

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_predicate(int op, int elem_bytes, const void* a, const void* b, const void* c, void* out,
                      const tcx_hip_broadcast3_t* plan, tcx_stream_t stream) {
  using namespace tcx;
  if (op < TCX_PRED_EQUAL || op > TCX_PRED_WHERE) return fail(TCX_INVALID_ARGUMENT, "unknown predicate");
  if (elem_bytes != 1 && elem_bytes != 4) return fail(TCX_INVALID_ARGUMENT, "element size must be 1 or 4 bytes");
  if (plan == nullptr || plan->rank < 0 || plan->rank > TCX_HIP_MAX_RANK)
    return fail(TCX_INVALID_ARGUMENT, "predicate plan rank must be in [0, 8]");
  PredicateMeta m{};
  m.rank = plan->rank;
  std::int64_t n = 1;
  for (int d = 0; d < plan->rank; ++d) {
    if (plan->shape[d] < 0) return fail(TCX_INVALID_ARGUMENT, "predicate extents must be non-negative");
    m.shape[d] = plan->shape[d];
    for (int k = 0; k < 3; ++k) m.strides[k][d] = plan->strides[k][d];
    n *= plan->shape[d];
  }
  if (n == 0) return TCX_OK;
  const int inputs = op == TCX_PRED_WHERE ? 3 : op == TCX_PRED_LOGICAL_NOT ? 1 : 2;
  if (a == nullptr || out == nullptr || (inputs > 1 && b == nullptr) || (inputs > 2 && c == nullptr))
    return fail(TCX_INVALID_ARGUMENT, "predicate buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  // elem_bytes is the compared dtype's size (comparisons) or the branch size
  // (where); the 4-byte compare distinguishes float32 with op flag bit 8.
  if (elem_bytes == 1)
    hipLaunchKernelGGL((predicate_kernel<std::uint8_t>), grid_of(n), dim3(256), 0, s, op, a, b, c, out, m, n);
  else if (op == TCX_PRED_WHERE || (plan->flags & TCX_PRED_FLAG_INT32))
    hipLaunchKernelGGL((predicate_kernel<std::int32_t>), grid_of(n), dim3(256), 0, s, op, a, b, c, out, m, n);
  else
    hipLaunchKernelGGL((predicate_kernel<float>), grid_of(n), dim3(256), 0, s, op, a, b, c, out, m, n);
  return check(hipGetLastError(), "predicate launch");
}

int tcx_hip_bool_reduce(int all, const uint8_t* x, uint8_t* out, const int64_t* meta, int32_t rank, int64_t groups,
                        int64_t reduce, tcx_stream_t stream) {
  using namespace tcx;
  if (rank < 0 || rank > TCX_HIP_MAX_RANK) return fail(TCX_INVALID_ARGUMENT, "boolean reduction rank must be in [0, 8]");
  if (groups < 0 || reduce < 0) return fail(TCX_INVALID_ARGUMENT, "boolean reduction extents must be non-negative");
  if (groups == 0) return TCX_OK;
  if (out == nullptr || (reduce > 0 && (x == nullptr || (rank > 0 && meta == nullptr))))
    return fail(TCX_INVALID_ARGUMENT, "boolean reduction buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  ReduceMeta m{};
  m.rank = rank;
  for (int i = 0; i < 2 * rank; ++i) m.pairs[i] = meta[i];
  hipLaunchKernelGGL(bool_reduce_kernel, dim3(grid_for(groups, 4, 256 * 16)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), all, x, out, m, groups, reduce);
  return check(hipGetLastError(), "boolean reduction launch");
}

int64_t tcx_hip_mask_chunks(int64_t n) { return n <= 0 ? 0 : (n + tcx::kChunk - 1) / tcx::kChunk; }

int tcx_hip_mask_count(const uint8_t* mask, int64_t n, int64_t* chunk_counts, tcx_stream_t stream) {
  using namespace tcx;
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "mask extent must be non-negative");
  if (n == 0) return TCX_OK;
  if (mask == nullptr || chunk_counts == nullptr) return fail(TCX_INVALID_ARGUMENT, "mask buffers are null");
  const std::int64_t chunks = tcx_hip_mask_chunks(n);
  if (chunks > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "mask is too large");
  if (int rc = ready(); rc != TCX_OK) return rc;
  hipLaunchKernelGGL(mask_count_kernel, dim3(static_cast<unsigned>(chunks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mask, n, chunk_counts);
  return check(hipGetLastError(), "mask count launch");
}

int tcx_hip_masked_select(int elem_bytes, const void* in, const uint8_t* mask, int64_t n, int64_t block,
                          const int64_t* chunk_offsets, int64_t total, int64_t* index, void* out,
                          tcx_stream_t stream) {
  using namespace tcx;
  if (elem_bytes != 1 && elem_bytes != 4) return fail(TCX_INVALID_ARGUMENT, "element size must be 1 or 4 bytes");
  if (n < 0 || block < 0 || total < 0 || total > n) return fail(TCX_INVALID_ARGUMENT, "masked select extents are inconsistent");
  if (n == 0 || total == 0) return TCX_OK;
  if (mask == nullptr || chunk_offsets == nullptr || index == nullptr)
    return fail(TCX_INVALID_ARGUMENT, "masked select buffers are null");
  if (block > 0 && (in == nullptr || out == nullptr)) return fail(TCX_INVALID_ARGUMENT, "masked select buffers are null");
  const std::int64_t chunks = tcx_hip_mask_chunks(n);
  if (chunks > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "mask is too large");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(mask_index_kernel, dim3(static_cast<unsigned>(chunks)), dim3(256), 0, s, mask, n, chunk_offsets,
                     index, total);
  if (int rc = check(hipGetLastError(), "mask index launch"); rc != TCX_OK) return rc;
  if (block == 0) return TCX_OK;
  if (elem_bytes == 4)
    hipLaunchKernelGGL((row_gather_kernel<std::uint32_t>), grid_of(total * block), dim3(256), 0, s,
                       static_cast<const std::uint32_t*>(in), index, static_cast<std::uint32_t*>(out), total, block);
  else
    hipLaunchKernelGGL((row_gather_kernel<std::uint8_t>), grid_of(total * block), dim3(256), 0, s,
                       static_cast<const std::uint8_t*>(in), index, static_cast<std::uint8_t*>(out), total, block);
  return check(hipGetLastError(), "masked select launch");
}

}  // extern "C"
