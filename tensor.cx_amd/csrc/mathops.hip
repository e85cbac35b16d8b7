// log / sqrt / abs, clip and topk: the math extension of the reference
// (backends/cpu/cpu_math.cpp:27-76 under the plans of core/math.cpp:13-71).
//
// Values are handled as 32-bit words, as the reference does: abs clears the
// sign bit (float32) or negates in uint32 (int32, so INT32_MIN stays), clip and
// topk order words with the reference's total order (+0 == -0, NaN handled
// apart), so the results are bit-exact. log uses OCML's logf (within 1 ulp of
// glibc's logf); sqrt is IEEE correctly rounded, as std::sqrt is.
//
//   math_unary_kernel  grid-stride elementwise log / sqrt / abs
//   clip_kernel        three-way broadcast clip(x, lo, hi)
//   topk_kernel        one 256-thread block per (outer, inner) row: k rounds of
//                      exact selection of the next element in the order, then
//                      (sorted == 0) an index-order compaction of the chosen set.
//                      O(k * reduce) work per row: correctness-first.

#include "common.hpp"

namespace tcx {
namespace {

__device__ __forceinline__ bool word_nan(std::uint32_t a, bool fp) {
  return fp && (a & 0x7fffffffU) > 0x7f800000U;
}

// Monotone key of the reference's float order (cpu_math.cpp:15-20): -0 maps
// to +0, negative words are inverted, positive words get the top bit set.
__device__ __forceinline__ std::uint32_t order_key(std::uint32_t a) {
  if ((a & 0x7fffffffU) == 0) a = 0;
  return (a & 0x80000000U) ? ~a : (a ^ 0x80000000U);
}

__device__ __forceinline__ bool word_less(std::uint32_t a, std::uint32_t b, bool fp) {
  if (!fp) return static_cast<std::int32_t>(a) < static_cast<std::int32_t>(b);
  return order_key(a) < order_key(b);
}

template <int kCode, bool kFp>
__device__ __forceinline__ std::uint32_t math_word(std::uint32_t a) {
  if constexpr (kCode == TCX_MATH_ABS) {
    if constexpr (kFp) return a & 0x7fffffffU;
    return (a & 0x80000000U) ? 0U - a : a;
  } else {
    const float f = __builtin_bit_cast(float, a);
    const float r = kCode == TCX_MATH_LOG ? logf(f) : __builtin_sqrtf(f);
    return __builtin_bit_cast(std::uint32_t, r);
  }
}

template <int kCode, bool kFp>
__global__ __launch_bounds__(256) void math_unary_kernel(const std::uint32_t* __restrict__ x,
                                                         std::uint32_t* __restrict__ out, std::int64_t n) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = math_word<kCode, kFp>(x[i]);
}

struct ClipMeta {
  std::int64_t shape[TCX_HIP_MAX_RANK];
  std::int64_t x[TCX_HIP_MAX_RANK];
  std::int64_t lo[TCX_HIP_MAX_RANK];
  std::int64_t hi[TCX_HIP_MAX_RANK];
  std::int32_t rank;
};

// cpu_math.cpp:45-50: a NaN value stays; a NaN bound, or a bound the value
// does not strictly exceed (lo) / stay below (hi), replaces it; lo first.
template <bool kFp>
__global__ __launch_bounds__(256) void clip_kernel(const std::uint32_t* __restrict__ x,
                                                   const std::uint32_t* __restrict__ lo,
                                                   const std::uint32_t* __restrict__ hi,
                                                   std::uint32_t* __restrict__ out, ClipMeta m, std::int64_t n) {
  const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    std::int64_t flat = i, ox = 0, ol = 0, oh = 0;
    for (int a = m.rank - 1; a >= 0; --a) {
      const std::int64_t c = flat % m.shape[a];
      flat /= m.shape[a];
      ox += c * m.x[a];
      ol += c * m.lo[a];
      oh += c * m.hi[a];
    }
    std::uint32_t v = x[ox];
    const std::uint32_t l = lo[ol], h = hi[oh];
    if (!word_nan(v, kFp)) v = (word_nan(l, kFp) || !word_less(l, v, kFp)) ? l : v;
    if (!word_nan(v, kFp)) v = (word_nan(h, kFp) || !word_less(v, h, kFp)) ? h : v;
    out[i] = v;
  }
}

// ------------------------------------------------------------------ topk
struct Cand {
  std::uint32_t word;
  std::int32_t index;  // -1: none
};

// The reference comparator (cpu_math.cpp:58-64): true when a comes before b.
template <bool kFp>
__device__ __forceinline__ bool before(Cand a, Cand b, bool largest) {
  if (a.index < 0) return false;
  if (b.index < 0) return true;
  const bool an = word_nan(a.word, kFp), bn = word_nan(b.word, kFp);
  if (an != bn) return largest ? an : bn;
  if (!an && (word_less(a.word, b.word, kFp) || word_less(b.word, a.word, kFp)))
    return largest ? word_less(b.word, a.word, kFp) : word_less(a.word, b.word, kFp);
  return a.index < b.index;
}

template <bool kFp>
__device__ Cand block_best(Cand c, bool largest, Cand* lds) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    Cand o;
    o.word = static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(c.word), offset, kWave));
    o.index = __shfl_xor(c.index, offset, kWave);
    // Both partners keep the same winner: the order is total on valid indices.
    if (before<kFp>(o, c, largest)) c = o;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();  // the previous round's readers are done with lds
  if (lane == 0) lds[wave] = c;
  __syncthreads();
  Cand r = lds[0];
#pragma unroll
  for (int w = 1; w < 4; ++w)
    if (before<kFp>(lds[w], r, largest)) r = lds[w];
  return r;
}

template <bool kFp>
__global__ __launch_bounds__(256) void topk_kernel(const std::uint32_t* __restrict__ x,
                                                   std::uint32_t* __restrict__ values,
                                                   std::int32_t* __restrict__ indices, std::int64_t reduce,
                                                   std::int64_t inner, std::int64_t k, int largest_flag,
                                                   int sorted) {
  __shared__ Cand lds[4];
  __shared__ std::int32_t wave_counts[4];
  const bool largest = largest_flag != 0;
  const std::int64_t g = blockIdx.x;  // (outer, inner) row
  const std::int64_t base = (g / inner) * reduce * inner + g % inner;
  const std::int64_t dest0 = (g / inner) * k * inner + g % inner;
  const int t = threadIdx.x;
  Cand prev{0U, -1};
  for (std::int64_t j = 0; j < k; ++j) {
    Cand best{0U, -1};
    for (std::int64_t i = t; i < reduce; i += 256) {
      const Cand c{x[base + i * inner], static_cast<std::int32_t>(i)};
      if ((prev.index < 0 || before<kFp>(prev, c, largest)) && before<kFp>(c, best, largest)) best = c;
    }
    prev = block_best<kFp>(best, largest, lds);
    if (sorted && t == 0) {
      values[dest0 + j * inner] = prev.word;
      indices[dest0 + j * inner] = prev.index;
    }
  }
  if (sorted || k == 0) return;
  // Unsorted: the chosen set is every element not after the k-th pick, listed
  // in index order (cpu_math.cpp:66).
  const int lane = t & 63, wave = t >> 6;
  std::int64_t written = 0;
  for (std::int64_t start = 0; start < reduce; start += 256) {
    const std::int64_t i = start + t;
    bool take = false;
    std::uint32_t w = 0;
    if (i < reduce) {
      w = x[base + i * inner];
      const Cand c{w, static_cast<std::int32_t>(i)};
      take = c.index == prev.index || before<kFp>(c, prev, largest);
    }
    const unsigned long long ballot = __ballot(take);
    const int below = __popcll(ballot & ((1ULL << lane) - 1ULL));
    __syncthreads();
    if (lane == 0) wave_counts[wave] = __popcll(ballot);
    __syncthreads();
    std::int64_t offset = written;
    for (int v = 0; v < wave; ++v) offset += wave_counts[v];
    const std::int64_t pos = offset + below;
    if (take && pos < k) {  // exactly k are taken; the bound keeps every store in range
      values[dest0 + pos * inner] = w;
      indices[dest0 + pos * inner] = static_cast<std::int32_t>(i);
    }
    written += wave_counts[0] + wave_counts[1] + wave_counts[2] + wave_counts[3];
  }
}

template <int kCode>
void launch_unary(bool fp, const void* x, void* out, std::int64_t n, hipStream_t s) {
  const dim3 grid(grid_for(n, 256, 256 * 32));
  const auto* xi = static_cast<const std::uint32_t*>(x);
  auto* o = static_cast<std::uint32_t*>(out);
  if (fp)
    hipLaunchKernelGGL((math_unary_kernel<kCode, true>), grid, dim3(256), 0, s, xi, o, n);
  else
    hipLaunchKernelGGL((math_unary_kernel<kCode, false>), grid, dim3(256), 0, s, xi, o, n);
}

int check_dtype(int dtype) {
  if (dtype != TCX_FLOAT32 && dtype != TCX_INT32) return fail(TCX_INVALID_ARGUMENT, "math operations require float32 or int32");
  return TCX_OK;
}

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_math_unary(int op, int dtype, const void* x, void* out, int64_t n, tcx_stream_t stream) {
  using namespace tcx;
  if (int rc = check_dtype(dtype); rc != TCX_OK) return rc;
  if (op != TCX_MATH_LOG && op != TCX_MATH_SQRT && op != TCX_MATH_ABS)
    return fail(TCX_INVALID_ARGUMENT, "unknown math unary operation");
  if (op != TCX_MATH_ABS && dtype != TCX_FLOAT32) return fail(TCX_INVALID_ARGUMENT, "log/sqrt only support float32 tensors");
  if (n < 0) return fail(TCX_INVALID_ARGUMENT, "element count must be non-negative");
  if (n == 0) return TCX_OK;
  if (x == nullptr || out == nullptr) return fail(TCX_INVALID_ARGUMENT, "math buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  const bool fp = dtype == TCX_FLOAT32;
  if (op == TCX_MATH_LOG) launch_unary<TCX_MATH_LOG>(fp, x, out, n, s);
  else if (op == TCX_MATH_SQRT) launch_unary<TCX_MATH_SQRT>(fp, x, out, n, s);
  else launch_unary<TCX_MATH_ABS>(fp, x, out, n, s);
  return check(hipGetLastError(), "math unary launch");
}

int tcx_hip_clip(int dtype, const void* x, const void* lo, const void* hi, void* out, int32_t rank,
                 const int64_t* out_shape, const int64_t* x_strides, const int64_t* lo_strides,
                 const int64_t* hi_strides, tcx_stream_t stream) {
  using namespace tcx;
  if (int rc = check_dtype(dtype); rc != TCX_OK) return rc;
  if (rank < 0 || rank > TCX_HIP_MAX_RANK) return fail(TCX_INVALID_ARGUMENT, "clip rank must be in [0, 8]");
  if (rank > 0 && (out_shape == nullptr || x_strides == nullptr || lo_strides == nullptr || hi_strides == nullptr))
    return fail(TCX_INVALID_ARGUMENT, "clip metadata is null");
  ClipMeta m{};
  m.rank = rank;
  std::int64_t n = 1;
  for (int i = 0; i < rank; ++i) {
    if (out_shape[i] < 0) return fail(TCX_INVALID_ARGUMENT, "clip extents must be non-negative");
    m.shape[i] = out_shape[i];
    m.x[i] = x_strides[i];
    m.lo[i] = lo_strides[i];
    m.hi[i] = hi_strides[i];
    n *= out_shape[i];
  }
  if (n == 0) return TCX_OK;
  if (x == nullptr || lo == nullptr || hi == nullptr || out == nullptr)
    return fail(TCX_INVALID_ARGUMENT, "clip buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for(n, 256, 256 * 32));
  const auto* xi = static_cast<const std::uint32_t*>(x);
  const auto* li = static_cast<const std::uint32_t*>(lo);
  const auto* hi_words = static_cast<const std::uint32_t*>(hi);
  auto* o = static_cast<std::uint32_t*>(out);
  if (dtype == TCX_FLOAT32)
    hipLaunchKernelGGL((clip_kernel<true>), grid, dim3(256), 0, s, xi, li, hi_words, o, m, n);
  else
    hipLaunchKernelGGL((clip_kernel<false>), grid, dim3(256), 0, s, xi, li, hi_words, o, m, n);
  return check(hipGetLastError(), "clip launch");
}

int tcx_hip_topk(int dtype, const void* x, void* values, int32_t* indices, int64_t outer, int64_t reduce,
                 int64_t inner, int64_t k, int largest, int sorted, tcx_stream_t stream) {
  using namespace tcx;
  if (int rc = check_dtype(dtype); rc != TCX_OK) return rc;
  if (outer < 0 || reduce < 0 || inner < 0) return fail(TCX_INVALID_ARGUMENT, "topk extents must be non-negative");
  if (reduce > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "topk index range exceeds int32");
  if (k < 0 || k > reduce) return fail(TCX_INVALID_ARGUMENT, "topk k must be between zero and the axis size");
  const std::int64_t rows = outer * inner;
  if (rows == 0 || k == 0) return TCX_OK;
  if (rows > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "topk has too many rows");
  if (x == nullptr || values == nullptr || indices == nullptr) return fail(TCX_INVALID_ARGUMENT, "topk buffers are null");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  const auto* xi = static_cast<const std::uint32_t*>(x);
  auto* v = static_cast<std::uint32_t*>(values);
  if (dtype == TCX_FLOAT32)
    hipLaunchKernelGGL((topk_kernel<true>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, xi, v, indices,
                       reduce, inner, k, largest, sorted);
  else
    hipLaunchKernelGGL((topk_kernel<false>), dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, xi, v, indices,
                       reduce, inner, k, largest, sorted);
  return check(hipGetLastError(), "topk launch");
}

}  // extern "C"
