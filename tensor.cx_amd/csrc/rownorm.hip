// Row softmax, RMSNorm and LayerNorm (reference cpu_backend.cpp:125-240), with
// the optional affine weight/bias of the kAffine*Norm composites
// (core/inference.cpp:103-122) fused into the same pass.
//
// Contiguous rows (inner == 1) of up to 64*4*kMaxChunks elements: one wave per
// row holds the whole row in registers (kChunks 16-byte loads per lane), so
// each element is read from HBM once and written once; the row statistics use
// wave-wide butterfly reductions. Longer rows use one 256-thread block per
// row and re-read the row (mostly from L2). Strided rows (inner > 1) use one
// lane per row in the reference's exact element order.
//
// Per-element arithmetic follows the reference step by step (exp(x - max),
// sum, division; (x - mean) * scale; x * scale), each step rounded separately
// (built with -ffp-contract=off). Statistics are summed in a fixed tree order,
// which stays within allclose(rtol=1e-5, atol=1e-5) of the sequential sums.

#include "common.hpp"

namespace tcx {
namespace {

constexpr int kMaxChunks = 32;  // rows up to 8192 floats stay in registers

enum class RowOp { kSoftmax, kRms, kLayer };

struct RowArgs {
  const float* x;
  const float* gamma;
  const float* beta;
  float* out;
  std::int64_t rows, n;
  float eps;
};

__device__ __forceinline__ float wave_max_nan(float v) {
  // NaN-first maximum: any NaN in the row makes the result NaN.
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    const float o = __shfl_xor(v, offset, kWave);
    v = (is_nan(o) || o > v) ? o : v;
  }
  return v;
}

__device__ __forceinline__ float finish_scale_ln(float ssd, std::int64_t n, float eps, bool& nan_row) {
  const float denom = ssd / static_cast<float>(n) + eps;
  nan_row = denom == 0.F;
  return 1.0F / sqrtf(denom);
}

// One wave per row, row cached in registers: kChunks float4 per lane.
template <RowOp kOp, int kChunks, bool kVec>
__global__ __launch_bounds__(256) void row_cached_kernel(RowArgs a) {
  const int lane = threadIdx.x & 63;
  const std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const std::int64_t n = a.n;
  const float* __restrict__ x = a.x + row * n;
  float* __restrict__ out = a.out + row * n;
  float v[kChunks][4];
  // Element (c, q) sits at column 4*(lane + 64c) + q (vector rows) or at
  // lane + 64*(4c + q) (scalar rows); `valid` masks the row tail.
  auto column = [&](int c, int q) -> std::int64_t {
    return kVec ? 4 * (lane + 64 * static_cast<std::int64_t>(c)) + q
                : lane + 64 * (4 * static_cast<std::int64_t>(c) + q);
  };
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    if constexpr (kVec) {
      const std::int64_t i = column(c, 0);
      float4_t t = {0.F, 0.F, 0.F, 0.F};
      if (i < n) t = *reinterpret_cast<const float4_t*>(x + i);
      v[c][0] = t.x; v[c][1] = t.y; v[c][2] = t.z; v[c][3] = t.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const std::int64_t i = column(c, q);
        v[c][q] = i < n ? x[i] : 0.F;
      }
    }
  }

  if constexpr (kOp == RowOp::kSoftmax) {
    float m = -__builtin_inff();
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (column(c, q) < n && (is_nan(v[c][q]) || v[c][q] > m)) m = v[c][q];
    m = wave_max_nan(m);
    float s = 0.F;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (column(c, q) < n) {
          v[c][q] = expf(v[c][q] - m);
          s += v[c][q];
        }
      }
    const float denom = wave_sum(s);
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] / denom;
  } else if constexpr (kOp == RowOp::kRms) {
    float s = 0.F;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float t = v[c][q] * v[c][q];
        s += t;  // masked elements are zero
      }
    const float ss = wave_sum(s);
    const float scale = 1.0F / sqrtf(ss / static_cast<float>(n) + a.eps);
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] * scale;
  } else {
    const float first = x[0];
    float s = 0.F;
    bool equal = true;
#pragma unroll
    for (int c = 0; c < kChunks; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s += v[c][q];
        if (column(c, q) < n) equal = equal && v[c][q] == first;
      }
    const float mean = wave_sum(s) / static_cast<float>(n);
    const bool all_equal = __all(equal);
    if (all_equal && __builtin_isfinite(first)) {
      const float fillv = a.eps == 0.F ? __builtin_nanf("") : 0.F;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = fillv;
    } else {
      float d2 = 0.F;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (column(c, q) < n) {
            const float d = v[c][q] - mean;
            d2 += d * d;
          }
        }
      bool nan_row = false;
      const float scale = finish_scale_ln(wave_sum(d2), n, a.eps, nan_row);
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[c][q] = nan_row ? __builtin_nanf("") : (v[c][q] - mean) * scale;
    }
  }

  // Affine steps (multiply then add, each rounded) and the store.
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    if constexpr (kVec) {
      const std::int64_t i = column(c, 0);
      if (i >= n) continue;
      float4_t t = {v[c][0], v[c][1], v[c][2], v[c][3]};
      if (a.gamma) {
        const float4_t g = *reinterpret_cast<const float4_t*>(a.gamma + i);
        t.x = t.x * g.x; t.y = t.y * g.y; t.z = t.z * g.z; t.w = t.w * g.w;
      }
      if (a.beta) {
        const float4_t b = *reinterpret_cast<const float4_t*>(a.beta + i);
        t.x = t.x + b.x; t.y = t.y + b.y; t.z = t.z + b.z; t.w = t.w + b.w;
      }
      __builtin_nontemporal_store(t, reinterpret_cast<float4_t*>(out + i));
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const std::int64_t i = column(c, q);
        if (i >= n) continue;
        float t = v[c][q];
        if (a.gamma) t = t * a.gamma[i];
        if (a.beta) t = t + a.beta[i];
        out[i] = t;
      }
    }
  }
}

// Rows too long for registers: one block per row, three passes over the row.
__device__ float block_reduce(float v, bool is_max, float* scratch) {
  v = is_max ? wave_max_nan(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) {
    const float o = scratch[w];
    r = is_max ? ((is_nan(o) || o > r) ? o : r) : r + o;
  }
  return r;
}

template <RowOp kOp>
__global__ __launch_bounds__(256) void row_block_kernel(RowArgs a) {
  __shared__ float scratch[4];
  __shared__ int eq_flag;
  const std::int64_t row = blockIdx.x;
  const std::int64_t n = a.n;
  const float* __restrict__ x = a.x + row * n;
  float* __restrict__ out = a.out + row * n;
  const int t = threadIdx.x;
  if constexpr (kOp == RowOp::kSoftmax) {
    float m = -__builtin_inff();
    for (std::int64_t i = t; i < n; i += 256) {
      const float e = x[i];
      if (is_nan(e) || e > m) m = e;
    }
    m = block_reduce(m, true, scratch);
    float s = 0.F;
    for (std::int64_t i = t; i < n; i += 256) s += expf(x[i] - m);
    const float denom = block_reduce(s, false, scratch);
    for (std::int64_t i = t; i < n; i += 256) out[i] = expf(x[i] - m) / denom;
  } else if constexpr (kOp == RowOp::kRms) {
    float s = 0.F;
    for (std::int64_t i = t; i < n; i += 256) {
      const float e = x[i];
      const float sq = e * e;
      s += sq;
    }
    const float ss = block_reduce(s, false, scratch);
    const float scale = 1.0F / sqrtf(ss / static_cast<float>(n) + a.eps);
    for (std::int64_t i = t; i < n; i += 256) {
      float r = x[i] * scale;
      if (a.gamma) r = r * a.gamma[i];
      out[i] = r;
    }
    return;
  } else {
    if (t == 0) eq_flag = 1;
    const float first = x[0];
    float s = 0.F;
    bool equal = true;
    for (std::int64_t i = t; i < n; i += 256) {
      s += x[i];
      equal = equal && x[i] == first;
    }
    const float mean = block_reduce(s, false, scratch) / static_cast<float>(n);
    if (!equal) eq_flag = 0;
    __syncthreads();
    if (eq_flag && __builtin_isfinite(first)) {
      const float fillv = a.eps == 0.F ? __builtin_nanf("") : 0.F;
      for (std::int64_t i = t; i < n; i += 256) {
        float r = fillv;
        if (a.gamma) r = r * a.gamma[i];
        if (a.beta) r = r + a.beta[i];
        out[i] = r;
      }
      return;
    }
    float d2 = 0.F;
    for (std::int64_t i = t; i < n; i += 256) {
      const float d = x[i] - mean;
      d2 += d * d;
    }
    bool nan_row = false;
    const float scale = finish_scale_ln(block_reduce(d2, false, scratch), n, a.eps, nan_row);
    for (std::int64_t i = t; i < n; i += 256) {
      float r = nan_row ? __builtin_nanf("") : (x[i] - mean) * scale;
      if (a.gamma) r = r * a.gamma[i];
      if (a.beta) r = r + a.beta[i];
      out[i] = r;
    }
    return;
  }
}

// Strided rows: one lane per (outer, inner) row in the reference's order.
template <RowOp kOp>
__global__ __launch_bounds__(256) void row_lane_kernel(RowArgs a, std::int64_t reduce, std::int64_t inner) {
  const std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= a.rows) return;  // rows = outer * inner
  const std::int64_t base = (id / inner) * reduce * inner + id % inner;
  const float* __restrict__ x = a.x + base;
  float* __restrict__ out = a.out + base;
  if constexpr (kOp == RowOp::kSoftmax) {
    float m = -__builtin_inff();
    for (std::int64_t r = 0; r < reduce; ++r) {
      const float e = x[r * inner];
      if (is_nan(e)) {
        m = e;
        break;
      }
      m = (m < e) ? e : m;
    }
    float denom = 0.F;
    for (std::int64_t r = 0; r < reduce; ++r) denom += expf(x[r * inner] - m);
    for (std::int64_t r = 0; r < reduce; ++r) out[r * inner] = expf(x[r * inner] - m) / denom;
  } else if constexpr (kOp == RowOp::kRms) {
    float ss = 0.F;
    for (std::int64_t r = 0; r < reduce; ++r) {
      const float e = x[r * inner];
      const float sq = e * e;
      ss += sq;
    }
    const float scale = 1.0F / sqrtf(ss / static_cast<float>(reduce) + a.eps);
    for (std::int64_t r = 0; r < reduce; ++r) {
      float t = x[r * inner] * scale;
      if (a.gamma) t = t * a.gamma[r];
      out[r * inner] = t;
    }
  } else {
    const float first = x[0];
    float s = 0.F;
    bool equal = true;
    for (std::int64_t r = 0; r < reduce; ++r) {
      const float e = x[r * inner];
      s += e;
      equal = equal && e == first;
    }
    if (equal && __builtin_isfinite(first)) {
      const float fillv = a.eps == 0.F ? __builtin_nanf("") : 0.F;
      for (std::int64_t r = 0; r < reduce; ++r) {
        float t = fillv;
        if (a.gamma) t = t * a.gamma[r];
        if (a.beta) t = t + a.beta[r];
        out[r * inner] = t;
      }
      return;
    }
    const float mean = s / static_cast<float>(reduce);
    float d2 = 0.F;
    for (std::int64_t r = 0; r < reduce; ++r) {
      const float d = x[r * inner] - mean;
      d2 += d * d;
    }
    bool nan_row = false;
    const float scale = finish_scale_ln(d2, reduce, a.eps, nan_row);
    for (std::int64_t r = 0; r < reduce; ++r) {
      float t = nan_row ? __builtin_nanf("") : (x[r * inner] - mean) * scale;
      if (a.gamma) t = t * a.gamma[r];
      if (a.beta) t = t + a.beta[r];
      out[r * inner] = t;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }

template <RowOp kOp, int kChunks>
void launch_cached(const RowArgs& a, bool vec, hipStream_t s) {
  const dim3 grid(grid_for(a.rows, 4, 0x7fffffff));
  if (vec)
    hipLaunchKernelGGL((row_cached_kernel<kOp, kChunks, true>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((row_cached_kernel<kOp, kChunks, false>), grid, dim3(256), 0, s, a);
}

template <RowOp kOp>
int run_rows(RowArgs a, std::int64_t outer, std::int64_t reduce, std::int64_t inner, hipStream_t s) {
  if (outer == 0 || reduce == 0 || inner == 0) return TCX_OK;
  const int status = ready();
  if (status != TCX_OK) return status;
  if (inner != 1) {
    a.rows = outer * inner;
    hipLaunchKernelGGL((row_lane_kernel<kOp>), dim3(grid_for(a.rows, 256, 0x7fffffff)), dim3(256), 0, s,
                       a, reduce, inner);
    return check(hipGetLastError(), "row lane kernel launch");
  }
  a.rows = outer;
  a.n = reduce;
  const bool vec = reduce % 4 == 0 && aligned16(a.x) && aligned16(a.out) &&
                   (a.gamma == nullptr || aligned16(a.gamma)) && (a.beta == nullptr || aligned16(a.beta));
  const std::int64_t chunks = (reduce + 255) / 256;
  if (chunks > kMaxChunks) {
    if (outer > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "too many rows");
    hipLaunchKernelGGL((row_block_kernel<kOp>), dim3(static_cast<unsigned>(outer)), dim3(256), 0, s, a);
    return check(hipGetLastError(), "row block kernel launch");
  }
  if (chunks <= 1) launch_cached<kOp, 1>(a, vec, s);
  else if (chunks <= 2) launch_cached<kOp, 2>(a, vec, s);
  else if (chunks <= 4) launch_cached<kOp, 4>(a, vec, s);
  else if (chunks <= 8) launch_cached<kOp, 8>(a, vec, s);
  else if (chunks <= 16) launch_cached<kOp, 16>(a, vec, s);
  else launch_cached<kOp, 32>(a, vec, s);
  return check(hipGetLastError(), "row kernel launch");
}

int check_extents(std::int64_t outer, std::int64_t reduce, std::int64_t inner, const void* x, const void* out) {
  if (outer < 0 || reduce < 0 || inner < 0) return fail(TCX_INVALID_ARGUMENT, "row extents must be non-negative");
  if (outer && reduce && inner && (x == nullptr || out == nullptr))
    return fail(TCX_INVALID_ARGUMENT, "row op buffers are null");
  return TCX_OK;
}

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_softmax_f32(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner,
                        tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  RowArgs a{x, nullptr, nullptr, out, 0, 0, 0.F};
  return run_rows<RowOp::kSoftmax>(a, outer, reduce, inner, static_cast<hipStream_t>(stream));
}

int tcx_hip_rmsnorm_f32(const float* x, const float* gamma, float* out, int64_t outer, int64_t reduce,
                        int64_t inner, float eps, tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  if (!(eps >= 0.F) || __builtin_isinf(eps)) return fail(TCX_INVALID_ARGUMENT, "epsilon must be finite and non-negative");
  RowArgs a{x, gamma, nullptr, out, 0, 0, eps};
  return run_rows<RowOp::kRms>(a, outer, reduce, inner, static_cast<hipStream_t>(stream));
}

int tcx_hip_layernorm_f32(const float* x, const float* gamma, const float* beta, float* out, int64_t outer,
                          int64_t reduce, int64_t inner, float eps, tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  if (!(eps >= 0.F) || __builtin_isinf(eps)) return fail(TCX_INVALID_ARGUMENT, "epsilon must be finite and non-negative");
  RowArgs a{x, gamma, beta, out, 0, 0, eps};
  return run_rows<RowOp::kLayer>(a, outer, reduce, inner, static_cast<hipStream_t>(stream));
}

}  // extern "C"
