// Row softmax, RMSNorm and LayerNorm (reference cpu_backend.cpp:125-240), with
// the optional affine weight/bias of the kAffine*Norm composites
// (core/inference.cpp:103-122) fused into the same pass.
//
// Contiguous rows (inner == 1) stay in registers, so each element is read from
// HBM once and written once: rows of up to 1024 elements take one wave per row
// (kChunks 16-byte loads per lane, wave-wide butterfly statistics); rows of up
// to kMaxSplit elements take one 256-thread block per row (four waves, whose
// partial statistics meet in LDS). Longer rows use one block per row that
// re-reads the row (mostly from L2). Strided rows (inner > 1) use one lane per
// row in the reference's exact element order.
//
// Per-element arithmetic follows the reference step by step (exp(x - max),
// sum, division; (x - mean) * scale; x * scale), each step rounded separately
// (built with -ffp-contract=off). Statistics are summed in a fixed tree order,
// which stays within allclose(rtol=1e-5, atol=1e-5) of the sequential sums.

#include "common.hpp"

namespace tcx {
namespace {

constexpr int kMaxWaveChunks = 4;  // one wave per row up to 1024 floats
constexpr int kMaxSplit = 16;      // one block per row up to 256*4*16 floats

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

// One wave per row, row cached in registers (kChunks float4 per lane).
// Blocks are persistent: each of the grid's blocks walks rows
// blockIdx*4 + wave, stepping by the grid, so the affine weight and bias are
// staged into LDS once per block instead of being re-read for every row.
template <RowOp kOp, int kChunks, bool kVec, bool kFull>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void
row_cached_kernel(RowArgs a) {
  extern __shared__ float4_t affine4[];  // gamma [n] then beta [n], when present
  float* affine = reinterpret_cast<float*>(affine4);
  const int lane = threadIdx.x & 63;
  const std::int64_t n = a.n;
  const bool has_g = a.gamma != nullptr, has_b = a.beta != nullptr;
  if (has_g || has_b) {
    for (std::int64_t i = threadIdx.x; i < n; i += 256) {
      if (has_g) affine[i] = a.gamma[i];
      if (has_b) affine[n + i] = a.beta[i];
    }
    __syncthreads();
  }
  // Element (c, q) sits at column 4*(lane + 64c) + q (vector rows) or at
  // lane + 64*(4c + q) (scalar rows); columns >= n are masked. kFull rows
  // (n == 256 * kChunks, 16-byte aligned) have no masked elements.
  auto column = [&](int c, int q) -> int {
    return kVec ? 4 * (lane + 64 * c) + q : lane + 64 * (4 * c + q);
  };
  const int ni = static_cast<int>(n);
  auto valid = [&](int c, int q) -> bool {
    if constexpr (kFull) return true;
    return kVec ? column(c, 0) < ni : column(c, q) < ni;
  };
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
  for (std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row < a.rows;
       row += step) {
    const float* __restrict__ x = a.x + row * n;
    float* __restrict__ out = a.out + row * n;
    float v[kChunks][4];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if constexpr (kVec) {
        const int i = column(c, 0);
        float4_t t = {0.F, 0.F, 0.F, 0.F};
        if (valid(c, 0)) t = stream_load(reinterpret_cast<const float4_t*>(x + i));
        v[c][0] = t.x; v[c][1] = t.y; v[c][2] = t.z; v[c][3] = t.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v[c][q] = valid(c, q) ? x[column(c, q)] : 0.F;
        }
      }
    }

    if constexpr (kOp == RowOp::kSoftmax) {
      float m = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (valid(c, q) && (is_nan(v[c][q]) || v[c][q] > m)) m = v[c][q];
      m = wave_max_nan(m);
      float sum = 0.F;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (valid(c, q)) {
            v[c][q] = exp_softmax(v[c][q] - m);
            sum += v[c][q];
          }
        }
      // One correctly rounded reciprocal per row; each output is e * (1/denom),
      // within 1.5 ulp of the reference's e / denom.
      const float inv = 1.0F / wave_sum(sum);
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] * inv;
    } else if constexpr (kOp == RowOp::kRms) {
      float sum = 0.F;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t = v[c][q] * v[c][q];
          sum += t;  // masked elements are zero
        }
      const float ss = wave_sum(sum);
      const float scale = 1.0F / sqrtf(ss / static_cast<float>(n) + a.eps);
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] * scale;
    } else {
      const float first = x[0];
      float sum = 0.F;
      bool equal = true;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sum += v[c][q];
          if (valid(c, q)) equal = equal && v[c][q] == first;
        }
      const float mean = wave_sum(sum) / static_cast<float>(n);
      float d2 = 0.F;
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (valid(c, q)) {
            const float d = v[c][q] - mean;
            d2 += d * d;
          }
        }
      bool nan_row = false;
      const float scale = finish_scale_ln(wave_sum(d2), n, a.eps, nan_row);
      // Row-uniform special cases as selects: an all-equal finite row gives 0
      // (NaN when eps is 0); a zero variance + eps gives NaN.
      const bool const_row = __all(equal) && __builtin_isfinite(first);
      const bool special = const_row || nan_row;
      const float special_value = const_row && a.eps != 0.F ? 0.F : __builtin_nanf("");
#pragma unroll
      for (int c = 0; c < kChunks; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = special ? special_value : (v[c][q] - mean) * scale;
    }

    // Affine steps (multiply then add, each rounded) and the store.
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
      if constexpr (kVec) {
        const int i = column(c, 0);
        if (!valid(c, 0)) continue;
        float4_t t = {v[c][0], v[c][1], v[c][2], v[c][3]};
        if (has_g) {
          const float4_t g = affine4[i / 4];
          t.x = t.x * g.x; t.y = t.y * g.y; t.z = t.z * g.z; t.w = t.w * g.w;
        }
        if (has_b) {
          const float4_t b = affine4[(ni + i) / 4];
          t.x = t.x + b.x; t.y = t.y + b.y; t.z = t.z + b.z; t.w = t.w + b.w;
        }
        __builtin_nontemporal_store(t, reinterpret_cast<float4_t*>(out + i));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (!valid(c, q)) continue;
          const int i = column(c, q);
          float t = v[c][q];
          if (has_g) t = t * affine[i];
          if (has_b) t = t + affine[ni + i];
          out[i] = t;
        }
      }
    }
    // Keep the next row's loads from being hoisted into this row's live range.
    asm volatile("" ::: "memory");
  }
}

// One 256-thread block per row, the row cached in registers: thread t holds
// kPer float4 at columns 4*(t + 256c) (vector rows) or 4*kPer floats at
// t + 256*(4c + q) (scalar rows). Each wave reduces its part with butterflies
// and the four wave partials meet in LDS, combined in wave order. Blocks are
// persistent (a few per CU walk the rows, stepping by the grid), which keeps
// the set of rows in flight, and the HBM pages they touch, small. For kPer <= 4
// the affine weight and bias of a thread's columns stay in registers across
// rows; wider rows re-read them (L2-resident) for every row.
template <RowOp kOp, int kPer, bool kVec, bool kFull>
__global__ __launch_bounds__(256) void row_split_kernel(RowArgs a) {
  constexpr bool kAffRegs = kPer <= 4;
  // Statistics exchange, double-buffered by row parity so a wave that runs
  // ahead never overwrites a slot another wave has yet to read.
  __shared__ float red[2][2][4];  // [row parity][statistic][wave]
  __shared__ int same[2][4];      // LayerNorm all-equal flag per wave
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const std::int64_t n = a.n;
  const int ni = static_cast<int>(n);
  auto column = [&](int c, int q) -> int { return kVec ? 4 * (t + 256 * c) + q : t + 256 * (4 * c + q); };
  auto valid = [&](int c, int q) -> bool {
    if constexpr (kFull) return true;
    return kVec ? column(c, 0) < ni : column(c, q) < ni;
  };
  const bool has_g = a.gamma != nullptr, has_b = a.beta != nullptr;
  auto load_affine = [&](const float* p, int c, float fallback, float (&dst)[4]) {
    if constexpr (kVec) {
      float4_t w = {fallback, fallback, fallback, fallback};
      if (p != nullptr && valid(c, 0)) w = *reinterpret_cast<const float4_t*>(p + column(c, 0));
      dst[0] = w.x; dst[1] = w.y; dst[2] = w.z; dst[3] = w.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) dst[q] = (p != nullptr && valid(c, q)) ? p[column(c, q)] : fallback;
    }
  };
  float g[kAffRegs ? kPer : 1][4], b[kAffRegs ? kPer : 1][4];
  if constexpr (kAffRegs) {
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      load_affine(a.gamma, c, 1.F, g[c]);
      load_affine(a.beta, c, 0.F, b[c]);
    }
  }
  auto combine = [&](float v, int par, int stat, bool is_max) -> float {
    if (lane == 0) red[par][stat][wave] = v;
    __syncthreads();
    float r = red[par][stat][0];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float o = red[par][stat][w];
      r = is_max ? ((is_nan(o) || o > r) ? o : r) : r + o;
    }
    return r;
  };

  // Rows of up to 4 float4 per thread prefetch the block's next row into a
  // second register set while the current row reduces and stores (global
  // loads stay in flight across the barriers). Wider rows load in place.
  constexpr bool kPrefetch = kPer <= 4;
  auto load_row = [&](std::int64_t row, float (&dst)[kPer][4], float& first) {
    const float* __restrict__ x = a.x + row * n;
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      if constexpr (kVec) {
        float4_t q = {0.F, 0.F, 0.F, 0.F};
        if (valid(c, 0)) q = stream_load(reinterpret_cast<const float4_t*>(x + column(c, 0)));
        dst[c][0] = q.x; dst[c][1] = q.y; dst[c][2] = q.z; dst[c][3] = q.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[c][q] = valid(c, q) ? x[column(c, q)] : 0.F;
      }
    }
    if constexpr (kOp == RowOp::kLayer) first = x[0];
  };
  float v[kPer][4], nv[kPrefetch ? kPer : 1][4];
  float first = 0.F, next_first = 0.F;
  if (kPrefetch && blockIdx.x < a.rows) load_row(blockIdx.x, v, first);

  int par = 0;
  for (std::int64_t row = blockIdx.x; row < a.rows; row += gridDim.x, par ^= 1) {
    float* __restrict__ out = a.out + row * n;
    if constexpr (kPrefetch) {
      const std::int64_t next = row + gridDim.x;
      if (next < a.rows) load_row(next, nv, next_first);
    } else {
      load_row(row, v, first);
    }

    if constexpr (kOp == RowOp::kSoftmax) {
      float m = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (valid(c, q) && (is_nan(v[c][q]) || v[c][q] > m)) m = v[c][q];
      m = combine(wave_max_nan(m), par, 0, true);
      float sum = 0.F;
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (valid(c, q)) {
            v[c][q] = exp_softmax(v[c][q] - m);
            sum += v[c][q];
          }
        }
      // One correctly rounded reciprocal per row; each output is e * (1/denom),
      // within 1.5 ulp of the reference's e / denom.
      const float inv = 1.0F / combine(wave_sum(sum), par, 1, false);
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] * inv;
    } else if constexpr (kOp == RowOp::kRms) {
      float sum = 0.F;
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float sq = v[c][q] * v[c][q];
          sum += sq;  // masked elements are zero
        }
      const float ss = combine(wave_sum(sum), par, 0, false);
      const float scale = 1.0F / sqrtf(ss / static_cast<float>(n) + a.eps);
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = v[c][q] * scale;
    } else {
      float sum = 0.F;
      bool equal = true;
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sum += v[c][q];  // masked elements are zero
          if (valid(c, q)) equal = equal && v[c][q] == first;
        }
      const bool wave_equal = __all(equal);
      if (lane == 0) same[par][wave] = wave_equal ? 1 : 0;
      const float mean = combine(wave_sum(sum), par, 0, false) / static_cast<float>(n);
      const bool all_equal = same[par][0] && same[par][1] && same[par][2] && same[par][3];
      float d2 = 0.F;
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (valid(c, q)) {
            const float d = v[c][q] - mean;
            d2 += d * d;
          }
        }
      bool nan_row = false;
      const float scale = finish_scale_ln(combine(wave_sum(d2), par, 1, false), n, a.eps, nan_row);
      // Row-uniform special cases as selects: an all-equal finite row gives 0
      // (NaN when eps is 0); a zero variance + eps gives NaN.
      const bool const_row = all_equal && __builtin_isfinite(first);
      const bool special = const_row || nan_row;
      const float special_value = const_row && a.eps != 0.F ? 0.F : __builtin_nanf("");
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = special ? special_value : (v[c][q] - mean) * scale;
    }

    // Affine steps (multiply then add, each rounded) and the store.
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      float gc[4], bc[4];
      if constexpr (kAffRegs) {
#pragma unroll
        for (int q = 0; q < 4; ++q) { gc[q] = g[c][q]; bc[q] = b[c][q]; }
      } else {
        if (has_g) load_affine(a.gamma, c, 1.F, gc);
        if (has_b) load_affine(a.beta, c, 0.F, bc);
      }
      float r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        r[q] = v[c][q];
        if (has_g) r[q] = r[q] * gc[q];
        if (has_b) r[q] = r[q] + bc[q];
      }
      if constexpr (kVec) {
        if (!valid(c, 0)) continue;
        const float4_t o = {r[0], r[1], r[2], r[3]};
        __builtin_nontemporal_store(o, reinterpret_cast<float4_t*>(out + column(c, 0)));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (valid(c, q)) out[column(c, q)] = r[q];
      }
    }
    if constexpr (kPrefetch) {
#pragma unroll
      for (int c = 0; c < kPer; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) v[c][q] = nv[c][q];
      first = next_first;
    }
    // Keep later rows' loads from being hoisted into this row's live range.
    asm volatile("" ::: "memory");
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
  // Grid-stride over rows = outer * inner (the launcher caps the grid).
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; id < a.rows; id += step) {
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
        continue;
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
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }

// Persistent grid: as many blocks as fit on the device at once (cached per
// kernel instance and LDS size), never more than there are 4-row groups.
template <RowOp kOp, int kChunks, bool kVec, bool kFull>
void launch_cached_as(const RowArgs& a, hipStream_t s) {
  const std::size_t lds = (a.gamma || a.beta) ? static_cast<std::size_t>(2 * a.n) * sizeof(float) : 0;
  thread_local int cached_blocks = 0;
  thread_local std::size_t cached_lds = ~std::size_t{0};
  if (cached_lds != lds) {
    int per_cu = 0, cus = 0, device = 0;
    (void)hipGetDevice(&device);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, row_cached_kernel<kOp, kChunks, kVec, kFull>, 256, lds) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    cached_blocks = per_cu * (cus > 0 ? cus : 256);
    cached_lds = lds;
  }
  const std::int64_t groups = (a.rows + 3) / 4;
  const unsigned grid = static_cast<unsigned>(groups < cached_blocks ? groups : cached_blocks);
  hipLaunchKernelGGL((row_cached_kernel<kOp, kChunks, kVec, kFull>), dim3(grid), dim3(256), lds, s, a);
}

// Persistent split grid: kSplitBlocksPerCu blocks per CU (fewer if the
// occupancy calculator allows fewer), never more than there are rows. A few
// blocks per CU keep enough loads in flight while the rows being streamed at
// any moment stay close together.
constexpr int kSplitBlocksPerCu = 3;

template <RowOp kOp, int kPer, bool kVec, bool kFull>
void launch_split_as(const RowArgs& a, hipStream_t s) {
  thread_local int cached_blocks = 0;
  if (cached_blocks == 0) {
    int per_cu = 0, cus = 0, device = 0;
    (void)hipGetDevice(&device);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, row_split_kernel<kOp, kPer, kVec, kFull>, 256, 0) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    if (per_cu > kSplitBlocksPerCu) per_cu = kSplitBlocksPerCu;
    cached_blocks = per_cu * (cus > 0 ? cus : 256);
  }
  const unsigned grid = static_cast<unsigned>(a.rows < cached_blocks ? a.rows : cached_blocks);
  hipLaunchKernelGGL((row_split_kernel<kOp, kPer, kVec, kFull>), dim3(grid), dim3(256), 0, s, a);
}

// Scalar (unaligned) rows keep one address per element live, so only rows of
// up to kMaxScalarSplit float4 per thread use the split kernel unaligned.
constexpr int kMaxScalarSplit = 4;

template <RowOp kOp, int kPer>
int launch_split(const RowArgs& a, bool vec, hipStream_t s) {
  if (vec && a.n == 1024 * kPer) {
    launch_split_as<kOp, kPer, true, true>(a, s);
  } else if (vec) {
    launch_split_as<kOp, kPer, true, false>(a, s);
  } else {
    if constexpr (kPer > kMaxScalarSplit) return fail(TCX_INTERNAL, "unaligned row too wide for the split kernel");
    else launch_split_as<kOp, kPer, false, false>(a, s);
  }
  return check(hipGetLastError(), "row kernel launch");
}

template <RowOp kOp, int kChunks>
void launch_cached(const RowArgs& a, bool vec, hipStream_t s) {
  if (vec && a.n == 256 * kChunks)
    launch_cached_as<kOp, kChunks, true, true>(a, s);
  else if (vec)
    launch_cached_as<kOp, kChunks, true, false>(a, s);
  else
    launch_cached_as<kOp, kChunks, false, false>(a, s);
}

template <RowOp kOp>
int run_rows(RowArgs a, std::int64_t outer, std::int64_t reduce, std::int64_t inner, hipStream_t s) {
  if (outer == 0 || reduce == 0 || inner == 0) return TCX_OK;
  const int status = ready();
  if (status != TCX_OK) return status;
  if (inner != 1) {
    a.rows = outer * inner;
    hipLaunchKernelGGL((row_lane_kernel<kOp>), dim3(grid_for(a.rows, 256, kStrideBlocks)), dim3(256), 0, s,
                       a, reduce, inner);
    return check(hipGetLastError(), "row lane kernel launch");
  }
  a.rows = outer;
  a.n = reduce;
  const bool vec = reduce % 4 == 0 && aligned16(a.x) && aligned16(a.out) &&
                   (a.gamma == nullptr || aligned16(a.gamma)) && (a.beta == nullptr || aligned16(a.beta));
  const std::int64_t chunks = (reduce + 255) / 256;  // per lane, one wave per row
  const std::int64_t per = (reduce + 1023) / 1024;    // per thread, one block per row
  if (chunks <= 1) launch_cached<kOp, 1>(a, vec, s);
  else if (chunks <= 2) launch_cached<kOp, 2>(a, vec, s);
  else if (chunks <= kMaxWaveChunks) launch_cached<kOp, 4>(a, vec, s);
  else if (per <= 2) return launch_split<kOp, 2>(a, vec, s);
  else if (per <= 4) return launch_split<kOp, 4>(a, vec, s);
  else if (vec && per <= 8) return launch_split<kOp, 8>(a, vec, s);
  else if (vec && per <= kMaxSplit) return launch_split<kOp, 16>(a, vec, s);
  else {
    // Rows wider than the register budget (or unaligned rows wider than
    // kMaxScalarSplit float4 per thread): one block per row, re-read passes.
    if (outer > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "too many rows");
    hipLaunchKernelGGL((row_block_kernel<kOp>), dim3(static_cast<unsigned>(outer)), dim3(256), 0, s, a);
    return check(hipGetLastError(), "row block kernel launch");
  }
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
