// Row softmax, RMSNorm and LayerNorm (reference cpu_backend.cpp:125-240), with
// the optional affine weight/bias of the kAffine*Norm composites
// (core/inference.cpp:103-122) fused into the same pass.
//
// Contiguous rows (inner == 1) stay in registers, so each element is read from
// HBM once and written once: rows of up to 1536 elements take L lanes each,
// 64 / L rows per wave (row_group_kernel, 16-byte loads at any alignment,
// butterfly statistics over the row's lanes); rows of
// up to 3072 elements (4096 with an affine weight or bias) take one 256-thread
// block per row (four waves, whose partial statistics meet in LDS). Longer
// rows take one 512-thread block per row that holds the whole row in
// registers, from about 41 K floats with the rest in LDS (two blocks per CU
// to about 61 K, 69 K for LayerNorm; one, with more registers, past 90 K)
// (row_resident_kernel, to about 139 K floats); longer ones one 1024-thread
// block per row that reads it once per pass (row_block_kernel).
// Strided rows (inner > 1) run
// col_norm_kernel: column tiles whose waves fold per-column statistics over
// runs of rows, then write the row from them in a second walk (rows split
// over blocks, with a workspace, when tiles are few).
//
// Per-element arithmetic follows the reference step by step (exp(x - max),
// sum, division; (x - mean) * scale; x * scale), each step rounded separately
// (built with -ffp-contract=off). Statistics are summed in a fixed tree order,
// which stays within allclose(rtol=1e-5, atol=1e-5) of the sequential sums.

#include <algorithm>

#include "common.hpp"

namespace tcx {
namespace {

constexpr std::int64_t kGroupMax = 1536;  // row_group_kernel up to this length
constexpr int kMaxSplit = 4;       // one block per row up to 256*4*4 floats

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

// Statistics of a row held by a group of L lanes (L a power of two, aligned
// groups): butterflies in which both partners add the same operands, so the
// row's lanes agree bit for bit.
__device__ __forceinline__ float group_sum(float v, int L) {
  for (int offset = L >> 1; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}
__device__ __forceinline__ float group_max_nan(float v, int L) {
  for (int offset = L >> 1; offset > 0; offset >>= 1) {
    const float o = __shfl_xor(v, offset, kWave);
    v = (is_nan(o) || o > v) ? o : v;
  }
  return v;
}
__device__ __forceinline__ bool group_all(bool v, int L) {
  int f = v ? 1 : 0;
  for (int offset = L >> 1; offset > 0; offset >>= 1) f &= __shfl_xor(f, offset, kWave);
  return f != 0;
}

// One 256-thread block per row, the row cached in registers: thread t holds
// kPer float4 at columns 4*(t + 256c) (vector rows) or 4*kPer floats at
// t + 256*(4c + q) (scalar rows). Each wave reduces its part with butterflies
// and the four wave partials meet in LDS, combined in wave order. Blocks are
// persistent (a few per CU walk the rows, stepping by the grid), which keeps
// the set of rows in flight, and the HBM pages they touch, small. The affine
// weight and bias of a thread's columns stay in registers across rows, and the
// block's next row loads into a second register set while the current one
// reduces and stores (global loads stay in flight across the barriers).
// Rows of 4 float4 per thread load and store non-temporally; rows of 2 (the
// 1537-2048 floats this kernel takes there) with the default policy:
// [8192, 2048] LayerNorm + weight/bias 25.5 -> 22.4 us, softmax 25.9 ->
// 23.0, where [16384, 4096] LayerNorm + weight/bias lost 87.1 -> 92.6 us
// without the non-temporal hint.
template <RowOp kOp, int kPer, bool kVec, bool kFull>
__global__ __launch_bounds__(256) void row_split_kernel(RowArgs a) {
  static_assert(kPer <= kMaxSplit, "two register copies of the row and the affine terms per thread");
  constexpr bool kNT = kPer > 2;
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
  float g[kPer][4], b[kPer][4];
#pragma unroll
  for (int c = 0; c < kPer; ++c) {
    load_affine(a.gamma, c, 1.F, g[c]);
    load_affine(a.beta, c, 0.F, b[c]);
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

  auto load_row = [&](std::int64_t row, float (&dst)[kPer][4], float& first) {
    const float* __restrict__ x = a.x + row * n;
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      if constexpr (kVec) {
        float4_t q = {0.F, 0.F, 0.F, 0.F};
        if (valid(c, 0)) {
          const auto* src = reinterpret_cast<const float4_t*>(x + column(c, 0));
          q = kNT ? stream_load(src) : *src;
        }
        dst[c][0] = q.x; dst[c][1] = q.y; dst[c][2] = q.z; dst[c][3] = q.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) dst[c][q] = valid(c, q) ? x[column(c, q)] : 0.F;
      }
    }
    if constexpr (kOp == RowOp::kLayer) first = x[0];
  };
  float v[kPer][4], nv[kPer][4];
  float first = 0.F, next_first = 0.F;
  if (blockIdx.x < a.rows) load_row(blockIdx.x, v, first);

  int par = 0;
  for (std::int64_t row = blockIdx.x; row < a.rows; row += gridDim.x, par ^= 1) {
    float* __restrict__ out = a.out + row * n;
    const std::int64_t next = row + gridDim.x;
    if (next < a.rows) load_row(next, nv, next_first);

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
      float r[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        r[q] = v[c][q];
        if (has_g) r[q] = r[q] * g[c][q];
        if (has_b) r[q] = r[q] + b[c][q];
      }
      if constexpr (kVec) {
        if (!valid(c, 0)) continue;
        const float4_t o = {r[0], r[1], r[2], r[3]};
        auto* dst = reinterpret_cast<float4_t*>(out + column(c, 0));
        if constexpr (kNT) __builtin_nontemporal_store(o, dst);
        else *dst = o;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (valid(c, q)) out[column(c, q)] = r[q];
      }
    }
#pragma unroll
    for (int c = 0; c < kPer; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) v[c][q] = nv[c][q];
    first = next_first;
    // Keep later rows' loads from being hoisted into this row's live range.
    asm volatile("" ::: "memory");
  }
}

// Block-wide maximum (NaN first) or sum of one value per thread.
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

// Threads of the long-row block: 1024 keep four times the loads of 256 in
// flight per row, which matters when a few hundred rows fill the GPU.
constexpr int kRowBlockThreads = 1024;
constexpr int kNonTemporal = 2;  // buffer instruction cache policy: nt

// Walks row x[0, n) with the kRowBlockThreads threads of a block: the elements before
// x's first 16-byte boundary (threads 0-2, f1(value, i)), whole float4s four
// deep per thread (f4(vector, i) for elements i .. i + 3, all four loads of
// a round issued before any is used), then the last elements (threads 0-2).
// Scalar loads one per iteration ran [1000, 100003] softmax at 14 % of HBM.
template <typename F4, typename F1>
__device__ __forceinline__ void block_row_walk(const float* __restrict__ x, std::int64_t n, F4&& f4, F1&& f1) {
  const int t = threadIdx.x;
  std::int64_t head = static_cast<std::int64_t>(((16U - (reinterpret_cast<std::uintptr_t>(x) & 15U)) & 15U) / 4);
  if (head > n) head = n;
  const std::int64_t vectors = (n - head) / 4;
  const float4_t* __restrict__ body = reinterpret_cast<const float4_t*>(x + head);
  std::int64_t k = t;
  constexpr int T = kRowBlockThreads;
  for (; k + 3 * T < vectors; k += 4 * T) {
    const float4_t a = stream_load(body + k), b = stream_load(body + k + T), c = stream_load(body + k + 2 * T),
                   d = stream_load(body + k + 3 * T);
    f4(a, head + 4 * k);
    f4(b, head + 4 * (k + T));
    f4(c, head + 4 * (k + 2 * T));
    f4(d, head + 4 * (k + 3 * T));
  }
  float4_t last[3];
#pragma unroll
  for (int u = 0; u < 3; ++u)
    if (k + T * u < vectors) last[u] = stream_load(body + k + T * u);
#pragma unroll
  for (int u = 0; u < 3; ++u)
    if (k + T * u < vectors) f4(last[u], head + 4 * (k + T * u));
  if (t < head) f1(x[t], static_cast<std::int64_t>(t));
  const std::int64_t tail = head + 4 * vectors;
  if (t < n - tail) f1(x[tail + t], tail + t);
}

// exp(d) for -150 <= d <= 88 (the caller clamps): 2^t exp(r) with
// t = d log2(e) and r = d - t ln(2) taken in two parts (Cody and Waite), so
// that exp(r) = 1 + r to within 2^-35 (|r| < 2^-16). Within 1.5 ulp of exp(d)
// where the result is normal; 0 below 2^-126 (and at d = -150).
__device__ __forceinline__ float exp_reduced(float d) {
  constexpr float kLog2e = 1.44269502F;
  constexpr float kLn2Hi = 0.693145752F;    // 0x3f317200: ln 2 to 16 bits
  constexpr float kLn2Lo = 1.42860677e-6F;  // ln 2 - kLn2Hi
  const float t = d * kLog2e;
  const float e = __builtin_amdgcn_exp2f(t);
  const float r = fmaf(-t, kLn2Lo, fmaf(-t, kLn2Hi, d));
  return fmaf(e, r, e);
}

// Rows longer than a CU's registers and LDS hold (past about 139 K floats):
// one block per row, passes over the row read from HBM each time (softmax: a
// running maximum and rescaled sum, write; RMSNorm: sum of squares, write;
// LayerNorm: sum, squared deviations, write).
template <RowOp kOp>
__global__ __launch_bounds__(kRowBlockThreads) void row_block_kernel(RowArgs a) {
  constexpr int kWaves = kRowBlockThreads / 64;
  __shared__ float scratch[kWaves];
  __shared__ int eq_flag;
  const std::int64_t row = blockIdx.x;
  const std::int64_t n = a.n;
  const float* __restrict__ x = a.x + row * n;
  float* __restrict__ out = a.out + row * n;
  auto walk = [&](auto&& f4, auto&& f1) { block_row_walk(x, n, f4, f1); };
  // Writes f(value) for every element of the row, times the weight and plus
  // the bias when present, as float4 at x's float4 offsets (16-byte buffer
  // accesses need only 4-byte alignment in out, gamma and beta).
  const float* __restrict__ g = a.gamma;
  const float* __restrict__ b = a.beta;
  auto rsrc_of = [&](const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                             static_cast<int>(4 * n), 0x00020000);
  };
  auto write_row = [&](auto&& f) {
    if (n >= (std::int64_t{1} << 29)) {  // past 32-bit buffer offsets: element by element
      walk(
          [&](const float4_t& v, std::int64_t i) {
            const float q[4] = {v.x, v.y, v.z, v.w};
            for (int e = 0; e < 4; ++e) {
              float r = f(q[e]);
              if (g) r = r * g[i + e];
              if (b) r = r + b[i + e];
              out[i + e] = r;
            }
          },
          [&](float v, std::int64_t i) {
            float r = f(v);
            if (g) r = r * g[i];
            if (b) r = r + b[i];
            out[i] = r;
          });
      return;
    }
    const auto o_rsrc = rsrc_of(out);
    const auto g_rsrc = rsrc_of(g ? g : out);
    const auto b_rsrc = rsrc_of(b ? b : out);
    using b128_t = decltype(__builtin_amdgcn_raw_buffer_load_b128(o_rsrc, 0, 0, 0));
    walk(
        [&](const float4_t& v, std::int64_t i) {
          float4_t r = {f(v.x), f(v.y), f(v.z), f(v.w)};
          const int off = static_cast<int>(4 * i);
          if (g) {
            const auto gv = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, off, 0, 0));
            r = float4_t{r.x * gv.x, r.y * gv.y, r.z * gv.z, r.w * gv.w};
          }
          if (b) {
            const auto bv = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, off, 0, 0));
            r = float4_t{r.x + bv.x, r.y + bv.y, r.z + bv.z, r.w + bv.w};
          }
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128_t, r), o_rsrc, off, 0, kNonTemporal);
        },
        [&](float v, std::int64_t i) {
          float r = f(v);
          if (g) r = r * g[i];
          if (b) r = r + b[i];
          out[i] = r;
        });
  };
  if constexpr (kOp == RowOp::kSoftmax) {
    // One read pass for the maximum and the sum: each thread keeps (m, s),
    // s relative to its running maximum m and rescaled when m grows (a sum
    // begun under m = -inf starts over). A separate maximum pass read every
    // row three times: [1000, 100000] 284 us at 35 % of HBM.
    float m = -__builtin_inff(), s = 0.F;
    auto grow = [&](float top) {
      if ((is_nan(top) && !is_nan(m)) || top > m) {
        s = m == -__builtin_inff() ? 0.F : s * exp_softmax(m - top);
        m = top;
      }
    };
    auto nan_max = [](float p, float q) { return (is_nan(q) || q > p) ? q : p; };
    walk(
        [&](const float4_t& v, std::int64_t) {
          grow(nan_max(nan_max(v.x, v.y), nan_max(v.z, v.w)));
          s += (exp_softmax(v.x - m) + exp_softmax(v.y - m)) + (exp_softmax(v.z - m) + exp_softmax(v.w - m));
        },
        [&](float v, std::int64_t) {
          grow(v);
          s += exp_softmax(v - m);
        });
    // Merge (m, s) over the wave, then the block's waves in order.
    auto merge = [&](float om, float os) {
      const float top = nan_max(m, om);
      if (top == -__builtin_inff()) {
        s = s + os;
      } else {
        const float mine = m == -__builtin_inff() ? 0.F : s * exp_softmax(m - top);
        const float other = om == -__builtin_inff() ? 0.F : os * exp_softmax(om - top);
        s = mine + other;
      }
      m = top;
    };
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) merge(__shfl_xor(m, offset, kWave), __shfl_xor(s, offset, kWave));
    __shared__ float wave_ms[2][kWaves];
    if ((threadIdx.x & 63) == 0) {
      wave_ms[0][threadIdx.x >> 6] = m;
      wave_ms[1][threadIdx.x >> 6] = s;
    }
    __syncthreads();
    m = wave_ms[0][0];
    s = wave_ms[1][0];
    for (int w = 1; w < kWaves; ++w) merge(wave_ms[0][w], wave_ms[1][w]);
    // One correctly rounded reciprocal per row; each output is e * (1/denom),
    // within 1.5 ulp of the reference's e / denom.
    const float inv = 1.0F / s;
    write_row([&](float v) { return exp_softmax(v - m) * inv; });
  } else if constexpr (kOp == RowOp::kRms) {
    float s0 = 0.F, s1 = 0.F;
    walk(
        [&](const float4_t& v, std::int64_t) { s0 += v.x * v.x + v.y * v.y; s1 += v.z * v.z + v.w * v.w; },
        [&](float v, std::int64_t) { s0 += v * v; });
    const float ss = block_reduce(s0 + s1, false, scratch);
    const float scale = 1.0F / sqrtf(ss / static_cast<float>(n) + a.eps);
    write_row([&](float v) { return v * scale; });
  } else {
    if (threadIdx.x == 0) eq_flag = 1;
    const float first = x[0];
    float s0 = 0.F, s1 = 0.F;
    bool equal = true;
    walk(
        [&](const float4_t& v, std::int64_t) {
          s0 += v.x + v.y;
          s1 += v.z + v.w;
          equal = equal && v.x == first && v.y == first && v.z == first && v.w == first;
        },
        [&](float v, std::int64_t) {
          s0 += v;
          equal = equal && v == first;
        });
    const float mean = block_reduce(s0 + s1, false, scratch) / static_cast<float>(n);
    if (!equal) eq_flag = 0;
    __syncthreads();
    if (eq_flag && __builtin_isfinite(first)) {
      const float fillv = a.eps == 0.F ? __builtin_nanf("") : 0.F;
      write_row([&](float) { return fillv; });
      return;
    }
    float d0 = 0.F, d1 = 0.F;
    walk(
        [&](const float4_t& v, std::int64_t) {
          const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
          d0 += dx * dx + dy * dy;
          d1 += dz * dz + dw * dw;
        },
        [&](float v, std::int64_t) {
          const float d = v - mean;
          d0 += d * d;
        });
    bool nan_row = false;
    const float scale = finish_scale_ln(block_reduce(d0 + d1, false, scratch), n, a.eps, nan_row);
    write_row([&](float v) { return nan_row ? __builtin_nanf("") : (v - mean) * scale; });
  }
}

// Rows too long for one block's LDS and up to about 139 K floats: one block
// of T threads per row (512, or 1024 for the widest softmax and RMSNorm
// rows) holds the whole row, its first 4 T P floats (after the elements
// before its first 16-byte boundary) in registers, float4 k = t + T c in
// thread t's v[c], and the rest in LDS, loaded straight from HBM
// (buffer_load ... lds) in 1 KB wave chunks, chunk j by wave j mod (T / 64),
// so that each lane reads back only what its own loads wrote and no barrier
// is needed. A CU's registers (512 KB) and LDS (160 KB) together hold such a
// row, so it is read from HBM once and written once.
//
// One row per CU at a time leaves no other block to overlap the row's
// arithmetic with its loads, so the first statistics pass takes each float4
// as it arrives: the LDS chunks (issued first, so landing first), then the
// register chunks in order. For softmax that pass already takes the
// exponentials, against the maximum m0 of the wave's first register float4s
// (256 elements): e = exp(x - m0) in place, and the thread's sum of them. The
// block maximum M then rescales: denom = sum over threads of
// sum_t * exp(m0_t - M) in a fixed order, out = e * (exp(m0_t - M) / denom).
// A thread whose own maximum lies more than kResidentShift above m0 reloads
// its elements from HBM before any output is written and takes them against
// its own maximum, so e stays below exp(32) and exp(m0_t - M) keeps the
// precision of the outputs that matter; on ordinary data no thread does (one
// that did stalled its row for several microseconds). A row whose maximum is
// not finite (a NaN, +inf, or -inf throughout) is NaN throughout, as in the
// reference.
//
// Loads and stores go through buffer resources (one address register for the
// row, range-checked: float4s past the row read as zero and are not stored).
// The affine weight and bias (which of them is present is a template
// argument) are read as float4 beside each output float4.
constexpr int kResidentThreads = 512;
constexpr float kResidentShift = 32.0F;
constexpr int kAffGamma = 1, kAffBeta = 2;


// One wave's 1 KB load from HBM straight into LDS at lds (a wave-uniform
// address): lane l's 16 bytes at byte voffset of r land at lds + 16 l.
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0,
                                           kNonTemporal);
}

// Waves per SIMD a block of P float4 per thread leaves room for: rows held in
// 12 or 20 float4 per thread (at most 24576 or 40960 floats in registers,
// up to kPairLdsChunks KB more in LDS) run three or two blocks per CU, so one
// row's arithmetic overlaps another's loads, and so does 24 (LayerNorm rows
// held partly in LDS); 4 or 8 (rows of 3073 to 8192 or 16384 floats) four.
constexpr int resident_waves_per_eu(int P) { return P <= 8 ? 8 : P <= 12 ? 6 : P <= 24 ? 4 : 2; }

// LDS per block (1 KB chunks of 64 float4) for rows held at 20 or 24 float4
// per thread plus LDS: two blocks, with their static arrays, fit in the
// 160 KB of a CU.
constexpr int kPairLdsChunks = 79;

// Rows past the two-block routes: 1024 threads of 24 float4 (16 waves per
// CU, at most 128 VGPRs) plus LDS, to 139008 floats. With inputs rotated,
// against the 512 threads of 44 float4 that held these rows before (the same
// register share, 8 waves): softmax [512, 128256] 98.1 -> 91.9 us, [1000,
// 100003] 164.7 -> 157.5, [300, 130000] 77.0 -> 66.3; RMSNorm [512, 128256]
// 94.8 -> 92.7, [2048, 70000] 210.7 -> 203.3; RMSNorm + weight [512,
// 128256] 98.3 -> 97.3; LayerNorm + weight/bias [512, 128256] 104.5 ->
// 101.5, [2048, 70000] 234.7 -> 224.8, [256, 139000] (re-read before) 100.7
// -> 59.2. LayerNorm fits only with the block folds' LDS reads fenced four
// at a time (12 dwords spilled before: [512, 128256] 110.4 us).
constexpr int kWideThreads = 1024;
constexpr int kWideVec = 24;

template <RowOp kOp, int kAff, int P, int kT = kResidentThreads>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(resident_waves_per_eu(P))))
void row_resident_kernel(RowArgs a) {
  constexpr int T = kT, kWaves = T / 64;
  constexpr bool kG = (kAff & kAffGamma) != 0, kB = (kAff & kAffBeta) != 0;
  extern __shared__ float4_t rest4[];
  __shared__ float scratch[kWaves];
  __shared__ int equal_waves[kWaves];
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const std::int64_t row = blockIdx.x;
  const int n = static_cast<int>(a.n);  // below 2^29 (the launcher checks)
  const float* __restrict__ x = a.x + row * a.n;
  float* __restrict__ out = a.out + row * a.n;
  int head = static_cast<int>(((16U - (reinterpret_cast<std::uintptr_t>(x) & 15U)) & 15U) / 4);
  if (head > n) head = n;
  const int vectors = (n - head) / 4, tail = head + 4 * vectors;
  const int first = T * P;  // float4s from here on are in LDS
  const int lds_chunks = vectors > first ? (vectors - first + 63) / 64 : 0;
  auto rsrc_of = [](const float* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), bytes, 0x00020000);
  };
  const auto x_rsrc = rsrc_of(x + head, vectors * 16);
  using b128_t = decltype(__builtin_amdgcn_raw_buffer_load_b128(x_rsrc, 0, 0, 0));
  auto load4 = [&](int k) {
    return __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, k * 16, 0, kNonTemporal));
  };
  // Thread t's index, copied opaquely for each pass over the register
  // chunks: the compiler would otherwise keep all P chunk offsets live from
  // the loads to the stores.
  auto opaque_t = [&] {
    int u = t;
    asm volatile("" : "+v"(u));
    return u;
  };

  // LDS chunks first (they land first), then the register part, then the
  // elements before the first 16-byte boundary and after the last whole
  // float4 (threads 0-2, clamped loads used only where in range). A partial
  // last LDS chunk reads zero past the row, into LDS the launch reserves.
  for (int j = wave; j < lds_chunks; j += kWaves)
    load_lds16(x_rsrc, rest4 + 64 * j, (first + 64 * j + lane) * 16);
  float4_t v[P];
#pragma unroll
  for (int c = 0; c < P; ++c) v[c] = load4(t + T * c);
  const bool has_h = t < head, has_t = t < n - tail;
  float hv = x[has_h ? t : 0], tv = x[has_t ? tail + t : 0];
  // Register chunks below full are in range for every thread (a uniform
  // test), chunk full only for some.
  const int full = vectors / T < P ? vectors / T : P;
  auto in_regs = [&](int c) { return c < full || (c == full && t + T * c < vectors); };

  // Applies f(float4&, float4 index) to this thread's float4s (its LDS slots,
  // then its registers in arrival order) and g(float&) to its head and tail
  // elements.
  auto for_each = [&](auto&& f, auto&& g) {
    for (int j = wave; j < lds_chunks; j += kWaves)
      if (first + 64 * j + lane < vectors) f(rest4[64 * j + lane]);
    // An opaque copy of full per pass: the per-chunk tests are then scalar
    // compares used once, not P lane masks the compiler keeps across passes.
    int f_full = full;
    asm volatile("" : "+s"(f_full));
#pragma unroll
    for (int c = 0; c < P; ++c) {
      if (c < f_full) {
        f(v[c]);
      } else if (c == f_full && t + T * c < vectors) {
        f(v[c]);
      }
    }
    if (has_h) g(hv);
    if (has_t) g(tv);
  };
  auto block_sum = [&](float s) {
    s = wave_sum(s);
    if (lane == 0) scratch[wave] = s;
    __syncthreads();
    // The waves' sums in wave order, at most four LDS reads in flight: all
    // sixteen at once (1024 threads) kept 16 VGPRs live beside the row and
    // made LayerNorm spill.
    float r = scratch[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      r += scratch[w];
      if (w % 4 == 3) asm volatile("" ::: "memory");
    }
    __syncthreads();  // scratch is reused
    return r;
  };

  // Writes r(value) for every element, times the weight and plus the bias.
  // The output, weight and bias float4s sit at x's float4 offsets, which are
  // 16-byte aligned in x but only 4-byte aligned in the others when they
  // start at another offset within 16 bytes: a 16-byte buffer access needs
  // only 4-byte alignment.
  const float* __restrict__ gamma = a.gamma;
  const float* __restrict__ beta = a.beta;
  auto write = [&](auto&& r) {
    auto aff1 = [&](float q, int i) {
      if constexpr (kG) q = q * gamma[i];
      if constexpr (kB) q = q + beta[i];
      return q;
    };
    const auto o_rsrc = rsrc_of(out + head, vectors * 16);
    const auto g_rsrc = rsrc_of(kG ? gamma + head : out + head, vectors * 16);
    const auto b_rsrc = rsrc_of(kB ? beta + head : out + head, vectors * 16);
    auto put = [&](const float4_t& q, int k) {
      float4_t o = {r(q.x), r(q.y), r(q.z), r(q.w)};
      if constexpr (kG) {
        const auto g = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, k * 16, 0, 0));
        o = float4_t{o.x * g.x, o.y * g.y, o.z * g.z, o.w * g.w};
      }
      if constexpr (kB) {
        const auto b = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, k * 16, 0, 0));
        o = float4_t{o.x + b.x, o.y + b.y, o.z + b.z, o.w + b.w};
      }
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128_t, o), o_rsrc, k * 16, 0, kNonTemporal);
    };
    for (int j = wave; j < lds_chunks; j += kWaves) put(rest4[64 * j + lane], first + 64 * j + lane);
    if constexpr (kOp == RowOp::kRms && kG && (P == 12 || P == 20)) {
      // RMSNorm with a weight at 12 or 20 float4 per thread, in two phases:
      // the outputs times the weight replace the row in registers, four
      // chunks at a time (two at 20) with no store among their loads, then
      // every output float4 is stored back to back. Each group's results
      // pass through an opaque step with a memory clobber before the next
      // group's loads, so the compiler neither sinks the products below later
      // loads nor keeps every weight float4 live (which spilled). With inputs
      // rotated past the Infinity Cache, against one chunk at a time and the
      // grouped form below: [4096, 32000] 186.6 -> 174.0 us, [4096, 20001]
      // 125.1 -> 122.3 us, outputs unchanged. LayerNorm, whose extra state
      // left too few registers ([4096, 32000] 182.4 -> 205.0 us with spills),
      // and 44 float4 per thread ([512, 128256] RMSNorm + weight 98.6 -> 99.1
      // us) keep the other forms.
      constexpr int kPhase = P == 20 ? 2 : 4;
#pragma unroll
      for (int c0 = 0; c0 < P; c0 += kPhase) {
#pragma unroll
        for (int c = c0; c < c0 + kPhase; ++c) {
          const int k = opaque_t() + T * c;
          const auto g = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, k * 16, 0, 0));
          const float4_t q = v[c];
          v[c] = float4_t{r(q.x) * g.x, r(q.y) * g.y, r(q.z) * g.z, r(q.w) * g.w};
        }
#pragma unroll
        for (int c = c0; c < c0 + kPhase; ++c) asm volatile("" : "+v"(v[c]) : : "memory");
      }
#pragma unroll
      for (int c = 0; c < P; ++c)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128_t, v[c]), o_rsrc, (opaque_t() + T * c) * 16, 0,
                                               kNonTemporal);  // past the row: not stored
    } else if constexpr ((kG || kB) && P <= 12) {
      // Weight and bias of kGroup chunks are loaded before any of their
      // stores: a load cannot move above an earlier buffer store (the
      // compiler takes them to alias), so one chunk at a time waited an L2
      // round trip per store. With inputs rotated past the Infinity Cache:
      // [8192, 5120] LayerNorm + weight/bias 62.7 -> 60.4 us, [2048, 12288]
      // RMSNorm + weight 36.5 -> 34.9, [4096, 20001] LayerNorm 129.8 ->
      // 127.8; at 20 and 44 float4 per thread it lost as often as it won
      // ([4096, 32000] LayerNorm 182.2 -> 186.9, [1000, 100003] 175.7 ->
      // 181.6 us).
      constexpr int kGroup = 4;
      const int u = opaque_t();
#pragma unroll
      for (int c0 = 0; c0 < P; c0 += kGroup) {
        float4_t gw[kGroup], bw[kGroup];
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
          if (c0 + g >= P) break;
          const int k = u + T * (c0 + g);
          if constexpr (kG)
            gw[g] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(g_rsrc, k * 16, 0, 0));
          if constexpr (kB)
            bw[g] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, k * 16, 0, 0));
        }
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
          if (c0 + g >= P) break;
          const float4_t& q = v[c0 + g];
          float4_t o = {r(q.x), r(q.y), r(q.z), r(q.w)};
          if constexpr (kG) o = float4_t{o.x * gw[g].x, o.y * gw[g].y, o.z * gw[g].z, o.w * gw[g].w};
          if constexpr (kB) o = float4_t{o.x + bw[g].x, o.y + bw[g].y, o.z + bw[g].z, o.w + bw[g].w};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128_t, o), o_rsrc, (u + T * (c0 + g)) * 16, 0,
                                                 kNonTemporal);  // past the row: not stored
        }
      }
    } else {
#pragma unroll
      for (int c = 0, u = opaque_t(); c < P; ++c) put(v[c], u + T * c);  // past the row: not stored
    }
    if (has_h) out[t] = aff1(r(hv), t);
    if (has_t) out[tail + t] = aff1(r(tv), tail + t);
  };

  if constexpr (kOp == RowOp::kSoftmax) {
    // NaN-propagating maxima (v_maximum3_f32): a NaN anywhere makes M NaN.
    auto vmax = [](float p, float q) { return __builtin_elementwise_maximum(p, q); };
    auto max4 = [&](float m, const float4_t& q) { return vmax(vmax(vmax(vmax(m, q.x), q.y), q.z), q.w); };
    // The reference maximum m0 is the wave's over its first float4s (v[0] is
    // in range: the row has more than T float4s).
    float m0 = wave_max_nan(max4(v[0].x, v[0]));
    float mt = m0, s0 = 0.F, s1 = 0.F;
    // Clamped at -150 (exp 0): -inf elements give exactly 0; a NaN is caught
    // by the maximum instead.
    auto ex = [](float d) { return exp_reduced(fmaxf(d, -150.F)); };
    auto exps = [&](float4_t& q, float m) {
      q = float4_t{ex(q.x - m), ex(q.y - m), ex(q.z - m), ex(q.w - m)};
      s0 += q.x + q.y;
      s1 += q.z + q.w;
    };
    for_each(
        [&](float4_t& q) {
          mt = max4(mt, q);
          exps(q, m0);
        },
        [&](float& q) {
          mt = vmax(mt, q);
          q = ex(q - m0);
          s0 += q;
        });
    if (mt - m0 > kResidentShift && __builtin_isfinite(mt)) {
      // Reload and take the exponentials against the thread's own maximum.
      m0 = mt;
      s0 = 0.F;
      s1 = 0.F;
      for (int j = wave; j < lds_chunks; j += kWaves)
        if (first + 64 * j + lane < vectors) {
          float4_t q = load4(first + 64 * j + lane);
          exps(q, m0);
          rest4[64 * j + lane] = q;
        }
#pragma unroll
      for (int c = 0, u = opaque_t(); c < P; ++c)
        if (in_regs(c)) {
          v[c] = load4(u + T * c);
          exps(v[c], m0);
        }
      if (has_h) {
        hv = ex(x[t] - m0);
        s0 += hv;
      }
      if (has_t) {
        tv = ex(x[tail + t] - m0);
        s0 += tv;
      }
    }
    float m = wave_max_nan(mt);
    if (lane == 0) scratch[wave] = m;
    __syncthreads();
    m = scratch[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      m = vmax(m, scratch[w]);
      if (w % 4 == 3) asm volatile("" ::: "memory");
    }
    __syncthreads();
    if (!__builtin_isfinite(m)) {
      write([](float) { return __builtin_nanf(""); });
      return;
    }
    const float w = ex(m0 - m);  // 0 for a thread of -inf only (m0 = -inf)
    // One correctly rounded reciprocal per row.
    const float f = w * (1.0F / block_sum((s0 + s1) * w));
    write([&](float e) { return e * f; });
  } else if constexpr (kOp == RowOp::kRms) {
    float s0 = 0.F, s1 = 0.F;
    for_each([&](const float4_t& q) { s0 += q.x * q.x + q.y * q.y; s1 += q.z * q.z + q.w * q.w; },
             [&](float q) { s0 += q * q; });
    const float scale = 1.0F / sqrtf(block_sum(s0 + s1) / static_cast<float>(n) + a.eps);
    write([&](float q) { return q * scale; });
  } else {
    const float x0 = x[0];
    float s0 = 0.F, s1 = 0.F;
    bool equal = true;
    for_each(
        [&](const float4_t& q) {
          s0 += q.x + q.y;
          s1 += q.z + q.w;
          equal = equal && q.x == x0 && q.y == x0 && q.z == x0 && q.w == x0;
        },
        [&](float q) {
          s0 += q;
          equal = equal && q == x0;
        });
    const bool wave_equal = __all(equal);  // all 64 lanes vote: outside the lane-0 branch
    if (lane == 0) equal_waves[wave] = wave_equal ? 1 : 0;
    const float mean = block_sum(s0 + s1) / static_cast<float>(n);
    bool all_equal = true;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      all_equal = all_equal && equal_waves[w] != 0;
      if (w % 4 == 3) asm volatile("" ::: "memory");
    }
    if (all_equal && __builtin_isfinite(x0)) {
      // An all-equal finite row: 0, or NaN when eps is 0 (cpu_backend.cpp:205-213).
      const float fill = a.eps == 0.F ? __builtin_nanf("") : 0.F;
      write([&](float) { return fill; });
      return;
    }
    float d0 = 0.F, d1 = 0.F;
    for_each(
        [&](const float4_t& q) {
          const float dx = q.x - mean, dy = q.y - mean, dz = q.z - mean, dw = q.w - mean;
          d0 += dx * dx + dy * dy;
          d1 += dz * dz + dw * dw;
        },
        [&](float q) {
          const float d = q - mean;
          d0 += d * d;
        });
    bool nan_row = false;
    const float scale = finish_scale_ln(block_sum(d0 + d1), n, a.eps, nan_row);
    write([&](float q) { return nan_row ? __builtin_nanf("") : (q - mean) * scale; });
  }
}

// ------------------------------------------------------------ strided rows
// Row ops over a middle axis (inner > 1), x as [outer, R, inner]: the row of
// (outer o, column j) is R elements, inner apart. A column tile is W columns
// (64 lanes x 4 with 16-byte loads when inner is a multiple of 4 and x and
// out are 16-byte aligned, else x 1; or the power of two at or above a
// narrower inner, the wave then stepping G = 64 x kVec / W rows at a time).
// A block of kNormWaves waves takes one (split, tile) pair; its waves take
// the split's row groups in turn (as the column reductions) and lane (g, c)
// of wave w walks rows rb + w G + g + i G kNormWaves of column c with
// kNormDepth rows loaded at once.
//
// Column statistics fold lane -> row groups (butterfly) -> waves (LDS, in
// order) -> splits (in order); then each element is written from them in a
// last walk over the rows. Softmax takes one statistics walk (a running
// maximum with its rescaled sum of exponentials), RMSNorm one (sum of
// squares), LayerNorm two as the reference: the sum, then the squared
// deviations from the rounded mean, which a near-constant row's output
// depends on. With one split (col_norm_kernel kMode 0) one block does every
// walk; with several, statistics launches (kMode 1) write per-split
// statistics to the workspace, col_norm_finalize_kernel folds them into
// per-column parameters, and a write launch (kMode 2) reads those.
constexpr int kNormWaves = 8;
constexpr int kNormDepth = 8;
constexpr std::int64_t kNormTargetBlocks = 512;  // two 8-wave blocks per CU on 256 CUs
constexpr std::int64_t kNormMinRows = 64;        // rows per split, times G
constexpr std::int64_t kNormMaxWorkspace = std::int64_t{16} << 20;

// Statistics of one column over some of its rows:
//   softmax  a = running maximum m (NaN once a NaN is seen), b = sum of
//            e^(x - m) over the elements other than -inf (rescaled when m
//            grows), so the row's denominator is sum_p b_p e^(m_p - M)
//   rms      a = sum of x^2
//   layer    walk 0: a = sum of x, c = a value of the rows, n bit 31 set
//            while every element equals c (n counts rows); walk 1: a = sum of
//            (x - mean)^2
struct NormStat {
  float a, b, c;
  std::uint32_t n;
};
constexpr std::uint32_t kAllEqual = 0x80000000U;

// Per-column parameters of the write walk: softmax (m, 1 / denominator);
// rms (scale); layer (mean, scale), or a fill value for a row of equal
// finite elements (0; NaN when eps is 0) or a zero variance + eps (NaN).
struct NormParams {
  float p0, p1, fill;
  int special;
};

struct ColNormArgs {
  const float* x;
  const float* gamma;
  const float* beta;
  float* out;
  NormStat* stats;     // [splits][outer * inner] (kMode 1)
  NormParams* params;  // [outer * inner] (kMode 1 walk 1, kMode 2)
  std::int64_t outer, R, inner, split_rows, splits, blocks;
  float eps;
  int W;
  int walk;            // kMode 1: LayerNorm's statistics walk (0 or 1)
};

template <RowOp kOp>
__device__ __forceinline__ NormStat empty_stat() {
  if constexpr (kOp == RowOp::kSoftmax) return NormStat{-__builtin_inff(), 0.F, 0.F, 0U};
  else return NormStat{0.F, 0.F, 0.F, kAllEqual};
}

// Folds statistics b (of later rows) into a.
template <RowOp kOp>
__device__ __forceinline__ void fold_stat(NormStat& a, const NormStat& b) {
  if constexpr (kOp == RowOp::kSoftmax) {
    if (is_nan(a.a)) return;
    if (is_nan(b.a)) {
      a = b;
      return;
    }
    const float m = a.a < b.a ? b.a : a.a;
    // A side with no element other than -inf adds nothing (its b is 0, and
    // e^(-inf - m) would be NaN when m is -inf too).
    const float ta = a.a == -__builtin_inff() ? 0.F : a.b * exp_softmax(a.a - m);
    const float tb = b.a == -__builtin_inff() ? 0.F : b.b * exp_softmax(b.a - m);
    a.a = m;
    a.b = ta + tb;
  } else if constexpr (kOp == RowOp::kRms) {
    a.a = a.a + b.a;
  } else {
    const std::uint32_t na = a.n & ~kAllEqual, nb = b.n & ~kAllEqual;
    if (nb == 0) return;
    if (na == 0) {
      a = b;
      return;
    }
    const bool equal = (a.n & kAllEqual) && (b.n & kAllEqual) && a.c == b.c;
    a.a = a.a + b.a;
    a.n = (na + nb) | (equal ? kAllEqual : 0U);
  }
}

template <RowOp kOp>
__device__ __forceinline__ NormStat shfl_stat(const NormStat& v, int off) {
  NormStat r;
  r.a = __shfl_xor(v.a, off, kWave);
  r.b = kOp == RowOp::kSoftmax ? __shfl_xor(v.b, off, kWave) : 0.F;
  r.c = kOp == RowOp::kLayer ? __shfl_xor(v.c, off, kWave) : 0.F;
  r.n = kOp == RowOp::kLayer ? static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(v.n), off, kWave)) : 0U;
  return r;
}

// Parameters from a column's folded statistics: for LayerNorm, walk 0 sets
// the mean and the equal-row fill, walk 1 the scale (into p, which holds
// walk 0's parameters).
template <RowOp kOp>
__device__ __forceinline__ void norm_params(NormParams& p, const NormStat& st, int walk, std::int64_t R, float eps) {
  if constexpr (kOp == RowOp::kSoftmax) {
    p = NormParams{st.a, 1.0F / st.b, 0.F, 0};  // one correctly rounded reciprocal, as the row kernels
  } else if constexpr (kOp == RowOp::kRms) {
    p = NormParams{1.0F / sqrtf(st.a / static_cast<float>(R) + eps), 0.F, 0.F, 0};
  } else if (walk == 0) {
    const bool const_row = (st.n & kAllEqual) && __builtin_isfinite(st.c);
    p = NormParams{st.a / static_cast<float>(R), 0.F, const_row && eps != 0.F ? 0.F : __builtin_nanf(""),
                   const_row ? 1 : 0};
  } else {
    bool nan_row = false;
    p.p1 = finish_scale_ln(st.a, R, eps, nan_row);
    if (nan_row && !p.special) {
      p.special = 1;
      p.fill = __builtin_nanf("");
    }
  }
}

template <RowOp kOp, int kVec, int kMode>
__device__ __forceinline__ void col_norm_block(const ColNormArgs& a, std::int64_t b,
                                               NormStat (&lds)[kNormWaves][64 * kVec],
                                               NormParams (&params)[64 * kVec]) {
  const int W = a.W;
  const int G = 64 * kVec / W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lanes_per_row = W / kVec;
  const int g = lane / lanes_per_row, cl = (lane % lanes_per_row) * kVec;
  const int t = threadIdx.x;
  const std::int64_t inner = a.inner, R = a.R;
  const std::int64_t tiles_per_outer = (inner + W - 1) / W;
  const std::int64_t col_tiles = a.outer * tiles_per_outer;
  const std::int64_t split = b / col_tiles, tile = b % col_tiles;
  const std::int64_t o = tile / tiles_per_outer, tile_col = (tile % tiles_per_outer) * W;
  const std::int64_t rb = split * a.split_rows, re = min(R, rb + a.split_rows);
  // This lane's rows: row0, row0 + GS, ... below re, GS = G x kNormWaves
  // (the block's waves take row groups in turn, streaming neighbouring rows
  // together).
  const std::int64_t GS = static_cast<std::int64_t>(G) * kNormWaves;
  const std::int64_t row0 = rb + wave * G + g;
  const std::int64_t n = row0 < re ? (re - row0 + GS - 1) / GS : 0;
  // Lanes past the last column read the last kVec columns (in bounds: inner
  // is a multiple of kVec) and store nothing.
  const std::int64_t j = tile_col + cl;
  const bool col_in = j < inner;
  const bool t_in = t < W && tile_col + t < inner;  // thread t folds column tile_col + t
  const std::int64_t offset = o * R * inner + row0 * inner + (col_in ? j : inner - kVec);
  const float* __restrict__ xb = a.x + offset;
  const std::int64_t step = GS * inner;
  auto load_row = [&](std::int64_t i, float (&v)[kVec]) {
    if constexpr (kVec == 4) {
      const float4_t q = stream_load(reinterpret_cast<const float4_t*>(xb + i * step));
      v[0] = q.x;
      v[1] = q.y;
      v[2] = q.z;
      v[3] = q.w;
    } else {
      v[0] = stream_load(xb + i * step);
    }
  };

  // One statistics walk over this lane's rows, folded to column t's block
  // statistics (valid for t_in threads; the call is block-wide).
  auto stats_walk = [&](int walk, const float (&mean)[kVec]) -> NormStat {
    NormStat st[kVec];
#pragma unroll
    for (int c = 0; c < kVec; ++c) st[c] = empty_stat<kOp>();
    float first[kVec];
    if (kOp == RowOp::kLayer && walk == 0 && n > 0) {
      load_row(0, first);
#pragma unroll
      for (int c = 0; c < kVec; ++c) st[c].c = first[c];
    }
    for (std::int64_t i = 0; i < n; i += kNormDepth) {
      float v[kNormDepth][kVec];
#pragma unroll
      for (int u = 0; u < kNormDepth; ++u) load_row(min(i + u, n - 1), v[u]);  // clamped past the run
#pragma unroll
      for (int c = 0; c < kVec; ++c) {
        if constexpr (kOp == RowOp::kSoftmax) {
          float bm = st[c].a;
#pragma unroll
          for (int u = 0; u < kNormDepth; ++u)
            if (i + u < n && (is_nan(v[u][c]) || v[u][c] > bm)) bm = v[u][c];
          if (is_nan(bm)) {
            st[c].a = st[c].b = bm;
          } else {
            if (bm > st[c].a) {
              st[c].b = st[c].b * exp_softmax(st[c].a - bm);
              st[c].a = bm;
            }
#pragma unroll
            for (int u = 0; u < kNormDepth; ++u)
              if (i + u < n && v[u][c] != -__builtin_inff()) st[c].b += exp_softmax(v[u][c] - st[c].a);
          }
        } else if constexpr (kOp == RowOp::kRms) {
#pragma unroll
          for (int u = 0; u < kNormDepth; ++u)
            if (i + u < n) {
              const float sq = v[u][c] * v[u][c];
              st[c].a += sq;
            }
        } else if (walk == 0) {
#pragma unroll
          for (int u = 0; u < kNormDepth; ++u)
            if (i + u < n) {
              st[c].a += v[u][c];
              if (v[u][c] != first[c]) st[c].n &= ~kAllEqual;
            }
        } else {
#pragma unroll
          for (int u = 0; u < kNormDepth; ++u)
            if (i + u < n) {
              const float d = v[u][c] - mean[c];
              const float dd = d * d;
              st[c].a += dd;
            }
        }
      }
    }
    if constexpr (kOp == RowOp::kLayer) {
#pragma unroll
      for (int c = 0; c < kVec; ++c) st[c].n = (st[c].n & kAllEqual) | static_cast<std::uint32_t>(n);
    }
    // Row groups of the wave: a butterfly over the lane bits above the
    // column, each pair folded in row order (group 0 ends with the wave's).
    for (int off = lanes_per_row; off < 64; off <<= 1) {
#pragma unroll
      for (int c = 0; c < kVec; ++c) {
        const NormStat other = shfl_stat<kOp>(st[c], off);
        if (g & (off / lanes_per_row)) {
          NormStat mine = other;
          fold_stat<kOp>(mine, st[c]);
          st[c] = mine;
        } else {
          fold_stat<kOp>(st[c], other);
        }
      }
    }
    if (g == 0) {
#pragma unroll
      for (int c = 0; c < kVec; ++c) lds[wave][cl + c] = st[c];
    }
    __syncthreads();
    NormStat total = empty_stat<kOp>();
    if (t_in) {
      total = lds[0][t];
#pragma unroll
      for (int w = 1; w < kNormWaves; ++w) fold_stat<kOp>(total, lds[w][t]);
    }
    __syncthreads();  // lds is free again
    return total;
  };

  const float no_mean[kVec] = {};
  if constexpr (kMode == 1) {
    float mean[kVec] = {};
    if (kOp == RowOp::kLayer && a.walk == 1) {
#pragma unroll
      for (int c = 0; c < kVec; ++c) mean[c] = a.params[o * inner + (col_in ? j : inner - kVec) + c].p0;
    }
    const NormStat total = stats_walk(a.walk, mean);
    if (t_in) a.stats[split * a.outer * inner + o * inner + tile_col + t] = total;
    return;
  } else if constexpr (kMode == 0) {
    const NormStat total = stats_walk(0, no_mean);
    if (t_in) norm_params<kOp>(params[t], total, 0, R, a.eps);
    if constexpr (kOp == RowOp::kLayer) {
      __syncthreads();
      float mean[kVec];
#pragma unroll
      for (int c = 0; c < kVec; ++c) mean[c] = params[cl + c].p0;
      const NormStat dev = stats_walk(1, mean);
      if (t_in) norm_params<kOp>(params[t], dev, 1, R, a.eps);
    }
  } else {
    if (t_in) params[t] = a.params[o * inner + tile_col + t];
  }
  __syncthreads();

  // The write walk over this lane's rows.
  NormParams pc[kVec];
#pragma unroll
  for (int c = 0; c < kVec; ++c) pc[c] = params[cl + c];
  float* __restrict__ ob = a.out + offset;
  for (std::int64_t i = 0; i < n; i += kNormDepth) {
    float v[kNormDepth][kVec];
#pragma unroll
    for (int u = 0; u < kNormDepth; ++u) load_row(min(i + u, n - 1), v[u]);
#pragma unroll
    for (int u = 0; u < kNormDepth; ++u) {
      if (i + u >= n) continue;
      const std::int64_t r = row0 + (i + u) * GS;
      const float gr = a.gamma ? a.gamma[r] : 1.F;
      const float br = a.beta ? a.beta[r] : 0.F;
      float y[kVec];
#pragma unroll
      for (int c = 0; c < kVec; ++c) {
        float e;
        if constexpr (kOp == RowOp::kSoftmax) {
          e = exp_softmax(v[u][c] - pc[c].p0) * pc[c].p1;
        } else if constexpr (kOp == RowOp::kRms) {
          e = v[u][c] * pc[c].p0;
        } else {
          e = pc[c].special ? pc[c].fill : (v[u][c] - pc[c].p0) * pc[c].p1;
        }
        // Affine steps (multiply then add, each rounded).
        if (a.gamma) e = e * gr;
        if (a.beta) e = e + br;
        y[c] = e;
      }
      if (!col_in) continue;
      float* __restrict__ q = ob + (i + u) * step;
      if constexpr (kVec == 4) {
        const float4_t o4 = {y[0], y[1], y[2], y[3]};
        __builtin_nontemporal_store(o4, reinterpret_cast<float4_t*>(q));
      } else {
        __builtin_nontemporal_store(y[0], q);
      }
    }
  }
}

// Folds each column's split statistics into its parameters: L lanes per
// column (a power of two up to 64, about eight splits each), lane k folding
// splits k, k + L, ... in order, then the L lanes by a butterfly.
template <RowOp kOp>
__global__ __launch_bounds__(256) void col_norm_finalize_kernel(const NormStat* __restrict__ stats,
                                                                NormParams* __restrict__ params,
                                                                std::int64_t outputs, std::int64_t splits,
                                                                std::int64_t R, float eps, int L, int walk) {
  const int k = threadIdx.x & (L - 1);
  const std::int64_t per_pass = static_cast<std::int64_t>(gridDim.x) * (blockDim.x / L);
  // Every lane runs the same passes (the butterfly needs the whole wave):
  // lanes past the last column fold a clamped one and store nothing.
  const std::int64_t passes = (outputs + per_pass - 1) / per_pass;
  for (std::int64_t pass = 0; pass < passes; ++pass) {
    const std::int64_t id0 = pass * per_pass + static_cast<std::int64_t>(blockIdx.x) * (blockDim.x / L) + threadIdx.x / L;
    const std::int64_t id = id0 < outputs ? id0 : outputs - 1;
    NormStat total = empty_stat<kOp>();
    std::int64_t sp = k;
    for (; sp + 7 * L < splits; sp += 8 * L) {
      NormStat q[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) q[u] = stats[(sp + u * L) * outputs + id];
#pragma unroll
      for (int u = 0; u < 8; ++u) fold_stat<kOp>(total, q[u]);
    }
    for (; sp < splits; sp += L) fold_stat<kOp>(total, stats[sp * outputs + id]);
    for (int off = 1; off < L; off <<= 1) fold_stat<kOp>(total, shfl_stat<kOp>(total, off));
    if (k == 0 && id0 < outputs) {
      NormParams p = walk == 1 ? params[id] : NormParams{};
      norm_params<kOp>(p, total, walk, R, eps);
      params[id] = p;
    }
  }
}

template <RowOp kOp, int kVec, int kMode>
__global__ __launch_bounds__(64 * kNormWaves) void col_norm_kernel(ColNormArgs a) {
  __shared__ NormStat lds[kNormWaves][64 * kVec];
  __shared__ NormParams params[64 * kVec];
  // Block-stride over (split, tile) pairs; the launcher caps the grid.
  for (std::int64_t b = blockIdx.x; b < a.blocks; b += gridDim.x) {
    col_norm_block<kOp, kVec, kMode>(a, b, lds, params);
    __syncthreads();  // lds and params are rewritten by the next pair
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }

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

// Scalar (unaligned) rows take the split kernel too, four floats per group
// (one float per load).
template <RowOp kOp, int kPer>
int launch_split(const RowArgs& a, bool vec, hipStream_t s) {
  if (vec && a.n == 1024 * kPer)
    launch_split_as<kOp, kPer, true, true>(a, s);
  else if (vec)
    launch_split_as<kOp, kPer, true, false>(a, s);
  else
    launch_split_as<kOp, kPer, false, false>(a, s);
  return check(hipGetLastError(), "row kernel launch");
}

// Columns of a strided tile: 64 x 4 with 16-byte loads, else 64; a
// narrower inner takes the power of two at or above it.
std::int64_t norm_width(std::int64_t inner, bool vec) {
  const std::int64_t full = vec ? 256 : 64;
  if (inner >= full) return full;
  std::int64_t w = 1;
  while (w < inner) w *= 2;
  return w;
}

struct NormPlan {
  std::int64_t splits, split_rows;
};

// Rows of a strided tile are split by doubling while tiles x splits is
// below kNormTargetBlocks, each split keeps at least kNormMinRows x G rows
// and the workspace (split statistics plus one parameter record per column)
// stays within kNormMaxWorkspace. Planned for 16-byte loads whenever inner
// is a multiple of 4, so the workspace query needs no pointers.
NormPlan plan_norm(std::int64_t outer, std::int64_t reduce, std::int64_t inner) {
  const bool vec = inner % 4 == 0;
  const std::int64_t width = norm_width(inner, vec);
  const std::int64_t g = (vec ? 256 : 64) / width;
  const std::int64_t tiles = outer * ((inner + width - 1) / width);
  const std::int64_t entry = static_cast<std::int64_t>(sizeof(NormStat));
  std::int64_t splits = 1;
  while (tiles * splits < kNormTargetBlocks && reduce / (2 * splits) >= kNormMinRows * g &&
         (2 * splits + 1) * outer * inner * entry <= kNormMaxWorkspace)
    splits *= 2;
  const std::int64_t rows = (reduce + splits - 1) / splits;
  return NormPlan{(reduce + rows - 1) / rows, rows};
}

std::int64_t norm_workspace(std::int64_t outer, std::int64_t reduce, std::int64_t inner) {
  if (outer <= 0 || reduce <= 0 || inner <= 1) return 0;
  const NormPlan plan = plan_norm(outer, reduce, inner);
  if (plan.splits == 1) return 0;
  return (plan.splits + 1) * outer * inner * static_cast<std::int64_t>(sizeof(NormStat));
}

template <RowOp kOp>
int run_cols(const RowArgs& r, std::int64_t outer, std::int64_t reduce, std::int64_t inner, void* workspace,
             std::size_t workspace_bytes, bool split, hipStream_t s) {
  NormPlan plan{1, reduce};
  if (split) plan = plan_norm(outer, reduce, inner);
  if (plan.split_rows / kNormWaves >= INT32_MAX)
    return fail(TCX_INVALID_ARGUMENT, "strided row op has too many rows per split");
  const std::int64_t outputs = outer * inner;
  NormStat* stats = nullptr;
  NormParams* params = nullptr;
  if (plan.splits > 1) {
    const std::int64_t need = norm_workspace(outer, reduce, inner);
    if (workspace == nullptr || workspace_bytes < static_cast<std::size_t>(need))
      return fail(TCX_INVALID_ARGUMENT, "row op workspace is smaller than tcx_hip_rownorm_workspace_bytes");
    stats = static_cast<NormStat*>(workspace);
    params = reinterpret_cast<NormParams*>(stats + plan.splits * outputs);
  }
  // 16-byte loads and stores need inner a multiple of 4 and aligned x and
  // out; gamma and beta are read one element per row. Otherwise the 4-byte
  // kernel runs with the same splits.
  const bool vec = inner % 4 == 0 && aligned16(r.x) && aligned16(r.out);
  const std::int64_t width = norm_width(inner, vec);
  const std::int64_t blocks = outer * ((inner + width - 1) / width) * plan.splits;
  ColNormArgs a{r.x, r.gamma, r.beta, r.out, stats, params, outer, reduce, inner, plan.split_rows, plan.splits,
                blocks, r.eps, static_cast<int>(width), 0};
  const dim3 grid(static_cast<unsigned>(blocks < kStrideBlocks ? blocks : kStrideBlocks));
  const dim3 block(64 * kNormWaves);
  auto launch = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, s, a); };
  if (plan.splits == 1) {
    vec ? launch(col_norm_kernel<kOp, 4, 0>) : launch(col_norm_kernel<kOp, 1, 0>);
    return check(hipGetLastError(), "strided row kernel launch");
  }
  int lanes = 1;  // about eight splits per lane, at most a wave per column
  while (lanes < 64 && 16 * lanes <= plan.splits) lanes *= 2;
  // Statistics walks, each folded into the parameters (LayerNorm: the sum,
  // then the squared deviations from the mean).
  for (int walk = 0; walk < (kOp == RowOp::kLayer ? 2 : 1); ++walk) {
    a.walk = walk;
    vec ? launch(col_norm_kernel<kOp, 4, 1>) : launch(col_norm_kernel<kOp, 1, 1>);
    int rc = check(hipGetLastError(), "strided row statistics launch");
    if (rc != TCX_OK) return rc;
    hipLaunchKernelGGL((col_norm_finalize_kernel<kOp>), dim3(grid_for(outputs * lanes, 256, kStrideBlocks)),
                       dim3(256), 0, s, stats, params, outputs, plan.splits, reduce, r.eps, lanes, walk);
    rc = check(hipGetLastError(), "strided row finalize launch");
    if (rc != TCX_OK) return rc;
  }
  vec ? launch(col_norm_kernel<kOp, 4, 2>) : launch(col_norm_kernel<kOp, 1, 2>);
  return check(hipGetLastError(), "strided row write launch");
}

// Calls f(kernel, affine bits) for each resident-row kernel of P float4 per
// thread (kT threads) that the op launches.
using RowKernel = void (*)(RowArgs);
template <RowOp kOp, int P, int kT = kResidentThreads, typename F>
void resident_variants(F&& f) {
  f(static_cast<RowKernel>(&row_resident_kernel<kOp, 0, P, kT>), 0);
  if constexpr (kOp != RowOp::kSoftmax)
    f(static_cast<RowKernel>(&row_resident_kernel<kOp, kAffGamma, P, kT>), kAffGamma);
  if constexpr (kOp == RowOp::kLayer) {
    f(static_cast<RowKernel>(&row_resident_kernel<kOp, kAffBeta, P, kT>), kAffBeta);
    f(static_cast<RowKernel>(&row_resident_kernel<kOp, kAffGamma | kAffBeta, P, kT>), kAffGamma | kAffBeta);
  }
}

// Rows of 1-1536 elements at any alignment: L lanes per row, 64 / L rows
// per wave; lane l of a row's group holds elements 4l + 4Lu .. + 3 (u < kV),
// read with 16-byte buffer loads (4-byte alignment suffices) through a
// resource based at the group's first row. Elements past the row are
// masked to zero; a float4 wholly past it is not loaded, and the one that
// crosses the row's end is stored element by element (whole float4s take
// 16-byte buffer stores), so no other row's elements are written. The
// waves are persistent (as many blocks as stay resident); at two shapes
// (below) they load their next row group into a second register set before
// the current group's reductions. Row statistics are butterflies over the
// group's L lanes, in the per-element steps of the other row kernels. Loads
// and stores take the default cache policy: with the non-temporal one, whose
// partial-line writes these rows make at every row boundary, [100000, 100]
// softmax ran 26.7 against 17.0 us and [1000000, 50] 108.1 against 89.4 us
// on MI355X (inputs rotated past the Infinity Cache).
template <RowOp kOp, int kL, int kV, int kAff>
__global__ __launch_bounds__(256) void row_group_kernel(RowArgs a) {
  constexpr int kRows = 64 / kL;
  constexpr int kOut = 0x7fffffff;
  constexpr bool kG = (kAff & kAffGamma) != 0, kB = (kAff & kAffBeta) != 0;
  using b128_t = unsigned int __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l = lane % kL, gr = lane / kL;
  const int n = static_cast<int>(a.n);  // at most 1536
  auto col = [&](int u) { return 4 * l + 4 * kL * u; };
  // The weight and bias go to LDS once per (persistent) block: gamma at 0,
  // beta at nq (n rounded up to 4), so both read as aligned float4s.
  extern __shared__ float4_t affine4[];
  float* const affine = reinterpret_cast<float*>(affine4);
  const int nq = (n + 3) / 4 * 4;
  if constexpr (kG || kB) {
    for (int i = threadIdx.x; i < n; i += 256) {
      if constexpr (kG) affine[i] = a.gamma[i];
      if constexpr (kB) affine[nq + i] = a.beta[i];
    }
    __syncthreads();
  }
  auto rsrc_at = [&](const float* base, std::int64_t row0, int nrows) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + row0 * a.n), static_cast<short>(0),
                                             nrows * n * 4, 0x00020000);
  };
  const std::int64_t groups = (a.rows + kRows - 1) / kRows;
  auto rows_in = [&](std::int64_t t) {
    const std::int64_t left = a.rows - t * kRows;
    return left < kRows ? static_cast<int>(left) : kRows;
  };
  auto load = [&](std::int64_t t, float (&v)[kV][4]) {
    const int nrows = rows_in(t);
    const auto r = rsrc_at(a.x, t * kRows, nrows);
    const bool live = gr < nrows;
#pragma unroll
    for (int u = 0; u < kV; ++u) {
      const int j0 = col(u);
      const int off = live && j0 < n ? (gr * n + j0) * 4 : kOut;
      const float4_t q = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
#pragma unroll
      for (int e = 0; e < 4; ++e) v[u][e] = j0 + e < n ? q[e] : 0.F;
    }
  };
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
  std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * 4 + wave;
  // The next group's loads go out before this group's reductions at 8 lanes
  // x 4 float4 and 64 x 6; other shapes measured as fast or faster loading in
  // place (with inputs rotated past the Infinity Cache: [100000, 100] softmax
  // 16.9 against 20.6 us with and without, [8192, 1500] 19.1 against 20.8;
  // [16384, 1023] 27.0 against 25.0, [25000, 700] 26.9 against 25.4).
  constexpr bool kPrefetch = (kL == 8 && kV == 4) || kV == 6;
  float v[kV][4], nv[kPrefetch ? kV : 1][4];
  if (kPrefetch && t < groups) load(t, v);
  for (; t < groups; t += step) {
    if constexpr (kPrefetch) {
      if (t + step < groups) load(t + step, nv);
    } else {
      load(t, v);
    }
    const int nrows = rows_in(t);
    const bool live = gr < nrows;
    auto valid = [&](int u, int e) { return col(u) + e < n; };
    if constexpr (kOp == RowOp::kSoftmax) {
      float m = -__builtin_inff();
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (valid(u, e) && (is_nan(v[u][e]) || v[u][e] > m)) m = v[u][e];
      m = group_max_nan(m, kL);
      float sum = 0.F;
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (valid(u, e)) {
            v[u][e] = exp_softmax(v[u][e] - m);
            sum += v[u][e];
          }
      const float inv = 1.0F / group_sum(sum, kL);
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = v[u][e] * inv;
    } else if constexpr (kOp == RowOp::kRms) {
      float sum = 0.F;
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sq = v[u][e] * v[u][e];
          sum += sq;  // masked elements are zero
        }
      const float scale = 1.0F / sqrtf(group_sum(sum, kL) / static_cast<float>(n) + a.eps);
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = v[u][e] * scale;
    } else {
      // Element 0 of the row sits in the group's first lane.
      const float first = __shfl(v[0][0], lane & ~(kL - 1), kWave);
      float sum = 0.F;
      bool equal = true;
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum += v[u][e];  // masked elements are zero
          if (valid(u, e)) equal = equal && v[u][e] == first;
        }
      const float mean = group_sum(sum, kL) / static_cast<float>(n);
      float d2 = 0.F;
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (valid(u, e)) {
            const float d = v[u][e] - mean;
            d2 += d * d;
          }
      bool nan_row = false;
      const float scale = finish_scale_ln(group_sum(d2, kL), n, a.eps, nan_row);
      const bool const_row = group_all(equal, kL) && __builtin_isfinite(first);
      const bool special = const_row || nan_row;
      const float special_value = const_row && a.eps != 0.F ? 0.F : __builtin_nanf("");
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = special ? special_value : (v[u][e] - mean) * scale;
    }
    // Affine steps (multiply then add, each rounded) and the store.
    const auto o = rsrc_at(a.out, t * kRows, nrows);
#pragma unroll
    for (int u = 0; u < kV; ++u) {
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[e] = v[u][e];
      }
      const int j0 = col(u);
      if constexpr (kG) {
        const float4_t w = affine4[j0 / 4];  // past n: unset lanes of LDS, not stored
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = r[e] * w[e];
      }
      if constexpr (kB) {
        const float4_t w = affine4[nq / 4 + j0 / 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = r[e] + w[e];
      }
      if (!live || j0 >= n) continue;
      const int off = (gr * n + j0) * 4;
      if (j0 + 4 <= n) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(b128_t, float4_t{r[0], r[1], r[2], r[3]}), o, off,
                                               0, 0);
      } else {
#pragma unroll
        for (int e = 0; e < 3; ++e)
          if (j0 + e < n) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, r[e]), o, off + 4 * e, 0,
                                                                0);
      }
    }
    if constexpr (kPrefetch) {
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[u][e] = nv[u][e];
    }
    // Keep later groups' loads from being hoisted into this group's live range.
    asm volatile("" ::: "memory");
  }
}

template <RowOp kOp, int kL, int kV, int kAff>
void launch_group_as(const RowArgs& a, hipStream_t s) {
  const std::size_t lds = (kAff != 0 ? 2 : 0) * static_cast<std::size_t>((a.n + 3) / 4 * 4) * sizeof(float);
  thread_local int cached_blocks = 0;
  if (cached_blocks == 0) {
    int per_cu = 0, cus = 0, device = 0;
    (void)hipGetDevice(&device);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, row_group_kernel<kOp, kL, kV, kAff>, 256,
                                                     kAff != 0 ? 2 * kGroupMax * 4 : 0) !=
            hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    cached_blocks = per_cu * (cus > 0 ? cus : 256);
  }
  const std::int64_t groups = (a.rows + 64 / kL - 1) / (64 / kL);
  const std::int64_t need = (groups + 3) / 4;
  const unsigned grid = static_cast<unsigned>(need < cached_blocks ? need : cached_blocks);
  hipLaunchKernelGGL((row_group_kernel<kOp, kL, kV, kAff>), dim3(grid), dim3(256), lds, s, a);
}

template <RowOp kOp, int kL, int kV>
void launch_group(const RowArgs& a, hipStream_t s) {
  const int aff = (a.gamma ? kAffGamma : 0) + (a.beta ? kAffBeta : 0);
  if (aff == 0) launch_group_as<kOp, kL, kV, 0>(a, s);
  if constexpr (kOp != RowOp::kSoftmax)
    if (aff == kAffGamma) launch_group_as<kOp, kL, kV, kAffGamma>(a, s);
  if constexpr (kOp == RowOp::kLayer) {
    if (aff == kAffBeta) launch_group_as<kOp, kL, kV, kAffBeta>(a, s);
    if (aff == (kAffGamma | kAffBeta)) launch_group_as<kOp, kL, kV, kAffGamma | kAffBeta>(a, s);
  }
}

// (L, kV): up to 64 elements one float4 per lane (L = n / 4 rounded up to a
// power of two, 64 / L rows per wave), then the smallest that covers the row,
// as for the packed reductions, except 193-256 at 32 x 2 ([65536, 200]
// softmax 24.0 -> 20.0 us against 16 x 4). Against lanes of one float4 (or
// four floats at k, k + L, ... for unaligned rows) with non-temporal loads
// and stores, inputs rotated past the Infinity Cache: [1000000, 50] softmax
// 105.7 -> 93.9 us, [4194304, 8] LayerNorm 53.0 -> 44.9, softmax 45.6 ->
// 42.8. Two float4 per lane from 33 elements lost at 50 and 63 (105 -> 112
// and 121 -> 138 us); 8 x 5-6 for 129-192 and 16 x 5-6 for 257-384 lost
// ([100000, 130] softmax 24.2 -> 26.6 us, [50000, 300] 22.9 -> 25.5,
// [40000, 350] LayerNorm 21.9 -> 27.2) but at [65536, 180] softmax.
template <RowOp kOp>
void launch_group_for(const RowArgs& a, std::int64_t n, hipStream_t s) {
  if (n <= 4) launch_group<kOp, 1, 1>(a, s);
  else if (n <= 8) launch_group<kOp, 2, 1>(a, s);
  else if (n <= 16) launch_group<kOp, 4, 1>(a, s);
  else if (n <= 32) launch_group<kOp, 8, 1>(a, s);
  else if (n <= 64) launch_group<kOp, 16, 1>(a, s);
  else if (n <= 128) launch_group<kOp, 8, 4>(a, s);
  else if (n <= 192) launch_group<kOp, 16, 3>(a, s);
  else if (n <= 256) launch_group<kOp, 32, 2>(a, s);
  else if (n <= 384) launch_group<kOp, 32, 3>(a, s);
  else if (n <= 512) launch_group<kOp, 32, 4>(a, s);
  else if (n <= 768) launch_group<kOp, 64, 3>(a, s);
  else if (n <= 1024) launch_group<kOp, 64, 4>(a, s);
  else launch_group<kOp, 64, 6>(a, s);
}

template <RowOp kOp>
int run_rows(RowArgs a, std::int64_t outer, std::int64_t reduce, std::int64_t inner, void* workspace,
             std::size_t workspace_bytes, bool split, hipStream_t s) {
  if (outer == 0 || reduce == 0 || inner == 0) return TCX_OK;
  const int status = ready();
  if (status != TCX_OK) return status;
  if (inner != 1) return run_cols<kOp>(a, outer, reduce, inner, workspace, workspace_bytes, split, s);
  a.rows = outer;
  a.n = reduce;
  const bool vec = reduce % 4 == 0 && aligned16(a.x) && aligned16(a.out) &&
                   (a.gamma == nullptr || aligned16(a.gamma)) && (a.beta == nullptr || aligned16(a.beta));
  const std::int64_t per = (reduce + 1023) / 1024;    // per thread, one block per row
  if (reduce <= kGroupMax) {
    launch_group_for<kOp>(a, reduce, s);
  } else if (reduce > 3072 && reduce <= 4 * kResidentThreads * 8 &&
           (reduce > 4096 || (a.gamma == nullptr && a.beta == nullptr))) {
    // Rows of 3073-16384 floats: held in registers by row_resident_kernel,
    // one 512-thread block per row, whose float4 body starts at the row's
    // first 16-byte boundary. Off 16-byte alignment (an odd length, or a
    // buffer off 16 bytes) the split kernel takes a row one float per load
    // ([16384, 4097] softmax 176 -> 91 us); aligned, the single read of the
    // row still beats the split kernel's per-row phases ([2048, 12288]
    // softmax 44.4 -> 34.1 us, LayerNorm 49.9 -> 39.0 us; [8192, 8192]
    // softmax 95.9 -> 90.8 us). Up to 4096 floats with a weight or bias the
    // split kernel stays: it keeps them in registers across rows, where this
    // kernel reads them from L2 for each row ([8192, 3001] LayerNorm 40
    // against 54 us; with this kernel's weight/bias loads grouped, inputs
    // rotated, [16384, 4096] LayerNorm + weight/bias 92.8 against 100.9 us,
    // [32768, 3500] 161.4 against 195.0); so do rows of up to 3072 (one float4 per thread here:
    // [4096, 2049] RMSNorm 13.4 against 15.4 us).
    if (outer > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "too many rows");
    const int aff = (a.gamma ? kAffGamma : 0) + (a.beta ? kAffBeta : 0);
    auto launch_resident = [&](auto p) {
      resident_variants<kOp, decltype(p)::value>([&](RowKernel kernel, int k) {
        if (k == aff) hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(outer)), dim3(kResidentThreads), 0, s, a);
      });
    };
    if (reduce <= 4 * kResidentThreads * 4)
      launch_resident(std::integral_constant<int, 4>{});
    else
      launch_resident(std::integral_constant<int, 8>{});
  } else if (per <= 2) return launch_split<kOp, 2>(a, vec, s);
  else if (per <= kMaxSplit) return launch_split<kOp, kMaxSplit>(a, vec, s);
  else {
    // Rows of more than 16384 floats: one block per row holding the row, 512
    // threads of 12 or 20 float4 of registers (up to 24576 and 40960 floats;
    // three and two blocks per CU), then of 20 or 24 with the rest in LDS
    // (two blocks per CU), then 1024 threads of 24 with the rest in LDS
    // within the device's per-block LDS (its static arrays and a margin
    // aside); longer rows are re-read.
    if (outer > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "too many rows");
    thread_local int lds_limit[64] = {};
    int device = 0;
    (void)hipGetDevice(&device);
    int& limit = lds_limit[device & 63];
    if (limit == 0) {
      int bytes = 0;
      if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, device) != hipSuccess) bytes = 0;
      limit = bytes > 0 ? bytes : -1;
      if (limit > 0) {
        resident_variants<kOp, kWideVec, kWideThreads>([&](RowKernel kernel, int) {
          (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    limit - 1024);
        });
        const int pair_bytes = std::min(kPairLdsChunks * 1024, limit - 1024);
        resident_variants<kOp, 20>([&](RowKernel kernel, int) {
          (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                                    pair_bytes);
        });
        if constexpr (kOp == RowOp::kLayer)
          resident_variants<kOp, 24>([&](RowKernel kernel, int) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, pair_bytes);
          });
      }
    }
    const int aff = (a.gamma ? kAffGamma : 0) + (a.beta ? kAffBeta : 0);
    auto launch_resident = [&](auto p, unsigned lds_bytes) {
      resident_variants<kOp, decltype(p)::value>([&](RowKernel kernel, int k) {
        if (k == aff)
          hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(outer)), dim3(kResidentThreads), lds_bytes, s, a);
      });
    };
    // Rows past the registers of 20 (LayerNorm also 24) float4 per thread
    // keep two blocks per CU with the rest in LDS, so one row's writes
    // overlap another's reads, where that measured faster (inputs rotated)
    // than one block per CU: against 512 threads of 44 float4, softmax
    // [2048, 50257] 170.1 -> 159.6 us, [4096, 41000] 280.7 -> 250.0;
    // LayerNorm + weight/bias [2048, 50257] 198.4 -> 169.2, at 24 [2048,
    // 65536] 235.7 -> 210.5, [1024, 69000] 125.4 -> 116.2; RMSNorm + weight
    // [2048, 50257] 166.3 -> 161.7; against the 1024-thread route below,
    // softmax [4096, 45000] 288.4 -> 276.8, LayerNorm + weight/bias 350.4 ->
    // 291.9, [2048, 50257] 191.5 -> 169.3, [1024, 69000] 124.3 -> 114.9.
    // Plain RMSNorm (0.5-3 % behind 44 float4), softmax at 24 ([2048,
    // 65536] 205.1 -> 218.0 against 44 float4) and RMSNorm + weight at 24
    // take the 1024-thread route instead.
    const std::int64_t regs20 = static_cast<std::int64_t>(kResidentThreads) * 20;
    const std::int64_t regs24 = static_cast<std::int64_t>(kResidentThreads) * 24;
    const bool pair20 = kOp != RowOp::kRms || a.gamma != nullptr;
    const std::int64_t pair_chunks = limit > 0 ? std::min<std::int64_t>(kPairLdsChunks, (limit - 1024) / 1024) : 0;
    // LDS holds the float4s past the registers' share, in whole 1 KB DMA
    // instructions (a row has at most reduce / 4 float4s).
    auto pair_bytes = [&](std::int64_t regs) {
      return static_cast<unsigned>((reduce / 4 - regs + 63) / 64 * 1024);  // reduce / 4 > regs here
    };
    if (reduce / 4 <= static_cast<std::int64_t>(kResidentThreads) * 12)
      launch_resident(std::integral_constant<int, 12>{}, 0U);
    else if (reduce / 4 <= regs20)
      launch_resident(std::integral_constant<int, 20>{}, 0U);
    else if (pair20 && reduce / 4 <= regs20 + 64 * pair_chunks)
      launch_resident(std::integral_constant<int, 20>{}, pair_bytes(regs20));
    else if (kOp == RowOp::kLayer && reduce / 4 > regs24 && reduce / 4 <= regs24 + 64 * pair_chunks) {
      if constexpr (kOp == RowOp::kLayer) launch_resident(std::integral_constant<int, 24>{}, pair_bytes(regs24));
    } else if (limit > 0 &&
               reduce / 4 <= static_cast<std::int64_t>(kWideThreads) * kWideVec + 64 * ((limit - 1024) / 1024)) {
      // Rows past those: 1024 threads of 24 float4, the rest in LDS.
      const std::int64_t past = reduce / 4 - static_cast<std::int64_t>(kWideThreads) * kWideVec;
      const unsigned wide_bytes = static_cast<unsigned>(past > 0 ? (past + 63) / 64 * 1024 : 0);
      resident_variants<kOp, kWideVec, kWideThreads>([&](RowKernel kernel, int k) {
        if (k == aff)
          hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(outer)), dim3(kWideThreads), wide_bytes, s, a);
      });
    } else {
      hipLaunchKernelGGL((row_block_kernel<kOp>), dim3(static_cast<unsigned>(outer)), dim3(kRowBlockThreads), 0, s,
                         a);
    }
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

size_t tcx_hip_rownorm_workspace_bytes(int64_t outer, int64_t reduce, int64_t inner) {
  return static_cast<size_t>(tcx::norm_workspace(outer, reduce, inner));
}

namespace {

int softmax_entry(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner, void* ws,
                  size_t wsb, bool split, tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  RowArgs a{x, nullptr, nullptr, out, 0, 0, 0.F};
  return run_rows<RowOp::kSoftmax>(a, outer, reduce, inner, ws, wsb, split, static_cast<hipStream_t>(stream));
}

int rmsnorm_entry(const float* x, const float* gamma, float* out, int64_t outer, int64_t reduce, int64_t inner,
                  float eps, void* ws, size_t wsb, bool split, tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  if (!(eps >= 0.F) || __builtin_isinf(eps)) return fail(TCX_INVALID_ARGUMENT, "epsilon must be finite and non-negative");
  RowArgs a{x, gamma, nullptr, out, 0, 0, eps};
  return run_rows<RowOp::kRms>(a, outer, reduce, inner, ws, wsb, split, static_cast<hipStream_t>(stream));
}

int layernorm_entry(const float* x, const float* gamma, const float* beta, float* out, int64_t outer,
                    int64_t reduce, int64_t inner, float eps, void* ws, size_t wsb, bool split,
                    tcx_stream_t stream) {
  using namespace tcx;
  const int rc = check_extents(outer, reduce, inner, x, out);
  if (rc != TCX_OK) return rc;
  if (!(eps >= 0.F) || __builtin_isinf(eps)) return fail(TCX_INVALID_ARGUMENT, "epsilon must be finite and non-negative");
  RowArgs a{x, gamma, beta, out, 0, 0, eps};
  return run_rows<RowOp::kLayer>(a, outer, reduce, inner, ws, wsb, split, static_cast<hipStream_t>(stream));
}

}  // namespace

int tcx_hip_softmax_f32(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner,
                        tcx_stream_t stream) {
  return softmax_entry(x, out, outer, reduce, inner, nullptr, 0, false, stream);
}

int tcx_hip_rmsnorm_f32(const float* x, const float* gamma, float* out, int64_t outer, int64_t reduce,
                        int64_t inner, float eps, tcx_stream_t stream) {
  return rmsnorm_entry(x, gamma, out, outer, reduce, inner, eps, nullptr, 0, false, stream);
}

int tcx_hip_layernorm_f32(const float* x, const float* gamma, const float* beta, float* out, int64_t outer,
                          int64_t reduce, int64_t inner, float eps, tcx_stream_t stream) {
  return layernorm_entry(x, gamma, beta, out, outer, reduce, inner, eps, nullptr, 0, false, stream);
}

int tcx_hip_softmax_f32_ws(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner,
                           void* workspace, size_t workspace_bytes, tcx_stream_t stream) {
  return softmax_entry(x, out, outer, reduce, inner, workspace, workspace_bytes, true, stream);
}

int tcx_hip_rmsnorm_f32_ws(const float* x, const float* gamma, float* out, int64_t outer, int64_t reduce,
                           int64_t inner, float eps, void* workspace, size_t workspace_bytes,
                           tcx_stream_t stream) {
  return rmsnorm_entry(x, gamma, out, outer, reduce, inner, eps, workspace, workspace_bytes, true, stream);
}

int tcx_hip_layernorm_f32_ws(const float* x, const float* gamma, const float* beta, float* out, int64_t outer,
                             int64_t reduce, int64_t inner, float eps, void* workspace, size_t workspace_bytes,
                             tcx_stream_t stream) {
  return layernorm_entry(x, gamma, beta, out, outer, reduce, inner, eps, workspace, workspace_bytes, true, stream);
}

}  // extern "C"
