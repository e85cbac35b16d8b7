// Shared helpers for the gfx950 kernels and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "launch_grid.hpp"
#include "tensorcx_hip.h"

namespace tcx {

// Thread-local failure message behind tcx_hip_last_error().
void set_error(std::string message);
int fail(int code, std::string message);
// Maps a hipError_t to a StatusCode value, recording the message.
int check(hipError_t error, const char* what);
// Validates a launch on this thread (runtime ready, not in a forked child).
int ready();
// True in a process forked from the one that loaded the library; every entry
// point that reaches the HIP runtime refuses to run there.
bool forked();
int refuse_forked();

constexpr int kWave = 64;

using float4_t = float __attribute__((ext_vector_type(4)));
using int4_t = int __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bool is_nan(float v) { return v != v; }

// Streaming loads of data read exactly once. TCX_STREAM_NT selects the
// non-temporal form (global_load ... nt), which keeps one-pass operands from
// displacing reusable lines in L2 and the Infinity Cache.
#ifndef TCX_STREAM_NT
#define TCX_STREAM_NT 1
#endif
template <typename V>
__device__ __forceinline__ V stream_load(const V* p) {
#if TCX_STREAM_NT
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

// e^x for softmax arguments (x <= 0): v_exp_f32 of t = x*log2(e) with the
// rounding error of that product, recovered exactly by an FMA plus the low
// part of log2(e), applied as a first-order correction. About 2 ulp, against
// the ~1 ulp of a correctly rounded expf.
__device__ __forceinline__ float exp_softmax(float x) {
  constexpr float kLog2e = 1.44269502F;        // float(log2 e)
  constexpr float kLog2eLo = 1.925963033e-8F;  // log2 e - kLog2e
  constexpr float kLn2 = 0.693147181F;
  const float t = x * kLog2e;
  const float e = __builtin_amdgcn_exp2f(t);
  const float err = fmaf(x, kLog2e, -t) + x * kLog2eLo;
  return t >= -125.0F ? fmaf(e, err * kLn2, e) : e;  // underflow, -inf and NaN keep e
}

// Wave-wide butterfly sums: both partners add the same two operands, so every
// lane ends with identical bits and the order is fixed for a given layout.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}
__device__ __forceinline__ std::uint32_t wave_sum_u32(std::uint32_t v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1)
    v += static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(v), offset, kWave));
  return v;
}

// (value, index) candidate of an extremum search with the reference's rules
// (cpu_math.cpp:14-20,48-54; cpu_backend.cpp:1181-1194): a NaN beats every
// number and the first NaN wins; otherwise the larger (kMax/kArgmax) or smaller
// (kMin) value wins, +0 and -0 compare equal, and ties keep the lowest index.
template <bool kLargest>
__device__ __forceinline__ bool better_f32(float v, std::int64_t i, float best, std::int64_t bi) {
  const bool vn = is_nan(v), bn = is_nan(best);
  if (vn != bn) return vn;
  if (!vn) {
    if (kLargest ? (v > best) : (v < best)) return true;
    if (kLargest ? (v < best) : (v > best)) return false;
  }
  return i < bi;
}
template <bool kLargest>
__device__ __forceinline__ bool better_i32(int v, std::int64_t i, int best, std::int64_t bi) {
  if (kLargest ? (v > best) : (v < best)) return true;
  if (kLargest ? (v < best) : (v > best)) return false;
  return i < bi;
}

}  // namespace tcx
