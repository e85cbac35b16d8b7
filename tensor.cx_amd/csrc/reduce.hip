// Reductions: sum / max / mean / min / argmax over float32 and int32.
//
// Semantics (reference cpu_backend.cpp:1099-1249, cpu_math.cpp:27-76):
//   sum    float32: fp32 additions from +0; int32: wraps modulo 2^32
//   mean   float32 sum / float(count); NaN for an empty reduction
//   max    value at the first index attaining the maximum; a NaN wins and the
//          first NaN is returned; +0 and -0 compare equal (first kept)
//   min    the same with the minimum
//   argmax int32 index of that element
// max/min/argmax and int32 sums are order-free under these rules, so the
// parallel paths are bit-exact. A float32 sum depends on order: rows longer
// than kSequentialMax use a fixed tree order (per-lane strided partials, then a
// butterfly), strided (inner > 1) reductions of more than kSequentialMax rows
// a fixed interleaved order (per-lane sequences of rows, folded in a fixed
// order), and
// shorter reductions keep the reference's exact left-to-right order, one lane
// per output.
//
// Paths:
//   packed_row_kernel  inner == 1, rows of kSequentialMax + 1 .. kPackedRowMax:
//                      8 to 64 lanes per row, 16-byte loads, butterfly folds
//   row_kernel         inner == 1, longer rows: wave segments reduced by one
//                      wave each with 16-byte loads; items of one segment per
//                      wave (rows below kBlockRowMin) or four per 4-wave block
//                      (longer rows) taken in turn by a persistent grid; rows
//                      split into more items when there are too few rows to
//                      fill the GPU (partials in workspace)
//   finish_kernel      combines per-row item partials in a fixed order
//   col_kernel         inner > 1, more than kSequentialMax rows: a block per
//                      tile of 64 or 256 columns, its waves folding runs of
//                      rows (rows split over blocks when tiles are few)
//   col_finish_kernel  combines the column splits' partials in split order
//   short_row_kernel   inner == 1, rows of at most kSequentialMax: 64 rows per
//                      wave staged in LDS, each lane folding one row in the
//                      reference's element order
//   lane_kernel        inner > 1, at most kSequentialMax rows: one lane per
//                      output, reference element order
//   axes_kernel        any axis selection through reduction-plan metadata

#include <mutex>
#include <string>
#include <type_traits>

#include "common.hpp"

namespace tcx {
namespace {

constexpr std::int64_t kSequentialMax = 64;   // rows up to this length keep exact order
// Wave segments that too few long rows are split into (over all rows): one
// per wave of the row path's persistent grid on 256 CUs (7 blocks of 4 waves
// per 4 CUs), so each wave streams one segment and the finish step folds few
// partials. Measured against 8192 segments (4.6 per wave) on MI355X: full
// max 66.1 -> 75.9 % of HBM peak, int32 full max 72.1 -> 75.3 %, 2 x 33 M min
// 68.6 -> 76.2 %; 3584 segments lost 7 points on 64 x 1 M max.
constexpr std::int64_t kTargetSegments = 1792;
// Rows of at least this many elements are reduced a block at a time, four
// wave segments of at least 8192 elements per block item. Shorter segments
// cost extremum searches their per-segment tail (the wave's key reduction):
// with block items from 8192 elements, [8192, 8192] max fell from 77.9 to
// 57.0 % of HBM peak; from 32768, every shape measured kept or gained.
constexpr std::int64_t kBlockRowMin = 32768;
constexpr std::int64_t kMinSegment = 4096;    // fewest elements per wave segment of a split row

// Partial result of one (row, segment) of an extremum search: (value bits,
// index); index < 0 marks an empty candidate. Sum partials are stored instead
// as dense 32-bit words (float bits or uint32) at the start of the workspace.
struct Partial {
  std::uint32_t bits;
  std::uint32_t pad;
  std::int64_t index;
};

template <typename T>
__device__ __forceinline__ T from_bits(std::uint32_t b) {
  return __builtin_bit_cast(T, b);
}
template <typename T>
__device__ __forceinline__ std::uint32_t to_bits(T v) {
  return __builtin_bit_cast(std::uint32_t, v);
}

template <typename T, bool kLargest>
__device__ __forceinline__ bool lane_takes(T v, T best) {
  // Within one lane indices only grow, so ties keep the earlier element.
  if constexpr (sizeof(T) == 4 && __is_same(T, float)) {
    // As lane masks, two compares: !(v <= best) holds for v > best and for a
    // NaN on either side, so it takes a larger or NaN v unless best is
    // already NaN. (The select form, is_nan(v) ? !is_nan(best) : v > best,
    // compiled to booleans kept as 0/1 integers: six selects per element;
    // [8192, 8192] over axis 0 max 53.0 -> 49.7 us.)
    const bool beats = kLargest ? !(v <= best) : !(v >= best);
    return beats & !is_nan(best);
  } else {
    return kLargest ? v > best : v < best;
  }
}

template <typename T, bool kLargest>
__device__ __forceinline__ bool cand_better(T v, std::int64_t i, T best, std::int64_t bi) {
  if (i < 0) return false;
  if (bi < 0) return true;
  if constexpr (__is_same(T, float))
    return better_f32<kLargest>(v, i, best, bi);
  else
    return better_i32<kLargest>(v, i, best, bi);
}

// Rank key of an extremum candidate's value bits: the larger key is the
// better candidate, and equal keys go to the lower index, which is the order
// cand_better defines. NaN ranks above every number (for min as for max), -0
// and +0 share a key, other values map monotonically (the sign-flipped bit
// pattern, inverted for min). An empty candidate is (key 0, kNoIndex): only
// the int32 extreme (INT_MIN for max, INT_MAX for min) also has key 0, and it
// wins on the index.
constexpr std::int64_t kNoIndex = INT64_MAX;
template <typename T, bool kLargest>
__device__ __forceinline__ std::uint32_t rank_key(std::uint32_t bits) {
  std::uint32_t o;
  if constexpr (__is_same(T, float)) {
    const std::uint32_t mag = bits & 0x7FFFFFFFU;
    if (mag > 0x7F800000U) return 0xFFFFFFFFU;
    if (mag == 0) bits = 0;
    o = (bits & 0x80000000U) ? ~bits : bits | 0x80000000U;
  } else {
    o = bits ^ 0x80000000U;
  }
  return kLargest ? o : ~o;
}

template <typename T, bool kLargest>
__device__ __forceinline__ void wave_extremum(T& best, std::int64_t& bi) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    const T ov = from_bits<T>(static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(to_bits(best)), offset, kWave)));
    const std::int64_t oi = __shfl_xor(bi, offset, kWave);
    if (cand_better<T, kLargest>(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
}

// ------------------------------------------------------------- row path
template <typename T>
using vec4 = T __attribute__((ext_vector_type(4)));

// The last vectors of a lane's walk, issued together: the 16-byte vectors at
// element offsets i, i + 256, ... below end (at most kCount of them) are all
// loaded before use(vector, k) sees them in order k = 0, 1, ... Taken one per
// loop iteration, each load waited for the one before, which left every row's
// last kilo-element (and rows of a few thousand elements) latency-bound.
template <int kCount, typename V, typename E, typename F>
__device__ __forceinline__ void last_vectors(const E* __restrict__ p, std::int64_t i, std::int64_t end, F&& use) {
  V v[kCount];
#pragma unroll
  for (int k = 0; k < kCount; ++k)
    if (i + k * 256 < end) v[k] = stream_load(reinterpret_cast<const V*>(p + i + k * 256));
#pragma unroll
  for (int k = 0; k < kCount; ++k)
    if (i + k * 256 < end) use(v[k], k);
}

// One wave's reduction of elements [begin, end) of row p (an empty range
// gives 0, or an extremum candidate with index -1). Sums return their bits
// (float or uint32) in .bits; extrema return (value bits, row index).
// kVec: p + begin is 16-byte aligned and end - begin a multiple of 4.
template <int kOp, typename T, bool kVec>
__device__ __forceinline__ Partial wave_reduce_body(const T* __restrict__ p, std::int64_t begin, std::int64_t end,
                                                    int lane) {
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  constexpr bool kLargest = kOp != TCX_REDUCE_MIN;

  if constexpr (kSum) {
    if constexpr (__is_same(T, float)) {
      float s0 = 0.F, s1 = 0.F, s2 = 0.F, s3 = 0.F;
      if constexpr (kVec) {
        std::int64_t i = begin + lane * 4;
        for (; i + 3 * 256 < end; i += 4 * 256) {
          const vec4<float> a = stream_load(reinterpret_cast<const vec4<float>*>(p + i));
          const vec4<float> b = stream_load(reinterpret_cast<const vec4<float>*>(p + i + 256));
          const vec4<float> c = stream_load(reinterpret_cast<const vec4<float>*>(p + i + 512));
          const vec4<float> d = stream_load(reinterpret_cast<const vec4<float>*>(p + i + 768));
          s0 += a.x; s1 += a.y; s2 += a.z; s3 += a.w;
          s0 += b.x; s1 += b.y; s2 += b.z; s3 += b.w;
          s0 += c.x; s1 += c.y; s2 += c.z; s3 += c.w;
          s0 += d.x; s1 += d.y; s2 += d.z; s3 += d.w;
        }
        // i + 768 >= end: at most three vectors remain.
        last_vectors<3, vec4<float>>(p, i, end, [&](const vec4<float>& a, int) {
          s0 += a.x; s1 += a.y; s2 += a.z; s3 += a.w;
        });
      } else {
        for (std::int64_t i = begin + lane; i < end; i += 64) s0 += p[i];
      }
      return Partial{to_bits(wave_sum((s0 + s1) + (s2 + s3))), 0U, 0};
    } else {
      std::uint32_t s = 0;
      if constexpr (kVec) {
        const unsigned* __restrict__ q = reinterpret_cast<const unsigned*>(p);
        std::int64_t i = begin + lane * 4;
        for (; i + 3 * 256 < end; i += 4 * 256) {
          const vec4<unsigned> a = stream_load(reinterpret_cast<const vec4<unsigned>*>(q + i));
          const vec4<unsigned> b = stream_load(reinterpret_cast<const vec4<unsigned>*>(q + i + 256));
          const vec4<unsigned> c = stream_load(reinterpret_cast<const vec4<unsigned>*>(q + i + 512));
          const vec4<unsigned> d = stream_load(reinterpret_cast<const vec4<unsigned>*>(q + i + 768));
          s += (a.x + a.y) + (a.z + a.w);
          s += (b.x + b.y) + (b.z + b.w);
          s += (c.x + c.y) + (c.z + c.w);
          s += (d.x + d.y) + (d.z + d.w);
        }
        last_vectors<3, vec4<unsigned>>(q, i, end, [&](const vec4<unsigned>& a, int) {
          s += (a.x + a.y) + (a.z + a.w);
        });
      } else {
        for (std::int64_t i = begin + lane; i < end; i += 64) s += static_cast<std::uint32_t>(p[i]);
      }
      return Partial{wave_sum_u32(s), 0U, 0};
    }
  } else {
    // Lane-local search in increasing index order; indices are kept relative
    // to the segment start in 32 bits (segments are capped below 2^31).
    T best{};
    int li = -1;
    auto visit = [&](T v, int j) {
      if (li < 0 || lane_takes<T, kLargest>(v, best)) {
        best = v;
        li = j;
      }
    };
    const int len = static_cast<int>(end - begin);
    const T* __restrict__ q = p + begin;
    bool exact = true;  // run the exact scan below
    int fast_index = -1;  // fast path result (segment-relative index, value)
    T fast_value{};
    if constexpr (kVec && __is_same(T, float)) {
      // Fast float path: four independent (value, index) chains per lane, one
      // per float4 component, each seeing its elements in increasing index
      // order. A strict compare keeps the earlier index on ties and treats +0
      // and -0 as equal, which is the reference's rule for NaN-free data.
      // NaNs are only flagged here: a wave that saw one re-scans its segment
      // with the exact loop.
      // Chain c of this lane holds element lane*4 + c + cr[c]; the offsets r
      // stepped through are wave-uniform, so they live in scalar registers.
      // Chains start at -inf (+inf for min) with no element: one that never
      // takes an element saw only that infinity (or a NaN, which the re-scan
      // handles), so its candidate is its first element.
      constexpr float kStart = kLargest ? -__builtin_inff() : __builtin_inff();
      float cb[4] = {kStart, kStart, kStart, kStart};
      int cr[4] = {-1, -1, -1, -1};
      bool nan_seen = false;
      const int lane4 = lane * 4;
      auto step = [&](int c, float v, int r) {
        const bool take = kLargest ? v > cb[c] : v < cb[c];
        cb[c] = take ? v : cb[c];
        cr[c] = take ? r : cr[c];
        nan_seen |= v != v;
      };
      int r = 0;
      // Every lane's four groups are in range while r + 1024 <= len. The
      // next four loads are issued before the current four are scanned.
      auto scan4 = [&](const vec4<float>& a, const vec4<float>& b, const vec4<float>& c, const vec4<float>& d,
                       int at) {
        step(0, a.x, at); step(1, a.y, at); step(2, a.z, at); step(3, a.w, at);
        step(0, b.x, at + 256); step(1, b.y, at + 256); step(2, b.z, at + 256); step(3, b.w, at + 256);
        step(0, c.x, at + 512); step(1, c.y, at + 512); step(2, c.z, at + 512); step(3, c.w, at + 512);
        step(0, d.x, at + 768); step(1, d.y, at + 768); step(2, d.z, at + 768); step(3, d.w, at + 768);
      };
      auto ld = [&](int at) { return stream_load(reinterpret_cast<const vec4<float>*>(q + lane4 + at)); };
      if (len >= 1024) {
        vec4<float> a = ld(0), b = ld(256), c = ld(512), d = ld(768);
        for (; r + 2048 <= len; r += 1024) {
          const vec4<float> a2 = ld(r + 1024), b2 = ld(r + 1280), c2 = ld(r + 1536), d2 = ld(r + 1792);
          scan4(a, b, c, d, r);
          a = a2; b = b2; c = c2; d = d2;
        }
        scan4(a, b, c, d, r);
        r += 1024;
      }
      // r + 1024 > len: at most four vectors remain.
      last_vectors<4, vec4<float>>(q, lane4 + r, len, [&](const vec4<float>& a, int k) {
        const int at = r + k * 256;
        step(0, a.x, at); step(1, a.y, at); step(2, a.z, at); step(3, a.w, at);
      });
      exact = __any(nan_seen);
      if (!exact) {
        // NaN-free wave: one order-preserving 64-bit key per candidate, the
        // value (+0 and -0 merged) above the complemented index, so a plain
        // maximum picks the extreme value and, among equal ones, the lowest
        // index. Key 0 means no candidate (real keys are >= 2^32).
        auto key_of = [](float v, int idx) -> std::uint64_t {
          std::uint32_t u = to_bits(v);
          if (u == 0x80000000U) u = 0;
          u = (u & 0x80000000U) ? ~u : (u | 0x80000000U);
          if constexpr (!kLargest) u = ~u;
          return (static_cast<std::uint64_t>(u) << 32) | (0xFFFFFFFFU - static_cast<std::uint32_t>(idx));
        };
        std::uint64_t key = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const std::uint64_t k = lane4 < len ? key_of(cb[c], lane4 + c + (cr[c] < 0 ? 0 : cr[c])) : 0;
          key = k > key ? k : key;
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
          const std::uint64_t o = __shfl_xor(key, offset, kWave);
          key = o > key ? o : key;
        }
        // The winning element sits in chain (win & 3) of lane (win & 255) / 4;
        // its own bits give the value (and the sign of a zero).
        fast_index = key ? static_cast<int>(0xFFFFFFFFU - static_cast<std::uint32_t>(key)) : -1;
        const int c = fast_index & 3;
        const float mine = c == 0 ? cb[0] : c == 1 ? cb[1] : c == 2 ? cb[2] : cb[3];
        fast_value = __shfl(mine, (fast_index & 255) >> 2, kWave);
      }
    }
    if (!exact) {
    } else if constexpr (kVec) {
      int j = lane * 4;
      for (; j + 3 * 256 < len; j += 4 * 256) {
        const vec4<T> a = stream_load(reinterpret_cast<const vec4<T>*>(q + j));
        const vec4<T> b = stream_load(reinterpret_cast<const vec4<T>*>(q + j + 256));
        const vec4<T> c = stream_load(reinterpret_cast<const vec4<T>*>(q + j + 512));
        const vec4<T> d = stream_load(reinterpret_cast<const vec4<T>*>(q + j + 768));
        visit(a.x, j); visit(a.y, j + 1); visit(a.z, j + 2); visit(a.w, j + 3);
        visit(b.x, j + 256); visit(b.y, j + 257); visit(b.z, j + 258); visit(b.w, j + 259);
        visit(c.x, j + 512); visit(c.y, j + 513); visit(c.z, j + 514); visit(c.w, j + 515);
        visit(d.x, j + 768); visit(d.y, j + 769); visit(d.z, j + 770); visit(d.w, j + 771);
      }
      last_vectors<3, vec4<T>>(q, j, len, [&](const vec4<T>& a, int k) {
        const int at = j + k * 256;
        visit(a.x, at); visit(a.y, at + 1); visit(a.z, at + 2); visit(a.w, at + 3);
      });
    } else {
      for (int j = lane; j < len; j += 64) visit(q[j], j);
    }
    std::int64_t bi;
    if (!exact) {
      best = fast_value;
      bi = fast_index < 0 ? -1 : begin + fast_index;
    } else {
      bi = li < 0 ? -1 : begin + li;
      wave_extremum<T, kLargest>(best, bi);
    }
    return Partial{to_bits(best), 0U, bi};
  }
}

// wave_reduce_body for any range: a range that is not 16-byte aligned (rows
// whose length is not a multiple of 4) splits into a head of at most three
// elements up to the next 16-byte boundary, a body of whole float4s run by
// the 16-byte path, and a tail of at most three; lanes 0-2 take the head and
// lanes 3-5 the tail, folded in after the body (sums) or as candidates with
// their row indices (extrema, so ties and NaNs keep the reference's rule).
// One element per lane per step instead ran [8192, 8191] sum at 17 % of HBM.
template <int kOp, typename T, bool kVec>
__device__ __forceinline__ Partial wave_reduce(const T* __restrict__ p, std::int64_t begin, std::int64_t end,
                                               int lane) {
  if constexpr (kVec) {
    return wave_reduce_body<kOp, T, true>(p, begin, end, lane);
  } else {
    constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
    constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
    const auto addr = reinterpret_cast<std::uintptr_t>(p + begin);
    std::int64_t head = static_cast<std::int64_t>(((16U - (addr & 15U)) & 15U) / sizeof(T));
    if (head > end - begin) head = end - begin;
    const std::int64_t body_begin = begin + head;
    const std::int64_t body_end = body_begin + (end - body_begin) / 4 * 4;
    // This lane's head or tail element, if any, loaded before the body's.
    std::int64_t idx = -1;
    if (lane < head) idx = begin + lane;
    else if (lane >= 3 && lane < 3 + (end - body_end)) idx = body_end + (lane - 3);
    const T edge = idx >= 0 ? p[idx] : T{};
    const Partial body = wave_reduce_body<kOp, T, true>(p, body_begin, body_end, lane);
    if constexpr (kSum) {
      if constexpr (__is_same(T, float)) {
        const float extra = wave_sum(idx >= 0 ? edge : 0.F);
        return Partial{to_bits(from_bits<float>(body.bits) + extra), 0U, 0};
      } else {
        const std::uint32_t extra = wave_sum_u32(idx >= 0 ? static_cast<std::uint32_t>(edge) : 0U);
        return Partial{body.bits + extra, 0U, 0};
      }
    } else {
      // The head and tail candidates sit in lanes 0-5: a 64-bit key maximum
      // (rank key above the complemented segment-relative index, as in
      // packed_row_kernel) over lanes 0-7 in three steps, the winner's bits
      // from its lane; lane 0, which publishes the result, then holds it.
      const std::int64_t rel = idx - begin;
      std::uint64_t key = idx >= 0 ? (static_cast<std::uint64_t>(rank_key<T, kLargest>(to_bits(edge))) << 32) |
                                         (0xFFFFFFFFU - static_cast<std::uint32_t>(rel))
                                   : 0;
#pragma unroll
      for (int offset = 4; offset > 0; offset >>= 1) {
        const std::uint64_t o = __shfl_xor(key, offset, kWave);
        key = o > key ? o : key;
      }
      const std::int64_t won = key ? static_cast<std::int64_t>(0xFFFFFFFFU - static_cast<std::uint32_t>(key)) : -1;
      const int owner = won < 0 ? 0 : won < head ? static_cast<int>(won) : static_cast<int>(3 + won - (body_end - begin));
      const T best = from_bits<T>(static_cast<std::uint32_t>(__shfl(static_cast<int>(to_bits(edge)), owner, kWave)));
      const std::int64_t bi = won < 0 ? -1 : begin + won;
      T v = from_bits<T>(body.bits);
      std::int64_t vi = body.index;
      if (cand_better<T, kLargest>(best, bi, v, vi)) {
        v = best;
        vi = bi;
      }
      return Partial{to_bits(v), 0U, vi};
    }
  }
}

// Writes the final value of `row` from its combined result.
template <int kOp, typename T>
__device__ __forceinline__ void store_row(void* out, std::int64_t row, const Partial& r, std::int64_t reduce) {
  if constexpr (kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN) {
    if constexpr (__is_same(T, float)) {
      const float s = from_bits<float>(r.bits);
      static_cast<float*>(out)[row] = kOp == TCX_REDUCE_MEAN ? s / static_cast<float>(reduce) : s;
    } else {
      static_cast<int*>(out)[row] = static_cast<int>(r.bits);
    }
  } else if constexpr (kOp == TCX_REDUCE_ARGMAX) {
    static_cast<int*>(out)[row] = static_cast<int>(r.index);
  } else {
    static_cast<T*>(out)[row] = from_bits<T>(r.bits);
  }
}

// Combines the four wave partials of a block item in wave order: sums as
// (w0 + w1) + (w2 + w3), extrema by cand_better (empty candidates lose).
template <int kOp, typename T>
__device__ __forceinline__ Partial combine_waves(const Partial (&w)[4]) {
  if constexpr (kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN) {
    if constexpr (__is_same(T, float)) {
      const float s = (from_bits<float>(w[0].bits) + from_bits<float>(w[1].bits)) +
                      (from_bits<float>(w[2].bits) + from_bits<float>(w[3].bits));
      return Partial{to_bits(s), 0U, 0};
    } else {
      return Partial{(w[0].bits + w[1].bits) + (w[2].bits + w[3].bits), 0U, 0};
    }
  } else {
    constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
    Partial best = w[0];
#pragma unroll
    for (int v = 1; v < 4; ++v)
      if (cand_better<T, kLargest>(from_bits<T>(w[v].bits), w[v].index, from_bits<T>(best.bits), best.index))
        best = w[v];
    return best;
  }
}

// The row path. Each row is cut into `segments` wave segments of seg_len
// elements (the last ones may be short or empty), reduced by wave_reduce.
//   kBlock false: one wave per (row, segment) item, the waves of a persistent
//   grid taking items in turn.
//   kBlock true: one 4-wave block per item of four consecutive segments, the
//   blocks of a persistent grid taking items in turn; the block adds its four
//   wave partials in wave order. A block finishes a long row four times
//   sooner than a wave, so the last round of items leaves fewer waves idle.
// With one item per row the row's result is stored; otherwise each item's
// partial goes to the workspace (sums as dense 32-bit words, extrema as
// records) for finish_kernel.
template <int kOp, typename T, bool kVec, bool kBlock>
__global__ __launch_bounds__(256) void row_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                  Partial* __restrict__ partials, std::int64_t rows,
                                                  std::int64_t reduce, std::int64_t segments, std::int64_t seg_len) {
  constexpr bool kSumWords = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto publish = [&](std::int64_t row, std::int64_t item, std::int64_t per_row, const Partial& r) {
    if (per_row == 1)
      store_row<kOp, T>(out, row, r, reduce);
    else if constexpr (kSumWords)
      reinterpret_cast<std::uint32_t*>(partials)[item] = r.bits;
    else
      partials[item] = r;
  };
  if constexpr (!kBlock) {
    // Grid-stride over the waves' items (the launcher caps the grid); the
    // bound is wave-uniform, so every lane of a wave runs the same iterations.
    const std::int64_t items = rows * segments;
    const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
    for (std::int64_t gw = static_cast<std::int64_t>(blockIdx.x) * 4 + wave; gw < items; gw += step) {
      const std::int64_t row = gw / segments, seg = gw % segments;
      const std::int64_t begin = seg * seg_len;
      const Partial r = wave_reduce<kOp, T, kVec>(x + row * reduce, begin, min(reduce, begin + seg_len), lane);
      if (lane == 0) publish(row, gw, segments, r);
    }
  } else {
    // Block-uniform bound: every thread reaches each barrier. The wave
    // partials alternate between two slots, so thread 0 reads an item's
    // slot while the waves fill the other one with the next item's.
    __shared__ Partial slot[2][4];
    const std::int64_t per_row = segments / 4;
    const std::int64_t items = rows * per_row;
    int parity = 0;
    for (std::int64_t item = blockIdx.x; item < items; item += gridDim.x, parity ^= 1) {
      const std::int64_t row = item / per_row;
      const std::int64_t begin = min(reduce, ((item % per_row) * 4 + wave) * seg_len);
      const Partial r = wave_reduce<kOp, T, kVec>(x + row * reduce, begin, min(reduce, begin + seg_len), lane);
      if (lane == 0) slot[parity][wave] = r;
      __syncthreads();
      if (threadIdx.x == 0) publish(row, item, per_row, combine_waves<kOp, T>(slot[parity]));
    }
  }
}

// One block of kFinishThreads threads per row combines that row's item
// partials in a fixed order, so the result is deterministic: a sum's thread t
// keeps kUnroll accumulators, accumulator u folding partials t + u * 256,
// t + (u + kUnroll) * 256, ... (all kUnroll loads of a round in flight; one
// round covers 2048 partials, the full-tensor sum has 443), then the accumulators, the
// lanes and the waves combine pairwise. Extremum records fold on (rank key,
// index) in a few selects per record: a lone block's time is its dependent
// instruction path, and the former fold, exec-masked branches around every
// comparison (1210 instructions), took 9.2 us at 8192 records against 6.7 us
// for this one (146).
constexpr int kFinishThreads = 256;
template <int kOp, typename T>
__global__ __launch_bounds__(kFinishThreads) void finish_kernel(const Partial* __restrict__ partials,
                                                                void* __restrict__ out, std::int64_t rows,
                                                                std::int64_t reduce, std::int64_t segments) {
  constexpr int kThreads = kFinishThreads, kWaves = kThreads / 64, kUnroll = 8;
  if (static_cast<std::int64_t>(blockIdx.x) >= rows) return;
  const std::int64_t row = blockIdx.x;
  __shared__ Partial waves[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
  if constexpr (kSum) {
    // Sum partials are dense 32-bit words (float bits or uint32).
    const std::uint32_t* w = reinterpret_cast<const std::uint32_t*>(partials) + row * segments;
    using Acc = std::conditional_t<__is_same(T, float), float, std::uint32_t>;
    Acc acc[kUnroll] = {};
    for (std::int64_t base = threadIdx.x; base < segments; base += kUnroll * kThreads) {
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const std::int64_t i = base + u * kThreads;
        if (i < segments) acc[u] += __builtin_bit_cast(Acc, w[i]);
      }
    }
#pragma unroll
    for (int u = kUnroll / 2; u > 0; u >>= 1)
#pragma unroll
      for (int v = 0; v < u; ++v) acc[v] += acc[v + u];
    Acc t;
    if constexpr (__is_same(T, float))
      t = wave_sum(acc[0]);
    else
      t = wave_sum_u32(acc[0]);
    if (lane == 0) waves[wave] = Partial{__builtin_bit_cast(std::uint32_t, t), 0U, 0};
    __syncthreads();
    if (threadIdx.x == 0) {
      // Pairwise over the waves: (w0 + w1) + (w2 + w3).
      const Acc w01 = __builtin_bit_cast(Acc, waves[0].bits) + __builtin_bit_cast(Acc, waves[1].bits);
      const Acc w23 = __builtin_bit_cast(Acc, waves[2].bits) + __builtin_bit_cast(Acc, waves[3].bits);
      store_row<kOp, T>(out, row, Partial{__builtin_bit_cast(std::uint32_t, w01 + w23), 0U, 0}, reduce);
    }
  } else {
    const Partial* p = partials + row * segments;
    std::uint32_t bk = 0, bb = 0;
    std::int64_t bi = kNoIndex;
    auto take = [&](std::uint32_t k, std::uint32_t b, std::int64_t i) {
      const bool win = k > bk || (k == bk && i < bi);
      bk = win ? k : bk;
      bb = win ? b : bb;
      bi = win ? i : bi;
    };
#pragma unroll 1
    for (std::int64_t i = threadIdx.x; i < segments; i += kThreads) {
      const Partial r = p[i];
      const bool empty = r.index < 0;
      take(empty ? 0U : rank_key<T, kLargest>(r.bits), r.bits, empty ? kNoIndex : r.index);
    }
#pragma unroll 1
    for (int offset = 32; offset > 0; offset >>= 1) {
      const std::uint32_t k = static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(bk), offset, kWave));
      const std::uint32_t b = static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(bb), offset, kWave));
      take(k, b, __shfl_xor(bi, offset, kWave));
    }
    if (lane == 0) waves[wave] = Partial{bb, bk, bi};
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll 1
      for (int v = 1; v < kWaves; ++v) take(waves[v].pad, waves[v].bits, waves[v].index);
      store_row<kOp, T>(out, row, Partial{bb, 0U, bi == kNoIndex ? -1 : bi}, reduce);
    }
  }
}

// ------------------------------------------------------- strided path
// Reductions over a middle axis (inner > 1) of more than kSequentialMax rows,
// x as [outer, R, inner]: the R elements of one output lie inner elements
// apart. One block of kColWaves waves per column tile (64 x kVec consecutive
// columns of one outer index; a lane holds kVec columns, so a wave reads 256
// or 1024 contiguous bytes of each row). When column tiles are too few to
// fill the GPU, `splits` blocks share a tile's rows, in contiguous runs of
// split_rows; inside a block the waves interleave over the run's rows (wave w
// takes rows w, w + 8, ...: the block's waves stream neighbouring rows
// together). A lane folds its rows in order with kColDepth loads in flight;
// the waves' results are folded in wave order through LDS and the splits' in
// split order by col_finish_kernel. Extrema and int32 sums are exact in any
// order; a float32 sum takes this fixed order.
// Interleaved against contiguous runs per wave: [8192, 8192] over axis 0 sum
// 62.6 -> 48.5 us, max 58.5 -> 54.0 us; 16 x 512 x 8192 sum 59.3 -> 45.0 us;
// other shapes within 4 %.
// Eight waves per block and eight 16-byte loads in flight per lane: against
// sixteen loads, large strided reductions on MI355X took 0.93x the time
// (geometric mean of 18 cases of 16-268 MB; 8192 x 8200 columns sum 67.3
// -> 52.7 us, [32768, 2052] max 82.0 -> 72.2 us, the worst 8192 x 8192
// columns sum 52.0 -> 62.4 us); two or four vectors per row per lane (2-4
// KB contiguous per wave row), 16-wave blocks and 256 or 1024 target blocks
// measured no better.
constexpr int kColWaves = 8;
constexpr int kColDepth = 8;
constexpr std::int64_t kColMaxGrid = std::int64_t{1} << 22;

template <int kOp, typename T>
__device__ __forceinline__ void fold_into(Partial& into, const Partial& c) {
  constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
  if constexpr (kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN) {
    if constexpr (__is_same(T, float))
      into.bits = to_bits(from_bits<float>(into.bits) + from_bits<float>(c.bits));
    else
      into.bits += c.bits;
  } else if (cand_better<T, kLargest>(from_bits<T>(c.bits), c.index, from_bits<T>(into.bits), into.index)) {
    into = c;
  }
}

// Output `id` from its fold over all R rows.
template <int kOp, typename T>
__device__ __forceinline__ void store_output(void* out, std::int64_t id, const Partial& r, std::int64_t R) {
  if constexpr (kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN) {
    if constexpr (__is_same(T, float)) {
      const float v = from_bits<float>(r.bits);
      static_cast<float*>(out)[id] = kOp == TCX_REDUCE_MEAN ? v / static_cast<float>(R) : v;
    } else {
      static_cast<int*>(out)[id] = static_cast<int>(r.bits);
    }
  } else if constexpr (kOp == TCX_REDUCE_ARGMAX) {
    static_cast<int*>(out)[id] = static_cast<int>(r.index);
  } else {
    static_cast<T*>(out)[id] = from_bits<T>(r.bits);
  }
}

template <typename T, int kVec>
__device__ __forceinline__ void load_cols(const T* __restrict__ p, T (&v)[kVec]) {
  if constexpr (kVec == 4) {
    const vec4<T> q = stream_load(reinterpret_cast<const vec4<T>*>(p));
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  } else {
    v[0] = stream_load(p);
  }
}

// One (split, column tile) pair. A wave takes G rows at a time, W columns of
// each (W * G = 64 * kVec; W = 64 * kVec when inner is at least that, else
// the power of two at or above inner, so narrow tensors still give every lane
// a column), and the block's waves take consecutive row groups in turn: lane
// (g, c) of wave w folds rows rb + w G + g + i G kColWaves of column c,
// kColDepth of its rows loaded at once. For a float32 sum the order is
// fixed: each lane's rows in order, the wave's row groups by a butterfly,
// the waves in order, then the splits.
template <int kOp, typename T, int kVec>
__device__ __forceinline__ void col_block(const T* __restrict__ x, void* __restrict__ out,
                                          Partial* __restrict__ partials, std::int64_t outer, std::int64_t R,
                                          std::int64_t inner, std::int64_t split_rows, int W, std::int64_t b,
                                          Partial (&lds)[kColWaves][64 * kVec]) {
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
  constexpr int kRows = kColDepth;
  const int G = 64 * kVec / W;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lanes_per_row = W / kVec;
  const int g = lane / lanes_per_row, cl = (lane % lanes_per_row) * kVec;
  const std::int64_t tiles_per_outer = (inner + W - 1) / W;
  const std::int64_t col_tiles = outer * tiles_per_outer;
  const std::int64_t split = b / col_tiles, tile = b % col_tiles;
  const std::int64_t o = tile / tiles_per_outer, tile_col = (tile % tiles_per_outer) * W;
  const std::int64_t rb = split * split_rows, re = min(R, rb + split_rows);
  // This lane's rows: a, a + GS, a + 2 GS, ... below re (n of them), GS = G
  // x kColWaves: the block's waves interleave by row groups, so they stream
  // neighbouring rows together.
  const std::int64_t GS = static_cast<std::int64_t>(G) * kColWaves;
  const std::int64_t a = rb + wave * G + g;
  const std::int64_t n = a < re ? (re - a + GS - 1) / GS : 0;
  // Lanes past the last column read the last kVec columns (in bounds: inner
  // is a multiple of kVec) and their results are not stored.
  const std::int64_t j = tile_col + cl;
  const T* __restrict__ base = x + o * R * inner + a * inner + (j < inner ? j : inner - kVec);
  const std::int64_t step = GS * inner;
  auto load_row = [&](std::int64_t i, T (&v)[kVec]) { load_cols<T, kVec>(base + i * step, v); };
  Partial acc[kVec];
  if constexpr (kSum) {
    using Acc = std::conditional_t<__is_same(T, float), float, std::uint32_t>;
    Acc sum[kVec];
#pragma unroll
    for (int c = 0; c < kVec; ++c) sum[c] = 0;
    std::int64_t i = 0;
    for (; i + kRows <= n; i += kRows) {
      T v[kRows][kVec];
#pragma unroll
      for (int u = 0; u < kRows; ++u) load_row(i + u, v[u]);
#pragma unroll
      for (int u = 0; u < kRows; ++u)
#pragma unroll
        for (int c = 0; c < kVec; ++c) sum[c] += static_cast<Acc>(v[u][c]);
    }
    if (i < n) {  // the last partial batch: loads clamped to row n - 1
      T v[kRows][kVec];
#pragma unroll
      for (int u = 0; u < kRows; ++u) load_row(min(i + u, n - 1), v[u]);
#pragma unroll
      for (int u = 0; u < kRows; ++u)
        if (i + u < n)
#pragma unroll
          for (int c = 0; c < kVec; ++c) sum[c] += static_cast<Acc>(v[u][c]);
    }
#pragma unroll
    for (int c = 0; c < kVec; ++c) acc[c] = Partial{__builtin_bit_cast(std::uint32_t, sum[c]), 0U, 0};
  } else {
    // A lane without rows (more waves or splits than rows) gives empty
    // candidates.
#pragma unroll
    for (int c = 0; c < kVec; ++c) acc[c] = Partial{0U, 0U, -1};
    if (n > 0) {
      // Candidates hold the lane's row count (below 2^31: a lane takes at
      // most split_rows / kColWaves rows, checked at launch); the row index
      // is a + count x GS.
      T best[kVec];
      int bi[kVec];
      load_row(0, best);
#pragma unroll
      for (int c = 0; c < kVec; ++c) bi[c] = 0;
      auto visit = [&](const T (&v)[kVec], int i) {
#pragma unroll
        for (int c = 0; c < kVec; ++c)
          if (lane_takes<T, kLargest>(v[c], best[c])) {
            best[c] = v[c];
            bi[c] = i;
          }
      };
      int i = 1;
      for (; i + kRows <= n; i += kRows) {
        T v[kRows][kVec];
#pragma unroll
        for (int u = 0; u < kRows; ++u) load_row(i + u, v[u]);
#pragma unroll
        for (int u = 0; u < kRows; ++u) visit(v[u], i + u);
      }
      if (i < n) {
        T v[kRows][kVec];
#pragma unroll
        for (int u = 0; u < kRows; ++u) load_row(min<std::int64_t>(i + u, n - 1), v[u]);
#pragma unroll
        for (int u = 0; u < kRows; ++u)
          if (i + u < n) visit(v[u], i + u);
      }
#pragma unroll
      for (int c = 0; c < kVec; ++c)
        acc[c] = Partial{to_bits(best[c]), 0U, a + static_cast<std::int64_t>(bi[c]) * GS};
    }
  }
  // The G row groups of a wave fold by a butterfly over the lane bits that
  // select the group (a fixed order); group 0's lanes then hold the wave's
  // result for their columns.
  for (int sh = lanes_per_row; sh < 64; sh <<= 1) {
#pragma unroll
    for (int c = 0; c < kVec; ++c) {
      Partial other;
      other.bits = static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(acc[c].bits), sh, kWave));
      other.pad = 0U;
      other.index = kSum ? 0 : __shfl_xor(acc[c].index, sh, kWave);
      fold_into<kOp, T>(acc[c], other);
    }
  }
  if (g == 0) {
#pragma unroll
    for (int c = 0; c < kVec; ++c) lds[wave][cl + c] = acc[c];
  }
  __syncthreads();
  // Thread t < W folds column tile_col + t over the waves, in wave order.
  const int t = threadIdx.x;
  if (t >= W || tile_col + t >= inner) return;
  Partial total = lds[0][t];
#pragma unroll
  for (int w = 1; w < kColWaves; ++w) fold_into<kOp, T>(total, lds[w][t]);
  const std::int64_t id = o * inner + tile_col + t;
  if (split_rows >= R)
    store_output<kOp, T>(out, id, total, R);
  else
    partials[split * outer * inner + id] = total;
}

template <int kOp, typename T, int kVec>
__global__ __launch_bounds__(64 * kColWaves) void col_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                             Partial* __restrict__ partials, std::int64_t outer,
                                                             std::int64_t R, std::int64_t inner,
                                                             std::int64_t split_rows, int W, std::int64_t blocks) {
  __shared__ Partial lds[kColWaves][64 * kVec];
  // Block-stride over (split, tile) pairs: a grid of at most kColMaxGrid
  // blocks keeps gridDim.x x blockDim.x inside 32 bits.
  for (std::int64_t b = blockIdx.x; b < blocks; b += gridDim.x) {
    col_block<kOp, T, kVec>(x, out, partials, outer, R, inner, split_rows, W, b, lds);
    __syncthreads();  // lds is rewritten by the next pair
  }
}

// Folds each output's split partials: L lanes per output (a power of two up
// to 64, so that many splits are read in one pass), lane k folding splits k,
// k + L, ... in order, then the L lanes by a butterfly (a fixed order).
template <int kOp, typename T>
__global__ __launch_bounds__(256) void col_finish_kernel(const Partial* __restrict__ partials, void* __restrict__ out,
                                                         std::int64_t outputs, std::int64_t splits, std::int64_t R,
                                                         int L) {
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  const int k = threadIdx.x & (L - 1);
  const std::int64_t per_pass = static_cast<std::int64_t>(gridDim.x) * (blockDim.x / L);
  // Every lane runs the same number of passes (the butterfly needs the whole
  // wave): lanes past the last output fold a clamped one and store nothing.
  const std::int64_t passes = (outputs + per_pass - 1) / per_pass;
  for (std::int64_t pass = 0; pass < passes; ++pass) {
    const std::int64_t id0 = pass * per_pass + static_cast<std::int64_t>(blockIdx.x) * (blockDim.x / L) + threadIdx.x / L;
    const std::int64_t id = id0 < outputs ? id0 : outputs - 1;
    Partial total{0U, 0U, kSum ? 0 : -1};
    if (k < splits) {
      total = partials[k * outputs + id];
      std::int64_t sp = k + L;
      for (; sp + 7 * L < splits; sp += 8 * L) {  // eight loads in flight, folded in order
        Partial q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = partials[(sp + u * L) * outputs + id];
#pragma unroll
        for (int u = 0; u < 8; ++u) fold_into<kOp, T>(total, q[u]);
      }
      for (; sp < splits; sp += L) fold_into<kOp, T>(total, partials[sp * outputs + id]);
    }
    for (int off = 1; off < L; off <<= 1) {
      Partial other;
      other.bits = static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(total.bits), off, kWave));
      other.pad = 0U;
      other.index = kSum ? 0 : __shfl_xor(total.index, off, kWave);
      fold_into<kOp, T>(total, other);
    }
    if (k == 0 && id0 < outputs) store_output<kOp, T>(out, id, total, R);
  }
}

// ------------------------------------------------------ exact-order paths
// Sequential per-output loop in the reference's element order.
template <int kOp, typename T>
__device__ __forceinline__ void sequential(const T* __restrict__ x, std::int64_t count,
                                           std::int64_t stride, void* out, std::int64_t id) {
  if constexpr (kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN) {
    if constexpr (__is_same(T, float)) {
      if (kOp == TCX_REDUCE_MEAN && count == 0) {
        static_cast<float*>(out)[id] = __builtin_nanf("");
        return;
      }
      float s = 0.F;
      for (std::int64_t r = 0; r < count; ++r) s += x[r * stride];
      static_cast<float*>(out)[id] = kOp == TCX_REDUCE_MEAN ? s / static_cast<float>(count) : s;
    } else {
      std::uint32_t s = 0;
      for (std::int64_t r = 0; r < count; ++r) s += static_cast<std::uint32_t>(x[r * stride]);
      static_cast<int*>(out)[id] = static_cast<int>(s);
    }
  } else if constexpr (kOp == TCX_REDUCE_MAX) {
    if constexpr (__is_same(T, float)) {
      float best = -__builtin_inff();
      for (std::int64_t r = 0; r < count; ++r) {
        const float v = x[r * stride];
        if (is_nan(v)) {
          best = v;
          break;
        }
        best = (best < v) ? v : best;  // std::max keeps the first of equals
      }
      static_cast<float*>(out)[id] = best;
    } else {
      int best = static_cast<int>(0x80000000U);
      for (std::int64_t r = 0; r < count; ++r) {
        const int v = x[r * stride];
        best = (best < v) ? v : best;
      }
      static_cast<int*>(out)[id] = best;
    }
  } else {
    constexpr bool kLargest = kOp == TCX_REDUCE_ARGMAX;
    T best = x[0];
    std::int64_t bi = 0;
    for (std::int64_t r = 1; r < count; ++r) {
      const T v = x[r * stride];
      bool take;
      if constexpr (__is_same(T, float))
        take = !is_nan(best) && (is_nan(v) || (kLargest ? best < v : v < best));
      else
        take = kLargest ? best < v : v < best;
      if (take) {
        best = v;
        bi = r;
      }
    }
    if constexpr (kOp == TCX_REDUCE_ARGMAX)
      static_cast<int*>(out)[id] = static_cast<int>(bi);
    else
      static_cast<T*>(out)[id] = best;
  }
}

template <int kOp, typename T>
__global__ __launch_bounds__(256) void lane_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                   std::int64_t outer, std::int64_t reduce,
                                                   std::int64_t inner) {
  const std::int64_t items = outer * inner;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t id = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; id < items; id += step) {
    const T* base = x + (id / inner) * reduce * inner + id % inner;
    sequential<kOp, T>(base, reduce, inner, out, id);
  }
}

// Contiguous rows (inner == 1) of 2 .. kSequentialMax elements: each wave
// stages 64 whole rows (one tile of 64 x R contiguous elements) in LDS with
// coalesced loads, 64 / R rows per load instruction, then each lane folds
// its own row from LDS in the reference's order (sequential). Rows sit at an
// odd LDS stride (R or R + 1), so the lanes' reads of one column fall in
// distinct banks. The waves of a block take tiles independently; a block of
// kShortWaves waves takes at most 2 x 64 x 65 x 4 bytes (33 KB) of LDS.
constexpr int kShortWaves = 2;
// Below this row length one lane per row reads its row's few contiguous
// words well enough. Sum, lanes against staged tiles on MI355X: [4194304, 4]
// 23.7 / 32.3 us, [2097152, 6] 17.1 / 18.3 us, [2097152, 8] 36.0 / 17.7 us,
// [2097152, 12] 46.0 / 19.7 us, [262144, 64] 70.6 / 19.2 us.
constexpr std::int64_t kShortRowMin = 8;

template <int kOp, typename T>
__global__ __launch_bounds__(64 * kShortWaves) void short_row_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                                     std::int64_t rows, int R) {
  // Dynamic LDS, 64 x stride elements per wave: short rows take little, so
  // more waves fit on a CU.
  extern __shared__ unsigned char short_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int stride = R | 1;
  const int per_step = 64 / R;             // rows per load instruction
  const int q = lane / R, m = lane % R;    // this lane's row within a step, and its column
  const bool loads = q < per_step;
  T* tile = reinterpret_cast<T*>(short_lds) + wave * 64 * stride;
  const std::int64_t tiles = (rows + 63) / 64;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * kShortWaves;
  for (std::int64_t tl = static_cast<std::int64_t>(blockIdx.x) * kShortWaves + wave; tl < tiles; tl += step) {
    const std::int64_t row0 = tl * 64;
    const int nrows = static_cast<int>(rows - row0 < 64 ? rows - row0 : 64);
    const T* __restrict__ src = x + row0 * R;
    for (int r = 0; r < nrows; r += 16 * per_step) {  // sixteen loads in flight per lane
      T v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int rr = r + u * per_step + q;
        if (loads && rr < nrows) v[u] = src[rr * R + m];
      }
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int rr = r + u * per_step + q;
        if (loads && rr < nrows) tile[rr * stride + m] = v[u];
      }
    }
    // The wave's LDS writes are visible to all its lanes before they read.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane < nrows) sequential<kOp, T>(tile + lane * stride, R, 1, out, row0 + lane);
    // Every lane has read its row before the next tile is staged.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Contiguous rows (inner == 1) of kSequentialMax + 1 .. kPackedRowMax
// elements: L lanes per row, 64 / L rows per wave. Lane l of a row's group
// takes elements 4l + 4Lu .. + 3 (u < kV, all loaded before any is used)
// with 16-byte loads through a buffer resource based at the wave's first
// row, whatever the rows' alignment (a 16-byte buffer load needs 4-byte
// alignment), so a row group reads 16 L contiguous bytes per instruction.
// Elements past the row (the next row's, or past the range, which read zero)
// are masked; a float4 wholly past the row is not loaded. L and kV are the
// smallest that cover the row ((8, 4) up to 128 elements, then (16, 3),
// (16, 4), (32, 3), (32, 4), (64, 3), (64, 4), (64, 6), (64, 8)), which
// keeps the per-element work of masked elements low. The group then folds
// its lanes by butterfly: sums in a fixed tree (every lane ends with the same
// bits: each lane adds its elements in order first), extrema by 64-bit keys
// (below), so ties and NaNs keep the reference's lowest-index rule. Against
// 4-byte loads at stride L (16-64 lanes, up to 8-32 loads), in one process
// on MI355X: [100000, 130] sum 11.5 -> 9.0 us, max 13.5 -> 11.3; [200000,
// 100] int32 argmax 22.8 -> 12.7; [50000, 257] max 14.2 -> 11.3; [10000,
// 1500] max 13.1 -> 11.1 us. One wave per row had spent each row's load
// latency and two wave-wide folds on 130 elements: [100000, 130] sum ran at
// 8.6 % and max at 4.8 % of HBM.
constexpr std::int64_t kPackedRowMax = 2048;

template <int kOp, typename T, int kL, int kV>
__global__ __launch_bounds__(256) void packed_row_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                         std::int64_t rows, int R) {
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  constexpr bool kLargest = kOp != TCX_REDUCE_MIN;
  constexpr int kRows = 64 / kL;
  constexpr int kOut = 0x7fffffff;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l = lane % kL, g = lane / kL;
  const std::int64_t tiles = (rows + kRows - 1) / kRows;
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * 4;
  // The bound is wave-uniform: every lane of a wave takes part in each
  // butterfly, lanes past the last row with empty values.
  for (std::int64_t t = static_cast<std::int64_t>(blockIdx.x) * 4 + wave; t < tiles; t += step) {
    const std::int64_t row0 = t * kRows;
    const std::int64_t row = row0 + g;
    const bool live = row < rows;
    const int nrows = rows - row0 < kRows ? static_cast<int>(rows - row0) : kRows;
    const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(x + row0 * R), static_cast<short>(0),
                                                        nrows * R * static_cast<int>(sizeof(T)), 0x00020000);
    T v[kV][4];
#pragma unroll
    for (int u = 0; u < kV; ++u) {
      const int j0 = 4 * l + 4 * kL * u;
      const int off = live && j0 < R ? (g * R + j0) * static_cast<int>(sizeof(T)) : kOut;
      // The whole vector is cast before its elements are taken: element
      // reads of the builtin's result itself compiled to one 4-byte load
      // whose value stood in for all four elements.
      using vec4 = T __attribute__((ext_vector_type(4)));
      const vec4 q = __builtin_bit_cast(vec4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
#pragma unroll
      for (int e = 0; e < 4; ++e) v[u][e] = q[e];
    }
    Partial r{0U, 0U, 0};
    if constexpr (kSum) {
      if constexpr (__is_same(T, float)) {
        float s = 0.F;
#pragma unroll
        for (int u = 0; u < kV; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (4 * l + 4 * kL * u + e < R) s += v[u][e];
#pragma unroll
        for (int offset = kL / 2; offset > 0; offset >>= 1) s += __shfl_xor(s, offset, kWave);
        r.bits = to_bits(s);
      } else {
        std::uint32_t s = 0;
#pragma unroll
        for (int u = 0; u < kV; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (4 * l + 4 * kL * u + e < R) s += static_cast<std::uint32_t>(v[u][e]);
#pragma unroll
        for (int offset = kL / 2; offset > 0; offset >>= 1)
          s += static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(s), offset, kWave));
        r.bits = s;
      }
    } else {
      // One 64-bit key per element: its rank key above the complemented row
      // index, so the largest key is the extreme value and, among equal
      // ranks (ties, +0 and -0, every NaN), the lowest index. Real keys are
      // nonzero (the low word alone is), 0 marks no element. The winner's
      // own bits (a NaN's payload, a zero's sign) come from the lane that
      // holds it. Against (value, index) butterflies under cand_better:
      // [100000, 130] max 26.5 -> 16.7 us on MI355X.
      std::uint64_t key = 0;
      T best{};
#pragma unroll
      for (int u = 0; u < kV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * l + 4 * kL * u + e;
          if (live && j < R) {
            const std::uint64_t k = (static_cast<std::uint64_t>(rank_key<T, kLargest>(to_bits(v[u][e]))) << 32) |
                                    (0xFFFFFFFFU - static_cast<std::uint32_t>(j));
            if (k > key) {
              key = k;
              best = v[u][e];
            }
          }
        }
#pragma unroll
      for (int offset = kL / 2; offset > 0; offset >>= 1) {
        const std::uint64_t o = __shfl_xor(key, offset, kWave);
        key = o > key ? o : key;
      }
      const int bi = key ? static_cast<int>(0xFFFFFFFFU - static_cast<std::uint32_t>(key)) : -1;
      // Element j sits in lane (j / 4) % L of the group.
      const int owner = (lane & ~(kL - 1)) + (bi < 0 ? 0 : (bi / 4) % kL);
      r.bits = static_cast<std::uint32_t>(__shfl(static_cast<int>(to_bits(best)), owner, kWave));
      r.index = bi;
    }
    if (live && l == 0) store_row<kOp, T>(out, row, r, R);
  }
}

struct AxesMeta {
  std::int64_t extent[TCX_HIP_MAX_FOLDED_RANK];
  std::int64_t stride[TCX_HIP_MAX_FOLDED_RANK];
  std::int32_t outer_rank, rank;
};

__device__ __forceinline__ std::int64_t meta_offset(std::int64_t index, const AxesMeta& m, int begin,
                                                    int end) {
  std::int64_t value = 0;
  for (int axis = end - 1; axis >= begin; --axis) {
    value += (index % m.extent[axis]) * m.stride[axis];
    index /= m.extent[axis];
  }
  return value;
}

// Output g of an axis selection: the `count` selected elements of group g in
// the reference's order.
template <int kOp, typename T>
__device__ __forceinline__ void axes_item(const T* __restrict__ x, void* __restrict__ out, const AxesMeta& meta,
                                          std::int64_t g, std::int64_t count) {
  const T* base = x + meta_offset(g, meta, 0, meta.outer_rank);
  constexpr bool kSum = kOp == TCX_REDUCE_SUM || kOp == TCX_REDUCE_MEAN;
  auto item = [&](std::int64_t r) { return base[meta_offset(r, meta, meta.outer_rank, meta.rank)]; };
  if constexpr (kSum) {
    if constexpr (__is_same(T, float)) {
      float s = 0.F;
      for (std::int64_t r = 0; r < count; ++r) s += item(r);
      float v = s;
      if (kOp == TCX_REDUCE_MEAN) v = count ? s / static_cast<float>(count) : __builtin_nanf("");
      static_cast<float*>(out)[g] = v;
    } else {
      std::uint32_t s = 0;
      for (std::int64_t r = 0; r < count; ++r) s += static_cast<std::uint32_t>(item(r));
      static_cast<int*>(out)[g] = static_cast<int>(s);
    }
  } else if constexpr (kOp == TCX_REDUCE_MAX) {
    if constexpr (__is_same(T, float)) {
      float best = -__builtin_inff();
      for (std::int64_t r = 0; r < count; ++r) {
        const float v = item(r);
        if (is_nan(v)) {
          best = v;
          break;
        }
        best = (best < v) ? v : best;
      }
      static_cast<float*>(out)[g] = best;
    } else {
      int best = static_cast<int>(0x80000000U);
      for (std::int64_t r = 0; r < count; ++r) {
        const int v = item(r);
        best = (best < v) ? v : best;
      }
      static_cast<int*>(out)[g] = best;
    }
  } else {
    constexpr bool kLargest = kOp == TCX_REDUCE_ARGMAX;
    T best = item(0);
    std::int64_t bi = 0;
    for (std::int64_t r = 1; r < count; ++r) {
      const T v = item(r);
      bool take;
      if constexpr (__is_same(T, float))
        take = !is_nan(best) && (is_nan(v) || (kLargest ? best < v : v < best));
      else
        take = kLargest ? best < v : v < best;
      if (take) {
        best = v;
        bi = r;
      }
    }
    if constexpr (kOp == TCX_REDUCE_ARGMAX)
      static_cast<int*>(out)[g] = static_cast<int>(bi);
    else
      static_cast<T*>(out)[g] = best;
  }
}

template <int kOp, typename T>
__global__ __launch_bounds__(256) void axes_kernel(const T* __restrict__ x, void* __restrict__ out,
                                                   AxesMeta meta, std::int64_t groups,
                                                   std::int64_t count) {
  const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * blockDim.x;
  for (std::int64_t g = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; g < groups; g += step)
    axes_item<kOp, T>(x, out, meta, g, count);
}

// ------------------------------------------------------------ planning
struct RowPlan {
  bool row_path;
  bool block_items;        // row_kernel<..., kBlock = true>
  std::int64_t segments;   // wave segments per row (4 per item with block_items)
  std::int64_t seg_len;    // elements per wave segment, a multiple of 1024 when segments > 1
  std::int64_t partials;   // items per row: 1 means row_kernel stores the row itself
};

RowPlan plan_rows(std::int64_t outer, std::int64_t reduce, std::int64_t inner) {
  RowPlan p{false, false, 1, reduce, 1};
  if (inner != 1 || reduce <= kPackedRowMax) return p;
  p.row_path = true;
  // 32-bit in-segment indices: segments stay at or below 2^30 elements.
  constexpr std::int64_t kMaxSegment = std::int64_t{1} << 30;
  if (reduce >= kBlockRowMin || (reduce > 2 * kMinSegment && outer < kTargetSegments)) {
    // Block items: four wave segments each, about kTargetSegments wave
    // segments in all when the rows are too few to fill the grid (rows of
    // 8193-32767 elements take block items only then).
    p.block_items = true;
    std::int64_t items = 1;
    if (outer < kTargetSegments / 4) {
      items = (kTargetSegments / 4 + outer - 1) / outer;
      const std::int64_t most = (reduce + 4 * kMinSegment - 1) / (4 * kMinSegment);
      if (items > most) items = most;
    }
    // A multiple of 1024 elements keeps 16-byte alignment and whole
    // unrolled strides inside each wave segment.
    std::int64_t len = (reduce + 4 * items - 1) / (4 * items);
    len = (len + 1023) / 1024 * 1024;
    if (len > kMaxSegment) len = kMaxSegment;
    p.partials = (reduce + 4 * len - 1) / (4 * len);
    p.segments = 4 * p.partials;
    p.seg_len = len;
    return p;
  }
  // Rows of at most 8192 elements, or enough rows to fill the grid: one wave
  // per row.
  return p;
}

bool aligned16(const void* q) { return (reinterpret_cast<std::uintptr_t>(q) & 15U) == 0; }

// Strided (inner > 1) reductions of more than kSequentialMax rows. A column
// tile is W columns: 64 x kVec (256 when inner is a multiple of 4, so lanes
// load 16 bytes, else 64), or the power of two at or above a narrower inner,
// the wave then stepping G = 64 x kVec / W rows at a time. The rows of each
// tile are split `splits` ways (by doubling) while tiles x splits is below
// kColTargetBlocks (two 8-wave blocks per CU on 256 CUs), each split keeps
// at least kColMinRows x G rows (a batch of kColDepth loads per lane) and
// the split partials fit the no-allocation scratch.
constexpr std::int64_t kColTargetBlocks = 512;
constexpr std::int64_t kColMinRows = 64;

// Columns of a full tile: 64 lanes x 4 (inner a multiple of 4, 16-byte
// loads) or x 1.
std::int64_t col_full(bool vec) { return vec ? 256 : 64; }

std::int64_t col_width(std::int64_t inner, std::int64_t full) {
  if (inner >= full) return full;
  std::int64_t w = 1;
  while (w < inner) w *= 2;
  return w;
}

struct ColPlan {
  bool col_path;
  std::int64_t splits;      // > 1: partials in workspace, folded by col_finish_kernel
  std::int64_t split_rows;  // rows per split (the last may be shorter)
};

ColPlan plan_cols(std::int64_t outer, std::int64_t reduce, std::int64_t inner) {
  ColPlan p{false, 1, reduce};
  if (inner <= 1 || reduce <= kSequentialMax) return p;
  p.col_path = true;
  const std::int64_t full = col_full(inner % 4 == 0);
  const std::int64_t width = col_width(inner, full);
  const std::int64_t col_tiles = outer * ((inner + width - 1) / width);
  const std::int64_t min_rows = kColMinRows * (full / width);
  const std::int64_t partial_cap =
      static_cast<std::int64_t>(TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE / sizeof(Partial));
  std::int64_t splits = 1;
  while (col_tiles * splits < kColTargetBlocks && reduce / (2 * splits) >= min_rows &&
         2 * splits * outer * inner <= partial_cap)
    splits *= 2;
  p.split_rows = (reduce + splits - 1) / splits;
  p.splits = (reduce + p.split_rows - 1) / p.split_rows;
  return p;
}

// Blocks of the row path's persistent grid: 7 per 4 CUs (1792 waves on 256
// CUs), each wave (or block) streaming its items in turn. Fewer streams
// open at once read HBM faster than one wave per item. Measured against one
// wave per item on 8192 x 8192 f32: sum 81.1 -> 83.8 %, max 77.9 -> 80.0 %,
// the 67 M-element full sum 75.6 -> 78.0 %, 65536 x 4096 84.7 -> 86.3 %,
// 32768 x 2048 83.9 -> 86.1 %. Two blocks per CU did as well on 8192 x 8192
// but lost 1 point at 65536 x 4096; one per CU lost 7-17 points.
unsigned row_grid_blocks() {
  thread_local int cached[64] = {};
  int device = 0;
  (void)hipGetDevice(&device);
  int& blocks = cached[device & 63];
  if (blocks == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus < 1)
      cus = 256;
    blocks = (7 * cus + 3) / 4;
  }
  return static_cast<unsigned>(blocks);
}

// Bytes of partials a plan keeps in workspace (0 for single-launch plans).
std::int64_t workspace_need(std::int64_t outer, std::int64_t reduce, std::int64_t inner) {
  const std::int64_t entry = static_cast<std::int64_t>(sizeof(Partial));
  const ColPlan cols = plan_cols(outer, reduce, inner);
  if (cols.col_path) return cols.splits > 1 ? cols.splits * outer * inner * entry : 0;
  const RowPlan rows = plan_rows(outer, reduce, inner);
  return rows.row_path && rows.partials > 1 ? outer * rows.partials * entry : 0;
}

template <int kOp, typename T>
int launch_cols(const T* x, void* out, std::int64_t outer, std::int64_t reduce, std::int64_t inner,
                const ColPlan& plan, void* workspace, std::size_t workspace_bytes, hipStream_t s) {
  if (plan.split_rows / kColWaves >= INT32_MAX)
    return fail(TCX_INVALID_ARGUMENT, "strided reduction has too many rows per split for 32-bit row counts");
  Partial* partials = nullptr;
  if (plan.splits > 1) {
    const std::size_t need = static_cast<std::size_t>(plan.splits * outer * inner) * sizeof(Partial);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(TCX_INVALID_ARGUMENT, "reduce workspace is smaller than tcx_hip_reduce_workspace_bytes");
    partials = static_cast<Partial*>(workspace);
  }
  // An unaligned base with inner a multiple of 4 runs the 4-byte kernel with
  // the splits planned for 16-byte loads.
  const bool vec = inner % 4 == 0 && aligned16(x);
  const std::int64_t full = col_full(vec);
  const std::int64_t width = col_width(inner, full);
  const std::int64_t blocks = outer * ((inner + width - 1) / width) * plan.splits;
  const dim3 grid(static_cast<unsigned>(blocks < kColMaxGrid ? blocks : kColMaxGrid));
  const int w = static_cast<int>(width);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(64 * kColWaves), 0, s, x, out, partials, outer, reduce, inner,
                       plan.split_rows, w, blocks);
  };
  if (vec)
    launch(col_kernel<kOp, T, 4>);
  else
    launch(col_kernel<kOp, T, 1>);
  int rc = check(hipGetLastError(), "reduce column kernel launch");
  if (rc != TCX_OK || plan.splits == 1) return rc;
  // Lanes per output: two to four splits per lane, at most a wave. The fold
  // is latency-bound (a few MB of partials); against eight to sixteen splits
  // per lane: [8192, 8192] over axis 0 sum 48.4 -> 47.4 us, max 54.4 -> 52.9
  // us, [4096, 256] 9.0 -> 7.4 us, [4, 65536, 7] 9.2 -> 7.7 us.
  int lanes = 1;
  while (lanes < 64 && 4 * lanes <= plan.splits) lanes *= 2;
  const std::int64_t outputs = outer * inner;
  hipLaunchKernelGGL((col_finish_kernel<kOp, T>), dim3(grid_for(outputs * lanes, 256, kStrideBlocks)), dim3(256), 0,
                     s, partials, out, outputs, plan.splits, reduce, lanes);
  return check(hipGetLastError(), "reduce column finish kernel launch");
}

template <int kOp, typename T>
int launch_reduce(const T* x, void* out, std::int64_t outer, std::int64_t reduce, std::int64_t inner,
                  void* workspace, std::size_t workspace_bytes, hipStream_t s) {
  const ColPlan cols = plan_cols(outer, reduce, inner);
  if (cols.col_path) return launch_cols<kOp, T>(x, out, outer, reduce, inner, cols, workspace, workspace_bytes, s);
  const RowPlan plan = plan_rows(outer, reduce, inner);
  if (!plan.row_path) {
    if (inner == 1 && reduce > kSequentialMax) {
      auto packed = [&](auto kernel, std::int64_t rows_per_wave) {
        hipLaunchKernelGGL(kernel, dim3(grid_for((outer + rows_per_wave - 1) / rows_per_wave, 4, kStrideBlocks)),
                           dim3(256), 0, s, x, out, outer, static_cast<int>(reduce));
        return check(hipGetLastError(), "reduce packed row kernel launch");
      };
      if (reduce <= 128) return packed(packed_row_kernel<kOp, T, 8, 4>, 8);
      if (reduce <= 192) return packed(packed_row_kernel<kOp, T, 16, 3>, 4);
      if (reduce <= 256) return packed(packed_row_kernel<kOp, T, 16, 4>, 4);
      if (reduce <= 384) return packed(packed_row_kernel<kOp, T, 32, 3>, 2);
      if (reduce <= 512) return packed(packed_row_kernel<kOp, T, 32, 4>, 2);
      if (reduce <= 768) return packed(packed_row_kernel<kOp, T, 64, 3>, 1);
      if (reduce <= 1024) return packed(packed_row_kernel<kOp, T, 64, 4>, 1);
      if (reduce <= 1536) return packed(packed_row_kernel<kOp, T, 64, 6>, 1);
      return packed(packed_row_kernel<kOp, T, 64, 8>, 1);
    }
    if (inner == 1 && reduce >= kShortRowMin) {
      const std::int64_t tiles = (outer + 63) / 64;
      const std::size_t lds = static_cast<std::size_t>(kShortWaves) * 64 * (reduce | 1) * sizeof(T);
      hipLaunchKernelGGL((short_row_kernel<kOp, T>), dim3(grid_for(tiles, kShortWaves, kStrideBlocks)),
                         dim3(64 * kShortWaves), lds, s, x, out, outer, static_cast<int>(reduce));
      return check(hipGetLastError(), "reduce short row kernel launch");
    }
    hipLaunchKernelGGL((lane_kernel<kOp, T>), dim3(grid_for(outer * inner, 256, kStrideBlocks)), dim3(256), 0,
                       s, x, out, outer, reduce, inner);
    return check(hipGetLastError(), "reduce lane kernel launch");
  }
  Partial* partials = nullptr;
  if (plan.partials > 1) {
    const std::size_t need = static_cast<std::size_t>(outer * plan.partials) * sizeof(Partial);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(TCX_INVALID_ARGUMENT, "reduce workspace is smaller than tcx_hip_reduce_workspace_bytes");
    partials = static_cast<Partial*>(workspace);
  }
  const bool vec = reduce % 4 == 0 && aligned16(x);
  // A grid of at most row_grid_blocks() blocks, sized so that every round of
  // items keeps all of its waves (or blocks) busy: 4096 rows of 16384 floats
  // take 3 rounds of 1366 waves, not 2 full rounds of 1792 and a third of
  // 512. Against the full grid: [4096, 16384] sum 70.4 -> 78.7 % and max
  // 69.2 -> 75.8 %, [16384, 8192] 83.0 -> 84.6 %, [1000, 32768] sum 71.2 ->
  // 75.3 %, [3000, 20000] 76.7 -> 79.0 %.
  auto balanced = [](std::int64_t work, std::int64_t per_block, std::int64_t cap_blocks) {
    const std::int64_t slots = cap_blocks * per_block;
    const std::int64_t rounds = (work + slots - 1) / slots;
    return grid_for((work + rounds - 1) / rounds, per_block, cap_blocks);
  };
  const dim3 grid(plan.block_items ? balanced(outer * plan.partials, 1, row_grid_blocks())
                                   : balanced(outer * plan.segments, 4, row_grid_blocks()));
  auto launch_rows = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(256), 0, s, x, out, partials, outer, reduce, plan.segments, plan.seg_len);
  };
  if (plan.block_items)
    vec ? launch_rows(row_kernel<kOp, T, true, true>) : launch_rows(row_kernel<kOp, T, false, true>);
  else
    vec ? launch_rows(row_kernel<kOp, T, true, false>) : launch_rows(row_kernel<kOp, T, false, false>);
  int rc = check(hipGetLastError(), "reduce row kernel launch");
  if (rc != TCX_OK || plan.partials == 1) return rc;
  hipLaunchKernelGGL((finish_kernel<kOp, T>), dim3(static_cast<unsigned>(outer)), dim3(kFinishThreads), 0, s,
                     partials, out, outer, reduce, plan.partials);
  return check(hipGetLastError(), "reduce finish kernel launch");
}

// The no-allocation scratch: the segment partials of the two-launch row path
// (row_kernel writes them, finish_kernel combines them), for every plan
// whose workspace query is at most TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE.
constexpr std::size_t kScratchBytes = TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE;

}  // namespace
}  // namespace tcx

// One copy per device, held until the process ends. Each call writes the
// partials it reads, so nothing needs clearing between calls.
static __device__ __align__(256) unsigned char scratch[tcx::kScratchBytes];

namespace tcx {
namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_device[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) on the first no-allocation call there.
// Host code passes this address, never the symbol itself, to kernels.
int scratch_address(void** address) {
  int device = 0;
  int rc = check(hipGetDevice(&device), "hipGetDevice");
  if (rc != TCX_OK) return rc;
  if (device < 0 || device >= kMaxDevices) return fail(TCX_UNAVAILABLE, "device index outside the scratch table");
  std::lock_guard lock(scratch_mutex);
  if (scratch_device[device] == nullptr) {
    void* found = nullptr;
    rc = check(hipGetSymbolAddress(&found, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc != TCX_OK) return rc;
    scratch_device[device] = found;
  }
  *address = scratch_device[device];
  return TCX_OK;
}

// tcx_hip_reduce with the static scratch as its workspace: the same kernels,
// the same partials and combine order, so the same bits.
template <int kOp, typename T>
int launch_reduce_noalloc(const T* x, void* out, std::int64_t outer, std::int64_t reduce, std::int64_t inner,
                          hipStream_t s) {
  const std::int64_t need = workspace_need(outer, reduce, inner);
  if (need == 0) return launch_reduce<kOp, T>(x, out, outer, reduce, inner, nullptr, 0, s);
  if (need > TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE)
    return fail(TCX_INVALID_ARGUMENT, "reduction plan needs " + std::to_string(need) +
                                          " bytes of partials; the no-allocation scratch holds " +
                                          std::to_string(TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE));
  void* base = nullptr;
  const int rc = scratch_address(&base);
  if (rc != TCX_OK) return rc;
  return launch_reduce<kOp, T>(x, out, outer, reduce, inner, base, kScratchBytes, s);
}

template <int kOp, typename T>
int launch_any(const T* x, void* out, std::int64_t outer, std::int64_t reduce, std::int64_t inner, void* ws,
               std::size_t wsb, bool noalloc, hipStream_t s) {
  if (noalloc) return launch_reduce_noalloc<kOp, T>(x, out, outer, reduce, inner, s);
  return launch_reduce<kOp, T>(x, out, outer, reduce, inner, ws, wsb, s);
}

template <typename T>
int dispatch_reduce(int op, const T* x, void* out, std::int64_t outer, std::int64_t reduce,
                    std::int64_t inner, void* ws, std::size_t wsb, bool noalloc, hipStream_t s) {
  switch (op) {
    case TCX_REDUCE_SUM: return launch_any<TCX_REDUCE_SUM, T>(x, out, outer, reduce, inner, ws, wsb, noalloc, s);
    case TCX_REDUCE_MAX: return launch_any<TCX_REDUCE_MAX, T>(x, out, outer, reduce, inner, ws, wsb, noalloc, s);
    case TCX_REDUCE_MIN: return launch_any<TCX_REDUCE_MIN, T>(x, out, outer, reduce, inner, ws, wsb, noalloc, s);
    case TCX_REDUCE_ARGMAX:
      return launch_any<TCX_REDUCE_ARGMAX, T>(x, out, outer, reduce, inner, ws, wsb, noalloc, s);
    default: break;
  }
  if constexpr (__is_same(T, float)) {
    if (op == TCX_REDUCE_MEAN)
      return launch_any<TCX_REDUCE_MEAN, T>(x, out, outer, reduce, inner, ws, wsb, noalloc, s);
  }
  return fail(TCX_INVALID_ARGUMENT, "unsupported reduction for this dtype");
}

template <typename T>
int dispatch_axes(int op, const T* x, void* out, const AxesMeta& m, std::int64_t groups,
                  std::int64_t count, hipStream_t s) {
  const dim3 grid(grid_for(groups, 256, kStrideBlocks));
  switch (op) {
    case TCX_REDUCE_SUM: hipLaunchKernelGGL((axes_kernel<TCX_REDUCE_SUM, T>), grid, dim3(256), 0, s, x, out, m, groups, count); break;
    case TCX_REDUCE_MAX: hipLaunchKernelGGL((axes_kernel<TCX_REDUCE_MAX, T>), grid, dim3(256), 0, s, x, out, m, groups, count); break;
    case TCX_REDUCE_MIN: hipLaunchKernelGGL((axes_kernel<TCX_REDUCE_MIN, T>), grid, dim3(256), 0, s, x, out, m, groups, count); break;
    case TCX_REDUCE_ARGMAX: hipLaunchKernelGGL((axes_kernel<TCX_REDUCE_ARGMAX, T>), grid, dim3(256), 0, s, x, out, m, groups, count); break;
    case TCX_REDUCE_MEAN:
      if constexpr (__is_same(T, float)) {
        hipLaunchKernelGGL((axes_kernel<TCX_REDUCE_MEAN, T>), grid, dim3(256), 0, s, x, out, m, groups, count);
        break;
      }
      [[fallthrough]];
    default:
      return fail(TCX_INVALID_ARGUMENT, "unsupported reduction for this dtype");
  }
  return check(hipGetLastError(), "reduce axes kernel launch");
}

int validate(int op, int dtype, std::int64_t count) {
  if (dtype != TCX_FLOAT32 && dtype != TCX_INT32)
    return fail(TCX_INVALID_ARGUMENT, "reductions require float32 or int32 tensors");
  if (op < TCX_REDUCE_SUM || op > TCX_REDUCE_ARGMAX) return fail(TCX_INVALID_ARGUMENT, "unknown reduction op");
  if (op == TCX_REDUCE_MEAN && dtype != TCX_FLOAT32)
    return fail(TCX_INVALID_ARGUMENT, "mean only supports float32 tensors");
  if ((op == TCX_REDUCE_MAX || op == TCX_REDUCE_MIN || op == TCX_REDUCE_ARGMAX) && count == 0)
    return fail(TCX_INVALID_ARGUMENT, "max/min/argmax require a non-empty reduction");
  return TCX_OK;
}

}  // namespace
}  // namespace tcx

extern "C" {

size_t tcx_hip_reduce_workspace_bytes(int op, int dtype, int64_t outer, int64_t reduce, int64_t inner) {
  (void)op;
  (void)dtype;
  if (outer <= 0 || reduce <= 0 || inner <= 0) return 0;
  return static_cast<size_t>(tcx::workspace_need(outer, reduce, inner));
}

namespace {
int reduce_entry(int op, int dtype, const void* x, void* out, int64_t outer, int64_t reduce, int64_t inner,
                 void* workspace, size_t workspace_bytes, bool noalloc, tcx_stream_t stream) {
  using namespace tcx;
  if (outer < 0 || reduce < 0 || inner < 0) return fail(TCX_INVALID_ARGUMENT, "reduce extents must be non-negative");
  int rc = validate(op, dtype, reduce);
  if (rc != TCX_OK) return rc;
  if (outer == 0 || inner == 0) return TCX_OK;
  if (x == nullptr && reduce != 0) return fail(TCX_INVALID_ARGUMENT, "reduce input is null");
  if (out == nullptr) return fail(TCX_INVALID_ARGUMENT, "reduce output is null");
  rc = ready();
  if (rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (dtype == TCX_FLOAT32)
    return dispatch_reduce<float>(op, static_cast<const float*>(x), out, outer, reduce, inner, workspace,
                                  workspace_bytes, noalloc, s);
  return dispatch_reduce<int>(op, static_cast<const int*>(x), out, outer, reduce, inner, workspace,
                              workspace_bytes, noalloc, s);
}
}  // namespace

int tcx_hip_reduce(int op, int dtype, const void* x, void* out, int64_t outer, int64_t reduce,
                   int64_t inner, void* workspace, size_t workspace_bytes, tcx_stream_t stream) {
  return reduce_entry(op, dtype, x, out, outer, reduce, inner, workspace, workspace_bytes, false, stream);
}

int tcx_hip_reduce_noalloc(int op, int dtype, const void* x, void* out, int64_t outer, int64_t reduce,
                           int64_t inner, tcx_stream_t stream) {
  return reduce_entry(op, dtype, x, out, outer, reduce, inner, nullptr, 0, true, stream);
}

int tcx_hip_reduce_axes(int op, int dtype, const void* x, void* out, const int64_t* meta,
                        int32_t outer_rank, int32_t rank, int64_t groups, int64_t reduction_size,
                        tcx_stream_t stream) {
  using namespace tcx;
  if (rank < 0 || rank > TCX_HIP_MAX_FOLDED_RANK || outer_rank < 0 || outer_rank > rank)
    return fail(TCX_INVALID_ARGUMENT, "reduction rank exceeds the supported maximum");
  if (groups < 0 || reduction_size < 0) return fail(TCX_INVALID_ARGUMENT, "reduce extents must be non-negative");
  int rc = validate(op, dtype, reduction_size);
  if (rc != TCX_OK) return rc;
  if (groups == 0) return TCX_OK;
  if (out == nullptr || (x == nullptr && reduction_size != 0))
    return fail(TCX_INVALID_ARGUMENT, "reduce buffers are null");
  AxesMeta m{};
  m.outer_rank = outer_rank;
  m.rank = rank;
  for (int i = 0; i < rank; ++i) {
    m.extent[i] = meta[2 * i];
    m.stride[i] = meta[2 * i + 1];
    if (m.extent[i] <= 0) return fail(TCX_INVALID_ARGUMENT, "reduction metadata extents must be positive");
  }
  rc = ready();
  if (rc != TCX_OK) return rc;
  const auto s = static_cast<hipStream_t>(stream);
  if (dtype == TCX_FLOAT32)
    return dispatch_axes<float>(op, static_cast<const float*>(x), out, m, groups, reduction_size, s);
  return dispatch_axes<int>(op, static_cast<const int*>(x), out, m, groups, reduction_size, s);
}

}  // extern "C"
