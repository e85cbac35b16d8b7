// Fused attention: out = softmax(scale * Q K^T [causal]) V without
// materialising the scores, on v_mfma_f32_16x16x4_f32.
//
// Semantics are those of the reference composite (core/inference.cpp:123-161
// over backends/cpu/cpu_inference.cpp:22-47) for unmasked and causal
// attention: a score is dot(q, k) * scale (rounded), a key after the query is
// -inf under causal, a row with any NaN score is NaN, a row whose maximum is
// -inf is 0 * V, otherwise exp(s - max) / sum, times V. The sums run in a
// different order (online softmax over key tiles), inside the reference
// test's allclose(rtol=2e-4, atol=2e-5).
//
// Layout. A block owns 16 queries per wave of one batch matrix and walks
// the keys in tiles of 64, staged through padded LDS with a register prefetch
// of the next tile. Each wave computes S^T = K Q^T for its 16 queries, so lane
// l holds S^T[key 16b + 4(l/16) + v][query l%16] (output layout of the MFMA):
// those are exactly the A operands (P[query l%16][key]) that the P V MFMAs
// need, when the k index of step (b, v) is taken as key 16b + 4(l/16) + v. The
// feature sum of S^T uses the same trick: lane l supplies features
// 16t + 4(l/16) + e of K and Q at step (t, e), read as one float4 each. The
// output tile t holds features kT*j + t in its column j (kT = D/16 tiles), so
// a lane reads its V operands, and writes its outputs, as kT contiguous floats.
// Masked keys keep p = 0, so a non-finite V propagates as in the reference's
// P @ V: tiles the causal mask only partly covers run in full; a tile wholly
// after the block's last query skips the MFMAs and only marks the feature
// columns where its V rows hold a non-finite value (0 * inf or 0 * NaN is NaN
// in every output row of the block). Blocks start with the longest query
// tiles under causal masking.

#include "common.hpp"

namespace tcx {
namespace {

constexpr int kKTile = 64;  // keys per tile
// Waves per block (16 queries each), measured on MI355X at 16 x 2048 x 128:
// 8 waves share each K/V tile over 128 queries (97 TFLOP/s unmasked against 93
// with 4); causal runs use 4, so twice as many blocks let the balanced block
// order pair long and short query tiles on each CU (78 against 53 TFLOP/s).
constexpr int kWavesFull = 8;
constexpr int kWavesCausal = 4;
constexpr int kPad = 4;     // LDS row padding (floats)

using mfma_acc = float __attribute__((ext_vector_type(4)));

struct FlashArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  std::int64_t rows, cols;
  float scale;
  int causal;
};

using float2_t = float __attribute__((ext_vector_type(2)));

// N contiguous floats (N = 2, 4 or 8) with 8- or 16-byte accesses.
template <int N>
__device__ __forceinline__ void load_row(const float* p, float (&v)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int t = 0; t < N; t += 4) {
      const float4_t w = *reinterpret_cast<const float4_t*>(p + t);
      v[t] = w.x;
      v[t + 1] = w.y;
      v[t + 2] = w.z;
      v[t + 3] = w.w;
    }
  } else {
    static_assert(N == 2);
    const float2_t w = *reinterpret_cast<const float2_t*>(p);
    v[0] = w.x;
    v[1] = w.y;
  }
}

template <int N>
__device__ __forceinline__ void store_row(float* p, const float (&v)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int t = 0; t < N; t += 4)
      *reinterpret_cast<float4_t*>(p + t) = float4_t{v[t], v[t + 1], v[t + 2], v[t + 3]};
  } else {
    static_assert(N == 2);
    *reinterpret_cast<float2_t*>(p) = float2_t{v[0], v[1]};
  }
}

template <int D, int kWaves>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 8))) void flash_attention_kernel(
    FlashArgs a) {
  constexpr int kThreads = 64 * kWaves;
  constexpr int kQTile = 16 * kWaves;  // queries per block (16 per wave)
  constexpr int kLd = D + kPad;
  constexpr int kT = D / 16;                    // float4 groups of features per lane
  constexpr int kLoads = kKTile * D / 4 / kThreads;  // float4 per thread per K (or V) tile
  static_assert(D % 16 == 0 && kLoads >= 1);
  __shared__ float ks[kKTile * kLd];
  __shared__ float vs[kKTile * kLd];
  __shared__ int bad_column[D];  // a wholly masked tile had a non-finite V here

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;  // MFMA row / k-group of this lane
  // Under causal masking the last query tiles see the most keys. Work items
  // are ranked by their key-tile count; the first half of the grid takes them
  // heaviest first and the second half lightest first, so the two blocks that
  // share a CU (launch ids L and L + grid/2) carry about the same total work.
  std::int64_t batch = blockIdx.y, qtile = blockIdx.x;
  if (a.causal) {
    const std::int64_t n = static_cast<std::int64_t>(gridDim.x) * gridDim.y;
    const std::int64_t id = static_cast<std::int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    const std::int64_t half = (n + 1) / 2;
    const std::int64_t rank = id < half ? id : n - 1 - (id - half);
    qtile = gridDim.x - 1 - rank / gridDim.y;
    batch = rank % gridDim.y;
  }
  const std::int64_t q0 = qtile * kQTile + wave * 16;
  const std::int64_t q_last = min(qtile * kQTile + kQTile, a.rows) - 1;  // the block's last query
  for (int d = tid; d < D; d += kThreads) bad_column[d] = 0;
  const float* __restrict__ qb = a.q + batch * a.rows * D;
  const float* __restrict__ kb = a.k + batch * a.cols * D;
  const float* __restrict__ vb = a.v + batch * a.cols * D;

  // Q fragment: features 16t + 4g .. +3 of query q0 + r.
  float4_t qf[kT];
  {
    const std::int64_t qrow = q0 + r;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      qf[t] = float4_t{0.F, 0.F, 0.F, 0.F};
      if (qrow < a.rows) qf[t] = *reinterpret_cast<const float4_t*>(qb + qrow * D + 16 * t + 4 * g);
    }
  }

  mfma_acc o[kT];
#pragma unroll
  for (int t = 0; t < kT; ++t) o[t] = mfma_acc{0.F, 0.F, 0.F, 0.F};
  const float neg_inf = -__builtin_inff();
  float m = neg_inf, l = 0.F;
  bool nan_row = false;
  const std::int64_t query = q0 + r;  // the query whose statistics this lane keeps

  // Tile staging: thread tid moves float4 f = tid + kThreads i (row f / (D/4)).
  float4_t kr[kLoads], vr[kLoads];
  auto fetch = [&](std::int64_t j0) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int f = tid + kThreads * i;
      const std::int64_t row = j0 + f / (D / 4);
      const int c = (f % (D / 4)) * 4;
      kr[i] = float4_t{0.F, 0.F, 0.F, 0.F};
      vr[i] = float4_t{0.F, 0.F, 0.F, 0.F};
      if (row < a.cols) {
        kr[i] = *reinterpret_cast<const float4_t*>(kb + row * D + c);
        vr[i] = *reinterpret_cast<const float4_t*>(vb + row * D + c);
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int f = tid + kThreads * i;
      const int row = f / (D / 4), c = (f % (D / 4)) * 4;
      *reinterpret_cast<float4_t*>(&ks[row * kLd + c]) = kr[i];
      *reinterpret_cast<float4_t*>(&vs[row * kLd + c]) = vr[i];
    }
  };

  const std::int64_t tiles = (a.cols + kKTile - 1) / kKTile;
  // Under causal masking tiles past the block's last query are not run.
  const std::int64_t run = a.causal ? min(tiles, q_last / kKTile + 1) : tiles;
  if (run > 0) fetch(0);
  for (std::int64_t tile = 0; tile < run; ++tile) {
    const std::int64_t j0 = tile * kKTile;
    __syncthreads();  // the previous tile's readers are done
    stage();
    __syncthreads();
    if (tile + 1 < run) fetch(j0 + kKTile);

    // S^T for 64 keys (4 blocks of 16) x the wave's 16 queries. The four
    // block accumulators take turns, so consecutive MFMAs are independent.
    mfma_acc s[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) s[b] = mfma_acc{0.F, 0.F, 0.F, 0.F};
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      float4_t kf[4];
#pragma unroll
      for (int b = 0; b < 4; ++b)
        kf[b] = *reinterpret_cast<const float4_t*>(&ks[(16 * b + r) * kLd + 16 * t + 4 * g]);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int b = 0; b < 4; ++b) s[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[b][e], qf[t][e], s[b], 0, 0, 0);
    }
    // Scores, masks and the tile maximum for query `query`: key j0 + kk is
    // kept when kk < limit (inside the sequence, and not after the query).
    std::int64_t lim = a.cols - j0;
    if (a.causal) lim = min(lim, query - j0 + 1);
    const int limit = static_cast<int>(max<std::int64_t>(min<std::int64_t>(lim, kKTile), 0));
    float tmax = neg_inf;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float product = s[b][v] * a.scale;
        float sc = product;
        if (16 * b + 4 * g + v >= limit) sc = neg_inf;
        if (is_nan(sc)) nan_row = true;
        s[b][v] = sc;
        tmax = fmaxf(tmax, sc);  // NaN never wins fmaxf; NaN rows are flagged
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m, tmax);
    const bool none = m_new == neg_inf;  // every key so far masked: p = 0
    const float alpha = none ? 1.F : exp_softmax(m - m_new);
    float psum = 0.F;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = none ? 0.F : exp_softmax(s[b][v] - m_new);
        s[b][v] = p;
        psum += p;
      }
    psum += __shfl_xor(psum, 16, kWave);
    psum += __shfl_xor(psum, 32, kWave);
    l = l * alpha + psum;
    m = m_new;
    // Rescale the output rows: lane l holds queries 4g + v of the tile.
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float av = __shfl(alpha, 4 * g + v, kWave);
#pragma unroll
      for (int t = 0; t < kT; ++t) o[t][v] *= av;
    }
    // O += P V: step (b, v) sums key 16b + 4g + v of lane group g; tile t
    // takes feature kT*r + t, so the lane's V operands are contiguous.
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float* vrow = &vs[(16 * b + 4 * g + v) * kLd + kT * r];
        float vv[kT];
        load_row<kT>(vrow, vv);
#pragma unroll
        for (int t = 0; t < kT; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(s[b][v], vv[t], o[t], 0, 0, 0);
      }
  }

  // Keys after every query of the block (p = 0): only a non-finite V there
  // changes the result. Thread tid always covers features 4 (tid % (D/4)) .. +3
  // (kThreads is a multiple of D/4).
  if (run < tiles) {
    const int c = (tid % (D / 4)) * 4;
    bool bad = false;
    for (std::int64_t row = run * kKTile + tid / (D / 4); row < a.cols; row += kThreads / (D / 4)) {
      const float4_t w = *reinterpret_cast<const float4_t*>(vb + row * D + c);
      bad = bad || !__builtin_isfinite(w.x) || !__builtin_isfinite(w.y) || !__builtin_isfinite(w.z) ||
            !__builtin_isfinite(w.w);
      if (bad) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (!__builtin_isfinite(w[e])) bad_column[c + e] = 1;  // same value from every writer
      }
    }
  }
  __syncthreads();  // bad_column is complete
  // Row statistics of the four lanes sharing a query agree; the NaN flag is
  // combined over them.
  int nan_bits = nan_row ? 1 : 0;
  nan_bits |= __shfl_xor(nan_bits, 16, kWave);
  nan_bits |= __shfl_xor(nan_bits, 32, kWave);
  float* __restrict__ ob = a.out + batch * a.rows * D;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int src = 4 * g + v;  // lane holding query 4g + v's statistics
    const float lv = __shfl(l, src, kWave);
    const float mv = __shfl(m, src, kWave);
    const int nv = __shfl(nan_bits, src, kWave);
    const std::int64_t qrow = q0 + 4 * g + v;
    if (qrow >= a.rows) continue;
    float y[kT];
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      if (nv || bad_column[kT * r + t]) y[t] = __builtin_nanf("");
      else if (mv == neg_inf) y[t] = o[t][v] * 0.F;  // 0 * V (NaN if V is not finite)
      else y[t] = o[t][v] / lv;
    }
    store_row<kT>(ob + qrow * D + kT * r, y);
  }
}

template <int D, int kWaves>
int launch_flash(const FlashArgs& a, std::int64_t batch, hipStream_t s) {
  constexpr int kQTile = 16 * kWaves;
  const std::int64_t qtiles = (a.rows + kQTile - 1) / kQTile;
  if (qtiles > 0x7fffffff || batch > 65535) return fail(TCX_INVALID_ARGUMENT, "attention grid is too large");
  hipLaunchKernelGGL((flash_attention_kernel<D, kWaves>),
                     dim3(static_cast<unsigned>(qtiles), static_cast<unsigned>(batch)), dim3(64 * kWaves), 0, s, a);
  return check(hipGetLastError(), "flash attention launch");
}

}  // namespace
}  // namespace tcx

extern "C" {

int tcx_hip_flash_attention_supported(int64_t features, int64_t value_features) {
  return features == value_features && (features == 32 || features == 64 || features == 128) ? 1 : 0;
}

int tcx_hip_flash_attention_f32(const float* q, const float* k, const float* v, float* out, int64_t batch,
                                int64_t rows, int64_t cols, int64_t features, float scale, int causal,
                                tcx_stream_t stream) {
  using namespace tcx;
  if (batch < 0 || rows < 0 || cols < 0) return fail(TCX_INVALID_ARGUMENT, "attention extents must be non-negative");
  if (!tcx_hip_flash_attention_supported(features, features))
    return fail(TCX_INVALID_ARGUMENT, "fused attention supports 32, 64 or 128 features");
  if (batch == 0 || rows == 0) return TCX_OK;
  if (q == nullptr || out == nullptr || (cols > 0 && (k == nullptr || v == nullptr)))
    return fail(TCX_INVALID_ARGUMENT, "attention buffers are null");
  for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(k), static_cast<const void*>(v),
                        static_cast<const void*>(out)})
    if (p != nullptr && (reinterpret_cast<std::uintptr_t>(p) & 15U) != 0)
      return fail(TCX_INVALID_ARGUMENT, "fused attention buffers must be 16-byte aligned");
  if (int rc = ready(); rc != TCX_OK) return rc;
  const FlashArgs a{q, k, v, out, rows, cols, scale, causal != 0};
  const auto s = static_cast<hipStream_t>(stream);
  if (a.causal) {
    if (features == 32) return launch_flash<32, kWavesCausal>(a, batch, s);
    if (features == 64) return launch_flash<64, kWavesCausal>(a, batch, s);
    return launch_flash<128, kWavesCausal>(a, batch, s);
  }
  if (features == 32) return launch_flash<32, kWavesFull>(a, batch, s);
  if (features == 64) return launch_flash<64, kWavesFull>(a, batch, s);
  return launch_flash<128, kWavesFull>(a, batch, s);
}

}  // extern "C"
