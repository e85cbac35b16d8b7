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
// Layout. A block owns 16 queries per wave of one batch matrix and walks the
// keys in tiles of kKeys (64, or 32 where two blocks must share a CU). K and V
// tiles go straight from HBM into LDS (buffer_load ... lds) and each tile's
// softmax overlaps the next tile's score MFMAs (details at the kernel). Each
// wave computes S^T = K Q^T for its 16 queries, so lane l holds
// S^T[key 16b + 4(l/16) + v][query l%16] (output layout of the MFMA): those
// are exactly the A operands (P[query l%16][key]) that the P V MFMAs need,
// when the k index of step (b, v) is taken as key 16b + 4(l/16) + v. The
// feature sum of S^T uses the same trick: lane l supplies features
// 16t + 4(l/16) + e of K and Q at step (t, e), read as one float4 each.
// Masked keys keep p = 0, so a non-finite V propagates as in the reference's
// P @ V: tiles the causal mask only partly covers run in full; a tile wholly
// after the block's last query skips the MFMAs and only marks the feature
// columns where its V rows hold a non-finite value (0 * inf or 0 * NaN is NaN
// in every output row of the block). Blocks start with the longest query
// tiles under causal masking.

#include "common.hpp"

namespace tcx {
namespace {

using mfma_acc = float __attribute__((ext_vector_type(4)));

struct FlashArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  std::int64_t rows, cols;
  std::int64_t qtiles, batch;  // work items: qtiles query tiles of each batch matrix
  float scale;
  int causal;
  int xcd_blocks;   // group the blocks of one batch matrix on one XCD
  int heavy_first;  // causal: more blocks than fit at once, heaviest first
};

using float2_t = float __attribute__((ext_vector_type(2)));

// N contiguous floats (N = 2, 4 or 8) with 8- or 16-byte stores.
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

// exp(x) for x <= 0 (or NaN) as exp2(x log2 e): rounding the product costs at
// most |t| 2^-24 ln 2 relative on a term exp(-t), 1e-6 for the terms above
// 2^-24 of the largest, far inside the reference's rtol 2e-4.
__device__ __forceinline__ float exp_attention(float x) {
  constexpr float kLog2e = 1.44269502F;  // float(log2 e)
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

// K/V tiles are loaded straight into LDS (buffer_load ... lds) and the loop
// is pipelined so that matrix cores stay busy through the softmax: while the scores of key tile j go through the softmax (VALU), the
// same wave's MFMAs already compute the scores of tile j + 1. K therefore runs
// one tile ahead of V: iteration j reads K tile j + 1 and V tile j, and loads
// K tile j + 2 and V tile j + 1 into the other halves of two-stage buffers,
// with one barrier per tile. Rows are unpadded and their 16-byte chunks
// XOR-swizzled by row (period 16), which keeps the K reads (16 rows, one
// chunk each) and the V reads (16 chunks of one row) conflict-free. Keys past
// the sequence read as zero (buffer range check).
template <int D>
__device__ __forceinline__ int kv_chunk(int row, int c) {
  if constexpr (D / 4 >= 16) return c ^ (row & 15);
  else return c ^ ((row >> 1) & 7);
}

// Output tile t of lane r holds feature output_feature(r, t): four
// consecutive features per 16-byte chunk, chunk r of each 64-feature half
// (features kT r + t for D = 32).
template <int kT>
__device__ __forceinline__ int output_feature(int r, int t) {
  if constexpr (kT >= 4) return 64 * (t / 4) + 4 * r + (t % 4);
  else return kT * r + t;
}

// Online-softmax state of a wave's 16 queries: the output accumulators in
// MFMA layout and the running maximum and sum (the lanes of query j hold its
// m and l).
template <int kT>
struct FlashState {
  mfma_acc o[kT];
  float m, l;
};

template <int kT>
__device__ __forceinline__ void flash_init(FlashState<kT>& st) {
#pragma unroll
  for (int t = 0; t < kT; ++t) st.o[t] = mfma_acc{0.F, 0.F, 0.F, 0.F};
  st.m = -__builtin_inff();
  st.l = 0.F;
}

// Key tiles [t_begin, t_end) of query tile `qtile` of batch matrix `batch`,
// folded into the state of the calling wave's 16 queries by the block's
// kWaves waves (thread tid) on two K and two V stages. kKeys keys per tile
// (64, or 32 to fit two blocks per CU), kB = kKeys / 16 MFMA blocks of keys.
// With scan_tail, the V rows after the range (keys the causal mask hides from
// every query of the tile) mark the feature columns holding an inf or NaN in
// bad_column, cleared by the caller. The segment opens with a barrier, so a
// segment may follow another on the same stages.

template <int D, int kWaves, int kKeys, bool kCausal>
__device__ __forceinline__ void flash_segment(const FlashArgs& a, float (&ks)[2][kKeys * D],
                                              float (&vs)[2][kKeys * D], int* bad_column, int tid,
                                              std::int64_t batch, std::int64_t qtile, std::int64_t t_begin,
                                              std::int64_t t_end, bool scan_tail, FlashState<D / 16>& st) {
  constexpr int kQTile = 16 * kWaves;
  constexpr int kT = D / 16;
  constexpr int kB = kKeys / 16;
  static_assert(kKeys == 32 || kKeys == 64);
  constexpr int kChunks = D / 4;                         // 16-byte chunks per K/V row
  constexpr int kRowsPerInst = 64 / kChunks;             // rows one wave instruction fills
  constexpr int kInst = kKeys / kRowsPerInst / kWaves;   // instructions per wave per K (or V) tile
  static_assert(D % 16 == 0 && kInst >= 1 && kInst * kRowsPerInst * kWaves == kKeys);
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const std::int64_t q0 = qtile * kQTile + wave * 16;
  const std::int64_t tiles = (a.cols + kKeys - 1) / kKeys;
  const float* __restrict__ qb = a.q + batch * a.rows * D;
  const float* __restrict__ kb = a.k + batch * a.cols * D;
  const float* __restrict__ vb = a.v + batch * a.cols * D;

  float4_t qf[kT];
  {
    const std::int64_t qrow = q0 + r;
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      // Unconditional loads (a row past the end reads row 0, then zero):
      // loads under a divergent branch would make the compiler wait for
      // every outstanding load inside the key loop.
      const std::int64_t qc = qrow < a.rows ? qrow : 0;
      qf[t] = *reinterpret_cast<const float4_t*>(qb + qc * D + 16 * t + 4 * g);
      if (qrow >= a.rows) qf[t] = float4_t{0.F, 0.F, 0.F, 0.F};
    }
  }
  mfma_acc (&o)[kT] = st.o;
  float& m = st.m;
  float& l = st.l;
  const float neg_inf = -__builtin_inff();
  const std::int64_t query = q0 + r;

  // DMA. Each tile is read through a buffer resource based at the tile's
  // first key row (64-bit address), whose num_records covers the keys left in
  // the sequence (at most one tile), so keys past the end read as zero and no
  // offset exceeds one tile. Instruction p of a wave fills rows
  // (p * kWaves + wave) * kRowsPerInst .. + kRowsPerInst - 1 of the tile;
  // lane i writes chunk slot i % kChunks of row i / kChunks, which holds
  // global chunk kv_chunk(row, slot).
  using int4v = int __attribute__((ext_vector_type(4)));
  auto rsrc_at = [&](const float* base, std::int64_t tile) {
    const std::int64_t j0 = tile * kKeys;
    const std::int64_t left = a.cols - j0;  // > 0 for every issued tile
    const int bytes = static_cast<int>((left < kKeys ? left : kKeys) * (D * 4));
    const auto addr = reinterpret_cast<std::uint64_t>(base + j0 * D);
    return int4v{static_cast<int>(addr), static_cast<int>(addr >> 32), bytes, 0x00020000};
  };
  int voff[kInst];
#pragma unroll
  for (int p = 0; p < kInst; ++p) {
    const int row = (p * kWaves + wave) * kRowsPerInst + lane / kChunks;
    voff[p] = (row * D + 4 * kv_chunk<D>(row, lane % kChunks)) * 4;
  }
  auto lds_of = [](const void* ptr) {
    return static_cast<unsigned>(reinterpret_cast<std::uintptr_t>((__attribute__((address_space(3))) const void*)ptr));
  };
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  auto dma16 = [](const int4v& rsrc, unsigned lds_byte, int off, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(lds_byte), "v"(off), "s"(rsrc), "s"(soff) : "memory", "m0");
  };
#pragma clang diagnostic pop
  auto issue = [&](const float* base, float* stage, std::int64_t tile) {
    const int4v rsrc = rsrc_at(base, tile);
#pragma unroll
    for (int p = 0; p < kInst; ++p) {
      const unsigned row_byte = static_cast<unsigned>((p * kWaves + wave) * kRowsPerInst * D * 4);
      dma16(rsrc, lds_of(stage) + row_byte, voff[p], 0);
    }
  };

  // Lane exchanges: xor 16 inside each half-wave (swizzle, bit-mask mode:
  // and 0x1f, xor 0x10), xor 32 and the broadcast of query 4g + v's factor
  // to lane group g through precomputed permute addresses.
  auto xor16 = [](float x) { return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), 0x401f)); };
  const int xor32_addr = (lane ^ 32) << 2;
  auto xor32 = [&](float x) { return __int_as_float(__builtin_amdgcn_ds_bpermute(xor32_addr, __float_as_int(x))); };
  int row_addr[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) row_addr[v] = (4 * g + v) << 2;

  // Fragment reads. K: the kB 16-key blocks of feature group t (lane (r, g)
  // reads chunk 4t + g of key 16b + r). V: key row 16b + 4g + v, features
  // output_feature(r, t): chunks r, 16 + r, ... (half of chunk r / 2 for
  // D = 32), so the 16 lanes of a row read 16 different chunks.
  auto read_k = [&](const float* __restrict__ kt_, int t, float4_t (&kf)[kB]) {
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int row = 16 * b + r;
      kf[b] = *reinterpret_cast<const float4_t*>(&kt_[row * D + 4 * kv_chunk<D>(row, 4 * t + g)]);
    }
  };
  auto read_v = [&](const float* __restrict__ vt_, int step, float (&vv)[kT]) {
    const int row = 16 * (step / 4) + 4 * g + step % 4;
    if constexpr (kT >= 4) {
#pragma unroll
      for (int h = 0; h < kT / 4; ++h) {
        const float4_t w = *reinterpret_cast<const float4_t*>(&vt_[row * D + 4 * kv_chunk<D>(row, 16 * h + r)]);
        vv[4 * h] = w.x; vv[4 * h + 1] = w.y; vv[4 * h + 2] = w.z; vv[4 * h + 3] = w.w;
      }
    } else {
      const float2_t w =
          *reinterpret_cast<const float2_t*>(&vt_[row * D + 4 * kv_chunk<D>(row, r / 2) + 2 * (r % 2)]);
      vv[0] = w.x; vv[1] = w.y;
    }
  };

  // The online softmax of one tile as kSteps small steps, so that they can be
  // spread between the MFMAs of the next tile's scores (kB = 4 numbering):
  //   0-3       scale (and mask) of key block b, running tile maximum
  //   4         row maximum over the four lane groups, new running maximum,
  //             rescale factor alpha
  //   5         alpha of query 4g + v to lane group g
  //   6..5+kT   rescale output tile t
  //   6+kT..9+kT  p = exp(s - max) of key block b, partial row sum
  //   10+kT     row sum over the lane groups, l and m updated
  // Every key so far masked (m_new = -inf): the finite stand-in m_sub keeps
  // p = exp(-inf) = 0 without a per-score select, and alpha = 0 leaves the
  // zero rows zero (or NaN). A NaN score is skipped by fmaxf but gives p = NaN,
  // so l and the whole row turn NaN; so does a +inf score (inf - inf).
  constexpr int kSteps = 2 * kB + 3 + kT;
  float tmax = neg_inf, m_new = neg_inf, m_sub = 0.F, alpha = 1.F, psum = 0.F;
  float av[4];
  int limit = kKeys;
  auto begin_tile = [&](std::int64_t tile) {
    const std::int64_t j0 = tile * kKeys;
    std::int64_t lim = a.cols - j0;
    if constexpr (kCausal) {
      if (query - j0 + 1 < lim) lim = query - j0 + 1;
    }
    limit = static_cast<int>(lim < 0 ? 0 : (lim > kKeys ? kKeys : lim));
    tmax = neg_inf;
    psum = 0.F;
  };
  // kMask: the tile may hold keys past the sequence or after the query.
  auto step = [&]<int I, bool kMask>(mfma_acc (&s)[kB]) {
    if constexpr (I < kB) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float sc = s[I][v] * a.scale;
        if constexpr (kMask) {
          if (16 * I + 4 * g + v >= limit) sc = neg_inf;
        }
        s[I][v] = sc;
        tmax = fmaxf(tmax, sc);
      }
    } else if constexpr (I == kB) {
      tmax = fmaxf(tmax, xor16(tmax));
      tmax = fmaxf(tmax, xor32(tmax));
      m_new = fmaxf(m, tmax);
      m_sub = m_new == neg_inf ? 0.F : m_new;
      alpha = exp_attention(m - m_sub);
    } else if constexpr (I == kB + 1) {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        av[v] = __int_as_float(__builtin_amdgcn_ds_bpermute(row_addr[v], __float_as_int(alpha)));
    } else if constexpr (I < kB + 2 + kT) {
#pragma unroll
      for (int v = 0; v < 4; ++v) o[I - kB - 2][v] *= av[v];
    } else if constexpr (I < 2 * kB + 2 + kT) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float p = exp_attention(s[I - kB - 2 - kT][v] - m_sub);
        s[I - kB - 2 - kT][v] = p;
        psum += p;
      }
    } else {
      psum += xor16(psum);
      psum += xor32(psum);
      l = l * alpha + psum;
      m = m_new;
    }
  };
  auto all_steps = [&]<int... I>(mfma_acc (&s)[kB], std::integer_sequence<int, I...>) {
    (step.template operator()<I, true>(s), ...);
  };

  // O += P V in 4 kB steps (key 16b + 4g + v of lane group g at step 4b + v),
  // each reading the next step's V operands before its own MFMAs.
  auto accumulate = [&]<int... I>(const float* __restrict__ vt_, const mfma_acc (&p)[kB], float (&vv)[2][kT],
                                  std::integer_sequence<int, I...>) {
    auto one = [&]<int J>() {
      if constexpr (J + 1 < 4 * kB) read_v(vt_, J + 1, vv[(J + 1) & 1]);
#pragma unroll
      for (int t = 0; t < kT; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(p[J / 4][J % 4], vv[J & 1][t], o[t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    };
    (one.template operator()<I>(), ...);
  };

  // The next tile's scores in kQuads = kT kB quads of four MFMAs (feature
  // group t = J / kB, k steps 4 / kB (J % kB) .. + 4 / kB - 1, every key
  // block), with softmax step I of the current tile in quad I kQuads / kSteps
  // and the K reads of group t + 1 in the first quad of group t; the last quad
  // also reads the first P V step's V operands.
  constexpr int kQuads = kT * kB;
  auto scores_with_softmax = [&]<bool kMask, int... Q>(const float* __restrict__ kt_, const float* __restrict__ vt_,
                                                       mfma_acc (&s_next)[kB], mfma_acc (&s)[kB],
                                                       float4_t (&kf)[2][kB], float (&vv)[2][kT],
                                                       std::bool_constant<kMask>, std::integer_sequence<int, Q...>) {
    auto quad = [&]<int J>() {
      constexpr int t = J / kB, e0 = (J % kB) * (4 / kB);
      if constexpr (J % kB == 0 && t + 1 < kT) read_k(kt_, t + 1, kf[(t + 1) & 1]);
      if constexpr (J == kQuads - 1) read_v(vt_, 0, vv[0]);
#pragma unroll
      for (int e = e0; e < e0 + 4 / kB; ++e)
#pragma unroll
        for (int b = 0; b < kB; ++b)
          s_next[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[t & 1][b][e], qf[t][e], s_next[b], 0, 0, 0);
      [&]<int... I>(std::integer_sequence<int, I...>) {
        ([&] {
          if constexpr (I * kQuads / kSteps == J) step.template operator()<I, kMask>(s);
        }(), ...);
      }(std::make_integer_sequence<int, kSteps>{});
      __builtin_amdgcn_sched_barrier(0);
    };
    (quad.template operator()<Q>(), ...);
  };
  // Scores of one tile without interleaving (first tile).
  auto scores = [&](const float* __restrict__ kt_, mfma_acc (&s)[kB]) {
#pragma unroll
    for (int b = 0; b < kB; ++b) s[b] = mfma_acc{0.F, 0.F, 0.F, 0.F};
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      float4_t kf[kB];
      read_k(kt_, t, kf);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int b = 0; b < kB; ++b) s[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[b][e], qf[t][e], s[b], 0, 0, 0);
    }
  };

  // Every tile but the last of the segment is full unless masked causally.
  mfma_acc s_cur[kB], s_next[kB];
  float4_t kf[2][kB];
  float vv[2][kT];
  // The stages may still be read by this team's previous segment.
  __syncthreads();
  if (t_begin < t_end) {
    issue(kb, ks[0], t_begin);
    issue(vb, vs[0], t_begin);
    if (t_begin + 1 < t_end) issue(kb, ks[1], t_begin + 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // K 0, V 0 and K 1 have landed
    scores(ks[0], s_cur);
    __syncthreads();  // every wave is done with K stage 0
  } else {
    __syncthreads();
  }
  // Iteration `tile` (stage parity counted from t_begin): K tile + 1 sits in
  // stage (tile + 1) & 1, V tile in stage tile & 1; K tile + 2 and V tile + 1
  // load into the other stages, whose last readers finished before the
  // previous barrier.
  std::int64_t tile = t_begin;
  for (; tile + 1 < t_end; ++tile) {
    const int st = static_cast<int>((tile - t_begin) & 1);
    issue(vb, vs[st ^ 1], tile + 1);
    if (tile + 2 < t_end) issue(kb, ks[st], tile + 2);
    begin_tile(tile);
#pragma unroll
    for (int b = 0; b < kB; ++b) s_next[b] = mfma_acc{0.F, 0.F, 0.F, 0.F};
    read_k(ks[st ^ 1], 0, kf[0]);
    // Under causal masking only tiles reaching past the block's first query
    // need the mask: a wave-uniform branch between two schedules at D = 128
    // (+2 %). At D = 64 the second schedule raised the register count from
    // 127 to 157, which costs a block per CU (-18 %), so D < 128 masks all.
    if (kCausal && (D < 128 || (tile + 1) * kKeys - 1 > qtile * kQTile))
      scores_with_softmax(ks[st ^ 1], vs[st], s_next, s_cur, kf, vv, std::true_type{},
                          std::make_integer_sequence<int, kQuads>{});
    else
      scores_with_softmax(ks[st ^ 1], vs[st], s_next, s_cur, kf, vv, std::false_type{},
                          std::make_integer_sequence<int, kQuads>{});
    accumulate(vs[st], s_cur, vv, std::make_integer_sequence<int, 4 * kB>{});
#pragma unroll
    for (int b = 0; b < kB; ++b) s_cur[b] = s_next[b];
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads have landed
    __syncthreads();                // and every wave is done with this iteration's stages
  }
  if (tile < t_end) {
    const int st = static_cast<int>((tile - t_begin) & 1);
    begin_tile(tile);
    all_steps(s_cur, std::make_integer_sequence<int, kSteps>{});
    read_v(vs[st], 0, vv[0]);
    accumulate(vs[st], s_cur, vv, std::make_integer_sequence<int, 4 * kB>{});
  }

  if (scan_tail && t_end < tiles) {
    // Columns of the V rows past the last run tile that hold an inf or NaN
    // (exponent all ones), eight independent loads in flight per thread and
    // no branch in the loop (a branch on each load's value serialised the
    // scan behind the load latency: 10 % of the causal kernel at D = 32).
    const int c = (tid % (D / 4)) * 4;
    constexpr int kPass = (64 * kWaves) / (D / 4);  // rows per pass of the block
    constexpr unsigned kExp = 0x7f800000U;
    unsigned flag[4] = {0U, 0U, 0U, 0U};
    auto mark = [&](const float4_t& w) {
#pragma unroll
      for (int e = 0; e < 4; ++e) flag[e] |= (__float_as_uint(w[e]) & kExp) == kExp ? 1U : 0U;
    };
    std::int64_t row = t_end * kKeys + tid / (D / 4);
    for (; row + 7 * kPass < a.cols; row += 8 * kPass) {
      float4_t w[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = *reinterpret_cast<const float4_t*>(vb + (row + u * kPass) * D + c);
#pragma unroll
      for (int u = 0; u < 8; ++u) mark(w[u]);
    }
    for (; row < a.cols; row += kPass) mark(*reinterpret_cast<const float4_t*>(vb + row * D + c));
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (flag[e]) bad_column[c + e] = 1;
  }
}

// Stores the calling wave's 16 output rows of query tile `qtile` from its
// state (NaN in the columns bad_column marks, 0 * V for an all-masked row).
template <int D, int kWaves>
__device__ __forceinline__ void flash_store(const FlashArgs& a, const int* bad_column, int tid, std::int64_t batch,
                                            std::int64_t qtile, const FlashState<D / 16>& st) {
  constexpr int kT = D / 16;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, g = lane >> 4;
  const std::int64_t q0 = qtile * (16 * kWaves) + wave * 16;
  const float neg_inf = -__builtin_inff();
  float* __restrict__ ob = a.out + batch * a.rows * D;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int src = 4 * g + v;
    const float lv = __shfl(st.l, src, kWave);
    const float mv = __shfl(st.m, src, kWave);
    const std::int64_t qrow = q0 + 4 * g + v;
    if (qrow >= a.rows) continue;
    float y[kT];
#pragma unroll
    for (int t = 0; t < kT; ++t) {
      if (bad_column[output_feature<kT>(r, t)]) y[t] = __builtin_nanf("");
      else if (mv == neg_inf) y[t] = st.o[t][v] * 0.F;
      else y[t] = st.o[t][v] / lv;
    }
    float* const orow = ob + qrow * D;
    if constexpr (kT >= 4) {
#pragma unroll
      for (int h = 0; h < kT / 4; ++h)
        *reinterpret_cast<float4_t*>(orow + output_feature<kT>(r, 4 * h)) =
            float4_t{y[4 * h], y[4 * h + 1], y[4 * h + 2], y[4 * h + 3]};
    } else {
      store_row<kT>(orow + kT * r, y);
    }
  }
}

// One block per query tile.
template <int D, int kWaves, int kKeys, bool kCausal>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 8))) void flash_attention_kernel(
    FlashArgs a) {
  constexpr int kQTile = 16 * kWaves;
  __shared__ float ks[2][kKeys * D];
  __shared__ float vs[2][kKeys * D];
  __shared__ int bad_column[D];
  const int tid = threadIdx.x;
  // One block per work item on a 1-D grid of n = qtiles x batch blocks; the
  // launch id maps to an item (batch-major by default).
  const std::int64_t n = a.qtiles * a.batch;
  const std::int64_t id = blockIdx.x;
  std::int64_t batch = id / a.qtiles, qtile = id % a.qtiles;
  if (a.xcd_blocks) {
    // Launch id L runs on XCD L % 8: give XCD x the consecutive (batch-major)
    // work items x * n/8 .. (x + 1) * n/8 - 1, so that the query tiles of one
    // batch matrix share its K and V in that XCD's L2 (n % 8 == 0).
    const std::int64_t item = (id % 8) * (n / 8) + id / 8;
    batch = item / a.qtiles;
    qtile = item % a.qtiles;
  }
  if constexpr (kCausal) {
    // Under causal masking the last query tiles see the most keys. Work items
    // are ranked by their key-tile count. When every block fits on the device
    // at once, the first half of the grid takes them heaviest first and the
    // second half lightest first, so the two blocks that share a CU (launch
    // ids L and L + n/2) carry about the same total work. With more blocks
    // than fit, the grid runs heaviest first throughout, so that the light
    // items fill the CUs the heavy ones leave (longest job first: 16 x 4096 x
    // 128 720 -> 658 us, 48 x 2048 x 128 536 -> 482 us on MI355X).
    const std::int64_t half = (n + 1) / 2;
    const std::int64_t rank = a.heavy_first || id < half ? id : n - 1 - (id - half);
    qtile = a.qtiles - 1 - rank / a.batch;
    batch = rank % a.batch;
  }
  const std::int64_t q_last = min(qtile * kQTile + kQTile, a.rows) - 1;
  const std::int64_t tiles = (a.cols + kKeys - 1) / kKeys;
  // Under causal masking tiles past the block's last query are not run.
  const std::int64_t run = kCausal ? min(tiles, q_last / kKeys + 1) : tiles;
  for (int d = tid; d < D; d += 64 * kWaves) bad_column[d] = 0;
  FlashState<D / 16> st;
  flash_init(st);
  flash_segment<D, kWaves, kKeys, kCausal>(a, ks, vs, bad_column, tid, batch, qtile, 0, run, true, st);
  __syncthreads();
  flash_store<D, kWaves>(a, bad_column, tid, batch, qtile, st);
}

template <int D, int kWaves, int kKeys, bool kCausal>
int launch_flash(FlashArgs a, std::int64_t batch, hipStream_t s) {
  constexpr int kQTile = 16 * kWaves;
  a.qtiles = (a.rows + kQTile - 1) / kQTile;
  a.batch = batch;
  if (a.qtiles > 0x7fffffff / batch) return fail(TCX_INVALID_ARGUMENT, "attention grid is too large");
  const std::int64_t blocks = a.qtiles * batch;
  // Causal blocks keep their heavy/light order instead.
  a.xcd_blocks = !kCausal && blocks % 8 == 0 ? 1 : 0;
  if constexpr (kCausal) {
    thread_local int slots = 0;
    if (slots == 0) {
      int per_cu = 0, cus = 0, device = 0;
      (void)hipGetDevice(&device);
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || cus < 1)
        cus = 256;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, flash_attention_kernel<D, kWaves, kKeys, kCausal>,
                                                        64 * kWaves, 0) != hipSuccess ||
          per_cu < 1)
        per_cu = 2;
      slots = per_cu * cus;
    }
    a.heavy_first = blocks > slots ? 1 : 0;
  }
  hipLaunchKernelGGL((flash_attention_kernel<D, kWaves, kKeys, kCausal>), dim3(static_cast<unsigned>(blocks)),
                     dim3(64 * kWaves), 0, s, a);
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
  const FlashArgs a{q, k, v, out, rows, cols, 0, 0, scale, causal != 0, 0, 0};
  const auto s = static_cast<hipStream_t>(stream);
  // Tile shapes measured on MI355X at 2048 x 2048. Unmasked: 8 waves and
  // 64-key tiles for D = 128 and 64 (one block per CU at D = 128: 110 against
  // 107 TFLOP/s with 4 waves and 32-key tiles), 4 waves and 32-key tiles for
  // D = 32 (94 against 90). Causal: 4 waves and 32-key tiles (64 KB of LDS at
  // D = 128), so that two blocks share each CU in the heavy/light order (89
  // TFLOP/s at 16 x 2048 x 128 against 86 for a register-staged 4-wave kernel,
  // 92 against 71 at 32 x 2048 x 64).
  if (a.causal) {
    if (features == 32) return launch_flash<32, 4, 32, true>(a, batch, s);
    if (features == 64) return launch_flash<64, 4, 32, true>(a, batch, s);
    return launch_flash<128, 4, 32, true>(a, batch, s);
  }
  if (features == 32) return launch_flash<32, 4, 32, false>(a, batch, s);
  if (features == 64) return launch_flash<64, 8, 64, false>(a, batch, s);
  return launch_flash<128, 8, 64, false>(a, batch, s);
}

}  // extern "C"
