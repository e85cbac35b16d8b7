// fp32 MFMA GEMM kernel template (v_mfma_f32_16x16x4_f32); included by
// gemm.hip, which owns the C entry point and the per-shape tile choice.
#pragma once

#include <type_traits>

#include "common.hpp"


namespace tcx {
namespace gemm {

struct GemmArgs {
  const float* lhs;
  const float* rhs;
  float* out;
  const float* bias;
  std::int64_t m, n, k;
  std::int64_t tiles_m, tiles_n, total_tiles;
  std::int32_t batch_rank, activation;
  std::int64_t batch_shape[TCX_HIP_MAX_BATCH_RANK];
  std::int64_t lhs_bs[TCX_HIP_MAX_BATCH_RANK];
  std::int64_t rhs_bs[TCX_HIP_MAX_BATCH_RANK];
  // Direct kernel with a K split: `splits` blocks per output tile each sum
  // K / splits of k and write their partial tile to partial[split] (laid out
  // like out); split_reduce_kernel then adds them. splits <= 1: no split.
  std::int32_t splits;
  float* partial;
};

using floatx4 = float __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float activate(float v, int act) {
  if (act == TCX_ACT_SILU) return v / (1.0F + expf(-v));
  if (act == TCX_ACT_GELU) {
    // Same operation order as cpu_backend.cpp:1000-1003.
    const float cubic = 0.044715F * v * v * v;
    const float inner = 0.7978845608028654F * (v + cubic);
    return 0.5F * v * (1.0F + tanhf(inner));
  }
  return v;
}

// Position inside a wave tile of element e (0 <= e < T) owned by MFMA lane
// row/column r (0..15) for a T-wide fragment. For T >= 4 the elements come in
// float4 groups 64 positions apart, so the 16 lanes sharing a k read 256
// contiguous bytes per group (one conflict-free ds_read_b128 each); for T = 2
// a lane's pair is adjacent.
template <int T>
__device__ __forceinline__ int frag_pos(int r, int e) {
  if constexpr (T >= 4)
    return (e >> 2) * 64 + r * 4 + (e & 3);
  else
    return r * T + e;
}

// XOR swizzle of the m (or n) index of tiles stored transposed (k-major from
// k-contiguous global rows), with rows padded by 8 floats: the k-quad (k/4)
// flips bits 3-4 of m for 16-wide k-tiles and bits 2-4 for 32-wide ones. With
// the thread-to-element map of load_tile the scalar transposed stores of a
// 32-wide k-tile land on distinct banks (SQ_LDS_BANK_CONFLICT reads 0 for
// them), and an XOR by a multiple of 4 keeps every aligned group of 4
// contiguous for the 16-byte fragment reads.
template <int BK>
__device__ __forceinline__ int swz(int k, int m) {
  return m ^ (((k >> 2) & 7) << (BK >= 32 ? 2 : 3));
}

// Reads the T fragment values of lane row r from LDS row `row` (already
// offset to the wave tile); `sw` is the row's swizzle (0 when unswizzled).
template <int T>
__device__ __forceinline__ void load_frag(const float* row, int r, int sw, float (&v)[T]) {
  if constexpr (T >= 4) {
#pragma unroll
    for (int g = 0; g < T / 4; ++g) {
      const float4_t t = *reinterpret_cast<const float4_t*>(row + ((g * 64 + r * 4) ^ sw));
      v[4 * g] = t.x; v[4 * g + 1] = t.y; v[4 * g + 2] = t.z; v[4 * g + 3] = t.w;
    }
  } else {
    const float2 t = *reinterpret_cast<const float2*>(row + ((r * T) ^ sw));
    v[0] = t.x; v[1] = t.y;
  }
}

// KS > 1 splits K inside the block: KS groups of waves each cover the whole
// block tile, group g taking rows [g*BK, (g+1)*BK) of every staged k-tile of
// KS*BK, and the groups' partial tiles are added through LDS in group order at
// the end (deterministic). It multiplies the waves per CU for shapes with few
// output tiles without any extra HBM traffic.
template <int BM, int BN, int BK, int WM, int WN, int kMinWaves, bool kTransB, bool kVec, int KS = 1>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64 * KS)
__attribute__((amdgpu_waves_per_eu(kMinWaves, 8))) void gemm_f32_kernel(GemmArgs a) {
  constexpr int kWavesN = BN / WN;
  constexpr int kGroupWaves = (BM / WM) * kWavesN;  // waves covering the block tile once
  constexpr int kThreads = kGroupWaves * 64 * KS;
  constexpr int BKT = BK * KS;  // k extent staged per iteration
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int LDA = BM + 8, LDB = BN + 8;
  static_assert(BK % 4 == 0 && (BM * BKT) % (4 * kThreads) == 0 && (BN * BKT) % (4 * kThreads) == 0);
  constexpr int kAVec = BM * BKT / 4 / kThreads;  // float4 loads per thread for A
  constexpr int kBVec = BN * BKT / 4 / kThreads;
  constexpr int kAScalar = BM * BKT / kThreads;
  constexpr int kBScalar = BN * BKT / kThreads;
  constexpr int kAReg = kVec ? kAVec * 4 : kAScalar;
  constexpr int kBReg = kVec ? kBVec * 4 : kBScalar;
  constexpr int kElems = TM * TN * 4;  // accumulator floats per lane
  constexpr int kStage = 2 * BKT * (LDA + LDB);
  constexpr int kReduce = (KS - 1) * kGroupWaves * kElems * 64;

  // Two staging buffers for A and B; after the k loop the same memory holds
  // the split-K partial tiles.
  __shared__ float smem[kStage > kReduce ? kStage : kReduce];
  auto As = reinterpret_cast<float (*)[BKT][LDA]>(smem);
  auto Bs = reinterpret_cast<float (*)[BKT][LDB]>(smem + 2 * BKT * LDA);

  // Blocks go round-robin to the 8 XCDs; give each XCD a contiguous run of
  // tile ids so the blocks sharing an L2 also share A row panels and B column
  // panels. The remap is a bijection when the grid is a multiple of 8.
  const std::int64_t grid = a.total_tiles;
  const std::int64_t bid = blockIdx.x;
  const std::int64_t tile = (grid % 8 == 0) ? (bid % 8) * (grid / 8) + bid / 8 : bid;
  const std::int64_t per_batch = a.tiles_m * a.tiles_n;
  const std::int64_t batch = tile / per_batch;
  const std::int64_t t = tile % per_batch;
  constexpr std::int64_t kGroupM = 8;
  const std::int64_t group_tiles = kGroupM * a.tiles_n;
  const std::int64_t first_m = (t / group_tiles) * kGroupM;
  const std::int64_t gm = min(a.tiles_m - first_m, kGroupM);
  const std::int64_t tm = first_m + (t % group_tiles) % gm;
  const std::int64_t tn = (t % group_tiles) / gm;

  std::int64_t lhs_off = 0, rhs_off = 0;
  {
    std::int64_t b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
  }
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const float* __restrict__ A = a.lhs + lhs_off;
  const float* __restrict__ B = a.rhs + rhs_off;
  float* __restrict__ C = a.out + batch * M * N;
  const std::int64_t m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x;
  float ra[kAReg], rb[kBReg];

  // Global -> registers for k-tile starting at k0 (zero outside the matrix).
  auto load_tile = [&](std::int64_t k0) {
    if constexpr (kVec) {
#pragma unroll
      for (int p = 0; p < kAVec; ++p) {
        const int idx = tid + p * kThreads;
        const int row = idx / (BKT / 4), kq = idx % (BKT / 4);
        const std::int64_t gm_ = m0 + row, gk = k0 + kq * 4;
        float4_t v = {0.F, 0.F, 0.F, 0.F};
        if (gm_ < M && gk < K) v = *reinterpret_cast<const float4_t*>(A + gm_ * K + gk);
        ra[4 * p + 0] = v.x; ra[4 * p + 1] = v.y; ra[4 * p + 2] = v.z; ra[4 * p + 3] = v.w;
      }
#pragma unroll
      for (int p = 0; p < kBVec; ++p) {
        const int idx = tid + p * kThreads;
        float4_t v = {0.F, 0.F, 0.F, 0.F};
        if constexpr (kTransB) {
          const int row = idx / (BKT / 4), kq = idx % (BKT / 4);
          const std::int64_t gn = n0 + row, gk = k0 + kq * 4;
          if (gn < N && gk < K) v = *reinterpret_cast<const float4_t*>(B + gn * K + gk);
        } else {
          const int krow = idx / (BN / 4), nq = idx % (BN / 4);
          const std::int64_t gk = k0 + krow, gn = n0 + nq * 4;
          if (gk < K && gn < N) v = *reinterpret_cast<const float4_t*>(B + gk * N + gn);
        }
        rb[4 * p + 0] = v.x; rb[4 * p + 1] = v.y; rb[4 * p + 2] = v.z; rb[4 * p + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int p = 0; p < kAScalar; ++p) {
        const int idx = tid + p * kThreads;
        const int row = idx / BKT, kk = idx % BKT;
        const std::int64_t gm_ = m0 + row, gk = k0 + kk;
        ra[p] = (gm_ < M && gk < K) ? A[gm_ * K + gk] : 0.F;
      }
#pragma unroll
      for (int p = 0; p < kBScalar; ++p) {
        const int idx = tid + p * kThreads;
        if constexpr (kTransB) {
          const int row = idx / BKT, kk = idx % BKT;
          const std::int64_t gn = n0 + row, gk = k0 + kk;
          rb[p] = (gn < N && gk < K) ? B[gn * K + gk] : 0.F;
        } else {
          const int krow = idx / BN, nn = idx % BN;
          const std::int64_t gk = k0 + krow, gn = n0 + nn;
          rb[p] = (gk < K && gn < N) ? B[gk * N + gn] : 0.F;
        }
      }
    }
  };

  // Registers -> LDS buffer `buf`, A and (transposed) B stored k-major.
  auto store_tile = [&](int buf) {
    if constexpr (kVec) {
#pragma unroll
      for (int p = 0; p < kAVec; ++p) {
        const int idx = tid + p * kThreads;
        const int row = idx / (BKT / 4), kq = idx % (BKT / 4);
#pragma unroll
        for (int q = 0; q < 4; ++q) As[buf][kq * 4 + q][swz<BKT>(kq * 4 + q, row)] = ra[4 * p + q];
      }
#pragma unroll
      for (int p = 0; p < kBVec; ++p) {
        const int idx = tid + p * kThreads;
        if constexpr (kTransB) {
          const int row = idx / (BKT / 4), kq = idx % (BKT / 4);
#pragma unroll
          for (int q = 0; q < 4; ++q) Bs[buf][kq * 4 + q][swz<BKT>(kq * 4 + q, row)] = rb[4 * p + q];
        } else {
          const int krow = idx / (BN / 4), nq = idx % (BN / 4);
          const float4_t v = {rb[4 * p], rb[4 * p + 1], rb[4 * p + 2], rb[4 * p + 3]};
          *reinterpret_cast<float4_t*>(&Bs[buf][krow][nq * 4]) = v;
        }
      }
    } else {
#pragma unroll
      for (int p = 0; p < kAScalar; ++p) {
        const int idx = tid + p * kThreads;
        As[buf][idx % BKT][swz<BKT>(idx % BKT, idx / BKT)] = ra[p];
      }
#pragma unroll
      for (int p = 0; p < kBScalar; ++p) {
        const int idx = tid + p * kThreads;
        if constexpr (kTransB)
          Bs[buf][idx % BKT][swz<BKT>(idx % BKT, idx / BKT)] = rb[p];
        else
          Bs[buf][idx / BN][idx % BN] = rb[p];
      }
    }
  };

  const int lane = tid & 63, wave = tid >> 6;
  const int group = wave / kGroupWaves, gwave = wave % kGroupWaves;
  const int wm = gwave / kWavesN, wn = gwave % kWavesN;
  const int r = lane & 15, kl = lane >> 4;
  floatx4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.F, 0.F, 0.F, 0.F};

  // Tile kt+1 sits in registers while tile kt's MFMAs run; its LDS stores
  // and the global loads of tile kt+2 both go before the barrier, so after
  // the barrier a wave only waits for its first fragment reads.
  const std::int64_t k_tiles = (K + BKT - 1) / BKT;
  if (k_tiles > 0) {
    load_tile(0);
    store_tile(0);
    if (k_tiles > 1) load_tile(BKT);
    __syncthreads();
  }
  for (std::int64_t kt = 0; kt < k_tiles; ++kt) {
    const int buf = static_cast<int>(kt & 1);
#pragma unroll
    for (int s = 0; s < BK / 4; ++s) {
      const int k = group * BK + s * 4 + kl;
      const int sw = swz<BKT>(k, 0);
      float av[TM], bv[TN];
      load_frag<TM>(&As[buf][k][wm * WM], r, sw, av);
      load_frag<TN>(&Bs[buf][k][wn * WN], r, kTransB ? sw : 0, bv);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < k_tiles) store_tile(buf ^ 1);
    if (kt + 2 < k_tiles) load_tile((kt + 2) * BKT);
    __syncthreads();
  }
  if constexpr (KS > 1) {
    // Groups 1..KS-1 hand their partial tiles to group 0 through LDS (free
    // after the loop's last barrier, or unused when K == 0); group 0 adds
    // them in group order and alone runs the epilogue.
    float* red = smem;
    auto slot = [&](int g, int i, int j, int q) {
      return (((g - 1) * kGroupWaves + gwave) * kElems + (i * TN + j) * 4 + q) * 64 + lane;
    };
    if (group > 0) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) red[slot(group, i, j, q)] = acc[i][j][q];
    }
    __syncthreads();
    if (group > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[i][j][q] += red[slot(g, i, j, q)];
  }

  // Epilogue: bias add then activation, as kAdd then kSilu/kGelu would round.
  // Register q of block (i, j) holds tile row frag_pos<TM>(4*kl + q, i) and
  // tile column frag_pos<TN>(r, j).
  const std::int64_t col_base = n0 + wn * WN;
  float bias[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const std::int64_t col = col_base + frag_pos<TN>(r, j);
    bias[j] = (a.bias != nullptr && col < N) ? a.bias[col] : 0.F;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const std::int64_t row = m0 + wm * WM + frag_pos<TM>(kl * 4 + q, i);
      if (row >= M) continue;
      float v[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float x = acc[i][j][q];
        if (a.bias != nullptr) x = x + bias[j];
        v[j] = activate(x, a.activation);
      }
      float* dst = C + row * N + col_base;
      if constexpr (TN >= 4) {
#pragma unroll
        for (int g = 0; g < TN / 4; ++g) {
          const std::int64_t col = g * 64 + r * 4;
          if (kVec && col_base + col + 3 < N) {
            *reinterpret_cast<float4_t*>(dst + col) = float4_t{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (col_base + col + e < N) dst[col + e] = v[4 * g + e];
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = frag_pos<TN>(r, j);
          if (col_base + col < N) dst[col] = v[j];
        }
      }
    }
  }
}

// Full-tile GEMM with global -> LDS direct loads (buffer_load ... lds), for
// B given as [k, n] or transposed, when every tile is full and rows are
// 16-byte aligned (128x128 tiles for every such shape of >= 256 tiles and for
// the K split; the template also builds 256x256 tiles). Each tile's loads are
// issued into the other LDS stage right after a barrier and land while the
// current stage's MFMAs run: no staging registers, no LDS store
// instructions, no wait before the barrier beyond the loads themselves.
//
// LDS layout: A m-major ([m][k], the eight 16-byte chunks of a 32-wide row
// XOR-swizzled by (m / 2) % 8, so both the DMA writes and the fragment reads
// are conflict-free), a [k, n] B k-major with unpadded rows, a transposed B
// like A. A fragment read of a [k, n] B gives each 16-lane group 256
// contiguous bytes of one k row: conflict-free with rows 4 * BN bytes apart,
// two cycles per pass with rows padded by 8 floats (SQ_LDS_BANK_CONFLICT was
// 40 % of SQ_LDS_IDX_ACTIVE at 4096^3 with the padding). One wave instruction fills 8 rows of A (64 lanes x
// 16 B, contiguous) or one k row of a [k, n] B (64 lanes for 256 columns,
// the first 32 for 128). A lane reads 4 consecutive k of one A row in one ds_read_b128, so inside
// each 16-k group MFMA step s of lane group kl uses k = 4 * kl + s for A and B
// alike (a permutation of the k order, covered by the parity bound).
//
// The two stages are separate LDS arrays and the k loop handles them in
// pairs. The loads are issued as assembly: the compiler adds no waits for
// them, and the loop waits (vmcnt 0) right before each barrier.
template <int BM, int BN, int BK, int WM, int WN, int kMinWaves, bool kTransB>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64)
__attribute__((amdgpu_waves_per_eu(kMinWaves, 8))) void gemm_f32_direct_kernel(GemmArgs a) {
  constexpr int kWavesN = BN / WN, kWaves = (BM / WM) * kWavesN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int LDB = BN;
  constexpr int kChunks = BK / 4;
  // A [k, n] B takes one k row per wave instruction (all 64 lanes for 256
  // floats, the first 32 for 128) and 16-byte output stores; a transposed B
  // is loaded like A (8 rows per instruction).
  static_assert(kChunks == 8 && (kTransB || ((BN == 256 || BN == 128) && TN % 4 == 0)),
                "one wave instruction = 8 rows of A or one row of B");
  constexpr int kARows = 64 / kChunks;          // A rows per wave instruction
  constexpr int kAInst = BM / kARows / kWaves;  // A instructions per wave and tile
  // B instructions per wave and tile: one k-row each ([k, n] B), or 8
  // n-rows each for a transposed B stored like A.
  constexpr int kBInst = kTransB ? BN / kARows / kWaves : BK / kWaves;
  static_assert(kAInst * kARows * kWaves == BM && (kTransB ? kBInst * kARows * kWaves == BN : kBInst * kWaves == BK));
  using BTile = std::conditional_t<kTransB, float[BN][BK], float[BK][LDB]>;
  __shared__ float A0[BM][BK], A1[BM][BK];
  __shared__ BTile B0, B1;

  // Work items are (split, batch, tile), split-major, in the XCD-aware tile
  // order of gemm_f32_kernel. A grid of fewer blocks than items is persistent:
  // block b runs XCD b % 8's items (b / 8) + j (gridDim / 8), so each round
  // of an XCD's blocks covers consecutive items that share panels in its L2.
  // Item counts fit 31 bits (the launcher checks). The transposed-B variant
  // runs one item per block: its loop state would not fit the registers left
  // beside the 252 it uses (the persistent build reloaded spills in the k loop).
  constexpr bool kPersist = !kTransB;
  const int items = static_cast<int>(a.total_tiles);
  const int blocks = static_cast<int>(gridDim.x), bid = static_cast<int>(blockIdx.x);
  int item = bid, item_step = blocks, item_end = items;
  if (items % 8 == 0 && blocks % 8 == 0) {
    const int xcd = bid % 8, xcd_items = items / 8;
    item = xcd * xcd_items + bid / 8;
    item_step = blocks / 8;
    item_end = (xcd + 1) * xcd_items;
  }
  const int splits = a.splits > 1 ? a.splits : 1;
  const int per_split = items / splits;
  const int per_batch = static_cast<int>(a.tiles_m * a.tiles_n);
  const int tiles_m = static_cast<int>(a.tiles_m), tiles_n = static_cast<int>(a.tiles_n);
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const bool partial = splits > 1;
  // Each item's k range: [k_base, k_base + K / splits).
  const int k_len = static_cast<int>(K / splits);

  using int4v = int __attribute__((ext_vector_type(4)));
  auto rsrc_of = [](const float* base) {
    const auto addr = reinterpret_cast<std::uint64_t>(base);
    return int4v{static_cast<int>(addr), static_cast<int>(addr >> 32), 0x7fffffff, 0x00020000};
  };
  // Per-item state: buffer resources based at the item's A row panel and B
  // column panel (32-bit byte offsets per lane and a scalar offset per
  // instruction and tile; the launcher checks that both panels span less than
  // 2^31 bytes), its k base and the origin of its output tile.
  int4v a_rsrc{}, b_rsrc{};
  int k_base = 0, tile_n0 = 0;
  float* out_tile = nullptr;
  auto setup = [&](int it) {
    const int split = it / per_split;
    const int tile = it - split * per_split;
    const int batch = tile / per_batch;
    const int t = tile - batch * per_batch;
    constexpr int kGroupM = 8;
    const int group_tiles = kGroupM * tiles_n;
    const int first_m = (t / group_tiles) * kGroupM;
    const int gm = min(tiles_m - first_m, kGroupM);
    const int tm = first_m + (t % group_tiles) % gm;
    const int tn = (t % group_tiles) / gm;
    std::int64_t lhs_off = 0, rhs_off = 0;
    int b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const int e = static_cast<int>(a.batch_shape[ax]);
      const int c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
    const std::int64_t m0 = static_cast<std::int64_t>(tm) * BM, n0 = static_cast<std::int64_t>(tn) * BN;
    float* const c_mat = partial ? a.partial + (static_cast<std::int64_t>(split) * (per_split / per_batch) + batch) * M * N
                                 : a.out + static_cast<std::int64_t>(batch) * M * N;
    out_tile = c_mat + m0 * N + n0;
    tile_n0 = tn * BN;
    k_base = split * k_len;
    a_rsrc = rsrc_of(a.lhs + lhs_off + m0 * K);
    b_rsrc = rsrc_of(kTransB ? a.rhs + rhs_off + n0 * K : a.rhs + rhs_off + n0);
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  auto achunk = [](int row, int kc) { return kc ^ ((row >> 1) & 7); };

  // Lane of instruction p writes A row (p * kWaves + wave) * 8 + lane / 8; the
  // chunk swizzle of that row does not depend on p.
  const int a_row = wave * kARows + lane / kChunks;
  const int a_voff = (a_row * static_cast<int>(K) + 4 * achunk(a_row, lane % kChunks)) * 4;
  const int b_row = a_row;  // transposed B: same lane map as A over n rows
  const int b_voff = kTransB ? (b_row * static_cast<int>(K) + 4 * achunk(b_row, lane % kChunks)) * 4
                             : (wave * static_cast<int>(N) + 4 * lane) * 4;
  auto lds_of = [](const void* p) {
    return static_cast<unsigned>(reinterpret_cast<std::uintptr_t>((__attribute__((address_space(3))) const void*)p));
  };
  // 16 bytes per lane from rsrc + voff + soff into LDS at lds_byte + 16 * lane.
  // M0 is reserved by the compiler (clang warns about naming it) and only
  // these loads use it here; listing it records that the asm writes it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  auto dma16 = [](const int4v& rsrc, unsigned lds_byte, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(lds_byte), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
  };
#pragma clang diagnostic pop
  auto issue = [&](float (&As)[BM][BK], BTile& Bs, int k_rel) {
    const int k0 = k_base + k_rel;
    __builtin_amdgcn_sched_barrier(0);
    const unsigned a_lds = lds_of(&As[0][0]) + static_cast<unsigned>(wave * kARows * BK * 4);
#pragma unroll
    for (int p = 0; p < kAInst; ++p)
      dma16(a_rsrc, a_lds + p * kWaves * kARows * BK * 4, a_voff,
            __builtin_amdgcn_readfirstlane((p * kWaves * kARows * static_cast<int>(K) + k0) * 4));
    if constexpr (kTransB) {
      const unsigned b_lds = lds_of(&Bs[0][0]) + static_cast<unsigned>(wave * kARows * BK * 4);
#pragma unroll
      for (int p = 0; p < kBInst; ++p)
        dma16(b_rsrc, b_lds + p * kWaves * kARows * BK * 4, b_voff,
              __builtin_amdgcn_readfirstlane((p * kWaves * kARows * static_cast<int>(K) + k0) * 4));
    } else {
      const unsigned b_lds = lds_of(&Bs[0][0]) + static_cast<unsigned>(wave * LDB * 4);
#pragma unroll
      for (int p = 0; p < kBInst; ++p) {
        const int soff = __builtin_amdgcn_readfirstlane((p * kWaves + k0) * static_cast<int>(N) * 4);
        // Lanes past the row stay off: the DMA writes LDS at M0 + 16 * lane,
        // which for them would be the next row.
        if (BN == 256 || lane < BN / 4) dma16(b_rsrc, b_lds + p * kWaves * LDB * 4, b_voff, soff);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int r = lane & 15, kl = lane >> 4;
  floatx4 acc[TM][TN];

  // Block i of the wave covers tile rows 16 i + (0..15). B columns keep the
  // frag_pos map for a [k, n] B (16-byte fragment reads and output stores);
  // a transposed B is read like A, block j covering columns 16 j + (0..15).
  auto compute = [&](const float (&As)[BM][BK], const BTile& Bs) {
#pragma unroll
    for (int g = 0; g < BK / 16; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      float4_t a4[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WM + 16 * i + r;
        a4[i] = *reinterpret_cast<const float4_t*>(&As[row][achunk(row, g * 4 + kl) * 4]);
      }
      if constexpr (kTransB) {
        float4_t b4[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int col = wn * WN + 16 * j + r;
          b4[j] = *reinterpret_cast<const float4_t*>(&Bs[col][achunk(col, g * 4 + kl) * 4]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i][s], b4[j][s], acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          float bv[TN];
          load_frag<TN>(&Bs[g * 16 + 4 * kl + s][wn * WN], r, 0, bv);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i][s], bv[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  };

  const int k_tiles = k_len / BK;
  setup(item);  // gridDim <= items: every block has a first item
  issue(A0, B0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const std::int64_t col_off = wn * WN;
  auto col_of = [&](int jj) { return kTransB ? 16 * jj + r : frag_pos<TN>(r, jj); };
  for (;;) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int jj = 0; jj < TN; ++jj) acc[i][jj] = floatx4{0.F, 0.F, 0.F, 0.F};
    // Pairs of k-tiles: stage 0 is read while stage 1 loads, then the reverse.
    int kt = 0;
    for (; kt + 2 <= k_tiles; kt += 2) {
      issue(A1, B1, (kt + 1) * BK);
      compute(A0, B0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (kt + 2 < k_tiles) issue(A0, B0, (kt + 2) * BK);
      compute(A1, B1);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    if (kt < k_tiles) compute(A0, B0);  // odd count: the last tile sits in stage 0

    // Epilogue as in gemm_f32_kernel (full tiles: no bounds checks); a split
    // item stores its raw partial sums. The next item's first k-tile is
    // issued before the stores, and only those loads are waited for: the
    // vector memory counter completes in issue order, so vmcnt(stores) leaves
    // this item's stores draining under the next item's MFMAs.
    float* const out_c = out_tile + static_cast<std::int64_t>(wm * WM + kl * 4) * N + col_off;
    const bool epilogue = !partial;
    const bool with_bias = epilogue && a.bias != nullptr;
    float bias[TN];
#pragma unroll
    for (int jj = 0; jj < TN; ++jj) bias[jj] = with_bias ? a.bias[tile_n0 + col_off + col_of(jj)] : 0.F;
    item += item_step;
    const bool next = kPersist && item < item_end;
    if (next) {
      // The bias loads complete here, before the tile loads go out, so that
      // waiting for them does not wait for those loads.
      if (with_bias) __builtin_amdgcn_s_waitcnt(0);
      if (k_tiles % 2 != 0) __syncthreads();  // every wave is done reading stage 0
      setup(item);
      issue(A0, B0, 0);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int row = 16 * i + q;  // + wm WM + 4 kl, in out_c
        float v[TN];
#pragma unroll
        for (int jj = 0; jj < TN; ++jj) {
          float x = acc[i][jj][q];
          if (epilogue) {
            if (with_bias) x = x + bias[jj];
            x = activate(x, a.activation);
          }
          v[jj] = x;
        }
        float* dst = out_c + row * N;
        if constexpr (kTransB) {
#pragma unroll
          for (int jj = 0; jj < TN; ++jj) dst[16 * jj + r] = v[jj];
        } else {
#pragma unroll
          for (int g = 0; g < TN / 4; ++g)
            *reinterpret_cast<float4_t*>(dst + g * 64 + r * 4) =
                float4_t{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
        }
      }
    }
    if (!next) break;
    // Stores per wave: TM * 4 rows of TN / 4 16-byte stores (TN 4-byte stores
    // for a transposed B); the count field holds at most 63.
    constexpr int kStores = kTransB ? TM * 4 * TN : TM * 4 * (TN / 4);
    constexpr int kVm = kStores < 63 ? kStores : 63;
    __builtin_amdgcn_s_waitcnt((kVm & 15) | (7 << 4) | (15 << 8) | ((kVm >> 4) << 14));
    __syncthreads();
  }
}

// out = act(partial[0] + ... + partial[splits - 1] (+ bias)) for the K-split
// direct GEMM, the partial sums added in split order and the bias after them
// (the unsplit epilogue's order: full sum, bias, activation). count4 float4s
// of out; n % 4 == 0.
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ partial, float* __restrict__ out,
                                                           const float* __restrict__ bias, std::int64_t count4,
                                                           std::int64_t n, int splits, int act) {
  const auto* p4 = reinterpret_cast<const float4_t*>(partial);
  auto* o4 = reinterpret_cast<float4_t*>(out);
  for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * 256 + threadIdx.x; i < count4;
       i += static_cast<std::int64_t>(gridDim.x) * 256) {
    float4_t v = stream_load(p4 + i);
    for (int sp = 1; sp < splits; ++sp) v += stream_load(p4 + sp * count4 + i);
    if (bias != nullptr) {
      const float* b = bias + (4 * i) % n;  // any alignment
      v += float4_t{b[0], b[1], b[2], b[3]};
    }
    o4[i] = float4_t{activate(v.x, act), activate(v.y, act), activate(v.z, act), activate(v.w, act)};
  }
}

// True when gemm_f32_direct_kernel<BM, BN, BK, ...> can take the problem:
// full tiles, k > 0, and byte offsets inside one A row panel (BM x K) and one
// B column panel (K x N, or BN x K transposed) below 2^31.
template <int BM, int BN, int BK>
bool direct_fits(std::int64_t m, std::int64_t n, std::int64_t k) {
  return m % BM == 0 && n % BN == 0 && k % BK == 0 && k > 0 &&
         static_cast<double>(BM) * k * 4 < 2147483647.0 && static_cast<double>(k) * n * 4 < 2147483647.0;
}

// Launches the direct kernel; with splits > 1 (K % (BK * splits) == 0 and a
// workspace of splits x batches x m x n floats in args.partial) it runs
// splits blocks per tile over K / splits each, then split_reduce_kernel.
template <int BM, int BN, int BK, int WM, int WN, int kMinWaves>
int launch_direct(GemmArgs& args, bool trans_b, hipStream_t stream) {
  if (!direct_fits<BM, BN, BK>(args.m, args.n, args.k))
    return fail(TCX_INTERNAL, "direct gemm needs full tiles and 31-bit panel offsets");
  const std::int64_t splits = args.splits > 1 ? args.splits : 1;
  if (splits > 1 && (args.k % (BK * splits) != 0 || args.partial == nullptr))
    return fail(TCX_INTERNAL, "split gemm needs K a multiple of the split k-tiles and a workspace");
  const std::int64_t batches = args.total_tiles;  // caller passes the batch count
  args.tiles_m = args.m / BM;
  args.tiles_n = args.n / BN;
  args.total_tiles = args.tiles_m * args.tiles_n * batches * splits;
  if (args.total_tiles > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  const int threads = (BM / WM) * (BN / WN) * 64;
  std::int64_t blocks = args.total_tiles;
  // A [k, n] B needs 256- or 128-wide tiles of 4-column fragments.
  constexpr bool kKnB = (BN == 256 || BN == 128) && (WN / 16) % 4 == 0;
  if constexpr (kKnB) {
    // [k, n] B with more items than blocks that fit at once: a persistent
    // grid of that many blocks (batched 32 x 1024^3: 512 items on 256 CUs,
    // two per block).
    thread_local int fit = 0;
    if (fit == 0) {
      int per_cu = 0, cus = 0, device = 0;
      (void)hipGetDevice(&device);
      (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, gemm_f32_direct_kernel<BM, BN, BK, WM, WN, kMinWaves, false>, threads, 0) != hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      fit = per_cu * (cus > 0 ? cus : 256);
    }
    if (!trans_b && blocks > fit) blocks = fit;
  }
  const dim3 grid(static_cast<unsigned>(blocks)), block(threads);
  if constexpr (kKnB) {
    if (trans_b)
      hipLaunchKernelGGL((gemm_f32_direct_kernel<BM, BN, BK, WM, WN, kMinWaves, true>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((gemm_f32_direct_kernel<BM, BN, BK, WM, WN, kMinWaves, false>), grid, block, 0, stream, args);
  } else {
    if (!trans_b) return fail(TCX_INTERNAL, "this direct gemm tile takes a transposed B only");
    hipLaunchKernelGGL((gemm_f32_direct_kernel<BM, BN, BK, WM, WN, kMinWaves, true>), grid, block, 0, stream, args);
  }
  int rc = check(hipGetLastError(), "gemm_f32 direct launch");
  if (rc != TCX_OK || splits == 1) return rc;
  const std::int64_t count4 = batches * args.m * args.n / 4;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(grid_for(count4, 256, 256 * 16)), dim3(256), 0, stream, args.partial,
                     args.out, args.bias, count4, args.n, static_cast<int>(splits), args.activation);
  return check(hipGetLastError(), "gemm_f32 split reduce launch");
}

// Direct-to-LDS GEMM for BM x 64 output tiles of any shape (edge tiles
// included), BM = 64 or 32: BM / 4 waves in four K groups of BM / 16 32x32
// waves, each group taking 16 of every 64 staged k (its partial tile is added
// in group order at the end, as in gemm_f32_kernel with KS = 4). Tiles go from
// HBM to LDS with buffer_load ... lds. 64x64 tiles: 16 waves, four stages
// (128 KB, one block per CU), two k-tiles between barriers, two 16-byte
// instructions per wave and stage. 32x64 tiles: 8 waves, three stages (72 KB,
// two blocks per CU), one k-tile per barrier with two in flight, three
// instructions per wave and stage. The half-height tiles serve launches whose
// last round of 64x64 tiles would be mostly empty: the blocks of that round
// then run half the work each, alone on their CUs.
//   Edges: each operand panel is read through a buffer resource whose
//   num_records ends at the matrix, so rows past M (and past N for a
//   transposed B) read as zero through the VGPR offset alone. Lanes whose k
//   is past K in an A row (or a transposed B row), and lanes of a [k, n] B
//   whose k row is past K or whose column chunk is past N, get an
//   out-of-range VGPR offset and read zero too: a value past K, which may be
//   infinite (the next batch's B rows, say), never meets the zero of the
//   other operand, and no load leaves the operand's own rows.
//   LDS layouts (conflict-free reads): A [BM rows][64 k] (a transposed B
//   [64 rows][64 k])
//   with the 16-byte chunk c of row r at c ^ (r & 15); a [k, n] B
//   [64 k][64 n] with chunk c of k row kr at c ^ (8 ((kr >> 2) & 1)), which
//   puts the two k rows one 32-lane read pass takes in opposite halves of
//   the banks.
//   Output column of MFMA column r in block j: 32 wn + 2r + j for a [k, n] B
//   (a lane's two columns are adjacent, one 8-byte read per k), 32 wn + 16j +
//   r for a transposed B.
template <bool kTransB, int BM>
__global__ __launch_bounds__(16 * BM) __attribute__((amdgpu_waves_per_eu(4, 8))) void gemm_f32_direct64_kernel(
    GemmArgs a) {
  static_assert(BM == 64 || BM == 32);
  constexpr int BN = 64, KS = 4, BKT = 64, kStages = BM == 64 ? 4 : 3;
  constexpr int kWaves = BM / 4, kGroupWaves = kWaves / KS;
  constexpr int kBInst = 64 / (4 * kWaves);  // B instructions per wave and stage
  constexpr std::int64_t kGroupM = 512 / BM;  // tile rows per group: 512 rows of A
  // One array, so that the group reduction can span both operands' stages.
  __shared__ float smem[kStages * (BM + 64) * BKT];
  auto As = reinterpret_cast<float (*)[BM][BKT]>(smem);
  auto Bs = reinterpret_cast<float (*)[64][64]>(smem + kStages * BM * BKT);  // [n][k] transposed, [k][n] otherwise

  const std::int64_t grid = a.total_tiles;
  const std::int64_t bid = blockIdx.x;
  const std::int64_t tile = (grid % 8 == 0) ? (bid % 8) * (grid / 8) + bid / 8 : bid;
  const std::int64_t per_batch = a.tiles_m * a.tiles_n;
  const std::int64_t batch = tile / per_batch;
  const std::int64_t t = tile % per_batch;
  const std::int64_t group_tiles = kGroupM * a.tiles_n;
  const std::int64_t first_m = (t / group_tiles) * kGroupM;
  const std::int64_t gm = min(a.tiles_m - first_m, kGroupM);
  const std::int64_t tm = first_m + (t % group_tiles) % gm;
  const std::int64_t tn = (t % group_tiles) / gm;
  std::int64_t lhs_off = 0, rhs_off = 0;
  {
    std::int64_t b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
  }
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const float* __restrict__ A = a.lhs + lhs_off;
  const float* __restrict__ B = a.rhs + rhs_off;
  float* __restrict__ C = a.out + batch * M * N;
  const std::int64_t m0 = tm * BM, n0 = tn * BN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave / kGroupWaves, gwave = wave % kGroupWaves;
  const int wm = gwave / 2, wn = gwave % 2;
  const int r = lane & 15, kl = lane >> 4;

  using int4v = int __attribute__((ext_vector_type(4)));
  auto rsrc_of = [](const float* base, std::int64_t bytes) {
    const auto addr = reinterpret_cast<std::uint64_t>(base);
    return int4v{static_cast<int>(addr), static_cast<int>(addr >> 32), static_cast<int>(bytes), 0x00020000};
  };
  // Panels: A rows m0.. (M - m0 rows), B columns n0.. (a [k, n] B: through
  // its last element) or rows n0.. (transposed: N - n0 rows). The launcher
  // checks that every panel spans less than 2^31 bytes.
  const int4v a_rsrc = rsrc_of(A + m0 * K, (M - m0) * K * 4);
  const int4v b_rsrc = kTransB ? rsrc_of(B + n0 * K, (N - n0) * K * 4) : rsrc_of(B + n0, (K * N - n0) * 4);
  // Instruction of wave w: rows 4w .. 4w + 3 of the stage's A tile and rows
  // 4 kWaves h + 4w .. + 3 of its B tile (h < kBInst); lane i fills chunk slot
  // i % 16 of row 4w + i / 16 (+ 4 kWaves h). The chunk swizzles read the
  // row's low five bits, which 4 kWaves h (0 or 32) leaves alone, so a lane's
  // B rows share one chunk.
  const int row = 4 * wave + lane / 16, slot = lane % 16;
  const int a_chunk = slot ^ (row & 15);
  const int a_voff = (row * static_cast<int>(K) + 4 * a_chunk) * 4;
  const int b_chunk = kTransB ? a_chunk : slot ^ (8 * ((row >> 2) & 1));
  int b_voff[kBInst];
#pragma unroll
  for (int h = 0; h < kBInst; ++h) {
    const int b_row = 4 * kWaves * h + row;
    b_voff[h] = (b_row * static_cast<int>(kTransB ? K : N) + 4 * b_chunk) * 4;
  }
  auto lds_of = [](const void* p) {
    return static_cast<unsigned>(reinterpret_cast<std::uintptr_t>((__attribute__((address_space(3))) const void*)p));
  };
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  auto dma16 = [](const int4v& rsrc, unsigned lds_byte, int voff, int soff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(lds_byte), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
  };
#pragma clang diagnostic pop
  // An offset past every panel (voff + soff stays below 2^32): a zero read.
  constexpr int kOut = 0x7fffffff;
  auto issue = [&](int stage, int k0) {
    const unsigned row_byte = static_cast<unsigned>(4 * wave * 64 * 4);
    const bool a_in = k0 + 4 * a_chunk < K;
    dma16(a_rsrc, lds_of(&As[stage][0][0]) + row_byte, a_in ? a_voff : kOut, __builtin_amdgcn_readfirstlane(k0 * 4));
#pragma unroll
    for (int h = 0; h < kBInst; ++h) {
      const unsigned b_byte = row_byte + static_cast<unsigned>(4 * kWaves * h * 64 * 4);
      if constexpr (kTransB) {
        dma16(b_rsrc, lds_of(&Bs[stage][0][0]) + b_byte, a_in ? b_voff[h] : kOut,
              __builtin_amdgcn_readfirstlane(k0 * 4));
      } else {
        // k rows past K and column chunks past N take the out-of-range
        // offset on the VGPR side alone, so the zero fill does not depend on
        // whether the range check counts the SGPR offset.
        const bool b_in = k0 + 4 * kWaves * h + row < K && n0 + 4 * b_chunk < N;
        dma16(b_rsrc, lds_of(&Bs[stage][0][0]) + b_byte, b_in ? b_voff[h] : kOut,
              __builtin_amdgcn_readfirstlane(k0 * static_cast<int>(N) * 4));
      }
    }
  };

  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.F, 0.F, 0.F, 0.F};
  // A wave's operands of one k-tile: a[i][q] and b[j][q] feed the MFMA of
  // block (i, j) at k step q.
  struct Frag {
    float4_t a[2], b[2];
  };
  auto load = [&](int stage, Frag& f) {
    const int kc = group * 4 + kl;  // this lane's k chunk of the group's 16 k
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ar = wm * 32 + 16 * i + r;
      f.a[i] = *reinterpret_cast<const float4_t*>(&As[stage][ar][4 * (kc ^ (ar & 15))]);
    }
    if constexpr (kTransB) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int bc = wn * 32 + 16 * j + r;
        f.b[j] = *reinterpret_cast<const float4_t*>(&Bs[stage][bc][4 * (kc ^ (bc & 15))]);
      }
    } else {
      // Indexing the stage as 8-byte pairs keeps every read a ds_read_b64
      // (as float offsets the compiler split the q > 0 reads into
      // ds_read2_b32, whose single-dword passes put the k rows of lane
      // groups kl and kl + 2 on the same banks).
      using float2v = float __attribute__((ext_vector_type(2)));
      const auto* pairs = reinterpret_cast<const float2v*>(&Bs[stage][0][0]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kr = group * 16 + 4 * kl + q;
        const int c = wn * 8 + r / 2;  // chunk of columns 32 wn + 2r, + 1
        const float2v bv = pairs[kr * 32 + 2 * (c ^ (8 * ((kr >> 2) & 1))) + (r & 1)];
        f.b[0][q] = bv.x;
        f.b[1][q] = bv.y;
      }
    }
  };
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][q], f.b[j][q], acc[i][j], 0, 0, 0);
  };
  auto compute = [&](int stage) {
    Frag f;
    load(stage, f);
    mma(f);
  };

  const int k_tiles = static_cast<int>((K + BKT - 1) / BKT);
  if constexpr (BM == 32) {
    // One k-tile per barrier over three stages, two tiles in flight: the
    // barrier of tile kt frees the stage of tile kt - 1 for tile kt + 2. The
    // other block on the CU covers this block's barrier waits.
    issue(0, 0);
    if (k_tiles > 1) issue(1, BKT);
    for (int kt = 0; kt < k_tiles; ++kt) {
      if (kt + 1 < k_tiles) __builtin_amdgcn_s_waitcnt(0x0F70 | (kBInst + 1));  // tile kt + 1 may still be out
      else __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (kt + 2 < k_tiles) issue((kt + 2) % kStages, (kt + 2) * BKT);
      compute(kt % kStages);
    }
  } else {
  // Two k-tiles per barrier over four stages: tiles kt and kt + 1 are read
  // between two barriers while tiles kt + 2 and kt + 3 land in the stages of
  // kt - 2 and kt - 1, free since the last barrier. Each wave runs 32 MFMAs
  // between barriers and a load has two tiles' MFMAs to land (one tile per
  // barrier, three tiles ahead, measured 26.0 against 24.0 us at 1000^3).
  // Each wave has two loads per tile in flight.
  for (int p = 0; p < kStages && p < k_tiles; ++p) issue(p, p * BKT);
  int kt0 = 0;
  if (k_tiles >= 4) {
    // The first pair starts as soon as tile 0 has landed; tile 1 lands
    // under tile 0's MFMAs, tiles 2 and 3 under tile 1's (one barrier more;
    // 1000^3 24.2 -> 24.0 us, 1024^3 23.5 -> 23.1 us).
    __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6): tile 0
    __syncthreads();
    compute(0);
    __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4): tile 1
    __syncthreads();
    compute(1);
    __builtin_amdgcn_s_waitcnt(0);  // tiles 2 and 3
    __syncthreads();
    kt0 = 2;
  } else {
    // Tiles 0 and 1 have landed: vmcnt(4) with four tiles in flight, vmcnt(2)
    // with three.
    if (k_tiles > 3) __builtin_amdgcn_s_waitcnt(0x0F74);
    else if (k_tiles == 3) __builtin_amdgcn_s_waitcnt(0x0F72);
    else __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (int kt = kt0; kt < k_tiles; kt += 2) {
    if (kt >= 2 && kt + 2 < k_tiles) issue((kt + 2) % kStages, (kt + 2) * BKT);
    if (kt >= 2 && kt + 3 < k_tiles) issue((kt + 3) % kStages, (kt + 3) * BKT);
    // Both tiles' fragment reads go out before the first MFMA (the stage of
    // a missing odd tile is read but not used): the second tile's reads land
    // under the first tile's MFMAs (1000^3: 23.8 -> 23.55 us).
    Frag f0, f1;
    load(kt % kStages, f0);
    load((kt + 1) % kStages, f1);
    __builtin_amdgcn_sched_barrier(0);
    mma(f0);
    if (kt + 1 < k_tiles) mma(f1);
    __builtin_amdgcn_s_waitcnt(0);  // tiles kt + 2 and kt + 3 have landed
    __syncthreads();
  }
  }
  if constexpr (BM == 32) __syncthreads();  // every wave is done with the stages

  // Every group passes its partial tile through LDS (the stages are free
  // after the last barrier); group g then adds the four partials of rows
  // 16 g .. 16 g + 15 of its tile in group order (the sum order of an
  // unsplit k loop over the groups' ranges, the same bits whichever group
  // adds) and stores them, so the adds and stores are spread over all
  // waves.
  float* red = smem;  // KS x kGroupWaves waves x 64 lanes x 16 floats: 64 or 32 KB
  auto red_at = [&](int g, int w, int i, int j, int q, int ln) {
    return red + ((((g * kGroupWaves + w) * 16 + (i * 2 + j) * 4 + q) * 64) + ln);
  };
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) *red_at(group, gwave, i, j, q, lane) = acc[i][j][q];
  __syncthreads();
  // This wave now owns the outputs of (wave gwave, i, q) = rows
  // wm * 32 + 16 i + 4 kl + q of the tile handled by wave gwave of every
  // group, for the q given by its group: q == group.
  const int q = group;
  auto col_of = [&](int j) { return kTransB ? 16 * j + r : 2 * r + j; };
  float bias[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const std::int64_t col = n0 + wn * 32 + col_of(j);
    bias[j] = a.bias != nullptr && col < N ? a.bias[col] : 0.F;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const std::int64_t orow = m0 + wm * 32 + 16 * i + 4 * kl + q;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float x = *red_at(0, gwave, i, j, q, lane);
#pragma unroll
      for (int g = 1; g < KS; ++g) x += *red_at(g, gwave, i, j, q, lane);
      const std::int64_t col = n0 + wn * 32 + col_of(j);
      if (orow >= M || col >= N) continue;
      if (a.bias != nullptr) x = x + bias[j];
      C[orow * N + col] = activate(x, a.activation);
    }
  }
}

// True when gemm_f32_direct64_kernel can take the problem: 16-byte rows
// (k and n multiples of 4, 16-byte aligned operands, checked by the caller)
// and every byte offset into a panel, a tile's 64 rows included, below 2^31.
inline bool direct64_fits(std::int64_t m, std::int64_t n, std::int64_t k) {
  constexpr double kLimit = 2147483647.0;
  const double rows_m = static_cast<double>(m < 64 ? 64 : m), rows_n = static_cast<double>(n < 64 ? 64 : n);
  return m > 0 && n > 0 && k > 0 && k % 4 == 0 && n % 4 == 0 && rows_m * k * 4 < kLimit &&
         rows_n * k * 4 < kLimit && (static_cast<double>(k) + 64) * n * 4 < kLimit;
}

// half: 32x64 tiles instead of 64x64.
inline int launch_direct64(GemmArgs& args, bool trans_b, bool half, hipStream_t stream) {
  if (!direct64_fits(args.m, args.n, args.k))
    return fail(TCX_INTERNAL, "direct 64x64 gemm needs 16-byte rows and 31-bit panel offsets");
  const int bm = half ? 32 : 64;
  args.tiles_m = (args.m + bm - 1) / bm;
  args.tiles_n = (args.n + 63) / 64;
  args.total_tiles = args.tiles_m * args.tiles_n * args.total_tiles;  // caller passes the batch count
  if (args.total_tiles > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  const dim3 grid(static_cast<unsigned>(args.total_tiles)), block(16 * bm);
  if (half && trans_b)
    hipLaunchKernelGGL((gemm_f32_direct64_kernel<true, 32>), grid, block, 0, stream, args);
  else if (half)
    hipLaunchKernelGGL((gemm_f32_direct64_kernel<false, 32>), grid, block, 0, stream, args);
  else if (trans_b)
    hipLaunchKernelGGL((gemm_f32_direct64_kernel<true, 64>), grid, block, 0, stream, args);
  else
    hipLaunchKernelGGL((gemm_f32_direct64_kernel<false, 64>), grid, block, 0, stream, args);
  return check(hipGetLastError(), "gemm_f32 direct 64-column tile launch");
}

// Small GEMMs (fewer than 128 output tiles of 64x64): one 32x32 output tile
// per block of KS waves, the waves splitting K into KS contiguous runs of
// 16-k chunks. A wave loads its own operands straight into registers (A and
// a transposed B: one 16-byte load per lane, 16-row block and chunk; a
// [k, n] B: four 8-byte loads per chunk, a lane's two columns adjacent), kG
// chunks per load group and two groups in flight, so a K of up to 64 KS
// takes one memory round trip, with no LDS staging and no barrier before the
// epilogue. MFMA step q of chunk c takes k = 16 c + 4 (lane / 16) + q, as in
// the other kernels. The partial tiles meet in LDS and are added in wave
// order (a fixed order for a given KS), with bias and activation, by all KS
// waves.
//   Edges as in gemm_f32_direct64_kernel: buffer resources end at the
// operand panels, so rows past M or N read zero; lanes past K, [k, n] B
// columns past N and chunks past the wave's run take an out-of-range offset
// (zero, no memory access), so every group issues the same loads.
template <bool kTransB, int KS, int kG>
__global__ __launch_bounds__(64 * KS) void gemm_f32_small_kernel(GemmArgs a) {
  const std::int64_t per_batch = a.tiles_m * a.tiles_n;
  const std::int64_t grid = a.total_tiles;
  const std::int64_t bid = blockIdx.x;
  // Consecutive tiles per XCD (launch id L runs on XCD L % 8), grouped eight
  // tile rows deep, so an XCD's blocks share A and B panels in its L2.
  const std::int64_t tile = grid % 8 == 0 ? (bid % 8) * (grid / 8) + bid / 8 : bid;
  const std::int64_t batch = tile / per_batch, t = tile % per_batch;
  constexpr std::int64_t kGroupM = 8;
  const std::int64_t group_tiles = kGroupM * a.tiles_n;
  const std::int64_t first_m = (t / group_tiles) * kGroupM;
  const std::int64_t gm = min(a.tiles_m - first_m, kGroupM);
  const std::int64_t tm = first_m + (t % group_tiles) % gm;
  const std::int64_t tn = (t % group_tiles) / gm;
  std::int64_t lhs_off = 0, rhs_off = 0;
  {
    std::int64_t b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
  }
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const std::int64_t m0 = tm * 32, n0 = tn * 32;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, kl = lane >> 4;
  auto rsrc_of = [](const float* base, std::int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
  };
  // The launcher checks that every panel spans less than 2^31 bytes.
  const auto a_rsrc = rsrc_of(a.lhs + lhs_off + m0 * K, (M - m0) * K * 4);
  const auto b_rsrc = kTransB ? rsrc_of(a.rhs + rhs_off + n0 * K, (N - n0) * K * 4)
                              : rsrc_of(a.rhs + rhs_off + n0, (K * N - n0) * 4);
  constexpr int kOut = 0x7fffffff;
  const int Ki = static_cast<int>(K), Ni = static_cast<int>(N);
  // This wave's chunks: [c_begin, c_end), at least one when KS <= chunks.
  const int chunks = (Ki + 15) / 16;
  const int c_begin = wave * chunks / KS, c_end = (wave + 1) * chunks / KS;
  const bool b_col_in = n0 + 2 * r < N;

  struct Frag {
    float4_t a[2], b[2];
  };
  auto load = [&](int c, Frag& f) {
    const int k = 16 * c + 4 * kl;
    const bool k_in = c < c_end && k < Ki;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      f.a[i] = __builtin_bit_cast(
          float4_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, k_in ? ((16 * i + r) * Ki + k) * 4 : kOut, 0, 0));
    if constexpr (kTransB) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        f.b[j] = __builtin_bit_cast(
            float4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, k_in ? ((16 * j + r) * Ki + k) * 4 : kOut, 0, 0));
    } else {
      using float2v = float __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool in = c < c_end && k + q < Ki && b_col_in;
        const float2v v = __builtin_bit_cast(
            float2v, __builtin_amdgcn_raw_buffer_load_b64(b_rsrc, in ? ((k + q) * Ni + 2 * r) * 4 : kOut, 0, 0));
        f.b[0][q] = v.x;
        f.b[1][q] = v.y;
      }
    }
  };
  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.F, 0.F, 0.F, 0.F};
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][q], f.b[j][q], acc[i][j], 0, 0, 0);
  };
  // Load groups of kG chunks, two in flight; a chunk's MFMAs run only when it
  // is in this wave's run (zero-filled chunks past it are loaded, not used).
  Frag f0[kG], f1[kG];
  auto load_group = [&](int c0, Frag (&f)[kG]) {
#pragma unroll
    for (int u = 0; u < kG; ++u) load(c0 + u, f[u]);
  };
  auto mma_group = [&](int c0, const Frag (&f)[kG]) {
#pragma unroll
    for (int u = 0; u < kG; ++u)
      if (c0 + u < c_end) mma(f[u]);
  };
  load_group(c_begin, f0);
  for (int c0 = c_begin; c0 < c_end; c0 += 2 * kG) {
    load_group(c0 + kG, f1);
    mma_group(c0, f0);
    load_group(c0 + 2 * kG, f0);
    if (c0 + kG < c_end) mma_group(c0 + kG, f1);
  }

  // Output (i, j, q) of lane (r, kl): row 16 i + 4 kl + q, column 16 j + r
  // (transposed B) or 2 r + j ([k, n] B) of the tile.
  auto store = [&](int i, int j, int q, float x) {
    const std::int64_t row = m0 + 16 * i + 4 * kl + q;
    const std::int64_t col = n0 + (kTransB ? 16 * j + r : 2 * r + j);
    if (row >= M || col >= N) return;
    if (a.bias != nullptr) x = x + a.bias[col];
    a.out[batch * M * N + row * N + col] = activate(x, a.activation);
  };
  if constexpr (KS == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) store(i, j, q, acc[i][j][q]);
  } else {
    __shared__ float red[KS][16][64];  // partial (i, j, q) of each wave, per lane
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave][(i * 2 + j) * 4 + q][lane] = acc[i][j][q];
    __syncthreads();
    // Wave w adds and stores outputs e = w, w + KS, ... of the 16 per lane.
    for (int e = wave; e < 16; e += KS) {
      float x = red[0][e][lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) x += red[w][e][lane];
      store(e / 8, (e / 4) % 2, e % 4, x);
    }
  }
}

// True when gemm_f32_small_kernel can take the problem: 16-byte rows and
// every byte offset into a panel below 2^31 (rows of a 32-row tile included).
inline bool small_fits(std::int64_t m, std::int64_t n, std::int64_t k) {
  constexpr double kLimit = 2147483647.0;
  const double rows_m = static_cast<double>(m < 32 ? 32 : m), rows_n = static_cast<double>(n < 32 ? 32 : n);
  return m > 0 && n > 0 && k > 0 && k % 4 == 0 && n % 4 == 0 && rows_m * k * 4 < kLimit &&
         rows_n * k * 4 < kLimit && (static_cast<double>(k) + 16) * n * 4 < kLimit;
}

template <bool kTransB, int KS>
void launch_small_as(GemmArgs& args, hipStream_t stream) {
  // Two groups of four chunks in flight (160 VGPRs) up to two waves per SIMD
  // (KS <= 8); two chunks per group at 16 waves per block.
  constexpr int kG = KS <= 8 ? 4 : 2;
  hipLaunchKernelGGL((gemm_f32_small_kernel<kTransB, KS, kG>), dim3(static_cast<unsigned>(args.total_tiles)),
                     dim3(64 * KS), 0, stream, args);
}

// KS: enough waves for about sixteen per CU over the launch (512^3: 8.4
// against 9.5 us with eight), at most one per 16-k chunk and at most 16.
inline int launch_small(GemmArgs& args, bool trans_b, hipStream_t stream) {
  if (!small_fits(args.m, args.n, args.k))
    return fail(TCX_INTERNAL, "small gemm needs 16-byte rows and 31-bit panel offsets");
  args.tiles_m = (args.m + 31) / 32;
  args.tiles_n = (args.n + 31) / 32;
  args.total_tiles = args.tiles_m * args.tiles_n * args.total_tiles;  // caller passes the batch count
  if (args.total_tiles > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  const std::int64_t chunks = (args.k + 15) / 16;
  int ks = 1;
  while (ks < 16 && ks * 2 <= chunks && args.total_tiles * ks < 4096) ks *= 2;
  switch (ks) {
    case 1: trans_b ? launch_small_as<true, 1>(args, stream) : launch_small_as<false, 1>(args, stream); break;
    case 2: trans_b ? launch_small_as<true, 2>(args, stream) : launch_small_as<false, 2>(args, stream); break;
    case 4: trans_b ? launch_small_as<true, 4>(args, stream) : launch_small_as<false, 4>(args, stream); break;
    case 8: trans_b ? launch_small_as<true, 8>(args, stream) : launch_small_as<false, 8>(args, stream); break;
    default: trans_b ? launch_small_as<true, 16>(args, stream) : launch_small_as<false, 16>(args, stream); break;
  }
  return check(hipGetLastError(), "gemm_f32 small launch");
}

// Streaming GEMM for one skinny operand: at most 32 rows of A against a
// transposed B (the decode-time linear x W^T), or at most 32 columns of B.
//   P[j][i] = sum_k X[j][k] W[i][k]: W [I, K] row-major (the long operand,
//   each row read once from HBM), X the skinny one (J <= 16 kMB rows, read
//   through the caches), row-major [J, K] or, with kXCols, held as [K, J] (a
//   [k, n] B of few columns).
//   kOutJI: W is the transposed B and X the lhs, out[j][i]; otherwise W is the
//   lhs, out[i][j].
// One block per 16 rows of W (and batch) of KS waves that split K into
// contiguous runs of 16-k chunks, as in gemm_f32_small_kernel. Lane (r, kl)
// holds W[i0 + r][16c + 4kl .. + 3] of chunk c as the MFMA's A operand (one
// 16-byte load) and X[16g + r][16c + 4kl .. + 3] as its B operand for row
// group g, so MFMA step q takes k = 16c + 4kl + q for both; output (g, v) of
// lane (r, kl) is P[16g + r][i0 + 4kl + v]. kG chunks per load group, two
// groups in flight. The KS partial tiles meet in LDS and are added in wave
// order with the bias and activation. Rows of W past I, rows of X past J and
// k past K read zero through the buffer range checks and an out-of-range
// offset.
template <bool kXCols, bool kOutJI, int kMB, int KS, int kG>
__global__ __launch_bounds__(64 * KS) void gemm_f32_stream_kernel(GemmArgs a) {
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const std::int64_t I = kOutJI ? N : M, J = kOutJI ? M : N;
  const std::int64_t i_blocks = (I + 15) / 16;
  const std::int64_t bid = blockIdx.x;
  const std::int64_t batch = bid / i_blocks, i0 = (bid % i_blocks) * 16;
  std::int64_t lhs_off = 0, rhs_off = 0;
  {
    std::int64_t b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
  }
  const float* const W = kOutJI ? a.rhs + rhs_off : a.lhs + lhs_off;
  const float* const X = kOutJI ? a.lhs + lhs_off : a.rhs + rhs_off;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, kl = lane >> 4;
  auto rsrc_of = [](const float* base, std::int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
  };
  // The launcher checks that 64 rows of K floats span less than 2^31 bytes.
  const std::int64_t w_rows = I - i0 < 16 ? I - i0 : 16;
  const auto w_rsrc = rsrc_of(W + i0 * K, w_rows * K * 4);
  const auto x_rsrc = rsrc_of(X, J * K * 4);
  constexpr int kOut = 0x7fffffff;
  const int Ki = static_cast<int>(K), Ji = static_cast<int>(J);
  const int chunks = (Ki + 15) / 16;
  const int c_begin = wave * chunks / KS, c_end = (wave + 1) * chunks / KS;

  struct Frag {
    float4_t w, x[kMB];
  };
  auto load = [&](int c, Frag& f) {
    const int k = 16 * c + 4 * kl;
    const bool k_in = c < c_end && k < Ki;
    f.w = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(w_rsrc, k_in ? (r * Ki + k) * 4 : kOut,
                                                                             0, 0));
#pragma unroll
    for (int g = 0; g < kMB; ++g) {
      const int j = 16 * g + r;
      if constexpr (kXCols) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          f.x[g][q] = __builtin_bit_cast(
              float, __builtin_amdgcn_raw_buffer_load_b32(x_rsrc, k_in && j < Ji ? ((k + q) * Ji + j) * 4 : kOut, 0, 0));
      } else {
        f.x[g] = __builtin_bit_cast(
            float4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, k_in && j < Ji ? (j * Ki + k) * 4 : kOut, 0, 0));
      }
    }
  };
  floatx4 acc[kMB];
#pragma unroll
  for (int g = 0; g < kMB; ++g) acc[g] = floatx4{0.F, 0.F, 0.F, 0.F};
  auto mma = [&](const Frag& f) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int g = 0; g < kMB; ++g)
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.w[q], f.x[g][q], acc[g], 0, 0, 0);
  };
  Frag f0[kG], f1[kG];
  auto load_group = [&](int c0, Frag (&f)[kG]) {
#pragma unroll
    for (int u = 0; u < kG; ++u) load(c0 + u, f[u]);
  };
  auto mma_group = [&](int c0, const Frag (&f)[kG]) {
#pragma unroll
    for (int u = 0; u < kG; ++u)
      if (c0 + u < c_end) mma(f[u]);
  };
  load_group(c_begin, f0);
  for (int c0 = c_begin; c0 < c_end; c0 += 2 * kG) {
    load_group(c0 + kG, f1);
    mma_group(c0, f0);
    load_group(c0 + 2 * kG, f0);
    if (c0 + kG < c_end) mma_group(c0 + kG, f1);
  }

  auto store = [&](int g, int v, float x) {
    const std::int64_t i = i0 + 4 * kl + v, j = 16 * g + r;
    if (i >= I || j >= J) return;
    const std::int64_t row = kOutJI ? j : i, col = kOutJI ? i : j;
    if (a.bias != nullptr) x = x + a.bias[col];
    a.out[batch * M * N + row * N + col] = activate(x, a.activation);
  };
  if constexpr (KS == 1) {
#pragma unroll
    for (int g = 0; g < kMB; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) store(g, v, acc[g][v]);
  } else {
    __shared__ float red[KS][kMB * 4][64];  // partial (g, v) of each wave, per lane
#pragma unroll
    for (int g = 0; g < kMB; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][g * 4 + v][lane] = acc[g][v];
    __syncthreads();
    for (int e = wave; e < kMB * 4; e += KS) {
      float x = red[0][e][lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) x += red[w][e][lane];
      store(e / 4, e % 4, x);
    }
  }
}

// Streaming GEMM for the decode-time linear out = X W^T (X: J <= 16 kMB rows
// of A, W: the transposed B, I rows), with both operands staged in LDS. The
// operand layout of gemm_f32_stream_kernel makes every load instruction
// touch 16 rows of 64 B; here each wave moves 64-k spans of its 16 W rows and
// of X into its own LDS stage by DMA (buffer_load ... lds), four rows x 256 B
// per instruction, and reads the MFMA operands back with ds_read_b128. Lane
// i of instruction u fills slot i % 16 of row 4u + i / 16, which holds the
// row's 16-byte chunk slot ^ row, so the operand reads (chunk 4c + kl of row
// r, at slot (4c + kl) ^ r) are conflict-free. Three stages per wave, two
// spans in flight, no barrier in the loop: a wave reads only what its own
// loads wrote, after its own vmcnt wait. Lane (r, kl) takes k = 64s + 16c +
// 4kl + q at MFMA step (c, q), as gemm_f32_stream_kernel does; chunks of even
// and odd c accumulate separately (two dependence chains) and are added at
// the end. KS waves split the spans into contiguous runs and meet in LDS, in
// wave order. Rows of W past I, rows of X past J and k past K read zero.
// Against gemm_f32_stream_kernel on MI355X: 16x4096x4096 20.8 -> 16.2 us,
// 32x4096x4096 28.5 -> 19.3, 16x14336x4096 66.2 -> 54.4, 32x11008x4096
// 76.1 -> 54.0, 24x2048x2048 13.7 -> 10.7.
template <int kMB, int KS>
__global__ __launch_bounds__(64 * KS) void gemm_f32_stream_lds_kernel(GemmArgs a) {
  constexpr int kStages = 3, kSpan = 64, kTile = 16 * kSpan;
  constexpr int kPer = (1 + kMB) * kTile;  // floats of one stage: W, then kMB row groups of X
  __shared__ float lds[KS * kStages * kPer];
  const std::int64_t M = a.m, N = a.n, K = a.k;
  const std::int64_t I = N, J = M;
  const std::int64_t i_blocks = (I + 15) / 16;
  const std::int64_t bid = blockIdx.x;
  const std::int64_t batch = bid / i_blocks, i0 = (bid % i_blocks) * 16;
  std::int64_t lhs_off = 0, rhs_off = 0;
  {
    std::int64_t b = batch;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lhs_off += c * a.lhs_bs[ax];
      rhs_off += c * a.rhs_bs[ax];
    }
  }
  const float* const W = a.rhs + rhs_off;
  const float* const X = a.lhs + lhs_off;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, kl = lane >> 4;
  using int4v = int __attribute__((ext_vector_type(4)));
  auto rsrc_of = [](const float* base, std::int64_t bytes) {
    const auto addr = reinterpret_cast<std::uint64_t>(base);
    return int4v{static_cast<int>(addr), static_cast<int>(addr >> 32), static_cast<int>(bytes), 0x00020000};
  };
  // The launcher checks that 32 rows of K floats span less than 2^31 bytes.
  const std::int64_t w_rows = I - i0 < 16 ? I - i0 : 16;
  const int4v w_rsrc = rsrc_of(W + i0 * K, w_rows * K * 4);
  const int4v x_rsrc = rsrc_of(X, J * K * 4);
  constexpr int kOut = 0x7fffffff;
  const int Ki = static_cast<int>(K), Ji = static_cast<int>(J);
  const int spans = (Ki + kSpan - 1) / kSpan;
  const int s_begin = wave * spans / KS, s_end = (wave + 1) * spans / KS;
  float* const mine = lds + wave * kStages * kPer;
  auto lds_of = [](const void* ptr) {
    return static_cast<unsigned>(reinterpret_cast<std::uintptr_t>((__attribute__((address_space(3))) const void*)ptr));
  };
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  auto dma16 = [](const int4v& rsrc, unsigned lds_byte, int voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :: "s"(lds_byte), "v"(voff), "s"(rsrc), "s"(0) : "memory", "m0");
  };
#pragma clang diagnostic pop
  const int slot = lane % 16;
  auto issue = [&](int s, int stage) {
    const int k0 = s * kSpan;
    float* const base = mine + stage * kPer;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = 4 * u + lane / 16;
      const int k = k0 + 4 * (slot ^ row);
      const bool k_in = k < Ki;  // K % 4 == 0: a chunk is whole or past K
      dma16(w_rsrc, lds_of(base) + u * 1024, k_in ? (row * Ki + k) * 4 : kOut);
#pragma unroll
      for (int g = 0; g < kMB; ++g) {
        const int j = 16 * g + row;
        dma16(x_rsrc, lds_of(base + (1 + g) * kTile) + u * 1024, k_in && j < Ji ? (j * Ki + k) * 4 : kOut);
      }
    }
  };
  floatx4 acc[2][kMB];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int g = 0; g < kMB; ++g) acc[h][g] = floatx4{0.F, 0.F, 0.F, 0.F};
  auto compute = [&](int stage) {
    const float* const base = mine + stage * kPer;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int off = r * kSpan + 4 * ((4 * c + kl) ^ r);
      const float4_t w = *reinterpret_cast<const float4_t*>(base + off);
      float4_t x[kMB];
#pragma unroll
      for (int g = 0; g < kMB; ++g) x[g] = *reinterpret_cast<const float4_t*>(base + (1 + g) * kTile + off);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int g = 0; g < kMB; ++g)
          acc[c & 1][g] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[q], x[g][q], acc[c & 1][g], 0, 0, 0);
    }
  };
  constexpr int kInst = 4 * (1 + kMB);  // DMA instructions per span
  if (s_begin < s_end) issue(s_begin, 0);
  if (s_begin + 1 < s_end) issue(s_begin + 1, 1);
  for (int s = s_begin; s < s_end; ++s) {
    // Span s has landed (span s + 1's loads may still be out).
    if (s + 1 < s_end) __builtin_amdgcn_s_waitcnt(0x0F70 | kInst);
    else __builtin_amdgcn_s_waitcnt(0x0F70);
    asm volatile("" ::: "memory");  // the stage's LDS reads stay after the wait
    compute((s - s_begin) % kStages);
    // The stage of span s - 1, whose reads this wave has consumed.
    if (s + 2 < s_end) issue(s + 2, (s + 2 - s_begin) % kStages);
  }
#pragma unroll
  for (int g = 0; g < kMB; ++g) acc[0][g] = acc[0][g] + acc[1][g];

  auto store = [&](int g, int v, float x) {
    const std::int64_t i = i0 + 4 * kl + v, j = 16 * g + r;
    if (i >= I || j >= J) return;
    if (a.bias != nullptr) x = x + a.bias[i];
    a.out[batch * M * N + j * N + i] = activate(x, a.activation);
  };
  if constexpr (KS == 1) {
#pragma unroll
    for (int g = 0; g < kMB; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) store(g, v, acc[0][g][v]);
  } else {
    __syncthreads();  // every wave is done with its stages
    float* const red = lds;  // KS x kMB * 4 x 64 floats
#pragma unroll
    for (int g = 0; g < kMB; ++g)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(wave * kMB * 4 + g * 4 + v) * 64 + lane] = acc[0][g][v];
    __syncthreads();
    for (int e = wave; e < kMB * 4; e += KS) {
      float x = red[e * 64 + lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) x += red[(w * kMB * 4 + e) * 64 + lane];
      store(e / 4, e % 4, x);
    }
  }
}

// Matrix-vector products: y[i] = act(dot(R[i], v) + bias) for every row i of
// a row-major R [I, K], batched. The decode-time linear x W^T with one row of
// x (R = W, v = x, y = that row of the output), and A b with one column of b
// (R = A, v = b, y = that column). Lanes stream K in 16-byte loads, so one
// wave instruction reads 1 KB of one row (eight whole 128-byte lines; the
// MFMA operand layout of gemm_f32_stream_kernel reads 16 rows x 64 B per
// instruction). KW waves of a 4-wave block split a row's K into contiguous
// runs (KW = 1, 2 or 4, more when rows are few); lane sums add in a fixed
// tree, the waves' in wave order. Eight loads per lane in flight. v is
// contiguous (a row of x, or the column of a [k, 1] b); y_stride is the
// element stride of y in the output; bias is per row (bias_per_row) or one
// value.
template <int KW>
__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ R, const float* __restrict__ v,
                                                       float* __restrict__ y, const float* __restrict__ bias,
                                                       std::int64_t rows, std::int64_t K, std::int64_t batches,
                                                       std::int64_t r_batch, std::int64_t v_batch,
                                                       std::int64_t y_batch, std::int64_t y_stride, int bias_per_row,
                                                       int act) {
  constexpr int kRowsPerBlock = 4 / KW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int part = wave % KW;
  const std::int64_t row_in_grid = static_cast<std::int64_t>(blockIdx.x) * kRowsPerBlock + wave / KW;
  const std::int64_t batch = row_in_grid / rows, i = row_in_grid % rows;
  __shared__ float partial[4];
  float sum = 0.F;
  if (batch < batches) {
    const float* __restrict__ rp = R + batch * r_batch + i * K;
    const float* __restrict__ vp = v + batch * v_batch;
    // This wave's run of K: whole 1024-element strides first, 4-element
    // groups after (K % 4 == 0).
    const std::int64_t run = (K / 4 + KW - 1) / KW * 4;
    const std::int64_t k_begin = part * run, k_end = min(K, k_begin + run);
    float s[8] = {};
    std::int64_t k = k_begin + 4 * lane;
    for (; k + 7 * 256 < k_end; k += 8 * 256) {
      float4_t w[8], x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) w[u] = stream_load(reinterpret_cast<const float4_t*>(rp + k + 256 * u));
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const float4_t*>(vp + k + 256 * u);
#pragma unroll
      for (int u = 0; u < 8; ++u) s[u] += (w[u].x * x[u].x + w[u].y * x[u].y) + (w[u].z * x[u].z + w[u].w * x[u].w);
    }
    for (; k < k_end; k += 256) {
      const float4_t w = stream_load(reinterpret_cast<const float4_t*>(rp + k));
      const float4_t x = *reinterpret_cast<const float4_t*>(vp + k);
      s[0] += (w.x * x.x + w.y * x.y) + (w.z * x.z + w.w * x.w);
    }
    sum = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  }
  sum = wave_sum(sum);
  if constexpr (KW > 1) {
    if (lane == 0) partial[wave] = sum;
    __syncthreads();
    if (part != 0 || lane != 0 || batch >= batches) return;
    sum = partial[wave];
#pragma unroll
    for (int w = 1; w < KW; ++w) sum += partial[wave + w];
  } else {
    if (lane != 0 || batch >= batches) return;
  }
  if (bias != nullptr) sum = sum + bias[bias_per_row ? i : 0];
  y[batch * y_batch + i * y_stride] = activate(sum, act);
}

// Many small products (M, N, K <= kTinyMax): P whole items per block are
// staged in LDS (A [P][M][K], B [P][K][N], a transposed B transposed on the
// way in), then each thread computes outputs of the block's items in output
// order, summing its k in order as separately rounded products and sums
// (the reference's loop order, -ffp-contract=off). One 64x64 tile per item
// wastes most of an MFMA tile on 8x8 items and pays a block's latency per
// item: 65536 batches of 8x8x8 took 3.6 ms on the tiled kernel, 16 us here;
// four columns per thread (kQuad) took 64^3 x 4096 from 145 to 88 us. Dense
// batches of a [k, n] B (kDense) stage the block's A items and B items as two
// contiguous runs with 16-byte loads instead of one float per load: 65536 x
// 8x8x8 16.2 -> 14.1 us, 10000 x 1x64x64 60.3 -> 49.0, 65536 x 5x7x3 13.5 ->
// 11.5, 16384 x 16^3 18.1 -> 16.1 us on MI355X.
constexpr std::int64_t kTinyMax = 64;
constexpr int kTinyFloats = 8192;  // 32 KB of LDS per block

constexpr int kTinyItems = 256;    // most items per block

template <bool kTransB, bool kQuad, bool kDense>
__global__ __launch_bounds__(256) void gemm_f32_tiny_kernel(GemmArgs a, int P) {
  // kDense: the staging's float4s may run up to three floats past a region.
  __shared__ __attribute__((aligned(16))) float lds[kTinyFloats + 8];
  __shared__ std::int64_t item_off[2][kDense ? 1 : kTinyItems];  // each item's A and B offsets
  const int M = static_cast<int>(a.m), N = static_cast<int>(a.n), K = static_cast<int>(a.k);
  const int a_size = M * K, b_size = K * N, item_size = a_size + b_size;
  const std::int64_t items = a.total_tiles;
  const std::int64_t first = static_cast<std::int64_t>(blockIdx.x) * P;
  const int count = static_cast<int>(items - first < P ? items - first : P);
  const int T = static_cast<int>(blockDim.x);
  // Item p's A at a_at(p), its B ([K][N]) at b_at(p): interleaved per item,
  // or (kDense) all A, then all B from a 16-byte boundary.
  const int b_base = (P * a_size + 3) / 4 * 4;
  auto a_at = [&](int p) { return kDense ? p * a_size : p * item_size; };
  auto b_at = [&](int p) { return kDense ? b_base + p * b_size : p * item_size + a_size; };
  if constexpr (kDense) {
    // Dense batches: the block's A items and B items are two contiguous
    // runs, staged with 16-byte buffer loads (4-byte alignment suffices).
    const int na = count * a_size, nb = count * b_size;
    const auto ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.lhs + first * a_size),
                                                      static_cast<short>(0), na * 4, 0x00020000);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.rhs + first * b_size),
                                                      static_cast<short>(0), nb * 4, 0x00020000);
    for (int f = 4 * static_cast<int>(threadIdx.x); f < na; f += 4 * T)
      *reinterpret_cast<float4_t*>(lds + f) =
          __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(ra, 4 * f, 0, 0));
    for (int f = 4 * static_cast<int>(threadIdx.x); f < nb; f += 4 * T)
      *reinterpret_cast<float4_t*>(lds + b_base + f) =
          __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rb, 4 * f, 0, 0));
  }
  for (int p = threadIdx.x; !kDense && p < count; p += blockDim.x) {
    std::int64_t b = first + p, lo = 0, ro = 0;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t c = b % e;
      b /= e;
      lo += c * a.lhs_bs[ax];
      ro += c * a.rhs_bs[ax];
    }
    item_off[0][p] = lo;
    item_off[1][p] = ro;
  }
  __syncthreads();
  // Stage item p's A at lds[p * item_size] and its B (as [K][N]) after it:
  // one flat walk over the block's elements, eight loads in flight; each
  // thread's (item, offset) advances by the block size without a division.
  const int total = kDense ? 0 : count * item_size;
  const int dp = T / item_size, dr = T % item_size;
  int sp = static_cast<int>(threadIdx.x) / item_size, sr = static_cast<int>(threadIdx.x) % item_size;
  for (int e0 = threadIdx.x; e0 < total; e0 += 8 * T) {
    float v[8];
    int dst[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (e0 + u * T < total) {
        if (sr < a_size) {
          v[u] = a.lhs[item_off[0][sp] + sr];
          dst[u] = sp * item_size + sr;
        } else {
          const int rb = sr - a_size;
          v[u] = a.rhs[item_off[1][sp] + rb];
          if constexpr (kTransB) {
            const int nn = rb / K, kk = rb - nn * K;  // B is [N][K]
            dst[u] = sp * item_size + a_size + kk * N + nn;
          } else {
            dst[u] = sp * item_size + sr;
          }
        }
      }
      sp += dp;
      sr += dr;
      if (sr >= item_size) {
        sr -= item_size;
        ++sp;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (e0 + u * T < total) lds[dst[u]] = v[u];
  }
  __syncthreads();
  // Outputs in output order: this thread's (item, row, column) advances by
  // the block size the same way. kQuad: a thread computes four adjacent
  // columns (N, M K and K N multiples of 4, so every staged row and output
  // row is 16-byte aligned), one broadcast A read and one float4 B read per
  // four multiply-adds, each output's k still in order.
  constexpr int Q = kQuad ? 4 : 1;
  const int NQ = N / Q;
  const int outs = M * NQ;
  const int op = T / outs, orem = T % outs, oi = orem / NQ, oj = orem % NQ;
  int p = static_cast<int>(threadIdx.x) / outs;
  int i = (static_cast<int>(threadIdx.x) % outs) / NQ, j = static_cast<int>(threadIdx.x) % NQ;
  for (int e = threadIdx.x; e < count * outs; e += T) {
    const float* A = lds + a_at(p) + i * K;
    float* o = a.out + (first + p) * static_cast<std::int64_t>(M) * N + i * N + j * Q;
    if constexpr (kQuad) {
      const float4_t* B = reinterpret_cast<const float4_t*>(lds + b_at(p)) + j;
      float4_t acc = {0.F, 0.F, 0.F, 0.F};
      for (int k = 0; k < K; ++k) {
        const float x = A[k];
        const float4_t bv = B[k * NQ];
        acc.x += x * bv.x;
        acc.y += x * bv.y;
        acc.z += x * bv.z;
        acc.w += x * bv.w;
      }
      if (a.bias != nullptr) {
        acc.x = acc.x + a.bias[4 * j];
        acc.y = acc.y + a.bias[4 * j + 1];
        acc.z = acc.z + a.bias[4 * j + 2];
        acc.w = acc.w + a.bias[4 * j + 3];
      }
      acc.x = activate(acc.x, a.activation);
      acc.y = activate(acc.y, a.activation);
      acc.z = activate(acc.z, a.activation);
      acc.w = activate(acc.w, a.activation);
      *reinterpret_cast<float4_t*>(o) = acc;
    } else {
      const float* B = lds + b_at(p) + j;
      float acc = 0.F;
      for (int k = 0; k < K; ++k) acc += A[k] * B[k * N];
      if (a.bias != nullptr) acc = acc + a.bias[j];
      *o = activate(acc, a.activation);
    }
    p += op;
    i += oi;
    j += oj;
    if (j >= NQ) {
      j -= NQ;
      ++i;
    }
    if (i >= M) {
      i -= M;
      ++p;
    }
  }
}

// Products with K <= kSmallK (unbatched, N a multiple of 4, 16-byte aligned
// B rows and output): each thread owns four output columns, holds their K x 4
// B values in registers and walks rows, so the output is written once as a
// float4 stream and A rows come from cache. Rows of at least 256 float4 take
// a column tile of 256 per block and stride over rows (blockIdx.y);
// narrower rows put 256 / (N / 4) rows in a block. Each output sums its k in
// order as separately rounded products and sums, the reference's loop. A
// grid of about 2048 blocks makes each block load its B columns once for
// many rows (one row per block took 26.8 us at 4096 x 4096 x 4, 15.2 us so).
constexpr std::int64_t kSmallK = 16;

template <bool kTransB>
__global__ __launch_bounds__(256) void gemm_f32_smallk_kernel(GemmArgs a, int rows_per_block) {
  const std::int64_t M = a.m, N = a.n;
  const int K = static_cast<int>(a.k);
  const std::int64_t CQ = N / 4;
  std::int64_t cq, row0, row_step;
  if (rows_per_block == 0) {
    cq = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    row0 = blockIdx.y;
    row_step = gridDim.y;
  } else {
    cq = threadIdx.x % CQ;
    const int rb = static_cast<int>(threadIdx.x / CQ);
    if (rb >= rows_per_block) return;
    row0 = static_cast<std::int64_t>(blockIdx.y) * rows_per_block + rb;
    row_step = static_cast<std::int64_t>(gridDim.y) * rows_per_block;
  }
  if (cq >= CQ) return;
  float4_t b[kSmallK];
#pragma unroll
  for (int k = 0; k < kSmallK; ++k) {
    b[k] = float4_t{0.F, 0.F, 0.F, 0.F};
    if (k < K) {
      if constexpr (kTransB) {  // B is [N][K]
        const float* col = a.rhs + 4 * cq * K + k;
        b[k] = float4_t{col[0], col[K], col[2 * K], col[3 * K]};
      } else {
        b[k] = reinterpret_cast<const float4_t*>(a.rhs + k * N)[cq];
      }
    }
  }
  float4_t bias = {0.F, 0.F, 0.F, 0.F};
  if (a.bias != nullptr) bias = float4_t{a.bias[4 * cq], a.bias[4 * cq + 1], a.bias[4 * cq + 2], a.bias[4 * cq + 3]};
  // Two rows per step: both rows' A values are loaded before either is used.
  for (std::int64_t m = row0; m < M; m += 2 * row_step) {
    const std::int64_t m2 = m + row_step < M ? m + row_step : m;  // a lone last row repeats itself
    float x0[kSmallK], x1[kSmallK];
#pragma unroll
    for (int k = 0; k < kSmallK; ++k) {
      x0[k] = k < K ? a.lhs[m * K + k] : 0.F;
      x1[k] = k < K ? a.lhs[m2 * K + k] : 0.F;
    }
    float4_t acc[2] = {{0.F, 0.F, 0.F, 0.F}, {0.F, 0.F, 0.F, 0.F}};
#pragma unroll
    for (int k = 0; k < kSmallK; ++k) {
      if (k < K) {
        acc[0].x += x0[k] * b[k].x;
        acc[0].y += x0[k] * b[k].y;
        acc[0].z += x0[k] * b[k].z;
        acc[0].w += x0[k] * b[k].w;
        acc[1].x += x1[k] * b[k].x;
        acc[1].y += x1[k] * b[k].y;
        acc[1].z += x1[k] * b[k].z;
        acc[1].w += x1[k] * b[k].w;
      }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float4_t v = acc[r];
      if (a.bias != nullptr) {
        v.x = v.x + bias.x; v.y = v.y + bias.y; v.z = v.z + bias.z; v.w = v.w + bias.w;
      }
      v.x = activate(v.x, a.activation);
      v.y = activate(v.y, a.activation);
      v.z = activate(v.z, a.activation);
      v.w = activate(v.w, a.activation);
      if (r == 0 || m2 != m) __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(a.out + (r ? m2 : m) * N) + cq);
    }
  }
}

inline int launch_smallk(GemmArgs& args, bool trans_b, hipStream_t stream) {
  if (args.k < 1 || args.k > kSmallK || args.n % 4 != 0)
    return fail(TCX_INTERNAL, "small-K gemm needs 1 <= K <= 16 and N a multiple of 4");
  const std::int64_t CQ = args.n / 4;
  int rows_per_block = 0;
  unsigned gx = 1;
  std::int64_t rows_in_y = args.m;
  if (CQ >= 256) {
    gx = static_cast<unsigned>((CQ + 255) / 256);
  } else {
    rows_per_block = static_cast<int>(256 / CQ);
    rows_in_y = (args.m + rows_per_block - 1) / rows_per_block;
  }
  // About 2048 blocks (eight per CU): each loads its B columns once and
  // strides over many rows.
  const std::int64_t gy_cap = 2048 / gx > 0 ? 2048 / gx : 1;
  const std::int64_t gy = rows_in_y < gy_cap ? rows_in_y : (gy_cap < 65535 ? gy_cap : 65535);
  const dim3 grid(gx, static_cast<unsigned>(gy < 65535 ? gy : 65535));
  if (trans_b)
    hipLaunchKernelGGL((gemm_f32_smallk_kernel<true>), grid, dim3(256), 0, stream, args, rows_per_block);
  else
    hipLaunchKernelGGL((gemm_f32_smallk_kernel<false>), grid, dim3(256), 0, stream, args, rows_per_block);
  return check(hipGetLastError(), "gemm_f32 small-K launch");
}

// One row of A against a row-major B per batch (M == 1, [k, n] B): out[j]
// = sum_k x[k] B[k, j]. A block of 1024 threads takes 1024 columns (a float4
// per thread) of one batch item, in four groups of 256 threads each summing
// a quarter of K in order with eight float4 rows of B in flight; the groups'
// partials are added in group order through LDS. The tiled kernels padded
// the one row to a 64-row tile: 64 batches of 1 x 4096 x 4096 took 3.97 ms.
constexpr int kVecMatGroups = 4;

__global__ __launch_bounds__(1024) void gemm_f32_vecmat_kernel(GemmArgs a) {
  __shared__ float4_t part[kVecMatGroups - 1][256];
  const std::int64_t N = a.n, K = a.k, CQ = N / 4;
  const int t = threadIdx.x & 255, group = threadIdx.x >> 8;
  const std::int64_t c = static_cast<std::int64_t>(blockIdx.x) * 256 + t;
  for (std::int64_t item = blockIdx.y; item < a.total_tiles; item += gridDim.y) {
    std::int64_t b = item, lo = 0, ro = 0;
    for (int ax = a.batch_rank - 1; ax >= 0; --ax) {
      const std::int64_t e = a.batch_shape[ax];
      const std::int64_t cc = b % e;
      b /= e;
      lo += cc * a.lhs_bs[ax];
      ro += cc * a.rhs_bs[ax];
    }
    const float* x = a.lhs + lo;
    const float4_t* B = reinterpret_cast<const float4_t*>(a.rhs + ro);
    // This block's k range: all of K, or split blockIdx.z of a.splits.
    std::int64_t ks0 = 0, ks1 = K;
    if (a.splits > 1) {
      const std::int64_t per = (K + a.splits - 1) / a.splits;
      ks0 = blockIdx.z * per < K ? blockIdx.z * per : K;
      ks1 = ks0 + per < K ? ks0 + per : K;
    }
    const std::int64_t kq = (ks1 - ks0 + kVecMatGroups - 1) / kVecMatGroups;
    const std::int64_t k0 = ks0 + group * kq < ks1 ? ks0 + group * kq : ks1;
    const std::int64_t k1 = k0 + kq < ks1 ? k0 + kq : ks1;
    const std::int64_t cl = c < CQ ? c : CQ - 1;  // lanes past the last column read a valid one
    float4_t acc = {0.F, 0.F, 0.F, 0.F};
    std::int64_t k = k0;
    for (; k + 8 <= k1; k += 8) {
      float4_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = stream_load(B + (k + u) * CQ + cl);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float xv = x[k + u];
        acc.x += xv * v[u].x;
        acc.y += xv * v[u].y;
        acc.z += xv * v[u].z;
        acc.w += xv * v[u].w;
      }
    }
    for (; k < k1; ++k) {
      const float4_t v = stream_load(B + k * CQ + cl);
      const float xv = x[k];
      acc.x += xv * v.x;
      acc.y += xv * v.y;
      acc.z += xv * v.z;
      acc.w += xv * v.w;
    }
    if (group > 0) part[group - 1][t] = acc;
    __syncthreads();
    if (group == 0 && c < CQ) {
#pragma unroll
      for (int g = 0; g < kVecMatGroups - 1; ++g) {
        const float4_t p = part[g][t];
        acc.x += p.x;
        acc.y += p.y;
        acc.z += p.z;
        acc.w += p.w;
      }
      if (a.splits > 1) {  // a partial sum: split_reduce_kernel adds the splits in order
        reinterpret_cast<float4_t*>(a.partial + (blockIdx.z * a.total_tiles + item) * N)[c] = acc;
      } else {
        if (a.bias != nullptr) {
          acc.x = acc.x + a.bias[4 * c];
          acc.y = acc.y + a.bias[4 * c + 1];
          acc.z = acc.z + a.bias[4 * c + 2];
          acc.w = acc.w + a.bias[4 * c + 3];
        }
        acc.x = activate(acc.x, a.activation);
        acc.y = activate(acc.y, a.activation);
        acc.z = activate(acc.z, a.activation);
        acc.w = activate(acc.w, a.activation);
        reinterpret_cast<float4_t*>(a.out + item * N)[c] = acc;
      }
    }
    __syncthreads();  // part is rewritten by the next item
  }
}

// K splits of the vector-matrix kernel for items x 1024-column chunks too
// few to fill the GPU: the smallest power of two giving >= 256 blocks, each
// split keeping >= 128 rows of B, at most 128. Measured against 512 blocks
// of >= 64 rows and 1024 of >= 32: 1 x 4096 x 4096 22.5 / 27.4 / 42.3 us,
// 1 x 8192 x 8192 48.6 / 70.2 / 68.3 us (more splits only add partials).
inline std::int64_t vecmat_splits(std::int64_t items, std::int64_t n, std::int64_t k) {
  const std::int64_t blocks = items * ((n / 4 + 255) / 256);
  std::int64_t splits = 1;
  while (blocks * splits < 256 && splits < 128 && k / (2 * splits) >= 128) splits *= 2;
  return splits;
}

inline int launch_vecmat(GemmArgs& args, hipStream_t stream) {
  if (args.m != 1 || args.n % 4 != 0 || args.k < 1) return fail(TCX_INTERNAL, "vector-matrix gemm needs M == 1");
  const std::int64_t chunks = (args.n / 4 + 255) / 256;
  const std::int64_t items = args.total_tiles;  // the caller passes the batch count
  const int splits = args.splits > 1 ? args.splits : 1;
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(items < 65535 ? items : 65535),
                  static_cast<unsigned>(splits));
  hipLaunchKernelGGL(gemm_f32_vecmat_kernel, grid, dim3(256 * kVecMatGroups), 0, stream, args);
  int rc = check(hipGetLastError(), "gemm_f32 vector-matrix launch");
  if (rc != TCX_OK || splits == 1) return rc;
  const std::int64_t count4 = items * args.n / 4;
  hipLaunchKernelGGL(split_reduce_kernel, dim3(grid_for(count4, 256, 256 * 16)), dim3(256), 0, stream, args.partial,
                     args.out, args.bias, count4, args.n, splits, args.activation);
  return check(hipGetLastError(), "gemm_f32 vector-matrix split reduce launch");
}

inline bool tiny_fits(std::int64_t m, std::int64_t n, std::int64_t k) {
  return m >= 1 && n >= 1 && k >= 1 && m <= kTinyMax && n <= kTinyMax && k <= kTinyMax &&
         m * k + k * n <= kTinyFloats;
}

inline int launch_tiny(GemmArgs& args, bool trans_b, hipStream_t stream) {
  const std::int64_t item = args.m * args.k + args.k * args.n;
  if (!tiny_fits(args.m, args.n, args.k) || item <= 0)
    return fail(TCX_INTERNAL, "tiny gemm needs M, N, K <= 64");
  const std::int64_t items = args.total_tiles;  // the caller passes the batch count
  // Items per block: as many as the LDS holds, at most enough for about 16
  // outputs per thread and at most kTinyItems, and at least one.
  // Four columns per thread where rows stay 16-byte aligned and a block's
  // items still give its 256 threads a four-column output each (fewer left
  // most threads idle: 10000 items of 1 x 64 x 64, one item per block,
  // 60 -> 69 us).
  bool quad = args.n % 4 == 0 && (args.m * args.k) % 4 == 0 && (args.k * args.n) % 4 == 0 &&
              (reinterpret_cast<std::uintptr_t>(args.out) & 15U) == 0;
  auto items_per_block = [&](std::int64_t per_item) {  // thread outputs per item
    std::int64_t P = kTinyFloats / item;
    const std::int64_t by_outputs = (16 * 256 + per_item - 1) / per_item;
    if (P > by_outputs) P = by_outputs;
    if (P > kTinyItems) P = kTinyItems;
    return P < 1 ? std::int64_t{1} : P;
  };
  std::int64_t P = items_per_block(args.m * args.n / 4);
  if (!quad || P * (args.m * args.n / 4) < 256) {
    quad = false;
    P = items_per_block(args.m * args.n);
  }
  const std::int64_t blocks = (items + P - 1) / P;
  if (blocks > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, args, static_cast<int>(P));
  };
  // Dense batches (natural strides) of a [k, n] B stage their two runs with
  // 16-byte loads; the block's A and B regions then span at most P * (a + b)
  // + 5 floats (the B region starts at a 16-byte boundary and the last float4
  // may run 3 past it), inside the kernel's LDS slack.
  bool dense = !trans_b;
  {
    std::int64_t ea = args.m * args.k, eb = args.k * args.n;
    for (int ax = args.batch_rank - 1; ax >= 0; --ax) {
      dense = dense && args.lhs_bs[ax] == ea && args.rhs_bs[ax] == eb;
      ea *= args.batch_shape[ax];
      eb *= args.batch_shape[ax];
    }
  }
  if (trans_b)
    quad ? launch(gemm_f32_tiny_kernel<true, true, false>) : launch(gemm_f32_tiny_kernel<true, false, false>);
  else if (dense)
    quad ? launch(gemm_f32_tiny_kernel<false, true, true>) : launch(gemm_f32_tiny_kernel<false, false, true>);
  else
    quad ? launch(gemm_f32_tiny_kernel<false, true, false>) : launch(gemm_f32_tiny_kernel<false, false, false>);
  return check(hipGetLastError(), "gemm_f32 tiny launch");
}


// rows x batches dot products of K (K % 4 == 0, R, v and every batch offset
// 16-byte aligned): KW waves per row, more when rows are few.
inline int launch_gemv(const float* R, const float* v, float* y, const float* bias, std::int64_t rows,
                       std::int64_t K, std::int64_t batches, std::int64_t r_batch, std::int64_t v_batch,
                       std::int64_t y_batch, std::int64_t y_stride, bool bias_per_row, int act, hipStream_t stream) {
  const std::int64_t total = rows * batches;
  const int kw = total >= 4096 ? 1 : total >= 2048 ? 2 : 4;
  const std::int64_t blocks = (total * kw + 3) / 4;
  if (blocks > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  const dim3 grid(static_cast<unsigned>(blocks));
  const int bpr = bias_per_row ? 1 : 0;
  if (kw == 1)
    hipLaunchKernelGGL(gemv_f32_kernel<1>, grid, dim3(256), 0, stream, R, v, y, bias, rows, K, batches, r_batch,
                       v_batch, y_batch, y_stride, bpr, act);
  else if (kw == 2)
    hipLaunchKernelGGL(gemv_f32_kernel<2>, grid, dim3(256), 0, stream, R, v, y, bias, rows, K, batches, r_batch,
                       v_batch, y_batch, y_stride, bpr, act);
  else
    hipLaunchKernelGGL(gemv_f32_kernel<4>, grid, dim3(256), 0, stream, R, v, y, bias, rows, K, batches, r_batch,
                       v_batch, y_batch, y_stride, bpr, act);
  return check(hipGetLastError(), "gemv launch");
}

// Skinny rows or columns the streaming kernel takes: up to two row groups.
// With four (33-64) its MFMAs outweigh the streamed bytes and the tiled
// kernels were faster (48x4096x4096 transposed: 38.1 against 34.3 us).
constexpr std::int64_t kStreamMaxSkinny = 32;

// True when gemm_f32_stream_kernel can take a K: whole 16-byte groups of k
// and kStreamMaxSkinny rows of K floats (the skinny operand's buffer range)
// below 2^31 bytes.
inline bool stream_fits(std::int64_t k) {
  return k > 0 && k % 4 == 0 && static_cast<double>(kStreamMaxSkinny) * static_cast<double>(k) * 4 < 2147483647.0;
}

template <bool kXCols, bool kOutJI, int kMB, int KS>
void launch_stream_as(const GemmArgs& args, std::int64_t blocks, hipStream_t stream) {
  // Two groups of four chunks in flight for one row group of X, of two
  // chunks for two (the registers of four waves per SIMD at KS = 16).
  constexpr int kG = kMB == 1 ? 4 : 2;
  hipLaunchKernelGGL((gemm_f32_stream_kernel<kXCols, kOutJI, kMB, KS, kG>), dim3(static_cast<unsigned>(blocks)),
                     dim3(64 * KS), 0, stream, args);
}

template <bool kXCols, bool kOutJI, int kMB>
void launch_stream_ks(const GemmArgs& args, std::int64_t blocks, int ks, hipStream_t stream) {
  switch (ks) {
    case 1: launch_stream_as<kXCols, kOutJI, kMB, 1>(args, blocks, stream); break;
    case 2: launch_stream_as<kXCols, kOutJI, kMB, 2>(args, blocks, stream); break;
    case 4: launch_stream_as<kXCols, kOutJI, kMB, 4>(args, blocks, stream); break;
    case 8: launch_stream_as<kXCols, kOutJI, kMB, 8>(args, blocks, stream); break;
    default: launch_stream_as<kXCols, kOutJI, kMB, 16>(args, blocks, stream); break;
  }
}

// kOutJI: W is the transposed B (at most 32 rows of A); otherwise W is A (at
// most 32 columns of B, kXCols when B is [k, n]). args.total_tiles holds the
// batch count. KS as for the small kernel: about sixteen waves per CU over
// the launch, at most one per 16-k chunk and at most 16.
template <bool kXCols, bool kOutJI>
int launch_stream(GemmArgs& args, hipStream_t stream) {
  const std::int64_t I = kOutJI ? args.n : args.m, J = kOutJI ? args.m : args.n;
  if (J > kStreamMaxSkinny || !stream_fits(args.k))
    return fail(TCX_INTERNAL, "streaming gemm needs at most 32 skinny rows");
  const std::int64_t blocks = (I + 15) / 16 * args.total_tiles;
  if (blocks > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  if constexpr (kOutJI && !kXCols) {
    // The LDS-staged kernel while every block stays resident (24 KB of LDS
    // per wave for one row group of X, 36 KB for two; 160 KB per CU), with up
    // to four waves per block. One wave per block with at most four rows of
    // X left the register kernel ahead (4x14336x4096: 56.6 against 48.1 us).
    const std::int64_t capacity = 256 * (J <= 16 ? 6 : 4);
    const std::int64_t spans = (args.k + 63) / 64;
    int waves = 1;
    while (waves < 4 && waves * 2 <= spans && blocks * waves * 2 <= capacity) waves *= 2;
    if (blocks <= capacity && (waves > 1 || J > 4)) {
      auto go = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(64 * waves), 0, stream, args);
      };
      if (J <= 16)
        go(waves == 1 ? gemm_f32_stream_lds_kernel<1, 1>
                      : waves == 2 ? gemm_f32_stream_lds_kernel<1, 2> : gemm_f32_stream_lds_kernel<1, 4>);
      else
        go(waves == 1 ? gemm_f32_stream_lds_kernel<2, 1>
                      : waves == 2 ? gemm_f32_stream_lds_kernel<2, 2> : gemm_f32_stream_lds_kernel<2, 4>);
      return check(hipGetLastError(), "gemm_f32 streaming launch");
    }
  }
  const std::int64_t chunks = (args.k + 15) / 16;
  int ks = 1;
  while (ks < 16 && ks * 2 <= chunks && blocks * ks < 4096) ks *= 2;
  if (J <= 16)
    launch_stream_ks<kXCols, kOutJI, 1>(args, blocks, ks, stream);
  else
    launch_stream_ks<kXCols, kOutJI, 2>(args, blocks, ks, stream);
  return check(hipGetLastError(), "gemm_f32 streaming launch");
}

template <int BM, int BN, int BK, int WM, int WN, int kMinWaves, bool kVecOnly = false, int KS = 1>
int launch_config(GemmArgs& args, bool trans_b, bool vec, hipStream_t stream) {
  args.tiles_m = (args.m + BM - 1) / BM;
  args.tiles_n = (args.n + BN - 1) / BN;
  const std::int64_t batches = args.total_tiles;  // caller passes the batch count here
  args.total_tiles = args.tiles_m * args.tiles_n * batches;
  if (args.total_tiles > 0x7fffffff) return fail(TCX_INVALID_ARGUMENT, "gemm grid is too large");
  const dim3 grid(static_cast<unsigned>(args.total_tiles));
  const dim3 block((BM / WM) * (BN / WN) * 64 * KS);
  if constexpr (kVecOnly) {
    if (!vec) return fail(TCX_INTERNAL, "gemm tile requires 16-byte aligned operands");
    if (trans_b)
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, true, true, KS>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, false, true, KS>), grid, block, 0, stream, args);
  } else if (trans_b) {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, true, true, KS>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, true, false, KS>), grid, block, 0, stream, args);
  } else {
    if (vec)
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, false, true, KS>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WM, WN, kMinWaves, false, false, KS>), grid, block, 0, stream, args);
  }
  return check(hipGetLastError(), "gemm_f32 launch");
}

}  // namespace gemm
}  // namespace tcx
