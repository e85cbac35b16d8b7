// fp32 GEMM on gfx950 matrix cores (v_mfma_f32_16x16x4_f32).
//
// C[b] = act(A[b] @ B[b] + bias) with A [m,k] row-major, B [k,n] row-major
// (matmul, reference cpu_backend.cpp:1251-1276) or B given as W [n,k]
// (kLinear, core/inference.cpp:89-102, read in place instead of copying Wᵀ).
//
// The kernel (gemm_kernel.hpp): block tile BM x BN, k-tile BK, staged through
// LDS in two buffers, so one barrier per k-tile covers both the
// write-after-read and read-after-write hazards. Each wave owns a WM x WN tile
// as (WM/16) x (WN/16) MFMA blocks whose accumulators stay in registers for
// the whole k loop; with an in-block K split, KS such wave groups share the
// block tile and add their partial tiles at the end.
//
// MFMA operand layout (16x16x4 f32): lane l supplies A[row l%16][k l/16] and
// B[k l/16][col l%16] and receives D[4*(l/16)+v][l%16] in register v. The
// kernel maps MFMA row r of block i to tile row r*TM + i (and column c of
// block j to tile column c*TN + j), so a lane's TM A values for one k are
// adjacent in LDS (one ds_read_b128 for TM = 4) and its TN outputs of one row
// are adjacent in C (one 16-byte store).
//
// Rounding: each output is a sum of exact-product MFMA partials in fp32 (and,
// with a K split, of KS fp32 partial sums added in a fixed order); the result
// differs from the reference's sequential k order only by summation order,
// which the parity bound max|dC| <= 1e-4 * sqrt(K) * rms(A) * rms(B) covers.


#include <cmath>

#include "gemm_kernel.hpp"

namespace tcx {
namespace {
using gemm::GemmArgs;
using gemm::launch_config;

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15U) == 0; }

// Long-operand rows (16 per block) from which the streaming kernel takes a
// skinny GEMM.
constexpr std::int64_t kStreamMinRows = 256;
// Batched products of items up to 64 x 64 x 64 run the tiny kernel from this
// many items on (fewer items leave the tiled kernels enough tiles).
constexpr std::int64_t kTinyMinBatches = 64;
// Products with K <= 16 stream their output from this many outputs on.
constexpr std::int64_t kSmallKMinOutputs = 65536;
// One-row products against a row-major B take the vector-matrix kernel from
// this many 1024-column blocks on.
constexpr std::int64_t kVecMatMinBlocks = 128;

// Shapes of >= 256 full 128x128 tiles: the direct kernel on 128x128 tiles of
// eight waves (64x32 for a transposed B, 32x64 for a [k, n] B; 64-68 KB of
// LDS and 79-84 registers, so two blocks share a CU), persistent past the
// blocks that fit. Against the 256x256 direct tiles (one block per CU):
// 4096^3 940.0 -> 931.3 us, batched 32x1024^3 495.9 -> 482.8,
// 4096x4096x1024 250.6 -> 243.3 (transposed 258.8 -> 253.5), 8192x8192x1024
// 979.5 -> 959.7; against the K split: 4096x1024x4096 260.2 -> 243.7
// (transposed 265.0 -> 249.6), 2048^3 145.6 -> 125.8.
bool direct128_fits(const tcx_hip_gemm_desc_t* d, std::int64_t batches) {
  return gemm::direct_fits<128, 128, 32>(d->m, d->n, d->k) && (d->m / 128) * (d->n / 128) * batches >= 256;
}

// K split of the direct 128x128 kernel for shapes with fewer than 256 full
// 128x128 tiles and a long K: the smallest power of two that gives >= 512
// items (two blocks per CU; at most 16 splits) when every split keeps >= 384
// of K in whole k-tiles, else the smallest split count that gives >= 384
// items under the same rule (else see below). 1 = none. (First built on
// 256x256 tiles with a 256-block target: 1024x1024x8192 546 -> 261 us at 8
// splits.) Swept over
// split counts 1-8 on MI355X: the 384 floor (512 before) and the fallback
// took 1536^3 88.7 -> 81.5 us (4 splits), 2048x1536x1536 90.2 -> 84.3 (4),
// 1792^3 148.8 -> 121.5 (4), and left 1024^3 (no split), 1024x1024x2048
// (no split) and the other measured shapes as they were.
//   With >= 256 full tiles the unsplit direct kernel runs them in rounds of
// 256 CUs, and a last round that leaves most CUs idle is worth splitting
// K: the split count s in {1, 2, 3, 4, 8} (>= 384 of K in whole k-tiles per
// split) minimising idle(T s / 256) + 0.02 s, where idle(x) = (ceil(x) - x)
// / ceil(x) is the share of the last round left idle and 0.02 s charges the
// partial tiles' traffic. The constants fit a sweep of s = 1-8 on MI355X:
// 3072^3 522 -> 438 us (s = 4), 2304x2304x4096 468 -> 362 (2),
// 3072x2048x2048 238 -> 194 (2), 2560^3 295 -> 288 (4); 4096x3072x1024
// (three full rounds) stays unsplit, 183 against 213 us with s = 2.
std::int64_t gemm_splits(const tcx_hip_gemm_desc_t* d, std::int64_t batches) {
  if (!gemm::direct_fits<128, 128, 32>(d->m, d->n, d->k) || d->n % 4 != 0) return 1;
  const std::int64_t tiles = (d->m / 128) * (d->n / 128) * batches;
  auto whole = [&](std::int64_t splits) { return d->k % (32 * splits) == 0 && d->k / splits >= 384; };
  if (direct128_fits(d, batches)) {
    auto cost = [&](std::int64_t splits) {
      const double x = static_cast<double>(tiles * splits) / 256.0, rounds = std::ceil(x);
      return (rounds - x) / rounds + 0.02 * static_cast<double>(splits);
    };
    std::int64_t best = 1;
    for (const std::int64_t splits : {2, 3, 4, 8})
      if (whole(splits) && cost(splits) < cost(best) - 1e-9) best = splits;
    return best;
  }
  std::int64_t splits = 1;
  while (tiles * splits < 512 && splits < 16) splits *= 2;
  if (splits > 1 && whole(splits)) return splits;
  for (splits = 2; splits <= 16; ++splits)
    if (tiles * splits >= 384 && whole(splits)) return splits;
  // Failing both, with fewer 64x64 tiles than CUs for the unsplit kernels,
  // the most splits that still give >= 256 items (128 x 4096 x 4096: 32
  // tiles, 8 splits, 72.2 -> 43.4 us transposed; 1024 x 1024 x 2048, whose
  // 256 64x64 tiles fill the CUs, stays unsplit: 40.3 against 42.7 us).
  if (tiles * 4 < 256)
    for (splits = 16; splits >= 2; --splits)
      if (tiles * splits >= 256 && whole(splits)) return splits;
  return 1;
}

// Unbatched products whose K or N is not a multiple of 4 cannot use 16-byte
// rows and run the scalar-load kernels (1025^3: 62 us against 23 us for
// 1024^3). With a workspace, large ones run zero-padded copies instead: A [M][K4],
// B [K4][N4] (or [N4][K4]) and the output [M][N4] in the workspace, the
// aligned routes on those, then the output stripped back to [M][N] with the
// bias and activation applied as the kernels' epilogue applies them. The
// padded k terms are 0 x 0. Only products of at least kPadMinWork
// multiply-adds pay for the copies and three extra launches: measured on
// MI355X, padded against scalar loads, 4096 x 4095 x 4096 1058 against 1276
// us, 2048 x 2049 x 2048 249 / 267, 3000 x 3001 x 1000 241 / 253; around
// 10^9 multiply-adds it lost (1000 x 1001 x 999 transposed 40 / 32 us).
constexpr std::int64_t kPadMinWork = std::int64_t{1} << 32;
constexpr std::int64_t kPadAlign = 64;  // floats: 256-byte aligned regions

struct PadPlan {
  bool pad;
  std::int64_t k4, n4, a_floats, b_floats, c_floats;
};

PadPlan pad_plan(const tcx_hip_gemm_desc_t* d) {
  PadPlan p{false, 0, 0, 0, 0, 0};
  if (d->batch_rank != 0 || (d->k % 4 == 0 && d->n % 4 == 0) || d->m * d->n * d->k < kPadMinWork) return p;
  auto up = [](std::int64_t v, std::int64_t q) { return (v + q - 1) / q * q; };
  p.pad = true;
  p.k4 = up(d->k, 4);
  p.n4 = up(d->n, 4);
  p.a_floats = up(d->m * p.k4, kPadAlign);
  p.b_floats = up(p.k4 * p.n4, kPadAlign);
  p.c_floats = up(d->m * p.n4, kPadAlign);
  return p;
}

// out [rows_out][cols_out] = in [rows][cols] (row stride ld), zero past it.
__global__ __launch_bounds__(256) void pad_copy_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                       std::int64_t rows, std::int64_t cols, std::int64_t ld,
                                                       std::int64_t rows_out, std::int64_t cols_out) {
  for (std::int64_t r = blockIdx.y; r < rows_out; r += gridDim.y)
    for (std::int64_t c = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < cols_out;
         c += static_cast<std::int64_t>(gridDim.x) * blockDim.x)
      out[r * cols_out + c] = r < rows && c < cols ? in[r * ld + c] : 0.F;
}

// out [rows][cols] = act(in [rows][ld] + bias[col]): the kernels' epilogue
// (bias added, then the activation) on the padded output.
__global__ __launch_bounds__(256) void strip_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                    const float* __restrict__ bias, std::int64_t rows,
                                                    std::int64_t cols, std::int64_t ld, int act) {
  for (std::int64_t r = blockIdx.y; r < rows; r += gridDim.y)
    for (std::int64_t c = static_cast<std::int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < cols;
         c += static_cast<std::int64_t>(gridDim.x) * blockDim.x) {
      float x = in[r * ld + c];
      if (bias != nullptr) x = x + bias[c];
      out[r * cols + c] = gemm::activate(x, act);
    }
}

dim3 grid2d(std::int64_t rows, std::int64_t cols) {
  const std::int64_t gx = (cols + 255) / 256 < 64 ? (cols + 255) / 256 : 64;
  const std::int64_t gy = rows < 4096 ? rows : 4096;
  return dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
}

std::int64_t batch_product(const tcx_hip_gemm_desc_t* d) {
  std::int64_t batches = 1;
  for (int i = 0; i < d->batch_rank; ++i) batches *= d->batch_shape[i];
  return batches;
}

}  // namespace
}  // namespace tcx

extern "C" size_t tcx_hip_gemm_workspace_bytes(const tcx_hip_gemm_desc_t* d) {
  using namespace tcx;
  if (d == nullptr || d->m <= 0 || d->n <= 0 || d->k <= 0 || d->batch_rank < 0 ||
      d->batch_rank > TCX_HIP_MAX_BATCH_RANK)
    return 0;
  const std::int64_t batches = batch_product(d);
  if (batches <= 0) return 0;
  const PadPlan pad = pad_plan(d);
  if (pad.pad) return static_cast<size_t>(pad.a_floats + pad.b_floats + pad.c_floats) * sizeof(float);
  bool rhs_strides_vec = true;
  for (int i = 0; i < d->batch_rank; ++i) rhs_strides_vec = rhs_strides_vec && d->rhs_batch_strides[i] % 4 == 0;
  if (d->m == 1 && d->rhs_transposed == 0 && d->n >= 512 && d->n % 4 == 0 && rhs_strides_vec &&
      batches * ((d->n / 4 + 255) / 256) < kVecMatMinBlocks) {
    const std::int64_t splits = gemm::vecmat_splits(batches, d->n, d->k);
    return splits > 1 ? static_cast<size_t>(splits * batches * d->n) * sizeof(float) : 0;
  }
  const std::int64_t splits = gemm_splits(d, batches);
  if (splits == 1) return 0;
  return static_cast<size_t>(splits * batches * d->m * d->n) * sizeof(float);
}

extern "C" int tcx_hip_gemm_f32(const float* lhs, const float* rhs, float* out,
                                const tcx_hip_gemm_desc_t* d, tcx_stream_t stream) {
  return tcx_hip_gemm_f32_ws(lhs, rhs, out, d, nullptr, 0, stream);
}

extern "C" int tcx_hip_gemm_f32_ws(const float* lhs, const float* rhs, float* out, const tcx_hip_gemm_desc_t* d,
                                   void* workspace, size_t workspace_bytes, tcx_stream_t stream) {
  using namespace tcx;
  if (d == nullptr) return fail(TCX_INVALID_ARGUMENT, "gemm descriptor is null");
  if (d->m < 0 || d->n < 0 || d->k < 0 || d->batch_count < 0)
    return fail(TCX_INVALID_ARGUMENT, "gemm extents must be non-negative");
  if (d->batch_rank < 0 || d->batch_rank > TCX_HIP_MAX_BATCH_RANK)
    return fail(TCX_INVALID_ARGUMENT, "gemm batch rank exceeds the supported maximum");
  if (d->activation < TCX_ACT_NONE || d->activation > TCX_ACT_GELU)
    return fail(TCX_INVALID_ARGUMENT, "unknown gemm activation");
  std::int64_t batches = 1;
  for (int i = 0; i < d->batch_rank; ++i) batches *= d->batch_shape[i];
  if (batches != d->batch_count) return fail(TCX_INVALID_ARGUMENT, "gemm batch_count mismatch");
  if (d->m == 0 || d->n == 0 || batches == 0) return TCX_OK;
  if (const PadPlan pad = pad_plan(d); pad.pad && d->k > 0 && lhs != nullptr && rhs != nullptr && out != nullptr &&
      workspace != nullptr && aligned16(workspace) &&
      workspace_bytes >= static_cast<size_t>(pad.a_floats + pad.b_floats + pad.c_floats) * sizeof(float)) {
    const int status = ready();
    if (status != TCX_OK) return status;
    const auto s = static_cast<hipStream_t>(stream);
    float* a4 = static_cast<float*>(workspace);
    float* b4 = a4 + pad.a_floats;
    float* c4 = b4 + pad.b_floats;
    const bool trans = d->rhs_transposed != 0;
    hipLaunchKernelGGL(pad_copy_kernel, grid2d(d->m, pad.k4), dim3(256), 0, s, lhs, a4, d->m, d->k, d->k, d->m,
                       pad.k4);
    if (trans)
      hipLaunchKernelGGL(pad_copy_kernel, grid2d(pad.n4, pad.k4), dim3(256), 0, s, rhs, b4, d->n, d->k, d->k,
                         pad.n4, pad.k4);
    else
      hipLaunchKernelGGL(pad_copy_kernel, grid2d(pad.k4, pad.n4), dim3(256), 0, s, rhs, b4, d->k, d->n, d->n,
                         pad.k4, pad.n4);
    int rc = check(hipGetLastError(), "gemm pad launch");
    if (rc != TCX_OK) return rc;
    tcx_hip_gemm_desc_t padded = *d;
    padded.k = pad.k4;
    padded.n = pad.n4;
    padded.bias = nullptr;
    padded.activation = TCX_ACT_NONE;
    rc = tcx_hip_gemm_f32_ws(a4, b4, c4, &padded, nullptr, 0, stream);
    if (rc != TCX_OK) return rc;
    hipLaunchKernelGGL(strip_kernel, grid2d(d->m, d->n), dim3(256), 0, s, c4, out, d->bias, d->m, d->n, pad.n4,
                       d->activation);
    return check(hipGetLastError(), "gemm strip launch");
  }
  if (lhs == nullptr && d->k != 0) return fail(TCX_INVALID_ARGUMENT, "gemm lhs is null");
  if (rhs == nullptr && d->k != 0) return fail(TCX_INVALID_ARGUMENT, "gemm rhs is null");
  if (out == nullptr) return fail(TCX_INVALID_ARGUMENT, "gemm output is null");
  const int status = ready();
  if (status != TCX_OK) return status;

  GemmArgs args{};
  args.lhs = lhs;
  args.rhs = rhs;
  args.out = out;
  args.bias = d->bias;
  args.m = d->m;
  args.n = d->n;
  args.k = d->k;
  args.batch_rank = d->batch_rank;
  args.activation = d->activation;
  bool strides_vec = true;
  for (int i = 0; i < d->batch_rank; ++i) {
    args.batch_shape[i] = d->batch_shape[i];
    args.lhs_bs[i] = d->lhs_batch_strides[i];
    args.rhs_bs[i] = d->rhs_batch_strides[i];
    strides_vec = strides_vec && d->lhs_batch_strides[i] % 4 == 0 && d->rhs_batch_strides[i] % 4 == 0;
  }
  // 16-byte loads need every row start 16-byte aligned: k rows for A (and W),
  // n rows for B and C.
  const bool vec = strides_vec && d->k % 4 == 0 && d->n % 4 == 0 && aligned16(lhs) &&
                   aligned16(rhs) && aligned16(out);
  const bool trans_b = d->rhs_transposed != 0;
  args.total_tiles = batches;
  const auto s = static_cast<hipStream_t>(stream);
  // Tile choice (swept on MI355X over the config shapes): full 128x128 tiles
  // on the direct-to-LDS kernel when there are >= 256 of them; else, with a
  // workspace and a long K, the direct 256x256 kernel split over K. Partial
  // tiles take the register-staged kernels: 256x256 blocks of eight 64x128
  // waves (133 KB of LDS, 2 waves/SIMD) for >= 256 tiles, then, as fewer
  // output tiles leave the CUs short of waves, smaller tiles that split K
  // inside the block: 128x128 blocks of two groups of eight 32x64 waves
  // (4 waves/SIMD) when there are enough of those (below), else 64x64 blocks
  // of four groups of four 32x32 waves when there are >= 128 of those
  // (1000^3), else 32x32 blocks of eight one-wave groups with 32-wide k-tiles
  // (small shapes; 512^3: 17.9 -> 11.8 us). The in-block split gained 7 % on
  // 4096x1024x4096 and 21 % on 1000^3 over the same tiles without it.
  // One row of A against a transposed B, or one column of B: a
  // matrix-vector product, the long operand's rows streamed in whole cache
  // lines (one or no batch axis).
  if (d->batch_rank <= 1 && strides_vec && d->k % 4 == 0 && aligned16(lhs) && aligned16(rhs)) {
    const std::int64_t lbs = d->batch_rank == 1 ? d->lhs_batch_strides[0] : 0;
    const std::int64_t rbs = d->batch_rank == 1 ? d->rhs_batch_strides[0] : 0;
    if (trans_b && d->m == 1)
      return gemm::launch_gemv(rhs, lhs, out, d->bias, d->n, d->k, batches, rbs, lbs, d->n, 1, true,
                               d->activation, s);
    if (d->n == 1)
      return gemm::launch_gemv(lhs, rhs, out, d->bias, d->m, d->k, batches, lbs, rbs, d->m, 1, false,
                               d->activation, s);
  }
  // One row of A against a row-major B per batch item (rows of 512+
  // columns), with enough items x 1024-column chunks to give every CU a
  // block.
  bool rhs_strides_vec = true;  // A's row is read a word at a time: only B's rows need 16 bytes
  for (int i = 0; i < d->batch_rank; ++i) rhs_strides_vec = rhs_strides_vec && d->rhs_batch_strides[i] % 4 == 0;
  if (d->m == 1 && !trans_b && d->n >= 512 && d->n % 4 == 0 && aligned16(rhs) && aligned16(out) &&
      rhs_strides_vec) {
    if (batches * ((d->n / 4 + 255) / 256) >= kVecMatMinBlocks) return gemm::launch_vecmat(args, s);
    // Fewer blocks: K split over blocks, partials in the caller's workspace.
    const std::int64_t splits = gemm::vecmat_splits(batches, d->n, d->k);
    const size_t need = static_cast<size_t>(splits * batches * d->n) * sizeof(float);
    if (splits > 1 && workspace != nullptr && aligned16(workspace) && workspace_bytes >= need) {
      args.splits = static_cast<std::int32_t>(splits);
      args.partial = static_cast<float*>(workspace);
      return gemm::launch_vecmat(args, s);
    }
  }
  // A short K (unbatched, row-major B): the output streamed as float4 from B
  // columns held in registers. Against the tiled kernels: 4096 x 4096 x 4
  // 26.5 -> 15.2 us, x 8 26.5 -> 17.0, x 16 26.6 -> 23.8, 1000000 x 16 x 16
  // 114 -> 36. A transposed B's strided column loads made 3000 x 1028 x 16
  // take 67 us, so it keeps the tiled route.
  if (d->batch_rank == 0 && !trans_b && d->k >= 1 && d->k <= gemm::kSmallK && d->n % 4 == 0 && aligned16(out) &&
      aligned16(rhs) && d->m * d->n >= kSmallKMinOutputs)
    return gemm::launch_smallk(args, false, s);
  // Many small products: whole items staged in LDS, several per block.
  if (batches >= kTinyMinBatches && gemm::tiny_fits(d->m, d->n, d->k)) return gemm::launch_tiny(args, trans_b, s);
  // One skinny operand against a long one: at most 32 rows of A against a
  // transposed B (the decode-time linear x W^T), or at most 32 columns of B.
  // The streaming kernel reads the long operand's rows once, 16 per block.
  // Against the tiled kernels: 1x4096x4096 transposed 25.0 -> 17.1 us,
  // 16x4096x4096 31.8 -> 20.7, 1x11008x4096 49.8 -> 34.7, 4096x16x4096
  // 31.8 -> 20.4, 2048x1x2048 28.3 -> 13.3, 64 batches of 8x1024x1024
  // transposed 255.8 -> 57.6.
  constexpr std::int64_t kSkinny = gemm::kStreamMaxSkinny;
  if (strides_vec && gemm::stream_fits(d->k) && aligned16(lhs)) {
    if (trans_b && d->m <= kSkinny && d->n >= kStreamMinRows && aligned16(rhs))
      return gemm::launch_stream<false, true>(args, s);
    if (d->n <= kSkinny && d->m >= kStreamMinRows) {
      if (!trans_b) return gemm::launch_stream<true, false>(args, s);
      if (aligned16(rhs)) return gemm::launch_stream<false, false>(args, s);
    }
  }
  // Many tiles of a short K (<= 64) and a narrow N (<= 64): the 64x64 tiles
  // spend a block's life on one k-tile's latency; the small kernel's 32x32
  // tiles (register-direct, little LDS, several blocks per CU) halve it:
  // 1000000 x 64 x 64 468 -> 251 us. With wide rows it lost (4096 x 4096 x 64:
  // 30 -> 61 us), so it stays narrow.
  if (vec && d->k <= 64 && d->n <= 64 && gemm::small_fits(d->m, d->n, d->k) &&
      ((d->m + 63) / 64) * ((d->n + 63) / 64) * batches > 768)
    return gemm::launch_small(args, trans_b, s);
  const std::int64_t tiles_256 = ((d->m + 255) / 256) * ((d->n + 255) / 256) * batches;
  // (Unaligned shapes take the scalar-load variant, which does not fit the
  // 256x256 tile's registers; they use the 128x128 tile.)
  // K split over several blocks of the direct 128x128 kernel (gemm_splits)
  // when the caller brought the workspace (tcx_hip_gemm_workspace_bytes).
  if (vec && workspace != nullptr && aligned16(workspace)) {
    const std::int64_t splits = gemm_splits(d, batches);
    const size_t need = static_cast<size_t>(splits * batches * d->m * d->n) * sizeof(float);
    if (splits > 1 && workspace_bytes >= need) {
      args.splits = static_cast<std::int32_t>(splits);
      args.partial = static_cast<float*>(workspace);
      if (trans_b) return gemm::launch_direct<128, 128, 32, 64, 32, 2>(args, true, s);
      return gemm::launch_direct<128, 128, 32, 32, 64, 2>(args, false, s);
    }
  }
  // Full 128x128 tiles, >= 256 of them: the direct-to-LDS kernel (see
  // direct128_fits).
  if (vec && direct128_fits(d, batches)) {
    if (trans_b) return gemm::launch_direct<128, 128, 32, 64, 32, 2>(args, true, s);
    return gemm::launch_direct<128, 128, 32, 32, 64, 2>(args, false, s);
  }
  if (vec && tiles_256 >= 256) return launch_config<256, 256, 32, 64, 128, 2, true>(args, trans_b, true, s);
  // 128x128 tiles when there are >= 256 of them and the last round of 256
  // blocks is >= 90 % full (3000x3000x1000: 576 tiles fill 75 % and ran 221 us
  // against 203 us with 64x64 tiles).
  const std::int64_t tiles_128 = ((d->m + 127) / 128) * ((d->n + 127) / 128) * batches;
  if (tiles_128 >= 256 && tiles_128 * 10 >= (tiles_128 + 255) / 256 * 256 * 9)
    return launch_config<128, 128, 16, 32, 64, 2, false, 2>(args, trans_b, vec, s);
  const std::int64_t tiles_64 = ((d->m + 63) / 64) * ((d->n + 63) / 64) * batches;
  if (tiles_64 < 128) {
    if (vec && gemm::small_fits(d->m, d->n, d->k)) return gemm::launch_small(args, trans_b, s);
    return launch_config<32, 32, 32, 32, 32, 2, false, 8>(args, trans_b, vec, s);
  }
  // Up to three rounds of 64x64 tiles: the direct-to-LDS 64x64 kernel, edge
  // tiles included (1000^3: 30.0 -> 28.5 us, transposed 31.2 -> 28.1 us,
  // 768^3 23.4 -> 22.6 us). With more rounds the register-staged kernel
  // measured as fast or faster (3000x3000x1000: 203 against 212 us). When a
  // last round of at most 128 tiles follows full ones, 32x64 tiles (two
  // blocks per CU) run that round as lone half tiles: 1100^3 48.0 -> 39.1 us,
  // 1200^3 50.2 -> 40.8, 1600^3 92.4 -> 82.0, 4 x 500x600x700 34.2 -> 27.6 us;
  // with a fuller last round, or one round, 64x64 tiles stay ahead by 2-6 %
  // (1280^3, 1400^3, 1700^3; 1000^3 23.5 against 24.6 us).
  if (vec && tiles_64 <= 768 && gemm::direct64_fits(d->m, d->n, d->k)) {
    // Skinny shapes whose 64x64 tiles are mostly padding run the small
    // kernel's 32x32 tiles when those waste at most two thirds as much
    // (8192x4x1000: 23.0 -> 13.1 us, 4x8192x1000: 22.5 -> 10.5 us; 1000^3
    // stays on 64x64 tiles, 24.2 against 33.8 us).
    const std::int64_t tiles_32 = ((d->m + 31) / 32) * ((d->n + 31) / 32) * batches;
    if (8 * tiles_64 > 3 * tiles_32 && gemm::small_fits(d->m, d->n, d->k)) return gemm::launch_small(args, trans_b, s);
    const std::int64_t last = tiles_64 % 256;
    return gemm::launch_direct64(args, trans_b, tiles_64 > 256 && last > 0 && last <= 128, s);
  }
  return launch_config<64, 64, 16, 32, 32, 4, false, 4>(args, trans_b, vec, s);
}
