// Known-answer test of the CPU oracle (oracle/oracle.cpp), test
// infrastructure: built with ASan and UBSan by tests/cpp/sanitize.mk and run
// by tests/test_host_sanitizers.py, with one and with several threads.
//
// The answers come from the reference's own known-answer tests and from what
// the mathematics fixes, not from the oracle's formulas:
//   matmul [[1,2],[3,4]]·[[5,6],[7,8]] = [[19,22],[43,50]]
//     (cpu_backend.cpp:593-621), dyadic operands whose products and sums are
//     exact in float32 (batched_matmul_contract.h:25-26), broadcast batches;
//   sum over axis 1 of [[1..3],[4..6]] = [6, 15] (cpu_backend.cpp:566-591),
//     multi-axis {60, 92, 124} (test_backend_contract.cpp:352-385), int32
//     wrap modulo 2^32 (test_multi_axis_reductions.py:133-140);
//   max: the first NaN wins, signed zeros keep the first occurrence;
//   min/argmax: ties keep the lowest index, a NaN is sticky
//     (test_math_ops.py:62-91,226-234);
//   softmax of a constant row is 1/n, rows sum to 1; RMSNorm of [3, 4] is
//     [3, 4]/sqrt(12.5 + eps); LayerNorm of constant rows is 0, or NaN with
//     eps = 0 (test_cuda_primitives.py:104-111).

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <vector>

using Dim = std::int64_t;

extern "C" {
void oracle_matmul_f32(const float* a, const float* b, float* out, Dim batches, Dim m, Dim n, Dim k,
                       const Dim* lhs_offsets, const Dim* rhs_offsets, int threads);
void oracle_reduce_f32(int op, const float* x, float* out, Dim outer, Dim reduce, Dim inner, int threads);
void oracle_reduce_i32(int op, const std::int32_t* x, std::int32_t* out, Dim outer, Dim reduce, Dim inner,
                       int threads);
void oracle_reduce_axes(int op, int dtype, const void* x, void* out, const Dim* meta, int outer_rank,
                        int rank, Dim groups, Dim reduction_size, int threads);
void oracle_argext(int code, int dtype, const std::uint32_t* x, std::uint32_t* out, const Dim* meta,
                   int rank, Dim groups, Dim reduce, int threads);
void oracle_softmax(const float* x, float* out, Dim outer, Dim reduce, Dim inner, int threads);
void oracle_rmsnorm(const float* x, float* out, Dim outer, Dim reduce, Dim inner, float eps, int threads);
void oracle_layernorm(const float* x, float* out, Dim outer, Dim reduce, Dim inner, float eps, int threads);
}

namespace {

int failures = 0;

#define CHECK(cond)                                                                      \
  do {                                                                                   \
    if (!(cond)) {                                                                       \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond);     \
      ++failures;                                                                        \
    }                                                                                    \
  } while (0)

std::uint32_t word(float v) {
  std::uint32_t w;
  std::memcpy(&w, &v, sizeof w);
  return w;
}

void matmul(int threads) {
  const float a[] = {1, 2, 3, 4}, b[] = {5, 6, 7, 8};
  float c[4];
  const Dim zero = 0;
  oracle_matmul_f32(a, b, c, 1, 2, 2, 2, &zero, &zero, threads);
  CHECK(c[0] == 19 && c[1] == 22 && c[2] == 43 && c[3] == 50);

  // Dyadic operands: every product and partial sum is exact in float32, so
  // the result equals the float64 sum in any order. Two batches of A against
  // one broadcast B (rhs batch offset 0 for both).
  constexpr Dim M = 17, K = 23, N = 19;
  std::vector<float> A(2 * M * K), B(K * N), C(2 * M * N);
  for (Dim i = 0; i < 2 * M * K; ++i) A[i] = static_cast<float>(i % 11 - 5) / 8.0F;
  for (Dim i = 0; i < K * N; ++i) B[i] = static_cast<float>(i % 7 - 3) / 8.0F;
  const Dim lhs[] = {0, M * K}, rhs[] = {0, 0};
  oracle_matmul_f32(A.data(), B.data(), C.data(), 2, M, N, K, lhs, rhs, threads);
  for (Dim b2 = 0; b2 < 2; ++b2)
    for (Dim i = 0; i < M; ++i)
      for (Dim j = 0; j < N; ++j) {
        double s = 0;
        for (Dim k = 0; k < K; ++k) s += double(A[b2 * M * K + i * K + k]) * double(B[k * N + j]);
        CHECK(double(C[b2 * M * N + i * N + j]) == s);
      }
  // K = 0: zeros.
  float z[6] = {1, 1, 1, 1, 1, 1};
  const float unused = 0.0F;
  oracle_matmul_f32(&unused, &unused, z, 1, 2, 3, 0, &zero, &zero, threads);
  for (float v : z) CHECK(v == 0.0F);
}

void reductions(int threads) {
  const float x[] = {1, 2, 3, 4, 5, 6};
  float out[2];
  oracle_reduce_f32(0, x, out, 2, 3, 1, threads);
  CHECK(out[0] == 6 && out[1] == 15);
  oracle_reduce_f32(2, x, out, 2, 3, 1, threads);
  CHECK(out[0] == 2 && out[1] == 5);
  oracle_reduce_f32(1, x, out, 2, 3, 1, threads);
  CHECK(out[0] == 3 && out[1] == 6);
  // First axis of [2, 3] -> [3]: inner stride.
  float cols[3];
  oracle_reduce_f32(0, x, cols, 1, 2, 3, threads);
  CHECK(cols[0] == 5 && cols[1] == 7 && cols[2] == 9);

  // max: the first NaN wins and stops the walk; signed zeros keep the first.
  const float nan = std::numeric_limits<float>::quiet_NaN();
  const float special[] = {1, nan, 7, -0.0F, 0.0F, -1};
  float m[2];
  oracle_reduce_f32(1, special, m, 2, 3, 1, threads);
  CHECK(std::isnan(m[0]) && word(m[1]) == word(-0.0F));

  // Multi-axis: arange(24).reshape(2, 3, 4) summed over axes (0, 2) is
  // {60, 92, 124}. Kept axis 1 (extent 3, stride 4), reduced axes 0 (2, 12)
  // and 2 (4, 1).
  std::vector<float> r(24);
  for (int i = 0; i < 24; ++i) r[i] = static_cast<float>(i);
  const Dim meta[] = {3, 4, 2, 12, 4, 1};
  float sums[3];
  oracle_reduce_axes(0, 0, r.data(), sums, meta, 1, 3, 3, 8, threads);
  CHECK(sums[0] == 60 && sums[1] == 92 && sums[2] == 124);

  // int32: the sum wraps modulo 2^32; max is signed.
  const std::int32_t ints[] = {std::numeric_limits<std::int32_t>::max(), 1, -5, -7};
  std::int32_t isum[2], imax[2];
  oracle_reduce_i32(0, ints, isum, 2, 2, 1, threads);
  CHECK(isum[0] == std::numeric_limits<std::int32_t>::min() && isum[1] == -12);
  oracle_reduce_i32(1, ints, imax, 2, 2, 1, threads);
  CHECK(imax[0] == std::numeric_limits<std::int32_t>::max() && imax[1] == -5);
  // An empty mean is NaN.
  float empty_mean = 0;
  const Dim meta1[] = {1, 1, 0, 1};
  oracle_reduce_axes(2, 0, x, &empty_mean, meta1, 1, 2, 1, 0, threads);
  CHECK(std::isnan(empty_mean));
}

void argext(int threads) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  // Rows: ties (argmax keeps index 1), a NaN (sticky at index 2), signed zeros
  // for min (the first of -0/+0 wins).
  const float x[] = {1, 5, 5, 2, 3, 1, nan, 9, 0.0F, -0.0F, 1, 2};
  std::uint32_t w[12];
  for (int i = 0; i < 12; ++i) w[i] = word(x[i]);
  const Dim meta[] = {3, 4, 4, 1};
  std::uint32_t idx[3], mins[3];
  oracle_argext(4, 0, w, idx, meta, 2, 3, 4, threads);
  CHECK(idx[0] == 1 && idx[1] == 2 && idx[2] == 3);
  oracle_argext(3, 0, w, mins, meta, 2, 3, 4, threads);
  CHECK(mins[0] == word(1.0F) && (mins[1] & 0x7fffffffu) > 0x7f800000u && mins[2] == word(0.0F));
  // int32 argmax: ties keep the lowest index.
  const std::int32_t ints[] = {-3, 8, 8, -9};
  std::uint32_t iw[4], ii[1];
  std::memcpy(iw, ints, sizeof iw);
  const Dim meta2[] = {1, 4, 4, 1};
  oracle_argext(4, 1, iw, ii, meta2, 2, 1, 4, threads);
  CHECK(ii[0] == 1);
}

void rows(int threads) {
  // Softmax: a constant row gives exactly 1/n; a row sums to 1.
  const float c[] = {2, 2, 2, 2};
  float s[4];
  oracle_softmax(c, s, 1, 4, 1, threads);
  for (float v : s) CHECK(v == 0.25F);
  const float x[] = {-3, 0.5F, 7, 1e-3F, 2};
  float p[5];
  oracle_softmax(x, p, 1, 5, 1, threads);
  double total = 0;
  for (float v : p) total += v;
  CHECK(std::fabs(total - 1.0) < 1e-6);
  CHECK(p[2] > p[4] && p[4] > p[1] && p[1] > p[3] && p[3] > p[0]);

  // RMSNorm of [3, 4]: mean square 12.5.
  const float r[] = {3, 4};
  float rn[2];
  oracle_rmsnorm(r, rn, 1, 2, 1, 0.0F, threads);
  CHECK(std::fabs(rn[0] - 3.0 / std::sqrt(12.5)) < 1e-6 && std::fabs(rn[1] - 4.0 / std::sqrt(12.5)) < 1e-6);

  // LayerNorm: constant finite rows give 0, or NaN when eps = 0; [1, 3] gives
  // [-1, 1] / sqrt(1 + eps).
  const float k[] = {0.3F, 0.3F, 0.3F, 1e38F, 1e38F, 1e38F};
  float ln[6];
  oracle_layernorm(k, ln, 2, 3, 1, 1e-5F, threads);
  for (float v : ln) CHECK(v == 0.0F);
  oracle_layernorm(k, ln, 2, 3, 1, 0.0F, threads);
  for (float v : ln) CHECK(std::isnan(v));
  const float two[] = {1, 3};
  float l2[2];
  oracle_layernorm(two, l2, 1, 2, 1, 0.0F, threads);
  CHECK(l2[0] == -1.0F && l2[1] == 1.0F);
}

}  // namespace

int main() {
  for (int threads : {1, 4}) {
    matmul(threads);
    reductions(threads);
    argext(threads);
    rows(threads);
  }
  if (failures != 0) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("oracle known-answer test passed\n");
  return 0;
}
