// Host test of the launchers' grid arithmetic (tensor.cx_amd/csrc/launch_grid.hpp):
// every grid-stride launch stays within HIP's 32-bit work-item count for any
// item count up to 2^62, and shapes below the cap keep one item per thread or
// wave (a single pass). Exit status 0 when every check holds.
#include <cstdint>
#include <cstdio>
#include <initializer_list>

#include "launch_grid.hpp"

namespace {

int failures = 0;

void expect(bool ok, const char* what, std::int64_t n, std::int64_t per_block) {
  if (!ok) {
    ++failures;
    std::printf("FAIL %s: n=%lld per_block=%lld\n", what, static_cast<long long>(n),
                static_cast<long long>(per_block));
  }
}

}  // namespace

int main() {
  using tcx::grid_for;
  // (items per block, threads per block) of the grid-stride launchers:
  // one item per thread (reduce lane/axes kernels, row_lane_kernel), one per
  // wave (row_kernel with wave items, four waves per block) and one per block
  // (row_kernel with block items).
  const std::int64_t shapes[][2] = {{256, 256}, {4, 256}, {1, 256}};
  std::int64_t sizes[64];
  int count = 0;
  for (std::int64_t v : {0LL, 1LL, 3LL, 4LL, 5LL, 255LL, 256LL, 257LL, 65535LL, 65536LL, 1LL << 20, (1LL << 24) - 1,
                         1LL << 24, (1LL << 24) + 1, (1LL << 26) + 3, 1LL << 30, (1LL << 32) - 1, 1LL << 32,
                         (1LL << 32) + 7, 3LL << 33, 1LL << 40, 1LL << 50, 1LL << 62})
    sizes[count++] = v;
  for (const auto& shape : shapes) {
    const std::int64_t per_block = shape[0], threads = shape[1];
    for (int i = 0; i < count; ++i) {
      const std::int64_t n = sizes[i];
      const std::int64_t blocks = grid_for(n, per_block, tcx::kStrideBlocks);
      expect(blocks >= 1, "at least one block", n, per_block);
      expect(blocks <= tcx::kStrideBlocks, "grid within the cap", n, per_block);
      expect(blocks * threads <= tcx::kMaxLaunchWorkItems, "work-items fit 32 bits", n, per_block);
      // A grid-stride loop of stride blocks * per_block reaches every item;
      // below the cap it is a single pass.
      const std::int64_t stride = blocks * per_block;
      expect(stride >= 1, "positive stride", n, per_block);
      if (n <= tcx::kStrideBlocks * per_block) expect(stride >= n, "one pass below the cap", n, per_block);
      else expect(blocks == tcx::kStrideBlocks, "full grid above the cap", n, per_block);
    }
  }
  // The uncapped default still covers what it is used for (elementwise grids
  // cap themselves below 2^20 blocks).
  expect(grid_for(1LL << 40, 256) == (1U << 20), "default cap", 1LL << 40, 256);
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
