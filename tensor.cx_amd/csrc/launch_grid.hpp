// Launch-size arithmetic of the kernel launchers (plain C++, no HIP types, so
// host tests compile it on its own).
#pragma once

#include <cstdint>

namespace tcx {

// HIP counts a launch's work-items (grid x block) in 32 bits.
constexpr std::int64_t kMaxLaunchWorkItems = (std::int64_t{1} << 32) - 1;

// Block cap of the grid-stride kernels of 256 threads (one item per thread or
// one per wave): 2^22 blocks are 2^30 work-items, and the kernels loop over
// the rest, so no shape is refused for its size.
constexpr std::int64_t kStrideBlocks = std::int64_t{1} << 22;
static_assert(kStrideBlocks * 256 <= kMaxLaunchWorkItems, "a capped 256-thread grid fits HIP's count");

// Enough blocks to cover n items with `per_block` each, at least 1 and at
// most cap.
constexpr unsigned grid_for(std::int64_t n, std::int64_t per_block, std::int64_t cap = 1 << 20) {
  std::int64_t g = (n + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<unsigned>(g);
}

}  // namespace tcx
