// Host test of the bounded pool behind tcx_hip_allocate (runtime.hip), through
// its injectable allocator seam: no device is touched. Built with ASan and
// UBSan by tests/cpp/sanitize.mk and run by tests/test_host_sanitizers.py.
//
// It checks the semantics the reference's MemoryPool has
// (cuda_memory_pool.cpp:21-163, exercised by test_cuda_memory_pool.cpp):
// exact-size reuse, the byte and block bounds of the cache, drain-and-retry
// once on out-of-memory, scope rules (single use, not nestable, exit on the
// owning thread), a pool that outlives destroy until its blocks return, free
// failures counted, and pools on many threads at once, with blocks returned
// from threads other than the one that allocated them.

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "tensorcx_hip.h"

namespace {

int failures = 0;

#define CHECK(cond)                                                          \
  do {                                                                       \
    if (!(cond)) {                                                           \
      std::fprintf(stderr, "%s:%d: CHECK failed: %s (last error: %s)\n",     \
                   __FILE__, __LINE__, #cond, tcx_hip_last_error());         \
      ++failures;                                                            \
    }                                                                        \
  } while (0)

// A host "device" with a byte budget; every block is real heap memory, so
// ASan sees a use after free or a double free of a pooled block.
struct FakeDevice {
  std::mutex mutex;
  size_t capacity = 0, used = 0;
  bool fail_free = false;
  std::set<void*> live;
};
FakeDevice* device = nullptr;
thread_local size_t last_size = 0;

int fake_allocate(void** ptr, size_t bytes) {
  std::lock_guard lock(device->mutex);
  if (device->used + bytes > device->capacity) return TCX_POOL_OOM;
  void* p = std::malloc(bytes + sizeof(size_t));
  if (p == nullptr) return TCX_POOL_OOM;
  std::memcpy(p, &bytes, sizeof(size_t));
  std::memset(static_cast<char*>(p) + sizeof(size_t), 0xA5, bytes);
  device->used += bytes;
  *ptr = static_cast<char*>(p) + sizeof(size_t);
  device->live.insert(*ptr);
  last_size = bytes;
  return TCX_OK;
}

int fake_free(void* ptr) {
  std::lock_guard lock(device->mutex);
  if (device->fail_free) return TCX_INTERNAL;
  if (device->live.erase(ptr) != 1) return TCX_INTERNAL;  // not ours, or freed twice
  char* base = static_cast<char*>(ptr) - sizeof(size_t);
  size_t bytes = 0;
  std::memcpy(&bytes, base, sizeof(size_t));
  device->used -= bytes;
  std::free(base);
  return TCX_OK;
}

int fake_clear_error() { return TCX_OK; }

const tcx_hip_pool_runtime_t kRuntime{fake_allocate, fake_free, fake_clear_error};

tcx_hip_pool_t* make_pool(size_t max_bytes, size_t max_blocks) {
  tcx_hip_pool_t* pool = nullptr;
  CHECK(tcx_hip_pool_create(max_bytes, max_blocks, &kRuntime, &pool) == TCX_OK);
  return pool;
}

tcx_hip_pool_stats_t stats_of(tcx_hip_pool_t* pool) {
  tcx_hip_pool_stats_t s{};
  CHECK(tcx_hip_pool_stats(pool, &s) == TCX_OK);
  return s;
}

struct Block {
  void* ptr = nullptr;
  tcx_hip_pool_t* owner = nullptr;
  size_t bytes = 0;
};

Block alloc(size_t bytes, int* code = nullptr) {
  Block b;
  b.bytes = bytes;
  const int rc = tcx_hip_allocate(bytes, &b.ptr, &b.owner);
  if (code != nullptr) *code = rc;
  else CHECK(rc == TCX_OK);
  if (rc == TCX_OK && b.ptr != nullptr) std::memset(b.ptr, 0x3C, bytes);  // the block is writable
  return b;
}

void release(const Block& b) { tcx_hip_release(b.ptr, b.bytes, b.owner); }

void exact_reuse_and_bounds() {
  FakeDevice dev;
  dev.capacity = 1 << 30;
  device = &dev;
  tcx_hip_pool_t* pool = make_pool(3000, 2);
  CHECK(tcx_hip_pool_enter(pool) == TCX_OK);
  Block b1 = alloc(1000);
  CHECK(b1.owner == pool);
  release(b1);
  Block b2 = alloc(1000);
  CHECK(b2.ptr == b1.ptr);
  Block b3 = alloc(999);
  CHECK(b3.ptr != b1.ptr);
  tcx_hip_pool_stats_t s = stats_of(pool);
  CHECK(s.hits == 1 && s.misses == 2 && s.in_use_bytes == 1999);
  Block b4 = alloc(2500);
  release(b2);
  release(b3);
  release(b4);
  s = stats_of(pool);
  CHECK(s.cached_blocks == 2 && s.cached_bytes == 1999 && s.uncached_returns == 1);
  CHECK(s.peak_in_use_bytes == 4499);
  CHECK(tcx_hip_pool_exit(pool) == TCX_OK);
  CHECK(stats_of(pool).cached_blocks == 0 && dev.used == 0);
  tcx_hip_pool_destroy(pool);
  CHECK(dev.live.empty());
}

void drain_and_retry_once() {
  FakeDevice dev;
  dev.capacity = 3000;
  device = &dev;
  tcx_hip_pool_t* pool = make_pool(1 << 20, 8);
  CHECK(tcx_hip_pool_enter(pool) == TCX_OK);
  Block b1 = alloc(2000);
  release(b1);
  Block b2 = alloc(2500);  // out of memory, the cache is drained, the retry succeeds
  tcx_hip_pool_stats_t s = stats_of(pool);
  CHECK(s.oom_retries == 1 && s.cached_blocks == 0 && s.allocation_calls == 3);
  int code = 0;
  Block b3 = alloc(2000, &code);  // nothing cached to drain: a plain failure
  CHECK(code == TCX_INTERNAL && b3.ptr == nullptr);
  CHECK(std::string(tcx_hip_last_error()).find("out of memory") != std::string::npos);
  CHECK(stats_of(pool).allocation_failures == 1);
  release(b2);
  CHECK(tcx_hip_pool_exit(pool) == TCX_OK);
  tcx_hip_pool_destroy(pool);
  CHECK(dev.used == 0 && dev.live.empty());
}

void scope_rules() {
  FakeDevice dev;
  dev.capacity = 1 << 20;
  device = &dev;
  tcx_hip_pool_t* a = make_pool(1 << 20, 8);
  tcx_hip_pool_t* b = make_pool(1 << 20, 8);
  CHECK(tcx_hip_pool_enter(a) == TCX_OK);
  CHECK(tcx_hip_pool_enter(b) == TCX_INVALID_ARGUMENT);  // nested
  CHECK(tcx_hip_pool_exit(b) == TCX_INVALID_ARGUMENT);   // not the active pool
  // Exit on another thread is refused: the pool belongs to this one.
  int other = TCX_OK;
  std::thread([&] { other = tcx_hip_pool_exit(a); }).join();
  CHECK(other == TCX_INVALID_ARGUMENT);
  CHECK(tcx_hip_pool_exit(a) == TCX_OK);
  CHECK(tcx_hip_pool_enter(a) == TCX_INVALID_ARGUMENT);  // single use
  tcx_hip_pool_t* bad = nullptr;
  CHECK(tcx_hip_pool_create(1, 0, nullptr, &bad) == TCX_INVALID_ARGUMENT && bad == nullptr);
  CHECK(tcx_hip_pool_create(1, 4097, nullptr, &bad) == TCX_INVALID_ARGUMENT && bad == nullptr);
  const tcx_hip_pool_runtime_t partial{fake_allocate, nullptr, fake_clear_error};
  CHECK(tcx_hip_pool_create(1, 1, &partial, &bad) == TCX_INVALID_ARGUMENT && bad == nullptr);
  tcx_hip_pool_destroy(a);
  tcx_hip_pool_destroy(b);
  tcx_hip_pool_destroy(nullptr);
  // Zero bytes: no allocation, no owner.
  void* p = reinterpret_cast<void*>(1);
  tcx_hip_pool_t* owner = reinterpret_cast<tcx_hip_pool_t*>(1);
  CHECK(tcx_hip_allocate(0, &p, &owner) == TCX_OK && p == nullptr && owner == nullptr);
  CHECK(dev.live.empty());
}

void outlives_destroy() {
  FakeDevice dev;
  dev.capacity = 1 << 20;
  device = &dev;
  tcx_hip_pool_t* pool = make_pool(1 << 20, 8);
  CHECK(tcx_hip_pool_enter(pool) == TCX_OK);
  Block b = alloc(4096);
  Block c = alloc(128);
  release(c);  // cached
  CHECK(tcx_hip_pool_exit(pool) == TCX_OK);
  tcx_hip_pool_destroy(pool);  // a block is still out: the pool stays until it returns
  CHECK(dev.used == 4096);
  release(b);  // freed (the pool is closed) and the pool goes away
  CHECK(dev.used == 0 && dev.live.empty());
}

void destroy_while_active() {
  FakeDevice dev;
  dev.capacity = 1 << 20;
  device = &dev;
  tcx_hip_pool_t* pool = make_pool(1 << 20, 8);
  CHECK(tcx_hip_pool_enter(pool) == TCX_OK);
  Block b = alloc(256);
  release(b);
  tcx_hip_pool_destroy(pool);  // exits the active scope, frees the cache
  CHECK(dev.used == 0 && dev.live.empty());
  tcx_hip_pool_t* next = make_pool(1 << 20, 8);  // the thread can enter a new pool
  CHECK(tcx_hip_pool_enter(next) == TCX_OK);
  CHECK(tcx_hip_pool_exit(next) == TCX_OK);
  tcx_hip_pool_destroy(next);
}

void free_failures_counted() {
  FakeDevice dev;
  dev.capacity = 1 << 20;
  device = &dev;
  tcx_hip_pool_t* pool = make_pool(1 << 20, 8);
  CHECK(tcx_hip_pool_enter(pool) == TCX_OK);
  Block b = alloc(64);
  void* kept = b.ptr;
  release(b);
  dev.fail_free = true;
  CHECK(tcx_hip_pool_trim(pool) == TCX_INTERNAL);
  tcx_hip_pool_stats_t s = stats_of(pool);
  CHECK(s.free_failures == 1 && s.failed_free_bytes == 64 && s.cached_blocks == 0);
  dev.fail_free = false;
  CHECK(tcx_hip_pool_exit(pool) == TCX_OK);
  tcx_hip_pool_destroy(pool);
  CHECK(fake_free(kept) == TCX_OK);  // the block the failed free left behind
  CHECK(dev.used == 0 && dev.live.empty());
}

// Pools on many threads at once, each caching its own blocks; blocks returned
// on other threads after their pool closed go back to the device.
void many_threads() {
  FakeDevice dev;
  dev.capacity = size_t{1} << 32;
  device = &dev;
  constexpr int kThreads = 8, kRounds = 200;
  std::vector<std::vector<Block>> handoff(kThreads);
  std::atomic<int> ready{0};
  std::vector<std::thread> threads;
  std::atomic<int> errors{0};
  for (int t = 0; t < kThreads; ++t) {
    threads.emplace_back([&, t] {
      tcx_hip_pool_t* pool = nullptr;
      if (tcx_hip_pool_create(1 << 20, 16, &kRuntime, &pool) != TCX_OK) {
        ++errors;
        return;
      }
      ready.fetch_add(1);
      while (ready.load() < kThreads) std::this_thread::yield();
      if (tcx_hip_pool_enter(pool) != TCX_OK) ++errors;
      for (int r = 0; r < kRounds; ++r) {
        const size_t bytes = 64 * (1 + (r + t) % 7);
        void* p = nullptr;
        tcx_hip_pool_t* owner = nullptr;
        if (tcx_hip_allocate(bytes, &p, &owner) != TCX_OK || owner != pool) {
          ++errors;
          continue;
        }
        std::memset(p, t, bytes);
        if (r % 50 == 0) handoff[t].push_back({p, owner, bytes});
        else tcx_hip_release(p, bytes, owner);
      }
      tcx_hip_pool_stats_t s{};
      tcx_hip_pool_stats(pool, &s);
      if (s.hits == 0 || s.cached_blocks > 16) ++errors;
      if (tcx_hip_pool_exit(pool) != TCX_OK) ++errors;
      tcx_hip_pool_destroy(pool);
    });
  }
  for (auto& th : threads) th.join();
  CHECK(errors.load() == 0);
  // Return the handed-off blocks from this thread, after their pools closed.
  for (auto& list : handoff)
    for (const Block& b : list) release(b);
  CHECK(dev.used == 0 && dev.live.empty());
}

}  // namespace

int main() {
  exact_reuse_and_bounds();
  drain_and_retry_once();
  scope_rules();
  outlives_destroy();
  destroy_while_active();
  free_failures_counted();
  many_threads();
  if (failures != 0) {
    std::fprintf(stderr, "%d check(s) failed\n", failures);
    return 1;
  }
  std::printf("pool host test passed\n");
  return 0;
}
