// C ABI runtime layer: status mapping, device discovery, per-thread streams,
// device allocation through the bounded pool, copies and events.

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "common.hpp"

namespace tcx {
namespace {
thread_local std::string last_error;
std::once_flag init_once;
int init_status = TCX_UNAVAILABLE;
std::string init_message;
// The process that loaded the library. A forked child inherits the parent's
// runtime state without its threads or device contexts, so every entry point
// refuses to run there, before any HIP call (the reference's CUDA backend
// refuses the same way, cuda_context.cpp:16-20).
const pid_t load_pid = getpid();
thread_local hipStream_t thread_stream = nullptr;
}  // namespace

void set_error(std::string message) { last_error = std::move(message); }

int fail(int code, std::string message) {
  last_error = std::move(message);
  return code;
}

int check(hipError_t error, const char* what) {
  if (error == hipSuccess) return TCX_OK;
  std::string message = std::string(what) + ": " + hipGetErrorString(error);
  switch (error) {
    case hipErrorNoDevice:
    case hipErrorInvalidDevice:
    case hipErrorInsufficientDriver:
      return fail(TCX_UNAVAILABLE, message);
    case hipErrorInvalidValue:
      return fail(TCX_INVALID_ARGUMENT, message);
    default:
      return fail(TCX_INTERNAL, message);
  }
}

bool forked() { return getpid() != load_pid; }

int refuse_forked() { return fail(TCX_UNAVAILABLE, "HIP requires a fresh process after fork"); }

int ready() { return tcx_hip_init(); }

}  // namespace tcx

// ------------------------------------------------------------ bounded pool
struct tcx_hip_pool {
  std::mutex mutex;
  std::atomic<long> refs{1};
  tcx_hip_pool_runtime_t runtime{};
  bool default_runtime{true};
  tcx_hip_pool_stats_t stats{};
  std::vector<std::pair<void*, size_t>> cached;
  bool used{false};
};

namespace {
thread_local tcx_hip_pool* active_pool = nullptr;

int hip_allocate(void** ptr, size_t bytes) {
  if (tcx::forked()) return tcx::refuse_forked();
  const hipError_t error = hipMalloc(ptr, bytes);
  if (error == hipErrorOutOfMemory) {
    tcx::set_error("hipMalloc: out of memory");
    return TCX_POOL_OOM;
  }
  return tcx::check(error, "hipMalloc");
}
int hip_free(void* ptr) { return tcx::forked() ? tcx::refuse_forked() : tcx::check(hipFree(ptr), "hipFree"); }
int hip_clear_error() {
  if (tcx::forked()) return tcx::refuse_forked();
  const hipError_t error = hipGetLastError();
  if (error == hipErrorOutOfMemory) return TCX_POOL_OOM;
  return tcx::check(error, "pending HIP error");
}

void pool_unref(tcx_hip_pool* pool) {
  if (pool->refs.fetch_sub(1) == 1) {
    for (auto& [ptr, bytes] : pool->cached) pool->runtime.free(ptr);
    delete pool;
  }
}

// Frees every cached block; keeps going after a failure and reports it.
int pool_trim_locked(tcx_hip_pool* pool) {
  int status = TCX_OK;
  for (auto& [ptr, bytes] : pool->cached) {
    ++pool->stats.free_calls;
    const int rc = pool->runtime.free(ptr);
    if (rc != TCX_OK) {
      ++pool->stats.free_failures;
      pool->stats.failed_free_bytes += bytes;
      status = TCX_INTERNAL;
    }
  }
  pool->cached.clear();
  pool->stats.cached_bytes = 0;
  pool->stats.cached_blocks = 0;
  if (status != TCX_OK) return tcx::fail(status, "HIP pool failed to free cached blocks");
  return TCX_OK;
}

int pool_allocate(tcx_hip_pool* pool, size_t bytes, void** ptr) {
  std::lock_guard lock(pool->mutex);
  if (!pool->stats.active || !bytes)
    return tcx::fail(TCX_INVALID_ARGUMENT, "inactive pool or zero-byte allocation");
  auto found = std::find_if(pool->cached.begin(), pool->cached.end(),
                            [=](const auto& b) { return b.second == bytes; });
  if (found != pool->cached.end()) {
    *ptr = found->first;
    pool->cached.erase(found);
    pool->stats.cached_bytes -= bytes;
    ++pool->stats.hits;
  } else {
    ++pool->stats.misses;
    ++pool->stats.allocation_calls;
    int rc = pool->runtime.allocate(ptr, bytes);
    if (rc == TCX_POOL_OOM && !pool->cached.empty()) {
      // Recover only from out-of-memory: drain the cache and retry once.
      const int pending = pool->runtime.clear_error();
      if (pending != TCX_OK && pending != TCX_POOL_OOM) {
        ++pool->stats.allocation_failures;
        return tcx::fail(TCX_INTERNAL, "HIP pool allocation found a prior device error");
      }
      const int drained = pool_trim_locked(pool);
      if (drained != TCX_OK) {
        ++pool->stats.allocation_failures;
        return drained;
      }
      ++pool->stats.oom_retries;
      ++pool->stats.allocation_calls;
      rc = pool->runtime.allocate(ptr, bytes);
    }
    if (rc != TCX_OK) {
      ++pool->stats.allocation_failures;
      return tcx::fail(rc == TCX_POOL_OOM ? TCX_INTERNAL : rc, "HIP pool allocation failed: out of memory");
    }
  }
  pool->stats.cached_blocks = pool->cached.size();
  pool->stats.in_use_bytes += bytes;
  pool->stats.peak_in_use_bytes = std::max(pool->stats.peak_in_use_bytes, pool->stats.in_use_bytes);
  pool->refs.fetch_add(1);
  return TCX_OK;
}

void pool_release(tcx_hip_pool* pool, void* ptr, size_t bytes, bool allow_cache) {
  {
    std::lock_guard lock(pool->mutex);
    pool->stats.in_use_bytes -= bytes;
    bool cache = allow_cache && pool->stats.active && pool->cached.size() < pool->stats.max_cached_blocks &&
                 bytes <= pool->stats.max_cached_bytes - pool->stats.cached_bytes;
    if (cache && pool->default_runtime && tcx::thread_stream != nullptr &&
        hipStreamQuery(tcx::thread_stream) != hipSuccess) {
      // Never cache a block that queued work may still touch.
      ++pool->stats.readiness_failures;
      cache = false;
    }
    if (cache) {
      pool->cached.emplace_back(ptr, bytes);
      pool->stats.cached_bytes += bytes;
      pool->stats.cached_blocks = pool->cached.size();
      pool->stats.peak_cached_bytes = std::max(pool->stats.peak_cached_bytes, pool->stats.cached_bytes);
    } else {
      ++pool->stats.uncached_returns;
      ++pool->stats.free_calls;
      if (pool->runtime.free(ptr) != TCX_OK) {
        ++pool->stats.free_failures;
        pool->stats.failed_free_bytes += bytes;
      }
    }
  }
  pool_unref(pool);
}
}  // namespace

extern "C" {

const char* tcx_hip_last_error(void) { return tcx::last_error.c_str(); }

int tcx_hip_init(void) {
  if (tcx::forked()) return tcx::refuse_forked();
  std::call_once(tcx::init_once, [] {
    hipError_t error = hipInit(0);
    int count = 0;
    if (error == hipSuccess) error = hipGetDeviceCount(&count);
    if (error != hipSuccess) {
      tcx::init_status = error == hipErrorNoDevice ? TCX_UNAVAILABLE : tcx::check(error, "hipInit");
      if (tcx::init_status == TCX_INTERNAL) tcx::init_status = TCX_UNAVAILABLE;
      tcx::init_message = std::string("HIP runtime unavailable: ") + hipGetErrorString(error);
    } else if (count == 0) {
      tcx::init_status = TCX_UNAVAILABLE;
      tcx::init_message = "no HIP device is visible";
    } else {
      tcx::init_status = TCX_OK;
    }
  });
  if (tcx::init_status != TCX_OK) return tcx::fail(tcx::init_status, tcx::init_message);
  return TCX_OK;
}

int tcx_hip_device_count(int* count) {
  *count = 0;
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  return tcx::check(hipGetDeviceCount(count), "hipGetDeviceCount");
}

int tcx_hip_device_info(int device, tcx_hip_device_info_t* info) {
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  std::memset(info, 0, sizeof(*info));
  hipDeviceProp_t prop;
  int rc = tcx::check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
  if (rc != TCX_OK) return rc;
  std::snprintf(info->name, sizeof(info->name), "%s", prop.name);
  std::snprintf(info->arch, sizeof(info->arch), "%s", prop.gcnArchName);
  info->compute_units = prop.multiProcessorCount;
  info->clock_khz = prop.clockRate;
  info->memory_clock_khz = prop.memoryClockRate;
  info->memory_bus_width = prop.memoryBusWidth;
  info->l2_bytes = prop.l2CacheSize;
  info->total_bytes = prop.totalGlobalMem;
  (void)hipRuntimeGetVersion(&info->runtime_version);
  (void)hipDriverGetVersion(&info->driver_version);
  int current = 0;
  (void)hipGetDevice(&current);
  if (current == device) {
    size_t free_bytes = 0, total = 0;
    if (hipMemGetInfo(&free_bytes, &total) == hipSuccess) info->free_bytes = free_bytes;
  }
  return TCX_OK;
}

int tcx_hip_stream(tcx_stream_t* stream) {
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  if (tcx::thread_stream == nullptr) {
    hipStream_t s = nullptr;
    const int rc = tcx::check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    if (rc != TCX_OK) return rc;
    tcx::thread_stream = s;
  }
  *stream = tcx::thread_stream;
  return TCX_OK;
}

int tcx_hip_stream_synchronize(tcx_stream_t stream) {
  if (tcx::forked()) return tcx::refuse_forked();
  return tcx::check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}

int tcx_hip_allocate(size_t bytes, void** ptr, tcx_hip_pool_t** owner) {
  *ptr = nullptr;
  *owner = nullptr;
  if (bytes == 0) return TCX_OK;
  if (active_pool != nullptr) {
    const int rc = pool_allocate(active_pool, bytes, ptr);
    if (rc == TCX_OK) *owner = active_pool;
    return rc;
  }
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  return tcx::check(hipMalloc(ptr, bytes), "hipMalloc");
}

void tcx_hip_release(void* ptr, size_t bytes, tcx_hip_pool_t* owner) {
  if (ptr == nullptr || tcx::forked()) return;  // a child does not own the parent's memory
  if (owner != nullptr) {
    pool_release(owner, ptr, bytes, true);
    return;
  }
  (void)hipFree(ptr);
}

void tcx_hip_release_uncached(void* ptr, size_t bytes, tcx_hip_pool_t* owner) {
  if (ptr == nullptr || tcx::forked()) return;
  if (owner != nullptr) {
    pool_release(owner, ptr, bytes, false);
    return;
  }
  (void)hipFree(ptr);
}

int tcx_hip_borrow_check(const void* ptr, size_t bytes) {
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  if (bytes != 0) {
    if (ptr == nullptr) return tcx::fail(TCX_INVALID_ARGUMENT, "borrowed HIP storage requires data");
    hipPointerAttribute_t attributes{};
    if (hipPointerGetAttributes(&attributes, ptr) != hipSuccess) {
      (void)hipGetLastError();  // an unknown pointer is an argument error, not a sticky one
      return tcx::fail(TCX_INVALID_ARGUMENT, "invalid borrowed HIP pointer");
    }
    if (attributes.type != hipMemoryTypeDevice || attributes.device != 0)
      return tcx::fail(TCX_INVALID_ARGUMENT, "borrowed HIP pointer must be device memory of device 0");
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(ptr)) != hipSuccess) {
      (void)hipGetLastError();
      return tcx::fail(TCX_INVALID_ARGUMENT, "borrowed HIP pointer has no allocation range");
    }
    const auto begin = reinterpret_cast<std::uintptr_t>(base), at = reinterpret_cast<std::uintptr_t>(ptr);
    if (at < begin || at - begin > size || bytes > size - (at - begin))
      return tcx::fail(TCX_INVALID_ARGUMENT, "borrowed HIP range exceeds its allocation");
  }
  // The producer may have queued its writes on any of its streams.
  return tcx::check(hipDeviceSynchronize(), "borrowed HIP readiness");
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, tcx_stream_t stream,
                const char* what) {
  if (bytes == 0) return TCX_OK;
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  const auto s = static_cast<hipStream_t>(stream);
  int rc = tcx::check(hipMemcpyAsync(dst, src, bytes, kind, s), what);
  if (rc != TCX_OK) return rc;
  return tcx::check(hipStreamSynchronize(s), what);
}

int tcx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, tcx_stream_t stream) {
  return copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "hipMemcpy host to device");
}
int tcx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, tcx_stream_t stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "hipMemcpy device to host");
}
int tcx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, tcx_stream_t stream) {
  return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "hipMemcpy device to device");
}

int tcx_hip_pool_create(size_t max_cached_bytes, size_t max_cached_blocks,
                        const tcx_hip_pool_runtime_t* runtime, tcx_hip_pool_t** pool) {
  *pool = nullptr;
  if (max_cached_blocks == 0 || max_cached_blocks > 4096)
    return tcx::fail(TCX_INVALID_ARGUMENT, "max_cached_blocks must be in [1, 4096]");
  if (runtime && (!runtime->allocate || !runtime->free || !runtime->clear_error))
    return tcx::fail(TCX_INVALID_ARGUMENT, "invalid pool runtime");
  auto* p = new (std::nothrow) tcx_hip_pool();
  if (!p) return tcx::fail(TCX_INTERNAL, "pool allocation failed");
  if (runtime) {
    p->runtime = *runtime;
    p->default_runtime = false;
  } else {
    p->runtime = {hip_allocate, hip_free, hip_clear_error};
  }
  p->stats.max_cached_bytes = max_cached_bytes;
  p->stats.max_cached_blocks = max_cached_blocks;
  p->cached.reserve(max_cached_blocks);  // caching a block never allocates host memory
  *pool = p;
  return TCX_OK;
}

int tcx_hip_pool_enter(tcx_hip_pool_t* pool) {
  std::lock_guard lock(pool->mutex);
  if (active_pool != nullptr)
    return tcx::fail(TCX_INVALID_ARGUMENT, "memory pools cannot be nested on the same thread");
  if (pool->used) return tcx::fail(TCX_INVALID_ARGUMENT, "memory pool contexts are single-use");
  if (pool->default_runtime) {
    const int status = tcx::ready();
    if (status != TCX_OK) return status;
  }
  pool->used = true;
  pool->stats.active = 1;
  active_pool = pool;
  return TCX_OK;
}

int tcx_hip_pool_exit(tcx_hip_pool_t* pool) {
  if (active_pool != pool)
    return tcx::fail(TCX_INVALID_ARGUMENT, "memory pool must exit on its owning thread");
  active_pool = nullptr;
  std::lock_guard lock(pool->mutex);
  pool->stats.active = 0;
  return pool_trim_locked(pool);
}

int tcx_hip_pool_trim(tcx_hip_pool_t* pool) {
  std::lock_guard lock(pool->mutex);
  return pool_trim_locked(pool);
}

int tcx_hip_pool_stats(const tcx_hip_pool_t* pool, tcx_hip_pool_stats_t* stats) {
  auto* p = const_cast<tcx_hip_pool_t*>(pool);
  std::lock_guard lock(p->mutex);
  *stats = p->stats;
  return TCX_OK;
}

void tcx_hip_pool_destroy(tcx_hip_pool_t* pool) {
  if (pool == nullptr) return;
  if (active_pool == pool) (void)tcx_hip_pool_exit(pool);
  {
    std::lock_guard lock(pool->mutex);
    pool->stats.active = 0;
    (void)pool_trim_locked(pool);
  }
  pool_unref(pool);
}

int tcx_hip_event_create(void** event) {
  const int status = tcx::ready();
  if (status != TCX_OK) return status;
  hipEvent_t e = nullptr;
  const int rc = tcx::check(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return rc;
}
int tcx_hip_event_record(void* event, tcx_stream_t stream) {
  if (tcx::forked()) return tcx::refuse_forked();
  return tcx::check(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
                    "hipEventRecord");
}
int tcx_hip_event_synchronize(void* event) {
  if (tcx::forked()) return tcx::refuse_forked();
  return tcx::check(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}
int tcx_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (tcx::forked()) return tcx::refuse_forked();
  return tcx::check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                    "hipEventElapsedTime");
}
int tcx_hip_event_destroy(void* event) {
  if (tcx::forked()) return tcx::refuse_forked();
  return tcx::check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

}  // extern "C"
