// Runtime profiling: thread-local, bounded host spans and backend device
// intervals. The interface is the one the reference's backends instrument
// against (reference cpp/tensorcx/core/profiling.h): ProfileScope spans,
// begin_profile/end_profile sessions and reserved device-interval slots, so
// the hip backend reports through the same `cx.profile()` surface.
#pragma once

#include <chrono>
#include <cstddef>
#include <cstdint>
#include <optional>
#include <vector>

#include "tensorcx/core/operation.h"

namespace tensorcx {

enum class ProfileCategory {
  kDispatch,
  kAllocation,
  kDeallocation,
  kCopy,
  kCopyAllocate,
  kCompute,
  kMemset,
  kSynchronize,
  kMemoryPool
};

// One host span. `name` and `backend` are static literals.
struct ProfileEvent {
  std::uint64_t id{}, parent_id{}, start_ns{}, duration_ns{}, self_ns{};
  ProfileCategory category{};
  const char* name{};
  const char* backend{};
  std::optional<std::uint64_t> bytes;
  std::optional<OpKind> operation;
};

struct ProfileResult {
  std::uint64_t elapsed_ns{}, dropped_events{};
  std::vector<ProfileEvent> events;
  struct DeviceEvent {
    std::uint64_t id{}, host_event_id{};
    const char* name{};
    const char* backend{};
    std::optional<OpKind> operation;
    std::optional<float> elapsed_ms;
    const char* error{"incomplete"};
  };
  bool device_timing{};
  std::uint64_t dropped_device_events{};
  std::vector<DeviceEvent> device_events;
};

// Starts this thread's session (no nesting); max_events in [1, 100000].
std::uint64_t begin_profile(std::size_t max_events, bool device_timing = false);
// Ends it, on the owning thread, outside every span.
ProfileResult end_profile(std::uint64_t token);
const char* profile_category_name(ProfileCategory category);
const char* profile_operation_name(OpKind operation);

struct ProfileSession;

// A reserved device-interval slot of the active session (empty when device
// timing is off or the slot budget is spent). The backend fills it before its
// synchronous call returns.
struct DeviceProfileToken {
  std::uint64_t session{};
  std::size_t index{};
  explicit operator bool() const noexcept { return session != 0; }
};
DeviceProfileToken reserve_device_profile(const char* name, const char* backend) noexcept;
void finish_device_profile(DeviceProfileToken token, std::optional<float> elapsed_ms, const char* error) noexcept;

// A host steady-clock span on this thread's session. Costs one TLS read when
// no session is active; never allocates (capacity is reserved up front) and
// never throws.
class ProfileScope {
 public:
  ProfileScope(ProfileCategory category, const char* name, const char* backend,
               std::optional<std::uint64_t> bytes = std::nullopt,
               std::optional<OpKind> operation = std::nullopt) noexcept;
  ~ProfileScope() noexcept;
  ProfileScope(const ProfileScope&) = delete;
  ProfileScope& operator=(const ProfileScope&) = delete;

  bool recording() const noexcept { return recorded_; }
  std::uint64_t event_id() const noexcept { return recorded_ ? slot_ + 1 : 0; }
  std::optional<OpKind> operation() const noexcept { return operation_; }
  void set_bytes(std::uint64_t bytes) noexcept;

 private:
  ProfileSession* session_{};
  ProfileScope* parent_{};
  std::chrono::steady_clock::time_point start_{};
  std::uint64_t nested_ns_{};
  std::size_t slot_{};
  bool recorded_{};
  std::optional<OpKind> operation_;
};

}  // namespace tensorcx
