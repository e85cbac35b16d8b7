// Device intervals of HipBackend::execute: one per executed operation, HIP
// events recorded on the execution stream before the first and after the last
// launch and read after the synchronising wait that ends every execute (the
// reference's DeviceTimer, backends/cuda/cuda_profiling.h:22-77). The event
// calls go through an Api type, the seam host tests use to fail any step.
#pragma once

#include <cmath>
#include <optional>

#include "tensorcx/core/profiling.h"
#include "tensorcx_hip.h"

namespace tensorcx::hip {

// The event calls of a device interval, through the C ABI.
struct HipEventApi {
  using Event = void*;
  static bool create(Event& event) noexcept { return tcx_hip_event_create(&event) == TCX_OK; }
  static bool record(Event event, tcx_stream_t stream) noexcept {
    return tcx_hip_event_record(event, stream) == TCX_OK;
  }
  static bool wait(Event event) noexcept { return tcx_hip_event_synchronize(event) == TCX_OK; }
  static bool elapsed(float& ms, Event start, Event stop) noexcept {
    return tcx_hip_event_elapsed_ms(start, stop, &ms) == TCX_OK;
  }
  static bool destroy(Event event) noexcept { return tcx_hip_event_destroy(event) == TCX_OK; }
};

// Inactive (no event calls at all) unless the thread's profile session times
// devices and has a slot left. A failed event call becomes the interval's
// error ("event_failed"); an operation that never reached stop() reports
// "launch_failed". Never throws and never changes the operation's status.
template <class Api = HipEventApi>
class DeviceInterval {
 public:
  explicit DeviceInterval(const char* name) noexcept : token_(reserve_device_profile(name, "hip")) {}
  ~DeviceInterval() { finish(); }
  DeviceInterval(const DeviceInterval&) = delete;
  DeviceInterval& operator=(const DeviceInterval&) = delete;

  bool active() const noexcept { return static_cast<bool>(token_); }

  // Before the first launch, on the stream the launches use.
  void start(tcx_stream_t stream) noexcept {
    if (!token_ || error_ || started_) return;
    started_ = true;
    if (!create(start_) || !create(stop_) || !Api::record(*start_, stream)) error_ = "event_failed";
  }
  // The interval cannot be measured (say, the stream was not available).
  void fail() noexcept {
    if (token_ && !error_) error_ = "event_failed";
  }
  // After the last launch was enqueued.
  void stop(tcx_stream_t stream) noexcept {
    if (!token_ || error_ || stopped_) return;
    if (!started_) {
      error_ = "event_failed";
      return;
    }
    stopped_ = true;
    if (!Api::record(*stop_, stream)) error_ = "event_failed";
  }

 private:
  bool create(std::optional<typename Api::Event>& slot) noexcept {
    typename Api::Event event{};
    if (!Api::create(event)) return false;
    slot = event;
    return true;
  }
  void finish() noexcept {
    if (token_) {
      const char* error = error_ ? error_ : !stopped_ ? "launch_failed" : nullptr;
      float ms = 0.F;
      if (!error && (!Api::wait(*stop_) || !Api::elapsed(ms, *start_, *stop_) || !std::isfinite(ms) || ms < 0.F))
        error = "event_failed";
      finish_device_profile(token_, error ? std::nullopt : std::optional<float>(ms), error);
      token_ = {};
    }
    if (stop_) (void)Api::destroy(*stop_);
    if (start_) (void)Api::destroy(*start_);
    start_.reset();
    stop_.reset();
  }

  DeviceProfileToken token_;
  std::optional<typename Api::Event> start_, stop_;
  const char* error_{};
  bool started_{}, stopped_{};
};

}  // namespace tensorcx::hip
