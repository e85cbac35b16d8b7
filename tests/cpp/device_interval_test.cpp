// Host test of HipBackend's device intervals through their event seam
// (tensor.cx_amd/cpp/tensorcx/backends/hip/hip_device_interval.h): a scripted
// event API fails at each step in turn, and every outcome is checked against
// the profile session's device event (error, elapsed time) and the event
// bookkeeping (every created event destroyed once, nothing timed before it
// was recorded). Exit status 0 when every check holds.
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "tensorcx/backends/hip/hip_device_interval.h"

namespace {

int failures = 0;
void expect(bool ok, const std::string& what) {
  if (!ok) {
    ++failures;
    std::printf("FAIL %s\n", what.c_str());
  }
}

// Scripted events: ids from 1; `fail_call` names the failing call by its
// position in the sequence of all calls (1-based), 0 for none.
struct Script {
  int fail_call = 0;
  int calls = 0;
  int next_id = 0;
  float elapsed = 2.5F;
  std::map<int, int> created, destroyed, recorded;
  std::vector<std::string> log;
  bool step(const char* name) {
    log.emplace_back(name);
    return ++calls != fail_call;
  }
};
Script script;

struct FakeEventApi {
  using Event = int;
  static bool create(Event& event) noexcept {
    if (!script.step("create")) return false;
    event = ++script.next_id;
    script.created[event]++;
    return true;
  }
  static bool record(Event event, tcx_stream_t) noexcept {
    if (!script.step("record")) return false;
    script.recorded[event]++;
    return true;
  }
  static bool wait(Event event) noexcept {
    if (!script.recorded.count(event)) ++failures, std::printf("FAIL wait on an unrecorded event\n");
    return script.step("wait");
  }
  static bool elapsed(float& ms, Event start, Event stop) noexcept {
    if (!script.recorded.count(start) || !script.recorded.count(stop))
      ++failures, std::printf("FAIL elapsed of unrecorded events\n");
    if (!script.step("elapsed")) return false;
    ms = script.elapsed;
    return true;
  }
  static bool destroy(Event event) noexcept {
    script.destroyed[event]++;
    return script.step("destroy");
  }
};

using Interval = tensorcx::hip::DeviceInterval<FakeEventApi>;

// One profiled operation: start, then stop unless `launched` is false.
tensorcx::ProfileResult::DeviceEvent run(int fail_call, bool launched, bool timing = true) {
  script = Script{};
  script.fail_call = fail_call;
  const auto token = tensorcx::begin_profile(16, timing);
  {
    Interval interval("hip_kernels");
    interval.start(nullptr);
    if (launched) interval.stop(nullptr);
  }
  const auto result = tensorcx::end_profile(token);
  if (!timing) {
    expect(result.device_events.empty(), "no device event without device timing");
    return {};
  }
  expect(result.device_events.size() == 1, "one device event per operation");
  return result.device_events.empty() ? tensorcx::ProfileResult::DeviceEvent{} : result.device_events[0];
}

bool balanced() {
  for (const auto& [id, n] : script.created)
    if (n != 1 || script.destroyed[id] != 1) return false;
  for (const auto& [id, n] : script.destroyed)
    if (!script.created.count(id)) return false;
  return true;
}

std::string str(const char* s) { return s ? s : "(none)"; }

}  // namespace

int main() {
  // Success: create, create, record, record, wait, elapsed, destroy, destroy.
  auto ok = run(0, true);
  expect(ok.error == nullptr && ok.elapsed_ms && *ok.elapsed_ms == 2.5F, "success reports the elapsed time");
  expect(script.calls == 8 && balanced(), "success creates, records, reads and destroys two events");
  expect(std::strcmp(ok.name, "hip_kernels") == 0 && std::strcmp(ok.backend, "hip") == 0, "interval name");
  // A failure at each call: no elapsed time, the error named, every created
  // event destroyed exactly once.
  const char* expected[] = {nullptr, "event_failed", "event_failed", "event_failed", "event_failed",
                            "event_failed", "event_failed", nullptr, nullptr};
  for (int call = 1; call <= 8; ++call) {
    const auto event = run(call, true);
    const std::string what = "failure at call " + std::to_string(call) + " (" +
                             (call <= static_cast<int>(script.log.size()) ? script.log[call - 1] : "?") + ")";
    if (call <= 6) {
      expect(str(event.error) == str(expected[call]), what + ": error " + str(event.error));
      expect(!event.elapsed_ms, what + ": no elapsed time");
    } else {
      // A failing destroy after a good reading keeps the reading.
      expect(event.error == nullptr && event.elapsed_ms, what + ": the reading stands");
    }
    expect(balanced(), what + ": every created event destroyed once");
  }
  // The operation never reached stop(): no reading, nothing waited on.
  const auto unlaunched = run(0, false);
  expect(str(unlaunched.error) == "launch_failed" && !unlaunched.elapsed_ms, "launch_failed without stop()");
  expect(balanced() && script.log.size() == 5, "launch_failed: no wait, both events destroyed");
  // A negative or non-finite reading is an event failure.
  script = Script{};
  {
    const auto token = tensorcx::begin_profile(16, true);
    script.elapsed = -1.F;
    {
      Interval interval("hip_kernels");
      interval.start(nullptr);
      interval.stop(nullptr);
    }
    const auto result = tensorcx::end_profile(token);
    expect(result.device_events.size() == 1 && str(result.device_events[0].error) == "event_failed",
           "a negative elapsed time is refused");
  }
  // Device timing off: the interval is inactive and makes no event call.
  run(0, true, false);
  expect(script.calls == 0, "no event call without device timing");
  std::printf("%s (%d failures)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
