// Dispatch-exact timing hook for the decode profile: when a thread arms start/stop
// events, the next GEMV launch on that thread goes through hipExtLaunchKernelGGL with
// them, so the events bracket exactly that dispatch on its stream (event records
// around an ordinary launch also count the queue gaps between dispatches).
//
// The same thread-local record also keeps the name and launch shape of the last
// kernel an entry point launched on the thread (am_gfx950_last_launch), so callers and
// tests can confirm which variant a shape reached.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace am {

struct LaunchTiming {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  bool used = false;
  // last launch on this thread
  char kernel[96] = {0};
  int64_t grid = 0;
  int32_t block_threads = 0;
  int32_t lds_bytes = 0;
};

// this thread's hook (disarmed: start == nullptr)
LaunchTiming& ThreadLaunchTiming() noexcept;

// Records the kernel name (printf format) and launch shape of a launch.
void RecordLaunch(int64_t grid, int32_t block_threads, int32_t lds_bytes, const char* fmt, ...) noexcept
    __attribute__((format(printf, 4, 5)));

}  // namespace am
