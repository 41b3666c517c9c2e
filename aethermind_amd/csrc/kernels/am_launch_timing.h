// Dispatch-exact timing hook for the decode profile: when a thread arms start/stop
// events, the next GEMV launch on that thread goes through hipExtLaunchKernelGGL with
// them, so the events bracket exactly that dispatch on its stream (event records
// around an ordinary launch also count the queue gaps between dispatches).
#pragma once

#include <hip/hip_runtime.h>

namespace am {

struct LaunchTiming {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
  bool used = false;
};

// this thread's hook (disarmed: start == nullptr)
LaunchTiming& ThreadLaunchTiming() noexcept;

}  // namespace am
