// The one place the host runtime takes device and pinned host memory, and
// instantiates HIP graphs (which take device memory of their own).  Every call is
// counted process-wide, so a test can show that steady-state decode allocates nothing
// (am_debug_alloc_stats in am_runtime.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "am_runtime.h"

namespace aethermind::hip_alloc {

hipError_t DeviceMallocRaw(void** p, size_t bytes);
hipError_t DeviceFree(void* p);
hipError_t PinnedMallocRaw(void** p, size_t bytes);
hipError_t PinnedFree(void* p);
hipError_t GraphInstantiate(hipGraphExec_t* exec, hipGraph_t graph);
void Snapshot(am_alloc_stats* out);

template <typename T>
hipError_t DeviceMalloc(T** p, size_t bytes) {
  return DeviceMallocRaw(reinterpret_cast<void**>(p), bytes);
}
template <typename T>
hipError_t PinnedMalloc(T** p, size_t bytes) {
  return PinnedMallocRaw(reinterpret_cast<void**>(p), bytes);
}

}  // namespace aethermind::hip_alloc
