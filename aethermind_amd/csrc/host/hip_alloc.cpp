#include "hip_alloc.h"

#include <mutex>
#include <unordered_map>

namespace aethermind::hip_alloc {
namespace {

struct Counters {
  std::mutex mu;
  std::unordered_map<void*, size_t> device_live, pinned_live;  // pointer -> bytes
  am_alloc_stats s{};
};

Counters& C() {
  static Counters c;
  return c;
}

}  // namespace

hipError_t DeviceMallocRaw(void** p, size_t bytes) {
  const hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return e;
  Counters& c = C();
  std::lock_guard<std::mutex> lock(c.mu);
  c.device_live[*p] = bytes;
  c.s.device_allocs += 1;
  c.s.device_bytes_live += static_cast<int64_t>(bytes);
  return e;
}

hipError_t DeviceFree(void* p) {
  if (p == nullptr) return hipSuccess;
  {
    Counters& c = C();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.device_live.find(p);
    if (it != c.device_live.end()) {
      c.s.device_bytes_live -= static_cast<int64_t>(it->second);
      c.device_live.erase(it);
    }
    c.s.device_frees += 1;
  }
  return hipFree(p);
}

hipError_t PinnedMallocRaw(void** p, size_t bytes) {
  const hipError_t e = hipHostMalloc(p, bytes, hipHostMallocDefault);
  if (e != hipSuccess) return e;
  Counters& c = C();
  std::lock_guard<std::mutex> lock(c.mu);
  c.pinned_live[*p] = bytes;
  c.s.pinned_allocs += 1;
  c.s.pinned_bytes_live += static_cast<int64_t>(bytes);
  return e;
}

hipError_t PinnedFree(void* p) {
  if (p == nullptr) return hipSuccess;
  {
    Counters& c = C();
    std::lock_guard<std::mutex> lock(c.mu);
    auto it = c.pinned_live.find(p);
    if (it != c.pinned_live.end()) {
      c.s.pinned_bytes_live -= static_cast<int64_t>(it->second);
      c.pinned_live.erase(it);
    }
    c.s.pinned_frees += 1;
  }
  return hipHostFree(p);
}

hipError_t GraphInstantiate(hipGraphExec_t* exec, hipGraph_t graph) {
  const hipError_t e = hipGraphInstantiate(exec, graph, nullptr, nullptr, 0);
  if (e == hipSuccess) {
    Counters& c = C();
    std::lock_guard<std::mutex> lock(c.mu);
    c.s.graph_instantiations += 1;
  }
  return e;
}

void Snapshot(am_alloc_stats* out) {
  Counters& c = C();
  std::lock_guard<std::mutex> lock(c.mu);
  *out = c.s;
}

}  // namespace aethermind::hip_alloc

extern "C" am_status_code am_debug_alloc_stats(am_alloc_stats* out) {
  if (out == nullptr) return AM_STATUS_INVALID_ARGUMENT;
  aethermind::hip_alloc::Snapshot(out);
  return AM_STATUS_OK;
}
