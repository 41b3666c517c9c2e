// gfx950 backend: the device-side counterpart of the reference CpuBackend
// (src/backend/cpu/cpu_backend.cpp:7-53).  It registers one KernelFunc per
// (OpType, KernelSelector) through AM_REGISTER_KERNEL; each KernelFunc unpacks the
// POD params built by BuildGfxParams plus the op attrs and calls the matching
// am_gfx950_* C entry point on the HIP stream carried by KernelContext::stream.
#pragma once

#include "am_core.h"
#include "am_gfx950.h"

namespace aethermind::gfx950 {

// Compact tensor reference inside the <= 512-byte params buffer.
struct ArgRef {
  void* p = nullptr;
  int32_t dt = -1;  // am_dtype
  int32_t rank = 0;
  int64_t d[3] = {0, 0, 0};
};

struct GfxParams {
  ArgRef in[7];
  ArgRef out[5];
  int32_t nin = 0, nout = 0;
};
static_assert(sizeof(GfxParams) <= kMaxKernelParamsSize, "params must fit the stack buffer");

Status BuildGfxParams(std::span<const TensorView> inputs, std::span<const MutableTensorView> outputs,
                      void* buffer) noexcept;

// Per-op attributes (ResolvedKernel::attrs bytes, like RmsNormOp::Prepare packing eps,
// rmsnorm_op.cpp:9-29).
struct NormAttrs { float eps; };
struct RopeAttrs { int64_t hq, hkv, d, max_pos; };
// Paged KV (am_gfx950_kv_pages): the cache inputs are block pools and `table` the
// device block table (row r = sequence r); a null table is the contiguous layout.
struct KvPaging {
  const int32_t* table = nullptr;
  int32_t block = 0, stride = 0;
  int64_t num_blocks = 0;
};
struct KvAttrs { int64_t hkv, d, cap; KvPaging pg; };
// batch > 1: q holds batch sequences of seq/batch rows each; sequence r's cache planes
// start cbs elements after sequence r-1's (cbs is the same batch stride for QkvAttrs).
struct AttnAttrs { int64_t hq, hkv, d, cap; int32_t splits; int64_t batch, cbs; KvPaging pg; };
struct QkvAttrs { float eps; int64_t hq, hkv, d, cap, cbs; KvPaging pg; };
struct DecodeLayersAttrs { float eps; int64_t layers, hidden, hq, hkv, d, ffn, cap; };

template <typename T>
std::vector<std::byte> PackAttrs(const T& v) {
  std::vector<std::byte> b(sizeof(T));
  std::memcpy(b.data(), &v, sizeof(T));
  return b;
}

class Gfx950Backend final : public Backend {
 public:
  Gfx950Backend();
  DeviceType device_type() const noexcept override { return DeviceType::kHIP; }
  const BackendCapabilities& capabilities() const noexcept override { return caps_; }
  KernelFunc ResolveKernel(OpType op, const KernelSelector& sel) const noexcept override;
  StatusOr<ResolvedKernel> ResolveKernelInfo(OpType op, const KernelSelector& sel) const noexcept override;
  const KernelRegistry* TryGetKernelRegistryForDebug() const noexcept override { return &KernelRegistry::Global(); }

 private:
  BackendCapabilities caps_{};
};

class Gfx950BackendFactory final : public BackendFactory {
 public:
  DeviceType device_type() const noexcept override { return DeviceType::kHIP; }
  std::unique_ptr<Backend> Create() const override { return std::make_unique<Gfx950Backend>(); }
};

// Executable operator: resolves at Prepare, runs through InvokeResolvedKernel with the
// step's tensor binding (operator.h:115-127 flow).
class DeviceOperator final : public Operator {
 public:
  DeviceOperator(OpType type, std::vector<std::byte> attrs) : type_(type), attrs_(std::move(attrs)) {}
  OpType Type() const noexcept override { return type_; }
  Status Prepare(Backend& backend, const KernelSelector& selector) override;
  Status Run(KernelContext& ctx, const RuntimeBindingContext& bindings, size_t step_index) const noexcept override;
  const ResolvedKernel& GetResolvedKernel() const noexcept override { return resolved_; }

 private:
  OpType type_;
  std::vector<std::byte> attrs_;
  ResolvedKernel resolved_{};
};

// Selector helpers for the gfx950 registrations.
KernelSelector HipSelector(DataType act, DataType weight, WeightFormat fmt, ExecPhase phase);

}  // namespace aethermind::gfx950
