// C++20 host contract layer: the subset of the reference AetherMind API that the
// Llama prefill/decode path touches, re-implemented for a device backend.
//
// Names, enumerator order and semantics follow the reference headers so that a
// gfx950 backend written against this header is a drop-in behind the reference's
// own registry:
//   Status/StatusCode         include/aethermind/base/status.h:39-60 (1:1 with am_status_code)
//   DeviceType                include/aethermind/base/device.h:23-28 (+kHIP appended)
//   IsaLevel/ExecPhase/WeightFormat/KernelSelector/SelectorMatches
//                             include/aethermind/backend/kernel_selector.h:12-71 (+kGfx950)
//   OpType                    include/aethermind/operators/op_type.h:22-40 (+fused ops appended)
//   KernelFunc/KernelParamsBuilder/kMaxKernelParamsSize
//                             include/aethermind/backend/kernel_types.h:21-51
//   KernelContext             include/aethermind/backend/kernel_context.h:14-22
//   KernelDescriptor          include/aethermind/backend/kernel_descriptor.h:12-57
//   KernelRegistry            src/backend/kernel_registry.cpp:30-142 (contract; flat sorted table here)
//   AM_REGISTER_KERNEL        include/aethermind/backend/kernel_static_registration.h:15-22
//   Backend/BackendFactory    include/aethermind/backend/backend.h:14-28, backend_factory.h:12-17
//   ResolvedKernel            include/aethermind/backend/resolved_kernel.h:11-28
//   Operator                  include/aethermind/operators/operator.h:36-128
//   ExecutionStep/Plan        include/aethermind/execution/execution_plan.h:14-44
//   LayerRunner/Executor      src/execution/layer_runner.cpp:9-93, executor.cpp:8-11
//   RuntimeBindingContext     include/aethermind/execution/runtime_binding_context.h:49-104
//   KVCacheLayout/View/Manager include/aethermind/execution/kv_cache_view.h,
//                             src/execution/kv_cache_{view,manager}.cpp (contract; here a
//                             device slot pool: one HBM allocation, one slot per sequence)
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <span>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <variant>
#include <vector>

#include "am_c_api.h"

namespace aethermind {

// ---------------------------------------------------------------- Status
enum class StatusCode : uint8_t {
  kOk = 0,
  kCancelled,
  kUnknown,
  kInvalidArgument,
  kDeadlineExceeded,
  kNotFound,
  kAlreadyExists,
  kPermissionDenied,
  kResourceExhausted,
  kFailedPrecondition,
  kAborted,
  kOutOfRange,
  kUnimplemented,
  kInternal,
  kUnavailable,
  kDataLoss,
  kOverflow,
  kUnauthenticated
};
static_assert(static_cast<int>(StatusCode::kOutOfRange) == AM_STATUS_OUT_OF_RANGE);
static_assert(static_cast<int>(StatusCode::kUnauthenticated) == AM_STATUS_UNAUTHENTICATED);

class Status {
 public:
  Status() = default;
  Status(StatusCode c, std::string m) : code_(c), msg_(std::move(m)) {}
  static Status Ok() { return {}; }
  static Status InvalidArgument(std::string m) { return {StatusCode::kInvalidArgument, std::move(m)}; }
  static Status NotFound(std::string m) { return {StatusCode::kNotFound, std::move(m)}; }
  static Status AlreadyExists(std::string m) { return {StatusCode::kAlreadyExists, std::move(m)}; }
  static Status FailedPrecondition(std::string m) { return {StatusCode::kFailedPrecondition, std::move(m)}; }
  static Status OutOfRange(std::string m) { return {StatusCode::kOutOfRange, std::move(m)}; }
  static Status ResourceExhausted(std::string m) { return {StatusCode::kResourceExhausted, std::move(m)}; }
  static Status Internal(std::string m) { return {StatusCode::kInternal, std::move(m)}; }
  static Status DataLoss(std::string m) { return {StatusCode::kDataLoss, std::move(m)}; }
  static Status Unimplemented(std::string m) { return {StatusCode::kUnimplemented, std::move(m)}; }
  static Status Overflow(std::string m) { return {StatusCode::kOverflow, std::move(m)}; }
  static Status FromC(am_status_code c, const char* m) {
    return c == AM_STATUS_OK ? Status() : Status(static_cast<StatusCode>(c), m ? m : "");
  }
  bool ok() const noexcept { return code_ == StatusCode::kOk; }
  StatusCode code() const noexcept { return code_; }
  const std::string& message() const noexcept { return msg_; }
  std::string ToString() const;
  am_status_code c_code() const noexcept { return static_cast<am_status_code>(code_); }

 private:
  StatusCode code_ = StatusCode::kOk;
  std::string msg_;
};

template <typename T>
class StatusOr {
 public:
  StatusOr(Status s) : v_(std::move(s)) {}  // NOLINT
  StatusOr(T v) : v_(std::move(v)) {}       // NOLINT
  bool ok() const noexcept { return std::holds_alternative<T>(v_); }
  Status status() const { return ok() ? Status::Ok() : std::get<Status>(v_); }
  T& value() { return std::get<T>(v_); }
  const T& value() const { return std::get<T>(v_); }
  T* operator->() { return &value(); }
  const T* operator->() const { return &value(); }
  T& operator*() { return value(); }

 private:
  std::variant<Status, T> v_;
};

#define AM_RETURN_IF_ERROR(expr)            \
  do {                                      \
    ::aethermind::Status am_s_ = (expr);    \
    if (!am_s_.ok()) return am_s_;          \
  } while (0)

bool CheckOverflowMul(size_t a, size_t b, size_t* out) noexcept;
bool CheckOverflowAdd(size_t a, size_t b, size_t* out) noexcept;

// ---------------------------------------------------------------- dtypes / device
enum class DLDataTypeCode : uint8_t { kInt = 0, kUInt = 1, kFloat = 2, kBFloat = 4 };

struct DataType {
  DLDataTypeCode code = DLDataTypeCode::kFloat;
  uint8_t bits = 0;
  uint16_t lanes = 0;
  constexpr DataType() = default;
  constexpr DataType(DLDataTypeCode c, uint8_t b, uint16_t l = 1) : code(c), bits(b), lanes(l) {}
  static constexpr DataType Float32() { return {DLDataTypeCode::kFloat, 32}; }
  static constexpr DataType Float(int b) { return {DLDataTypeCode::kFloat, static_cast<uint8_t>(b)}; }
  static constexpr DataType BFloat(int b) { return {DLDataTypeCode::kBFloat, static_cast<uint8_t>(b)}; }
  static constexpr DataType Int(int b) { return {DLDataTypeCode::kInt, static_cast<uint8_t>(b)}; }
  static constexpr DataType UInt(int b) { return {DLDataTypeCode::kUInt, static_cast<uint8_t>(b)}; }
  // data_type.h:117-120: nbytes = (bits*lanes+7)/8, so Int(4) occupies one byte per element.
  constexpr size_t nbytes() const { return (static_cast<size_t>(bits) * lanes + 7) / 8; }
  constexpr bool IsUndefined() const { return bits == 0; }
  friend constexpr bool operator==(const DataType& a, const DataType& b) {
    return a.code == b.code && a.bits == b.bits && a.lanes == b.lanes;
  }
};
std::string ToString(const DataType& d);
int32_t ToAmDtype(const DataType& d);  // am_dtype or -1

enum class DeviceType : uint8_t { kCPU = 0, kCUDA, kCANN, kUndefined, kHIP };
const char* ToString(DeviceType t) noexcept;

// ---------------------------------------------------------------- selector
enum class IsaLevel : uint8_t { kScalar = 0, kAVX2, kAVX512, kAMX, kGfx950 };
enum class ExecPhase : uint8_t { kPrefill = 0, kDecode, kBoth };
enum class WeightFormat : uint8_t { kPlain = 0, kPacked, kQuantizedInt8, kQuantizedInt4 };
const char* ToString(IsaLevel) noexcept;
const char* ToString(ExecPhase) noexcept;
const char* ToString(WeightFormat) noexcept;

inline bool PhaseMatches(ExecPhase candidate, ExecPhase request) noexcept {
  return candidate == request || candidate == ExecPhase::kBoth;
}

struct KernelSelector {
  DeviceType device_type = DeviceType::kUndefined;
  DataType act_dtype{};
  DataType weight_dtype{};
  WeightFormat weight_format = WeightFormat::kPlain;
  IsaLevel isa = IsaLevel::kScalar;
  ExecPhase phase = ExecPhase::kBoth;
  friend bool operator==(const KernelSelector& a, const KernelSelector& b) noexcept {
    return a.device_type == b.device_type && a.act_dtype == b.act_dtype && a.weight_dtype == b.weight_dtype &&
           a.weight_format == b.weight_format && a.isa == b.isa && a.phase == b.phase;
  }
};

inline bool SelectorMatches(const KernelSelector& candidate, const KernelSelector& request) noexcept {
  return candidate.device_type == request.device_type && candidate.act_dtype == request.act_dtype &&
         candidate.weight_dtype == request.weight_dtype && candidate.weight_format == request.weight_format &&
         PhaseMatches(candidate.phase, request.phase) && candidate.isa <= request.isa;
}
std::string ToString(const KernelSelector& s);

// ---------------------------------------------------------------- op types
enum class OpType : uint16_t {
  kUnknown = 0,
  kEmbedding,
  kRmsNorm,
  kLinear,
  kMatMul,
  kRoPE,
  kAttention,
  kSilu,
  kSiluMul,
  kElementwiseMul,
  kKVCacheUpdate,
  kAdd,
  kSoftmax,
  kArgmax,
  kReshape,
  kPermute,
  kReorder,
  // Fused decode ops emitted by the gfx950 fusion pass (appended: existing values stay stable).
  kFusedRmsNormQkvRoPEKVUpdate,
  kFusedLinearAdd,
  kFusedRmsNormGateUpSiluMul,
  kFusedRmsNormLmHeadArgmax,
  kEmbedToken,
  kFusedDecodeLayers,  // every layer of one decode token in one persistent launch
  kFusedLinearSplit,   // prefill: one weight whose row ranges are several Linears (q|k|v)
  kFusedLinearSiluMul, // prefill: Linear gate|up -> SiluMul
  kFusedLinearRoPEKVUpdate,  // prefill: Linear q|k|v -> RoPE -> KVCacheUpdate
};
const char* ToString(OpType op) noexcept;

// ---------------------------------------------------------------- tensors
// Borrowed view of device (or host) memory; mirrors tensor_view.h's TensorView /
// MutableTensorView with the shape kept inline (rank <= 4 on this path).
struct TensorView {
  const void* data_ = nullptr;
  DataType dtype_{};
  int64_t shape_[4] = {0, 0, 0, 0};
  int rank_ = 0;
  TensorView() = default;
  TensorView(const void* d, DataType t, std::initializer_list<int64_t> s) : data_(d), dtype_(t) {
    for (int64_t v : s) shape_[rank_++] = v;
  }
  const void* data() const { return data_; }
  DataType dtype() const { return dtype_; }
  int rank() const { return rank_; }
  int64_t dim(int i) const { return shape_[i]; }
  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < rank_; ++i) n *= shape_[i];
    return n;
  }
  bool is_valid() const { return rank_ >= 0 && !dtype_.IsUndefined(); }
};
struct MutableTensorView : TensorView {
  MutableTensorView() = default;
  MutableTensorView(void* d, DataType t, std::initializer_list<int64_t> s) : TensorView(d, t, s) {}
  void* mutable_data() const { return const_cast<void*>(data_); }
};

// ---------------------------------------------------------------- backend contract
class Stream {
 public:
  virtual ~Stream() = default;
};
// Device stream: one HIP stream per runtime; LayerRunner populates KernelContext::stream
// with it (the reference hard-wires nullptr at layer_runner.cpp:14).
class HipStream final : public Stream {
 public:
  explicit HipStream(void* s) : stream_(s) {}
  void* native() const noexcept { return stream_; }

 private:
  void* stream_ = nullptr;
};

struct WorkspaceBinding {
  void* data = nullptr;
  size_t size = 0;
};

struct KernelContext {
  DeviceType device_type = DeviceType::kUndefined;
  Stream* stream = nullptr;
  void* workspace = nullptr;
  WorkspaceBinding workspace_binding{};
  const void* packed_weights = nullptr;
  const void* kernel_params = nullptr;
  std::span<const std::byte> attrs{};
};

using KernelFunc = Status (*)(const KernelContext&) noexcept;
using KernelParamsBuilder = Status (*)(std::span<const TensorView> inputs,
                                       std::span<const MutableTensorView> outputs, void* params_buffer) noexcept;
inline constexpr size_t kMaxKernelParamsSize = 512;

struct KernelDescriptor {
  OpType op_type = OpType::kUnknown;
  KernelSelector selector{};
  KernelFunc kernel_func = nullptr;
  std::string name{};
  int priority = 0;  // higher wins; first registered wins ties
  KernelParamsBuilder params_builder = nullptr;
  size_t params_size = 0;
};
Status ValidateKernelDescriptor(const KernelDescriptor& d) noexcept;

// Kernel table.  Registration appends descriptors under a mutex until the first
// Freeze(); freezing sorts a flat copy by (op type, priority high to low, registration
// order) and records each op type's range, so Resolve is a lock-free scan of one
// contiguous range that returns the first matching entry.  Contract of the reference
// (kernel_registry.cpp:30-112): no registration after freeze (kFailedPrecondition),
// one descriptor per (op type, selector) (kAlreadyExists), no resolve before freeze,
// the highest priority wins and the earlier registration wins a tie (kNotFound when
// nothing matches).
class KernelRegistry {
 public:
  static KernelRegistry& Global() noexcept;
  Status Register(const KernelDescriptor& descriptor);
  StatusOr<const KernelDescriptor*> Resolve(OpType op_type, const KernelSelector& selector) const;
  Status Freeze();
  size_t size() const;
  bool frozen() const noexcept { return frozen_.load(std::memory_order_acquire); }
  StatusOr<std::vector<const KernelDescriptor*>> FindByOpType(OpType op_type) const;
  std::string DebugDump() const;

 private:
  static constexpr size_t kOpSlots = 64;  // OpType values are small integers
  struct Range {
    uint32_t begin = 0, end = 0;
  };
  mutable std::mutex mutex_;
  std::atomic<bool> frozen_{false};
  std::vector<KernelDescriptor> pending_;  // registration order
  std::vector<KernelDescriptor> table_;    // frozen, sorted
  Range ranges_[kOpSlots]{};
};

namespace kernel_registration_detail {
bool RegisterOrDie(const KernelDescriptor& d);
}

#define AM_REGISTER_KERNEL(unique_name, ...)                                                      \
  namespace {                                                                                     \
  [[maybe_unused]] static const bool am_kernel_reg_##unique_name =                                \
      ::aethermind::kernel_registration_detail::RegisterOrDie(__VA_ARGS__);                       \
  }

struct ResolvedKernel {
  OpType op_type = OpType::kUnknown;
  KernelFunc fn = nullptr;
  std::vector<std::byte> attrs{};
  const char* debug_name = nullptr;
  KernelParamsBuilder params_builder = nullptr;
  size_t params_size = 0;
};

struct BackendCapabilities {
  bool supports_packed_weights = true;
  bool supports_quantized_weights = true;
  bool supports_graph_capture = true;
};

class Backend {
 public:
  virtual ~Backend() = default;
  virtual DeviceType device_type() const noexcept = 0;
  virtual const BackendCapabilities& capabilities() const noexcept = 0;
  virtual KernelFunc ResolveKernel(OpType op_type, const KernelSelector& selector) const noexcept = 0;
  virtual StatusOr<ResolvedKernel> ResolveKernelInfo(OpType op_type, const KernelSelector& selector) const noexcept = 0;
  virtual const KernelRegistry* TryGetKernelRegistryForDebug() const noexcept = 0;
};

class BackendFactory {
 public:
  virtual ~BackendFactory() = default;
  virtual DeviceType device_type() const noexcept = 0;
  virtual std::unique_ptr<Backend> Create() const = 0;
};

// Backend registry with lazy creation (backend_registry.cpp:21-44).
class BackendRegistry {
 public:
  Status RegisterFactory(std::unique_ptr<BackendFactory> f);
  StatusOr<Backend*> GetBackend(DeviceType t);

 private:
  std::unordered_map<uint8_t, std::unique_ptr<BackendFactory>> factories_;
  std::unordered_map<uint8_t, std::unique_ptr<Backend>> backends_;
};

// ---------------------------------------------------------------- operators
class RuntimeBindingContext;

class Operator {
 public:
  virtual ~Operator() = default;
  virtual OpType Type() const noexcept = 0;
  virtual const char* Name() const noexcept { return ToString(Type()); }
  // Resolves and caches the kernel (plan-build time only).
  virtual Status Prepare(Backend& backend, const KernelSelector& selector) = 0;
  virtual Status Run(KernelContext& ctx, const RuntimeBindingContext& bindings, size_t step_index) const noexcept = 0;
  virtual const ResolvedKernel& GetResolvedKernel() const noexcept = 0;

 protected:
  // operator.h:115-127: builder placement-constructs the params on the stack,
  // ctx.kernel_params points at them for the duration of fn(ctx).
  Status InvokeResolvedKernel(KernelContext& ctx, std::span<const TensorView> inputs,
                              std::span<const MutableTensorView> outputs) const noexcept {
    const ResolvedKernel& resolved = GetResolvedKernel();
    alignas(std::max_align_t) std::byte buffer[kMaxKernelParamsSize];
    if (resolved.params_builder != nullptr) {
      AM_RETURN_IF_ERROR(resolved.params_builder(inputs, outputs, buffer));
      ctx.kernel_params = buffer;
    }
    return resolved.fn(ctx);
  }
};
using OperatorPtr = std::shared_ptr<const Operator>;

// ---------------------------------------------------------------- execution
struct StepTensorBinding {
  std::vector<TensorView> inputs;
  std::vector<MutableTensorView> outputs;
};

class RuntimeBindingContext {
 public:
  void SetStream(Stream* s) noexcept { stream_ = s; }
  Stream* stream() const noexcept { return stream_; }
  void SetWorkspace(void* p, size_t n) noexcept { ws_ = {p, n}; }
  StatusOr<WorkspaceBinding> BindWorkspace(size_t bytes) const noexcept {
    if (bytes > ws_.size) return Status::ResourceExhausted("workspace requirement exceeds the bound arena");
    return WorkspaceBinding{bytes ? ws_.data : nullptr, bytes};
  }
  void SetStepTensorBinding(size_t step, StepTensorBinding b);
  StatusOr<const StepTensorBinding*> GetStepTensorBinding(size_t step) const noexcept;
  void ClearStepTensorBindings() { bindings_.clear(); }

 private:
  Stream* stream_ = nullptr;
  WorkspaceBinding ws_{};
  std::vector<StepTensorBinding> bindings_;
};

struct ExecutionStep {
  KernelSelector selector{};
  OperatorPtr op{};
  const void* packed_weights = nullptr;
  size_t workspace_bytes = 0;
  const char* debug_name = nullptr;
};

class ExecutionPlan {
 public:
  static StatusOr<ExecutionPlan> Create(std::vector<ExecutionStep> steps);
  const std::vector<ExecutionStep>& steps() const noexcept { return steps_; }
  size_t size() const noexcept { return steps_.size(); }

 private:
  std::vector<ExecutionStep> steps_;
};

class LayerRunner {
 public:
  static Status Run(const ExecutionPlan& plan, RuntimeBindingContext& bindings) noexcept;
  static Status RunStep(size_t index, const ExecutionStep& step, RuntimeBindingContext& bindings) noexcept;
};

class Executor {
 public:
  static Status Execute(const ExecutionPlan& plan, RuntimeBindingContext& bindings) noexcept {
    return LayerRunner::Run(plan, bindings);
  }
};

// ---------------------------------------------------------------- KV cache
struct KVCacheLayout {
  size_t num_layers = 0, num_kv_heads = 0, max_tokens = 0, head_dim = 0;
  size_t head_dim_stride = 0, token_stride = 0, head_stride = 0, layer_stride = 0;
  DataType kv_dtype{};
  size_t alignment = 64;
  size_t ElementBytes() const noexcept { return kv_dtype.nbytes(); }
  Status Validate() const noexcept;
  StatusOr<size_t> Offset(size_t layer, size_t head, size_t pos, size_t dim) const noexcept;
  StatusOr<size_t> BytesPerPlane() const noexcept;
};

// Device KV slot pool.  One allocation holds num_slots slots; a slot is one sequence's
// key planes followed by its value planes, each [layers][kv heads][max_tokens][head_dim]
// with the KVCacheLayout strides above.  Slot s starts s * slot_bytes after slot 0, so
// a batched kernel reaches sequence r's planes at a fixed stride from sequence 0's.
struct KVCacheStorage {
  void* base = nullptr;
  size_t bytes_per_plane = 0;  // one K (or V) plane set, unpadded
  size_t value_offset = 0;     // bytes from a slot's key planes to its value planes
  size_t slot_bytes = 0;       // bytes between consecutive slots
  size_t num_slots = 0;
  bool is_initialized() const noexcept { return base != nullptr; }
  void* key(size_t slot) const noexcept { return static_cast<std::byte*>(base) + slot * slot_bytes; }
  void* value(size_t slot) const noexcept { return static_cast<std::byte*>(key(slot)) + value_offset; }
};

// One sequence's reservation: its token capacity, prompt length and committed position.
// The generation changes on every release, so views of an earlier reservation go stale.
struct SessionKVSlot {
  uint64_t generation = 0;
  bool in_use = false;
  size_t capacity_tokens = 0, prompt_len = 0, current_pos = 0;
  size_t index = 0;  // slot number inside the pool
};

class KVCacheView {
 public:
  KVCacheView() = default;
  KVCacheView(const KVCacheLayout* l, const KVCacheStorage* s, SessionKVSlot* slot) noexcept
      : layout_(l), storage_(s), slot_(slot), generation_(slot ? slot->generation : 0) {}
  bool valid() const noexcept;
  size_t current_pos() const noexcept { return valid() ? slot_->current_pos : 0; }
  size_t token_capacity() const noexcept { return valid() ? slot_->capacity_tokens : 0; }
  size_t slot() const noexcept { return valid() ? slot_->index : 0; }
  size_t max_tokens() const noexcept { return layout_ ? layout_->max_tokens : 0; }
  size_t num_layers() const noexcept { return layout_ ? layout_->num_layers : 0; }
  size_t num_kv_heads() const noexcept { return layout_ ? layout_->num_kv_heads : 0; }
  size_t head_dim() const noexcept { return layout_ ? layout_->head_dim : 0; }
  Status ValidateWrite(size_t layer, size_t head, size_t pos, size_t count) const noexcept;
  Status ValidateRead(size_t layer, size_t head, size_t begin, size_t end) const noexcept;
  // Device address of the [head][pos][dim] plane of `layer` (K or V) in this slot.
  StatusOr<void*> KeyPlane(size_t layer) const noexcept;
  StatusOr<void*> ValuePlane(size_t layer) const noexcept;
  Status CommitUntil(size_t new_pos) noexcept;
  void Invalidate() noexcept { *this = KVCacheView(); }

 private:
  Status CheckLive() const noexcept;
  StatusOr<void*> Plane(bool value, size_t layer) const noexcept;
  const KVCacheLayout* layout_ = nullptr;
  const KVCacheStorage* storage_ = nullptr;
  SessionKVSlot* slot_ = nullptr;
  uint64_t generation_ = 0;
};

// Allocation hooks so the manager logic runs (and is tested) without a GPU.
struct DeviceAllocator {
  void* (*alloc)(size_t bytes, void* user) = nullptr;
  void (*free)(void* p, void* user) = nullptr;
  void* user = nullptr;
};
DeviceAllocator HipDeviceAllocator();
DeviceAllocator HostTestAllocator();

// Static KV cache manager over a slot pool (the reference's KVCacheManager contract,
// kv_cache_manager.cpp:49-150, with one reservation per slot instead of one per
// manager).  With num_slots = 1 it behaves as the reference's: a second active
// reservation is refused.
class KVCacheManager {
 public:
  KVCacheManager() = default;
  explicit KVCacheManager(DeviceAllocator a) : alloc_(a) {}
  ~KVCacheManager();
  KVCacheManager(const KVCacheManager&) = delete;
  KVCacheManager& operator=(const KVCacheManager&) = delete;
  // (Re)builds the pool; refused while a reservation is active.
  Status Init(size_t num_layers, size_t num_kv_heads, size_t max_tokens, size_t head_dim, DataType kv_dtype,
              size_t alignment = 256, size_t num_slots = 1);
  // Reserves the lowest free slot (kFailedPrecondition when every slot is taken).
  StatusOr<KVCacheView> ReserveForSession(size_t prompt_len, size_t max_new_tokens) noexcept;
  // Reserves slot `slot` (a batched session keeps sequence r in slot r).
  StatusOr<KVCacheView> ReserveSlot(size_t slot, size_t prompt_len, size_t max_new_tokens) noexcept;
  Status ResetSession(KVCacheView& view) noexcept;
  Status ReleaseSession(KVCacheView& view) noexcept;
  const KVCacheLayout& layout() const noexcept { return layout_; }
  size_t capacity_tokens() const noexcept { return layout_.max_tokens; }
  size_t total_bytes() const noexcept { return initialized_ ? storage_.slot_bytes * storage_.num_slots : 0; }
  bool is_initialized() const noexcept { return initialized_; }
  const KVCacheStorage& storage() const noexcept { return storage_; }
  size_t num_slots() const noexcept { return slots_.size(); }
  size_t free_slots() const noexcept;

 private:
  void Release() noexcept;
  StatusOr<KVCacheView> Take(SessionKVSlot& s, size_t prompt_len, size_t max_new_tokens) noexcept;
  DeviceAllocator alloc_ = HipDeviceAllocator();
  KVCacheLayout layout_{};
  KVCacheStorage storage_{};
  std::vector<SessionKVSlot> slots_;
  bool initialized_ = false;
};

// Paged (block) KV storage, the Phase-2 direction of the reference's KV design
// (kv_cache_design.md sections 6.7 and 10; aethermind_prd.md:437-444): per layer a
// K pool and a V pool of num_blocks blocks of [kv heads][block_size][head_dim]
// elements, a free list of block ids, and one block table row of table_stride int32
// entries per sequence.  A sequence holds blocks for positions [0, n) only: blocks
// are taken when it grows (lowest free id first) and returned when it is released, so
// sequences of different lengths share one pool.  The device copy of the table is
// the caller's to refresh from host_table() after a change (dirty()).
class KVBlockManager {
 public:
  KVBlockManager() = default;
  explicit KVBlockManager(DeviceAllocator a) : alloc_(a) {}
  ~KVBlockManager();
  KVBlockManager(const KVBlockManager&) = delete;
  KVBlockManager& operator=(const KVBlockManager&) = delete;
  // block_size: a power of two of at least 32; max_tokens: positions per sequence.
  Status Init(size_t num_layers, size_t num_kv_heads, size_t head_dim, DataType kv_dtype, size_t block_size,
              size_t num_blocks, size_t max_seqs, size_t max_tokens);
  // Gives sequence `seq` blocks for positions [0, n).  kResourceExhausted when the
  // free blocks do not cover the growth (then nothing changes); kOutOfRange past
  // max_tokens or for a bad sequence.
  Status EnsureCapacity(size_t seq, size_t n) noexcept;
  // Returns every block of `seq` to the pool and clears its table row.
  Status ReleaseSequence(size_t seq) noexcept;

  void* key_pool(size_t layer) const noexcept;
  void* value_pool(size_t layer) const noexcept;
  int32_t* device_table() const noexcept { return table_dev_; }
  const std::vector<int32_t>& host_table() const noexcept { return table_; }
  bool dirty() const noexcept { return dirty_; }
  void clear_dirty() noexcept { dirty_ = false; }
  size_t block_size() const noexcept { return block_; }
  size_t num_blocks() const noexcept { return num_blocks_; }
  size_t table_stride() const noexcept { return stride_; }
  size_t free_blocks() const noexcept { return free_.size(); }
  size_t blocks_of(size_t seq) const noexcept { return seq < held_.size() ? held_[seq] : 0; }
  size_t pool_bytes() const noexcept { return pool_bytes_; }

 private:
  void Release() noexcept;
  DeviceAllocator alloc_ = HipDeviceAllocator();
  void* pools_ = nullptr;       // [layers][K, V][num_blocks][hkv][block][d]
  int32_t* table_dev_ = nullptr;
  size_t pool_bytes_ = 0, layer_bytes_ = 0;
  size_t block_ = 0, num_blocks_ = 0, stride_ = 0, max_tokens_ = 0;
  std::vector<int32_t> free_;   // free block ids, the lowest at the back
  std::vector<int32_t> table_;  // [max_seqs][stride], -1 = no block
  std::vector<size_t> held_;    // blocks per sequence
  bool dirty_ = false;
};

}  // namespace aethermind
