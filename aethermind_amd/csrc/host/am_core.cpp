// Implementation of the host contract layer (see am_core.h for the reference map).

#include "am_core.h"

#include <hip/hip_runtime.h>

#include "am_gfx950.h"

#include <cstdio>
#include <cstdlib>

namespace aethermind {

// ---------------------------------------------------------------- status / utils
std::string Status::ToString() const {
  static const char* names[] = {"OK",          "CANCELLED",          "UNKNOWN",          "INVALID_ARGUMENT",
                                "DEADLINE_EXCEEDED", "NOT_FOUND",     "ALREADY_EXISTS",   "PERMISSION_DENIED",
                                "RESOURCE_EXHAUSTED", "FAILED_PRECONDITION", "ABORTED",   "OUT_OF_RANGE",
                                "UNIMPLEMENTED", "INTERNAL",          "UNAVAILABLE",      "DATA_LOSS",
                                "OVERFLOW",    "UNAUTHENTICATED"};
  const int c = static_cast<int>(code_);
  std::string s = (c >= 0 && c < 18) ? names[c] : "?";
  if (!msg_.empty()) s += ": " + msg_;
  return s;
}

bool CheckOverflowMul(size_t a, size_t b, size_t* out) noexcept { return __builtin_mul_overflow(a, b, out); }
bool CheckOverflowAdd(size_t a, size_t b, size_t* out) noexcept { return __builtin_add_overflow(a, b, out); }

std::string ToString(const DataType& d) {
  const char* base = "?";
  switch (d.code) {
    case DLDataTypeCode::kInt: base = "int"; break;
    case DLDataTypeCode::kUInt: base = "uint"; break;
    case DLDataTypeCode::kFloat: base = "float"; break;
    case DLDataTypeCode::kBFloat: base = "bfloat"; break;
  }
  return std::string(base) + std::to_string(d.bits);
}

int32_t ToAmDtype(const DataType& d) {
  if (d == DataType::Float32()) return AM_DT_F32;
  if (d == DataType::BFloat(16)) return AM_DT_BF16;
  if (d == DataType::Float(16)) return AM_DT_F16;
  if (d == DataType::Int(8)) return AM_DT_I8;
  if (d == DataType::Int(4)) return AM_DT_I4;
  if (d == DataType::Int(32)) return AM_DT_I32;
  if (d == DataType::Int(64)) return AM_DT_I64;
  if (d == DataType::UInt(32)) return AM_DT_U32;
  if (d == DataType::UInt(8)) return AM_DT_U8;
  return -1;
}

const char* ToString(DeviceType t) noexcept {
  switch (t) {
    case DeviceType::kCPU: return "cpu";
    case DeviceType::kCUDA: return "cuda";
    case DeviceType::kCANN: return "cann";
    case DeviceType::kHIP: return "hip";
    default: return "undefined";
  }
}
const char* ToString(IsaLevel i) noexcept {
  static const char* n[] = {"scalar", "avx2", "avx512", "amx", "gfx950"};
  return static_cast<int>(i) < 5 ? n[static_cast<int>(i)] : "?";
}
const char* ToString(ExecPhase p) noexcept {
  static const char* n[] = {"prefill", "decode", "both"};
  return static_cast<int>(p) < 3 ? n[static_cast<int>(p)] : "?";
}
const char* ToString(WeightFormat f) noexcept {
  static const char* n[] = {"plain", "packed", "int8", "int4"};
  return static_cast<int>(f) < 4 ? n[static_cast<int>(f)] : "?";
}
std::string ToString(const KernelSelector& s) {
  return std::string("{device=") + ToString(s.device_type) + ", act=" + ToString(s.act_dtype) +
         ", weight=" + ToString(s.weight_dtype) + ", format=" + ToString(s.weight_format) +
         ", isa=" + ToString(s.isa) + ", phase=" + ToString(s.phase) + "}";
}

const char* ToString(OpType op) noexcept {
  switch (op) {
    case OpType::kEmbedding: return "Embedding";
    case OpType::kRmsNorm: return "RmsNorm";
    case OpType::kLinear: return "Linear";
    case OpType::kMatMul: return "MatMul";
    case OpType::kRoPE: return "RoPE";
    case OpType::kAttention: return "Attention";
    case OpType::kSilu: return "Silu";
    case OpType::kSiluMul: return "SiluMul";
    case OpType::kElementwiseMul: return "ElementwiseMul";
    case OpType::kKVCacheUpdate: return "KVCacheUpdate";
    case OpType::kAdd: return "Add";
    case OpType::kSoftmax: return "Softmax";
    case OpType::kArgmax: return "Argmax";
    case OpType::kReshape: return "Reshape";
    case OpType::kPermute: return "Permute";
    case OpType::kReorder: return "Reorder";
    case OpType::kFusedRmsNormQkvRoPEKVUpdate: return "FusedRmsNormQkvRoPEKVUpdate";
    case OpType::kFusedLinearAdd: return "FusedLinearAdd";
    case OpType::kFusedRmsNormGateUpSiluMul: return "FusedRmsNormGateUpSiluMul";
    case OpType::kFusedDecodeLayers: return "FusedDecodeLayers";
    case OpType::kFusedRmsNormLmHeadArgmax: return "FusedRmsNormLmHeadArgmax";
    case OpType::kEmbedToken: return "EmbedToken";
    default: return "Unknown";
  }
}

// ---------------------------------------------------------------- registry
Status ValidateKernelDescriptor(const KernelDescriptor& d) noexcept {
  if (d.op_type == OpType::kUnknown) return Status::InvalidArgument("Kernel descriptor op_type cannot be kUnknown");
  if (d.kernel_func == nullptr) return Status::InvalidArgument("Kernel descriptor function cannot be null");
  if (d.name.empty()) return Status::InvalidArgument("Kernel descriptor name cannot be empty");
  if (d.selector.device_type == DeviceType::kUndefined)
    return Status::InvalidArgument("Kernel descriptor device_type cannot be kUndefined");
  if (d.params_builder != nullptr) {
    if (d.params_size == 0) return Status::InvalidArgument("params_size must be > 0 when params_builder is set");
    if (d.params_size > kMaxKernelParamsSize) return Status::InvalidArgument("params_size exceeds kMaxKernelParamsSize");
  }
  return Status::Ok();
}

size_t KernelRegistry::KeyHash::operator()(const Key& k) const noexcept {
  size_t h = static_cast<size_t>(k.op);
  auto mix = [&h](size_t v) { h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2); };
  mix(static_cast<size_t>(k.sel.device_type));
  mix((static_cast<size_t>(k.sel.act_dtype.code) << 24) | (static_cast<size_t>(k.sel.act_dtype.bits) << 16) |
      k.sel.act_dtype.lanes);
  mix((static_cast<size_t>(k.sel.weight_dtype.code) << 24) | (static_cast<size_t>(k.sel.weight_dtype.bits) << 16) |
      k.sel.weight_dtype.lanes);
  mix(static_cast<size_t>(k.sel.weight_format));
  mix(static_cast<size_t>(k.sel.isa));
  mix(static_cast<size_t>(k.sel.phase));
  return h;
}

KernelRegistry& KernelRegistry::Global() noexcept {
  static KernelRegistry r;
  return r;
}

Status KernelRegistry::Register(const KernelDescriptor& d) {
  std::lock_guard<std::mutex> lock(mutex_);
  if (frozen_.load(std::memory_order_relaxed))
    return Status::FailedPrecondition("Cannot register kernel after registry has been frozen");
  AM_RETURN_IF_ERROR(ValidateKernelDescriptor(d));
  if (!keys_.insert(Key{d.op_type, d.selector}).second) return Status::AlreadyExists("Duplicate kernel registration");
  kernels_.push_back(d);
  return Status::Ok();
}

Status KernelRegistry::Freeze() {
  std::lock_guard<std::mutex> lock(mutex_);
  if (frozen_.load(std::memory_order_relaxed)) return Status::Ok();
  std::unordered_map<uint16_t, std::vector<size_t>> b;
  for (size_t i = 0; i < kernels_.size(); ++i) b[static_cast<uint16_t>(kernels_[i].op_type)].push_back(i);
  buckets_.swap(b);
  frozen_.store(true, std::memory_order_release);
  return Status::Ok();
}

StatusOr<const KernelDescriptor*> KernelRegistry::Resolve(OpType op_type, const KernelSelector& selector) const {
  if (!frozen_.load(std::memory_order_acquire))
    return Status::FailedPrecondition("Cannot resolve kernel before registry has been frozen");
  if (op_type == OpType::kUnknown) return Status::InvalidArgument("op_type cannot be kUnknown");
  if (selector.device_type == DeviceType::kUndefined) return Status::InvalidArgument("device_type cannot be kUndefined");
  const KernelDescriptor* best = nullptr;
  if (auto it = buckets_.find(static_cast<uint16_t>(op_type)); it != buckets_.end()) {
    for (size_t idx : it->second) {
      const KernelDescriptor& d = kernels_[idx];
      if (!SelectorMatches(d.selector, selector)) continue;
      if (best == nullptr || d.priority > best->priority) best = &d;
    }
  }
  if (best == nullptr)
    return Status::NotFound(std::string("No matching kernel registered for op_type=") + ToString(op_type) +
                            ", selector=" + ToString(selector));
  return best;
}

size_t KernelRegistry::size() const {
  std::lock_guard<std::mutex> lock(mutex_);
  return kernels_.size();
}

StatusOr<std::vector<const KernelDescriptor*>> KernelRegistry::FindByOpType(OpType op_type) const {
  if (!frozen_.load(std::memory_order_acquire))
    return Status::FailedPrecondition("Cannot find kernels by op_type before registry has been frozen");
  std::vector<const KernelDescriptor*> out;
  if (auto it = buckets_.find(static_cast<uint16_t>(op_type)); it != buckets_.end())
    for (size_t idx : it->second) out.push_back(&kernels_[idx]);
  return out;
}

std::string KernelRegistry::DebugDump() const {
  std::lock_guard<std::mutex> lock(mutex_);
  std::string out;
  for (size_t i = 0; i < kernels_.size(); ++i) {
    if (i) out += '\n';
    out += std::string(ToString(kernels_[i].op_type)) + " | " + kernels_[i].name + " | " +
           ToString(kernels_[i].selector) + " | priority=" + std::to_string(kernels_[i].priority);
  }
  return out;
}

namespace kernel_registration_detail {
bool RegisterOrDie(const KernelDescriptor& d) {
  const Status s = KernelRegistry::Global().Register(d);
  if (!s.ok()) {
    std::fprintf(stderr, "Kernel registration failed: %s\n", s.ToString().c_str());
    std::abort();
  }
  return true;
}
}  // namespace kernel_registration_detail

Status BackendRegistry::RegisterFactory(std::unique_ptr<BackendFactory> f) {
  if (!f) return Status::InvalidArgument("backend factory is null");
  const uint8_t k = static_cast<uint8_t>(f->device_type());
  factories_[k] = std::move(f);
  backends_.erase(k);
  return Status::Ok();
}

StatusOr<Backend*> BackendRegistry::GetBackend(DeviceType t) {
  const uint8_t k = static_cast<uint8_t>(t);
  if (auto it = backends_.find(k); it != backends_.end()) return it->second.get();
  auto f = factories_.find(k);
  if (f == factories_.end()) return Status::NotFound(std::string("No backend factory for device ") + ToString(t));
  auto b = f->second->Create();
  if (!b) return Status::Internal("backend factory returned null");
  Backend* raw = b.get();
  backends_[k] = std::move(b);
  return raw;
}

// ---------------------------------------------------------------- execution
void RuntimeBindingContext::SetStepTensorBinding(size_t step, StepTensorBinding b) {
  if (bindings_.size() <= step) bindings_.resize(step + 1);
  bindings_[step] = std::move(b);
}

StatusOr<const StepTensorBinding*> RuntimeBindingContext::GetStepTensorBinding(size_t step) const noexcept {
  if (step >= bindings_.size()) return Status::NotFound("no tensor binding for execution step");
  return &bindings_[step];
}

StatusOr<ExecutionPlan> ExecutionPlan::Create(std::vector<ExecutionStep> steps) {
  for (const auto& s : steps)
    if (s.op == nullptr) return Status::InvalidArgument("Execution step operator cannot be null");
  ExecutionPlan p;
  p.steps_ = std::move(steps);
  return p;
}

Status LayerRunner::Run(const ExecutionPlan& plan, RuntimeBindingContext& bindings) noexcept {
  const auto& steps = plan.steps();
  for (size_t i = 0; i < steps.size(); ++i) AM_RETURN_IF_ERROR(RunStep(i, steps[i], bindings));
  return Status::Ok();
}

Status LayerRunner::RunStep(size_t index, const ExecutionStep& step, RuntimeBindingContext& bindings) noexcept {
  if (step.op == nullptr) return Status::InvalidArgument("Execution step operator cannot be null");
  auto ws = bindings.BindWorkspace(step.workspace_bytes);
  if (!ws.ok()) return ws.status();
  const ResolvedKernel& resolved = step.op->GetResolvedKernel();
  KernelContext ctx{};
  ctx.device_type = step.selector.device_type;
  ctx.stream = bindings.stream();
  ctx.workspace_binding = ws.value();
  ctx.packed_weights = step.packed_weights;
  ctx.attrs = std::span<const std::byte>(resolved.attrs.data(), resolved.attrs.size());
  return step.op->Run(ctx, bindings, index);
}

// ---------------------------------------------------------------- KV cache
Status KVCacheLayout::Validate() const noexcept {
  if (num_layers == 0 || num_kv_heads == 0 || max_tokens == 0 || head_dim == 0)
    return Status::InvalidArgument("KV layout dimensions must be non-zero");
  if (alignment == 0 || (alignment & (alignment - 1)) != 0)
    return Status::InvalidArgument("KV layout alignment must be a non-zero power of two");
  if (kv_dtype.bits == 0 || kv_dtype.lanes == 0) return Status::InvalidArgument("KV layout dtype must be initialized");
  if (head_dim_stride < head_dim) return Status::InvalidArgument("KV head_dim_stride must be >= head_dim");
  return Status::Ok();
}

StatusOr<size_t> KVCacheLayout::Offset(size_t layer, size_t head, size_t pos, size_t dim) const noexcept {
  AM_RETURN_IF_ERROR(Validate());
  if (layer >= num_layers) return Status::OutOfRange("layer index out of range");
  if (head >= num_kv_heads) return Status::OutOfRange("kv_head index out of range");
  if (pos >= max_tokens) return Status::OutOfRange("seq_pos index out of range");
  if (dim >= head_dim) return Status::OutOfRange("dim index out of range");
  size_t off = 0, t = 0;
  if (CheckOverflowMul(layer, layer_stride, &off)) return Status::Overflow("KV layer offset overflowed size_t");
  if (CheckOverflowMul(head, head_stride, &t) || CheckOverflowAdd(off, t, &off))
    return Status::Overflow("KV head offset overflowed size_t");
  if (CheckOverflowMul(pos, token_stride, &t) || CheckOverflowAdd(off, t, &off))
    return Status::Overflow("KV token offset overflowed size_t");
  if (CheckOverflowMul(dim, ElementBytes(), &t) || CheckOverflowAdd(off, t, &off))
    return Status::Overflow("KV dim offset overflowed size_t");
  return off;
}

StatusOr<size_t> KVCacheLayout::BytesPerPlane() const noexcept {
  AM_RETURN_IF_ERROR(Validate());
  size_t b = 0;
  if (CheckOverflowMul(num_layers, layer_stride, &b)) return Status::Overflow("KV bytes-per-plane overflowed size_t");
  return b;
}

bool KVCacheView::valid() const noexcept {
  return layout_ && storage_ && storage_->is_initialized() && slot_ && slot_->in_use && slot_->generation == generation_;
}

Status KVCacheView::ValidateBase() const noexcept {
  if (!layout_ || !storage_ || !slot_) return Status::FailedPrecondition("KVCacheView is not bound to manager-owned state");
  if (!storage_->is_initialized()) return Status::FailedPrecondition("KVCacheView storage is not initialized");
  if (!(slot_->in_use && slot_->generation == generation_))
    return Status::FailedPrecondition("KVCacheView is stale or released");
  return layout_->Validate();
}

Status KVCacheView::ValidateWrite(size_t layer, size_t head, size_t pos, size_t count) const noexcept {
  AM_RETURN_IF_ERROR(ValidateBase());
  if (layer >= layout_->num_layers) return Status::OutOfRange("layer index out of range");
  if (head >= layout_->num_kv_heads) return Status::OutOfRange("kv_head index out of range");
  if (count == 0) return Status::InvalidArgument("KV write token_count must be non-zero");
  size_t end = 0;
  if (CheckOverflowAdd(pos, count, &end)) return Status::Overflow("KV write range overflowed size_t");
  if (end > slot_->capacity_tokens) return Status::OutOfRange("KV write exceeds reserved session token capacity");
  if (end > layout_->max_tokens) return Status::OutOfRange("KV write exceeds physical KV capacity");
  return Status::Ok();
}

Status KVCacheView::ValidateRead(size_t layer, size_t head, size_t begin, size_t end) const noexcept {
  AM_RETURN_IF_ERROR(ValidateBase());
  if (layer >= layout_->num_layers) return Status::OutOfRange("layer index out of range");
  if (head >= layout_->num_kv_heads) return Status::OutOfRange("kv_head index out of range");
  if (begin > end) return Status::InvalidArgument("KV read seq_begin must be <= seq_end");
  if (end > slot_->current_pos) return Status::OutOfRange("KV read exceeds committed token range");
  return Status::Ok();
}

StatusOr<void*> KVCacheView::KeyPlane(size_t layer) const noexcept {
  AM_RETURN_IF_ERROR(ValidateBase());
  if (layer >= layout_->num_layers) return Status::OutOfRange("layer index out of range");
  return static_cast<void*>(static_cast<std::byte*>(storage_->key) + layer * layout_->layer_stride);
}

StatusOr<void*> KVCacheView::ValuePlane(size_t layer) const noexcept {
  AM_RETURN_IF_ERROR(ValidateBase());
  if (layer >= layout_->num_layers) return Status::OutOfRange("layer index out of range");
  return static_cast<void*>(static_cast<std::byte*>(storage_->value) + layer * layout_->layer_stride);
}

Status KVCacheView::CommitUntil(size_t new_pos) noexcept {
  AM_RETURN_IF_ERROR(ValidateBase());
  if (new_pos < slot_->current_pos) return Status::InvalidArgument("KV commit position cannot move backwards");
  if (new_pos > slot_->capacity_tokens) return Status::OutOfRange("KV commit exceeds reserved session token capacity");
  slot_->current_pos = new_pos;
  return Status::Ok();
}

namespace {
void* HipAlloc(size_t n, void*) {
  void* p = nullptr;
  if (hipMalloc(&p, n == 0 ? 1 : n) != hipSuccess) return nullptr;
  return p;
}
void HipFree(void* p, void*) { (void)hipFree(p); }
void* HostAlloc(size_t n, void*) {
  void* p = nullptr;
  if (posix_memalign(&p, 256, n == 0 ? 1 : n) != 0) return nullptr;
  return p;
}
void HostFree(void* p, void*) { std::free(p); }
}  // namespace

DeviceAllocator HipDeviceAllocator() { return {&HipAlloc, &HipFree, nullptr}; }
DeviceAllocator HostTestAllocator() { return {&HostAlloc, &HostFree, nullptr}; }

KVCacheManager::~KVCacheManager() { FreeStorage(); }

void KVCacheManager::FreeStorage() noexcept {
  if (storage_.key) alloc_.free(storage_.key, alloc_.user);
  if (storage_.value) alloc_.free(storage_.value, alloc_.user);
  storage_ = {};
}

Status KVCacheManager::Init(size_t num_layers, size_t num_kv_heads, size_t max_tokens, size_t head_dim,
                            DataType kv_dtype, size_t alignment) {
  FreeStorage();
  layout_ = {};
  slot_ = {};
  total_bytes_ = 0;
  initialized_ = false;
  layout_.num_layers = num_layers;
  layout_.num_kv_heads = num_kv_heads;
  layout_.max_tokens = max_tokens;
  layout_.head_dim = head_dim;
  layout_.head_dim_stride = head_dim;
  layout_.kv_dtype = kv_dtype;
  layout_.alignment = alignment;
  const size_t eb = layout_.ElementBytes();
  if (eb == 0) return Status::InvalidArgument("KV dtype must have non-zero element bytes");
  if (CheckOverflowMul(layout_.head_dim_stride, eb, &layout_.token_stride) ||
      CheckOverflowMul(layout_.max_tokens, layout_.token_stride, &layout_.head_stride) ||
      CheckOverflowMul(layout_.num_kv_heads, layout_.head_stride, &layout_.layer_stride))
    return Status::Overflow("KV layout stride computation overflowed size_t");
  AM_RETURN_IF_ERROR(layout_.Validate());
  auto bpp = layout_.BytesPerPlane();
  if (!bpp.ok()) return bpp.status();
  size_t total = 0;
  if (CheckOverflowMul(bpp.value(), size_t{2}, &total)) return Status::Overflow("KV total bytes overflowed size_t");
  storage_.key = alloc_.alloc(bpp.value(), alloc_.user);
  storage_.value = alloc_.alloc(bpp.value(), alloc_.user);
  if (!storage_.key || !storage_.value) {
    FreeStorage();
    return Status::ResourceExhausted("Failed to allocate KV cache planes");
  }
  storage_.bytes_per_plane = bpp.value();
  total_bytes_ = total;
  initialized_ = true;
  return Status::Ok();
}

StatusOr<KVCacheView> KVCacheManager::ReserveForSession(size_t prompt_len, size_t max_new_tokens) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KVCacheManager is not initialized");
  if (slot_.in_use) return Status::FailedPrecondition("KVCacheManager already has an active session reservation");
  size_t req = 0;
  if (CheckOverflowAdd(prompt_len, max_new_tokens, &req)) return Status::Overflow("KV session reservation overflowed size_t");
  if (req == 0) return Status::InvalidArgument("KV session reservation must request at least one token");
  if (req > layout_.max_tokens) return Status::OutOfRange("KV session reservation exceeds physical KV capacity");
  ++slot_.generation;
  slot_.in_use = true;
  slot_.capacity_tokens = req;
  slot_.prompt_len = prompt_len;
  slot_.current_pos = prompt_len;
  return KVCacheView(&layout_, &storage_, &slot_);
}

Status KVCacheManager::ResetSession(KVCacheView& view) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KVCacheManager is not initialized");
  if (!view.valid()) return Status::FailedPrecondition("Cannot reset an invalid or stale KVCacheView");
  slot_.current_pos = slot_.prompt_len;
  return Status::Ok();
}

Status KVCacheManager::ReleaseSession(KVCacheView& view) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KVCacheManager is not initialized");
  if (!view.valid()) return Status::FailedPrecondition("Cannot release an invalid or stale KVCacheView");
  slot_ = SessionKVSlot{slot_.generation + 1, false, 0, 0, 0};
  view.Invalidate();
  return Status::Ok();
}

}  // namespace aethermind
