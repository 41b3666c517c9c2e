// Implementation of the host contract layer (see am_core.h for the reference map).

#include "am_core.h"

#include <hip/hip_runtime.h>

#include "am_gfx950.h"
#include "hip_alloc.h"

#include <algorithm>
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
    case OpType::kFusedLinearSplit: return "FusedLinearSplit";
    case OpType::kFusedLinearSiluMul: return "FusedLinearSiluMul";
    case OpType::kFusedLinearRoPEKVUpdate: return "FusedLinearRoPEKVUpdate";
    default: return "Unknown";
  }
}

// ---------------------------------------------------------------- registry
Status ValidateKernelDescriptor(const KernelDescriptor& d) noexcept {
  if (d.op_type == OpType::kUnknown) return Status::InvalidArgument("kernel descriptor: op type is unknown");
  if (d.kernel_func == nullptr) return Status::InvalidArgument("kernel descriptor: no kernel function");
  if (d.name.empty()) return Status::InvalidArgument("kernel descriptor: empty name");
  if (d.selector.device_type == DeviceType::kUndefined)
    return Status::InvalidArgument("kernel descriptor: device type is undefined");
  if (d.params_builder != nullptr && (d.params_size == 0 || d.params_size > kMaxKernelParamsSize))
    return Status::InvalidArgument("kernel descriptor: a params builder needs 0 < params_size <= " +
                                   std::to_string(kMaxKernelParamsSize));
  return Status::Ok();
}

KernelRegistry& KernelRegistry::Global() noexcept {
  static KernelRegistry registry;
  return registry;
}

Status KernelRegistry::Register(const KernelDescriptor& d) {
  std::lock_guard<std::mutex> lock(mutex_);
  if (frozen_.load(std::memory_order_relaxed))
    return Status::FailedPrecondition("kernel table is frozen; '" + d.name + "' registered too late");
  AM_RETURN_IF_ERROR(ValidateKernelDescriptor(d));
  if (static_cast<size_t>(d.op_type) >= kOpSlots)
    return Status::InvalidArgument("kernel descriptor: op type beyond the table's range");
  for (const KernelDescriptor& e : pending_)
    if (e.op_type == d.op_type && e.selector == d.selector)
      return Status::AlreadyExists("kernel '" + d.name + "' repeats the op type and selector of '" + e.name + "'");
  pending_.push_back(d);
  return Status::Ok();
}

Status KernelRegistry::Freeze() {
  std::lock_guard<std::mutex> lock(mutex_);
  if (frozen_.load(std::memory_order_relaxed)) return Status::Ok();
  // order: op type, then priority high to low, then registration order (stable sort)
  std::vector<KernelDescriptor> t = pending_;
  std::stable_sort(t.begin(), t.end(), [](const KernelDescriptor& a, const KernelDescriptor& b) {
    if (a.op_type != b.op_type) return static_cast<uint32_t>(a.op_type) < static_cast<uint32_t>(b.op_type);
    return a.priority > b.priority;
  });
  for (Range& r : ranges_) r = Range{};
  for (uint32_t i = 0; i < t.size();) {
    const size_t op = static_cast<size_t>(t[i].op_type);
    uint32_t j = i;
    while (j < t.size() && static_cast<size_t>(t[j].op_type) == op) ++j;
    ranges_[op] = Range{i, j};
    i = j;
  }
  table_ = std::move(t);
  frozen_.store(true, std::memory_order_release);
  return Status::Ok();
}

StatusOr<const KernelDescriptor*> KernelRegistry::Resolve(OpType op_type, const KernelSelector& selector) const {
  if (!frozen_.load(std::memory_order_acquire))
    return Status::FailedPrecondition("kernel table must be frozen before resolving");
  if (op_type == OpType::kUnknown) return Status::InvalidArgument("resolve: op type is unknown");
  if (selector.device_type == DeviceType::kUndefined) return Status::InvalidArgument("resolve: device type is undefined");
  const size_t op = static_cast<size_t>(op_type);
  if (op < kOpSlots)
    for (uint32_t i = ranges_[op].begin; i < ranges_[op].end; ++i)
      if (SelectorMatches(table_[i].selector, selector)) return &table_[i];
  return Status::NotFound(std::string("no kernel for ") + ToString(op_type) + " matches " + ToString(selector));
}

size_t KernelRegistry::size() const {
  std::lock_guard<std::mutex> lock(mutex_);
  return pending_.size();
}

StatusOr<std::vector<const KernelDescriptor*>> KernelRegistry::FindByOpType(OpType op_type) const {
  if (!frozen_.load(std::memory_order_acquire))
    return Status::FailedPrecondition("kernel table must be frozen before listing kernels");
  std::vector<const KernelDescriptor*> out;
  const size_t op = static_cast<size_t>(op_type);
  if (op < kOpSlots)
    for (uint32_t i = ranges_[op].begin; i < ranges_[op].end; ++i) out.push_back(&table_[i]);
  return out;
}

std::string KernelRegistry::DebugDump() const {
  std::lock_guard<std::mutex> lock(mutex_);
  std::string out;
  for (const KernelDescriptor& d : pending_) {
    if (!out.empty()) out += '\n';
    out += std::string(ToString(d.op_type)) + " | " + d.name + " | " + ToString(d.selector) +
           " | priority=" + std::to_string(d.priority);
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
// Layout arithmetic and checks follow the reference contract (kv_cache_view.cpp:17-75):
// the same strides, the same error codes for a dimension or index out of range and
// for size_t overflow.
Status KVCacheLayout::Validate() const noexcept {
  if (num_layers == 0 || num_kv_heads == 0 || max_tokens == 0 || head_dim == 0)
    return Status::InvalidArgument("KV layout: every dimension must be positive");
  if (alignment == 0 || (alignment & (alignment - 1)) != 0)
    return Status::InvalidArgument("KV layout: alignment must be a power of two");
  if (kv_dtype.bits == 0 || kv_dtype.lanes == 0) return Status::InvalidArgument("KV layout: element type not set");
  if (head_dim_stride < head_dim) return Status::InvalidArgument("KV layout: head_dim_stride below head_dim");
  return Status::Ok();
}

StatusOr<size_t> KVCacheLayout::Offset(size_t layer, size_t head, size_t pos, size_t dim) const noexcept {
  AM_RETURN_IF_ERROR(Validate());
  const size_t index[4] = {layer, head, pos, dim};
  const size_t limit[4] = {num_layers, num_kv_heads, max_tokens, head_dim};
  const size_t stride[4] = {layer_stride, head_stride, token_stride, ElementBytes()};
  static const char* const what[4] = {"layer", "kv head", "position", "dim"};
  size_t off = 0;
  for (int i = 0; i < 4; ++i) {
    if (index[i] >= limit[i]) return Status::OutOfRange(std::string("KV offset: ") + what[i] + " index out of range");
    size_t term = 0;
    if (CheckOverflowMul(index[i], stride[i], &term) || CheckOverflowAdd(off, term, &off))
      return Status::Overflow(std::string("KV offset: ") + what[i] + " term overflows size_t");
  }
  return off;
}

StatusOr<size_t> KVCacheLayout::BytesPerPlane() const noexcept {
  AM_RETURN_IF_ERROR(Validate());
  size_t b = 0;
  if (CheckOverflowMul(num_layers, layer_stride, &b)) return Status::Overflow("KV plane size overflows size_t");
  return b;
}

bool KVCacheView::valid() const noexcept { return CheckLive().ok(); }

Status KVCacheView::CheckLive() const noexcept {
  if (layout_ == nullptr || storage_ == nullptr || slot_ == nullptr)
    return Status::FailedPrecondition("KV view is not bound to a reservation");
  if (!storage_->is_initialized()) return Status::FailedPrecondition("KV view: the pool has no storage");
  if (!slot_->in_use || slot_->generation != generation_)
    return Status::FailedPrecondition("KV view belongs to a released reservation");
  return Status::Ok();
}

Status KVCacheView::ValidateWrite(size_t layer, size_t head, size_t pos, size_t count) const noexcept {
  AM_RETURN_IF_ERROR(CheckLive());
  AM_RETURN_IF_ERROR(layout_->Validate());
  if (layer >= layout_->num_layers || head >= layout_->num_kv_heads)
    return Status::OutOfRange("KV write: layer or kv head out of range");
  if (count == 0) return Status::InvalidArgument("KV write: no tokens");
  size_t end = 0;
  if (CheckOverflowAdd(pos, count, &end)) return Status::Overflow("KV write: end position overflows size_t");
  if (end > slot_->capacity_tokens || end > layout_->max_tokens)
    return Status::OutOfRange("KV write: rows " + std::to_string(pos) + ".." + std::to_string(end) +
                              " fall outside the reservation");
  return Status::Ok();
}

Status KVCacheView::ValidateRead(size_t layer, size_t head, size_t begin, size_t end) const noexcept {
  AM_RETURN_IF_ERROR(CheckLive());
  AM_RETURN_IF_ERROR(layout_->Validate());
  if (layer >= layout_->num_layers || head >= layout_->num_kv_heads)
    return Status::OutOfRange("KV read: layer or kv head out of range");
  if (begin > end) return Status::InvalidArgument("KV read: begin after end");
  if (end > slot_->current_pos)
    return Status::OutOfRange("KV read: position " + std::to_string(end) + " is past the committed " +
                              std::to_string(slot_->current_pos));
  return Status::Ok();
}

StatusOr<void*> KVCacheView::Plane(bool value, size_t layer) const noexcept {
  AM_RETURN_IF_ERROR(CheckLive());
  if (layer >= layout_->num_layers) return Status::OutOfRange("KV plane: layer out of range");
  void* base = value ? storage_->value(slot_->index) : storage_->key(slot_->index);
  return static_cast<void*>(static_cast<std::byte*>(base) + layer * layout_->layer_stride);
}

StatusOr<void*> KVCacheView::KeyPlane(size_t layer) const noexcept { return Plane(false, layer); }
StatusOr<void*> KVCacheView::ValuePlane(size_t layer) const noexcept { return Plane(true, layer); }

Status KVCacheView::CommitUntil(size_t new_pos) noexcept {
  AM_RETURN_IF_ERROR(CheckLive());
  if (new_pos < slot_->current_pos) return Status::InvalidArgument("KV commit: position would move backwards");
  if (new_pos > slot_->capacity_tokens) return Status::OutOfRange("KV commit: position past the reservation");
  slot_->current_pos = new_pos;
  return Status::Ok();
}

namespace {
void* HipAlloc(size_t n, void*) {
  void* p = nullptr;
  if (hip_alloc::DeviceMalloc(&p, n == 0 ? 1 : n) != hipSuccess) return nullptr;
  return p;
}
void HipFree(void* p, void*) { (void)hip_alloc::DeviceFree(p); }
void* HostAlloc(size_t n, void*) {
  void* p = nullptr;
  if (posix_memalign(&p, 256, n == 0 ? 1 : n) != 0) return nullptr;
  return p;
}
void HostFree(void* p, void*) { std::free(p); }
}  // namespace

DeviceAllocator HipDeviceAllocator() { return {&HipAlloc, &HipFree, nullptr}; }
DeviceAllocator HostTestAllocator() { return {&HostAlloc, &HostFree, nullptr}; }

KVCacheManager::~KVCacheManager() { Release(); }

void KVCacheManager::Release() noexcept {
  if (storage_.base != nullptr) alloc_.free(storage_.base, alloc_.user);
  storage_ = {};
  slots_.clear();
  layout_ = {};
  initialized_ = false;
}

size_t KVCacheManager::free_slots() const noexcept {
  size_t n = 0;
  for (const SessionKVSlot& s : slots_) n += s.in_use ? 0 : 1;
  return n;
}

Status KVCacheManager::Init(size_t num_layers, size_t num_kv_heads, size_t max_tokens, size_t head_dim,
                            DataType kv_dtype, size_t alignment, size_t num_slots) {
  for (const SessionKVSlot& s : slots_)
    if (s.in_use) return Status::FailedPrecondition("KV pool: cannot rebuild while a reservation is active");
  Release();
  if (num_slots == 0) return Status::InvalidArgument("KV pool: at least one slot");
  KVCacheLayout l;
  l.num_layers = num_layers;
  l.num_kv_heads = num_kv_heads;
  l.max_tokens = max_tokens;
  l.head_dim = head_dim;
  l.head_dim_stride = head_dim;
  l.kv_dtype = kv_dtype;
  l.alignment = alignment;
  if (l.ElementBytes() == 0) return Status::InvalidArgument("KV pool: element type has no size");
  // strides inside a plane set: dim, then position, then kv head, then layer
  if (CheckOverflowMul(l.head_dim_stride, l.ElementBytes(), &l.token_stride) ||
      CheckOverflowMul(l.max_tokens, l.token_stride, &l.head_stride) ||
      CheckOverflowMul(l.num_kv_heads, l.head_stride, &l.layer_stride))
    return Status::Overflow("KV pool: stride overflows size_t");
  AM_RETURN_IF_ERROR(l.Validate());
  auto plane = l.BytesPerPlane();
  if (!plane.ok()) return plane.status();
  // each plane set starts on an alignment boundary; a slot holds K then V
  size_t padded = 0, slot = 0, total = 0;
  if (CheckOverflowAdd(plane.value(), alignment - 1, &padded)) return Status::Overflow("KV pool: size overflows size_t");
  padded &= ~(alignment - 1);
  if (CheckOverflowMul(padded, size_t{2}, &slot) || CheckOverflowMul(slot, num_slots, &total))
    return Status::Overflow("KV pool: size overflows size_t");
  void* base = alloc_.alloc(total, alloc_.user);
  if (base == nullptr)
    return Status::ResourceExhausted("KV pool: could not allocate " + std::to_string(total) + " bytes");
  layout_ = l;
  storage_ = KVCacheStorage{base, plane.value(), padded, slot, num_slots};
  slots_.assign(num_slots, SessionKVSlot{});
  for (size_t i = 0; i < num_slots; ++i) slots_[i].index = i;
  initialized_ = true;
  return Status::Ok();
}

StatusOr<KVCacheView> KVCacheManager::Take(SessionKVSlot& s, size_t prompt_len, size_t max_new_tokens) noexcept {
  size_t want = 0;
  if (CheckOverflowAdd(prompt_len, max_new_tokens, &want)) return Status::Overflow("KV reserve: size overflows size_t");
  if (want == 0) return Status::InvalidArgument("KV reserve: no tokens requested");
  if (want > layout_.max_tokens)
    return Status::OutOfRange("KV reserve: " + std::to_string(want) + " tokens exceed the " +
                              std::to_string(layout_.max_tokens) + "-token cache");
  ++s.generation;
  s.in_use = true;
  s.capacity_tokens = want;
  s.prompt_len = prompt_len;
  s.current_pos = prompt_len;
  return KVCacheView(&layout_, &storage_, &s);
}

StatusOr<KVCacheView> KVCacheManager::ReserveForSession(size_t prompt_len, size_t max_new_tokens) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KV pool is not initialized");
  for (SessionKVSlot& s : slots_)
    if (!s.in_use) return Take(s, prompt_len, max_new_tokens);
  return Status::FailedPrecondition("KV pool: every slot holds an active reservation");
}

StatusOr<KVCacheView> KVCacheManager::ReserveSlot(size_t slot, size_t prompt_len, size_t max_new_tokens) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KV pool is not initialized");
  if (slot >= slots_.size()) return Status::OutOfRange("KV pool: slot index out of range");
  if (slots_[slot].in_use) return Status::FailedPrecondition("KV pool: the slot already holds a reservation");
  return Take(slots_[slot], prompt_len, max_new_tokens);
}

Status KVCacheManager::ResetSession(KVCacheView& view) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KV pool is not initialized");
  if (!view.valid()) return Status::FailedPrecondition("KV reset: the view is stale or unbound");
  SessionKVSlot& s = slots_[view.slot()];
  s.current_pos = s.prompt_len;
  return Status::Ok();
}

Status KVCacheManager::ReleaseSession(KVCacheView& view) noexcept {
  if (!initialized_) return Status::FailedPrecondition("KV pool is not initialized");
  if (!view.valid()) return Status::FailedPrecondition("KV release: the view is stale or unbound");
  SessionKVSlot& s = slots_[view.slot()];
  ++s.generation;
  s.in_use = false;
  s.capacity_tokens = s.prompt_len = s.current_pos = 0;
  view.Invalidate();
  return Status::Ok();
}

// ------------------------------------------------------------------ KVBlockManager
KVBlockManager::~KVBlockManager() { Release(); }

void KVBlockManager::Release() noexcept {
  if (pools_ != nullptr) alloc_.free(pools_, alloc_.user);
  if (table_dev_ != nullptr) alloc_.free(table_dev_, alloc_.user);
  pools_ = nullptr;
  table_dev_ = nullptr;
  pool_bytes_ = layer_bytes_ = 0;
  free_.clear();
  table_.clear();
  held_.clear();
  dirty_ = false;
}

Status KVBlockManager::Init(size_t num_layers, size_t num_kv_heads, size_t head_dim, DataType kv_dtype,
                            size_t block_size, size_t num_blocks, size_t max_seqs, size_t max_tokens) {
  Release();
  if (block_size < 32 || (block_size & (block_size - 1)) != 0)
    return Status::InvalidArgument("KV blocks: block_size must be a power of two of at least 32");
  if (num_layers == 0 || num_kv_heads == 0 || head_dim == 0 || num_blocks == 0 || max_seqs == 0 || max_tokens == 0)
    return Status::InvalidArgument("KV blocks: layers, heads, head_dim, blocks, sequences and tokens must be non-zero");
  if (num_blocks > static_cast<size_t>(INT32_MAX)) return Status::InvalidArgument("KV blocks: block ids must fit int32");
  const size_t esz = kv_dtype.nbytes();
  if (esz == 0) return Status::InvalidArgument("KV blocks: element type has no size");
  size_t block_bytes = 0, pool = 0;
  if (CheckOverflowMul(num_kv_heads * head_dim, block_size * esz, &block_bytes) ||
      CheckOverflowMul(block_bytes, num_blocks, &pool) || CheckOverflowMul(pool, 2 * num_layers, &pool_bytes_))
    return Status::Overflow("KV blocks: pool size overflows size_t");
  layer_bytes_ = pool * 2;
  block_ = block_size;
  num_blocks_ = num_blocks;
  max_tokens_ = max_tokens;
  stride_ = (max_tokens + block_size - 1) / block_size;
  pools_ = alloc_.alloc(pool_bytes_, alloc_.user);
  table_dev_ = static_cast<int32_t*>(alloc_.alloc(max_seqs * stride_ * sizeof(int32_t), alloc_.user));
  if (pools_ == nullptr || table_dev_ == nullptr) {
    Release();
    return Status::ResourceExhausted("KV blocks: device allocation failed");
  }
  free_.resize(num_blocks);
  for (size_t i = 0; i < num_blocks; ++i) free_[i] = static_cast<int32_t>(num_blocks - 1 - i);  // lowest at back
  table_.assign(max_seqs * stride_, -1);
  held_.assign(max_seqs, 0);
  dirty_ = true;
  return Status::Ok();
}

Status KVBlockManager::EnsureCapacity(size_t seq, size_t n) noexcept {
  if (pools_ == nullptr) return Status::FailedPrecondition("KV blocks: not initialised");
  if (seq >= held_.size()) return Status::OutOfRange("KV blocks: sequence out of range");
  if (n > max_tokens_) return Status::OutOfRange("KV write exceeds reserved session token capacity");
  const size_t need = (n + block_ - 1) / block_;
  if (need <= held_[seq]) return Status::Ok();
  if (need - held_[seq] > free_.size())
    return Status::ResourceExhausted("KV blocks: the pool has " + std::to_string(free_.size()) + " free blocks, " +
                                     std::to_string(need - held_[seq]) + " needed");
  for (size_t b = held_[seq]; b < need; ++b) {
    table_[seq * stride_ + b] = free_.back();
    free_.pop_back();
  }
  held_[seq] = need;
  dirty_ = true;
  return Status::Ok();
}

Status KVBlockManager::ReleaseSequence(size_t seq) noexcept {
  if (pools_ == nullptr) return Status::FailedPrecondition("KV blocks: not initialised");
  if (seq >= held_.size()) return Status::OutOfRange("KV blocks: sequence out of range");
  for (size_t b = held_[seq]; b-- > 0;) {
    int32_t& e = table_[seq * stride_ + b];
    free_.push_back(e);
    e = -1;
  }
  // keep the lowest ids at the back so the next taker gets them first
  std::sort(free_.begin(), free_.end(), std::greater<int32_t>());
  held_[seq] = 0;
  dirty_ = true;
  return Status::Ok();
}

void* KVBlockManager::key_pool(size_t layer) const noexcept {
  return pools_ == nullptr ? nullptr : static_cast<std::byte*>(pools_) + layer * layer_bytes_;
}
void* KVBlockManager::value_pool(size_t layer) const noexcept {
  return pools_ == nullptr ? nullptr : static_cast<std::byte*>(pools_) + layer * layer_bytes_ + layer_bytes_ / 2;
}

}  // namespace aethermind
