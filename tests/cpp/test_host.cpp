// Host-logic tests of the gfx950 build's C++ runtime contract layer.  No GPU needed:
// nothing here launches a kernel or allocates device memory (the KV manager runs on
// the host allocator hook).  The cases follow the reference's own unit tests:
//   registry resolve      tests/unit/backend/test_kernel_registry_resolve.cpp:36-118
//   KV layout / manager   tests/unit/execution/test_kv_cache_manager.cpp:13-123
//   executor order/errors tests/unit/execution/test_executor_backend_path.cpp:266-368
// Exit code 0 = all checks passed; every failure is printed with its line.
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "am_core.h"
#include "gfx950_backend.h"
#include "packed_cache.h"

using namespace aethermind;

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond)                                                      \
  do {                                                                   \
    ++g_checks;                                                          \
    if (!(cond)) {                                                       \
      ++g_failures;                                                      \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);        \
    }                                                                    \
  } while (0)

Status ScalarKernel(const KernelContext&) noexcept { return Status::Ok(); }
Status Avx2Kernel(const KernelContext&) noexcept { return Status::Ok(); }
Status DecodeOnlyKernel(const KernelContext&) noexcept { return Status::Ok(); }

KernelSelector MakeSelector(ExecPhase phase = ExecPhase::kBoth, IsaLevel isa = IsaLevel::kScalar) {
  KernelSelector s;
  s.device_type = DeviceType::kCPU;
  s.act_dtype = DataType::Float32();
  s.weight_dtype = DataType::Float32();
  s.weight_format = WeightFormat::kPlain;
  s.isa = isa;
  s.phase = phase;
  return s;
}

KernelDescriptor Desc(OpType op, KernelSelector sel, KernelFunc fn, const char* name, int priority) {
  KernelDescriptor d;
  d.op_type = op;
  d.selector = sel;
  d.kernel_func = fn;
  d.name = name;
  d.priority = priority;
  return d;
}

// ---------------------------------------------------------------- registry
void TestRegistry() {
  {  // a kBoth kernel serves a decode request
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kRmsNorm, MakeSelector(ExecPhase::kBoth), &ScalarKernel, "scalar", 1)).ok());
    CHECK(r.Freeze().ok());
    auto d = r.Resolve(OpType::kRmsNorm, MakeSelector(ExecPhase::kDecode));
    CHECK(d.ok() && d.value()->kernel_func == &ScalarKernel);
  }
  {  // ISA-compatible candidates: the higher priority wins
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kRmsNorm, MakeSelector(ExecPhase::kBoth, IsaLevel::kScalar), &ScalarKernel,
                          "scalar", 1)).ok());
    CHECK(r.Register(Desc(OpType::kRmsNorm, MakeSelector(ExecPhase::kBoth, IsaLevel::kAVX2), &Avx2Kernel, "avx2",
                          10)).ok());
    CHECK(r.Freeze().ok());
    auto d = r.Resolve(OpType::kRmsNorm, MakeSelector(ExecPhase::kPrefill, IsaLevel::kAVX512));
    CHECK(d.ok() && d.value()->kernel_func == &Avx2Kernel);
    // a scalar-only request cannot use the AVX2 kernel
    auto s = r.Resolve(OpType::kRmsNorm, MakeSelector(ExecPhase::kPrefill, IsaLevel::kScalar));
    CHECK(s.ok() && s.value()->kernel_func == &ScalarKernel);
  }
  {  // no ISA-compatible candidate -> kNotFound
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kRmsNorm, MakeSelector(ExecPhase::kBoth, IsaLevel::kAVX512), &Avx2Kernel,
                          "avx512-only", 10)).ok());
    CHECK(r.Freeze().ok());
    auto d = r.Resolve(OpType::kRmsNorm, MakeSelector(ExecPhase::kPrefill, IsaLevel::kAVX2));
    CHECK(!d.ok() && d.status().code() == StatusCode::kNotFound);
  }
  {  // a decode-only kernel does not serve prefill
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kRmsNorm, MakeSelector(ExecPhase::kDecode), &DecodeOnlyKernel, "decode-only", 5))
              .ok());
    CHECK(r.Freeze().ok());
    auto d = r.Resolve(OpType::kRmsNorm, MakeSelector(ExecPhase::kPrefill));
    CHECK(!d.ok() && d.status().code() == StatusCode::kNotFound);
  }
  {  // equal priority: the first registration wins
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kAdd, MakeSelector(ExecPhase::kBoth, IsaLevel::kScalar), &ScalarKernel, "first",
                          3)).ok());
    CHECK(r.Register(Desc(OpType::kAdd, MakeSelector(ExecPhase::kBoth, IsaLevel::kAVX2), &Avx2Kernel, "second", 3))
              .ok());
    CHECK(r.Freeze().ok());
    auto d = r.Resolve(OpType::kAdd, MakeSelector(ExecPhase::kDecode, IsaLevel::kAVX2));
    CHECK(d.ok() && d.value()->kernel_func == &ScalarKernel);
  }
  {  // duplicate (op, selector), registration after freeze, idempotent freeze, bad descriptors
    KernelRegistry r;
    CHECK(r.Register(Desc(OpType::kAdd, MakeSelector(), &ScalarKernel, "a", 1)).ok());
    auto dup = r.Register(Desc(OpType::kAdd, MakeSelector(), &Avx2Kernel, "b", 2));
    CHECK(!dup.ok() && dup.code() == StatusCode::kAlreadyExists);
    CHECK(r.Freeze().ok());
    CHECK(r.Freeze().ok());
    auto late = r.Register(Desc(OpType::kSiluMul, MakeSelector(), &ScalarKernel, "late", 1));
    CHECK(!late.ok() && late.code() == StatusCode::kFailedPrecondition);
    CHECK(r.size() == 1);

    KernelRegistry r2;
    auto nofn = r2.Register(Desc(OpType::kAdd, MakeSelector(), nullptr, "null-fn", 1));
    CHECK(!nofn.ok() && nofn.code() == StatusCode::kInvalidArgument);
    KernelDescriptor big = Desc(OpType::kAdd, MakeSelector(), &ScalarKernel, "too-big-params", 1);
    big.params_builder = &gfx950::BuildGfxParams;  // sizes are checked when a builder is set
    big.params_size = kMaxKernelParamsSize + 1;
    auto tb = r2.Register(big);
    CHECK(!tb.ok() && tb.code() == StatusCode::kInvalidArgument);
    big.params_size = 0;
    auto zero = r2.Register(big);
    CHECK(!zero.ok() && zero.code() == StatusCode::kInvalidArgument);
  }
}

// ---------------------------------------------------------------- KV cache
DataType KVType() { return DataType(DLDataTypeCode::kFloat, 16, 1); }

void TestKV() {
  {  // reference KAT: Offset(1,2,3,4) and bytes per plane
    KVCacheLayout l;
    l.num_layers = 2;
    l.num_kv_heads = 3;
    l.max_tokens = 4;
    l.head_dim = 5;
    l.head_dim_stride = 8;
    l.token_stride = 16;
    l.head_stride = 64;
    l.layer_stride = 192;
    l.kv_dtype = KVType();
    l.alignment = 64;
    auto off = l.Offset(1, 2, 3, 4);
    CHECK(off.ok() && off.value() == 192u + 128u + 48u + 8u);
    auto bpp = l.BytesPerPlane();
    CHECK(bpp.ok() && bpp.value() == 384u);
    CHECK(l.Offset(2, 0, 0, 0).status().code() == StatusCode::kOutOfRange);
    CHECK(l.Offset(0, 0, 0, 5).status().code() == StatusCode::kOutOfRange);
  }
  {  // init + reserve gives a valid view
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(2, 4, 32, 16, KVType(), 64).ok());
    auto v = m.ReserveForSession(8, 8);
    CHECK(v.ok());
    if (v.ok()) {
      CHECK(v->valid());
      CHECK(v->num_layers() == 2 && v->num_kv_heads() == 4 && v->head_dim() == 16);
      CHECK(v->max_tokens() == 32 && v->token_capacity() == 16 && v->current_pos() == 8);
    }
    CHECK(m.total_bytes() == 2u * 2 * 4 * 32 * 16 * 2);
    // layer planes are layer_stride apart inside one slab per plane
    auto k0 = v->KeyPlane(0), k1 = v->KeyPlane(1), v0 = v->ValuePlane(0);
    CHECK(k0.ok() && k1.ok() && v0.ok());
    CHECK(static_cast<char*>(k1.value()) - static_cast<char*>(k0.value()) ==
          static_cast<std::ptrdiff_t>(m.layout().layer_stride));
    CHECK(k0.value() != v0.value());
  }
  {  // a second active reservation is refused
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 1, 16, 8, KVType(), 64).ok());
    CHECK(m.ReserveForSession(4, 4).ok());
    auto second = m.ReserveForSession(2, 2);
    CHECK(!second.ok() && second.status().code() == StatusCode::kFailedPrecondition);
  }
  {  // reads only below the committed position, writes only inside the reservation
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 1, 16, 8, KVType(), 64).ok());
    auto v = m.ReserveForSession(4, 4);
    CHECK(v.ok());
    CHECK(v->ValidateRead(0, 0, 0, 4).ok());
    CHECK(v->ValidateRead(0, 0, 0, 5).code() == StatusCode::kOutOfRange);
    CHECK(v->ValidateWrite(0, 0, 4, 4).ok());
    CHECK(v->ValidateWrite(0, 0, 4, 5).code() == StatusCode::kOutOfRange);
    CHECK(v->CommitUntil(5).ok());
    CHECK(v->current_pos() == 5);
    CHECK(v->ValidateRead(0, 0, 0, 5).ok());
    CHECK(v->CommitUntil(4).code() == StatusCode::kInvalidArgument);  // never backwards
    CHECK(v->CommitUntil(9).code() == StatusCode::kOutOfRange);       // beyond the reservation
  }
  {  // reset rewinds to the prompt length
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 1, 32, 8, KVType(), 64).ok());
    auto v = m.ReserveForSession(6, 10);
    CHECK(v.ok());
    CHECK(v->CommitUntil(10).ok());
    CHECK(m.ResetSession(*v).ok());
    CHECK(v->current_pos() == 6);
  }
  {  // release invalidates the view (and every copy of it); a new reservation works
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 2, 24, 8, KVType(), 64).ok());
    auto v = m.ReserveForSession(3, 5);
    CHECK(v.ok());
    KVCacheView stale = v.value();
    CHECK(m.ReleaseSession(*v).ok());
    CHECK(!v->valid());
    CHECK(!stale.valid());
    CHECK(stale.KeyPlane(0).status().code() == StatusCode::kFailedPrecondition);
    auto next = m.ReserveForSession(2, 4);
    CHECK(next.ok() && next->valid() && next->current_pos() == 2);
    CHECK(!stale.valid());  // generation moved on
  }
  {  // reservations beyond the physical capacity
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 1, 8, 8, KVType(), 64).ok());
    auto v = m.ReserveForSession(6, 4);
    CHECK(!v.ok() && v.status().code() == StatusCode::kOutOfRange);
  }
  {  // slot pool: one allocation, slot r's planes a fixed stride after slot 0's
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(2, 2, 40, 8, KVType(), 256, 4).ok());
    CHECK(m.num_slots() == 4 && m.free_slots() == 4);
    const size_t plane = 2u * 2 * 40 * 8 * 2;           // 2560 bytes, padded to 2560
    CHECK(m.storage().slot_bytes == 2 * plane && m.total_bytes() == 4 * 2 * plane);
    std::vector<KVCacheView> vs;
    for (int r = 0; r < 4; ++r) {
      auto v = m.ReserveForSession(3, 5);
      CHECK(v.ok() && v->slot() == static_cast<size_t>(r));
      if (v.ok()) vs.push_back(v.value());
    }
    CHECK(m.free_slots() == 0);
    auto full = m.ReserveForSession(1, 1);
    CHECK(!full.ok() && full.status().code() == StatusCode::kFailedPrecondition);
    CHECK(vs.size() == 4);
    if (vs.size() == 4) {
      const auto base_k = static_cast<char*>(vs[0].KeyPlane(0).value());
      for (int r = 0; r < 4; ++r) {
        CHECK(static_cast<char*>(vs[r].KeyPlane(1).value()) - base_k ==
              static_cast<std::ptrdiff_t>(r * m.storage().slot_bytes + m.layout().layer_stride));
        CHECK(static_cast<char*>(vs[r].ValuePlane(0).value()) - static_cast<char*>(vs[r].KeyPlane(0).value()) ==
              static_cast<std::ptrdiff_t>(plane));
      }
      // slots are independent: commits and releases touch only their own slot
      CHECK(vs[2].CommitUntil(7).ok() && vs[1].current_pos() == 3 && vs[2].current_pos() == 7);
      CHECK(m.ReleaseSession(vs[1]).ok());
      CHECK(!vs[1].valid() && vs[0].valid() && vs[2].valid() && m.free_slots() == 1);
      auto again = m.ReserveSlot(1, 0, 40);
      CHECK(again.ok() && again->slot() == 1 && again->current_pos() == 0);
      auto taken = m.ReserveSlot(2, 0, 1);
      CHECK(!taken.ok() && taken.status().code() == StatusCode::kFailedPrecondition);
      auto bad = m.ReserveSlot(4, 0, 1);
      CHECK(!bad.ok() && bad.status().code() == StatusCode::kOutOfRange);
      // the pool is not rebuilt under active reservations
      CHECK(m.Init(1, 1, 8, 8, KVType(), 64).code() == StatusCode::kFailedPrecondition);
    }
  }
  {  // zero slots, zero dimensions, bad alignment
    KVCacheManager m(HostTestAllocator());
    CHECK(m.Init(1, 1, 8, 8, KVType(), 64, 0).code() == StatusCode::kInvalidArgument);
    CHECK(m.Init(1, 0, 8, 8, KVType(), 64).code() == StatusCode::kInvalidArgument);
    CHECK(m.Init(1, 1, 8, 8, KVType(), 48).code() == StatusCode::kInvalidArgument);
    CHECK(!m.ReserveForSession(1, 1).ok());
  }
}

// ---------------------------------------------------------------- executor
struct Trace {
  std::vector<size_t> order;
};

class FakeOp final : public Operator {
 public:
  FakeOp(Trace* t, size_t id, StatusCode result) : t_(t), id_(id), result_(result) {}
  OpType Type() const noexcept override { return OpType::kAdd; }
  Status Prepare(Backend&, const KernelSelector&) override { return Status::Ok(); }
  Status Run(KernelContext& ctx, const RuntimeBindingContext&, size_t step) const noexcept override {
    t_->order.push_back(id_);
    last_step = step;
    last_ws = ctx.workspace_binding.size;
    if (result_ != StatusCode::kOk) return Status(result_, "fake failure");
    return Status::Ok();
  }
  const ResolvedKernel& GetResolvedKernel() const noexcept override { return rk_; }
  mutable size_t last_step = 0, last_ws = 0;

 private:
  Trace* t_;
  size_t id_;
  StatusCode result_;
  ResolvedKernel rk_{};
};

void TestExecutor() {
  {  // steps run in plan order, each with its index and workspace binding
    Trace t;
    std::vector<ExecutionStep> steps;
    std::vector<std::shared_ptr<FakeOp>> ops;
    for (size_t i = 0; i < 5; ++i) {
      ops.push_back(std::make_shared<FakeOp>(&t, 10 + i, StatusCode::kOk));
      ExecutionStep s;
      s.op = ops.back();
      s.workspace_bytes = 16 * i;
      steps.push_back(s);
    }
    auto plan = ExecutionPlan::Create(std::move(steps));
    CHECK(plan.ok());
    RuntimeBindingContext b;
    std::vector<char> arena(256);
    b.SetWorkspace(arena.data(), arena.size());
    CHECK(Executor::Execute(plan.value(), b).ok());
    CHECK((t.order == std::vector<size_t>{10, 11, 12, 13, 14}));
    CHECK(ops[3]->last_step == 3 && ops[3]->last_ws == 48);
  }
  {  // the first failing step stops the run and its status comes back unchanged
    Trace t;
    std::vector<ExecutionStep> steps;
    for (size_t i = 0; i < 4; ++i) {
      ExecutionStep s;
      s.op = std::make_shared<FakeOp>(&t, i, i == 2 ? StatusCode::kOutOfRange : StatusCode::kOk);
      steps.push_back(s);
    }
    auto plan = ExecutionPlan::Create(std::move(steps));
    CHECK(plan.ok());
    RuntimeBindingContext b;
    auto st = Executor::Execute(plan.value(), b);
    CHECK(!st.ok() && st.code() == StatusCode::kOutOfRange);
    CHECK((t.order == std::vector<size_t>{0, 1, 2}));
  }
  {  // a step asking for more workspace than bound fails before it runs
    Trace t;
    ExecutionStep s;
    s.op = std::make_shared<FakeOp>(&t, 7, StatusCode::kOk);
    s.workspace_bytes = 1024;
    auto plan = ExecutionPlan::Create({s});
    CHECK(plan.ok());
    RuntimeBindingContext b;
    std::vector<char> arena(64);
    b.SetWorkspace(arena.data(), arena.size());
    auto st = Executor::Execute(plan.value(), b);
    CHECK(!st.ok() && st.code() == StatusCode::kResourceExhausted);
    CHECK(t.order.empty());
  }
  {  // a plan step without an operator is rejected
    ExecutionStep s;
    auto plan = ExecutionPlan::Create({s});
    if (plan.ok()) {
      RuntimeBindingContext b;
      CHECK(!Executor::Execute(plan.value(), b).ok());
    } else {
      CHECK(plan.status().code() == StatusCode::kInvalidArgument);
    }
  }
}

// ---------------------------------------------------------------- gfx950 registrations
void TestGfx950Registrations() {
  using gfx950::HipSelector;
  const DataType f32 = DataType::Float32(), bf16 = DataType::BFloat(16), i8 = DataType::Int(8), i4 = DataType::Int(4);
  gfx950::Gfx950Backend backend;  // freezes the global registry (static registrations done)
  const KernelRegistry& reg = KernelRegistry::Global();
  CHECK(reg.frozen());
  struct Case {
    OpType op;
    KernelSelector sel;
    const char* name;
  };
  const Case cases[] = {
      {OpType::kLinear, HipSelector(bf16, i4, WeightFormat::kQuantizedInt4, ExecPhase::kDecode), "gfx950::gemv_bf16_int4"},
      {OpType::kLinear, HipSelector(bf16, i4, WeightFormat::kQuantizedInt4, ExecPhase::kPrefill),
       "gfx950::gemm_mfma_bf16_int4"},
      {OpType::kLinear, HipSelector(bf16, i8, WeightFormat::kQuantizedInt8, ExecPhase::kDecode), "gfx950::gemv_bf16_int8"},
      {OpType::kLinear, HipSelector(f32, f32, WeightFormat::kPlain, ExecPhase::kDecode), "gfx950::gemv_f32_f32"},
      {OpType::kRmsNorm, HipSelector(bf16, bf16, WeightFormat::kPlain, ExecPhase::kDecode), "gfx950::rmsnorm_bf16"},
      {OpType::kAttention, HipSelector(bf16, bf16, WeightFormat::kPlain, ExecPhase::kPrefill),
       "gfx950::gqa_attention_bf16"},
      {OpType::kArgmax, HipSelector(f32, f32, WeightFormat::kPlain, ExecPhase::kDecode), "gfx950::argmax_f32"},
  };
  for (const Case& c : cases) {
    auto d = reg.Resolve(c.op, c.sel);
    CHECK(d.ok());
    if (d.ok()) {
      CHECK(d.value()->name == c.name);
      CHECK(d.value()->params_size <= kMaxKernelParamsSize);
      auto info = backend.ResolveKernelInfo(c.op, c.sel);
      CHECK(info.ok() && info->fn == d.value()->kernel_func);
    }
  }
  // a CPU request never resolves to a gfx950 kernel, and unknown combinations are kNotFound
  KernelSelector cpu = MakeSelector(ExecPhase::kDecode, IsaLevel::kAVX2);
  CHECK(reg.Resolve(OpType::kLinear, cpu).status().code() == StatusCode::kNotFound);
  KernelSelector odd = HipSelector(f32, i4, WeightFormat::kQuantizedInt8, ExecPhase::kDecode);
  CHECK(reg.Resolve(OpType::kLinear, odd).status().code() == StatusCode::kNotFound);
  // registration after the backend froze the registry fails
  auto late = KernelRegistry::Global().Register(
      Desc(OpType::kSoftmax, HipSelector(f32, f32, WeightFormat::kPlain, ExecPhase::kBoth), &ScalarKernel, "late", 1));
  CHECK(!late.ok() && late.code() == StatusCode::kFailedPrecondition);
  // the status codes cross the C ABI unchanged
  CHECK(Status(StatusCode::kOutOfRange, "x").c_code() == AM_STATUS_OUT_OF_RANGE);
  CHECK(Status::FromC(AM_STATUS_NOT_FOUND, "y").code() == StatusCode::kNotFound);
}

}  // namespace

// Packed weight cache header (host/packed_cache.h): round trip, and every corruption
// or foreign file that must be refused before any device memory is touched.
void TestPackedCacheHeader() {
  namespace P = aethermind::packed;
  P::Header h;
  h.payload_bytes = 4096;
  h.payload_checksum = 0x1234;
  h.cfg = am_model_config{2, 64, 4, 2, 16, 128, 100, 1e-5f, 500000.0, AM_DT_BF16, AM_WF_INT4, 32, 0, 0};
  uint8_t buf[P::kHeaderBytes];
  P::EncodeHeader(h, buf);
  {
    auto d = P::DecodeHeader(buf, sizeof(buf));
    CHECK(d.ok());
    if (d.ok()) {
      const auto& c = d.value().cfg;
      CHECK(d.value().payload_bytes == 4096 && d.value().payload_checksum == 0x1234);
      CHECK(c.num_layers == 2 && c.hidden == 64 && c.num_q_heads == 4 && c.num_kv_heads == 2 && c.head_dim == 16 &&
            c.ffn == 128 && c.vocab == 100 && c.rms_eps == 1e-5f && c.rope_theta == 500000.0 &&
            c.act_dtype == AM_DT_BF16 && c.weight_format == AM_WF_INT4 && c.group_size == 32);
    }
  }
  // every single-bit flip of the header is refused
  int refused = 0;
  for (size_t byte = 0; byte < P::kHeaderBytes; ++byte) {
    uint8_t b2[P::kHeaderBytes];
    std::memcpy(b2, buf, sizeof(b2));
    b2[byte] ^= 0x10;
    refused += P::DecodeHeader(b2, sizeof(b2)).ok() ? 0 : 1;
  }
  CHECK(refused == static_cast<int>(P::kHeaderBytes));
  CHECK(P::DecodeHeader(buf, 100).status().code() == StatusCode::kDataLoss);
  {
    uint8_t b2[P::kHeaderBytes];
    std::memcpy(b2, buf, sizeof(b2));
    b2[0] = 'X';
    CHECK(P::DecodeHeader(b2, sizeof(b2)).status().code() == StatusCode::kInvalidArgument);
  }
  auto with_cfg = [&](auto edit) {
    P::Header h2 = h;
    edit(h2);
    uint8_t b2[P::kHeaderBytes];
    P::EncodeHeader(h2, b2);
    return P::DecodeHeader(b2, sizeof(b2)).status();
  };
  CHECK(with_cfg([](P::Header& x) { x.cfg.num_kv_heads = 3; }).code() == StatusCode::kInvalidArgument);
  CHECK(with_cfg([](P::Header& x) { x.cfg.hidden = 0; }).code() == StatusCode::kInvalidArgument);
  CHECK(with_cfg([](P::Header& x) { x.cfg.weight_format = 9; }).code() == StatusCode::kInvalidArgument);
  CHECK(with_cfg([](P::Header& x) { x.cfg.act_dtype = AM_DT_F16; }).code() == StatusCode::kInvalidArgument);
  CHECK(with_cfg([](P::Header& x) { x.cfg.group_size = 0; }).code() == StatusCode::kInvalidArgument);
  CHECK(with_cfg([](P::Header& x) { x.payload_bytes = 1000; }).code() == StatusCode::kDataLoss);
  // the checksum: order- and content-sensitive, and streaming equals one shot
  std::vector<uint8_t> data(1 << 12);
  for (size_t i = 0; i < data.size(); ++i) data[i] = static_cast<uint8_t>(i * 131 + 7);
  const uint64_t c0 = P::Checksum(data.data(), data.size());
  P::PayloadHasher st;
  st.Update(data.data(), 1024);
  st.Update(data.data() + 1024, data.size() - 1024);
  CHECK(st.Finish() == c0);
  std::swap(data[100], data[3000]);
  CHECK(P::Checksum(data.data(), data.size()) != c0);
  // Inspect: whole file, truncated, padded, missing
  const std::string path = "/tmp/am_test_packed_" + std::to_string(::getpid()) + ".bin";
  auto write = [&](size_t payload) {
    FILE* f = std::fopen(path.c_str(), "wb");
    std::fwrite(buf, 1, sizeof(buf), f);
    std::vector<uint8_t> z(payload, 0);
    std::fwrite(z.data(), 1, z.size(), f);
    std::fclose(f);
  };
  write(4096);
  CHECK(P::Inspect(path).ok());
  write(4000);
  CHECK(P::Inspect(path).status().code() == StatusCode::kDataLoss);
  write(4096 + 256);
  CHECK(P::Inspect(path).status().code() == StatusCode::kDataLoss);
  std::remove(path.c_str());
  CHECK(P::Inspect(path).status().code() == StatusCode::kNotFound);
}

// Paged KV block manager (host/am_core.h): growth, exhaustion, release and reuse, the
// table rows, and the pool addresses.
void TestKVBlocks() {
  KVBlockManager m(HostTestAllocator());
  CHECK(m.Init(2, 8, 128, DataType::BFloat(16), 48, 10, 2, 1000).code() == StatusCode::kInvalidArgument);
  CHECK(m.Init(2, 8, 128, DataType::BFloat(16), 64, 10, 3, 1000).ok());
  CHECK(m.table_stride() == 16 && m.free_blocks() == 10 && m.dirty());
  CHECK(m.pool_bytes() == size_t{2} * 2 * 10 * 8 * 64 * 128 * 2);
  CHECK(static_cast<char*>(m.value_pool(0)) - static_cast<char*>(m.key_pool(0)) ==
        static_cast<ptrdiff_t>(10 * 8 * 64 * 128 * 2));
  CHECK(static_cast<char*>(m.key_pool(1)) - static_cast<char*>(m.key_pool(0)) ==
        static_cast<ptrdiff_t>(2 * 10 * 8 * 64 * 128 * 2));
  m.clear_dirty();
  CHECK(m.EnsureCapacity(0, 100).ok());  // 2 blocks: ids 0, 1
  CHECK(m.blocks_of(0) == 2 && m.free_blocks() == 8 && m.dirty());
  CHECK(m.host_table()[0] == 0 && m.host_table()[1] == 1 && m.host_table()[2] == -1);
  m.clear_dirty();
  CHECK(m.EnsureCapacity(0, 128).ok() && !m.dirty());  // still 2 blocks
  CHECK(m.EnsureCapacity(1, 65).ok());                 // ids 2, 3
  CHECK(m.host_table()[16] == 2 && m.host_table()[17] == 3);
  CHECK(m.EnsureCapacity(0, 129).ok() && m.host_table()[2] == 4);
  // exhaustion changes nothing
  CHECK(m.EnsureCapacity(2, 64 * 6).code() == StatusCode::kResourceExhausted);
  CHECK(m.blocks_of(2) == 0 && m.free_blocks() == 5);
  CHECK(m.EnsureCapacity(2, 1001).code() == StatusCode::kOutOfRange);
  CHECK(m.EnsureCapacity(3, 1).code() == StatusCode::kOutOfRange);
  // release returns blocks; the lowest free ids are reused first
  CHECK(m.ReleaseSequence(0).ok());
  CHECK(m.free_blocks() == 8 && m.blocks_of(0) == 0 && m.host_table()[0] == -1);
  CHECK(m.EnsureCapacity(2, 64 * 3).ok());
  CHECK(m.host_table()[32] == 0 && m.host_table()[33] == 1 && m.host_table()[34] == 4);
  CHECK(m.EnsureCapacity(0, 64 * 5).ok() && m.free_blocks() == 0);
  CHECK(m.EnsureCapacity(1, 64 * 3).code() == StatusCode::kResourceExhausted);
}

int main() {
  TestKVBlocks();
  TestPackedCacheHeader();
  TestRegistry();
  TestKV();
  TestExecutor();
  TestGfx950Registrations();
  std::printf("%d checks, %d failures\n", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
