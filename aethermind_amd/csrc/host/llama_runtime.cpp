// Llama-dense prefill/decode runtime on one GPU.
//
// * LlamaModel   = ModelInstance + BackendSidecar of the reference
//   (model_instance.h:10-32, backend_sidecar.h:14-32) for the device: weights are
//   generated/repacked straight into one HBM slab, with a per-weight identity
//   (layer, role) instead of the reference's (op, selector) dedup
//   (weight_prepack_planner.cpp:79-90).
// * Plans follow the per-layer node order of ModelGraphBuilder::BuildLlamaDense
//   (model_graph_builder.cpp:133-290, 356-415).  Every step is a DeviceOperator
//   resolved through the KernelRegistry at plan-build time (no hot-path lookups,
//   test_no_hotpath_resolve.cpp), executed by LayerRunner on the session's HIP stream.
//   The fused decode plan is the same node sequence after the gfx950 fusion pass:
//     RmsNorm+Linear q/k/v+RoPE+KVCacheUpdate -> one kernel,
//     Linear o + Add, Linear down + Add        -> GEMV with residual epilogue,
//     RmsNorm+Linear gate/up+SiluMul           -> one kernel,
//     RmsNorm+Linear lm_head+Argmax            -> one kernel.
// * Session = PrepareSession/Prefill/DecodeStep of executor_design.md:226-256: the
//   KV cache is reserved through KVCacheManager, decode state (token, position, step,
//   token history) lives in device memory, and the decode plan is captured once as a
//   HIP graph and replayed per token without host synchronisation.

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <cstddef>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

#include "am_core.h"
#include "am_runtime.h"
#include "gfx950_backend.h"
#include "am_launch_timing.h"
#include "hf_checkpoint.h"
#include "hip_alloc.h"
#include "packed_cache.h"

namespace am {
am_status_code SetLastError(am_status_code code, const char* msg);
int DeviceCUs();
}  // namespace am

namespace aethermind::llama {

using gfx950::DeviceOperator;
using gfx950::HipSelector;
using gfx950::PackAttrs;

#define AM_HIP_OK(expr)                                                              \
  do {                                                                               \
    hipError_t e_ = (expr);                                                          \
    if (e_ != hipSuccess) return Status::Internal(std::string(#expr) + ": " + hipGetErrorString(e_)); \
  } while (0)

#define AM_C_OK(expr)                                                        \
  do {                                                                       \
    am_status_code c_ = (expr);                                              \
    if (c_ != AM_STATUS_OK) return Status::FromC(c_, am_last_error_message()); \
  } while (0)

namespace {

constexpr uint64_t kEmbedId = 0x01;
constexpr uint64_t kLmHeadId = 0x02;
enum SynthRole : uint64_t { kRQ = 1, kRK, kRV, kRO, kRGate, kRUp, kRDown };
uint64_t LayerTensorId(int layer, SynthRole r) { return (static_cast<uint64_t>(layer + 1) << 8) | r; }

DataType ActType(int32_t dt) { return dt == AM_DT_BF16 ? DataType::BFloat(16) : DataType::Float32(); }
size_t ActBytes(int32_t dt) { return dt == AM_DT_BF16 ? 2 : 4; }

DataType WeightDType(int32_t fmt) {
  switch (fmt) {
    case AM_WF_F32: return DataType::Float32();
    case AM_WF_BF16: return DataType::BFloat(16);
    case AM_WF_INT8: return DataType::Int(8);
    default: return DataType::Int(4);
  }
}
WeightFormat SelFormat(int32_t fmt) {
  return fmt == AM_WF_INT8 ? WeightFormat::kQuantizedInt8
                           : (fmt == AM_WF_INT4 ? WeightFormat::kQuantizedInt4 : WeightFormat::kPlain);
}

struct Slab {
  void* base = nullptr;
  size_t size = 0, off = 0;
  void* Take(size_t bytes) {
    off = (off + 255) & ~size_t{255};
    void* p = static_cast<char*>(base) + off;
    off += bytes;
    return p;
  }
};

}  // namespace

class LlamaModel {
 public:
  am_model_config cfg{};
  hipStream_t stream = nullptr;
  Slab slab;
  void* embed = nullptr;
  std::vector<void*> in_norm, post_norm;
  void* final_norm = nullptr;
  std::vector<am_gfx950_weight> qkv, o, gate_up, down;
  am_gfx950_weight lm_head{};
  float* cos_tab = nullptr;
  float* sin_tab = nullptr;
  int64_t linear_bytes = 0;

  ~LlamaModel() {
    if (slab.base) (void)hip_alloc::DeviceFree(slab.base);
  }

  int64_t KvRows() const { return static_cast<int64_t>(cfg.num_kv_heads) * cfg.head_dim; }
  int64_t QRows() const { return static_cast<int64_t>(cfg.num_q_heads) * cfg.head_dim; }

  am_gfx950_weight RowView(const am_gfx950_weight& w, int64_t row0, int64_t rows) const {
    am_gfx950_weight v = w;
    int64_t rb = 0;
    switch (w.format) {
      case AM_WF_F32: rb = w.k * 4; break;
      case AM_WF_BF16: rb = w.k * 2; break;
      case AM_WF_INT8: rb = w.k; break;
      default: rb = w.k / 2; break;
    }
    v.data = static_cast<const char*>(w.data) + row0 * rb;
    if (w.format == AM_WF_INT8) v.scales = static_cast<const float*>(w.scales) + row0;
    if (w.format == AM_WF_INT4) v.scales = static_cast<const uint16_t*>(w.scales) + row0 * (w.k / w.group_size);
    v.n = rows;
    return v;
  }

  Status Validate() const {
    const auto& c = cfg;
    if (c.num_layers <= 0 || c.hidden <= 0 || c.num_q_heads <= 0 || c.num_kv_heads <= 0 || c.head_dim <= 0 ||
        c.ffn <= 0 || c.vocab <= 0)
      return Status::InvalidArgument("model config dimensions must be positive");
    if (c.num_q_heads % c.num_kv_heads != 0)
      return Status::InvalidArgument("num_attention_heads must be divisible by num_key_value_heads");
    if (c.act_dtype != AM_DT_F32 && c.act_dtype != AM_DT_BF16)
      return Status::InvalidArgument("act_dtype must be f32 or bf16");
    if (c.weight_format < AM_WF_F32 || c.weight_format > AM_WF_INT4) return Status::InvalidArgument("bad weight format");
    if (c.max_tokens <= 0 || c.max_prefill_chunk <= 0) return Status::InvalidArgument("max_tokens/max_prefill_chunk");
    if (!(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0)) return Status::InvalidArgument("eps/theta must be positive");
    if (c.weight_format == AM_WF_INT4 && (c.group_size <= 0 || c.hidden % c.group_size || c.ffn % c.group_size ||
                                          (c.num_q_heads * c.head_dim) % c.group_size))
      return Status::InvalidArgument("INT4 needs hidden/ffn/q width divisible by group_size");
    return Status::Ok();
  }

  static int64_t WBytes(int64_t n, int64_t k, int32_t fmt, int32_t g) {
    int64_t d = 0, s = 0;
    (void)am_gfx950_weight_bytes(n, k, fmt, g, &d, &s);
    return ((d + 255) & ~int64_t{255}) + ((s + 255) & ~int64_t{255});
  }

  Status AllocWeight(int64_t n, int64_t k, am_gfx950_weight* w) {
    int64_t d = 0, s = 0;
    AM_C_OK(am_gfx950_weight_bytes(n, k, cfg.weight_format, cfg.group_size, &d, &s));
    w->n = n;
    w->k = k;
    w->format = cfg.weight_format;
    w->group_size = cfg.group_size;
    w->data = slab.Take(static_cast<size_t>(d));
    w->scales = s > 0 ? slab.Take(static_cast<size_t>(s)) : nullptr;
    linear_bytes += d + s;
    return Status::Ok();
  }

  // Synthesize the logical weight (build SPEC stream of (seed, tensor_id)) into
  // scratch, then pack/quantize it into rows [row_off, row_off + rows) of dst.
  Status SynthInto(uint64_t seed, uint64_t tid, int64_t rows, int64_t k, void* scratch, const am_gfx950_weight& dst,
                   int64_t row_off) {
    const int32_t sdt = cfg.weight_format == AM_WF_F32 ? AM_DT_F32 : AM_DT_BF16;
    am_gfx950_synth_args sa{seed, tid, 0.02, 0, rows * k, scratch, sdt};
    AM_C_OK(am_gfx950_synth_normal(&sa, stream));
    am_gfx950_quantize_args qa{};
    qa.src = scratch;
    qa.src_dtype = sdt;
    qa.src_rows = rows;
    qa.dst = dst;
    qa.dst_row_offset = row_off;
    qa.dst_row_stride = 1;
    if (cfg.weight_format >= AM_WF_INT8)
      AM_C_OK(am_gfx950_quantize(&qa, stream));
    else
      AM_C_OK(am_gfx950_pack_plain(&qa, stream));
    return Status::Ok();
  }

  // One device slab for every weight of the model (layout in the file header).
  Status Allocate() {
    AM_RETURN_IF_ERROR(Validate());
    const auto& c = cfg;
    const int64_t H = c.hidden, F = c.ffn, V = c.vocab, L = c.num_layers, d = c.head_dim;
    const int64_t qkv_rows = QRows() + 2 * KvRows();
    const int32_t fmt = c.weight_format, g = c.group_size;
    const size_t ab = ActBytes(c.act_dtype);
    int64_t total = 0;
    total += V * H * static_cast<int64_t>(ab) + 256;
    total += (2 * L + 1) * (H * static_cast<int64_t>(ab) + 256);
    total += L * (WBytes(qkv_rows, H, fmt, g) + WBytes(H, QRows(), fmt, g) + WBytes(2 * F, H, fmt, g) +
                  WBytes(H, F, fmt, g));
    total += WBytes(V, H, fmt, g);
    total += 2 * (static_cast<int64_t>(c.max_tokens) * (d / 2) * 4 + 256);
    total += 4096;
    AM_HIP_OK(hip_alloc::DeviceMalloc(&slab.base, static_cast<size_t>(total)));
    slab.size = static_cast<size_t>(total);

    embed = slab.Take(static_cast<size_t>(V * H) * ab);
    in_norm.resize(static_cast<size_t>(L));
    post_norm.resize(static_cast<size_t>(L));
    qkv.resize(static_cast<size_t>(L));
    o.resize(static_cast<size_t>(L));
    gate_up.resize(static_cast<size_t>(L));
    down.resize(static_cast<size_t>(L));
    for (int64_t l = 0; l < L; ++l) {
      in_norm[l] = slab.Take(static_cast<size_t>(H) * ab);
      post_norm[l] = slab.Take(static_cast<size_t>(H) * ab);
      AM_RETURN_IF_ERROR(AllocWeight(qkv_rows, H, &qkv[l]));
      AM_RETURN_IF_ERROR(AllocWeight(H, QRows(), &o[l]));
      AM_RETURN_IF_ERROR(AllocWeight(2 * F, H, &gate_up[l]));
      AM_RETURN_IF_ERROR(AllocWeight(H, F, &down[l]));
    }
    final_norm = slab.Take(static_cast<size_t>(H) * ab);
    AM_RETURN_IF_ERROR(AllocWeight(V, H, &lm_head));
    cos_tab = static_cast<float*>(slab.Take(static_cast<size_t>(c.max_tokens) * (d / 2) * 4));
    sin_tab = static_cast<float*>(slab.Take(static_cast<size_t>(c.max_tokens) * (d / 2) * 4));
    if (slab.off > slab.size) return Status::Internal("weight slab overflow");
    return Status::Ok();
  }

  Status FillRope() {
    const auto& c = cfg;
    const int64_t d = c.head_dim;
    std::vector<float> ct(static_cast<size_t>(c.max_tokens) * (d / 2)), stb(ct.size());
    AM_C_OK(am_gfx950_rope_table(c.max_tokens, d, c.rope_theta, ct.data(), stb.data()));
    AM_HIP_OK(hipMemcpyAsync(cos_tab, ct.data(), ct.size() * 4, hipMemcpyHostToDevice, stream));
    AM_HIP_OK(hipMemcpyAsync(sin_tab, stb.data(), stb.size() * 4, hipMemcpyHostToDevice, stream));
    AM_HIP_OK(hipStreamSynchronize(stream));
    return Status::Ok();
  }

  Status CreateSynthetic(uint64_t seed) {
    AM_RETURN_IF_ERROR(Allocate());
    const auto& c = cfg;
    const int64_t H = c.hidden, F = c.ffn, V = c.vocab, L = c.num_layers;
    // scratch for one logical source matrix (largest: lm_head / embedding)
    const int64_t max_elems = std::max({V * H, F * H, QRows() * H});
    void* scratch = nullptr;
    AM_HIP_OK(hip_alloc::DeviceMalloc(&scratch, static_cast<size_t>(max_elems) * 4));
    Status st = [&]() -> Status {
      am_gfx950_synth_args ea{seed, kEmbedId, 0.02, 0, V * H, embed, c.act_dtype};
      AM_C_OK(am_gfx950_synth_normal(&ea, stream));
      for (int64_t l = 0; l < L; ++l) {
        const int li = static_cast<int>(l);
        AM_C_OK(am_gfx950_fill(in_norm[l], c.act_dtype, H, 1.0f, stream));
        AM_C_OK(am_gfx950_fill(post_norm[l], c.act_dtype, H, 1.0f, stream));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRQ), QRows(), H, scratch, qkv[l], 0));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRK), KvRows(), H, scratch, qkv[l], QRows()));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRV), KvRows(), H, scratch, qkv[l], QRows() + KvRows()));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRO), H, QRows(), scratch, o[l], 0));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRGate), F, H, scratch, gate_up[l], 0));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRUp), F, H, scratch, gate_up[l], F));
        AM_RETURN_IF_ERROR(SynthInto(seed, LayerTensorId(li, kRDown), H, F, scratch, down[l], 0));
      }
      AM_C_OK(am_gfx950_fill(final_norm, c.act_dtype, H, 1.0f, stream));
      AM_RETURN_IF_ERROR(SynthInto(seed, kLmHeadId, V, H, scratch, lm_head, 0));
      return FillRope();
    }();
    (void)hip_alloc::DeviceFree(scratch);
    return st;
  }

  // Streams a Hugging Face checkpoint into the slab: each tensor goes from the
  // memory-mapped shard through a pinned two-buffer ring (host copy of one buffer
  // overlaps the DMA of the other) into a device staging area, then is converted,
  // quantized and placed by the repack kernels (q|k|v concatenated, gate|up stacked,
  // norms and embedding in the activation dtype).
  Status LoadCheckpoint(const hf::Checkpoint& ck) {
    AM_RETURN_IF_ERROR(Allocate());
    const auto& c = cfg;
    const int64_t H = c.hidden, F = c.ffn, V = c.vocab, L = c.num_layers;
    const int32_t act_fmt = c.act_dtype == AM_DT_BF16 ? AM_WF_BF16 : AM_WF_F32;
    auto align = [](uint64_t b) { return (b + 255) & ~uint64_t{255}; };
    // The staging area holds any one tensor of the checkpoint, or the four tensors of
    // a GPTQ projection back to back; GPTQ projections also need an unpack area
    // (fp32 [n][k], or the logical INT4 bytes + fp16 scales).
    const uint32_t zero_offset = static_cast<uint32_t>(ck.config().gptq.zero_offset);
    uint64_t max_bytes = ck.max_tensor_bytes(), unpack_bytes = 0;
    for (int64_t l = 0; l < L && ck.has_gptq(); ++l)
      for (const char* p : {".self_attn.q_proj", ".self_attn.k_proj", ".self_attn.v_proj", ".self_attn.o_proj",
                            ".mlp.gate_proj", ".mlp.up_proj", ".mlp.down_proj"})
        if (const hf::GptqLinear* g = ck.Gptq(hf::LayerName(l, p))) {
          uint64_t b = 0;
          for (const hf::TensorView* v : {g->qweight, g->qzeros, g->scales, g->g_idx})
            if (v) b += align(v->bytes);
          max_bytes = std::max(max_bytes, b);
          unpack_bytes = std::max<uint64_t>(unpack_bytes, static_cast<uint64_t>(g->n * g->k) * 4);
        }
    constexpr size_t kRing = size_t{32} << 20;
    void* dsrc = nullptr;
    void* dunpack = nullptr;
    void* pinned[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    Status st = [&]() -> Status {
      AM_HIP_OK(hip_alloc::DeviceMalloc(&dsrc, static_cast<size_t>(max_bytes)));
      if (unpack_bytes > 0) AM_HIP_OK(hip_alloc::DeviceMalloc(&dunpack, static_cast<size_t>(unpack_bytes)));
      for (int i = 0; i < 2; ++i) {
        AM_HIP_OK(hip_alloc::PinnedMalloc(&pinned[i], kRing));
        AM_HIP_OK(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
      }
      int slot = 0;
      // tensor -> staging bytes [at, at + t.bytes)
      auto upload = [&](const hf::TensorView& t, uint64_t at) -> Status {
        if (at + t.bytes > max_bytes) return Status::Internal("tensor " + t.name + " exceeds the device staging area");
        for (uint64_t off = 0; off < t.bytes;) {
          const size_t n = static_cast<size_t>(std::min<uint64_t>(kRing, t.bytes - off));
          if (pending[slot]) AM_HIP_OK(hipEventSynchronize(ev[slot]));
          std::memcpy(pinned[slot], t.data + off, n);
          AM_HIP_OK(hipMemcpyAsync(static_cast<char*>(dsrc) + at + off, pinned[slot], n, hipMemcpyHostToDevice,
                                   stream));
          AM_HIP_OK(hipEventRecord(ev[slot], stream));
          pending[slot] = true;
          off += n;
          slot ^= 1;
        }
        return Status::Ok();
      };
      auto src_dtype = [](hf::StDType d) {
        return d == hf::StDType::kF32 ? AM_DT_F32 : d == hf::StDType::kF16 ? AM_DT_F16 : AM_DT_BF16;
      };
      // a float source matrix on the device -> rows [row_off, row_off + rows) of dst
      auto convert = [&](const void* src, int32_t sdt, int64_t rows, const am_gfx950_weight& dst,
                         int64_t row_off) -> Status {
        am_gfx950_quantize_args qa{};
        qa.src = src;
        qa.src_dtype = sdt;
        qa.src_rows = rows;
        qa.dst = dst;
        qa.dst_row_offset = row_off;
        qa.dst_row_stride = 1;
        if (dst.format >= AM_WF_INT8)
          AM_C_OK(am_gfx950_quantize(&qa, stream));
        else
          AM_C_OK(am_gfx950_pack_plain(&qa, stream));
        return Status::Ok();
      };
      // tensor -> rows [row_off, row_off + rows) of dst (the stream orders the next
      // upload after the kernel that reads the staging area)
      auto place = [&](const hf::TensorView& t, int64_t rows, const am_gfx950_weight& dst, int64_t row_off) -> Status {
        AM_RETURN_IF_ERROR(upload(t, 0));
        return convert(dsrc, src_dtype(t.dtype), rows, dst, row_off);
      };
      // A GPTQ projection -> rows [row_off, row_off + n) of dst.  When dst is INT4 with
      // the checkpoint's group size, F16 scales, in-order groups and every zero 8, the
      // GPTQ grid is this library's (q - 8 with the same fp16 scale), so the nibbles and
      // scales are repacked as they are.  Otherwise the weight is dequantized exactly to
      // fp32 (s * (q - z)) and converted like a dense fp32 tensor.
      auto place_gptq = [&](const hf::GptqLinear& g, const am_gfx950_weight& dst, int64_t row_off) -> Status {
        uint64_t at[4] = {0, 0, 0, 0}, cur = 0;
        const hf::TensorView* parts[4] = {g.qweight, g.qzeros, g.scales, g.g_idx};
        for (int i = 0; i < 4; ++i) {
          if (!parts[i]) continue;
          at[i] = cur;
          AM_RETURN_IF_ERROR(upload(*parts[i], cur));
          cur += align(parts[i]->bytes);
        }
        bool exact = dst.format == AM_WF_INT4 && dst.group_size == g.group && g.scales->dtype == hf::StDType::kF16;
        if (exact && g.g_idx) {
          const int32_t* gi = reinterpret_cast<const int32_t*>(g.g_idx->data);
          for (int64_t i = 0; i < g.k && exact; ++i) exact = gi[i] == i / g.group;
        }
        if (exact) {
          const uint32_t* zw = reinterpret_cast<const uint32_t*>(g.qzeros->data);
          const int64_t words = g.groups * (g.n / 8);
          for (int64_t i = 0; i < words && exact; ++i)
            for (int t = 0; t < 8 && exact; ++t) exact = (((zw[i] >> (4 * t)) + zero_offset) & 15u) == 8u;
        }
        char* base = static_cast<char*>(dsrc);
        am_gfx950_gptq_args a{};
        a.qweight = reinterpret_cast<const int32_t*>(base + at[0]);
        a.qzeros = reinterpret_cast<const int32_t*>(base + at[1]);
        a.scales = base + at[2];
        a.scales_dtype = src_dtype(g.scales->dtype);
        a.zero_offset = static_cast<int32_t>(zero_offset);
        a.g_idx = g.g_idx ? reinterpret_cast<const int32_t*>(base + at[3]) : nullptr;
        a.n = g.n;
        a.k = g.k;
        a.group_size = g.group;
        if (exact) {
          a.out_logical = static_cast<uint8_t*>(dunpack);
          a.out_scales = reinterpret_cast<uint16_t*>(static_cast<char*>(dunpack) + align(g.n * g.k / 2));
          AM_C_OK(am_gfx950_gptq_unpack(&a, stream));
          const am_gfx950_pack_int4_args pa{a.out_logical, a.out_scales, RowView(dst, row_off, g.n)};
          AM_C_OK(am_gfx950_pack_int4(&pa, stream));
          return Status::Ok();
        }
        a.out_f32 = static_cast<float*>(dunpack);
        AM_C_OK(am_gfx950_gptq_unpack(&a, stream));
        return convert(dunpack, AM_DT_F32, g.n, dst, row_off);
      };
      auto proj = [&](int64_t l, const char* name, int64_t rows, const am_gfx950_weight& dst, int64_t row_off) {
        const std::string prefix = hf::LayerName(l, name);
        if (const hf::GptqLinear* g = ck.Gptq(prefix)) return place_gptq(*g, dst, row_off);
        return place(ck.Get(prefix + ".weight"), rows, dst, row_off);
      };
      auto act = [&](void* p, int64_t rows) { return am_gfx950_weight{p, nullptr, rows, H, act_fmt, 0}; };
      auto get = [&](int64_t l, const char* sfx) -> const hf::TensorView& { return ck.Get(hf::LayerName(l, sfx)); };
      AM_RETURN_IF_ERROR(place(ck.Get("model.embed_tokens.weight"), V, act(embed, V), 0));
      for (int64_t l = 0; l < L; ++l) {
        AM_RETURN_IF_ERROR(place(get(l, ".input_layernorm.weight"), 1, act(in_norm[l], 1), 0));
        AM_RETURN_IF_ERROR(place(get(l, ".post_attention_layernorm.weight"), 1, act(post_norm[l], 1), 0));
        AM_RETURN_IF_ERROR(proj(l, ".self_attn.q_proj", QRows(), qkv[l], 0));
        AM_RETURN_IF_ERROR(proj(l, ".self_attn.k_proj", KvRows(), qkv[l], QRows()));
        AM_RETURN_IF_ERROR(proj(l, ".self_attn.v_proj", KvRows(), qkv[l], QRows() + KvRows()));
        AM_RETURN_IF_ERROR(proj(l, ".self_attn.o_proj", H, o[l], 0));
        AM_RETURN_IF_ERROR(proj(l, ".mlp.gate_proj", F, gate_up[l], 0));
        AM_RETURN_IF_ERROR(proj(l, ".mlp.up_proj", F, gate_up[l], F));
        AM_RETURN_IF_ERROR(proj(l, ".mlp.down_proj", H, down[l], 0));
      }
      AM_RETURN_IF_ERROR(place(ck.Get("model.norm.weight"), 1, act(final_norm, 1), 0));
      AM_RETURN_IF_ERROR(place(ck.LmHead(), V, lm_head, 0));
      return FillRope();  // synchronises the stream
    }();
    (void)hipStreamSynchronize(stream);
    for (int i = 0; i < 2; ++i) {
      if (ev[i]) (void)hipEventDestroy(ev[i]);
      if (pinned[i]) (void)hip_alloc::PinnedFree(pinned[i]);
    }
    if (dsrc) (void)hip_alloc::DeviceFree(dsrc);
    if (dunpack) (void)hip_alloc::DeviceFree(dunpack);
    return st;
  }

  // Slab bytes that hold weights: everything before the RoPE tables (which depend on
  // max_tokens and are recomputed at load).
  uint64_t WeightRegionBytes() const {
    return static_cast<uint64_t>(reinterpret_cast<const char*>(cos_tab) - static_cast<const char*>(slab.base));
  }

  // Pinned two-buffer ring for the cache file: chunk i of the weight region goes
  // through buffer i % 2, so the DMA of one buffer overlaps the file I/O of the other.
  struct Ring {
    static constexpr size_t kChunk = size_t{32} << 20;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    Status Init() {
      for (int i = 0; i < 2; ++i) {
        AM_HIP_OK(hip_alloc::PinnedMalloc(&buf[i], kChunk));
        AM_HIP_OK(hipEventCreateWithFlags(&ev[i], hipEventDisableTiming));
      }
      return Status::Ok();
    }
    ~Ring() {
      for (int i = 0; i < 2; ++i) {
        if (ev[i]) (void)hipEventSynchronize(ev[i]), (void)hipEventDestroy(ev[i]);
        if (buf[i]) (void)hip_alloc::PinnedFree(buf[i]);
      }
    }
  };

  // Writes the weight region to path (through path + ".tmp", renamed when complete).
  Status SavePackedCache(const std::string& path) {
    const uint64_t payload = WeightRegionBytes();
    const std::string tmp = path + ".tmp";
    const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd < 0) return Status::InvalidArgument("packed cache: cannot create " + tmp + ": " + std::strerror(errno));
    Ring ring;
    packed::PayloadHasher hasher;
    Status st = [&]() -> Status {
      AM_RETURN_IF_ERROR(ring.Init());
      AM_HIP_OK(hipStreamSynchronize(stream));
      const uint64_t n_chunks = (payload + Ring::kChunk - 1) / Ring::kChunk;
      auto issue = [&](uint64_t i) -> Status {
        const uint64_t off = i * Ring::kChunk, n = std::min<uint64_t>(Ring::kChunk, payload - off);
        AM_HIP_OK(hipMemcpyAsync(ring.buf[i & 1], static_cast<const char*>(slab.base) + off, n, hipMemcpyDeviceToHost,
                                 stream));
        AM_HIP_OK(hipEventRecord(ring.ev[i & 1], stream));
        return Status::Ok();
      };
      AM_RETURN_IF_ERROR(issue(0));
      for (uint64_t i = 0; i < n_chunks; ++i) {
        if (i + 1 < n_chunks) AM_RETURN_IF_ERROR(issue(i + 1));
        AM_HIP_OK(hipEventSynchronize(ring.ev[i & 1]));
        const uint64_t off = i * Ring::kChunk, n = std::min<uint64_t>(Ring::kChunk, payload - off);
        hasher.Update(ring.buf[i & 1], n);
        for (uint64_t done = 0; done < n;) {
          const ssize_t w = ::pwrite(fd, static_cast<const char*>(ring.buf[i & 1]) + done, n - done,
                                     static_cast<off_t>(packed::kHeaderBytes + off + done));
          if (w <= 0) return Status::Internal("packed cache: write failed: " + std::string(std::strerror(errno)));
          done += static_cast<uint64_t>(w);
        }
      }
      packed::Header h;
      h.payload_bytes = payload;
      h.payload_checksum = hasher.Finish();
      h.cfg = cfg;
      h.cfg.max_tokens = 0;
      h.cfg.max_prefill_chunk = 0;
      uint8_t hb[packed::kHeaderBytes];
      packed::EncodeHeader(h, hb);
      if (::pwrite(fd, hb, sizeof(hb), 0) != static_cast<ssize_t>(sizeof(hb)) || ::fsync(fd) != 0)
        return Status::Internal("packed cache: write failed: " + std::string(std::strerror(errno)));
      return Status::Ok();
    }();
    ::close(fd);
    if (st.ok() && ::rename(tmp.c_str(), path.c_str()) != 0)
      st = Status::Internal("packed cache: cannot rename " + tmp + " to " + path + ": " + std::strerror(errno));
    if (!st.ok()) ::unlink(tmp.c_str());
    return st;
  }

  // Allocates the model for cfg (shape and formats from the cache header) and streams
  // the cache's weight region into the slab, checking the payload checksum.
  Status LoadPackedCache(const std::string& path, const packed::Header& h) {
    AM_RETURN_IF_ERROR(Allocate());
    if (WeightRegionBytes() != h.payload_bytes)
      return Status::FailedPrecondition("packed cache: payload size does not match this library's weight layout");
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return Status::NotFound("packed cache: cannot open " + path + ": " + std::strerror(errno));
    Ring ring;
    packed::PayloadHasher hasher;
    Status st = [&]() -> Status {
      AM_RETURN_IF_ERROR(ring.Init());
      bool pending[2] = {false, false};
      for (uint64_t off = 0, i = 0; off < h.payload_bytes; off += Ring::kChunk, ++i) {
        const uint64_t n = std::min<uint64_t>(Ring::kChunk, h.payload_bytes - off);
        if (pending[i & 1]) AM_HIP_OK(hipEventSynchronize(ring.ev[i & 1]));
        for (uint64_t done = 0; done < n;) {
          const ssize_t r = ::pread(fd, static_cast<char*>(ring.buf[i & 1]) + done, n - done,
                                    static_cast<off_t>(packed::kHeaderBytes + off + done));
          if (r <= 0) return Status::DataLoss("packed cache: " + path + " ends inside its payload");
          done += static_cast<uint64_t>(r);
        }
        hasher.Update(ring.buf[i & 1], n);
        AM_HIP_OK(hipMemcpyAsync(static_cast<char*>(slab.base) + off, ring.buf[i & 1], n, hipMemcpyHostToDevice,
                                 stream));
        AM_HIP_OK(hipEventRecord(ring.ev[i & 1], stream));
        pending[i & 1] = true;
      }
      AM_HIP_OK(hipStreamSynchronize(stream));
      if (hasher.Finish() != h.payload_checksum) return Status::DataLoss("packed cache: payload checksum mismatch");
      return FillRope();
    }();
    ::close(fd);
    return st;
  }
};

// ------------------------------------------------------------------ session
class LlamaSession {
 public:
  LlamaModel* m = nullptr;
  hipStream_t stream = nullptr;
  std::unique_ptr<HipStream> hs;
  BackendRegistry backends;
  Backend* backend = nullptr;
  am_session_options opt{1, 1, 1, 0};
  int64_t B = 1;  // sequences decoded together

  // KV: one device slot pool, sequence r in slot r (its planes kv_row_elems elements
  // after sequence r-1's, the batch stride of the batched decode kernels)
  std::unique_ptr<KVCacheManager> kv;
  int64_t kv_row_elems = 0;
  std::vector<KVCacheView> views;
  // Paged KV (opt.kv_block_size > 0) instead: one block pool for every sequence; the
  // device block table is refreshed from a pinned mirror, on the stream, before the
  // work that first uses new blocks (table_ev: the last refresh has read the mirror)
  std::unique_ptr<KVBlockManager> blocks;
  int32_t* table_pinned = nullptr;
  hipEvent_t table_ev = nullptr;

  // device buffers
  void* act_slab = nullptr;
  int64_t* ids = nullptr;
  int64_t* positions = nullptr;
  void *h = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr, *tmp = nullptr;
  void *gate = nullptr, *up = nullptr, *act = nullptr;
  float* logits = nullptr;   // [B][vocab]
  int64_t* state = nullptr;  // token[B], pos[B], step
  int64_t* hist = nullptr;   // [B][max_tokens + 1]
  int32_t* err = nullptr;
  void* attn_ws = nullptr;
  size_t attn_ws_bytes = 0;
  void* gemm_ws = nullptr;  // split-K workspace of the prefill INT4 GEMMs
  size_t gemm_ws_bytes = 0;
  void* lm_ws = nullptr;
  void* am_ws = nullptr;
  int64_t am_ws_bytes = 0;

  // persistent all-layers decode (am_gfx950_decode_layers): device layer table and
  // exchange workspace (zero-filled at creation and after an aborted launch)
  bool persistent = false;
  void* dl_table = nullptr;
  void* dl_ws = nullptr;
  int64_t dl_ws_bytes = 0;

  // decode plan
  std::unique_ptr<ExecutionPlan> decode_plan;
  RuntimeBindingContext decode_bind;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  std::vector<int64_t> row_pos;     // host mirror of pos[r] after each host-visible sync point
  std::vector<uint8_t> row_ready;   // sequence r has been prefilled
  int64_t host_step = 0;            // decode steps since the last prefill (shared by all rows)

  ~LlamaSession() {
    if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
    if (graph) (void)hipGraphDestroy(graph);
    views.clear();
    kv.reset();
    if (table_ev) (void)hipEventSynchronize(table_ev), (void)hipEventDestroy(table_ev);
    blocks.reset();
    if (table_pinned) (void)hip_alloc::PinnedFree(table_pinned);
    if (act_slab) (void)hip_alloc::DeviceFree(act_slab);
    if (dl_table) (void)hip_alloc::DeviceFree(dl_table);
    if (dl_ws) (void)hip_alloc::DeviceFree(dl_ws);
  }

  int64_t HistStride() const { return static_cast<int64_t>(m->cfg.max_tokens) + 1; }
  int64_t* token_ptr(int64_t r = 0) const { return state + r; }
  int64_t* pos_ptr(int64_t r = 0) const { return state + B + r; }
  int64_t* step_ptr() const { return state + 2 * B; }
  int64_t* hist_ptr(int64_t r = 0) const { return hist + r * HistStride(); }
  int64_t host_pos() const { return row_pos.empty() ? 0 : row_pos[0]; }

  // Copies a changed block table to the device, ordered on the session stream.
  Status SyncTable() {
    if (!blocks || !blocks->dirty()) return Status::Ok();
    AM_HIP_OK(hipEventSynchronize(table_ev));  // the previous refresh has read the mirror
    const auto& t = blocks->host_table();
    std::memcpy(table_pinned, t.data(), t.size() * 4);
    AM_HIP_OK(hipMemcpyAsync(blocks->device_table(), table_pinned, t.size() * 4, hipMemcpyHostToDevice, stream));
    AM_HIP_OK(hipEventRecord(table_ev, stream));
    blocks->clear_dirty();
    return Status::Ok();
  }

  // Paging of the ops reading sequence `row` (batched ops: row 0, the table base).
  gfx950::KvPaging Paging(int64_t row) const {
    gfx950::KvPaging pg;
    if (!blocks) return pg;
    pg.table = blocks->device_table() + row * static_cast<int64_t>(blocks->table_stride());
    pg.block = static_cast<int32_t>(blocks->block_size());
    pg.stride = static_cast<int32_t>(blocks->table_stride());
    pg.num_blocks = static_cast<int64_t>(blocks->num_blocks());
    return pg;
  }

  // K and V cache bases of layer l for sequence `row`: its slot's planes, or the
  // layer's block pools when the KV is paged.
  Status Planes(int64_t l, int64_t row, void** kp, void** vp) const {
    if (blocks) {
      *kp = blocks->key_pool(static_cast<size_t>(l));
      *vp = blocks->value_pool(static_cast<size_t>(l));
      return Status::Ok();
    }
    auto k = views[static_cast<size_t>(row)].KeyPlane(static_cast<size_t>(l));
    auto v = views[static_cast<size_t>(row)].ValuePlane(static_cast<size_t>(l));
    if (!k.ok()) return k.status();
    if (!v.ok()) return v.status();
    *kp = k.value();
    *vp = v.value();
    return Status::Ok();
  }

  // Paged KV: blocks for the next n decode steps of every sequence.
  Status GrowForDecode(int64_t n) {
    if (!blocks) return Status::Ok();
    for (int64_t r = 0; r < B; ++r)
      AM_RETURN_IF_ERROR(blocks->EnsureCapacity(static_cast<size_t>(r), static_cast<size_t>(row_pos[r] + n)));
    return SyncTable();
  }

  Status Init(LlamaModel* model, const am_session_options* o) {
    m = model;
    stream = model->stream;
    hs = std::make_unique<HipStream>(stream);
    if (o) opt = *o;
    B = opt.batch > 1 ? opt.batch : 1;
    const auto& c = m->cfg;
    if (B > 16) return Status::InvalidArgument("session batch must be 1..16");
    if (B > 1 && (!opt.fused_decode || c.act_dtype != AM_DT_BF16 || c.weight_format == AM_WF_F32))
      return Status::Unimplemented("batched decode needs the fused plan, bf16 activations and bf16/int8/int4 weights");
    AM_RETURN_IF_ERROR(backends.RegisterFactory(std::make_unique<gfx950::Gfx950BackendFactory>()));
    auto b = backends.GetBackend(DeviceType::kHIP);
    if (!b.ok()) return b.status();
    backend = b.value();
    (void)am::DeviceCUs();

    if (opt.kv_block_size > 0) {
      // paged KV: a pool of blocks shared by the B sequences
      if (c.act_dtype != AM_DT_BF16) return Status::Unimplemented("paged KV needs bf16 activations");
      if (opt.persistent_decode > 0) return Status::Unimplemented("paged KV does not run with persistent_decode");
      const int64_t bs = opt.kv_block_size, per_seq = (c.max_tokens + bs - 1) / bs;
      const int64_t nb = opt.kv_pool_blocks > 0 ? opt.kv_pool_blocks : B * per_seq;
      blocks = std::make_unique<KVBlockManager>(HipDeviceAllocator());
      AM_RETURN_IF_ERROR(blocks->Init(c.num_layers, c.num_kv_heads, c.head_dim, ActType(c.act_dtype),
                                      static_cast<size_t>(bs), static_cast<size_t>(nb), static_cast<size_t>(B),
                                      static_cast<size_t>(c.max_tokens)));
      AM_HIP_OK(hip_alloc::PinnedMalloc(&table_pinned, blocks->host_table().size() * 4));
      AM_HIP_OK(hipEventCreateWithFlags(&table_ev, hipEventDisableTiming));
      AM_RETURN_IF_ERROR(SyncTable());
    } else {
      // KV: a pool of B slots of max_tokens positions, sequence r in slot r
      kv = std::make_unique<KVCacheManager>(HipDeviceAllocator());
      AM_RETURN_IF_ERROR(kv->Init(c.num_layers, c.num_kv_heads, c.max_tokens, c.head_dim, ActType(c.act_dtype), 256,
                                  static_cast<size_t>(B)));
      kv_row_elems = static_cast<int64_t>(kv->storage().slot_bytes / ActBytes(c.act_dtype));
      for (int64_t r = 0; r < B; ++r) {
        auto vw = kv->ReserveSlot(static_cast<size_t>(r), 0, static_cast<size_t>(c.max_tokens));
        if (!vw.ok()) return vw.status();
        views.push_back(vw.value());
      }
    }
    row_pos.assign(static_cast<size_t>(B), 0);
    row_ready.assign(static_cast<size_t>(B), 0);

    const int64_t S = std::max<int64_t>(c.max_prefill_chunk, B), H = c.hidden, F = c.ffn;
    const size_t ab = ActBytes(c.act_dtype);
    attn_ws_bytes = static_cast<size_t>(std::max(
        am_gfx950_attention_workspace_bytes(1, S, c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_tokens, 0),
        am_gfx950_attention_workspace_bytes(B, 1, c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_tokens, 0)));
    am_ws_bytes = am_gfx950_argmax_workspace_bytes(1);
    if (c.weight_format == AM_WF_INT4 || c.weight_format == AM_WF_INT8 || c.weight_format == AM_WF_BF16) {
      const int64_t g = c.weight_format == AM_WF_INT4 ? c.group_size : 128;
      for (auto nk : {std::pair<int64_t, int64_t>{m->QRows() + 2 * m->KvRows(), H}, {H, m->QRows()}, {2 * F, H}, {H, F}})
        gemm_ws_bytes = std::max(gemm_ws_bytes, static_cast<size_t>(am_gfx950_gemm_workspace_bytes(S, nk.first, nk.second, g)));
    }
    const size_t sizes[] = {
        static_cast<size_t>(S) * 8,                   // ids
        static_cast<size_t>(S) * 8,                   // positions
        static_cast<size_t>(S * H) * ab,              // h
        static_cast<size_t>(S * H) * ab,              // xn
        static_cast<size_t>(S * m->QRows()) * ab,     // q
        static_cast<size_t>(S * m->KvRows()) * ab,    // k
        static_cast<size_t>(S * m->KvRows()) * ab,    // v
        static_cast<size_t>(S * m->QRows()) * ab,     // attn
        static_cast<size_t>(S * H) * ab,              // tmp
        static_cast<size_t>(S * F) * ab,              // gate
        static_cast<size_t>(S * F) * ab,              // up
        static_cast<size_t>(S * F) * ab,              // act
        static_cast<size_t>(B * c.vocab) * 4,         // logits
        static_cast<size_t>(2 * B + 1) * 8,           // state
        static_cast<size_t>(B * HistStride()) * 8,    // hist
        64,                                           // err
        attn_ws_bytes,                                // attention workspace
        static_cast<size_t>(am_gfx950_lm_head_workspace_bytes()),
        static_cast<size_t>(am_ws_bytes),
        gemm_ws_bytes};                               // prefill GEMM split-K workspace
    constexpr int kParts = static_cast<int>(sizeof(sizes) / sizeof(sizes[0]));
    size_t total = 0;
    for (size_t s : sizes) total += (s + 255) & ~size_t{255};
    AM_HIP_OK(hip_alloc::DeviceMalloc(&act_slab, total));
    AM_HIP_OK(hipMemsetAsync(act_slab, 0, total, stream));
    Slab sl{act_slab, total, 0};
    void* ptrs[kParts];
    for (int i = 0; i < kParts; ++i) ptrs[i] = sl.Take(sizes[i]);
    ids = static_cast<int64_t*>(ptrs[0]);
    positions = static_cast<int64_t*>(ptrs[1]);
    h = ptrs[2];
    xn = ptrs[3];
    q = ptrs[4];
    k = ptrs[5];
    v = ptrs[6];
    attn = ptrs[7];
    tmp = ptrs[8];
    gate = ptrs[9];
    up = ptrs[10];
    act = ptrs[11];
    logits = static_cast<float*>(ptrs[12]);
    state = static_cast<int64_t*>(ptrs[13]);
    hist = static_cast<int64_t*>(ptrs[14]);
    err = static_cast<int32_t*>(ptrs[15]);
    attn_ws = ptrs[16];
    lm_ws = ptrs[17];
    am_ws = ptrs[18];
    gemm_ws = gemm_ws_bytes ? ptrs[19] : nullptr;
    decode_bind.SetStream(hs.get());
    decode_bind.SetWorkspace(attn_ws, attn_ws_bytes);
    AM_HIP_OK(hipStreamSynchronize(stream));
    AM_RETURN_IF_ERROR(SetupPersistent());
    return BuildDecodePlan();
  }

  am_gfx950_decode_layers_args DecodeLayersArgs() const {
    const auto& c = m->cfg;
    am_gfx950_decode_layers_args a{};
    a.layers = static_cast<const am_gfx950_decode_layer*>(dl_table);
    a.num_layers = c.num_layers;
    a.hidden = c.hidden;
    a.hq = c.num_q_heads;
    a.hkv = c.num_kv_heads;
    a.head_dim = c.head_dim;
    a.ffn = c.ffn;
    a.capacity = c.max_tokens;
    a.eps = c.rms_eps;
    a.cos_tab = m->cos_tab;
    a.sin_tab = m->sin_tab;
    a.pos = pos_ptr();
    a.h = h;
    a.workspace = dl_ws;
    a.workspace_bytes = dl_ws_bytes;
    a.dtype = c.act_dtype;
    return a;
  }

  // Decides whether batch-1 decode runs as one persistent launch for all layers
  // (option persistent_decode: 1 requested, else the per-op fused plan) and prepares
  // its device layer table and exchange workspace.
  Status SetupPersistent() {
    const auto& c = m->cfg;
    persistent = false;
    if (opt.persistent_decode <= 0) return Status::Ok();
    const bool required = true;
    if (B != 1 || !opt.fused_decode || c.act_dtype != AM_DT_BF16 || c.weight_format != AM_WF_INT4) {
      if (required)
        return Status::Unimplemented("persistent decode needs batch 1, the fused plan, bf16 activations and INT4 weights");
      return Status::Ok();
    }
    const size_t L = static_cast<size_t>(c.num_layers);
    std::vector<am_gfx950_decode_layer> host(L);
    for (size_t l = 0; l < L; ++l) {
      auto kp = views[0].KeyPlane(l);
      auto vp = views[0].ValuePlane(l);
      if (!kp.ok()) return kp.status();
      if (!vp.ok()) return vp.status();
      host[l] = am_gfx950_decode_layer{m->qkv[l], m->o[l], m->gate_up[l], m->down[l], m->in_norm[l], m->post_norm[l],
                                       kp.value(), vp.value()};
    }
    dl_ws_bytes = am_gfx950_decode_layers_workspace_bytes(c.hidden, c.num_q_heads, c.num_kv_heads, c.head_dim, c.ffn);
    if (dl_ws_bytes <= 0) {
      if (required) return Status::Unimplemented("persistent decode: unsupported head_dim or shape");
      return Status::Ok();
    }
    AM_HIP_OK(hip_alloc::DeviceMalloc(&dl_ws, static_cast<size_t>(dl_ws_bytes)));
    AM_HIP_OK(hip_alloc::DeviceMalloc(&dl_table, L * sizeof(am_gfx950_decode_layer)));
    const am_gfx950_decode_layers_args a = DecodeLayersArgs();
    if (am_gfx950_decode_layers_validate(&a, host.data()) != AM_STATUS_OK) {
      const std::string why = am_last_error_message();
      (void)hip_alloc::DeviceFree(dl_ws);
      (void)hip_alloc::DeviceFree(dl_table);
      dl_ws = dl_table = nullptr;
      dl_ws_bytes = 0;
      if (required) return Status::Unimplemented("persistent decode: " + why);
      return Status::Ok();
    }
    AM_HIP_OK(hipMemcpy(dl_table, host.data(), L * sizeof(am_gfx950_decode_layer), hipMemcpyHostToDevice));
    AM_HIP_OK(hipMemset(dl_ws, 0, static_cast<size_t>(dl_ws_bytes)));
    persistent = true;
    return Status::Ok();
  }

  // After a synchronised decode: a persistent launch whose blocks were not all
  // resident ends early with the workspace abort flag set.
  Status CheckPersistentAbort() {
    if (!persistent) return Status::Ok();
    int32_t ab = 0;
    if (am_gfx950_decode_layers_aborted(dl_ws, &ab) != AM_STATUS_OK) return Status::Internal(am_last_error_message());
    if (ab == 0) return Status::Ok();
    AM_HIP_OK(hipMemset(dl_ws, 0, static_cast<size_t>(dl_ws_bytes)));
    return Status::Internal("persistent decode: a cross-block wait timed out (the grid was not resident at once)");
  }

  // ---------------------------------------------------------------- plan building
  struct Builder {
    LlamaSession* s;
    ExecPhase phase;
    std::vector<ExecutionStep> steps;
    RuntimeBindingContext* bind;

    Status Add(OpType op, std::vector<std::byte> attrs, KernelSelector sel, const void* packed,
               std::vector<TensorView> ins, std::vector<MutableTensorView> outs, size_t ws_bytes = 0) {
      auto opr = std::make_shared<DeviceOperator>(op, std::move(attrs));
      AM_RETURN_IF_ERROR(opr->Prepare(*s->backend, sel));
      ExecutionStep st;
      st.selector = sel;
      st.op = opr;
      st.packed_weights = packed;
      st.workspace_bytes = ws_bytes;
      st.debug_name = opr->GetResolvedKernel().debug_name;
      bind->SetStepTensorBinding(steps.size(), StepTensorBinding{std::move(ins), std::move(outs)});
      steps.push_back(std::move(st));
      return Status::Ok();
    }
  };

  KernelSelector Sel(bool linear, ExecPhase ph) const {
    const DataType a = ActType(m->cfg.act_dtype);
    if (linear) return HipSelector(a, WeightDType(m->cfg.weight_format), SelFormat(m->cfg.weight_format), ph);
    return HipSelector(a, a, WeightFormat::kPlain, ph);
  }

  // Unfused per-layer body (reference node order) for `S` rows of sequence `row`
  // starting at device position *start (positions[] holds per-row positions).
  Status AddLayerUnfused(Builder& b, int64_t l, int64_t S, ExecPhase ph, const int64_t* pos_rows,
                         const int64_t* start, int64_t row) {
    const auto& c = m->cfg;
    const DataType A = ActType(c.act_dtype);
    const int64_t H = c.hidden, F = c.ffn, d = c.head_dim, Q = m->QRows(), KV = m->KvRows();
    void *kp = nullptr, *vp = nullptr;
    AM_RETURN_IF_ERROR(Planes(l, row, &kp, &vp));
    const gfx950::NormAttrs na{c.rms_eps};
    auto& W = s_views[static_cast<size_t>(l)];
    const TensorView hv(h, A, {S, H}), xnv(xn, A, {S, H});
    // Prefill on the MFMA GEMM fuses each Linear with its neighbour: q|k|v as one GEMM
    // over the concatenated weight, o and down with their residual Add, gate|up with
    // the SiluMul (the same op-boundary roundings).  INT4 (group a multiple of 64), INT8
    // and bf16 weights; INT8 and bf16 need every k a multiple of 128.
    const bool k128 = H % 128 == 0 && F % 128 == 0 && Q % 128 == 0;
    const bool fuse = ph == ExecPhase::kPrefill && c.act_dtype == AM_DT_BF16 && c.ffn % 64 == 0 &&
                      ((c.weight_format == AM_WF_INT4 && c.group_size % 64 == 0) ||
                       ((c.weight_format == AM_WF_INT8 || c.weight_format == AM_WF_BF16) && k128));
    AM_RETURN_IF_ERROR(b.Add(OpType::kRmsNorm, PackAttrs(na), Sel(false, ph), nullptr,
                             {hv, TensorView(m->in_norm[l], A, {H})}, {MutableTensorView(xn, A, {S, H})}));
    // the prefill GEMMs' inputs, with the split-K workspace when the session has one
    auto gemm_in = [&](TensorView x) {
      std::vector<TensorView> v{x};
      if (gemm_ws != nullptr) v.push_back(TensorView(gemm_ws, DataType::UInt(8), {static_cast<int64_t>(gemm_ws_bytes)}));
      return v;
    };
    const TensorView kplane(kp, A, {c.num_kv_heads, c.max_tokens, d});
    const TensorView vplane(vp, A, {c.num_kv_heads, c.max_tokens, d});
    // q|k|v GEMM with RoPE and the KV cache write in its epilogue (positions *start + i)
    const bool fuse_rope = fuse && (d == 64 || d == 128);
    if (fuse_rope) {
      const gfx950::QkvAttrs qa{c.rms_eps, c.num_q_heads, c.num_kv_heads, d, c.max_tokens, 0, Paging(row)};
      std::vector<TensorView> in = gemm_in(xnv);
      in.insert(in.begin() + 1, {TensorView(m->cos_tab, DataType::Float32(), {c.max_tokens, d / 2}),
                                 TensorView(m->sin_tab, DataType::Float32(), {c.max_tokens, d / 2}),
                                 TensorView(start, DataType::Int(64), {1}), kplane, vplane});
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearRoPEKVUpdate, PackAttrs(qa), Sel(true, ph), &m->qkv[l], in,
                               {MutableTensorView(q, A, {S, Q})}));
    } else if (fuse) {
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearSplit, {}, Sel(true, ph), &m->qkv[l], gemm_in(xnv),
                               {MutableTensorView(q, A, {S, Q}), MutableTensorView(k, A, {S, KV}),
                                MutableTensorView(v, A, {S, KV})}));
    } else {
      AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &W.q, {xnv}, {MutableTensorView(q, A, {S, Q})}));
      AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &W.k, {xnv}, {MutableTensorView(k, A, {S, KV})}));
      AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &W.v, {xnv}, {MutableTensorView(v, A, {S, KV})}));
    }
    if (!fuse_rope) {
      const gfx950::RopeAttrs ra{c.num_q_heads, c.num_kv_heads, d, c.max_tokens};
      AM_RETURN_IF_ERROR(b.Add(OpType::kRoPE, PackAttrs(ra), Sel(false, ph), nullptr,
                               {TensorView(q, A, {S, Q}), TensorView(k, A, {S, KV}),
                                TensorView(pos_rows, DataType::Int(64), {S}),
                                TensorView(m->cos_tab, DataType::Float32(), {c.max_tokens, d / 2}),
                                TensorView(m->sin_tab, DataType::Float32(), {c.max_tokens, d / 2})},
                               {MutableTensorView(q, A, {S, Q}), MutableTensorView(k, A, {S, KV})}));
      const gfx950::KvAttrs ka{c.num_kv_heads, d, c.max_tokens, Paging(row)};
      AM_RETURN_IF_ERROR(b.Add(OpType::kKVCacheUpdate, PackAttrs(ka), Sel(false, ph), nullptr,
                               {TensorView(k, A, {S, KV}), TensorView(v, A, {S, KV}), kplane, vplane,
                                TensorView(start, DataType::Int(64), {1})},
                               {}));
    }
    const gfx950::AttnAttrs aa{c.num_q_heads, c.num_kv_heads, d, c.max_tokens, 0, 1, 0, Paging(row)};
    AM_RETURN_IF_ERROR(b.Add(OpType::kAttention, PackAttrs(aa), Sel(false, ph), nullptr,
                             {TensorView(q, A, {S, Q}), kplane, vplane, TensorView(start, DataType::Int(64), {1})},
                             {MutableTensorView(attn, A, {S, Q})}, attn_ws_bytes));
    if (fuse) {
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearAdd, {}, Sel(true, ph), &m->o[l], gemm_in(TensorView(attn, A, {S, Q})),
                               {MutableTensorView(h, A, {S, H})}));
    } else {
      AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &m->o[l], {TensorView(attn, A, {S, Q})},
                               {MutableTensorView(tmp, A, {S, H})}));
      AM_RETURN_IF_ERROR(b.Add(OpType::kAdd, {}, Sel(false, ph), nullptr, {hv, TensorView(tmp, A, {S, H})},
                               {MutableTensorView(h, A, {S, H})}));
    }
    AM_RETURN_IF_ERROR(b.Add(OpType::kRmsNorm, PackAttrs(na), Sel(false, ph), nullptr,
                             {hv, TensorView(m->post_norm[l], A, {H})}, {MutableTensorView(xn, A, {S, H})}));
    if (fuse) {
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearSiluMul, {}, Sel(true, ph), &m->gate_up[l], gemm_in(xnv),
                               {MutableTensorView(act, A, {S, F})}));
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearAdd, {}, Sel(true, ph), &m->down[l],
                               gemm_in(TensorView(act, A, {S, F})), {MutableTensorView(h, A, {S, H})}));
      return Status::Ok();
    }
    AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &W.gate, {xnv}, {MutableTensorView(gate, A, {S, F})}));
    AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &W.up, {xnv}, {MutableTensorView(up, A, {S, F})}));
    AM_RETURN_IF_ERROR(b.Add(OpType::kSiluMul, {}, Sel(false, ph), nullptr,
                             {TensorView(gate, A, {S, F}), TensorView(up, A, {S, F})},
                             {MutableTensorView(act, A, {S, F})}));
    AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ph), &m->down[l], {TensorView(act, A, {S, F})},
                             {MutableTensorView(tmp, A, {S, H})}));
    AM_RETURN_IF_ERROR(b.Add(OpType::kAdd, {}, Sel(false, ph), nullptr, {hv, TensorView(tmp, A, {S, H})},
                             {MutableTensorView(h, A, {S, H})}));
    return Status::Ok();
  }

  // RmsNorm(final) -> Linear lm_head (fp32 logits) -> Argmax (+ advance decode state)
  // on the row `hrow` of h, for sequence `row`.
  Status AddHeadUnfused(Builder& b, int64_t hrow, ExecPhase ph, int64_t row) {
    const auto& c = m->cfg;
    const DataType A = ActType(c.act_dtype);
    const int64_t H = c.hidden;
    const size_t ab = ActBytes(c.act_dtype);
    void* hr = static_cast<char*>(h) + static_cast<size_t>(hrow * H) * ab;
    float* lg = logits + row * c.vocab;
    const gfx950::NormAttrs na{c.rms_eps};
    AM_RETURN_IF_ERROR(b.Add(OpType::kRmsNorm, PackAttrs(na), Sel(false, ph), nullptr,
                             {TensorView(hr, A, {1, H}), TensorView(m->final_norm, A, {H})},
                             {MutableTensorView(xn, A, {1, H})}));
    // lm_head GEMV for one row (decode-phase kernel: GEMV) with fp32 logits out.
    AM_RETURN_IF_ERROR(b.Add(OpType::kLinear, {}, Sel(true, ExecPhase::kDecode), &m->lm_head,
                             {TensorView(xn, A, {1, H})},
                             {MutableTensorView(lg, DataType::Float32(), {1, c.vocab})}));
    AM_RETURN_IF_ERROR(b.Add(OpType::kArgmax, {}, Sel(false, ph), nullptr,
                             {TensorView(lg, DataType::Float32(), {1, c.vocab}),
                              TensorView(am_ws, DataType::UInt(8), {am_ws_bytes})},
                             {MutableTensorView(token_ptr(row), DataType::Int(64), {1}),
                              MutableTensorView(hist_ptr(row), DataType::Int(64), {c.max_tokens}),
                              MutableTensorView(pos_ptr(row), DataType::Int(64), {1}),
                              MutableTensorView(step_ptr(), DataType::Int(64), {1})}));
    return Status::Ok();
  }

  struct LayerViews {
    am_gfx950_weight q, k, v, gate, up;
  };
  std::vector<LayerViews> s_views;

  void MakeViews() {
    const int64_t L = m->cfg.num_layers, Q = m->QRows(), KV = m->KvRows(), F = m->cfg.ffn;
    s_views.resize(static_cast<size_t>(L));
    for (int64_t l = 0; l < L; ++l) {
      auto& w = s_views[static_cast<size_t>(l)];
      w.q = m->RowView(m->qkv[l], 0, Q);
      w.k = m->RowView(m->qkv[l], Q, KV);
      w.v = m->RowView(m->qkv[l], Q + KV, KV);
      w.gate = m->RowView(m->gate_up[l], 0, F);
      w.up = m->RowView(m->gate_up[l], F, F);
    }
  }

  // Decode plan for the B sequences: one token of each per step.  B > 1 runs the
  // batched forms of the fused kernels (rows = B, per-row positions, sequence r's KV
  // planes kv_row_elems after sequence r-1's).
  Status BuildDecodePlan() {
    MakeViews();
    const auto& c = m->cfg;
    const DataType A = ActType(c.act_dtype);
    const int64_t H = c.hidden, F = c.ffn, d = c.head_dim, Q = m->QRows();
    decode_bind.ClearStepTensorBindings();
    Builder b{this, ExecPhase::kDecode, {}, &decode_bind};
    const auto ph = ExecPhase::kDecode;
    if (B == 1) {
      AM_RETURN_IF_ERROR(b.Add(OpType::kEmbedToken, {}, Sel(false, ph), nullptr,
                               {TensorView(token_ptr(), DataType::Int(64), {1}), TensorView(m->embed, A, {c.vocab, H}),
                                TensorView(err, DataType::Int(32), {1})},
                               {MutableTensorView(h, A, {1, H})}));
    } else {
      AM_RETURN_IF_ERROR(b.Add(OpType::kEmbedding, {}, Sel(false, ph), nullptr,
                               {TensorView(token_ptr(), DataType::Int(64), {B}), TensorView(m->embed, A, {c.vocab, H}),
                                TensorView(err, DataType::Int(32), {1})},
                               {MutableTensorView(h, A, {B, H})}));
    }
    if (persistent) {
      const gfx950::DecodeLayersAttrs da{c.rms_eps, c.num_layers, H, c.num_q_heads, c.num_kv_heads, d, F, c.max_tokens};
      AM_RETURN_IF_ERROR(b.Add(
          OpType::kFusedDecodeLayers, PackAttrs(da), Sel(true, ph), nullptr,
          {TensorView(h, A, {1, H}), TensorView(pos_ptr(), DataType::Int(64), {1}),
           TensorView(m->cos_tab, DataType::Float32(), {c.max_tokens, d / 2}),
           TensorView(m->sin_tab, DataType::Float32(), {c.max_tokens, d / 2}),
           TensorView(dl_table, DataType::UInt(8), {static_cast<int64_t>(c.num_layers * sizeof(am_gfx950_decode_layer))}),
           TensorView(dl_ws, DataType::UInt(8), {dl_ws_bytes})},
          {MutableTensorView(h, A, {1, H})}));
    }
    for (int64_t l = 0; l < c.num_layers && !persistent; ++l) {
      if (!opt.fused_decode) {
        AM_RETURN_IF_ERROR(AddLayerUnfused(b, l, 1, ph, pos_ptr(), pos_ptr(), 0));
        continue;
      }
      void *kp = nullptr, *vp = nullptr;
      AM_RETURN_IF_ERROR(Planes(l, 0, &kp, &vp));
      const TensorView kplane(kp, A, {c.num_kv_heads, c.max_tokens, d});
      const TensorView vplane(vp, A, {c.num_kv_heads, c.max_tokens, d});
      const gfx950::QkvAttrs qa{c.rms_eps, c.num_q_heads, c.num_kv_heads, d, c.max_tokens, kv_row_elems, Paging(0)};
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedRmsNormQkvRoPEKVUpdate, PackAttrs(qa), Sel(true, ph), &m->qkv[l],
                               {TensorView(h, A, {B, H}), TensorView(m->in_norm[l], A, {H}),
                                TensorView(pos_ptr(), DataType::Int(64), {B}),
                                TensorView(m->cos_tab, DataType::Float32(), {c.max_tokens, d / 2}),
                                TensorView(m->sin_tab, DataType::Float32(), {c.max_tokens, d / 2}), kplane, vplane},
                               {MutableTensorView(q, A, {B, Q})}));
      const gfx950::AttnAttrs aa{c.num_q_heads, c.num_kv_heads, d, c.max_tokens, 0, B, kv_row_elems, Paging(0)};
      AM_RETURN_IF_ERROR(b.Add(OpType::kAttention, PackAttrs(aa), Sel(false, ph), nullptr,
                               {TensorView(q, A, {B, Q}), kplane, vplane, TensorView(pos_ptr(), DataType::Int(64), {B})},
                               {MutableTensorView(attn, A, {B, Q})}, attn_ws_bytes));
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearAdd, {}, Sel(true, ph), &m->o[l], {TensorView(attn, A, {B, Q})},
                               {MutableTensorView(h, A, {B, H})}));
      const gfx950::NormAttrs na{c.rms_eps};
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedRmsNormGateUpSiluMul, PackAttrs(na), Sel(true, ph), &m->gate_up[l],
                               {TensorView(h, A, {B, H}), TensorView(m->post_norm[l], A, {H})},
                               {MutableTensorView(act, A, {B, F})}));
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedLinearAdd, {}, Sel(true, ph), &m->down[l], {TensorView(act, A, {B, F})},
                               {MutableTensorView(h, A, {B, H})}));
    }
    if (opt.fused_decode) {
      const gfx950::NormAttrs na{c.rms_eps};
      AM_RETURN_IF_ERROR(b.Add(OpType::kFusedRmsNormLmHeadArgmax, PackAttrs(na), Sel(true, ph), &m->lm_head,
                               {TensorView(h, A, {B, H}), TensorView(m->final_norm, A, {H}),
                                TensorView(lm_ws, DataType::UInt(8), {am_gfx950_lm_head_workspace_bytes()})},
                               {MutableTensorView(logits, DataType::Float32(), {B, c.vocab}),
                                MutableTensorView(token_ptr(), DataType::Int(64), {B}),
                                MutableTensorView(hist, DataType::Int(64), {B, HistStride()}),
                                MutableTensorView(pos_ptr(), DataType::Int(64), {B}),
                                MutableTensorView(step_ptr(), DataType::Int(64), {1})}));
    } else {
      AM_RETURN_IF_ERROR(AddHeadUnfused(b, 0, ph, 0));
    }
    auto plan = ExecutionPlan::Create(std::move(b.steps));
    if (!plan.ok()) return plan.status();
    decode_plan = std::make_unique<ExecutionPlan>(std::move(plan.value()));
    return Status::Ok();
  }

  // ---------------------------------------------------------------- execution
  // Prefill sequence `row` from position 0 (its own KV reservation); the other rows
  // keep their state.  The shared step counter restarts at 1.
  Status Prefill(int64_t row, const int64_t* prompt, int64_t n, int64_t* first_token) {
    const auto& c = m->cfg;
    if (row < 0 || row >= B) return Status::OutOfRange("prefill: sequence row out of range");
    if (n <= 0) return Status::InvalidArgument("prompt must contain at least one token");
    if (n + 1 > c.max_tokens) return Status::OutOfRange("KV session reservation exceeds physical KV capacity");
    for (int64_t i = 0; i < n; ++i)
      if (prompt[i] < 0 || prompt[i] >= c.vocab) return Status::OutOfRange("EmbeddingKernel token id is out of vocabulary range");
    const size_t ri = static_cast<size_t>(row);
    row_ready[ri] = 0;
    if (blocks) {
      // the row's blocks go back to the pool; the prompt takes blocks for [0, n)
      AM_RETURN_IF_ERROR(blocks->ReleaseSequence(ri));
      AM_RETURN_IF_ERROR(blocks->EnsureCapacity(ri, static_cast<size_t>(n)));
      AM_RETURN_IF_ERROR(SyncTable());
    } else {
      AM_RETURN_IF_ERROR(kv->ReleaseSession(views[ri]));
      auto vw = kv->ReserveSlot(ri, 0, static_cast<size_t>(c.max_tokens));
      if (!vw.ok()) return vw.status();
      views[ri] = vw.value();  // same slot planes: the decode plan and graph stay valid
    }
    const int64_t chunk = c.max_prefill_chunk;
    std::vector<int64_t> pos_host(static_cast<size_t>(chunk));
    for (int64_t p0 = 0; p0 < n; p0 += chunk) {
      const int64_t S = std::min(chunk, n - p0);
      for (int64_t i = 0; i < S; ++i) pos_host[static_cast<size_t>(i)] = p0 + i;
      AM_HIP_OK(hipMemcpyAsync(ids, prompt + p0, static_cast<size_t>(S) * 8, hipMemcpyHostToDevice, stream));
      AM_HIP_OK(hipMemcpyAsync(positions, pos_host.data(), static_cast<size_t>(S) * 8, hipMemcpyHostToDevice, stream));
      RuntimeBindingContext bind;
      bind.SetStream(hs.get());
      bind.SetWorkspace(attn_ws, attn_ws_bytes);
      Builder b{this, ExecPhase::kPrefill, {}, &bind};
      const DataType A = ActType(c.act_dtype);
      AM_RETURN_IF_ERROR(b.Add(OpType::kEmbedding, {}, Sel(false, ExecPhase::kPrefill), nullptr,
                               {TensorView(ids, DataType::Int(64), {S}), TensorView(m->embed, A, {c.vocab, c.hidden}),
                                TensorView(err, DataType::Int(32), {1})},
                               {MutableTensorView(h, A, {S, c.hidden})}));
      for (int64_t l = 0; l < c.num_layers; ++l)
        AM_RETURN_IF_ERROR(AddLayerUnfused(b, l, S, ExecPhase::kPrefill, positions, positions, row));
      const bool last = p0 + S == n;
      if (last) {
        // decode state before the head: pos = n-1, step = 0 (the head advances both)
        const int64_t zero = 0, pm1 = n - 1;
        AM_HIP_OK(hipMemcpyAsync(token_ptr(row), &zero, 8, hipMemcpyHostToDevice, stream));
        AM_HIP_OK(hipMemcpyAsync(pos_ptr(row), &pm1, 8, hipMemcpyHostToDevice, stream));
        AM_HIP_OK(hipMemcpyAsync(step_ptr(), &zero, 8, hipMemcpyHostToDevice, stream));
        AM_RETURN_IF_ERROR(AddHeadUnfused(b, S - 1, ExecPhase::kPrefill, row));
      }
      auto plan = ExecutionPlan::Create(std::move(b.steps));
      if (!plan.ok()) return plan.status();
      AM_RETURN_IF_ERROR(Executor::Execute(plan.value(), bind));
      AM_HIP_OK(hipStreamSynchronize(stream));  // pos_host / state staging reuse
    }
    if (!blocks) AM_RETURN_IF_ERROR(views[ri].CommitUntil(static_cast<size_t>(n)));
    int64_t tok = 0;
    AM_HIP_OK(hipMemcpy(&tok, token_ptr(row), 8, hipMemcpyDeviceToHost));
    int32_t e = 0;
    AM_HIP_OK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
    if (e != 0) return Status::OutOfRange("EmbeddingKernel token id is out of vocabulary range");
    row_pos[ri] = n;
    row_ready[ri] = 1;
    host_step = 1;
    if (first_token) *first_token = tok;
    return Status::Ok();
  }

  Status CheckDecode(int64_t n) const {
    const auto& c = m->cfg;
    for (int64_t r = 0; r < B; ++r) {
      if (!row_ready[static_cast<size_t>(r)]) return Status::FailedPrecondition("decode requires a prefilled session");
      if (row_pos[static_cast<size_t>(r)] + n > c.max_tokens)
        return Status::OutOfRange("KV write exceeds reserved session token capacity");
    }
    return Status::Ok();
  }

  Status Advance(int64_t n) {
    for (int64_t r = 0; r < B; ++r) {
      const size_t ri = static_cast<size_t>(r);
      row_pos[ri] += n;
      if (!blocks) AM_RETURN_IF_ERROR(views[ri].CommitUntil(static_cast<size_t>(row_pos[ri])));
    }
    return Status::Ok();
  }

  Status EnqueueDecode(int64_t n) {
    AM_RETURN_IF_ERROR(CheckDecode(n));
    AM_RETURN_IF_ERROR(GrowForDecode(n));
    if (opt.use_graph) {
      if (!graph_exec) {
        AM_HIP_OK(hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed));
        Status st = Executor::Execute(*decode_plan, decode_bind);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(stream, &g);
        if (!st.ok()) {
          if (g) (void)hipGraphDestroy(g);
          return st;
        }
        if (e != hipSuccess) return Status::Internal(std::string("graph capture failed: ") + hipGetErrorString(e));
        graph = g;
        AM_HIP_OK(hip_alloc::GraphInstantiate(&graph_exec, graph));
      }
      for (int64_t i = 0; i < n; ++i) AM_HIP_OK(hipGraphLaunch(graph_exec, stream));
    } else {
      for (int64_t i = 0; i < n; ++i) AM_RETURN_IF_ERROR(Executor::Execute(*decode_plan, decode_bind));
    }
    return Advance(n);
  }

  // n decode steps; out (host) receives [B][n] tokens, sequence-major.
  Status Decode(int64_t n, int64_t* out) {
    const int64_t first_step = host_step;
    AM_RETURN_IF_ERROR(EnqueueDecode(n));
    host_step += n;
    if (out)
      for (int64_t r = 0; r < B; ++r)
        AM_HIP_OK(hipMemcpyAsync(out + r * n, hist_ptr(r) + first_step, static_cast<size_t>(n) * 8,
                                 hipMemcpyDeviceToHost, stream));
    AM_HIP_OK(hipStreamSynchronize(stream));
    AM_RETURN_IF_ERROR(CheckPersistentAbort());
    int32_t e = 0;
    AM_HIP_OK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
    if (e != 0) return Status::OutOfRange("EmbeddingKernel token id is out of vocabulary range");
    return Status::Ok();
  }

  // Per-step device time of the decode plan, eager replay of the same steps on the
  // session stream.  Weight-GEMV and attention steps are timed with events bound to
  // their single dispatch (hipExtLaunchKernelGGL start/stop), other steps with events
  // around the step.
  Status Profile(int64_t n, double* ms_by_op, int64_t* count_by_op) {
    AM_RETURN_IF_ERROR(CheckDecode(n));
    AM_RETURN_IF_ERROR(GrowForDecode(n));
    const auto& steps = decode_plan->steps();
    std::vector<hipEvent_t> e0(steps.size(), nullptr), e1(steps.size(), nullptr);
    Status st;
    for (size_t i = 0; i < steps.size() && st.ok(); ++i)
      if (hipEventCreate(&e0[i]) != hipSuccess || hipEventCreate(&e1[i]) != hipSuccess)
        st = Status::Internal("profile: event creation failed");
    am::LaunchTiming& lt = am::ThreadLaunchTiming();
    for (int64_t it = 0; it < n && st.ok(); ++it) {
      for (size_t i = 0; i < steps.size() && st.ok(); ++i) {
        const OpType t = steps[i].op->Type();
        const bool timed = t == OpType::kFusedRmsNormQkvRoPEKVUpdate || t == OpType::kFusedLinearAdd ||
                           t == OpType::kFusedDecodeLayers || t == OpType::kFusedRmsNormGateUpSiluMul ||
                           (t == OpType::kFusedRmsNormLmHeadArgmax && B == 1) || t == OpType::kAttention;
        if (timed) {
          lt = {e0[i], e1[i], false};
          st = LayerRunner::RunStep(i, steps[i], decode_bind);
          const bool used = lt.used;
          lt = {};
          if (st.ok() && !used) st = Status::Internal("profile: a timed step did not take the timed launch");
        } else {
          (void)hipEventRecord(e0[i], stream);
          st = LayerRunner::RunStep(i, steps[i], decode_bind);
          (void)hipEventRecord(e1[i], stream);
        }
      }
      if (!st.ok()) break;
      if (hipStreamSynchronize(stream) != hipSuccess) {
        st = Status::Internal("profile: stream synchronize failed");
        break;
      }
      for (size_t i = 0; i < steps.size(); ++i) {
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, e0[i], e1[i]) != hipSuccess) {
          st = Status::Internal("profile: event timing failed");
          break;
        }
        const int op = static_cast<int>(steps[i].op->Type());
        if (op < 64) {
          ms_by_op[op] += ms;
          count_by_op[op] += 1;
        }
      }
    }
    lt = {};
    for (size_t i = 0; i < steps.size(); ++i) {
      if (e0[i]) (void)hipEventDestroy(e0[i]);
      if (e1[i]) (void)hipEventDestroy(e1[i]);
    }
    if (st.ok()) st = CheckPersistentAbort();
    if (st.ok()) {
      host_step += n;
      st = Advance(n);
    }
    return st;
  }
};

}  // namespace aethermind::llama

// ------------------------------------------------------------------ C ABI
using aethermind::Status;
using aethermind::llama::LlamaModel;
using aethermind::llama::LlamaSession;

struct am_runtime {
  int device = 0;
  hipStream_t stream = nullptr;
  am_config_t config{};  // load options of am_model_load
};
struct am_model {
  am_runtime* rt = nullptr;
  std::unique_ptr<LlamaModel> impl;
};
struct am_session {
  std::unique_ptr<LlamaSession> impl;
  uint32_t max_tokens = 0;  // am_session_config_t generation limits (PRD interface)
  int64_t eos = -1;
};

namespace {
am_status_code Ret(const Status& s) {
  if (s.ok()) return AM_STATUS_OK;
  return am::SetLastError(s.c_code(), s.message().c_str());
}
}  // namespace

extern "C" {

static am_config_t DefaultConfig(int32_t device) {
  am_config_t c{};
  c.struct_size = sizeof(am_config_t);
  c.device = device;
  c.act_dtype = AM_DT_BF16;
  c.weight_format = AM_WF_INT4;
  c.group_size = 128;
  c.max_tokens = 4096;
  c.max_prefill_chunk = 512;
  return c;
}

am_status_code am_runtime_open(int32_t device, am_runtime** out) {
  if (out == nullptr) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "runtime: null out");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return am::SetLastError(AM_STATUS_UNAVAILABLE, "no HIP device available");
  if (device < 0 || device >= n) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "runtime: bad device index");
  if (hipSetDevice(device) != hipSuccess) return am::SetLastError(AM_STATUS_INTERNAL, "hipSetDevice failed");
  auto* rt = new am_runtime();
  rt->device = device;
  rt->config = DefaultConfig(device);
  if (hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking) != hipSuccess) {
    delete rt;
    return am::SetLastError(AM_STATUS_INTERNAL, "hipStreamCreate failed");
  }
  *out = rt;
  return AM_STATUS_OK;
}

void am_runtime_destroy(am_runtime* rt) {
  if (!rt) return;
  (void)hipStreamSynchronize(rt->stream);
  (void)hipStreamDestroy(rt->stream);
  delete rt;
}

void* am_runtime_stream(am_runtime* rt) { return rt ? rt->stream : nullptr; }

am_status_code am_runtime_synchronize(am_runtime* rt) {
  if (!rt) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "runtime: null");
  const hipError_t e = hipStreamSynchronize(rt->stream);
  if (e != hipSuccess) return am::SetLastError(AM_STATUS_INTERNAL, hipGetErrorString(e));
  return AM_STATUS_OK;
}

am_status_code am_synth_token_ids_host(uint64_t seed, uint64_t stream, int64_t vocab, int64_t n, int64_t* out) {
  if (vocab <= 0 || n < 0 || (n > 0 && out == nullptr))
    return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "synth_token_ids_host: bad argument");
  auto mix = [](uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  };
  const uint64_t key = mix(mix(seed) ^ (0xF00D0000ull + stream));
  for (int64_t i = 0; i < n; ++i)
    out[i] = static_cast<int64_t>(((mix(key + static_cast<uint64_t>(i)) >> 32) * static_cast<uint64_t>(vocab)) >> 32);
  return AM_STATUS_OK;
}

am_status_code am_model_create_synthetic(am_runtime* rt, const am_model_config* cfg, uint64_t seed, am_model** out) {
  if (!rt || !cfg || !out) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model: null argument");
  auto m = std::make_unique<am_model>();
  m->rt = rt;
  m->impl = std::make_unique<LlamaModel>();
  m->impl->cfg = *cfg;
  m->impl->stream = rt->stream;
  const Status s = m->impl->CreateSynthetic(seed);
  if (!s.ok()) return Ret(s);
  *out = m.release();
  return AM_STATUS_OK;
}

namespace {
aethermind::hf::LoadRules RulesOf(uint32_t flags) {
  aethermind::hf::LoadRules r;
  r.strict_tensor_names = (flags & AM_LOAD_STRICT_TENSOR_NAMES) != 0;
  r.allow_unknown_tensors = (flags & AM_LOAD_REJECT_UNKNOWN_TENSORS) == 0;
  r.allow_quantized_tensors = (flags & AM_LOAD_ALLOW_QUANTIZED_TENSORS) != 0;
  return r;
}
am_model_config ShapeOf(const aethermind::hf::LlamaConfig& hc) {
  am_model_config mc{};
  mc.num_layers = static_cast<int32_t>(hc.num_layers);
  mc.hidden = static_cast<int32_t>(hc.hidden);
  mc.num_q_heads = static_cast<int32_t>(hc.num_q_heads);
  mc.num_kv_heads = static_cast<int32_t>(hc.num_kv_heads);
  mc.head_dim = static_cast<int32_t>(hc.head_dim);
  mc.ffn = static_cast<int32_t>(hc.ffn);
  mc.vocab = static_cast<int32_t>(hc.vocab);
  mc.rms_eps = static_cast<float>(hc.rms_eps);
  mc.rope_theta = hc.rope_theta;
  return mc;
}
constexpr uint32_t kKnownLoadFlags =
    AM_LOAD_STRICT_TENSOR_NAMES | AM_LOAD_REJECT_UNKNOWN_TENSORS | AM_LOAD_ALLOW_QUANTIZED_TENSORS;
}  // namespace

am_status_code am_model_load_hf_ex(am_runtime* rt, const char* model_dir, const am_model_load_options* opt,
                                   uint32_t flags, am_model** out) {
  if (!rt || !model_dir || !opt || !out) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_load_hf: null argument");
  if (flags & ~kKnownLoadFlags) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_load_hf: unknown load flags");
  auto ck = aethermind::hf::Checkpoint::Open(model_dir, RulesOf(flags));
  if (!ck.ok()) return Ret(ck.status());
  am_model_config mc = ShapeOf(ck.value()->config());
  mc.act_dtype = opt->act_dtype;
  mc.weight_format = opt->weight_format;
  mc.group_size = opt->group_size;
  mc.max_tokens = opt->max_tokens;
  mc.max_prefill_chunk = opt->max_prefill_chunk;
  auto m = std::make_unique<am_model>();
  m->rt = rt;
  m->impl = std::make_unique<LlamaModel>();
  m->impl->cfg = mc;
  m->impl->stream = rt->stream;
  const Status s = m->impl->LoadCheckpoint(*ck.value());
  if (!s.ok()) return Ret(s);
  *out = m.release();
  return AM_STATUS_OK;
}

am_status_code am_model_load_hf(am_runtime* rt, const char* model_dir, const am_model_load_options* opt,
                                am_model** out) {
  return am_model_load_hf_ex(rt, model_dir, opt, 0, out);
}

am_status_code am_hf_inspect_ex(const char* model_dir, uint32_t flags, am_model_config* cfg, int64_t* n_tensors,
                                int64_t* total_bytes) {
  if (!model_dir || !cfg) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "hf_inspect: null argument");
  if (flags & ~kKnownLoadFlags) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "hf_inspect: unknown load flags");
  auto ck = aethermind::hf::Checkpoint::Open(model_dir, RulesOf(flags));
  if (!ck.ok()) return Ret(ck.status());
  *cfg = ShapeOf(ck.value()->config());
  if (n_tensors) *n_tensors = static_cast<int64_t>(ck.value()->num_tensors());
  if (total_bytes) *total_bytes = static_cast<int64_t>(ck.value()->total_bytes());
  return AM_STATUS_OK;
}

am_status_code am_hf_inspect(const char* model_dir, am_model_config* cfg, int64_t* n_tensors, int64_t* total_bytes) {
  return am_hf_inspect_ex(model_dir, 0, cfg, n_tensors, total_bytes);
}

am_status_code am_model_save_packed_cache(am_model* m, const char* path) {
  if (!m || !path) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "save_packed_cache: null argument");
  return Ret(m->impl->SavePackedCache(path));
}

am_status_code am_packed_cache_inspect(const char* path, am_model_config* cfg, int64_t* payload_bytes) {
  if (!path || !cfg) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "packed_cache_inspect: null argument");
  auto h = aethermind::packed::Inspect(path);
  if (!h.ok()) return Ret(h.status());
  *cfg = h.value().cfg;
  if (payload_bytes) *payload_bytes = static_cast<int64_t>(h.value().payload_bytes);
  return AM_STATUS_OK;
}

am_status_code am_model_load_packed_cache(am_runtime* rt, const char* path, const am_model_load_options* opt,
                                          am_model** out) {
  if (!rt || !path || !opt || !out)
    return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "load_packed_cache: null argument");
  auto h = aethermind::packed::Inspect(path);
  if (!h.ok()) return Ret(h.status());
  const am_model_config& fc = h.value().cfg;
  if (opt->act_dtype != fc.act_dtype || opt->weight_format != fc.weight_format ||
      (fc.weight_format == AM_WF_INT4 && opt->group_size != fc.group_size)) {
    char msg[200];
    std::snprintf(msg, sizeof(msg),
                  "load_packed_cache: the cache holds act_dtype %d / weight_format %d / group %d, the options ask "
                  "for %d / %d / %d",
                  fc.act_dtype, fc.weight_format, fc.group_size, opt->act_dtype, opt->weight_format, opt->group_size);
    return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, msg);
  }
  auto m = std::make_unique<am_model>();
  m->rt = rt;
  m->impl = std::make_unique<LlamaModel>();
  m->impl->cfg = fc;
  m->impl->cfg.max_tokens = opt->max_tokens;
  m->impl->cfg.max_prefill_chunk = opt->max_prefill_chunk;
  m->impl->stream = rt->stream;
  const Status s = m->impl->LoadPackedCache(path, h.value());
  if (!s.ok()) return Ret(s);
  *out = m.release();
  return AM_STATUS_OK;
}

void am_model_destroy(am_model* m) {
  if (!m) return;
  (void)hipStreamSynchronize(m->rt->stream);
  delete m;
}

int64_t am_model_weight_bytes_total(am_model* m) { return m ? m->impl->linear_bytes : 0; }

am_status_code am_model_weight(am_model* m, int32_t layer, int32_t role, am_gfx950_weight* out) {
  if (!m || !out) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_weight: null argument");
  LlamaModel& M = *m->impl;
  if (role != AM_ROLE_LM_HEAD && (layer < 0 || layer >= M.cfg.num_layers))
    return am::SetLastError(AM_STATUS_OUT_OF_RANGE, "model_weight: layer out of range");
  const int64_t Q = M.QRows(), KV = M.KvRows(), F = M.cfg.ffn;
  const size_t l = static_cast<size_t>(layer);
  switch (role) {
    case AM_ROLE_QKV: *out = M.qkv[l]; break;
    case AM_ROLE_O: *out = M.o[l]; break;
    case AM_ROLE_GATE_UP: *out = M.gate_up[l]; break;
    case AM_ROLE_DOWN: *out = M.down[l]; break;
    case AM_ROLE_LM_HEAD: *out = M.lm_head; break;
    case AM_ROLE_Q: *out = M.RowView(M.qkv[l], 0, Q); break;
    case AM_ROLE_K: *out = M.RowView(M.qkv[l], Q, KV); break;
    case AM_ROLE_V: *out = M.RowView(M.qkv[l], Q + KV, KV); break;
    case AM_ROLE_GATE: *out = M.RowView(M.gate_up[l], 0, F); break;
    case AM_ROLE_UP: *out = M.RowView(M.gate_up[l], F, F); break;
    default: return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_weight: unknown role");
  }
  return AM_STATUS_OK;
}

am_status_code am_model_buffer(am_model* m, int32_t kind, int32_t layer, void** ptr, int64_t* bytes) {
  if (!m || !ptr || !bytes) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_buffer: null argument");
  LlamaModel& M = *m->impl;
  const int64_t ab = M.cfg.act_dtype == AM_DT_BF16 ? 2 : 4;
  const int64_t H = M.cfg.hidden;
  const bool per_layer = kind == AM_BUF_IN_NORM || kind == AM_BUF_POST_NORM;
  if (per_layer && (layer < 0 || layer >= M.cfg.num_layers))
    return am::SetLastError(AM_STATUS_OUT_OF_RANGE, "model_buffer: layer out of range");
  switch (kind) {
    case AM_BUF_EMBED: *ptr = M.embed; *bytes = static_cast<int64_t>(M.cfg.vocab) * H * ab; break;
    case AM_BUF_IN_NORM: *ptr = M.in_norm[static_cast<size_t>(layer)]; *bytes = H * ab; break;
    case AM_BUF_POST_NORM: *ptr = M.post_norm[static_cast<size_t>(layer)]; *bytes = H * ab; break;
    case AM_BUF_FINAL_NORM: *ptr = M.final_norm; *bytes = H * ab; break;
    case AM_BUF_ROPE_COS: *ptr = M.cos_tab; *bytes = static_cast<int64_t>(M.cfg.max_tokens) * (M.cfg.head_dim / 2) * 4; break;
    case AM_BUF_ROPE_SIN: *ptr = M.sin_tab; *bytes = static_cast<int64_t>(M.cfg.max_tokens) * (M.cfg.head_dim / 2) * 4; break;
    default: return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_buffer: unknown kind");
  }
  return AM_STATUS_OK;
}

am_status_code am_session_open(am_model* m, const am_session_options* opt, am_session** out) {
  if (!m || !out) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "session: null argument");
  auto s = std::make_unique<am_session>();
  s->impl = std::make_unique<LlamaSession>();
  const Status st = s->impl->Init(m->impl.get(), opt);
  if (!st.ok()) return Ret(st);
  *out = s.release();
  return AM_STATUS_OK;
}

void am_session_destroy(am_session* s) {
  if (!s) return;
  (void)hipStreamSynchronize(s->impl->stream);
  delete s;
}

am_status_code am_session_prefill(am_session* s, const int64_t* prompt, int64_t n, int64_t* first_token) {
  if (!s || !prompt) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "prefill: null argument");
  return Ret(s->impl->Prefill(0, prompt, n, first_token));
}

am_status_code am_session_prefill_row(am_session* s, int64_t row, const int64_t* prompt, int64_t n,
                                      int64_t* first_token) {
  if (!s || !prompt) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "prefill_row: null argument");
  return Ret(s->impl->Prefill(row, prompt, n, first_token));
}

int64_t am_session_batch(am_session* s) { return s ? s->impl->B : 0; }

am_status_code am_session_decode(am_session* s, int64_t n, int64_t* tokens_out) {
  if (!s || n < 0) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "decode: bad argument");
  if (n == 0) return AM_STATUS_OK;
  return Ret(s->impl->Decode(n, tokens_out));
}

am_status_code am_session_decode_async(am_session* s, int64_t n) {
  if (!s || n < 0) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "decode_async: bad argument");
  const Status st = s->impl->EnqueueDecode(n);
  if (st.ok()) s->impl->host_step += n;
  return Ret(st);
}

am_status_code am_session_generate_ids(am_session* s, const int64_t* prompt, int64_t n_prompt, int64_t max_new, int64_t eos,
                                   int64_t* tokens_out, int64_t* n_out) {
  if (!s || !prompt || !tokens_out || max_new <= 0) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "generate: bad argument");
  if (s->impl->B != 1) return am::SetLastError(AM_STATUS_UNIMPLEMENTED, "generate: single-sequence sessions only");
  int64_t first = 0;
  Status st = s->impl->Prefill(0, prompt, n_prompt, &first);
  if (!st.ok()) return Ret(st);
  tokens_out[0] = first;
  int64_t produced = 1;
  // EOS is checked every `chunk` steps: decode runs ahead without per-token syncs.
  const int64_t chunk = 16;
  while (produced < max_new && (eos < 0 || tokens_out[produced - 1] != eos)) {
    const int64_t n = std::min(chunk, max_new - produced);
    st = s->impl->Decode(n, tokens_out + produced);
    if (!st.ok()) return Ret(st);
    int64_t keep = n;
    if (eos >= 0)
      for (int64_t i = 0; i < n; ++i)
        if (tokens_out[produced + i] == eos) {
          keep = i + 1;
          break;
        }
    produced += keep;
    if (keep < n) break;
  }
  if (n_out) *n_out = produced;
  return AM_STATUS_OK;
}

am_status_code am_session_logits(am_session* s, float* out) {
  if (!s || !out) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "logits: null argument");
  auto& S = *s->impl;
  if (hipStreamSynchronize(S.stream) != hipSuccess ||
      hipMemcpy(out, S.logits, static_cast<size_t>(S.B * S.m->cfg.vocab) * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return am::SetLastError(AM_STATUS_INTERNAL, "logits copy failed");
  return AM_STATUS_OK;
}

int64_t am_session_position(am_session* s) { return s ? s->impl->host_pos() : -1; }

int64_t am_session_row_position(am_session* s, int64_t row) {
  if (!s || row < 0 || row >= s->impl->B) return -1;
  return s->impl->row_pos[static_cast<size_t>(row)];
}

int32_t am_session_persistent_decode(am_session* s) { return s && s->impl->persistent ? 1 : 0; }

int64_t am_session_decode_plan_size(am_session* s) {
  return s && s->impl->decode_plan ? static_cast<int64_t>(s->impl->decode_plan->size()) : 0;
}

am_status_code am_session_profile_decode(am_session* s, int64_t n, double* ms_by_op, int64_t* count_by_op) {
  if (!s || !ms_by_op || !count_by_op || n <= 0) return am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "profile: bad argument");
  return Ret(s->impl->Profile(n, ms_by_op, count_by_op));
}

// ---- the PRD's Phase-1 interface (aethermind_prd.md:298-320) over the calls above ----

am_runtime_t am_runtime_create(const am_config_t* config) {
  am_config_t c = DefaultConfig(0);
  if (config != nullptr) {
    // the first version of the struct ends before load_flags; later fields keep their
    // defaults when the caller's struct_size stops before them
    if (config->struct_size < offsetof(am_config_t, load_flags)) {
      (void)am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "am_config_t: struct_size too small");
      return nullptr;
    }
    std::memcpy(&c, config, std::min<size_t>(config->struct_size, sizeof(am_config_t)));
    c.struct_size = sizeof(am_config_t);
  }
  am_runtime* rt = nullptr;
  if (am_runtime_open(c.device, &rt) != AM_STATUS_OK) return nullptr;
  rt->config = c;
  return rt;
}

static void SetError(am_error_t* error, am_status_code code) {
  if (error != nullptr)
    *error = code == AM_STATUS_OK ? nullptr : am_gfx950_error_create(code, am_last_error_message());
}

am_model_t am_model_load(am_runtime_t runtime, const char* path, am_error_t* error) {
  if (error != nullptr) *error = nullptr;
  if (runtime == nullptr || path == nullptr) {
    SetError(error, am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "model_load: null runtime or path"));
    return nullptr;
  }
  const am_config_t& c = runtime->config;
  const am_model_load_options opt{c.act_dtype, c.weight_format, c.group_size, c.max_tokens, c.max_prefill_chunk};
  am_model* m = nullptr;
  const am_status_code rc = am_model_load_hf_ex(runtime, path, &opt, c.load_flags, &m);
  SetError(error, rc);
  return rc == AM_STATUS_OK ? m : nullptr;
}

void am_model_unload(am_model_t model) { am_model_destroy(model); }

am_session_t am_session_create(am_model_t model, const am_session_config_t* config) {
  if (config != nullptr && config->struct_size < sizeof(am_session_config_t)) {
    (void)am::SetLastError(AM_STATUS_INVALID_ARGUMENT, "am_session_config_t: struct_size too small");
    return nullptr;
  }
  const am_session_options opt{1, config != nullptr ? config->use_graph : 1, 1, 0};
  am_session* s = nullptr;
  if (am_session_open(model, &opt, &s) != AM_STATUS_OK) return nullptr;
  if (config != nullptr) {
    s->max_tokens = config->max_tokens;
    s->eos = config->eos_token_id;
  }
  return s;
}

int am_session_generate(am_session_t session, const uint32_t* input_tokens, size_t input_len,
                        uint32_t* output_tokens, size_t output_capacity, size_t* output_len,
                        am_error_t* error) {
  if (error != nullptr) *error = nullptr;
  if (output_len != nullptr) *output_len = 0;
  auto fail = [&](am_status_code code, const char* msg) {
    SetError(error, am::SetLastError(code, msg));
    return static_cast<int>(code);
  };
  if (session == nullptr || input_tokens == nullptr || output_tokens == nullptr || output_len == nullptr)
    return fail(AM_STATUS_INVALID_ARGUMENT, "generate: null argument");
  if (input_len == 0 || output_capacity == 0) return fail(AM_STATUS_INVALID_ARGUMENT, "generate: empty prompt or output");
  const int64_t cap = session->impl->m->cfg.max_tokens;
  if (input_len >= static_cast<size_t>(cap))
    return fail(AM_STATUS_OUT_OF_RANGE, "generate: the prompt leaves no KV capacity for a new token");
  // new tokens: the output capacity, the session's limit and the KV positions left
  // (the last generated token is never written to the cache)
  int64_t max_new = static_cast<int64_t>(std::min<size_t>(output_capacity, static_cast<size_t>(cap) - input_len));
  if (session->max_tokens > 0) max_new = std::min<int64_t>(max_new, session->max_tokens);
  std::vector<int64_t> prompt(input_tokens, input_tokens + input_len);
  std::vector<int64_t> out(static_cast<size_t>(max_new));
  int64_t n = 0;
  const am_status_code rc = am_session_generate_ids(session, prompt.data(), static_cast<int64_t>(input_len), max_new,
                                                    session->eos, out.data(), &n);
  if (rc != AM_STATUS_OK) {
    SetError(error, rc);
    return static_cast<int>(rc);
  }
  for (int64_t i = 0; i < n; ++i) output_tokens[i] = static_cast<uint32_t>(out[static_cast<size_t>(i)]);
  *output_len = static_cast<size_t>(n);
  return AM_STATUS_OK;
}

void am_error_free(am_error_t error) { am_gfx950_error_destroy(error); }

}  // extern "C"
