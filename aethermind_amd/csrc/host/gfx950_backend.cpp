// gfx950 backend KernelFuncs and their registrations.
//
// Registration mirrors the reference pattern (embedding_entry.cpp:142-158,
// rmsnorm_entry.cpp:193-227): one AM_REGISTER_KERNEL per (OpType, selector) with a
// params builder.  Selectors use DeviceType::kHIP and IsaLevel::kGfx950; Linear is
// registered per weight format and per phase (decode = GEMV, prefill = MFMA GEMM).

#include "gfx950_backend.h"

#include <cstring>

namespace aethermind::gfx950 {

namespace {

void* StreamOf(const KernelContext& ctx) {
  const auto* s = dynamic_cast<const HipStream*>(ctx.stream);
  return s ? s->native() : nullptr;
}

const GfxParams* P(const KernelContext& ctx) { return static_cast<const GfxParams*>(ctx.kernel_params); }

template <typename T>
bool ReadAttrs(const KernelContext& ctx, T* out) {
  if (ctx.attrs.size() != sizeof(T)) return false;
  std::memcpy(out, ctx.attrs.data(), sizeof(T));
  return true;
}

Status FromC(am_status_code c) { return Status::FromC(c, am_last_error_message()); }

Status NeedArgs(const GfxParams* p, int nin, int nout, const char* what) {
  if (p == nullptr) return Status::InvalidArgument(std::string(what) + " requires GfxParams in KernelContext.kernel_params");
  if (p->nin < nin || p->nout < nout) return Status::InvalidArgument(std::string(what) + ": wrong number of tensors");
  return Status::Ok();
}

const am_gfx950_weight* W(const KernelContext& ctx) { return static_cast<const am_gfx950_weight*>(ctx.packed_weights); }

// ---------------------------------------------------------------- per-op kernels
Status EmbeddingKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "EmbeddingKernel"));
  am_gfx950_embedding_args a{};
  a.ids = p->in[0].p;
  a.ids_dtype = p->in[0].dt;
  a.n_tokens = p->in[0].d[0];
  a.table = p->in[1].p;
  a.table_dtype = p->in[1].dt;
  a.vocab = p->in[1].d[0];
  a.hidden = p->in[1].d[1];
  a.out = p->out[0].p;
  a.out_dtype = p->out[0].dt;
  a.err_flag = p->nin > 2 ? static_cast<int32_t*>(p->in[2].p) : nullptr;
  a.check = 0;
  return FromC(am_gfx950_embedding(&a, StreamOf(ctx)));
}

Status EmbedTokenKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "EmbedTokenKernel"));
  return FromC(am_gfx950_embed_token(static_cast<const int64_t*>(p->in[0].p), p->in[1].p, p->in[1].dt,
                                     p->in[1].d[0], p->in[1].d[1], p->out[0].p,
                                     p->nin > 2 ? static_cast<int32_t*>(p->in[2].p) : nullptr, StreamOf(ctx)));
}

Status RmsNormKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "RmsNormKernel"));
  NormAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("RmsNormKernel requires eps in attrs");
  am_gfx950_rmsnorm_args a{};
  a.x = p->in[0].p;
  a.w = p->in[1].p;
  a.out = p->out[0].p;
  a.rows = p->in[0].d[0];
  a.hidden = p->in[0].d[1];
  a.x_stride = a.hidden;
  a.out_stride = a.hidden;
  a.eps = at.eps;
  a.x_dtype = p->in[0].dt;
  a.w_dtype = p->in[1].dt;
  a.out_dtype = p->out[0].dt;
  return FromC(am_gfx950_rmsnorm(&a, StreamOf(ctx)));
}

template <int MODE>
Status LinearKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 1, 1, "LinearKernel"));
  if (W(ctx) == nullptr) return Status::InvalidArgument("LinearKernel requires packed weights");
  am_gfx950_linear_args a{};
  a.x = p->in[0].p;
  a.x_dtype = p->in[0].dt;
  a.m = p->in[0].d[0];
  a.w = *W(ctx);
  a.out = p->out[0].p;
  a.out_dtype = p->out[0].dt;
  a.residual = p->nin > 1 ? p->in[1].p : nullptr;
  a.mode = MODE;
  if (p->out[0].d[1] != a.w.n || p->in[0].d[1] != a.w.k)
    return Status::InvalidArgument("LinearKernel: tensor shapes do not match the packed weight");
  return FromC(am_gfx950_linear(&a, StreamOf(ctx)));
}

Status RoPEKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 5, 2, "RoPEKernel"));
  RopeAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("RoPEKernel requires RopeAttrs");
  am_gfx950_rope_args a{};
  a.q = p->in[0].p;
  a.k = p->in[1].p;
  a.pos = static_cast<const int64_t*>(p->in[2].p);
  a.cos_tab = static_cast<const float*>(p->in[3].p);
  a.sin_tab = static_cast<const float*>(p->in[4].p);
  a.q_out = p->out[0].p;
  a.k_out = p->out[1].p;
  a.seq = p->in[0].d[0];
  a.hq = at.hq;
  a.hkv = at.hkv;
  a.head_dim = at.d;
  a.max_pos = at.max_pos;
  a.dtype = p->in[0].dt;
  return FromC(am_gfx950_rope(&a, StreamOf(ctx)));
}

am_gfx950_kv_pages PagesOf(const KvPaging& pg) {
  return am_gfx950_kv_pages{pg.table, pg.block, pg.stride, pg.num_blocks};
}

Status KVCacheUpdateKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 5, 0, "KVCacheUpdateKernel"));
  KvAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("KVCacheUpdateKernel requires KvAttrs");
  am_gfx950_kv_update_args a{};
  a.k = p->in[0].p;
  a.v = p->in[1].p;
  a.k_cache = p->in[2].p;
  a.v_cache = p->in[3].p;
  a.start_pos_dev = static_cast<const int64_t*>(p->in[4].p);
  a.seq = p->in[0].d[0];
  a.hkv = at.hkv;
  a.head_dim = at.d;
  a.capacity = at.cap;
  a.dtype = p->in[0].dt;
  const am_gfx950_kv_pages pages = PagesOf(at.pg);
  if (at.pg.table != nullptr) a.pages = &pages;
  return FromC(am_gfx950_kv_update(&a, StreamOf(ctx)));
}

Status AttentionKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 4, 1, "AttentionKernel"));
  AttnAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("AttentionKernel requires AttnAttrs");
  am_gfx950_attention_args a{};
  a.q = p->in[0].p;
  a.k_cache = p->in[1].p;
  a.v_cache = p->in[2].p;
  a.start_pos_dev = static_cast<const int64_t*>(p->in[3].p);
  a.out = p->out[0].p;
  a.seq = p->in[0].d[0];
  a.hq = at.hq;
  a.hkv = at.hkv;
  a.head_dim = at.d;
  a.capacity = at.cap;
  a.batch = 1;
  if (at.batch > 1) {
    if (a.seq % at.batch != 0) return Status::InvalidArgument("AttentionKernel: rows are not a whole batch");
    a.batch = at.batch;
    a.seq /= at.batch;
    a.cache_batch_stride = at.cbs;
  }
  a.dtype = p->in[0].dt;
  a.num_splits = at.splits;
  a.workspace = ctx.workspace_binding.data;
  a.workspace_bytes = static_cast<int64_t>(ctx.workspace_binding.size);
  const am_gfx950_kv_pages pages = PagesOf(at.pg);
  if (at.pg.table != nullptr) a.pages = &pages;
  return FromC(am_gfx950_attention(&a, StreamOf(ctx)));
}

Status AddKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "AddKernel"));
  am_gfx950_add_args a{p->in[0].p, p->in[1].p, p->out[0].p, p->out[0].d[0] * (p->out[0].rank > 1 ? p->out[0].d[1] : 1),
                       p->out[0].dt};
  return FromC(am_gfx950_add(&a, StreamOf(ctx)));
}

Status SiluMulKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "SiluMulKernel"));
  am_gfx950_silu_mul_args a{p->in[0].p, p->in[1].p, p->out[0].p,
                            p->out[0].d[0] * (p->out[0].rank > 1 ? p->out[0].d[1] : 1), p->out[0].dt};
  return FromC(am_gfx950_silu_mul(&a, StreamOf(ctx)));
}

// in[0] logits [rows, n], in[1] workspace (u8); out[0] ids [rows] (i64).  With a
// decode state bound (out[1..3] = tokens_hist, pos, step) the step also advances.
Status ArgmaxKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "ArgmaxKernel"));
  am_gfx950_argmax_args a{};
  a.x = p->in[0].p;
  a.dtype = p->in[0].dt;
  a.rows = p->in[0].rank > 1 ? p->in[0].d[0] : 1;
  a.n = p->in[0].rank > 1 ? p->in[0].d[1] : p->in[0].d[0];
  a.out = static_cast<int64_t*>(p->out[0].p);
  a.workspace = p->in[1].p;
  a.workspace_bytes = p->in[1].d[0];
  AM_RETURN_IF_ERROR(FromC(am_gfx950_argmax(&a, StreamOf(ctx))));
  if (p->nout >= 4)
    return FromC(am_gfx950_decode_advance(a.out, static_cast<int64_t*>(p->out[1].p), static_cast<int64_t*>(p->out[2].p),
                                          static_cast<int64_t*>(p->out[3].p), StreamOf(ctx)));
  return Status::Ok();
}

// ---------------------------------------------------------------- fused decode kernels
// in: h, norm_w, pos, cos, sin, k_plane, v_plane; out: q
Status FusedQkvKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 7, 1, "FusedRmsNormQkvRoPEKVUpdate"));
  QkvAttrs at{};
  if (!ReadAttrs(ctx, &at) || W(ctx) == nullptr) return Status::InvalidArgument("FusedQkv: attrs/weights missing");
  am_gfx950_fused_qkv_args a{};
  a.h = p->in[0].p;
  a.norm_w = p->in[1].p;
  a.eps = at.eps;
  a.w_qkv = *W(ctx);
  a.pos = static_cast<const int64_t*>(p->in[2].p);
  a.cos_tab = static_cast<const float*>(p->in[3].p);
  a.sin_tab = static_cast<const float*>(p->in[4].p);
  a.k_cache = p->in[5].p;
  a.v_cache = p->in[6].p;
  a.q_out = p->out[0].p;
  a.hq = at.hq;
  a.hkv = at.hkv;
  a.head_dim = at.d;
  a.capacity = at.cap;
  a.dtype = p->in[0].dt;
  a.rows = p->in[0].rank > 1 ? p->in[0].d[0] : 1;
  a.cache_batch_stride = at.cbs;
  const am_gfx950_kv_pages pages = PagesOf(at.pg);
  if (at.pg.table != nullptr) a.pages = &pages;
  return FromC(am_gfx950_fused_qkv(&a, StreamOf(ctx)));
}

// in: x; out: h (in/out residual)
Status FusedLinearAddKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 1, 1, "FusedLinearAdd"));
  if (W(ctx) == nullptr) return Status::InvalidArgument("FusedLinearAdd requires packed weights");
  am_gfx950_fused_linear_residual_args a{p->in[0].p, *W(ctx), p->out[0].p, p->out[0].dt,
                                         p->in[0].rank > 1 ? p->in[0].d[0] : 1};
  return FromC(am_gfx950_fused_linear_residual(&a, StreamOf(ctx)));
}

// Optional trailing input of the prefill GEMM ops: a u8 workspace [bytes] that lets the
// INT4 GEMM split K (am_gfx950_gemm_workspace_bytes).
void GemmWorkspace(const GfxParams* p, int index, void** ws, int64_t* bytes) {
  *ws = p->nin > index ? p->in[index].p : nullptr;
  *bytes = p->nin > index ? p->in[index].d[0] : 0;
}

// Prefill Linear -> Add on the MFMA GEMM: in: x (, workspace); out: h (in/out residual)
Status PrefillLinearAddKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 1, 1, "PrefillLinearAdd"));
  if (W(ctx) == nullptr) return Status::InvalidArgument("PrefillLinearAdd requires packed weights");
  am_gfx950_linear_args a{};
  a.x = p->in[0].p;
  a.x_dtype = p->in[0].dt;
  a.m = p->in[0].d[0];
  a.w = *W(ctx);
  a.out = p->out[0].p;
  a.out_dtype = p->out[0].dt;
  a.residual = p->out[0].p;
  a.mode = 2;
  GemmWorkspace(p, 1, &a.workspace, &a.workspace_bytes);
  if (p->out[0].d[1] != a.w.n || p->in[0].d[1] != a.w.k)
    return Status::InvalidArgument("PrefillLinearAdd: tensor shapes do not match the packed weight");
  return FromC(am_gfx950_linear(&a, StreamOf(ctx)));
}

// Prefill q|k|v: in: x (, workspace); out: the row ranges of the weight, in order (2 or 3 outputs)
Status FusedLinearSplitKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  if (p->nin < 1 || p->nout < 2 || p->nout > 3) return Status::InvalidArgument("FusedLinearSplit: needs 1 input, 2-3 outputs");
  if (W(ctx) == nullptr) return Status::InvalidArgument("FusedLinearSplit requires packed weights");
  am_gfx950_prefill_linear_args a{};
  a.x = p->in[0].p;
  a.m = p->in[0].d[0];
  a.w = *W(ctx);
  a.epilogue = AM_PREFILL_SPLIT;
  GemmWorkspace(p, 1, &a.workspace, &a.workspace_bytes);
  int64_t col = 0;
  for (int i = 0; i < p->nout; ++i) {
    a.out[i] = p->out[i].p;
    col += p->out[i].d[1];
    if (i < 2) a.split[i] = col;
  }
  if (p->nout == 2) a.split[1] = col;
  if (col != a.w.n || p->in[0].d[1] != a.w.k) return Status::InvalidArgument("FusedLinearSplit: outputs do not tile the weight rows");
  return FromC(am_gfx950_prefill_linear(&a, StreamOf(ctx)));
}

// Prefill q|k|v -> RoPE -> KVCacheUpdate (one sequence): in: x, cos, sin, start,
// k plane, v plane (, workspace); out: q [m][hq*d]
Status FusedLinearRoPEKVKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 6, 1, "FusedLinearRoPEKVUpdate"));
  if (W(ctx) == nullptr) return Status::InvalidArgument("FusedLinearRoPEKVUpdate requires packed weights");
  QkvAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("FusedLinearRoPEKVUpdate requires QkvAttrs");
  am_gfx950_prefill_rope_kv r{};
  r.cos_tab = static_cast<const float*>(p->in[1].p);
  r.sin_tab = static_cast<const float*>(p->in[2].p);
  r.max_pos = p->in[1].d[0];
  r.start_pos_dev = static_cast<const int64_t*>(p->in[3].p);
  r.k_cache = const_cast<void*>(p->in[4].p);
  r.v_cache = const_cast<void*>(p->in[5].p);
  r.hq = at.hq;
  r.hkv = at.hkv;
  r.head_dim = at.d;
  r.capacity = at.cap;
  const am_gfx950_kv_pages pages = PagesOf(at.pg);
  if (at.pg.table != nullptr) r.pages = &pages;
  am_gfx950_prefill_linear_args a{};
  a.x = p->in[0].p;
  a.m = p->in[0].d[0];
  a.w = *W(ctx);
  a.epilogue = AM_PREFILL_QKV_ROPE_KV;
  a.out[0] = p->out[0].p;
  a.rope_kv = &r;
  GemmWorkspace(p, 6, &a.workspace, &a.workspace_bytes);
  if (p->out[0].d[1] != at.hq * at.d || p->in[0].d[1] != a.w.k)
    return Status::InvalidArgument("FusedLinearRoPEKVUpdate: tensor shapes do not match the packed weight");
  return FromC(am_gfx950_prefill_linear(&a, StreamOf(ctx)));
}

// Prefill gate|up -> SiluMul: in: x (, workspace); out: act [m][n/2]
Status FusedLinearSiluMulKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 1, 1, "FusedLinearSiluMul"));
  if (W(ctx) == nullptr) return Status::InvalidArgument("FusedLinearSiluMul requires packed weights");
  am_gfx950_prefill_linear_args a{};
  a.x = p->in[0].p;
  a.m = p->in[0].d[0];
  a.w = *W(ctx);
  a.epilogue = AM_PREFILL_SILU_MUL;
  a.out[0] = p->out[0].p;
  GemmWorkspace(p, 1, &a.workspace, &a.workspace_bytes);
  if (2 * p->out[0].d[1] != a.w.n || p->in[0].d[1] != a.w.k)
    return Status::InvalidArgument("FusedLinearSiluMul: tensor shapes do not match the packed weight");
  return FromC(am_gfx950_prefill_linear(&a, StreamOf(ctx)));
}

// in: h, pos, cos, sin, layer table (device am_gfx950_decode_layer[layers]),
// workspace; out: h (the embedding in, the last layer's output out)
Status FusedDecodeLayersKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 6, 1, "FusedDecodeLayers"));
  DecodeLayersAttrs at{};
  if (!ReadAttrs(ctx, &at)) return Status::InvalidArgument("FusedDecodeLayers: attrs missing");
  am_gfx950_decode_layers_args a{};
  a.layers = static_cast<const am_gfx950_decode_layer*>(p->in[4].p);
  a.num_layers = at.layers;
  a.hidden = at.hidden;
  a.hq = at.hq;
  a.hkv = at.hkv;
  a.head_dim = at.d;
  a.ffn = at.ffn;
  a.capacity = at.cap;
  a.eps = at.eps;
  a.pos = static_cast<const int64_t*>(p->in[1].p);
  a.cos_tab = static_cast<const float*>(p->in[2].p);
  a.sin_tab = static_cast<const float*>(p->in[3].p);
  a.h = p->out[0].p;
  a.workspace = p->in[5].p;
  a.workspace_bytes = p->in[5].d[0];
  a.dtype = p->out[0].dt;
  return FromC(am_gfx950_decode_layers(&a, StreamOf(ctx)));
}

// in: h, norm_w; out: act
Status FusedGateUpKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 2, 1, "FusedRmsNormGateUpSiluMul"));
  NormAttrs at{};
  if (!ReadAttrs(ctx, &at) || W(ctx) == nullptr) return Status::InvalidArgument("FusedGateUp: attrs/weights missing");
  am_gfx950_fused_gate_up_args a{p->in[0].p, p->in[1].p, at.eps, *W(ctx), p->out[0].p, p->in[0].dt,
                                 p->in[0].rank > 1 ? p->in[0].d[0] : 1};
  return FromC(am_gfx950_fused_gate_up(&a, StreamOf(ctx)));
}

// in: h, norm_w, workspace; out: logits (f32, may be null), token, tokens_hist, pos, step
Status FusedLmHeadKernel(const KernelContext& ctx) noexcept {
  const GfxParams* p = P(ctx);
  AM_RETURN_IF_ERROR(NeedArgs(p, 3, 2, "FusedRmsNormLmHeadArgmax"));
  NormAttrs at{};
  if (!ReadAttrs(ctx, &at) || W(ctx) == nullptr) return Status::InvalidArgument("FusedLmHead: attrs/weights missing");
  am_gfx950_fused_lm_head_args a{};
  a.h = p->in[0].p;
  a.norm_w = p->in[1].p;
  a.eps = at.eps;
  a.w = *W(ctx);
  a.workspace = p->in[2].p;
  a.workspace_bytes = p->in[2].d[0];
  a.logits = static_cast<float*>(p->out[0].p);
  a.token_out = static_cast<int64_t*>(p->out[1].p);
  if (p->nout >= 5) {
    a.tokens_hist = static_cast<int64_t*>(p->out[2].p);
    a.pos = static_cast<int64_t*>(p->out[3].p);
    a.step = static_cast<int64_t*>(p->out[4].p);
    a.hist_stride = p->out[2].rank > 1 ? p->out[2].d[1] : 0;
  }
  a.dtype = p->in[0].dt;
  a.rows = p->in[0].rank > 1 ? p->in[0].d[0] : 1;
  return FromC(am_gfx950_fused_lm_head(&a, StreamOf(ctx)));
}

// ---------------------------------------------------------------- registrations
constexpr DataType kF32 = DataType::Float32();
constexpr DataType kBF16 = DataType::BFloat(16);
constexpr DataType kI8 = DataType::Int(8);
constexpr DataType kI4 = DataType::Int(4);

KernelDescriptor Desc(OpType op, KernelSelector sel, KernelFunc fn, const char* name, int prio = 100) {
  KernelDescriptor d;
  d.op_type = op;
  d.selector = sel;
  d.kernel_func = fn;
  d.name = name;
  d.priority = prio;
  d.params_builder = &BuildGfxParams;
  d.params_size = sizeof(GfxParams);
  return d;
}

}  // namespace

KernelSelector HipSelector(DataType act, DataType weight, WeightFormat fmt, ExecPhase phase) {
  KernelSelector s;
  s.device_type = DeviceType::kHIP;
  s.act_dtype = act;
  s.weight_dtype = weight;
  s.weight_format = fmt;
  s.isa = IsaLevel::kGfx950;
  s.phase = phase;
  return s;
}

Status BuildGfxParams(std::span<const TensorView> inputs, std::span<const MutableTensorView> outputs,
                      void* buffer) noexcept {
  if (inputs.size() > 7 || outputs.size() > 5) return Status::InvalidArgument("too many tensors for GfxParams");
  auto* p = ::new (buffer) GfxParams{};
  auto fill = [](ArgRef& r, const TensorView& t) {
    r.p = const_cast<void*>(t.data());
    r.dt = ToAmDtype(t.dtype());
    r.rank = t.rank();
    for (int i = 0; i < 3 && i < t.rank(); ++i) r.d[i] = t.dim(i);
  };
  for (size_t i = 0; i < inputs.size(); ++i) fill(p->in[i], inputs[i]);
  for (size_t i = 0; i < outputs.size(); ++i) fill(p->out[i], outputs[i]);
  p->nin = static_cast<int32_t>(inputs.size());
  p->nout = static_cast<int32_t>(outputs.size());
  return Status::Ok();
}

// ---------------------------------------------------------------- backend
Gfx950Backend::Gfx950Backend() {
  // Like CpuBackend (cpu_backend.cpp:7-10): the first backend freezes the global
  // registry, so every static registration above has already happened.
  (void)KernelRegistry::Global().Freeze();
}

KernelFunc Gfx950Backend::ResolveKernel(OpType op, const KernelSelector& sel) const noexcept {
  auto r = ResolveKernelInfo(op, sel);
  return r.ok() ? r->fn : nullptr;
}

StatusOr<ResolvedKernel> Gfx950Backend::ResolveKernelInfo(OpType op, const KernelSelector& sel) const noexcept {
  if (sel.device_type != DeviceType::kHIP) return Status::InvalidArgument("Gfx950Backend only resolves HIP selectors");
  auto d = KernelRegistry::Global().Resolve(op, sel);
  if (!d.ok()) return d.status();
  ResolvedKernel rk;
  rk.op_type = op;
  rk.fn = d.value()->kernel_func;
  rk.debug_name = d.value()->name.c_str();
  rk.params_builder = d.value()->params_builder;
  rk.params_size = d.value()->params_size;
  return rk;
}

Status DeviceOperator::Prepare(Backend& backend, const KernelSelector& selector) {
  auto r = backend.ResolveKernelInfo(type_, selector);
  if (!r.ok()) return r.status();
  resolved_ = std::move(r.value());
  resolved_.attrs = attrs_;
  return Status::Ok();
}

Status DeviceOperator::Run(KernelContext& ctx, const RuntimeBindingContext& bindings, size_t step_index) const noexcept {
  if (resolved_.fn == nullptr) return Status::FailedPrecondition("Operator Run called before Prepare");
  auto b = bindings.GetStepTensorBinding(step_index);
  if (!b.ok()) return b.status();
  return InvokeResolvedKernel(ctx, (*b)->inputs, (*b)->outputs);
}

}  // namespace aethermind::gfx950

// ---- registrations (static initialisation; the registry is frozen by the first backend) ----
namespace aethermind::gfx950 {
namespace {
using WF = WeightFormat;
using EP = ExecPhase;
}  // namespace
}  // namespace aethermind::gfx950

#define AM_GFX_REG(NAME, ...) AM_REGISTER_KERNEL(NAME, ::aethermind::gfx950::__VA_ARGS__)

namespace aethermind::gfx950 {
namespace {
// Embedding / EmbedToken: weight dtype = table dtype.
AM_REGISTER_KERNEL(HipEmbeddingF32, Desc(OpType::kEmbedding, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &EmbeddingKernel, "gfx950::embedding_f32"))
AM_REGISTER_KERNEL(HipEmbeddingBF16, Desc(OpType::kEmbedding, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &EmbeddingKernel, "gfx950::embedding_bf16"))
AM_REGISTER_KERNEL(HipEmbedTokenF32, Desc(OpType::kEmbedToken, HipSelector(kF32, kF32, WF::kPlain, EP::kDecode), &EmbedTokenKernel, "gfx950::embed_token_f32"))
AM_REGISTER_KERNEL(HipEmbedTokenBF16, Desc(OpType::kEmbedToken, HipSelector(kBF16, kBF16, WF::kPlain, EP::kDecode), &EmbedTokenKernel, "gfx950::embed_token_bf16"))
// RmsNorm (rmsnorm_entry.cpp:193-227 registers the CPU fp32 forms).
AM_REGISTER_KERNEL(HipRmsNormF32, Desc(OpType::kRmsNorm, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &RmsNormKernel, "gfx950::rmsnorm_f32"))
AM_REGISTER_KERNEL(HipRmsNormBF16, Desc(OpType::kRmsNorm, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &RmsNormKernel, "gfx950::rmsnorm_bf16"))
// Linear: decode = GEMV, prefill = MFMA GEMM (GEMV rows for fp32 activations).
AM_REGISTER_KERNEL(HipLinDecF32F32, Desc(OpType::kLinear, HipSelector(kF32, kF32, WF::kPlain, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_f32_f32"))
AM_REGISTER_KERNEL(HipLinDecF32BF16, Desc(OpType::kLinear, HipSelector(kF32, kBF16, WF::kPlain, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_f32_bf16"))
AM_REGISTER_KERNEL(HipLinDecF32I8, Desc(OpType::kLinear, HipSelector(kF32, kI8, WF::kQuantizedInt8, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_f32_int8"))
AM_REGISTER_KERNEL(HipLinDecF32I4, Desc(OpType::kLinear, HipSelector(kF32, kI4, WF::kQuantizedInt4, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_f32_int4"))
AM_REGISTER_KERNEL(HipLinDecBF16BF16, Desc(OpType::kLinear, HipSelector(kBF16, kBF16, WF::kPlain, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_bf16_bf16"))
AM_REGISTER_KERNEL(HipLinDecBF16I8, Desc(OpType::kLinear, HipSelector(kBF16, kI8, WF::kQuantizedInt8, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_bf16_int8"))
AM_REGISTER_KERNEL(HipLinDecBF16I4, Desc(OpType::kLinear, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kDecode), &LinearKernel<1>, "gfx950::gemv_bf16_int4"))
AM_REGISTER_KERNEL(HipLinPreF32F32, Desc(OpType::kLinear, HipSelector(kF32, kF32, WF::kPlain, EP::kPrefill), &LinearKernel<0>, "gfx950::linear_rows_f32_f32"))
AM_REGISTER_KERNEL(HipLinPreF32BF16, Desc(OpType::kLinear, HipSelector(kF32, kBF16, WF::kPlain, EP::kPrefill), &LinearKernel<0>, "gfx950::linear_rows_f32_bf16"))
AM_REGISTER_KERNEL(HipLinPreF32I8, Desc(OpType::kLinear, HipSelector(kF32, kI8, WF::kQuantizedInt8, EP::kPrefill), &LinearKernel<0>, "gfx950::linear_rows_f32_int8"))
AM_REGISTER_KERNEL(HipLinPreF32I4, Desc(OpType::kLinear, HipSelector(kF32, kI4, WF::kQuantizedInt4, EP::kPrefill), &LinearKernel<0>, "gfx950::linear_rows_f32_int4"))
AM_REGISTER_KERNEL(HipLinPreBF16BF16, Desc(OpType::kLinear, HipSelector(kBF16, kBF16, WF::kPlain, EP::kPrefill), &LinearKernel<0>, "gfx950::gemm_mfma_bf16_bf16"))
AM_REGISTER_KERNEL(HipLinPreBF16I8, Desc(OpType::kLinear, HipSelector(kBF16, kI8, WF::kQuantizedInt8, EP::kPrefill), &LinearKernel<0>, "gfx950::gemm_mfma_bf16_int8"))
AM_REGISTER_KERNEL(HipLinPreBF16I4, Desc(OpType::kLinear, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kPrefill), &LinearKernel<0>, "gfx950::gemm_mfma_bf16_int4"))
// RoPE / KVCacheUpdate / Attention / Add / SiluMul / Argmax
AM_REGISTER_KERNEL(HipRoPEF32, Desc(OpType::kRoPE, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &RoPEKernel, "gfx950::rope_f32"))
AM_REGISTER_KERNEL(HipRoPEBF16, Desc(OpType::kRoPE, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &RoPEKernel, "gfx950::rope_bf16"))
AM_REGISTER_KERNEL(HipKVF32, Desc(OpType::kKVCacheUpdate, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &KVCacheUpdateKernel, "gfx950::kv_update_f32"))
AM_REGISTER_KERNEL(HipKVBF16, Desc(OpType::kKVCacheUpdate, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &KVCacheUpdateKernel, "gfx950::kv_update_bf16"))
AM_REGISTER_KERNEL(HipAttnF32, Desc(OpType::kAttention, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &AttentionKernel, "gfx950::gqa_attention_f32"))
AM_REGISTER_KERNEL(HipAttnBF16, Desc(OpType::kAttention, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &AttentionKernel, "gfx950::gqa_attention_bf16"))
AM_REGISTER_KERNEL(HipAddF32, Desc(OpType::kAdd, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &AddKernel, "gfx950::add_f32"))
AM_REGISTER_KERNEL(HipAddBF16, Desc(OpType::kAdd, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &AddKernel, "gfx950::add_bf16"))
AM_REGISTER_KERNEL(HipSiluMulF32, Desc(OpType::kSiluMul, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &SiluMulKernel, "gfx950::silu_mul_f32"))
AM_REGISTER_KERNEL(HipSiluMulBF16, Desc(OpType::kSiluMul, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &SiluMulKernel, "gfx950::silu_mul_bf16"))
AM_REGISTER_KERNEL(HipArgmaxF32, Desc(OpType::kArgmax, HipSelector(kF32, kF32, WF::kPlain, EP::kBoth), &ArgmaxKernel, "gfx950::argmax_f32"))
AM_REGISTER_KERNEL(HipArgmaxBF16, Desc(OpType::kArgmax, HipSelector(kBF16, kBF16, WF::kPlain, EP::kBoth), &ArgmaxKernel, "gfx950::argmax_bf16"))
}  // namespace

#define AM_FUSED_REGS(TAG, ACT, WT, FMT)                                                                              \
  AM_REGISTER_KERNEL(HipQkv##TAG, Desc(OpType::kFusedRmsNormQkvRoPEKVUpdate, HipSelector(ACT, WT, FMT, EP::kDecode),  \
                                       &FusedQkvKernel, "gfx950::fused_norm_qkv_rope_kv_" #TAG))                      \
  AM_REGISTER_KERNEL(HipLinAdd##TAG, Desc(OpType::kFusedLinearAdd, HipSelector(ACT, WT, FMT, EP::kDecode),            \
                                          &FusedLinearAddKernel, "gfx950::fused_gemv_add_" #TAG))                     \
  AM_REGISTER_KERNEL(HipGateUp##TAG, Desc(OpType::kFusedRmsNormGateUpSiluMul, HipSelector(ACT, WT, FMT, EP::kDecode), \
                                          &FusedGateUpKernel, "gfx950::fused_norm_gateup_silu_" #TAG))                \
  AM_REGISTER_KERNEL(HipLmHead##TAG, Desc(OpType::kFusedRmsNormLmHeadArgmax, HipSelector(ACT, WT, FMT, EP::kDecode),  \
                                          &FusedLmHeadKernel, "gfx950::fused_norm_lmhead_argmax_" #TAG))

namespace {
AM_REGISTER_KERNEL(HipDecodeLayersBF16I4, Desc(OpType::kFusedDecodeLayers, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kDecode),
                                             &FusedDecodeLayersKernel, "gfx950::persistent_decode_layers_bf16_int4"))
AM_FUSED_REGS(f32_f32, kF32, kF32, WF::kPlain)
AM_FUSED_REGS(f32_bf16, kF32, kBF16, WF::kPlain)
AM_FUSED_REGS(f32_int8, kF32, kI8, WF::kQuantizedInt8)
AM_FUSED_REGS(f32_int4, kF32, kI4, WF::kQuantizedInt4)
AM_FUSED_REGS(bf16_bf16, kBF16, kBF16, WF::kPlain)
AM_FUSED_REGS(bf16_int8, kBF16, kI8, WF::kQuantizedInt8)
AM_FUSED_REGS(bf16_int4, kBF16, kI4, WF::kQuantizedInt4)
AM_REGISTER_KERNEL(HipPreLinAddBF16I4, Desc(OpType::kFusedLinearAdd, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kPrefill),
                                            &PrefillLinearAddKernel, "gfx950::gemm_add_bf16_int4"))
AM_REGISTER_KERNEL(HipPreSplitBF16I4, Desc(OpType::kFusedLinearSplit, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kPrefill),
                                           &FusedLinearSplitKernel, "gfx950::gemm_split_bf16_int4"))
AM_REGISTER_KERNEL(HipPreQkvRopeBF16I4, Desc(OpType::kFusedLinearRoPEKVUpdate, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kPrefill),
                                             &FusedLinearRoPEKVKernel, "gfx950::gemm_qkv_rope_kv_bf16_int4"))
AM_REGISTER_KERNEL(HipPreSiluBF16I4, Desc(OpType::kFusedLinearSiluMul, HipSelector(kBF16, kI4, WF::kQuantizedInt4, EP::kPrefill),
                                          &FusedLinearSiluMulKernel, "gfx950::gemm_silu_mul_bf16_int4"))
// the same prefill fusions for INT8 per-channel and bf16 weights (one GEMM kernel template)
#define AM_PREFILL_REGS(TAG, WT, FMT)                                                                                  \
  AM_REGISTER_KERNEL(HipPreLinAdd##TAG, Desc(OpType::kFusedLinearAdd, HipSelector(kBF16, WT, FMT, EP::kPrefill),        \
                                             &PrefillLinearAddKernel, "gfx950::gemm_add_" #TAG))                      \
  AM_REGISTER_KERNEL(HipPreSplit##TAG, Desc(OpType::kFusedLinearSplit, HipSelector(kBF16, WT, FMT, EP::kPrefill),       \
                                            &FusedLinearSplitKernel, "gfx950::gemm_split_" #TAG))                     \
  AM_REGISTER_KERNEL(HipPreQkvRope##TAG, Desc(OpType::kFusedLinearRoPEKVUpdate, HipSelector(kBF16, WT, FMT, EP::kPrefill), \
                                              &FusedLinearRoPEKVKernel, "gfx950::gemm_qkv_rope_kv_" #TAG))            \
  AM_REGISTER_KERNEL(HipPreSilu##TAG, Desc(OpType::kFusedLinearSiluMul, HipSelector(kBF16, WT, FMT, EP::kPrefill),      \
                                           &FusedLinearSiluMulKernel, "gfx950::gemm_silu_mul_" #TAG))
AM_PREFILL_REGS(bf16_int8, kI8, WF::kQuantizedInt8)
AM_PREFILL_REGS(bf16_bf16, kBF16, WF::kPlain)
}  // namespace

}  // namespace aethermind::gfx950
