// Per-op gfx950 kernels for the unfused (one kernel per reference node) path:
// Embedding, RmsNorm, RoPE, KVCacheUpdate, SiluMul, Add, Argmax, plus fills.
// All of them are HBM-bound streaming kernels: 16-byte vector accesses where the
// row length allows, one block per row for the row reductions.

#include <algorithm>
#include <cmath>

#include "am_kernel_common.h"
#include "am_launch_timing.h"

namespace am {
namespace {

// ---------------- Embedding ----------------
template <class Out, class Tab, typename Id>
__global__ __launch_bounds__(256) void embedding_kernel(const Id* ids, int64_t n_tokens,
                                                        const typename Tab::T* table, int64_t vocab,
                                                        int64_t hidden, typename Out::T* out,
                                                        int32_t* err) {
  const int64_t t = blockIdx.y;
  const int64_t id = static_cast<int64_t>(ids[t]);
  const bool ok = id >= 0 && id < vocab;
  if (!ok && err != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *err = 1;
  for (int64_t j = blockIdx.x * 256 + threadIdx.x; j < hidden; j += gridDim.x * 256) {
    const float v = ok ? Tab::load(table, id * hidden + j) : 0.0f;
    Out::store(out, t * hidden + j, v);
  }
}

template <class A>
__global__ __launch_bounds__(256) void embed_token_kernel(const int64_t* token, const typename A::T* table,
                                                          int64_t vocab, int64_t hidden,
                                                          typename A::T* h, int32_t* err) {
  const int64_t id = *token;
  const bool ok = id >= 0 && id < vocab;
  if (!ok && err != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *err = 1;
  for (int64_t j = blockIdx.x * 256 + threadIdx.x; j < hidden; j += gridDim.x * 256)
    h[j] = ok ? table[id * hidden + j] : typename A::T(0);
}

// ---------------- RMSNorm ----------------
template <class X, class W, class O>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const typename X::T* x, const typename W::T* w,
                                                      typename O::T* out, int64_t hidden,
                                                      int64_t xs, int64_t os, float eps) {
  __shared__ float red[4];
  const typename X::T* xr = x + blockIdx.x * xs;
  typename O::T* orow = out + blockIdx.x * os;
  float ss = 0.0f;
  for (int64_t j = threadIdx.x; j < hidden; j += 256) {
    const float v = X::load(xr, j);
    ss = fmaf(v, v, ss);
  }
  ss = block_sum_256(ss, red);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(hidden) + eps);
  for (int64_t j = threadIdx.x; j < hidden; j += 256)
    O::store(orow, j, (X::load(xr, j) * inv) * W::load(w, j));
}

// bf16 rows with hidden = 512 NV (prefill): one wave per row, the row and the gain
// held in registers as NV 16-byte pieces per lane, all loads issued at once; 16-byte
// stores.  The same formula and roundings as rmsnorm_kernel.
template <int NV>
__global__ __launch_bounds__(256) void rmsnorm_rows_bf16_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out,
                                                                int32_t rows, int64_t xs, int64_t os, float eps) {
  const int lane = threadIdx.x & 63;
  const int32_t row = static_cast<int32_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * xs);
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4 xv[NV], wv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) xv[v] = xr[lane + 64 * v];
#pragma unroll
  for (int v = 0; v < NV; ++v) wv[v] = wr[lane + 64 * v];
  float ss = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const uint32_t q[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float a = bf16_bits_to_f32(q[t] & 0xFFFFu), b = bf16_bits_to_f32(q[t] >> 16);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(NV * 512) + eps);
  uint4* orow = reinterpret_cast<uint4*>(out + row * os);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const uint32_t q[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
    const uint32_t g[4] = {wv[v].x, wv[v].y, wv[v].z, wv[v].w};
    uint32_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float lo = (bf16_bits_to_f32(q[t] & 0xFFFFu) * inv) * bf16_bits_to_f32(g[t] & 0xFFFFu);
      const float hi = (bf16_bits_to_f32(q[t] >> 16) * inv) * bf16_bits_to_f32(g[t] >> 16);
      o[t] = f32_to_bf16_bits(lo) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
    }
    orow[lane + 64 * v] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------- RoPE ----------------
// One thread per (token, head, i < d/2) pair: out[i] = x1 c - x2 s, out[i+d/2] = x2 c + x1 s.
template <class A>
__global__ __launch_bounds__(256) void rope_kernel(const typename A::T* x, typename A::T* out,
                                                   const int64_t* pos, const float* cos_tab,
                                                   const float* sin_tab, int64_t seq, int64_t heads,
                                                   int64_t d, int64_t max_pos, int32_t* bad) {
  const int64_t half = d / 2;
  const int64_t total = seq * heads * half;
  for (int64_t idx = blockIdx.x * 256 + threadIdx.x; idx < total; idx += gridDim.x * 256) {
    const int64_t i = idx % half;
    const int64_t sh = idx / half;  // s*heads + h
    const int64_t s = sh / heads;
    const int64_t p = pos[s];
    const int64_t base = sh * d;
    const float x1 = A::load(x, base + i);
    const float x2 = A::load(x, base + i + half);
    if (p < 0 || p >= max_pos) {
      if (bad != nullptr) *bad = 1;
      A::store(out, base + i, x1);
      A::store(out, base + i + half, x2);
      continue;
    }
    const float c = cos_tab[p * half + i];
    const float sn = sin_tab[p * half + i];
    float y1, y2;
    rope_rotate(x1, x2, c, sn, y1, y2);
    A::store(out, base + i, y1);
    A::store(out, base + i + half, y2);
  }
}

// ---------------- KV cache update ----------------
// 16-byte granules of one row of one head; cache plane [hkv][cap][d].
__global__ __launch_bounds__(256) void kv_update_kernel(const uint8_t* k, const uint8_t* v, uint8_t* kc,
                                                        uint8_t* vc, int64_t seq, int64_t hkv,
                                                        int64_t row_bytes, int64_t cap,
                                                        int64_t start, const int64_t* start_dev,
                                                        int32_t* err, KvRows kv, int64_t esz) {
  const int64_t st = start_dev != nullptr ? *start_dev : start;
  const int64_t g16 = row_bytes / 16;
  const int64_t total = seq * hkv * g16;
  for (int64_t idx = blockIdx.x * 256 + threadIdx.x; idx < total; idx += gridDim.x * 256) {
    const int64_t c = idx % g16;
    const int64_t sh = idx / g16;
    const int64_t h = sh % hkv;
    const int64_t s = sh / hkv;
    const int64_t p = st + s;
    if (p < 0 || p >= cap) {
      if (err != nullptr) *err = 1;
      continue;
    }
    const int64_t src = (s * hkv + h) * row_bytes + c * 16;
    const int64_t row = kv.WriteRow(0, h, p);
    if (row < 0) continue;
    const int64_t dst = row * esz + c * 16;
    *reinterpret_cast<uint4*>(kc + dst) = *reinterpret_cast<const uint4*>(k + src);
    *reinterpret_cast<uint4*>(vc + dst) = *reinterpret_cast<const uint4*>(v + src);
  }
}

// ---------------- SiluMul / Add ----------------
__device__ __forceinline__ float silu_ref(float g) {
  // const_eval_silu_mul.cpp:18-31: branch on the sign to avoid exp overflow.
  if (g >= 0.0f) return g / (1.0f + expf(-g));
  const float e = expf(g);
  return g * e / (1.0f + e);
}

template <class A>
__global__ __launch_bounds__(256) void silu_mul_kernel(const typename A::T* g, const typename A::T* u,
                                                       typename A::T* out, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    A::store(out, i, silu_ref(A::load(g, i)) * A::load(u, i));
}

template <class A>
__global__ __launch_bounds__(256) void add_kernel(const typename A::T* a, const typename A::T* b,
                                                  typename A::T* out, int64_t n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256)
    A::store(out, i, A::load(a, i) + A::load(b, i));
}

template <class A>
__global__ __launch_bounds__(256) void fill_kernel(typename A::T* out, int64_t n, float v) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) A::store(out, i, v);
}

// ---------------- Argmax ----------------
// grid (blocks_per_row, rows).  Each block reduces a slice, writes (value, index)
// to the workspace; the last block of a row (atomic ticket) reduces the partials
// and resets the ticket to zero for the next call.
struct ArgmaxWs {
  static constexpr int kMaxBlocks = 64;
};

template <class A>
__global__ __launch_bounds__(256) void argmax_kernel(const typename A::T* x, int64_t n, int64_t* out,
                                                     unsigned* tickets, float* pv, int64_t* pi) {
  __shared__ float sv[4];
  __shared__ int64_t si[4];
  __shared__ bool last;
  const int64_t r = blockIdx.y;
  const int nb = gridDim.x;
  const typename A::T* row = x + r * n;
  float bv = 0.0f;
  int64_t bi = -1;
  for (int64_t j = blockIdx.x * 256 + threadIdx.x; j < n; j += static_cast<int64_t>(nb) * 256) {
    const float v = A::load(row, j);
    if (argmax_better(v, j, bv, bi)) {
      bv = v;
      bi = j;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (oi >= 0 && argmax_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      if (si[w] >= 0 && argmax_better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    // device-coherent (sc1) stores, acknowledged before the relaxed ticket: the last
    // block's device-coherent loads then see every block's partial
    __hip_atomic_store(&pv[r * ArgmaxWs::kMaxBlocks + blockIdx.x], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&pi[r * ArgmaxWs::kMaxBlocks + blockIdx.x], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned t = __hip_atomic_fetch_add(&tickets[r], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = (t == static_cast<unsigned>(nb - 1));
  }
  __syncthreads();
  if (last && threadIdx.x == 0) {
    float fv = 0.0f;
    int64_t fi = -1;
    for (int b = 0; b < nb; ++b) {
      const float v = __hip_atomic_load(&pv[r * ArgmaxWs::kMaxBlocks + b], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      const int64_t i = __hip_atomic_load(&pi[r * ArgmaxWs::kMaxBlocks + b], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      if (i >= 0 && argmax_better(v, i, fv, fi)) {
        fv = v;
        fi = i;
      }
    }
    out[r] = fi < 0 ? 0 : fi;
    tickets[r] = 0u;
  }
}

int GridFor(int64_t n, int64_t per_block = 256, int64_t cap = 4096) {
  int64_t g = CeilDiv(n, per_block);
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

bool IsAct(int32_t dt) { return dt == AM_DT_F32 || dt == AM_DT_BF16; }

}  // namespace
}  // namespace am

using namespace am;

extern "C" am_status_code am_gfx950_embedding(const am_gfx950_embedding_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "embedding: null args");
  AM_CHECK_ARG(a->ids_dtype == AM_DT_I32 || a->ids_dtype == AM_DT_I64 || a->ids_dtype == AM_DT_U32,
               "embedding: token ids must be int32, int64, or uint32");
  AM_CHECK_ARG(IsAct(a->table_dtype) && IsAct(a->out_dtype), "embedding: table/out dtype must be f32 or bf16");
  AM_CHECK_ARG(a->vocab > 0 && a->hidden > 0, "embedding: requires positive vocab and hidden sizes");
  AM_CHECK_ARG(a->n_tokens >= 0 && a->n_tokens <= 65535, "embedding: token count out of range");
  if (a->n_tokens == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->ids && a->table && a->out, "embedding: null data pointer");
  hipStream_t s = AsStream(stream);
  int32_t* err = a->err_flag;
  if (a->check && err == nullptr) return SetLastError(AM_STATUS_INVALID_ARGUMENT, "embedding: check needs err_flag");
  if (a->check) {
    if (hipMemsetAsync(err, 0, sizeof(int32_t), s) != hipSuccess)
      return SetLastError(AM_STATUS_INTERNAL, "embedding: memset failed");
  }
  dim3 grid(static_cast<unsigned>(CeilDiv(a->hidden, 256 * 4)), static_cast<unsigned>(a->n_tokens));
#define AM_EMB(OUT, TAB, ID)                                                                    \
  hipLaunchKernelGGL((embedding_kernel<OUT, TAB, ID>), grid, dim3(256), 0, s,                 \
                     static_cast<const ID*>(a->ids), a->n_tokens,                              \
                     static_cast<const TAB::T*>(a->table), a->vocab, a->hidden,                \
                     static_cast<OUT::T*>(a->out), err)
#define AM_EMB_ID(OUT, TAB)                                                  \
  if (a->ids_dtype == AM_DT_I64) AM_EMB(OUT, TAB, int64_t);                  \
  else if (a->ids_dtype == AM_DT_I32) AM_EMB(OUT, TAB, int32_t);             \
  else AM_EMB(OUT, TAB, uint32_t)
  if (a->out_dtype == AM_DT_F32) {
    if (a->table_dtype == AM_DT_F32) { AM_EMB_ID(ActF32, ActF32); } else { AM_EMB_ID(ActF32, ActBF16); }
  } else {
    if (a->table_dtype == AM_DT_F32) { AM_EMB_ID(ActBF16, ActF32); } else { AM_EMB_ID(ActBF16, ActBF16); }
  }
#undef AM_EMB_ID
#undef AM_EMB
  AM_RETURN_IF_LAUNCH_FAILED("embedding");
  if (a->check) {
    int32_t host_flag = 0;
    if (hipMemcpyAsync(&host_flag, err, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
      return SetLastError(AM_STATUS_INTERNAL, "embedding: flag readback failed");
    if (host_flag != 0)
      return SetLastError(AM_STATUS_OUT_OF_RANGE, "EmbeddingKernel token id is out of vocabulary range");
  }
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_embed_token(const int64_t* token, const void* table, int32_t dtype,
                                                int64_t vocab, int64_t hidden, void* h, int32_t* err,
                                                void* stream) {
  AM_CHECK_ARG(token && table && h && vocab > 0 && hidden > 0 && IsAct(dtype), "embed_token: bad args");
  const dim3 grid(static_cast<unsigned>(CeilDiv(hidden, 256 * 4)));
  if (dtype == AM_DT_F32)
    hipLaunchKernelGGL(embed_token_kernel<ActF32>, grid, dim3(256), 0, AsStream(stream), token,
                       static_cast<const float*>(table), vocab, hidden, static_cast<float*>(h), err);
  else
    hipLaunchKernelGGL(embed_token_kernel<ActBF16>, grid, dim3(256), 0, AsStream(stream), token,
                       static_cast<const uint16_t*>(table), vocab, hidden, static_cast<uint16_t*>(h), err);
  AM_RETURN_IF_LAUNCH_FAILED("embed_token");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_rmsnorm(const am_gfx950_rmsnorm_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "rmsnorm: null args");
  AM_CHECK_ARG(IsAct(a->x_dtype) && IsAct(a->w_dtype) && IsAct(a->out_dtype), "rmsnorm: dtype must be f32 or bf16");
  AM_CHECK_ARG(a->rows >= 0 && a->hidden > 0, "rmsnorm: requires positive hidden size");
  AM_CHECK_ARG(a->eps > 0.0f && std::isfinite(a->eps), "rmsnorm: eps must be finite and positive");
  AM_CHECK_ARG(a->x_stride >= a->hidden && a->out_stride >= a->hidden, "rmsnorm: row stride smaller than hidden");
  AM_CHECK_ARG(a->rows <= 0x7FFFFFFF, "rmsnorm: too many rows");
  if (a->rows == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->x && a->w && a->out, "rmsnorm: null data pointer");
  hipStream_t s = AsStream(stream);
  // bf16 rows of 512, 1024, 2048, 4096 or 8192 values, 16-byte aligned: the wave-per-row kernel
  const int64_t nv = a->hidden / 512;
  const bool aligned = ((reinterpret_cast<uintptr_t>(a->x) | reinterpret_cast<uintptr_t>(a->w) |
                         reinterpret_cast<uintptr_t>(a->out)) & 15u) == 0 && a->x_stride % 8 == 0 && a->out_stride % 8 == 0;
  if (a->x_dtype == AM_DT_BF16 && a->w_dtype == AM_DT_BF16 && a->out_dtype == AM_DT_BF16 && aligned &&
      a->hidden % 512 == 0 && (nv == 1 || nv == 2 || nv == 4 || nv == 8 || nv == 16) &&
      a->rows * std::max(a->x_stride, a->out_stride) < (int64_t{1} << 31)) {
    const dim3 g4(static_cast<unsigned>(CeilDiv(a->rows, 4)));
    const auto* xp = static_cast<const uint16_t*>(a->x);
    const auto* wp = static_cast<const uint16_t*>(a->w);
    auto* op = static_cast<uint16_t*>(a->out);
    const int32_t rows = static_cast<int32_t>(a->rows);
    switch (nv) {
      case 1: hipLaunchKernelGGL(rmsnorm_rows_bf16_kernel<1>, g4, dim3(256), 0, s, xp, wp, op, rows, a->x_stride, a->out_stride, a->eps); break;
      case 2: hipLaunchKernelGGL(rmsnorm_rows_bf16_kernel<2>, g4, dim3(256), 0, s, xp, wp, op, rows, a->x_stride, a->out_stride, a->eps); break;
      case 4: hipLaunchKernelGGL(rmsnorm_rows_bf16_kernel<4>, g4, dim3(256), 0, s, xp, wp, op, rows, a->x_stride, a->out_stride, a->eps); break;
      case 8: hipLaunchKernelGGL(rmsnorm_rows_bf16_kernel<8>, g4, dim3(256), 0, s, xp, wp, op, rows, a->x_stride, a->out_stride, a->eps); break;
      default: hipLaunchKernelGGL(rmsnorm_rows_bf16_kernel<16>, g4, dim3(256), 0, s, xp, wp, op, rows, a->x_stride, a->out_stride, a->eps); break;
    }
    RecordLaunch(static_cast<int64_t>(g4.x), 256, 0, "rmsnorm_rows_bf16<nv=%d>", static_cast<int>(nv));
    AM_RETURN_IF_LAUNCH_FAILED("rmsnorm");
    return AM_STATUS_OK;
  }
  const dim3 grid(static_cast<unsigned>(a->rows));
#define AM_RMS(X, W, O)                                                                        \
  hipLaunchKernelGGL((rmsnorm_kernel<X, W, O>), grid, dim3(256), 0, s,                        \
                     static_cast<const X::T*>(a->x), static_cast<const W::T*>(a->w),           \
                     static_cast<O::T*>(a->out), a->hidden, a->x_stride, a->out_stride, a->eps)
  const int key = a->x_dtype * 4 + a->w_dtype * 2 + a->out_dtype;
  switch (key) {
    case 0: AM_RMS(ActF32, ActF32, ActF32); break;
    case 1: AM_RMS(ActF32, ActF32, ActBF16); break;
    case 2: AM_RMS(ActF32, ActBF16, ActF32); break;
    case 3: AM_RMS(ActF32, ActBF16, ActBF16); break;
    case 4: AM_RMS(ActBF16, ActF32, ActF32); break;
    case 5: AM_RMS(ActBF16, ActF32, ActBF16); break;
    case 6: AM_RMS(ActBF16, ActBF16, ActF32); break;
    default: AM_RMS(ActBF16, ActBF16, ActBF16); break;
  }
#undef AM_RMS
  AM_RETURN_IF_LAUNCH_FAILED("rmsnorm");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_rope_table(int64_t max_pos, int64_t head_dim, double theta,
                                               float* cos_tab, float* sin_tab) {
  AM_CHECK_ARG(max_pos > 0 && head_dim > 0 && head_dim % 2 == 0, "rope_table: bad shape");
  AM_CHECK_ARG(theta > 0.0 && std::isfinite(theta), "rope_table: theta must be finite and positive");
  AM_CHECK_ARG(cos_tab && sin_tab, "rope_table: null table");
  const int64_t half = head_dim / 2;
  for (int64_t i = 0; i < half; ++i) {
    const double inv_freq = 1.0 / std::pow(theta, 2.0 * static_cast<double>(i) / static_cast<double>(head_dim));
    for (int64_t p = 0; p < max_pos; ++p) {
      const double ang = static_cast<double>(p) * inv_freq;
      cos_tab[p * half + i] = static_cast<float>(std::cos(ang));
      sin_tab[p * half + i] = static_cast<float>(std::sin(ang));
    }
  }
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_rope(const am_gfx950_rope_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "rope: null args");
  AM_CHECK_ARG(IsAct(a->dtype), "rope: dtype must be f32 or bf16");
  AM_CHECK_ARG(a->seq >= 0 && a->hq > 0 && a->hkv > 0 && a->head_dim > 0 && a->head_dim % 2 == 0,
               "rope: bad shape");
  AM_CHECK_ARG(a->max_pos > 0, "rope: max_pos must be positive");
  if (a->seq == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->q && a->k && a->q_out && a->k_out && a->pos && a->cos_tab && a->sin_tab,
               "rope: null pointer");
  hipStream_t s = AsStream(stream);
  const int64_t half = a->head_dim / 2;
  for (int which = 0; which < 2; ++which) {
    const int64_t heads = which == 0 ? a->hq : a->hkv;
    const void* in = which == 0 ? a->q : a->k;
    void* out = which == 0 ? a->q_out : a->k_out;
    const int grid = GridFor(a->seq * heads * half);
    if (a->dtype == AM_DT_F32)
      hipLaunchKernelGGL(rope_kernel<ActF32>, dim3(grid), dim3(256), 0, s, static_cast<const float*>(in),
                         static_cast<float*>(out), a->pos, a->cos_tab, a->sin_tab, a->seq, heads,
                         a->head_dim, a->max_pos, nullptr);
    else
      hipLaunchKernelGGL(rope_kernel<ActBF16>, dim3(grid), dim3(256), 0, s,
                         static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), a->pos,
                         a->cos_tab, a->sin_tab, a->seq, heads, a->head_dim, a->max_pos, nullptr);
    AM_RETURN_IF_LAUNCH_FAILED("rope");
  }
  return AM_STATUS_OK;
}

namespace am {
am_status_code MakeKvRows(const am_gfx950_kv_pages* pages, int64_t cbs, int64_t cap, int64_t hkv, int64_t d,
                          KvRows* out) {
  KvRows r;
  r.cbs = cbs;
  r.cap = cap;
  r.hkv = static_cast<int32_t>(hkv);
  r.d = static_cast<int32_t>(d);
  if (pages != nullptr) {
    AM_CHECK_ARG(pages->block_table != nullptr, "kv pages: null block table");
    AM_CHECK_ARG(pages->block_size >= 32 && (pages->block_size & (pages->block_size - 1)) == 0,
                 "kv pages: block_size must be a power of two of at least 32");
    AM_CHECK_ARG(pages->table_stride > 0 && pages->num_blocks > 0, "kv pages: bad table stride or block count");
    AM_CHECK_ARG(cap <= static_cast<int64_t>(pages->table_stride) * pages->block_size,
                 "kv pages: capacity exceeds table_stride * block_size");
    r.table = pages->block_table;
    r.num_blocks = pages->num_blocks;
    r.stride = pages->table_stride;
    r.shift = __builtin_ctz(static_cast<unsigned>(pages->block_size));
    r.err = pages->err_flag;
  }
  *out = r;
  return AM_STATUS_OK;
}
}  // namespace am

extern "C" am_status_code am_gfx950_kv_update(const am_gfx950_kv_update_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "kv_update: null args");
  AM_CHECK_ARG(IsAct(a->dtype), "kv_update: dtype must be f32 or bf16");
  AM_CHECK_ARG(a->seq > 0 && a->hkv > 0 && a->head_dim > 0 && a->capacity > 0, "kv_update: bad shape");
  const int64_t esz = a->dtype == AM_DT_F32 ? 4 : 2;
  const int64_t row_bytes = a->head_dim * esz;
  AM_CHECK_ARG(row_bytes % 16 == 0, "kv_update: head_dim * element size must be a multiple of 16 bytes");
  AM_CHECK_ARG(a->k && a->v && a->k_cache && a->v_cache, "kv_update: null pointer");
  if (a->start_pos_dev == nullptr) {
    if (a->start_pos < 0 || a->start_pos + a->seq > a->capacity)
      return SetLastError(AM_STATUS_OUT_OF_RANGE, "KV write exceeds physical KV capacity");
  }
  KvRows kv;
  if (auto st = MakeKvRows(a->pages, 0, a->capacity, a->hkv, a->head_dim, &kv); st != AM_STATUS_OK) return st;
  if (kv.err == nullptr) kv.err = a->err_flag;
  const int grid = GridFor(a->seq * a->hkv * (row_bytes / 16));
  hipLaunchKernelGGL(kv_update_kernel, dim3(grid), dim3(256), 0, AsStream(stream),
                     static_cast<const uint8_t*>(a->k), static_cast<const uint8_t*>(a->v),
                     static_cast<uint8_t*>(a->k_cache), static_cast<uint8_t*>(a->v_cache), a->seq, a->hkv,
                     row_bytes, a->capacity, a->start_pos, a->start_pos_dev, a->err_flag, kv, esz);
  AM_RETURN_IF_LAUNCH_FAILED("kv_update");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_silu_mul(const am_gfx950_silu_mul_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && IsAct(a->dtype) && a->n >= 0, "silu_mul: bad args");
  if (a->n == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->gate && a->up && a->out, "silu_mul: null pointer");
  const int grid = GridFor(a->n);
  if (a->dtype == AM_DT_F32)
    hipLaunchKernelGGL(silu_mul_kernel<ActF32>, dim3(grid), dim3(256), 0, AsStream(stream),
                       static_cast<const float*>(a->gate), static_cast<const float*>(a->up),
                       static_cast<float*>(a->out), a->n);
  else
    hipLaunchKernelGGL(silu_mul_kernel<ActBF16>, dim3(grid), dim3(256), 0, AsStream(stream),
                       static_cast<const uint16_t*>(a->gate), static_cast<const uint16_t*>(a->up),
                       static_cast<uint16_t*>(a->out), a->n);
  AM_RETURN_IF_LAUNCH_FAILED("silu_mul");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_add(const am_gfx950_add_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && IsAct(a->dtype) && a->n >= 0, "add: bad args");
  if (a->n == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->a && a->b && a->out, "add: null pointer");
  const int grid = GridFor(a->n);
  if (a->dtype == AM_DT_F32)
    hipLaunchKernelGGL(add_kernel<ActF32>, dim3(grid), dim3(256), 0, AsStream(stream),
                       static_cast<const float*>(a->a), static_cast<const float*>(a->b),
                       static_cast<float*>(a->out), a->n);
  else
    hipLaunchKernelGGL(add_kernel<ActBF16>, dim3(grid), dim3(256), 0, AsStream(stream),
                       static_cast<const uint16_t*>(a->a), static_cast<const uint16_t*>(a->b),
                       static_cast<uint16_t*>(a->out), a->n);
  AM_RETURN_IF_LAUNCH_FAILED("add");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_fill(void* out, int32_t dtype, int64_t n, float value, void* stream) {
  AM_CHECK_ARG(IsAct(dtype) && n >= 0, "fill: bad args");
  if (n == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(out != nullptr, "fill: null pointer");
  const int grid = GridFor(n);
  if (dtype == AM_DT_F32)
    hipLaunchKernelGGL(fill_kernel<ActF32>, dim3(grid), dim3(256), 0, AsStream(stream), static_cast<float*>(out), n, value);
  else
    hipLaunchKernelGGL(fill_kernel<ActBF16>, dim3(grid), dim3(256), 0, AsStream(stream), static_cast<uint16_t*>(out), n, value);
  AM_RETURN_IF_LAUNCH_FAILED("fill");
  return AM_STATUS_OK;
}

extern "C" int64_t am_gfx950_argmax_workspace_bytes(int64_t rows) {
  // tickets (padded to 256 B) + partial values + partial indices
  return 256 * CeilDiv(rows * 4, 256) + rows * ArgmaxWs::kMaxBlocks * (4 + 8);
}

extern "C" am_status_code am_gfx950_argmax(const am_gfx950_argmax_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && IsAct(a->dtype), "argmax: bad args");
  AM_CHECK_ARG(a->rows >= 0 && a->rows <= 65535 && a->n > 0, "argmax: bad shape");
  if (a->rows == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->x && a->out && a->workspace, "argmax: null pointer");
  AM_CHECK_ARG(a->workspace_bytes >= am_gfx950_argmax_workspace_bytes(a->rows), "argmax: workspace too small");
  int nb = static_cast<int>(CeilDiv(a->n, 256 * 8));
  if (nb > ArgmaxWs::kMaxBlocks) nb = ArgmaxWs::kMaxBlocks;
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  unsigned* tickets = reinterpret_cast<unsigned*>(ws);
  const int64_t toff = 256 * CeilDiv(a->rows * 4, 256);
  int64_t* pi = reinterpret_cast<int64_t*>(ws + toff);
  float* pv = reinterpret_cast<float*>(ws + toff + a->rows * ArgmaxWs::kMaxBlocks * 8);
  const dim3 grid(static_cast<unsigned>(nb), static_cast<unsigned>(a->rows));
  if (a->dtype == AM_DT_F32)
    hipLaunchKernelGGL(argmax_kernel<ActF32>, grid, dim3(256), 0, AsStream(stream),
                       static_cast<const float*>(a->x), a->n, a->out, tickets, pv, pi);
  else
    hipLaunchKernelGGL(argmax_kernel<ActBF16>, grid, dim3(256), 0, AsStream(stream),
                       static_cast<const uint16_t*>(a->x), a->n, a->out, tickets, pv, pi);
  AM_RETURN_IF_LAUNCH_FAILED("argmax");
  return AM_STATUS_OK;
}

namespace am {
namespace {
__global__ void decode_advance_kernel(const int64_t* token, int64_t* hist, int64_t* pos, int64_t* step) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    const int64_t st = *step;
    if (hist != nullptr) hist[st] = *token;
    *step = st + 1;
    *pos = *pos + 1;
  }
}

// one thread per row; the shared step is read by every row before thread 0 bumps it
__global__ void decode_advance_rows_kernel(const int64_t* token, int64_t rows, int64_t* hist, int64_t hist_stride,
                                           int64_t* pos, int64_t* step) {
  const int64_t st = *step;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) {
    if (hist != nullptr) hist[r * hist_stride + st] = token[r];
    pos[r] = pos[r] + 1;
  }
  __syncthreads();
  if (threadIdx.x == 0) *step = st + 1;
}
}  // namespace
}  // namespace am

extern "C" am_status_code am_gfx950_decode_advance(const int64_t* token, int64_t* tokens_hist, int64_t* pos,
                                                   int64_t* step, void* stream) {
  AM_CHECK_ARG(token && pos && step, "decode_advance: null pointer");
  hipLaunchKernelGGL(decode_advance_kernel, dim3(1), dim3(64), 0, AsStream(stream), token, tokens_hist, pos, step);
  AM_RETURN_IF_LAUNCH_FAILED("decode_advance");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_decode_advance_rows(const int64_t* token, int64_t rows, int64_t* tokens_hist,
                                                        int64_t hist_stride, int64_t* pos, int64_t* step,
                                                        void* stream) {
  AM_CHECK_ARG(token && pos && step, "decode_advance_rows: null pointer");
  AM_CHECK_ARG(rows >= 1 && rows <= 65536, "decode_advance_rows: rows must be 1..65536");
  AM_CHECK_ARG(tokens_hist == nullptr || hist_stride > 0, "decode_advance_rows: hist_stride must be positive");
  hipLaunchKernelGGL(decode_advance_rows_kernel, dim3(1), dim3(256), 0, AsStream(stream), token, rows, tokens_hist,
                     hist_stride, pos, step);
  AM_RETURN_IF_LAUNCH_FAILED("decode_advance_rows");
  return AM_STATUS_OK;
}
