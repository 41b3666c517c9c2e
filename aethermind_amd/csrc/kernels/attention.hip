// GQA causal attention over the static KV cache (gfx950), split-K over positions.
//
// grid = (splits, kv_heads, batch*seq).  One 256-thread block owns one query row,
// one kv head (so all hq/hkv query heads of the group share every K/V load) and one
// contiguous slice of positions.  Inside the block:
//   * D/8 lanes cover one cache row (8 elements = 16 bytes of bf16 each), so a wave
//     reads 64/(D/8) consecutive rows per load instruction: for D = 128 that is four
//     256-byte rows = 1 KiB contiguous per instruction.  Each lane group loads U rows
//     before using any of them, so U KiB per wave are in flight at once.
//   * Each lane group keeps an fp32 online softmax (running max, sum, output slice)
//     in base 2: q is pre-scaled by log2(e)/sqrt(d), so every exponential is one
//     v_exp_f32.  Row dot products are summed over the lane group with DPP.
//     Groups are merged with xor shuffles, waves through LDS.
//   * The split count follows the live context (at least kMinPerSplit positions per
//     split); with one split the block writes the output, otherwise it writes a
//     partial record (m, l, o) and attention_combine_kernel, launched right after on
//     the same stream, merges the records.  No atomics, fences or zeroed scratch.

#include <cmath>

#include "am_kernel_common.h"

namespace am {
namespace {

struct AttnArgs {
  const void* q;
  const void* kc;
  const void* vc;
  void* out;
  int64_t seq, hq, hkv, cap, start;
  const int64_t* start_dev;
  int64_t cbs;  // cache batch stride (elements)
  int32_t splits;
  float scale;  // log2(e) / sqrt(d)
  float* part;
};

// Fewest cache positions one split block handles (short contexts use fewer splits).
constexpr int64_t kMinPerSplit = 64;
constexpr float kLog2e = 1.4426950408889634f;

template <class A>
__device__ __forceinline__ void load8(const typename A::T* p, float* out) {
  if constexpr (A::kDtype == AM_DT_BF16) {
    const uint4 v = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(p);
    const float4 b = *reinterpret_cast<const float4*>(p + 4);
    out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
    out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
  }
}

// Raw 16 bytes of one lane's slice of a cache row (bf16: 8 values; f32: 4 + 4).
template <class A>
struct RowSlice {
  uint4 a, b;
};
template <class A>
__device__ __forceinline__ RowSlice<A> load_slice(const typename A::T* p) {
  RowSlice<A> r;
  r.a = *reinterpret_cast<const uint4*>(p);
  if constexpr (A::kDtype != AM_DT_BF16) r.b = *reinterpret_cast<const uint4*>(p + 4);
  return r;
}
template <class A>
__device__ __forceinline__ void unpack_slice(const RowSlice<A>& r, float* out) {
  const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
  if constexpr (A::kDtype == AM_DT_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
  } else {
    const uint32_t v[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = __uint_as_float(w[i]);
      out[4 + i] = __uint_as_float(v[i]);
    }
  }
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Sum over aligned groups of LP lanes (LP = 8 or 16); every lane receives its sum.
template <int LP>
__device__ __forceinline__ float group_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror: the other quad of the 8-lane half
  if constexpr (LP == 16) v = dpp_add<0x140>(v);  // row_mirror: the other half of the row
  return v;
}

// merge (m2, l2, o2) into (m, l, o); base-2 exponentials
__device__ __forceinline__ void merge_state(float& m, float& l, float* o, float m2, float l2, const float* o2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float c1 = exp2f(m - mn), c2 = exp2f(m2 - mn);
  l = l * c1 + l2 * c2;
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = o[i] * c1 + o2[i] * c2;
  m = mn;
}

// live split count of a (row, kv head): every block and the combine agree on it
__device__ __forceinline__ int64_t live_splits(int64_t n_keys, int32_t splits) {
  int64_t ns = (n_keys + kMinPerSplit - 1) / kMinPerSplit;
  if (ns > splits) ns = splits;
  if (ns < 1) ns = 1;
  return ns;
}

__device__ __forceinline__ int64_t row_keys(const AttnArgs& p, int64_t b, int64_t s) {
  const int64_t start = p.start_dev != nullptr ? p.start_dev[b] : p.start;
  return start + s + 1 <= p.cap ? start + s + 1 : p.cap;
}

template <class A, int D, int G>
__global__ __launch_bounds__(256) void attention_kernel(AttnArgs p) {
  constexpr int LP = D / 8;      // lanes per cache row
  constexpr int PPW = 64 / LP;   // rows per wave step
  constexpr int U = 4;           // rows per lane group loaded before use
  constexpr int STEP = 4 * PPW;  // rows per block step
  using T = typename A::T;
  __shared__ float sm_m[4][G], sm_l[4][G];
  __shared__ float sm_o[4][G][D];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LP, ps = lane / LP;
  const int64_t qr = blockIdx.z;
  const int64_t b = qr / p.seq, s = qr % p.seq;
  const int64_t g = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t n_keys = row_keys(p, b, s);
  const int64_t nsplit = live_splits(n_keys, p.splits);
  if (split >= nsplit) return;  // surplus block for this context
  const int64_t per = (n_keys + nsplit - 1) / nsplit;
  const int64_t lo = split * per;
  const int64_t hi = lo + per < n_keys ? lo + per : n_keys;

  const T* qp = static_cast<const T*>(p.q) + (qr * p.hq + g * G) * D + sub * 8;
  float qv[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    load8<A>(qp + hh * D, qv[hh]);
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[hh][i] *= p.scale;
  }
  const T* kbase = static_cast<const T*>(p.kc) + b * p.cbs + g * p.cap * D + sub * 8;
  const T* vbase = static_cast<const T*>(p.vc) + b * p.cbs + g * p.cap * D + sub * 8;

  float m[G], l[G], o[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[hh][i] = 0.0f;
  }

  for (int64_t base = lo + wave * PPW + ps; base < hi; base += U * STEP) {
    RowSlice<A> kr[U], vr[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t pos = base + u * STEP;
      ok[u] = pos < hi;
      if (!ok[u]) pos = lo;  // in-bounds address, result discarded
      kr[u] = load_slice<A>(kbase + pos * D);
      vr[u] = load_slice<A>(vbase + pos * D);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kv[8], vv[8];
      unpack_slice<A>(kr[u], kv);
      unpack_slice<A>(vr[u], vv);
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d = fmaf(qv[hh][i], kv[i], d);
        d = group_sum<LP>(d);
        if (!ok[u]) d = -INFINITY;
        const float mn = fmaxf(m[hh], d);
        const float c = mn == -INFINITY ? 1.0f : exp2f(m[hh] - mn);
        const float e = ok[u] ? exp2f(d - mn) : 0.0f;
        l[hh] = fmaf(l[hh], c, e);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[hh][i] = fmaf(o[hh][i], c, e * vv[i]);
        m[hh] = mn;
      }
    }
  }
  // merge the PPW row streams of the wave (lanes sub, sub+LP, ...)
#pragma unroll
  for (int off = LP; off < 64; off <<= 1) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      const float m2 = __shfl_xor(m[hh], off, 64);
      const float l2 = __shfl_xor(l[hh], off, 64);
      float o2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o2[i] = __shfl_xor(o[hh][i], off, 64);
      merge_state(m[hh], l[hh], o[hh], m2, l2, o2);
    }
  }
  if (ps == 0) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      if (sub == 0) {
        sm_m[wave][hh] = m[hh];
        sm_l[wave][hh] = l[hh];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) sm_o[wave][hh][sub * 8 + i] = o[hh][i];
    }
  }
  __syncthreads();
  if (wave == 0 && ps == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w)
#pragma unroll
      for (int hh = 0; hh < G; ++hh) merge_state(m[hh], l[hh], o[hh], sm_m[w][hh], sm_l[w][hh], &sm_o[w][hh][sub * 8]);
    if (nsplit == 1) {
      T* out = static_cast<T*>(p.out) + (qr * p.hq + g * G) * D + sub * 8;
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        const float inv = l[hh] > 0.0f ? 1.0f / l[hh] : 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) A::store(out + hh * D, i, o[hh][i] * inv);
      }
    } else {
      // partial record per head: [m, l, o[D]]
      float* rec = p.part + (((qr * p.hkv + g) * p.splits + split) * G) * (D + 2);
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        if (sub == 0) {
          rec[hh * (D + 2)] = m[hh];
          rec[hh * (D + 2) + 1] = l[hh];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) rec[hh * (D + 2) + 2 + sub * 8 + i] = o[hh][i];
      }
    }
  }
}

// Merges the split records of one (query row, q head): grid = (hq, batch*seq), D
// threads, one output dimension each.  Rows that used a single split were written by
// attention_kernel and are left alone.
template <class A, int D>
__global__ __launch_bounds__(D) void attention_combine_kernel(AttnArgs p) {
  using T = typename A::T;
  const int64_t h = blockIdx.x, qr = blockIdx.y;
  const int64_t b = qr / p.seq, s = qr % p.seq;
  const int64_t n_keys = row_keys(p, b, s);
  const int64_t nsplit = live_splits(n_keys, p.splits);
  if (nsplit == 1) return;
  const int64_t G = p.hq / p.hkv;
  const int64_t g = h / G, hh = h % G;
  const float* base = p.part + ((qr * p.hkv + g) * p.splits * G + hh) * (D + 2);
  const int64_t rs = G * (D + 2);  // record stride between splits
  float mx = -INFINITY;
  for (int64_t sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, base[sp * rs]);
  float den = 0.0f, acc = 0.0f;
  if (mx != -INFINITY) {
    for (int64_t sp = 0; sp < nsplit; ++sp) {
      const float* rec = base + sp * rs;
      const float c = exp2f(rec[0] - mx);
      den = fmaf(rec[1], c, den);
      acc = fmaf(rec[2 + threadIdx.x], c, acc);
    }
  }
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  T* out = static_cast<T*>(p.out) + (qr * p.hq + h) * D;
  A::store(out, threadIdx.x, acc * inv);
}

int ChooseSplits(int64_t seq, int64_t cap, int32_t requested) {
  if (requested > 0) return requested;
  if (seq > 1) return 1;
  int64_t s = cap / kMinPerSplit;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return static_cast<int>(s);
}

template <class A, int D>
am_status_code LaunchD(int64_t G, dim3 grid, const AttnArgs& a, hipStream_t s) {
  switch (G) {
    case 1: hipLaunchKernelGGL((attention_kernel<A, D, 1>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attention_kernel<A, D, 2>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attention_kernel<A, D, 4>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((attention_kernel<A, D, 8>), grid, dim3(256), 0, s, a); break;
    default: return SetLastError(AM_STATUS_UNIMPLEMENTED, "attention: q heads per kv head must be 1, 2, 4 or 8");
  }
  AM_RETURN_IF_LAUNCH_FAILED("attention");
  if (a.splits > 1) {
    hipLaunchKernelGGL((attention_combine_kernel<A, D>), dim3(static_cast<unsigned>(a.hq), grid.z), dim3(D), 0, s, a);
    AM_RETURN_IF_LAUNCH_FAILED("attention combine");
  }
  return AM_STATUS_OK;
}

}  // namespace
}  // namespace am

using namespace am;

extern "C" int64_t am_gfx950_attention_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv,
                                                       int64_t head_dim, int64_t capacity, int32_t num_splits) {
  (void)hkv;
  const int splits = ChooseSplits(seq, capacity, num_splits);
  if (splits == 1) return 0;
  return batch * seq * hq * splits * (head_dim + 2) * 4;
}

extern "C" am_status_code am_gfx950_attention(const am_gfx950_attention_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "attention: null args");
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "attention: dtype must be f32 or bf16");
  AM_CHECK_ARG(a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0, "Attention num_attention_heads must be divisible by num_key_value_heads");
  AM_CHECK_ARG(a->head_dim == 64 || a->head_dim == 128, "attention: head_dim must be 64 or 128");
  AM_CHECK_ARG(a->seq > 0 && a->capacity > 0, "attention: bad shape");
  const int64_t batch = a->batch > 0 ? a->batch : 1;
  AM_CHECK_ARG(batch * a->seq <= 65535, "attention: too many query rows");
  AM_CHECK_ARG(a->q && a->k_cache && a->v_cache && a->out, "attention: null pointer");
  if (a->start_pos_dev == nullptr)
    AM_CHECK_ARG(a->start_pos >= 0 && a->start_pos + a->seq <= a->capacity, "KV read exceeds committed token range");
  const int splits = ChooseSplits(a->seq, a->capacity, a->num_splits);
  AM_CHECK_ARG(splits >= 1 && splits <= 1024, "attention: bad split count");
  const int64_t need = am_gfx950_attention_workspace_bytes(batch, a->seq, a->hq, a->hkv, a->head_dim, a->capacity,
                                                           a->num_splits);
  if (splits > 1) AM_CHECK_ARG(a->workspace != nullptr && a->workspace_bytes >= need, "attention: workspace too small");
  AttnArgs p{};
  p.q = a->q;
  p.kc = a->k_cache;
  p.vc = a->v_cache;
  p.out = a->out;
  p.seq = a->seq;
  p.hq = a->hq;
  p.hkv = a->hkv;
  p.cap = a->capacity;
  p.start = a->start_pos;
  p.start_dev = a->start_pos_dev;
  p.cbs = batch > 1 ? a->cache_batch_stride : 0;
  p.splits = splits;
  p.scale = kLog2e / sqrtf(static_cast<float>(a->head_dim));
  if (splits > 1) p.part = static_cast<float*>(a->workspace);
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(a->hkv), static_cast<unsigned>(batch * a->seq));
  const int64_t G = a->hq / a->hkv;
  hipStream_t s = AsStream(stream);
  if (a->dtype == AM_DT_BF16)
    return a->head_dim == 128 ? LaunchD<ActBF16, 128>(G, grid, p, s) : LaunchD<ActBF16, 64>(G, grid, p, s);
  return a->head_dim == 128 ? LaunchD<ActF32, 128>(G, grid, p, s) : LaunchD<ActF32, 64>(G, grid, p, s);
}
