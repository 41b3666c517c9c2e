// GQA causal attention over the static KV cache (gfx950), split-K over positions.
//
// grid = (splits, kv_heads, batch*seq).  One 512-thread block (8 waves) owns one
// query row, one kv head (so all hq/hkv query heads of the group share every K/V
// load) and one contiguous slice of positions.  Inside the block:
//   * D/8 lanes cover one cache row (8 elements = 16 bytes of bf16 each), so a wave
//     reads 64/(D/8) consecutive rows per load instruction: for D = 128 that is four
//     256-byte rows = 1 KiB contiguous per instruction.
//   * Positions go in batches of 8 waves x 64/(D/8) rows x U rows per lane group
//     (U shrinks as the query group grows, so two batches fit in registers).
//     q is loaded first, then two batches of K/V; the batch after next is issued as
//     soon as a buffer has been consumed, so the cache streams while the current
//     batch is reduced.  The loop exits sit before the issues, so the pending loads
//     always retire in order.
//   * Each lane group keeps an fp32 online softmax (running max, sum, output slice)
//     in base 2: q is pre-scaled by log2(e)/sqrt(d), so every exponential is one
//     v_exp_f32; a batch updates the running state once per head.  Row dot products
//     are summed over the lane group with DPP; lane groups are merged with permlane
//     swaps / DPP; the 8 waves through LDS, one (head, dim) per thread.
//   * The split count follows the live context (at least kMinPerSplit positions per
//     split); with one split the block writes the output.  Otherwise every block
//     writes a partial record (per head m, l, two pad words, o[D]) with device-coherent
//     stores, waits for them to complete and takes a ticket; the last block of the
//     (row, kv head) reads the records back with device-coherent loads, merges them
//     and resets the ticket.  Only the records and the ticket are device-coherent
//     accesses: no cache-wide writeback or invalidate, and no second launch.

#include <hip/hip_ext.h>

#include <cmath>
#include <cstdio>
#include <mutex>

#include "am_kernel_common.h"
#include "am_launch_timing.h"

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
  int32_t min_per_split;  // fewest positions one split block handles
  float scale;  // log2(e) / sqrt(d)
  float* part;
  unsigned* tickets;  // [rows][hkv], zero between calls
  KvRows kv;          // row addressing of the (possibly paged) cache
};

constexpr int kWaves = 8;
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Split records move as 8- and 16-byte buffer loads and stores carrying the sc1 cache
// policy (bit 4 of the builtins' aux operand on gfx950): the device-coherent accesses
// the relaxed agent-scope atomics compile to, several words at a time.  The
// descriptor's last dword is the raw-buffer format word (32-bit data, no swizzle).
constexpr int kCpolSc1 = 16;
constexpr int kRawBufferFlags = 0x00020000;
// Fewest cache positions one split block handles (contexts up to this length use a
// single block per (row, kv head) and need no cross-block merge), and the most
// splits: measured on MI355X, 128 positions per block and at most 16 blocks per
// (row, kv head) minimise decode time from 128 to 4096 positions.
constexpr int64_t kMinPerSplit = 128;
constexpr int kMaxSplits = 16;
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

// Raw bytes of one lane's 8-element slice of a cache row (bf16: 16 B; f32: 32 B).
template <class A>
struct RowSlice {
  uint4 a;
  uint4 b;  // f32 only
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

// Value held by lane (lane ^ OFF), OFF in {8, 16, 32}.
template <int OFF>
__device__ __forceinline__ float xor_partner(float v, int lane) {
  if constexpr (OFF == 8) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  } else if constexpr (OFF == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(((lane >> 4) & 1) ? r[0] : r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(lane < 32 ? r[1] : r[0]);
  }
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

// live split count of a (row, kv head): every block agrees on it
__device__ __forceinline__ int64_t live_splits(int64_t n_keys, int32_t splits, int32_t min_per_split) {
  int64_t ns = (n_keys + min_per_split - 1) / min_per_split;
  if (ns > splits) ns = splits;
  if (ns < 1) ns = 1;
  return ns;
}

__device__ __forceinline__ int64_t row_keys(const AttnArgs& p, int64_t b, int64_t s) {
  const int64_t start = p.start_dev != nullptr ? p.start_dev[b] : p.start;
  return start + s + 1 <= p.cap ? start + s + 1 : p.cap;
}

// Merge the NW per-wave states (sm_m, sm_l, sm_o) of one block, then write the output
// (one split) or the block's partial record, and let the last split block of the
// (row, kv head) merge the records.
template <class A, int D, int G, int NW>
__device__ __forceinline__ void finish_rows(const AttnArgs& p, const float (*sm_m)[G], const float (*sm_l)[G],
                                            const float (*sm_o)[G][D], bool& last, int64_t qr, int64_t g, int split,
                                            int64_t nsplit) {
  constexpr int NT = NW * 64;
  constexpr int RH = D + 4;  // floats per head in a partial record: m, l, 2 pad, o[D]
  using T = typename A::T;
  // Merge the waves of (head hh, dims d0 .. d0 + NE): the running maximum, the
  // rescaled denominator and output sums, in wave order.
  auto wave_merge = [&]<int NE>(int hh, int d0, float& mx, float& den, float (&acc)[NE]) {
    mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) mx = fmaxf(mx, sm_m[w][hh]);
    den = 0.0f;
#pragma unroll
    for (int e = 0; e < NE; ++e) acc[e] = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float c = exp2f(sm_m[w][hh] - mx);
        den = fmaf(sm_l[w][hh], c, den);
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[e] = fmaf(sm_o[w][hh][d0 + e], c, acc[e]);
      }
    }
  };
  if (nsplit == 1) {
    // one split: thread t owns (head, dim) pairs t, t + NT, ... and writes the output
    for (int t = threadIdx.x; t < G * D; t += NT) {
      const int hh = t / D, dd = t % D;
      float mx, den, acc[1];
      wave_merge(hh, dd, mx, den, acc);
      T* out = static_cast<T*>(p.out) + (qr * p.hq + g * G + hh) * D;
      A::store(out, dd, den > 0.0f ? acc[0] / den : 0.0f);
    }
    return;
  }
  // The block's partial record, published with device-coherent (sc1) stores: in 4-wave
  // blocks thread t owns 4 consecutive dims of one head (one 16-byte buffer store, and
  // the head's first thread stores m and l as one 8-byte store); 8-wave blocks have a
  // thread for every (head, dim) pair and keep 4-byte relaxed agent-scope stores (as
  // fast there in same-box A/B runs at batch 4; the wider accesses were about 1% slower).
  constexpr int DPT = NW >= 8 ? 1 : 4;
  static_assert(D % DPT == 0, "dims per thread must divide the head dimension");
  float* rec = p.part + (((qr * p.hkv + g) * p.splits + split) * G) * RH;
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(rec, 0, G * RH * 4, kRawBufferFlags);
  for (int t = threadIdx.x; t < G * D / DPT; t += NT) {
    const int hh = DPT * t / D, d0 = DPT * t % D;
    float mx, den, acc[DPT];
    wave_merge(hh, d0, mx, den, acc);
    if constexpr (DPT == 4) {
      if (d0 == 0)
        __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{__float_as_uint(mx), __float_as_uint(den)}, rrec, hh * RH * 4, 0,
                                              kCpolSc1);
      __builtin_amdgcn_raw_buffer_store_b128(
          u32x4_t{__float_as_uint(acc[0]), __float_as_uint(acc[1]), __float_as_uint(acc[2]), __float_as_uint(acc[3])},
          rrec, (hh * RH + 4 + d0) * 4, 0, kCpolSc1);
    } else {
      if (d0 == 0) {
        __hip_atomic_store(&rec[hh * RH], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&rec[hh * RH + 1], den, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __hip_atomic_store(&rec[hh * RH + 4 + d0], acc[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // every thread's record stores have completed before the block takes its ticket
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(&p.tickets[qr * p.hkv + g], 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    last = t == static_cast<unsigned>(nsplit - 1);
  }
  __syncthreads();
  if (!last) return;
  // Merge the splits: thread t owns the same dims; the records are read with
  // device-coherent (sc1) loads of the same widths, kMergeBatch splits at a time with
  // all of a batch's loads in flight together (slots past the last split reread it and
  // are skipped).  Each batch rescales the running sums to the batch's new maximum.
  constexpr int kMergeBatch = 8;
  const float* base0 = p.part + ((qr * p.hkv + g) * p.splits) * G * RH;
  const __amdgpu_buffer_rsrc_t rall = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(base0), 0, static_cast<int>(nsplit * G * RH * 4), kRawBufferFlags);
  for (int t = threadIdx.x; t < G * D / DPT; t += NT) {
    const int hh = DPT * t / D, d0 = DPT * t % D;
    float mx = -INFINITY, den = 0.0f, acc[DPT];
#pragma unroll
    for (int e = 0; e < DPT; ++e) acc[e] = 0.0f;
    for (int64_t s0 = 0; s0 < nsplit; s0 += kMergeBatch) {
      u32x2_t ml[kMergeBatch];
      uint32_t ov[kMergeBatch][DPT];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int r = static_cast<int>(s0 + u < nsplit ? s0 + u : nsplit - 1);
        const int off = (r * G * RH + hh * RH) * 4;
        if constexpr (DPT == 4) {
          ml[u] = __builtin_amdgcn_raw_buffer_load_b64(rall, off, 0, kCpolSc1);
          const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rall, off + (4 + d0) * 4, 0, kCpolSc1);
#pragma unroll
          for (int e = 0; e < 4; ++e) ov[u][e] = v[e];
        } else {
          const float* rr = base0 + off / 4;
          ml[u][0] = __float_as_uint(__hip_atomic_load(&rr[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          ml[u][1] = __float_as_uint(__hip_atomic_load(&rr[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
          ov[u][0] = __float_as_uint(__hip_atomic_load(&rr[4 + d0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
      }
      float bm = mx;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u)
        if (s0 + u < nsplit) bm = fmaxf(bm, __uint_as_float(ml[u][0]));
      if (bm == -INFINITY) continue;
      const float c0 = exp2f(mx - bm);  // 0 while nothing has been summed
      den *= c0;
#pragma unroll
      for (int e = 0; e < DPT; ++e) acc[e] *= c0;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (s0 + u < nsplit) {
          const float c = exp2f(__uint_as_float(ml[u][0]) - bm);
          den = fmaf(__uint_as_float(ml[u][1]), c, den);
#pragma unroll
          for (int e = 0; e < DPT; ++e) acc[e] = fmaf(__uint_as_float(ov[u][e]), c, acc[e]);
        }
      }
      mx = bm;
    }
    T* out = static_cast<T*>(p.out) + (qr * p.hq + g * G + hh) * D;
#pragma unroll
    for (int e = 0; e < DPT; ++e) A::store(out, d0 + e, den > 0.0f ? acc[e] / den : 0.0f);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&p.tickets[qr * p.hkv + g], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}


template <class A, int D, int G>
__global__ __launch_bounds__(kWaves * 64) void attention_kernel(AttnArgs p) {
  constexpr int LP = D / 8;                                 // lanes per cache row
  constexpr int PPW = 64 / LP;                              // rows per wave step
  // rows per lane group per batch: two batches of raw K/V rows stay in registers
  constexpr int UB = A::kDtype == AM_DT_BF16 ? 8 : 4;
  constexpr int U = G <= 2 ? UB : (G == 4 ? UB / 2 : UB / 4);
  constexpr int STEP = kWaves * PPW;                        // rows per block step
  constexpr int64_t BATCH = static_cast<int64_t>(STEP) * U;  // rows per batch
  using T = typename A::T;
  __shared__ float sm_m[kWaves][G], sm_l[kWaves][G];
  __shared__ float sm_o[kWaves][G][D];
  __shared__ bool last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane % LP, ps = lane / LP;
  const int64_t qr = blockIdx.z;
  const int64_t b = qr / p.seq, s = qr % p.seq;
  const int64_t g = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t n_keys = row_keys(p, b, s);
  const int64_t nsplit = live_splits(n_keys, p.splits, p.min_per_split);
  if (split >= nsplit) return;  // surplus block for this context
  const int64_t per = (n_keys + nsplit - 1) / nsplit;
  const int64_t lo = split * per;
  const int64_t hi = lo + per < n_keys ? lo + per : n_keys;
  const int64_t nb = (hi - lo + BATCH - 1) / BATCH;  // batches (>= 1)

  // q first: the memory counter retires in order, so the K/V batches behind it do not
  // delay the first use of q.
  const T* qp = static_cast<const T*>(p.q) + (qr * p.hq + g * G) * D + sub * 8;
  RowSlice<A> qraw[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) qraw[hh] = load_slice<A>(qp + hh * D);

  const T* kbase = static_cast<const T*>(p.kc) + b * p.cbs + g * p.cap * D + sub * 8;
  const T* vbase = static_cast<const T*>(p.vc) + b * p.cbs + g * p.cap * D + sub * 8;
  const int64_t row0 = wave * PPW + ps;  // this lane group's first row in a block step
  // Loads batch bi (clamped to the last batch; out-of-range rows read row lo).
  auto issue = [&](RowSlice<A> (&kr)[U], RowSlice<A> (&vr)[U], int64_t bi) {
    if (bi >= nb) bi = nb - 1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int64_t pos = lo + bi * BATCH + row0 + u * STEP;
      if (pos >= hi) pos = lo;
      kr[u] = load_slice<A>(kbase + pos * D);
      vr[u] = load_slice<A>(vbase + pos * D);
    }
  };
  RowSlice<A> ka[U], va[U], kb[U], vb[U];
  issue(ka, va, 0);
  issue(kb, vb, 1);

  float qv[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    unpack_slice<A>(qraw[hh], qv[hh]);
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[hh][i] *= p.scale;
  }
  float m[G], l[G], o[G][8];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    m[hh] = -INFINITY;
    l[hh] = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[hh][i] = 0.0f;
  }

  // One batch: all U dots per head first, then one running-state update per head.
  auto process = [&](const RowSlice<A> (&kr)[U], const RowSlice<A> (&vr)[U], int64_t bi) {
    float e[G][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kv[8];
      unpack_slice<A>(kr[u], kv);
      const bool ok = lo + bi * BATCH + row0 + u * STEP < hi;
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) d = fmaf(qv[hh][i], kv[i], d);
        d = group_sum<LP>(d);
        e[hh][u] = ok ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      float mn = m[hh];
#pragma unroll
      for (int u = 0; u < U; ++u) mn = fmaxf(mn, e[hh][u]);
      const float c = mn == -INFINITY ? 1.0f : exp2f(m[hh] - mn);
      float sum = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        e[hh][u] = e[hh][u] == -INFINITY ? 0.0f : exp2f(e[hh][u] - mn);
        sum += e[hh][u];
      }
      l[hh] = fmaf(l[hh], c, sum);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[hh][i] *= c;
      m[hh] = mn;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float vv[8];
      unpack_slice<A>(vr[u], vv);
#pragma unroll
      for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[hh][i] = fmaf(e[hh][u], vv[i], o[hh][i]);
    }
  };

  for (int64_t bi = 0;;) {
    process(ka, va, bi);
    if (bi + 2 >= nb) {
      if (bi + 1 < nb) process(kb, vb, bi + 1);
      break;
    }
    issue(ka, va, bi + 2);
    process(kb, vb, bi + 1);
    if (bi + 3 >= nb) {
      process(ka, va, bi + 2);
      break;
    }
    issue(kb, vb, bi + 3);
    bi += 2;
  }

  // merge the PPW row streams of the wave (lane groups sub, sub+LP, ...)
#pragma unroll
  for (int off = LP; off < 64; off <<= 1) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      float m2, l2, o2[8];
      if (off == 8) {
        m2 = xor_partner<8>(m[hh], lane);
        l2 = xor_partner<8>(l[hh], lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) o2[i] = xor_partner<8>(o[hh][i], lane);
      } else if (off == 16) {
        m2 = xor_partner<16>(m[hh], lane);
        l2 = xor_partner<16>(l[hh], lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) o2[i] = xor_partner<16>(o[hh][i], lane);
      } else {
        m2 = xor_partner<32>(m[hh], lane);
        l2 = xor_partner<32>(l[hh], lane);
#pragma unroll
        for (int i = 0; i < 8; ++i) o2[i] = xor_partner<32>(o[hh][i], lane);
      }
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

  finish_rows<A, D, G, kWaves>(p, sm_m, sm_l, sm_o, last, qr, g, split, nsplit);
}

// ---- decode: one query position per row, bf16 q and cache, both products on MFMA ----
//
// grid = (splits, kv_heads, batch).  A block of NW waves owns one (row, kv head) and a
// slice of positions; wave w takes the 32-position steps w, w + NW, ... of the slice,
// with the next step's K and V loads in flight while a step computes.  NW = 4 (one
// wave per SIMD, 264 registers) unless the grid already gives every CU a block
// (batched long contexts): then NW = 8 within 236 registers, two waves per SIMD and
// twice the K/V loads in flight per CU, the extra waves merged in LDS.
// No K or V byte is staged in LDS: their MFMA operands are built in the registers of
// the lane that loaded them.
//   * Scores: S^T = K Q^T on v_mfma_f32_16x16x32_bf16.  A = 16 cache rows (position
//     16 tt + i of the step is row i of tile tt; each lane loads 16 contiguous bytes
//     of its row per k step), B = the G query heads of the group (columns >= G
//     repeat head 0 and are never read), each wave's own copy in LDS.  Lane (j, h)
//     receives the scores of head j for positions 16 tt + 4 h + r, so the softmax
//     state of head j lives in the lanes with lane % 16 == j.  Products are exact and
//     sums fp32; the log2(e)/sqrt(d) scale is applied to the fp32 scores.
//   * O += P V on the same MFMA.  The reduction index runs over positions and its
//     order is free: k slot e of lane group h is position 16 (e >> 2) + 4 h + (e & 3),
//     exactly the positions whose scores lane (j, h) holds, so P never moves between
//     lanes (A = P split into bf16 hi + lo parts, two MFMAs, about 16 significant
//     bits).  The output column order is free too: lane n of tile t holds dimension
//     (D/16) n + t.  So B lane (n, h) needs V[its 8 positions][(D/16) n + t] for
//     t < D/16, which is exactly what it loads as 8 rows x D/16 contiguous columns
//     (16 lanes cover a whole row, coalesced); tile t's operand is column t of that
//     8 x D/16 block, gathered with byte permutes in the lane's own registers.
//   * The per-wave states are merged in LDS, and split blocks merge through the same
//     records and ticket as the general kernel.
constexpr int kDecWaves = 4;
// Split policy of the decode kernel, measured on MI355X with a cold cache (the layer's
// K/V evicted by the weight stream, as in decode) and in the replayed decode graph: at
// least 64 positions per split block and at most 8 split blocks per (row, kv head)
// minimise the kernel time from 64 to 4096 positions.  A split block costs a
// cross-block merge, so short contexts keep a single block.
constexpr int32_t kDecMinPerSplit = 64;
constexpr int kDecMaxSplits = 8;

// NW = 8: two waves per SIMD (236 VGPRs, no spills, against 264 for the 4-wave block,
// which holds one wave per SIMD), for grids that already give every CU a block.
template <int D, int G, int NW>
__global__ __launch_bounds__(NW * 64) void attention_decode_kernel(AttnArgs p) {
  constexpr int KK = D / 32;  // MFMA k steps of one score tile
  constexpr int CW = D / 16;  // V columns per lane = output tiles
  constexpr int VW = CW / 2;  // 32-bit words of one lane's V row piece
  __shared__ float sm_m[NW][G], sm_l[NW][G];
  __shared__ float sm_o[NW][G][D];
  __shared__ uint4 sq[NW][KK][64];  // each wave's copy of the score B operand
  __shared__ bool last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int j = lane & 15, h = lane >> 4;
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
  typedef __attribute__((ext_vector_type(4))) float f32x4_t;
  const int64_t qr = blockIdx.z;
  const int64_t b = qr / p.seq, s = qr % p.seq;
  const int64_t g = blockIdx.y;
  const int split = blockIdx.x;
  const int64_t n_keys = row_keys(p, b, s);
  // Slices are whole 32-position steps (a step then never straddles two cache blocks):
  // the slice length is rounded up to 32 and the live split count follows from it,
  // the same in every block of the (row, kv head).
  const int64_t ns0 = live_splits(n_keys, p.splits, p.min_per_split);
  const int64_t per = (((n_keys + ns0 - 1) / ns0) + 31) & ~int64_t{31};
  const int64_t nsplit = (n_keys + per - 1) / per;
  if (split >= nsplit) return;  // surplus block for this context
  const int64_t lo = split * per;
  const int64_t hi = lo + per < n_keys ? lo + per : n_keys;
  const int64_t nsteps = (hi - lo + 31) / 32;
  const int64_t my = nsteps > wave ? (nsteps - wave + NW - 1) / NW : 0;  // this wave's steps

  // B operand of the scores: lane (j, h) holds query head j of the group at
  // d = 32 kk + 8 h .. +8; columns j >= G repeat head 0 and only feed score columns,
  // softmax states and output rows that are never read.  Loaded first, so waiting for
  // it never waits for the cache loads behind it; every wave keeps its own copy in
  // LDS, so no block barrier (which would also drain the cache loads) is needed.
  const uint16_t* qp = static_cast<const uint16_t*>(p.q) + (qr * p.hq + g * G + (j < G ? j : 0)) * D + 8 * h;
  const uint4 q0 = *reinterpret_cast<const uint4*>(qp), q1 = *reinterpret_cast<const uint4*>(qp + 32);
  uint4 q2 = q0, q3 = q1;
  if constexpr (KK == 4) {
    q2 = *reinterpret_cast<const uint4*>(qp + 64);
    q3 = *reinterpret_cast<const uint4*>(qp + 96);
  }

  const uint16_t* kc0 = static_cast<const uint16_t*>(p.kc);
  const uint16_t* vc0 = static_cast<const uint16_t*>(p.vc);

  struct Buf {
    uint4 k[2][KK];    // two 16-row score tiles
    uint32_t v[8][VW];  // V[position of k slot c][CW j .. CW j + CW)
  };
  // Loads step i (clamped to this wave's last step; rows past the slice read row
  // hi - 1, whose scores are masked to -inf).  The step's 32 rows are contiguous from
  // its first row, whose offset (the same in K and V) is looked up once per step;
  // lanes add 32-bit row offsets to it.
  const int64_t last_row = hi - 1;
  auto issue = [&](Buf& bf, int64_t i) {
    if (i >= my) i = my - 1;
    const int64_t base = lo + 32 * (wave + i * NW);
    const int64_t off = p.kv.Row(b, g, base);
    const uint16_t* ks = kc0 + off;
    const uint16_t* vs = vc0 + off;
    const uint32_t lim = static_cast<uint32_t>(last_row - base);  // last readable row of the step
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const uint32_t r = min(static_cast<uint32_t>(16 * tt + j), lim);
      const uint16_t* kp = ks + (r * D + 8 * h);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) bf.k[tt][kk] = *reinterpret_cast<const uint4*>(kp + 32 * kk);
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t r = min(static_cast<uint32_t>(16 * (c >> 2) + 4 * h + (c & 3)), lim);
      const uint16_t* vp = vs + (r * D + CW * j);
      if constexpr (VW == 4) {
        const uint4 t = *reinterpret_cast<const uint4*>(vp);
        bf.v[c][0] = t.x, bf.v[c][1] = t.y, bf.v[c][2] = t.z, bf.v[c][3] = t.w;
      } else {
        const uint2 t = *reinterpret_cast<const uint2*>(vp);
        bf.v[c][0] = t.x, bf.v[c][1] = t.y;
      }
    }
  };

  float m_run = -INFINITY, l_run = 0.0f;  // head j's state over this lane's positions
  f32x4_t o[CW];                          // O[4h + r][CW j + t]
#pragma unroll
  for (int t = 0; t < CW; ++t) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Buf& bf, int64_t i) {
    // scores of positions base + 16 tt + 4 h + r for head j; lim = positions of the
    // step left in the slice, seen from this lane group's first row
    const int32_t lim = static_cast<int32_t>(hi - (lo + 32 * (wave + i * NW))) - 4 * h;
    float sc[2][4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, bf.k[tt][kk]),
                                                       __builtin_bit_cast(bf16x8_t, sq[wave][kk][lane]), acc, 0, 0,
                                                       0);
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[tt][r] = 16 * tt + r < lim ? acc[r] * p.scale : -INFINITY;
    }
    float bm = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
                     fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
    bm = fmaxf(bm, xor_partner<16>(bm, lane));
    bm = fmaxf(bm, xor_partner<32>(bm, lane));
    const float mn = fmaxf(m_run, bm);
    const float c = mn == -INFINITY ? 1.0f : exp2f(m_run - mn);
    float pr[2][4];
    float sum = 0.0f;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pr[tt][r] = sc[tt][r] == -INFINITY ? 0.0f : exp2f(sc[tt][r] - mn);
        sum += pr[tt][r];
      }
    l_run = fmaf(l_run, c, sum);
    m_run = mn;
    // rescale O rows 4h + r by their head's factor (held by lane 16 h + 4 h + r)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float cr = __shfl(c, 16 * h + 4 * h + r);
#pragma unroll
      for (int t = 0; t < CW; ++t) o[t][r] *= cr;
    }
    // A operand: element e of lane (j, h) is position 16 (e >> 2) + 4 h + (e & 3)
    bf16x8_t phi, plo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = pr[e >> 2][e & 3];
      const __bf16 hb = static_cast<__bf16>(v);
      phi[e] = hb;
      plo[e] = static_cast<__bf16>(v - static_cast<float>(hb));
    }
    // B operand of tile t: element e is V[k slot e][CW j + t], the t-th bf16 of row
    // piece e; pairs of k slots share a 32-bit word.
#pragma unroll
    for (int t = 0; t < CW; ++t) {
      uint32_t w[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const uint32_t a0 = bf.v[2 * e2][t >> 1], a1 = bf.v[2 * e2 + 1][t >> 1];
        w[e2] = (t & 1) ? ((a0 >> 16) | (a1 & 0xFFFF0000u)) : ((a0 & 0xFFFFu) | (a1 << 16));
      }
      const bf16x8_t vop = __builtin_bit_cast(bf16x8_t, make_uint4(w[0], w[1], w[2], w[3]));
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(phi, vop, o[t], 0, 0, 0);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(plo, vop, o[t], 0, 0, 0);
    }
  };

  // Steps alternate between two buffers; the step after next is issued once a buffer
  // is consumed.  The loop is entered and continued only with both buffers in flight
  // (ba older), so its waits leave the younger buffer's loads outstanding; the last
  // one or two steps are finished after it.  An issue past the wave's last step
  // reloads that step (cache hits, never used).  The scheduling barriers keep each
  // step's loads together where they are issued.
  auto stage_q = [&]() {
    sq[wave][0][lane] = q0;
    sq[wave][1][lane] = q1;
    if constexpr (KK == 4) {
      sq[wave][2][lane] = q2;
      sq[wave][3][lane] = q3;
    }
  };
  Buf ba, bb;
  if (my == 1) {
    issue(ba, 0);
    stage_q();
    compute(ba, 0);
  } else if (my > 1) {
    __builtin_amdgcn_sched_barrier(0);
    issue(ba, 0);
    __builtin_amdgcn_sched_barrier(0);
    issue(bb, 1);
    __builtin_amdgcn_sched_barrier(0);
    stage_q();
    int64_t i = 0;
    for (; i + 2 < my; i += 2) {
      compute(ba, i);
      issue(ba, i + 2);
      __builtin_amdgcn_sched_barrier(0);
      compute(bb, i + 1);
      issue(bb, i + 3);
      __builtin_amdgcn_sched_barrier(0);
    }
    compute(ba, i);
    if (i + 1 < my) compute(bb, i + 1);
  }

  // head j's sum over the four lane rows; all rows already share the running max
  l_run += xor_partner<16>(l_run, lane);
  l_run += xor_partner<32>(l_run, lane);
  if (h == 0 && j < G) {
    sm_m[wave][j] = m_run;
    sm_l[wave][j] = l_run;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 4 * h + r;
    if (q < G) {
#pragma unroll
      for (int t = 0; t < CW; ++t) sm_o[wave][q][CW * j + t] = o[t][r];
    }
  }
  __syncthreads();
  finish_rows<ActBF16, D, G, NW>(p, sm_m, sm_l, sm_o, last, qr, g, split, nsplit);
}

// ---- prefill / chunked prefill: many query rows, bf16, both products on MFMA ----
//
// One block owns QB consecutive query positions of one (row, kv head): NW waves, each
// with CG column groups of 16 MFMA columns (16/G positions x the G query heads of the
// kv group), so a K/V load serves G heads and NW*CG*16/G positions.  The block walks
// the key positions up to its last query's position in tiles of 32:
//   * Tile t+2 is loaded into registers while tile t is computed and tile t+1 waits in
//     LDS (two-deep prefetch; a tile is one cache block lookup, tiles start at
//     multiples of 32).  K is stored row-major and V transposed (V^T[d][key]); both are
//     XOR-swizzled in 16-byte slots, so the operand reads below are conflict-free.
//   * Scores S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with the key rows of score tile tt
//     permuted: MFMA row i is key 8(i/4) + 4 tt + i%4.  Lane (j, h) then holds the
//     scores of query column j for keys 8h .. 8h+7 (tile tt = 0 gives 8h..8h+3, tt = 1
//     gives 8h+4..8h+7): exactly the k slots of its A operand in P V, and its V operand
//     for output tile dt is V^T[16 dt + j][8h .. 8h+7], one 16-byte LDS read.  K and V
//     operands are read once per wave and shared by the wave's column groups.
//   * The causal mask is per column (key <= the column's position, key < the chunk
//     end), the online softmax is base 2 per column (scores pre-scaled by
//     log2(e)/sqrt(d)), P is split into bf16 hi + lo for the P V product.  Within a
//     key group waves own distinct queries: each wave normalises its columns and
//     writes them.
// Blocks are numbered kv head fastest: block b runs on XCD b % 8, so with 8 kv heads
// every block of one head shares one XCD's L2 (the head's K/V is read from HBM once),
// and the query blocks of a head are taken last-first (the longest causal ranges start
// first).
// KS = 2 runs two groups of NW waves over the same queries: group k takes the key
// tiles t with t % 2 == k through its own LDS buffers, and at the end the second
// group's softmax states are merged into the first's through LDS.  A block then keeps
// two waves per SIMD busy on half the tiles each, for launches that give a CU only one
// 4-wave block.
constexpr int kPreTile = 32;

// 16-byte slot of K row `key` holding dims 8s .. 8s+7 (s ^ this): the 16 rows of one
// score MFMA operand fall into 16 distinct slots.
template <int D>
__device__ __forceinline__ int kswz(int key) {
  if constexpr (D == 128)
    return (key & 3) | ((key >> 3) << 2);
  else
    return ((key >> 1) & 1) | ((key >> 3) << 1);
}
// 16-byte slot of V^T row d holding keys 8s .. 8s+7 (s ^ this)
__device__ __forceinline__ int vswz(int d) { return (d >> 2) & 3; }

template <int D, int G, int CG, int NW, int KS>
__global__ __launch_bounds__(NW * 64 * KS) void attention_prefill_kernel(AttnArgs p) {
  static_assert(KS == 1 || KS == 2, "one or two key groups");
  constexpr int NT = NW * 64;                // threads of one key group
  constexpr int QT = 16 / G;               // query positions per column group
  constexpr int QB = NW * CG * QT;         // query positions per block
  constexpr int KK = D / 32;               // MFMA k steps of one score tile
  constexpr int DT = D / 16;               // 16-wide output tiles
  constexpr int TP = kPreTile;             // key positions per tile
  constexpr int PR = D / 8;                // 16-byte pieces per cache row
  constexpr int PCH = TP * PR / NT;        // pieces per thread per tile (K and V each)
  static_assert(PCH >= 1 && TP * PR % NT == 0, "tile pieces must divide over the block");
  typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
  typedef __attribute__((ext_vector_type(4))) float f32x4_t;
  // per key group, two buffers each of K[key][d] and V^T[d][key], 16-byte slots swizzled
  __shared__ __align__(16) uint16_t sk_[KS][2][TP * D];
  __shared__ __align__(16) uint16_t sv_[KS][2][D * TP];

  // key group kg of the thread, and its index within the group
  const int kg = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / NT);
  auto sk = [&](int buf) { return &sk_[kg][buf][0]; };
  auto sv = [&](int buf) { return &sv_[kg][buf][0]; };
  const int tid = KS == 1 ? static_cast<int>(threadIdx.x) : static_cast<int>(threadIdx.x) % NT, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int j = lane & 15, h = lane >> 4;
  // block -> (row, q block, kv head): kv head fastest, q blocks last-first
  const int64_t nqb = (p.seq + QB - 1) / QB;
  const int64_t L = blockIdx.x;
  const int64_t g = L % p.hkv;
  const int64_t rest = L / p.hkv;
  const int64_t b = rest / nqb;
  const int64_t s0 = (nqb - 1 - rest % nqb) * QB;
  const int64_t start = p.start_dev != nullptr ? p.start_dev[b] : p.start;
  const int64_t s_last = s0 + QB - 1 < p.seq - 1 ? s0 + QB - 1 : p.seq - 1;
  int64_t kend = start + s_last + 1;  // keys the block needs: [0, kend)
  if (kend > p.cap) kend = p.cap;
  const int64_t ntiles = (kend + TP - 1) / TP;

  // column group c of this wave: positions s0 + (wave * CG + c) * QT + j / G; its score
  // B operand (query column j at d = 32 kk + 8 h .. +8; zero for missing queries)
  int64_t qpos[CG];
  bf16x8_t qop[CG][KK];
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    const int64_t s = s0 + (wave * CG + c) * QT + j / G;
    qpos[c] = s < p.seq ? start + s : -1;
    const int64_t sq = s < p.seq ? s : p.seq - 1;
    const uint16_t* qp =
        static_cast<const uint16_t*>(p.q) + ((b * p.seq + sq) * p.hq + g * G + j % G) * D + 8 * h;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      uint4 v = *reinterpret_cast<const uint4*>(qp + 32 * kk);
      if (qpos[c] < 0) v = make_uint4(0, 0, 0, 0);
      qop[c][kk] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  const uint16_t* kc0 = static_cast<const uint16_t*>(p.kc);
  const uint16_t* vc0 = static_cast<const uint16_t*>(p.vc);
  const int64_t last_row = kend - 1;
  // K piece c of the thread: tile row (tid / PR + c * NT / PR), dims 8 (tid % PR) .. +8
  // (a wave's lanes cover whole rows: row-major 16-byte LDS stores).  V piece c: key
  // q % 32, dims 8 (q / 32) .. +8 for q = c * NT + tid (a wave's lanes cover all 32 keys
  // of two 8-dim blocks, so the transposed 2-byte stores of one instruction fall into
  // two V^T rows rather than sixteen).  A tile's 32 rows are contiguous from its first
  // row (one offset lookup per tile).
  typedef u32x4_t Pieces[2][PCH];  // a vector type: copies stay in registers
  Pieces ra, rb;
  auto load_tile = [&](Pieces& r, int64_t t) {
    const int64_t off = p.kv.Row(b, g, t * TP);
    const uint32_t lim = static_cast<uint32_t>(min(last_row - t * TP, int64_t{TP - 1}));
#pragma unroll
    for (int c = 0; c < PCH; ++c) {
      const uint32_t row = min(static_cast<uint32_t>(tid / PR + c * (NT / PR)), lim);
      r[0][c] = *reinterpret_cast<const u32x4_t*>(kc0 + off + (row * D + 8 * (tid % PR)));
      const int q = c * NT + tid;
      const uint32_t vrow = min(static_cast<uint32_t>(q % TP), lim);
      r[1][c] = *reinterpret_cast<const u32x4_t*>(vc0 + off + (vrow * D + 8 * (q / TP)));
    }
  };
  auto store_tile = [&](const Pieces& r, int buf) {
#pragma unroll
    for (int c = 0; c < PCH; ++c) {
      const int key = tid / PR + c * (NT / PR), sl = tid % PR;
      *reinterpret_cast<u32x4_t*>(sk(buf) + key * D + 8 * (sl ^ kswz<D>(key))) = r[0][c];
      const int q = c * NT + tid, vkey = q % TP, vsl = q / TP;
      const uint32_t w[4] = {r[1][c].x, r[1][c].y, r[1][c].z, r[1][c].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 8 * vsl + e;
        sv(buf)[d * TP + 8 * ((vkey >> 3) ^ vswz(d)) + (vkey & 7)] =
            static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu));
      }
    }
  };

  // the wave's columns: all present, and the smallest position among them
  const int64_t wave_s0 = s0 + wave * CG * QT;
  const bool wave_full = wave_s0 + CG * QT - 1 < p.seq;
  const int64_t wave_qmin = start + wave_s0;
  float m_run[CG], l_run[CG];
  f32x4_t o[CG][DT];  // O[column 4h + r][16 dt + j]
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    m_run[c] = -INFINITY;
    l_run[c] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[c][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](int buf, int64_t t) {
    const uint16_t* kt = sk(buf);
    const uint16_t* vt = sv(buf);
    f32x4_t acc[CG][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int key = 8 * (j >> 2) + 4 * tt + (j & 3);  // this lane's A row
#pragma unroll
      for (int c = 0; c < CG; ++c) acc[c][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const uint4 a = *reinterpret_cast<const uint4*>(kt + key * D + 8 * ((4 * kk + h) ^ kswz<D>(key)));
#pragma unroll
        for (int c = 0; c < CG; ++c)
          acc[c][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), qop[c][kk], acc[c][tt],
                                                               0, 0, 0);
      }
    }
    // Tiles wholly below every column's position and the chunk end need no mask (all
    // but the last one or two tiles of a block); the test is wave-uniform.
    const bool full = wave_full && t * TP + TP - 1 <= wave_qmin && t * TP + TP <= kend;
    const int32_t tbase = static_cast<int32_t>(t * TP) + 8 * h;
    bf16x8_t phi[CG], plo[CG];
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      // lane (j, h), slot e = 4 tt + r: key 8h + e of query column j
      float sc[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) sc[e] = acc[c][e >> 2][e & 3] * p.scale;
      if (!full) {
        const int32_t lim = static_cast<int32_t>(min(qpos[c], kend - 1));  // keys <= lim are live
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (tbase + e > lim) sc[e] = -INFINITY;
      }
      float bm = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) bm = fmaxf(bm, sc[e]);
      bm = fmaxf(bm, xor_partner<16>(bm, lane));
      bm = fmaxf(bm, xor_partner<32>(bm, lane));
      const float mn = fmaxf(m_run[c], bm);
      // Rescale only when some column's maximum grew (multiplying by exp2(0) = 1 is
      // exact, so skipping it changes nothing); after the first tiles this is rare.
      if (__builtin_amdgcn_ballot_w64(mn > m_run[c]) != 0) {
        const float cf = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m_run[c] - mn);
        l_run[c] *= cf;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float cr = __shfl(cf, 16 * h + 4 * h + r);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[c][dt][r] *= cr;
        }
      }
      m_run[c] = mn;
      float sum = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = sc[e] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[e] - mn);
        sum += v;
        const __bf16 hb = static_cast<__bf16>(v);
        phi[c][e] = hb;
        plo[c][e] = static_cast<__bf16>(v - static_cast<float>(hb));
      }
      l_run[c] += sum;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d = 16 * dt + j;
      const bf16x8_t vop =
          __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(vt + d * TP + 8 * (h ^ vswz(d))));
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        o[c][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(phi[c], vop, o[c][dt], 0, 0, 0);
        o[c][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(plo[c], vop, o[c][dt], 0, 0, 0);
      }
    }
  };

  if constexpr (KS == 1) {
    // tile t: in LDS buffer t & 1; its registers were loaded two iterations earlier
    load_tile(ra, 0);
    if (ntiles > 1) load_tile(rb, 1);
    store_tile(ra, 0);
    __syncthreads();
    int64_t t = 0;
    for (; t + 1 < ntiles; t += 2) {
      // even tile t in buffer 0; rb holds tile t + 1
      if (t + 2 < ntiles) load_tile(ra, t + 2);
      compute(0, t);
      store_tile(rb, 1);
      __syncthreads();
      if (t + 3 < ntiles) load_tile(rb, t + 3);
      compute(1, t + 1);
      if (t + 2 < ntiles) store_tile(ra, 0);
      __syncthreads();
    }
    if (t < ntiles) compute(0, t);
  } else {
    // The group's u-th tile is tile u KS + kg, in LDS buffer u & 1, loaded as above.
    // Every group runs the loop of the group with the most tiles (the first), so all
    // threads meet at the same barriers.
    const int64_t nu = (ntiles + KS - 1) / KS;                            // group 0's tiles
    const int64_t nmine = ntiles > kg ? (ntiles - kg + KS - 1) / KS : 0;  // this group's
    auto gt = [&](int64_t u) { return u * KS + kg; };
    if (nmine > 0) load_tile(ra, gt(0));
    if (nmine > 1) load_tile(rb, gt(1));
    if (nmine > 0) store_tile(ra, 0);
    __syncthreads();
    int64_t u = 0;
    for (; u + 1 < nu; u += 2) {
      if (u + 2 < nmine) load_tile(ra, gt(u + 2));
      if (u < nmine) compute(0, gt(u));
      if (u + 1 < nmine) store_tile(rb, 1);
      __syncthreads();
      if (u + 3 < nmine) load_tile(rb, gt(u + 3));
      if (u + 1 < nmine) compute(1, gt(u + 1));
      if (u + 2 < nmine) store_tile(ra, 0);
      __syncthreads();
    }
    if (u < nmine) compute(0, gt(u));
  }

  if constexpr (KS == 2) {
    // the second group's states into LDS (lane-contiguous words per wave: o in the K
    // buffers, m and l in the V buffers), merged into the first group's on the same lanes
    constexpr int OW = CG * DT * 4;  // o words per lane
    static_assert(NW * OW * 64 * 4 <= static_cast<int>(sizeof(sk_)) &&
                      NW * 2 * CG * 64 * 4 <= static_cast<int>(sizeof(sv_)),
                  "merge records fit the tile buffers");
    float* reco = reinterpret_cast<float*>(&sk_[0][0][0]) + wave * OW * 64 + lane;
    float* recm = reinterpret_cast<float*>(&sv_[0][0][0]) + wave * 2 * CG * 64 + lane;
    __syncthreads();  // every group is done with its tiles
    if (kg == 1) {
#pragma unroll
      for (int c = 0; c < CG; ++c) {
        recm[(2 * c) * 64] = m_run[c];
        recm[(2 * c + 1) * 64] = l_run[c];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) reco[((c * DT + dt) * 4 + r) * 64] = o[c][dt][r];
      }
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int c = 0; c < CG; ++c) {
      // column j's scale factors (every lane of the column holds its maximum)
      const float m2 = recm[(2 * c) * 64], l2 = recm[(2 * c + 1) * 64];
      const float mn = fmaxf(m_run[c], m2);
      const float f1 = m_run[c] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[c] - mn);
      const float f2 = m2 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m2 - mn);
      l_run[c] = l_run[c] * f1 + l2 * f2;
      m_run[c] = mn;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // o[..][r] is column 4h + r: that column's factors
        const float c1 = __shfl(f1, 16 * h + 4 * h + r), c2 = __shfl(f2, 16 * h + 4 * h + r);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          o[c][dt][r] = o[c][dt][r] * c1 + reco[((c * DT + dt) * 4 + r) * 64] * c2;
      }
    }
  }

  // column j's sum over the four lane rows, then normalise and write
#pragma unroll
  for (int c = 0; c < CG; ++c) {
    float lr = l_run[c];
    lr += xor_partner<16>(lr, lane);
    lr += xor_partner<32>(lr, lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int q = 4 * h + r;  // this lane's output column
      const float lq = __shfl(lr, 16 * h + q);
      const int64_t sq = s0 + (wave * CG + c) * QT + q / G;
      if (sq >= p.seq) continue;
      uint16_t* out = static_cast<uint16_t*>(p.out) + ((b * p.seq + sq) * p.hq + g * G + q % G) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) out[16 * dt + j] = f32_to_bf16_bits(lq > 0.0f ? o[c][dt][r] / lq : 0.0f);
    }
  }
}

int64_t GridBlocks(dim3 g) { return static_cast<int64_t>(g.x) * g.y * g.z; }

// Launches through the dispatch-timing hook when the thread has armed it (the decode
// profile), so its events bracket exactly this dispatch.
template <class K>
void LaunchTimed(K kernel, dim3 grid, dim3 block, hipStream_t s, const AttnArgs& a) {
  LaunchTiming& lt = ThreadLaunchTiming();
  if (lt.start != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, lt.start, lt.stop, 0, a);
    lt.used = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, a);
  }
}

template <int D, int G, int CG, int NW, int KS>
void LaunchPrefillShape(int64_t blocks, const AttnArgs& a, hipStream_t s) {
  constexpr int QB = NW * CG * (16 / G);
  if constexpr (KS == 1)
    RecordLaunch(blocks, NW * 64, 0, "attention_prefill<d=%d,g=%d,qb=%d>", D, G, QB);
  else
    RecordLaunch(blocks, NW * 64 * KS, 0, "attention_prefill<d=%d,g=%d,qb=%d,ks=%d>", D, G, QB, KS);
  LaunchTimed(attention_prefill_kernel<D, G, CG, NW, KS>, dim3(static_cast<unsigned>(blocks)), dim3(NW * 64 * KS), s,
              a);
}

// Query positions per block: the largest of 16/G x {4, 8, 16} that still gives every CU
// a block (fewer re-reads of K/V per query), else the smallest, as two key groups of
// four waves.
template <int D, int G>
void LaunchPrefillG(const AttnArgs& a, int64_t batch, hipStream_t s) {
  const int64_t per = a.hkv * batch, cus = DeviceCUs();
  auto blocks = [&](int64_t qb) { return CeilDiv(a.seq, qb) * per; };
  constexpr int QT = 16 / G;
  // (a 512-thread block needs a whole 16-byte piece per thread per tile: D = 128)
  if (D == 128 && blocks(16 * QT) >= cus)
    LaunchPrefillShape<D, G, 2, D == 128 ? 8 : 4, 1>(blocks(16 * QT), a, s);
  else if (blocks(8 * QT) >= cus)
    LaunchPrefillShape<D, G, 2, 4, 1>(blocks(8 * QT), a, s);
  else
    LaunchPrefillShape<D, G, 1, 4, 2>(blocks(4 * QT), a, s);
}

template <int D>
am_status_code LaunchPrefill(int64_t G, int64_t batch, const AttnArgs& a, hipStream_t s) {
  switch (G) {
    case 1: LaunchPrefillG<D, 1>(a, batch, s); break;
    case 2: LaunchPrefillG<D, 2>(a, batch, s); break;
    case 4: LaunchPrefillG<D, 4>(a, batch, s); break;
    case 8: LaunchPrefillG<D, 8>(a, batch, s); break;
    default: return SetLastError(AM_STATUS_UNIMPLEMENTED, "attention: q heads per kv head must be 1, 2, 4 or 8");
  }
  AM_RETURN_IF_LAUNCH_FAILED("attention");
  return AM_STATUS_OK;
}

int ChooseSplits(int64_t seq, int64_t cap, int32_t requested) {
  if (requested > 0) return requested;
  if (seq > 1) return 1;
  int64_t s = cap / kMinPerSplit;
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return static_cast<int>(s);
}

template <int D, int NW>
am_status_code LaunchDecode(int64_t G, dim3 grid, const AttnArgs& a, hipStream_t s) {
  if constexpr (NW == kDecWaves)
    RecordLaunch(GridBlocks(grid), NW * 64, 0, "attention_decode<d=%d,g=%d,splits=%u>", D, static_cast<int>(G),
                 grid.x);
  else
    RecordLaunch(GridBlocks(grid), NW * 64, 0, "attention_decode<d=%d,g=%d,splits=%u,waves=%d>", D,
                 static_cast<int>(G), grid.x, NW);
  const dim3 block(NW * 64);
  switch (G) {
    case 1: LaunchTimed(attention_decode_kernel<D, 1, NW>, grid, block, s, a); break;
    case 2: LaunchTimed(attention_decode_kernel<D, 2, NW>, grid, block, s, a); break;
    case 4: LaunchTimed(attention_decode_kernel<D, 4, NW>, grid, block, s, a); break;
    case 8: LaunchTimed(attention_decode_kernel<D, 8, NW>, grid, block, s, a); break;
    default: return SetLastError(AM_STATUS_UNIMPLEMENTED, "attention: q heads per kv head must be 1, 2, 4 or 8");
  }
  AM_RETURN_IF_LAUNCH_FAILED("attention");
  return AM_STATUS_OK;
}

template <class A, int D>
am_status_code LaunchD(int64_t G, dim3 grid, const AttnArgs& a, hipStream_t s) {
  RecordLaunch(GridBlocks(grid), kWaves * 64, 0, "attention_valu<%s,d=%d,g=%d,splits=%u>",
               A::kDtype == AM_DT_BF16 ? "bf16" : "f32", D, static_cast<int>(G), grid.x);
  switch (G) {
    case 1: LaunchTimed(attention_kernel<A, D, 1>, grid, dim3(kWaves * 64), s, a); break;
    case 2: LaunchTimed(attention_kernel<A, D, 2>, grid, dim3(kWaves * 64), s, a); break;
    case 4: LaunchTimed(attention_kernel<A, D, 4>, grid, dim3(kWaves * 64), s, a); break;
    case 8: LaunchTimed(attention_kernel<A, D, 8>, grid, dim3(kWaves * 64), s, a); break;
    default: return SetLastError(AM_STATUS_UNIMPLEMENTED, "attention: q heads per kv head must be 1, 2, 4 or 8");
  }
  AM_RETURN_IF_LAUNCH_FAILED("attention");
  return AM_STATUS_OK;
}

}  // namespace
}  // namespace am

using namespace am;

extern "C" int64_t am_gfx950_attention_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv,
                                                       int64_t head_dim, int64_t capacity, int32_t num_splits) {
  const int splits = ChooseSplits(seq, capacity, num_splits);
  if (splits == 1) return 0;
  const int64_t tickets = 256 * CeilDiv(batch * seq * hkv * 4, 256);
  return tickets + batch * seq * hq * splits * (head_dim + 4) * 4;
}

// ---- zero-allocation variant -----------------------------------------------------
// The split tickets and records live in this file-scope device array instead of a
// caller workspace.  Its name is only a host-side handle: host code uses the address
// hipGetSymbolAddress returns for the current device (each device holds its own copy).
constexpr int64_t kNoAllocScratchBytes = int64_t{8} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

__global__ void scratch_zero_kernel(uint32_t* p, int64_t words) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < words) p[i] = 0u;
}

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up once per device.
am_status_code ScratchAddress(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return SetLastError(AM_STATUS_INTERNAL, "attention_noalloc: no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return SetLastError(AM_STATUS_INTERNAL, "attention_noalloc: hipGetSymbolAddress(scratch) failed");
    g_scratch_dev[dev] = ptr;
  }
  *out = g_scratch_dev[dev];
  return AM_STATUS_OK;
}
}  // namespace

extern "C" int64_t am_gfx950_attention_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" am_status_code am_gfx950_attention_noalloc(const am_gfx950_attention_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "attention_noalloc: null args");
  AM_CHECK_ARG(a->workspace == nullptr && a->workspace_bytes == 0,
               "attention_noalloc: pass no workspace (the split records use the library's device scratch)");
  AM_CHECK_ARG(a->hq > 0 && a->hkv > 0 && a->seq > 0 && a->capacity > 0 && a->head_dim > 0,
               "attention_noalloc: bad shape");
  const int64_t batch = a->batch > 0 ? a->batch : 1;
  AM_CHECK_ARG(batch * a->seq <= 65535, "attention: too many query rows");
  const int64_t need = am_gfx950_attention_workspace_bytes(batch, a->seq, a->hq, a->hkv, a->head_dim, a->capacity,
                                                           a->num_splits);
  if (need > kNoAllocScratchBytes) {
    char msg[160];
    std::snprintf(msg, sizeof(msg), "attention_noalloc: needs %lld bytes of split scratch, the maximum is %lld",
                  static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
    return SetLastError(AM_STATUS_RESOURCE_EXHAUSTED, msg);
  }
  hipStream_t s = AsStream(stream);
  if (s != nullptr) {
    int cur = -1, sdev = -1;
    if (hipGetDevice(&cur) != hipSuccess || hipStreamGetDevice(s, &sdev) != hipSuccess || cur != sdev)
      return SetLastError(AM_STATUS_INVALID_ARGUMENT, "attention_noalloc: the stream's device is not the current device");
  }
  am_gfx950_attention_args b = *a;
  if (need > 0) {
    void* ptr = nullptr;
    if (auto st = ScratchAddress(&ptr); st != AM_STATUS_OK) return st;
    // the tickets must start at zero: clear them with a kernel (capturable, no memset)
    const int64_t ticket_words = 64 * CeilDiv(batch * a->seq * a->hkv * 4, 256);
    hipLaunchKernelGGL(scratch_zero_kernel, dim3(static_cast<unsigned>(CeilDiv(ticket_words, 256))), dim3(256), 0, s,
                       static_cast<uint32_t*>(ptr), ticket_words);
    AM_RETURN_IF_LAUNCH_FAILED("attention_noalloc");
    b.workspace = ptr;
    b.workspace_bytes = kNoAllocScratchBytes;
  }
  return am_gfx950_attention(&b, stream);
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
  if (auto st = MakeKvRows(a->pages, p.cbs, a->capacity, a->hkv, a->head_dim, &p.kv); st != AM_STATUS_OK) return st;
  if (a->pages != nullptr)
    AM_CHECK_ARG(a->dtype == AM_DT_BF16, "attention: a paged KV cache needs bf16 activations");
  p.splits = splits;
  p.scale = kLog2e / sqrtf(static_cast<float>(a->head_dim));
  if (splits > 1) {
    uint8_t* ws = static_cast<uint8_t*>(a->workspace);
    p.tickets = reinterpret_cast<unsigned*>(ws);
    p.part = reinterpret_cast<float*>(ws + 256 * CeilDiv(batch * a->seq * a->hkv * 4, 256));
  }
  const int64_t G = a->hq / a->hkv;
  hipStream_t s = AsStream(stream);
  if (a->dtype == AM_DT_BF16 && a->seq == 1) {
    AM_CHECK_ARG(a->capacity * a->head_dim < (int64_t{1} << 31), "attention: cache too large for 32-bit offsets");
    // decode: MFMA kernel; an explicit split request is honoured down to 32 positions
    p.min_per_split = a->num_splits > 0 ? 32 : kDecMinPerSplit;
    if (a->num_splits <= 0 && p.splits > kDecMaxSplits) p.splits = kDecMaxSplits;
    const dim3 grid(static_cast<unsigned>(p.splits), static_cast<unsigned>(a->hkv), static_cast<unsigned>(batch));
    // Grids that give every CU a block (batched long contexts) run 8-wave blocks, two
    // waves per SIMD: twice the K/V loads in flight per CU, merged in LDS.
    if (a->num_splits <= 0 && GridBlocks(grid) >= DeviceCUs())
      return a->head_dim == 128 ? LaunchDecode<128, 8>(G, grid, p, s) : LaunchDecode<64, 8>(G, grid, p, s);
    return a->head_dim == 128 ? LaunchDecode<128, kDecWaves>(G, grid, p, s)
                              : LaunchDecode<64, kDecWaves>(G, grid, p, s);
  }
  if (a->dtype == AM_DT_BF16) {
    // prefill: MFMA kernel, one block per (16 query columns per wave) x kv head x row
    AM_CHECK_ARG(a->capacity * a->head_dim < (int64_t{1} << 31), "attention: cache too large for 32-bit offsets");
    return a->head_dim == 128 ? LaunchPrefill<128>(G, batch, p, s) : LaunchPrefill<64>(G, batch, p, s);
  }
  // fp32 activations: the VALU kernel
  const dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(a->hkv), static_cast<unsigned>(batch * a->seq));
  p.min_per_split = static_cast<int32_t>(kMinPerSplit);
  return a->head_dim == 128 ? LaunchD<ActF32, 128>(G, grid, p, s) : LaunchD<ActF32, 64>(G, grid, p, s);
}
