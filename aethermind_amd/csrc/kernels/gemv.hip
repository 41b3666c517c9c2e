// Decode-time (m = 1) weight-only GEMV for gfx950, HBM-bound.
//
// Layout of one launch:
//   * 256-thread blocks (4 wave64s).  The block stages the activation vector x (K
//     values) in LDS once, optionally applying the fused RMSNorm prologue, together
//     with one offset-correction term per 16-byte weight chunk.
//   * Work unit = a pair of output rows (RoPE pair, gate/up pair or two plain rows);
//     an iteration of a wave handles P pairs.  All 64 lanes of the wave read every
//     row: lane l owns the 16-byte chunks l, l+64, ... of each row, so each load
//     instruction moves 1 KiB of contiguous weights.  The lane -> chunk map is fixed,
//     so each lane copies its share of x from LDS into registers once and the inner
//     loop touches no LDS at all.
//   * For short rows (K <= 8192 INT4) the next iteration's weight loads are issued
//     before the current one is reduced (two register buffers), so every wave keeps
//     its rows' bytes in flight; long rows keep all their chunks in flight instead.
//   * Unpack is in registers: INT4 nibbles hold q+8, and (word >> 4t) & 0x000F000F
//     | 0x43004300 is the bf16 pair (136+q_even, 136+q_odd), fed to
//     v_dot2c_f32_bf16 with the bf16 activations; sum(x*(136+q)) - 136*sum(x) gives
//     sum(x*q) in fp32, then the fp16 group scale is applied per chunk.
//   * Row sums are reduced with DPP row rotations plus four readlanes; the epilogue
//     applies the reference op-boundary roundings of the nodes that were fused.

#include <cmath>

#include "am_kernel_common.h"

namespace am {
namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

enum Epi { kEpiStore = 0, kEpiResidual = 1, kEpiQkv = 2, kEpiGateUp = 3, kEpiLmHead = 4 };

struct GemvArgs {
  const void* x;
  const void* norm_w;
  float eps;
  const uint8_t* w;
  const void* scales;
  int64_t n, k;
  int32_t group;
  int64_t units;  // row pairs
  int64_t row_bytes;
  void* out;
  const void* residual;
  const float* cos_tab;
  const float* sin_tab;
  const int64_t* pos;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int32_t hq, hkv, d;
  int64_t cap;
  int64_t* token_out;
  int64_t* tokens_hist;
  int64_t* pos_inc;
  int64_t* step;
  unsigned* ticket;
  float* pv;
  int64_t* pi;
  int32_t out_f32;
};

// k values per 16-byte chunk of a weight row
template <int WF> struct Fmt;
template <> struct Fmt<AM_WF_F32> { static constexpr int kc = 4; static constexpr float off = 0.0f; };
template <> struct Fmt<AM_WF_BF16> { static constexpr int kc = 8; static constexpr float off = 0.0f; };
template <> struct Fmt<AM_WF_INT8> { static constexpr int kc = 16; static constexpr float off = 128.0f; };
template <> struct Fmt<AM_WF_INT4> { static constexpr int kc = 32; static constexpr float off = 8.0f; };

// x is kept as bf16 only where the dot uses v_dot2c_f32_bf16 (bf16 activations with
// bf16 or INT4 weights); elsewhere as fp32.
template <class A, int WF> struct XStore {
  static constexpr bool kBF16 = A::kDtype == AM_DT_BF16 && (WF == AM_WF_INT4 || WF == AM_WF_BF16);
  static constexpr int kBytes = kBF16 ? 2 : 4;
  static constexpr int kDW = Fmt<WF>::kc * kBytes / 4;  // dwords of x per weight chunk
  // offset subtracted per chunk: the bf16 INT4 path also carries the 128 exponent bias
  static constexpr float kOff = (kBF16 && WF == AM_WF_INT4) ? 136.0f : Fmt<WF>::off;
};

__device__ __forceinline__ bf16x2_t as_bf2(uint32_t u) { return __builtin_bit_cast(bf16x2_t, u); }

// Dot of one 16-byte weight chunk with its x values (kDW dwords at xd).
template <class A, int WF>
__device__ __forceinline__ float chunk_dot(const uint4 w, const uint32_t* xd) {
  using XS = XStore<A, WF>;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float acc = 0.0f;
  if constexpr (XS::kBF16) {
    if constexpr (WF == AM_WF_INT4) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
          const uint32_t pair = ((ws[t] >> (4 * pp)) & 0x000F000Fu) | 0x43004300u;
          acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(xd[4 * t + pp]), as_bf2(pair), acc, false);
        }
    } else {  // BF16 weights
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(xd[t]), as_bf2(ws[t]), acc, false);
    }
  } else {
    const float* xf = reinterpret_cast<const float*>(xd);
    if constexpr (WF == AM_WF_F32) {
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = fmaf(xf[t], __uint_as_float(ws[t]), acc);
    } else if constexpr (WF == AM_WF_BF16) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        acc = fmaf(xf[2 * t], __uint_as_float(ws[t] << 16), acc);
        acc = fmaf(xf[2 * t + 1], __uint_as_float(ws[t] & 0xFFFF0000u), acc);
      }
    } else if constexpr (WF == AM_WF_INT8) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int b = 0; b < 4; ++b)
          acc = fmaf(xf[4 * t + b], static_cast<float>((ws[t] >> (8 * b)) & 0xFFu), acc);
    } else {  // INT4, fp32 activations: nibble j of word t is k = 8t + {0,2,4,6,1,3,5,7}[j]
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kk = 8 * t + ((j < 4) ? 2 * j : 2 * (j - 4) + 1);
          acc = fmaf(xf[kk], static_cast<float>((ws[t] >> (4 * j)) & 0xFu), acc);
        }
    }
  }
  return acc;
}

// Sum over the 64 lanes: DPP inside each 16-lane row (quad swaps, then row
// rotations by 4 and 8), then the four row sums through readlane.  The result is
// wave-uniform.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
  const int b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

__device__ __forceinline__ float silu_ref(float g) {
  if (g >= 0.0f) return g / (1.0f + expf(-g));
  const float e = expf(g);
  return g * e / (1.0f + e);
}

// rows of pair u
template <int EPI>
__device__ __forceinline__ void pair_rows(const GemvArgs& p, int64_t u, int64_t& r0, int64_t& r1) {
  if constexpr (EPI == kEpiQkv) {
    const int64_t half = p.d / 2;
    const int64_t head = u / half, i = u % half;
    r0 = head * p.d + i;
    r1 = r0 + half;
  } else if constexpr (EPI == kEpiGateUp) {
    r0 = u;  // gate row u, up row u: rows [0, F) are gate, [F, 2F) are up
    r1 = u + p.n / 2;
  } else {
    r0 = 2 * u;
    r1 = 2 * u + 1;
  }
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// One load block: JB chunk-steps of both rows of P pairs (+ INT4 group scales).
template <int JB, int P, bool SC>
struct Frag {
  uint4 w[P][2][JB];
  uint32_t s[P][2][SC ? JB : 1];  // raw fp16 group-scale bits, converted at use
  float s8[P][2];                 // INT8 row scales
};

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}

// Streaming 16-byte weight load (read once per token: non-temporal hint).
__device__ __forceinline__ uint4 ld_stream(const uint8_t* row, int64_t c) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row) + c);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <class A, int WF, bool NORM, int EPI, int JM, int P>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs p) {
  using XS = XStore<A, WF>;
  using T = typename A::T;
  constexpr int kc = Fmt<WF>::kc;
  constexpr int XDW = XS::kDW;
  constexpr bool SC = WF == AM_WF_INT4;
  constexpr int JB = JM < 8 ? JM : 8;  // chunk-steps per load block
  constexpr int NB = JM / JB;          // load blocks per row
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[4];
  const int64_t K = p.k;
  const int64_t C = p.row_bytes / 16;  // chunks per row
  const int J = static_cast<int>((C + 63) / 64);
  // LDS: x | per-chunk corrections | residual (Residual epilogue) | cos,sin (Qkv epilogue)
  uint8_t* xl = smem;
  const int64_t off_corr = ((K * XS::kBytes + 15) / 16) * 16;
  const int64_t off_res = off_corr + ((C * 4 + 15) / 16) * 16;
  const int64_t off_cs = off_res + (EPI == kEpiResidual ? ((p.n * static_cast<int64_t>(sizeof(T)) + 15) / 16) * 16 : 0);
  float* corr_lds = reinterpret_cast<float*>(smem + off_corr);
  T* res_lds = reinterpret_cast<T*>(smem + off_res);
  float* cs_lds = reinterpret_cast<float*>(smem + off_cs);
  const int lane = threadIdx.x & 63;
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t TW = static_cast<int64_t>(gridDim.x) * 4;
  const int64_t niter = (p.units + P - 1) / P;
  const int ng = (WF == AM_WF_INT4) ? static_cast<int>(K / p.group) : 1;
  const int chunks_per_group = (WF == AM_WF_INT4) ? p.group / kc : 1;
  const uint16_t* sc16 = static_cast<const uint16_t*>(p.scales);

  // Loads chunk-steps [jb*JB, jb*JB + JB) of iteration `it` into f.  Every load is
  // unconditional (straight-line code, one wait at first use): out-of-range chunks
  // and rows read a clamped in-bounds address instead, and contribute nothing because
  // the lane's x registers for those chunks are zero and invalid rows are never
  // stored.
  auto issue = [&](Frag<JB, P, SC>& f, int64_t it, int jb) {
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
      int64_t u = it * P + pp;
      if (u >= p.units) u = p.units - 1;
      int64_t r0, r1;
      pair_rows<EPI>(p, u, r0, r1);
      if (r1 >= p.n) r1 = r0;
      const uint8_t* row0 = p.w + r0 * p.row_bytes;
      const uint8_t* row1 = p.w + r1 * p.row_bytes;
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int j = jb * JB + jj;
        int64_t c = lane + 64 * j;
        if (!(j < J && c < C)) c = 0;
        f.w[pp][0][jj] = ld_stream(row0, c);
        f.w[pp][1][jj] = ld_stream(row1, c);
        if constexpr (SC) {
          const int64_t g = c / chunks_per_group;
          f.s[pp][0][jj] = sc16[r0 * ng + g];
          f.s[pp][1][jj] = sc16[r1 * ng + g];
        }
      }
      if constexpr (WF == AM_WF_INT8) {
        if (jb == 0) {
          f.s8[pp][0] = static_cast<const float*>(p.scales)[r0];
          f.s8[pp][1] = static_cast<const float*>(p.scales)[r1];
        }
      }
    }
  };

  // Issue the first iteration's first load block before the prologue so HBM latency
  // overlaps the activation staging.
  Frag<JB, P, SC> fa;
  int64_t it = gw;
  if (it < niter) issue(fa, it, 0);

  // ---- prologue: x (optionally RMSNorm'd) -> LDS, per-chunk offset corrections ----
  const T* xin = static_cast<const T*>(p.x);
  float inv = 1.0f;
  if constexpr (NORM) {
    float ss = 0.0f;
    for (int64_t j = threadIdx.x; j < K; j += 256) {
      const float v = A::load(xin, j);
      ss = fmaf(v, v, ss);
    }
    ss = block_sum_256(ss, red);
    inv = 1.0f / sqrtf(ss / static_cast<float>(K) + p.eps);
  }
  const T* nw = static_cast<const T*>(p.norm_w);
  for (int64_t j = threadIdx.x; j < K; j += 256) {
    float v = A::load(xin, j);
    if constexpr (NORM) v = A::round((v * inv) * A::load(nw, j));
    if constexpr (XS::kBF16)
      reinterpret_cast<uint16_t*>(xl)[j] = f32_to_bf16_bits(v);
    else
      reinterpret_cast<float*>(xl)[j] = v;
  }
  // Epilogue operands come from LDS, so no global load is issued behind a prefetch
  // (the memory counter is in order: a later load would wait for the prefetch).
  // Each output row belongs to one wave, so staging the whole residual vector here
  // reads every row before its only writer updates it.
  int64_t posv = 0;
  if constexpr (EPI == kEpiResidual) {
    const T* res = static_cast<const T*>(p.residual);
    for (int64_t r = threadIdx.x; r < p.n; r += 256) res_lds[r] = res[r];
  }
  if constexpr (EPI == kEpiQkv) {
    posv = *p.pos;
    const int64_t half = p.d / 2;
    const int64_t pr = posv < p.cap ? posv : 0;
    for (int64_t i = threadIdx.x; i < half; i += 256) {
      cs_lds[i] = p.cos_tab[pr * half + i];
      cs_lds[half + i] = p.sin_tab[pr * half + i];
    }
  }
  __syncthreads();
  if constexpr (XS::kOff != 0.0f) {
    for (int64_t c = threadIdx.x; c < C; c += 256) {
      float s = 0.0f;
      for (int i = 0; i < kc; ++i) {
        const int64_t j = c * kc + i;
        s += XS::kBF16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(xl)[j])
                       : reinterpret_cast<const float*>(xl)[j];
      }
      corr_lds[c] = XS::kOff * s;
    }
    __syncthreads();
  }
  // this lane's x chunks into registers
  uint32_t xr[JM][XDW];
  float corr[JM];
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int64_t c = lane + 64 * j;
    const bool ok = j < J && c < C;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(xl) + c * XDW;
#pragma unroll
    for (int t = 0; t < XDW; ++t) xr[j][t] = ok ? src[t] : 0u;
    corr[j] = (XS::kOff != 0.0f && ok) ? corr_lds[c] : 0.0f;
  }

  float best_v = 0.0f;
  int64_t best_i = -1;

  // Accumulates load block jb of f into acc.
  auto accum = [&](const Frag<JB, P, SC>& f, int jb, float (&acc)[P][2]) {
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
#pragma unroll
      for (int jj = 0; jj < JB; ++jj) {
        const int j = jb * JB + jj;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          float dv = chunk_dot<A, WF>(f.w[pp][rr][jj], xr[j]);
          if constexpr (XS::kOff != 0.0f) dv -= corr[j];
          if constexpr (SC)
            acc[pp][rr] = fmaf(f16_bits_to_f32(f.s[pp][rr][jj]), dv, acc[pp][rr]);
          else
            acc[pp][rr] += dv;
        }
      }
      if constexpr (WF == AM_WF_INT8) {
        if (jb == NB - 1) {  // per-row scale after the last block of the row
          acc[pp][0] *= f.s8[pp][0];
          acc[pp][1] *= f.s8[pp][1];
        }
      }
    }
  };

  // Reduces acc across the wave and applies the epilogue of iteration itc.
  auto finish = [&](float (&acc)[P][2], int64_t itc) {
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
      acc[pp][0] = wave_sum_dpp(acc[pp][0]);
      acc[pp][1] = wave_sum_dpp(acc[pp][1]);
    }
#pragma unroll
    for (int pp = 0; pp < P; ++pp) {
      const int64_t u = itc * P + pp;
      if (u >= p.units) break;
      int64_t r0, r1;
      pair_rows<EPI>(p, u, r0, r1);
      const bool v1 = r1 < p.n;
      const float a0 = acc[pp][0], a1 = acc[pp][1];
      if constexpr (EPI == kEpiLmHead) {
        if (lane == 0) {
          float* lg = static_cast<float*>(p.out);
          if (lg != nullptr) {
            lg[r0] = a0;
            if (v1) lg[r1] = a1;
          }
        }
        if (argmax_better(a0, r0, best_v, best_i)) { best_v = a0; best_i = r0; }
        if (v1 && argmax_better(a1, r1, best_v, best_i)) { best_v = a1; best_i = r1; }
      } else if (lane == pp) {
        T* out = static_cast<T*>(p.out);
        if constexpr (EPI == kEpiStore) {
          if (p.out_f32) {
            float* of = static_cast<float*>(p.out);
            of[r0] = a0;
            if (v1) of[r1] = a1;
          } else {
            A::store(out, r0, a0);
            if (v1) A::store(out, r1, a1);
          }
        } else if constexpr (EPI == kEpiResidual) {
          A::store(out, r0, A::load(res_lds, r0) + A::round(a0));
          if (v1) A::store(out, r1, A::load(res_lds, r1) + A::round(a1));
        } else if constexpr (EPI == kEpiGateUp) {
          const float g = A::round(a0), up = A::round(a1);
          A::store(out, u, silu_ref(g) * up);
        } else if constexpr (EPI == kEpiQkv) {
          const int64_t half = p.d / 2;
          const int64_t head = u / half, i = u % half;
          const float y0 = A::round(a0), y1 = A::round(a1);
          if (head < p.hq + p.hkv) {
            const float c = cs_lds[i], s = cs_lds[half + i];
            const float o0 = y0 * c - y1 * s;
            const float o1 = y1 * c + y0 * s;
            if (head < p.hq) {
              T* q = static_cast<T*>(p.q_out);
              A::store(q, head * p.d + i, o0);
              A::store(q, head * p.d + i + half, o1);
            } else if (posv < p.cap) {
              T* kc = static_cast<T*>(p.k_cache);
              const int64_t base = ((head - p.hq) * p.cap + posv) * p.d;
              A::store(kc, base + i, o0);
              A::store(kc, base + i + half, o1);
            }
          } else if (posv < p.cap) {
            T* vc = static_cast<T*>(p.v_cache);
            const int64_t base = ((head - p.hq - p.hkv) * p.cap + posv) * p.d;
            A::store(vc, base + i, y0);
            A::store(vc, base + i + half, y1);
          }
        }
      }
    }
  };

  // Each iteration's loads are all issued before any of them is used; the next
  // iteration's first block is issued as soon as the registers are consumed, so its
  // latency overlaps the cross-lane reduction and the epilogue stores.
  while (it < niter) {
    float acc[P][2] = {};
#pragma unroll
    for (int jb = 0; jb < NB; ++jb) {
      if (jb > 0) issue(fa, it, jb);
      accum(fa, jb, acc);
    }
    const int64_t nx = it + TW;
    if (nx < niter) issue(fa, nx, 0);
    finish(acc, it);
    it = nx;
  }

  if constexpr (EPI == kEpiLmHead) {
    // block best -> partials; the last block (atomic ticket) reduces them, publishes
    // the token / advances the decode state, and resets the ticket for the next call.
    __shared__ float bv_s[4];
    __shared__ int64_t bi_s[4];
    __shared__ bool last;
    const int wave = threadIdx.x >> 6;
    if (lane == 0) {
      bv_s[wave] = best_v;
      bi_s[wave] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = 0.0f;
      int64_t bi = -1;
      for (int w = 0; w < 4; ++w)
        if (bi_s[w] >= 0 && argmax_better(bv_s[w], bi_s[w], bv, bi)) { bv = bv_s[w]; bi = bi_s[w]; }
      p.pv[blockIdx.x] = bv;
      p.pi[blockIdx.x] = bi;
      __threadfence();
      const unsigned t = atomicAdd(p.ticket, 1u);
      last = (t == gridDim.x - 1);
    }
    __syncthreads();
    if (last) {
      __threadfence();
      float bv = 0.0f;
      int64_t bi = -1;
      for (int64_t b = threadIdx.x; b < gridDim.x; b += 256) {
        const float v = __hip_atomic_load(&p.pv[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int64_t i = __hip_atomic_load(&p.pi[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (i >= 0 && argmax_better(v, i, bv, bi)) { bv = v; bi = i; }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int64_t oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && argmax_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
      }
      if (lane == 0) {
        bv_s[wave] = bv;
        bi_s[wave] = bi;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        float fv = 0.0f;
        int64_t fi = -1;
        for (int w = 0; w < 4; ++w)
          if (bi_s[w] >= 0 && argmax_better(bv_s[w], bi_s[w], fv, fi)) { fv = bv_s[w]; fi = bi_s[w]; }
        const int64_t tok = fi < 0 ? 0 : fi;
        p.token_out[0] = tok;
        if (p.tokens_hist != nullptr) {
          const int64_t st = *p.step;
          p.tokens_hist[st] = tok;
          *p.step = st + 1;
          *p.pos_inc = *p.pos_inc + 1;
        }
        *p.ticket = 0u;
      }
    }
  }
}

// ---- host-side launch ----
int64_t RowBytes(int32_t fmt, int64_t k) {
  switch (fmt) {
    case AM_WF_F32: return k * 4;
    case AM_WF_BF16: return k * 2;
    case AM_WF_INT8: return k;
    default: return k / 2;
  }
}

am_status_code ValidateWeight(const am_gfx950_weight& w) {
  AM_CHECK_ARG(w.data != nullptr && w.n > 0 && w.k > 0, "weight: null data or empty shape");
  AM_CHECK_ARG(w.format >= AM_WF_F32 && w.format <= AM_WF_INT4, "weight: unknown format");
  const int kc[4] = {4, 8, 16, 32};
  AM_CHECK_ARG(w.k % kc[w.format] == 0, "weight: in_features must fill whole 16-byte chunks");
  if (w.format == AM_WF_INT4) {
    AM_CHECK_ARG(w.group_size > 0 && w.group_size % 32 == 0 && w.k % w.group_size == 0,
                 "weight: INT4 group_size must be a multiple of 32 dividing in_features");
  }
  if (w.format >= AM_WF_INT8) AM_CHECK_ARG(w.scales != nullptr, "weight: quantized weight needs scales");
  AM_CHECK_ARG((reinterpret_cast<uintptr_t>(w.data) & 15u) == 0, "weight: data must be 16-byte aligned");
  return AM_STATUS_OK;
}

template <class A, int WF, bool NORM, int EPI, int JM, int P>
am_status_code LaunchJ(const GemvArgs& g, hipStream_t s) {
  using XS = XStore<A, WF>;
  const int64_t tb = A::kDtype == AM_DT_BF16 ? 2 : 4;
  int64_t lds = ((g.k * XS::kBytes + 15) / 16) * 16 + (((g.row_bytes / 16) * 4 + 15) / 16) * 16;
  if (EPI == kEpiResidual) lds += ((g.n * tb + 15) / 16) * 16;
  if (EPI == kEpiQkv) lds += g.d * 4;
  if (lds > 150 * 1024) return SetLastError(AM_STATUS_INVALID_ARGUMENT, "gemv: in_features too large for LDS staging");
  // Balanced grid of persistent waves: as many resident waves as the kernel's register
  // and LDS footprint allows (HBM latency is hidden by waves in flight), iterations
  // spread evenly over them.
  static thread_local int64_t cached_lds = -1;
  static thread_local int cached_blocks = 2;
  if (cached_lds != lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, gemv_kernel<A, WF, NORM, EPI, JM, P>, 256,
                                                     static_cast<size_t>(lds)) != hipSuccess || nb < 1)
      nb = 2;
    cached_blocks = nb;
    cached_lds = lds;
  }
  const int64_t niter = CeilDiv(g.units, P);
  const int64_t max_waves = static_cast<int64_t>(DeviceCUs()) * cached_blocks * 4;
  const int64_t ipw = CeilDiv(niter, max_waves);
  const int64_t waves = CeilDiv(niter, ipw);
  int64_t blocks = CeilDiv(waves, 4);
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL((gemv_kernel<A, WF, NORM, EPI, JM, P>), dim3(static_cast<unsigned>(blocks)), dim3(256),
                     static_cast<size_t>(lds), s, g);
  AM_RETURN_IF_LAUNCH_FAILED("gemv");
  return AM_STATUS_OK;
}

// Chunk-steps per row decide the register tiling: x stays in registers for up to
// 16 chunk-steps (bounded by 128 dwords of x per lane).
template <class A, int WF, bool NORM, int EPI>
am_status_code LaunchT(const GemvArgs& g, hipStream_t s) {
  using XS = XStore<A, WF>;
  const int64_t J = CeilDiv(g.row_bytes / 16, 64);
  if (J <= 2) return LaunchJ<A, WF, NORM, EPI, 2, 2>(g, s);
  if (J <= 4) return LaunchJ<A, WF, NORM, EPI, 4, 2>(g, s);
  if constexpr (8 * XS::kDW <= 128) {
    if (J <= 8) return LaunchJ<A, WF, NORM, EPI, 8, 1>(g, s);
  }
  if constexpr (16 * XS::kDW <= 128) {
    if (J <= 16) return LaunchJ<A, WF, NORM, EPI, 16, 1>(g, s);
  }
  if constexpr (32 * XS::kDW <= 128) {
    if (J <= 32) return LaunchJ<A, WF, NORM, EPI, 32, 1>(g, s);
  }
  return SetLastError(AM_STATUS_UNIMPLEMENTED, "gemv: in_features too large for register tiling of this format");
}

template <bool NORM, int EPI>
am_status_code Dispatch(int32_t act, int32_t fmt, const GemvArgs& g, hipStream_t s) {
  if (act == AM_DT_F32) {
    switch (fmt) {
      case AM_WF_F32: return LaunchT<ActF32, AM_WF_F32, NORM, EPI>(g, s);
      case AM_WF_BF16: return LaunchT<ActF32, AM_WF_BF16, NORM, EPI>(g, s);
      case AM_WF_INT8: return LaunchT<ActF32, AM_WF_INT8, NORM, EPI>(g, s);
      default: return LaunchT<ActF32, AM_WF_INT4, NORM, EPI>(g, s);
    }
  }
  switch (fmt) {
    case AM_WF_F32: return LaunchT<ActBF16, AM_WF_F32, NORM, EPI>(g, s);
    case AM_WF_BF16: return LaunchT<ActBF16, AM_WF_BF16, NORM, EPI>(g, s);
    case AM_WF_INT8: return LaunchT<ActBF16, AM_WF_INT8, NORM, EPI>(g, s);
    default: return LaunchT<ActBF16, AM_WF_INT4, NORM, EPI>(g, s);
  }
}

GemvArgs BaseArgs(const am_gfx950_weight& w) {
  GemvArgs g{};
  g.w = static_cast<const uint8_t*>(w.data);
  g.scales = w.scales;
  g.n = w.n;
  g.k = w.k;
  g.group = w.group_size;
  g.row_bytes = RowBytes(w.format, w.k);
  g.units = CeilDiv(w.n, 2);
  return g;
}

}  // namespace

// Linear rows for am_gfx950_linear (decode GEMV; also the row loop of small m).
am_status_code GemvLinearRow(const void* x, int32_t act, const am_gfx950_weight& w, void* out, int32_t out_dtype,
                             const void* residual, hipStream_t s) {
  if (auto st = ValidateWeight(w); st != AM_STATUS_OK) return st;
  GemvArgs g = BaseArgs(w);
  g.x = x;
  g.out = out;
  g.residual = residual;
  g.out_f32 = (out_dtype == AM_DT_F32 && act != AM_DT_F32) ? 1 : 0;
  if (residual != nullptr && g.out_f32)
    return SetLastError(AM_STATUS_INVALID_ARGUMENT, "linear: residual needs out dtype == activation dtype");
  if (residual != nullptr) return Dispatch<false, kEpiResidual>(act, w.format, g, s);
  return Dispatch<false, kEpiStore>(act, w.format, g, s);
}

}  // namespace am

using namespace am;

extern "C" am_status_code am_gfx950_fused_qkv(const am_gfx950_fused_qkv_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "fused_qkv: null args");
  if (auto st = ValidateWeight(a->w_qkv); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_qkv: dtype");
  AM_CHECK_ARG(a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0 && a->head_dim > 0 && a->head_dim % 2 == 0,
               "fused_qkv: bad head configuration");
  AM_CHECK_ARG(a->w_qkv.n == (a->hq + 2 * a->hkv) * a->head_dim, "fused_qkv: weight rows != (hq+2hkv)*d");
  AM_CHECK_ARG(a->h && a->norm_w && a->cos_tab && a->sin_tab && a->pos && a->q_out && a->k_cache && a->v_cache,
               "fused_qkv: null pointer");
  AM_CHECK_ARG(a->eps > 0.0f, "fused_qkv: eps must be positive");
  GemvArgs g = BaseArgs(a->w_qkv);
  g.units = a->w_qkv.n / 2;
  g.x = a->h;
  g.norm_w = a->norm_w;
  g.eps = a->eps;
  g.cos_tab = a->cos_tab;
  g.sin_tab = a->sin_tab;
  g.pos = a->pos;
  g.q_out = a->q_out;
  g.k_cache = a->k_cache;
  g.v_cache = a->v_cache;
  g.hq = static_cast<int32_t>(a->hq);
  g.hkv = static_cast<int32_t>(a->hkv);
  g.d = static_cast<int32_t>(a->head_dim);
  g.cap = a->capacity;
  return Dispatch<true, kEpiQkv>(a->dtype, a->w_qkv.format, g, AsStream(stream));
}

extern "C" am_status_code am_gfx950_fused_linear_residual(const am_gfx950_fused_linear_residual_args* a,
                                                          void* stream) {
  AM_CHECK_ARG(a != nullptr, "fused_linear_residual: null args");
  if (auto st = ValidateWeight(a->w); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_linear_residual: dtype");
  AM_CHECK_ARG(a->x && a->h, "fused_linear_residual: null pointer");
  GemvArgs g = BaseArgs(a->w);
  g.x = a->x;
  g.out = a->h;
  g.residual = a->h;
  return Dispatch<false, kEpiResidual>(a->dtype, a->w.format, g, AsStream(stream));
}

extern "C" am_status_code am_gfx950_fused_gate_up(const am_gfx950_fused_gate_up_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "fused_gate_up: null args");
  if (auto st = ValidateWeight(a->w_gate_up); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_gate_up: dtype");
  AM_CHECK_ARG(a->w_gate_up.n % 2 == 0, "fused_gate_up: gate/up weight needs an even row count");
  AM_CHECK_ARG(a->h && a->norm_w && a->act_out && a->eps > 0.0f, "fused_gate_up: bad pointer/eps");
  GemvArgs g = BaseArgs(a->w_gate_up);
  g.x = a->h;
  g.norm_w = a->norm_w;
  g.eps = a->eps;
  g.out = a->act_out;
  return Dispatch<true, kEpiGateUp>(a->dtype, a->w_gate_up.format, g, AsStream(stream));
}

extern "C" int64_t am_gfx950_lm_head_workspace_bytes(void) {
  // ticket (256 B) + up to 65536 block partials (value + index)
  return 256 + 65536LL * (4 + 8);
}

extern "C" am_status_code am_gfx950_fused_lm_head(const am_gfx950_fused_lm_head_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "fused_lm_head: null args");
  if (auto st = ValidateWeight(a->w); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_lm_head: dtype");
  AM_CHECK_ARG(a->h && a->norm_w && a->token_out && a->workspace && a->eps > 0.0f, "fused_lm_head: bad args");
  AM_CHECK_ARG(a->workspace_bytes >= am_gfx950_lm_head_workspace_bytes(), "fused_lm_head: workspace too small");
  AM_CHECK_ARG(a->tokens_hist == nullptr || (a->pos != nullptr && a->step != nullptr),
               "fused_lm_head: tokens_hist needs pos and step");
  GemvArgs g = BaseArgs(a->w);
  g.x = a->h;
  g.norm_w = a->norm_w;
  g.eps = a->eps;
  g.out = a->logits;
  g.token_out = a->token_out;
  g.tokens_hist = a->tokens_hist;
  g.pos_inc = a->pos;
  g.step = a->step;
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  g.ticket = reinterpret_cast<unsigned*>(ws);
  g.pi = reinterpret_cast<int64_t*>(ws + 256);
  g.pv = reinterpret_cast<float*>(ws + 256 + 65536LL * 8);
  return Dispatch<true, kEpiLmHead>(a->dtype, a->w.format, g, AsStream(stream));
}
