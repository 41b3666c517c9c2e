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

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <cmath>

#include "am_gemv_common.h"
#include "am_launch_timing.h"
#include <hip/hip_ext.h>

namespace am {
namespace {

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
  int32_t vec;  // x, norm_w, residual 16-byte aligned and whole 16-byte pieces
  KvRows kv;    // K/V row addressing of the q/k/v epilogue
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

// init + dot of one 16-byte weight chunk with its x values (kDW dwords at xd).
template <class A, int WF>
__device__ __forceinline__ float chunk_dot(const uint4 w, const uint32_t* xd, float init, const Unpack& up) {
  using XS = XStore<A, WF>;
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float acc = init;
  if constexpr (XS::kBF16) {
    if constexpr (WF == AM_WF_INT4) {
      acc = int4_chunk_dot_bf16(w, xd, init, up);
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

// rows of pair u
template <int EPI>
__device__ __forceinline__ void pair_rows(const GemvArgs& p, int64_t u, int64_t& r0, int64_t& r1) {
  if constexpr (EPI == kEpiQkv) {
    // 32-bit division: units and head_dim are far below 2^31 (checked on the host)
    const uint32_t half = static_cast<uint32_t>(p.d / 2);
    const uint32_t uu = static_cast<uint32_t>(u);
    const uint32_t head = uu / half, i = uu - head * half;
    r0 = static_cast<int64_t>(head) * p.d + i;
    r1 = r0 + half;
  } else if constexpr (EPI == kEpiGateUp) {
    r0 = u;  // gate row u, up row u: rows [0, F) are gate, [F, 2F) are up
    r1 = u + p.n / 2;
  } else {
    r0 = 2 * u;
    r1 = 2 * u + 1;
  }
}

// One load block: JB chunk-steps of both rows of P pairs (+ INT4 group scales).
template <int JB, int P, bool SC>
struct Frag {
  uint4 w[P][2][JB];
  uint32_t s[P][2][SC ? JB : 1];  // raw fp16 group-scale bits, converted at use
  float s8[P][2];                 // INT8 row scales
};

// Streaming 16-byte weight load (read once per token: non-temporal hint).
__device__ __forceinline__ uint4 ld_stream(const uint8_t* row, int64_t c) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row) + c);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Activation vector in LDS: chunk c (the kc values that meet 16-byte weight chunk c)
// occupies kc*kBytes contiguous bytes as NPC 16-byte pieces; piece i is stored in
// slot (i + (c >> 1)) % NPC so that lanes reading consecutive chunks start in
// different LDS banks.
template <class A, int WF>
struct XLds {
  using XS = XStore<A, WF>;
  static constexpr int kc = Fmt<WF>::kc;
  static constexpr int NPC = XS::kDW / 4;          // 16-byte pieces per chunk (1..8)
  static constexpr int CB = kc * XS::kBytes;       // bytes per chunk
  __device__ static __forceinline__ int64_t addr(int64_t j) {  // byte address of value j
    const int64_t c = j / kc;
    const int b = static_cast<int>(j % kc) * XS::kBytes;
    const int slot = ((b >> 4) + static_cast<int>(c >> 1)) % NPC;
    return c * CB + slot * 16 + (b & 15);
  }
  __device__ static __forceinline__ void store(uint8_t* xl, int64_t j, float v) {
    if constexpr (XS::kBF16)
      *reinterpret_cast<uint16_t*>(xl + addr(j)) = f32_to_bf16_bits(v);
    else
      *reinterpret_cast<float*>(xl + addr(j)) = v;
  }
  // the XS::kDW dwords of chunk c, in value order
  __device__ static __forceinline__ void load_chunk(const uint8_t* xl, int64_t c, uint32_t* xd) {
#pragma unroll
    for (int i = 0; i < NPC; ++i) {
      const int slot = (i + static_cast<int>(c >> 1)) % NPC;
      const uint4 v = *reinterpret_cast<const uint4*>(xl + c * CB + slot * 16);
      xd[4 * i] = v.x;
      xd[4 * i + 1] = v.y;
      xd[4 * i + 2] = v.z;
      xd[4 * i + 3] = v.w;
    }
  }
  // sum of the kc values of a chunk held in xd
  __device__ static __forceinline__ float chunk_sum(const uint32_t* xd) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < XS::kDW; ++i) {
      if constexpr (XS::kBF16) {
        s += __uint_as_float(xd[i] << 16);
        s += __uint_as_float(xd[i] & 0xFFFF0000u);
      } else {
        s += __uint_as_float(xd[i]);
      }
    }
    return s;
  }
};

// element e of a 16-byte piece of activations of type T, as float
template <class A>
__device__ __forceinline__ float piece_elem(const uint4& v, int e) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (A::kDtype == AM_DT_BF16)
    return __uint_as_float((e & 1) ? (w[e >> 1] & 0xFFFF0000u) : (w[e >> 1] << 16));
  else
    return __uint_as_float(w[e]);
}

// ONE: every wave has at most one load block (the launch covers all iterations with
// one per wave and x stays in registers), so there is no second buffer to prefetch.
template <class A, int WF, bool NORM, int EPI, int JM, int P, int NW, bool ONE = false>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(GemvArgs p) {
  constexpr int NT = NW * 64;  // threads per block
  using XS = XStore<A, WF>;
  using XL_ = XLds<A, WF>;
  using T = typename A::T;
  constexpr int kc = Fmt<WF>::kc;
  constexpr int XDW = XS::kDW;
  constexpr bool SC = WF == AM_WF_INT4;
  // x chunks live in registers when they fit in 32 dwords per lane, else they are
  // read from LDS per chunk-step inside the loop
  constexpr bool XL = JM * XDW > 32;
  // chunk-steps per load block with x in LDS: 2 (measured best for the 14336-long rows:
  // small blocks keep ~85 registers and a finer double-buffered pipeline)
  constexpr int JBX = 2;
  constexpr int JB = XL ? (JM < JBX ? JM : JBX) : JM;
  constexpr int NB = JM / JB;                      // load blocks per iteration
  constexpr int EPP = 16 / static_cast<int>(sizeof(T));               // activations per 16-byte piece
  constexpr int XP = (JM * 64 * kc + NT * EPP - 1) / (NT * EPP);  // x pieces per thread
  constexpr int RP = 1024 / NT > 0 ? 1024 / NT : 1;                // residual pieces per thread (first pass)
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[NW];
  const int tid = threadIdx.x;
  const int64_t K = p.k;
  const int64_t C = p.row_bytes / 16;  // chunks per row
  const int J = static_cast<int>((C + 63) / 64);
  // LDS: x | per-chunk offset corrections (INT formats) | residual | cos,sin
  uint8_t* xl = smem;
  const int64_t off_corr = ((K * XS::kBytes + 15) / 16) * 16;
  const int64_t off_res = off_corr + (XS::kOff != 0.0f ? ((C * 4 + 15) / 16) * 16 : 0);
  const int64_t off_cs = off_res + (EPI == kEpiResidual ? ((p.n * static_cast<int64_t>(sizeof(T)) + 15) / 16) * 16 : 0);
  float* corr_lds = reinterpret_cast<float*>(smem + off_corr);
  T* res_lds = reinterpret_cast<T*>(smem + off_res);
  float* cs_lds = reinterpret_cast<float*>(smem + off_cs);
  const int lane = tid & 63;
  // wave index made provably wave-uniform, so the loop below runs on scalar branches
  const int64_t gw = static_cast<int64_t>(blockIdx.x) * NW + __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t TW = static_cast<int64_t>(gridDim.x) * NW;
  const int64_t niter = (p.units + P - 1) / P;
  // 32-bit divisions (the host keeps K, units and the grid below 2^31): the 64-bit
  // forms cost a long scalar sequence ahead of the first loads
  const int ng = SC ? static_cast<int>(static_cast<uint32_t>(K) / static_cast<uint32_t>(p.group)) : 1;
  const int chunks_per_group = SC ? p.group / kc : 1;
  const uint16_t* sc16 = static_cast<const uint16_t*>(p.scales);
  // this wave's iterations are gw, gw + TW, ...; each is NB load blocks
  const int64_t nit_w =
      gw < niter ? static_cast<int64_t>(static_cast<uint32_t>(niter - 1 - gw) / static_cast<uint32_t>(TW)) + 1 : 0;
  const int64_t nblk = nit_w * NB;

  // ---- 1. prologue operands: all loads issued at once, before any weight load ----
  const T* xin = static_cast<const T*>(p.x);
  const T* nw = static_cast<const T*>(p.norm_w);
  const int64_t xpieces = K / EPP;
  uint4 xv[XP];
  uint4 nv[NORM ? XP : 1];
  u32x4_t rv[RP];  // a vector type: the copy into LDS stays in registers
  const int64_t rpieces = p.n / EPP;
  {
    // Straight-line loads on every path (the arrays stay in registers); without the
    // vector layout they read the (aligned) weight base instead and go unused.
    const uint4* xs = reinterpret_cast<const uint4*>(p.vec ? static_cast<const void*>(xin) : p.w);
    const uint4* ns = reinterpret_cast<const uint4*>(p.vec && NORM ? static_cast<const void*>(nw) : p.w);
    const int64_t xlast = p.vec ? xpieces - 1 : 0;
#pragma unroll
    for (int v = 0; v < XP; ++v) {
      int64_t pi = tid + NT * v;
      if (pi > xlast) pi = xlast;
      xv[v] = xs[pi];
      if constexpr (NORM) nv[v] = ns[pi];
    }
    if constexpr (EPI == kEpiResidual) {
      const u32x4_t* rs = reinterpret_cast<const u32x4_t*>(p.vec ? p.residual : static_cast<const void*>(p.w));
      const int64_t rlast = p.vec ? rpieces - 1 : 0;
#pragma unroll
      for (int v = 0; v < RP; ++v) {
        int64_t pi = tid + NT * v;
        if (pi > rlast) pi = rlast;
        rv[v] = rs[pi];
      }
    }
  }
  int64_t posv = 0;
  float cs_c = 0.0f, cs_s = 0.0f;
  if constexpr (EPI == kEpiQkv) {
    posv = *p.pos;
    const int64_t half = p.d / 2;
    const int64_t pr = posv < p.cap ? posv : 0;
    const int64_t i = tid < half ? tid : 0;
    cs_c = p.cos_tab[pr * half + i];
    cs_s = p.sin_tab[pr * half + i];
  }

  // ---- 2. first weight block ----
  // Loads chunk-steps [jb*JB, jb*JB + JB) of this wave's block b into f.  Every load
  // is unconditional (straight-line code, one wait at first use): out-of-range chunks
  // and rows read a clamped in-bounds address instead and contribute nothing, because
  // the lane's x values for those chunks are zero and invalid rows are never stored.
  // A block past the wave's last one re-reads that last block (a wave without work
  // reads the grid's last iteration).
  auto issue = [&](Frag<JB, P, SC>& f, int64_t b) {
    int64_t it;
    int jb = 0;
    if (nblk == 0) {
      it = niter - 1;
    } else {
      if (b >= nblk) b = nblk - 1;
      it = gw + (NB == 1 ? b : b / NB) * TW;
      if constexpr (NB > 1) jb = static_cast<int>(b % NB);
    }
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
          const int g = static_cast<int>(c) / chunks_per_group;
          f.s[pp][0][jj] = sc16[r0 * ng + g];
          f.s[pp][1][jj] = sc16[r1 * ng + g];
        }
      }
      if constexpr (WF == AM_WF_INT8) {
        f.s8[pp][0] = static_cast<const float*>(p.scales)[r0];
        f.s8[pp][1] = static_cast<const float*>(p.scales)[r1];
      }
    }
  };
  Frag<JB, P, SC> fa, fb;
  issue(fa, 0);

  // ---- 3. prologue: x (optionally RMSNorm'd) -> LDS, epilogue operands -> LDS ----
  // The vector pass runs on every path with clamped indices, so the register arrays
  // are consumed in straight-line code (nothing moves the loads behind the weights);
  // without the vector layout it only writes placeholders that the element pass
  // below overwrites.  Each 16-byte input piece is staged with one or two 16-byte LDS
  // stores; the per-chunk offset corrections are summed over the aligned lane group
  // that holds the chunk's pieces (consecutive threads hold consecutive pieces).
  {
    const bool vec = p.vec != 0;
    float inv = 1.0f;
    if constexpr (NORM) {
      float ss = 0.0f;
#pragma unroll
      for (int v = 0; v < XP; ++v) {
        const bool ok = vec && tid + NT * v < xpieces;
#pragma unroll
        for (int e = 0; e < EPP; ++e) {
          const float x = ok ? piece_elem<A>(xv[v], e) : 0.0f;
          ss = fmaf(x, x, ss);
        }
      }
      ss = block_sum<NW>(ss, red);
      inv = 1.0f / sqrtf(ss / static_cast<float>(K) + p.eps);
    }
    const int64_t xlast = vec ? xpieces - 1 : 0;
#pragma unroll
    for (int v = 0; v < XP; ++v) {
      const int64_t pi0 = tid + NT * v;
      const bool ok = vec && pi0 < xpieces;
      const int64_t pi = pi0 > xlast ? xlast : pi0;
      float xs[EPP];  // staged values (bf16-exact when LDS holds bf16)
      if constexpr (XS::kBF16) {
        uint32_t packed[4];
        if constexpr (NORM) {
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float x0 = (piece_elem<A>(xv[v], 2 * t) * inv) * piece_elem<A>(nv[v], 2 * t);
            const float x1 = (piece_elem<A>(xv[v], 2 * t + 1) * inv) * piece_elem<A>(nv[v], 2 * t + 1);
            const bf16x2_t h = {static_cast<__bf16>(x0), static_cast<__bf16>(x1)};  // RNE
            packed[t] = __builtin_bit_cast(uint32_t, h);
          }
        } else {
          packed[0] = xv[v].x; packed[1] = xv[v].y; packed[2] = xv[v].z; packed[3] = xv[v].w;
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          xs[2 * t] = __uint_as_float(packed[t] << 16);
          xs[2 * t + 1] = __uint_as_float(packed[t] & 0xFFFF0000u);
        }
        *reinterpret_cast<uint4*>(xl + XL_::addr(pi * EPP)) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      } else {
#pragma unroll
        for (int e = 0; e < EPP; ++e) {
          float x = piece_elem<A>(xv[v], e);
          if constexpr (NORM) x = A::round((x * inv) * piece_elem<A>(nv[v], e));
          xs[e] = x;
        }
#pragma unroll
        for (int h = 0; h < EPP / 4; ++h)
          *reinterpret_cast<float4*>(xl + XL_::addr(pi * EPP + 4 * h)) =
              make_float4(xs[4 * h], xs[4 * h + 1], xs[4 * h + 2], xs[4 * h + 3]);
      }
      if constexpr (XS::kOff != 0.0f) {
        constexpr int PPC = kc / EPP;  // input pieces per weight chunk: 2, 4 or 8
        float ps = 0.0f;
#pragma unroll
        for (int e = 0; e < EPP; ++e) ps += xs[e];
        if (!ok) ps = 0.0f;
        ps = dpp_add<0xB1>(ps);
        if constexpr (PPC >= 4) ps = dpp_add<0x4E>(ps);
        if constexpr (PPC >= 8) ps = dpp_add<0x141>(ps);
        if (ok && (tid % PPC) == 0) corr_lds[pi / PPC] = XS::kOff * ps;
      }
    }
    if constexpr (EPI == kEpiResidual) {
      const int64_t rlast = vec ? rpieces - 1 : 0;
#pragma unroll
      for (int v = 0; v < RP; ++v) {
        int64_t pi = tid + NT * v;
        if (pi > rlast) pi = rlast;
        reinterpret_cast<u32x4_t*>(res_lds)[pi] = rv[v];
      }
      if (vec) {
        const uint4* res = static_cast<const uint4*>(p.residual);
        for (int64_t pi = tid + NT * RP; pi < rpieces; pi += NT) reinterpret_cast<uint4*>(res_lds)[pi] = res[pi];
      }
    }
  }
  if (!p.vec) {
    // unaligned or ragged activations: element loops overwrite the placeholders
    __syncthreads();
    float inv = 1.0f;
    if constexpr (NORM) {
      float ss = 0.0f;
      for (int64_t j = tid; j < K; j += NT) {
        const float v = A::load(xin, j);
        ss = fmaf(v, v, ss);
      }
      ss = block_sum<NW>(ss, red);
      inv = 1.0f / sqrtf(ss / static_cast<float>(K) + p.eps);
    }
    for (int64_t j = tid; j < K; j += NT) {
      float v = A::load(xin, j);
      if constexpr (NORM) v = A::round((v * inv) * A::load(nw, j));
      XL_::store(xl, j, v);
    }
    if constexpr (EPI == kEpiResidual) {
      const T* res = static_cast<const T*>(p.residual);
      for (int64_t r = tid; r < p.n; r += NT) res_lds[r] = res[r];
    }
    if constexpr (XS::kOff != 0.0f) {
      __syncthreads();
      for (int64_t c = tid; c < C; c += NT) {
        uint32_t xd[XDW];
        XL_::load_chunk(xl, c, xd);
        corr_lds[c] = XS::kOff * XL_::chunk_sum(xd);
      }
    }
  }
  if constexpr (EPI == kEpiQkv) {
    const int64_t half = p.d / 2;
    if (tid < half) {
      cs_lds[tid] = cs_c;
      cs_lds[half + tid] = cs_s;
    }
  }
  __syncthreads();

  // ---- 4. second weight block, then this lane's x chunks ----
  if constexpr (!ONE) issue(fb, 1);
  uint32_t xr[XL ? 1 : JM][XDW];
  float corr[XL ? 1 : JM];
  if constexpr (!XL) {
#pragma unroll
    for (int j = 0; j < JM; ++j) {
      const int64_t c = lane + 64 * j;
      if (j < J && c < C) {
        XL_::load_chunk(xl, c, xr[j]);
        corr[j] = XS::kOff != 0.0f ? corr_lds[c] : 0.0f;
      } else {
#pragma unroll
        for (int t = 0; t < XDW; ++t) xr[j][t] = 0u;
        corr[j] = 0.0f;
      }
    }
  }

  float best_v = 0.0f;
  int64_t best_i = -1;

  const Unpack up;
  // Accumulates load block jb of f into acc.
  auto accum = [&](const Frag<JB, P, SC>& f, int jb, float (&acc)[P][2]) {
#pragma unroll
    for (int jj = 0; jj < JB; ++jj) {
      const int j = jb * JB + jj;
      uint32_t xc[XL ? XDW : 1];
      const uint32_t* xd;
      float cj;
      if constexpr (XL) {
        const int64_t c = lane + 64 * j;
        const bool ok = j < J && c < C;
        XL_::load_chunk(xl, ok ? c : 0, xc);
        if (!ok) {
#pragma unroll
          for (int t = 0; t < XDW; ++t) xc[t] = 0u;
        }
        xd = xc;
        cj = (XS::kOff != 0.0f && ok) ? corr_lds[c] : 0.0f;
      } else {
        xd = xr[jj];
        cj = corr[jj];
      }
#pragma unroll
      for (int pp = 0; pp < P; ++pp) {
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          // the offset correction seeds the accumulator: dv = dot - kOff * sum(x)
          const float dv = chunk_dot<A, WF>(f.w[pp][rr][jj], xd, XS::kOff != 0.0f ? -cj : 0.0f, up);
          if constexpr (SC)
            acc[pp][rr] = fmaf(f16_bits_to_f32(f.s[pp][rr][jj]), dv, acc[pp][rr]);
          else
            acc[pp][rr] += dv;
        }
      }
    }
    if constexpr (WF == AM_WF_INT8) {
      if (jb == NB - 1) {  // per-row scale after the last block of the row
#pragma unroll
        for (int pp = 0; pp < P; ++pp) {
          acc[pp][0] *= f.s8[pp][0];
          acc[pp][1] *= f.s8[pp][1];
        }
      }
    }
  };

  // Reduces acc across the wave, applies the epilogue of iteration itc in the lane
  // that owns each pair, zeroes acc.
  auto finish = [&](float (&acc)[P][2], int64_t itc) {
    float a0, a1;
    const int pp = reduce_pairs<P>(acc, lane, a0, a1);
#pragma unroll
    for (int q = 0; q < P; ++q) acc[q][0] = acc[q][1] = 0.0f;
    if (pp < 0) return;
    const int64_t u = itc * P + pp;
    if (u >= p.units) return;
    int64_t r0, r1;
    pair_rows<EPI>(p, u, r0, r1);
    const bool v1 = r1 < p.n;
    T* out = static_cast<T*>(p.out);
    if constexpr (EPI == kEpiLmHead) {
      float* lg = static_cast<float*>(p.out);
      if (lg != nullptr) {
        lg[r0] = a0;
        if (v1) lg[r1] = a1;
      }
      if (argmax_better(a0, r0, best_v, best_i)) { best_v = a0; best_i = r0; }
      if (v1 && argmax_better(a1, r1, best_v, best_i)) { best_v = a1; best_i = r1; }
    } else if constexpr (EPI == kEpiStore) {
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
        float o0, o1;
        rope_rotate(y0, y1, c, s, o0, o1);
        if (head < p.hq) {
          T* q = static_cast<T*>(p.q_out);
          A::store(q, head * p.d + i, o0);
          A::store(q, head * p.d + i + half, o1);
        } else if (posv < p.cap) {
          T* kc = static_cast<T*>(p.k_cache);
          const int64_t base = p.kv.WriteRow(0, head - p.hq, posv);
          if (base >= 0) {
            A::store(kc, base + i, o0);
            A::store(kc, base + i + half, o1);
          }
        }
      } else if (posv < p.cap) {
        T* vc = static_cast<T*>(p.v_cache);
        const int64_t base = p.kv.WriteRow(0, head - p.hq - p.hkv, posv);
        if (base >= 0) {
          A::store(vc, base + i, y0);
          A::store(vc, base + i + half, y1);
        }
      }
    }
  };
  auto blk_jb = [&](int64_t b) { return NB == 1 ? 0 : static_cast<int>(b % NB); };
  auto blk_it = [&](int64_t b) { return gw + (NB == 1 ? b : b / NB) * TW; };

  // ---- 5. main loop: blocks alternate between fa and fb; the block after next is
  // issued as soon as a buffer has been consumed, so one block is always in flight
  // while the other is reduced.  The exits sit before the issues, so on the path
  // that stays in the loop both buffers are always pending in the same order. ----
  float acc[P][2] = {};
  int64_t b = 0;
  if constexpr (ONE) {
    static_assert(NB == 1, "single-block launches keep x in registers");
    if (nblk > 0) {
      accum(fa, 0, acc);
      finish(acc, blk_it(0));
    }
  }
  while (!ONE && b < nblk) {
    accum(fa, blk_jb(b), acc);
    if (blk_jb(b) == NB - 1) finish(acc, blk_it(b));
    if (b + 2 >= nblk) {
      if (b + 1 < nblk) {
        accum(fb, blk_jb(b + 1), acc);
        if (blk_jb(b + 1) == NB - 1) finish(acc, blk_it(b + 1));
      }
      break;
    }
    issue(fa, b + 2);
    accum(fb, blk_jb(b + 1), acc);
    if (blk_jb(b + 1) == NB - 1) finish(acc, blk_it(b + 1));
    if (b + 3 >= nblk) {
      accum(fa, blk_jb(b + 2), acc);
      if (blk_jb(b + 2) == NB - 1) finish(acc, blk_it(b + 2));
      break;
    }
    issue(fb, b + 3);
    b += 2;
  }

  if constexpr (EPI == kEpiLmHead) {
    // block best -> partials; the last block (atomic ticket) reduces them, publishes
    // the token / advances the decode state, and resets the ticket for the next call.
    __shared__ float bv_s[NW];
    __shared__ int64_t bi_s[NW];
    __shared__ bool last;
    const int wave = threadIdx.x >> 6;
    // each pair lane holds the best of its rows: reduce over the wave first
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(best_v, o, 64);
      const int64_t oi = __shfl_xor(best_i, o, 64);
      if (oi >= 0 && argmax_better(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
    }
    if (lane == 0) {
      bv_s[wave] = best_v;
      bi_s[wave] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = 0.0f;
      int64_t bi = -1;
      for (int w = 0; w < NW; ++w)
        if (bi_s[w] >= 0 && argmax_better(bv_s[w], bi_s[w], bv, bi)) { bv = bv_s[w]; bi = bi_s[w]; }
      // device-coherent (sc1) stores, acknowledged before the relaxed ticket: the
      // last block's device-coherent loads then see every block's partial
      __hip_atomic_store(&p.pv[blockIdx.x], bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&p.pi[blockIdx.x], bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      const unsigned t = __hip_atomic_fetch_add(p.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = (t == gridDim.x - 1);
    }
    __syncthreads();
    if (last) {
      float bv = 0.0f;
      int64_t bi = -1;
      for (int64_t b = threadIdx.x; b < gridDim.x; b += NT) {
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
        for (int w = 0; w < NW; ++w)
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
  AM_CHECK_ARG(w.n < (int64_t{1} << 31) && w.k < (int64_t{1} << 31), "weight: dimensions must be below 2^31");
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

// ---- split-K GEMV for long rows ----
// When a lane's share of x no longer fits in registers (rows longer than 64 lanes x 2
// chunks), a block owns kSkRows consecutive rows and its NW*64 lanes split every row
// instead: lane slot t reads 16-byte chunk t of all kSkRows rows (each load
// instruction still moves 1 KiB of one row), holds the kc x values of chunk t in
// registers, and the block issues all of its rows' weight loads at once.  The row
// sums are folded over the lanes (permlane swaps, then DPP) and over the waves in LDS.
// 8 rows per block (512 blocks for the 8B down projection, two per CU): 0.36 us per
// launch faster than 16 (one block per CU), the same as 4, measured in the decode graph.
constexpr int kSkRows = 8;
constexpr int kSkWaves = 8;

template <class A, int WF, int EPI>
__global__ __launch_bounds__(kSkWaves * 64) void gemv_ksplit_kernel(GemvArgs p) {
  static_assert(EPI == kEpiStore || EPI == kEpiResidual, "split-K rows: plain or residual epilogue");
  using XS = XStore<A, WF>;
  using T = typename A::T;
  constexpr int kc = Fmt<WF>::kc;
  constexpr int XDW = XS::kDW;
  constexpr bool SC = WF == AM_WF_INT4;
  __shared__ float red[kSkWaves][kSkRows];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t C = p.row_bytes / 16;  // <= kSkWaves * 64 (host)
  const int64_t r_base = static_cast<int64_t>(blockIdx.x) * kSkRows;
  const bool active = tid < C;
  const int64_t c = active ? tid : 0;

  // Every load is unconditional and issued before any use: the epilogue operand (each
  // thread reads row tid % kSkRows, in bounds), x, then the block's weight chunks and
  // scales, each as a uniform row base plus a 32-bit lane offset.
  const uint32_t cu = static_cast<uint32_t>(c);
  float res = 0.0f;
  if constexpr (EPI == kEpiResidual) {
    const int64_t rr = r_base + (tid & (kSkRows - 1));
    res = A::load(static_cast<const T*>(p.residual), rr < p.n ? rr : p.n - 1);
  }
  uint32_t xd[XDW];
  {
    const uint4* xs = reinterpret_cast<const uint4*>(p.x) + cu * (XDW / 4);
#pragma unroll
    for (int i = 0; i < XDW / 4; ++i) {
      const uint4 v = xs[i];
      xd[4 * i] = v.x; xd[4 * i + 1] = v.y; xd[4 * i + 2] = v.z; xd[4 * i + 3] = v.w;
    }
  }
  uint4 w[kSkRows];
  uint32_t sb[SC ? kSkRows : 1];
  const int ng = SC ? static_cast<int>(static_cast<uint32_t>(p.k) / static_cast<uint32_t>(p.group)) : 1;
  const uint32_t g = SC ? cu / static_cast<uint32_t>(p.group / kc) : 0u;
  const uint16_t* sc16 = static_cast<const uint16_t*>(p.scales);
#pragma unroll
  for (int r = 0; r < kSkRows; ++r) {
    const int64_t row = r_base + r < p.n ? r_base + r : p.n - 1;
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p.w + row * p.row_bytes) + cu);
    w[r] = make_uint4(v.x, v.y, v.z, v.w);
  }
  if constexpr (SC) {
#pragma unroll
    for (int r = 0; r < kSkRows; ++r) {
      const int64_t row = r_base + r < p.n ? r_base + r : p.n - 1;
      sb[r] = (sc16 + row * ng)[g];
    }
  }

  // offset correction of this lane's chunk: kOff * sum(x)
  float corr = 0.0f;
  if constexpr (XS::kOff != 0.0f) {
    float sx = 0.0f;
    if constexpr (XS::kBF16) {
#pragma unroll
      for (int t = 0; t < XDW; ++t) sx += __uint_as_float(xd[t] << 16) + __uint_as_float(xd[t] & 0xFFFF0000u);
    } else {
#pragma unroll
      for (int t = 0; t < XDW; ++t) sx += __uint_as_float(xd[t]);
    }
    corr = XS::kOff * sx;
  }
  const Unpack up;
  float acc[kSkRows];
#pragma unroll
  for (int r = 0; r < kSkRows; ++r) {
    const float dv = chunk_dot<A, WF>(w[r], xd, -corr, up);
    acc[r] = SC ? f16_bits_to_f32(sb[r]) * dv : dv;
    if (!active) acc[r] = 0.0f;
  }

  // lanes: row 4 (lane / 16) + k of the block in every lane of that 16-lane row
  constexpr int RH = kSkRows / 2, RQ = kSkRows / 4;
  float xh[RH];
#pragma unroll
  for (int k = 0; k < RH; ++k) xh[k] = swap32_add(acc[k], acc[k + RH]);
  float z[RQ];
#pragma unroll
  for (int k = 0; k < RQ; ++k) z[k] = sum16(swap16_add(xh[k], xh[k + RQ]));
  if ((lane & 15) == 0) {
#pragma unroll
    for (int k = 0; k < RQ; ++k) red[wave][RQ * (lane >> 4) + k] = z[k];
  }
  __syncthreads();
  if (tid < kSkRows) {  // res holds row r_base + tid here
    const int64_t row = r_base + tid;
    if (row < p.n) {
      float a = 0.0f;
#pragma unroll
      for (int wv = 0; wv < kSkWaves; ++wv) a += red[wv][tid];
      if constexpr (WF == AM_WF_INT8) a *= static_cast<const float*>(p.scales)[row];
      if constexpr (EPI == kEpiResidual) {
        A::store(static_cast<T*>(p.out), row, res + A::round(a));
      } else if (p.out_f32) {
        static_cast<float*>(p.out)[row] = a;
      } else {
        A::store(static_cast<T*>(p.out), row, a);
      }
    }
  }
}

const char* EpiName(int epi) {
  switch (epi) {
    case kEpiStore: return "store";
    case kEpiResidual: return "residual";
    case kEpiQkv: return "qkv";
    case kEpiGateUp: return "gate_up";
    default: return "lm_head";
  }
}

const char* WfName(int wf) {
  switch (wf) {
    case AM_WF_F32: return "f32";
    case AM_WF_BF16: return "bf16";
    case AM_WF_INT8: return "int8";
    default: return "int4";
  }
}

template <class A, int WF, int EPI>
am_status_code LaunchKsplit(const GemvArgs& g, hipStream_t s) {
  const int64_t blocks = CeilDiv(g.n, kSkRows);
  RecordLaunch(blocks, kSkWaves * 64, 0, "gemv_ksplit<%s,%s,%s>", A::kDtype == AM_DT_BF16 ? "bf16" : "f32",
               WfName(WF), EpiName(EPI));
  LaunchTiming& lt = ThreadLaunchTiming();
  if (lt.start != nullptr) {
    hipExtLaunchKernelGGL((gemv_ksplit_kernel<A, WF, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kSkWaves * 64),
                          0, s, lt.start, lt.stop, 0, g);
    lt.used = true;
  } else {
    hipLaunchKernelGGL((gemv_ksplit_kernel<A, WF, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kSkWaves * 64), 0,
                       s, g);
  }
  AM_RETURN_IF_LAUNCH_FAILED("gemv");
  return AM_STATUS_OK;
}

template <class A, int WF, bool NORM, int EPI, int JM, int P, int NW, bool ONE>
am_status_code LaunchGrid(const GemvArgs& g, int64_t blocks, int64_t lds, hipStream_t s) {
  RecordLaunch(blocks, NW * 64, static_cast<int32_t>(lds), "gemv<%s,%s,%s,norm=%d,jm=%d,p=%d,nw=%d,one=%d>",
               A::kDtype == AM_DT_BF16 ? "bf16" : "f32", WfName(WF), EpiName(EPI), NORM ? 1 : 0, JM, P, NW,
               ONE ? 1 : 0);
  LaunchTiming& lt = ThreadLaunchTiming();
  if (lt.start != nullptr) {
    hipExtLaunchKernelGGL((gemv_kernel<A, WF, NORM, EPI, JM, P, NW, ONE>), dim3(static_cast<unsigned>(blocks)),
                          dim3(NW * 64), static_cast<size_t>(lds), s, lt.start, lt.stop, 0, g);
    lt.used = true;
  } else {
    hipLaunchKernelGGL((gemv_kernel<A, WF, NORM, EPI, JM, P, NW, ONE>), dim3(static_cast<unsigned>(blocks)),
                       dim3(NW * 64), static_cast<size_t>(lds), s, g);
  }
  AM_RETURN_IF_LAUNCH_FAILED("gemv");
  return AM_STATUS_OK;
}

template <class A, int WF, bool NORM, int EPI, int JM, int P, int NW>
am_status_code LaunchNW(const GemvArgs& g, int64_t lds, hipStream_t s) {
  // Persistent grid: at most the resident blocks per CU (one, for the large blocks),
  // iterations strided over the waves.
  static thread_local int64_t cached_lds = -1;
  static thread_local int cached_blocks = 1;
  if (cached_lds != lds) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, gemv_kernel<A, WF, NORM, EPI, JM, P, NW>, NW * 64,
                                                     static_cast<size_t>(lds)) != hipSuccess || nb < 1)
      nb = 1;
    cached_blocks = nb;
    cached_lds = lds;
  }
  const int64_t niter = CeilDiv(g.units, P);
  int64_t blocks = std::min<int64_t>(static_cast<int64_t>(DeviceCUs()) * cached_blocks, CeilDiv(niter, NW));
  if (blocks > 65536) blocks = 65536;
  // one load block per wave: x in registers (a single block per iteration) and no
  // wave with a second iteration
  constexpr bool XL = JM * XStore<A, WF>::kDW > 32;
  if constexpr (!XL) {
    if (blocks * NW >= niter) return LaunchGrid<A, WF, NORM, EPI, JM, P, NW, true>(g, blocks, lds, s);
  }
  return LaunchGrid<A, WF, NORM, EPI, JM, P, NW, false>(g, blocks, lds, s);
}

template <class A, int WF, bool NORM, int EPI, int JM, int P>
am_status_code LaunchJ(const GemvArgs& g, hipStream_t s) {
  using XS = XStore<A, WF>;
  const int64_t tb = A::kDtype == AM_DT_BF16 ? 2 : 4;
  int64_t lds = ((g.k * XS::kBytes + 15) / 16) * 16 + (XS::kOff != 0.0f ? (((g.row_bytes / 16) * 4 + 15) / 16) * 16 : 0);
  if (EPI == kEpiResidual) lds += ((g.n * tb + 15) / 16) * 16;
  if (EPI == kEpiQkv) lds += g.d * 4;
  if (lds > 150 * 1024) return SetLastError(AM_STATUS_INVALID_ARGUMENT, "gemv: in_features too large for LDS staging");
  GemvArgs ga = g;
  auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
  ga.vec = al16(g.x) && (g.k * tb) % 16 == 0 && (!NORM || al16(g.norm_w)) &&
           (EPI != kEpiResidual || (al16(g.residual) && (g.n * tb) % 16 == 0));
  // Large problems: one 8-wave block per CU, so x is staged once per CU (x-in-LDS
  // kernels as soon as every wave has an iteration, register-x kernels from two
  // iterations per wave).  Small ones: 4-wave blocks spread over every CU.  (Block
  // sizes and pairs per iteration were chosen by measurement on MI355X.)
  constexpr bool XL = JM * XS::kDW > 32;
  constexpr int NWB = (P == 2 && !XL && WF == AM_WF_INT4) ? 12 : 8;
  if (CeilDiv(g.units, P) >= static_cast<int64_t>(DeviceCUs()) * NWB * (XL ? 1 : 2))
    return LaunchNW<A, WF, NORM, EPI, JM, P, NWB>(ga, lds, s);
  return LaunchNW<A, WF, NORM, EPI, JM, P, 4>(ga, lds, s);
}

// Chunk-steps per row (J) pick the instantiation: JM >= J chunk-steps per lane,
// bounded so the prologue's x pieces per thread stay within 32 registers.
template <class A, int WF, bool NORM, int EPI>
am_status_code LaunchT(const GemvArgs& g, hipStream_t s) {
  using XS = XStore<A, WF>;
  const int64_t J = CeilDiv(g.row_bytes / 16, 64);
  // Long rows (more than two chunk-steps per lane): split each row over a block's
  // lanes, one chunk per lane.  That kernel reads x in its storage format (bf16
  // exactly where the dot takes bf16 pairs, fp32 for fp32 activations).
  constexpr bool kSkFormat = (A::kDtype == AM_DT_BF16) == XS::kBF16;
  if constexpr (!NORM && kSkFormat && (EPI == kEpiStore || EPI == kEpiResidual)) {
    const int64_t tb = A::kDtype == AM_DT_BF16 ? 2 : 4;
    auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; };
    const bool vec = al16(g.x) && (g.k * tb) % 16 == 0 && (EPI != kEpiResidual || al16(g.residual));
    if (J * XS::kDW > 32 && vec && g.row_bytes / 16 <= kSkWaves * 64 && g.n < (int64_t{1} << 31) / kSkRows) {
      GemvArgs ga = g;
      ga.vec = 1;
      return LaunchKsplit<A, WF, EPI>(ga, s);
    }
  }
  // One row pair per iteration keeps two weight buffers within ~100 registers, so
  // four to five waves fit per SIMD; the lm_head (argmax epilogue, 64k pairs) runs two
  // pairs per iteration.
  constexpr int PS = EPI == kEpiLmHead ? 2 : 1;
  if (J <= 2) return LaunchJ<A, WF, NORM, EPI, 2, PS>(g, s);
  if (J <= 4) return LaunchJ<A, WF, NORM, EPI, 4, 1>(g, s);
  // The prologue holds a thread's x input pieces (JM*64*kc values over >= 256
  // threads) in registers: at most 8 pieces, i.e. JM * kc <= 32 * (values per piece).
  constexpr int kEpp = 16 / static_cast<int>(sizeof(typename A::T));
  if constexpr (8 * Fmt<WF>::kc <= 32 * kEpp) {
    if (J <= 8) return LaunchJ<A, WF, NORM, EPI, 8, 1>(g, s);
  }
  if constexpr (16 * Fmt<WF>::kc <= 32 * kEpp) {
    if (J <= 16) return LaunchJ<A, WF, NORM, EPI, 16, 1>(g, s);
  }
  if constexpr (32 * Fmt<WF>::kc <= 32 * kEpp) {
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

LaunchTiming& ThreadLaunchTiming() noexcept {
  static thread_local LaunchTiming t;
  return t;
}

void RecordLaunch(int64_t grid, int32_t block_threads, int32_t lds_bytes, const char* fmt, ...) noexcept {
  LaunchTiming& t = ThreadLaunchTiming();
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(t.kernel, sizeof(t.kernel), fmt, ap);
  va_end(ap);
  t.grid = grid;
  t.block_threads = block_threads;
  t.lds_bytes = lds_bytes;
}

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
  AM_CHECK_ARG(a->rows >= 0, "fused_qkv: negative rows");
  if (auto st = ValidateWeight(a->w_qkv); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_qkv: dtype");
  AM_CHECK_ARG(a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0 && a->head_dim > 0 && a->head_dim % 2 == 0,
               "fused_qkv: bad head configuration");
  AM_CHECK_ARG(a->w_qkv.n == (a->hq + 2 * a->hkv) * a->head_dim, "fused_qkv: weight rows != (hq+2hkv)*d");
  AM_CHECK_ARG(a->head_dim <= 512, "fused_qkv: head_dim above 512");
  AM_CHECK_ARG(a->w_qkv.n < (int64_t{1} << 31), "fused_qkv: too many weight rows");
  AM_CHECK_ARG(a->h && a->norm_w && a->cos_tab && a->sin_tab && a->pos && a->q_out && a->k_cache && a->v_cache,
               "fused_qkv: null pointer");
  AM_CHECK_ARG(a->eps > 0.0f, "fused_qkv: eps must be positive");
  if (a->rows > 1) return BatchQkv(a, AsStream(stream));
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
  if (auto st = MakeKvRows(a->pages, 0, a->capacity, a->hkv, a->head_dim, &g.kv); st != AM_STATUS_OK) return st;
  return Dispatch<true, kEpiQkv>(a->dtype, a->w_qkv.format, g, AsStream(stream));
}

extern "C" am_status_code am_gfx950_fused_linear_residual(const am_gfx950_fused_linear_residual_args* a,
                                                          void* stream) {
  AM_CHECK_ARG(a != nullptr, "fused_linear_residual: null args");
  if (auto st = ValidateWeight(a->w); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16, "fused_linear_residual: dtype");
  AM_CHECK_ARG(a->x && a->h, "fused_linear_residual: null pointer");
  AM_CHECK_ARG(a->rows >= 0, "fused_linear_residual: negative rows");
  if (a->rows > 1) return BatchLinearResidual(a, AsStream(stream));
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
  AM_CHECK_ARG(a->rows >= 0, "fused_gate_up: negative rows");
  if (a->rows > 1) return BatchGateUp(a, AsStream(stream));
  GemvArgs g = BaseArgs(a->w_gate_up);
  g.x = a->h;
  g.norm_w = a->norm_w;
  g.eps = a->eps;
  g.out = a->act_out;
  return Dispatch<true, kEpiGateUp>(a->dtype, a->w_gate_up.format, g, AsStream(stream));
}

extern "C" am_status_code am_gfx950_last_launch(am_gfx950_launch_info* out) {
  AM_CHECK_ARG(out != nullptr, "last_launch: null out");
  const LaunchTiming& t = ThreadLaunchTiming();
  std::memcpy(out->kernel, t.kernel, sizeof(out->kernel));
  out->kernel[sizeof(out->kernel) - 1] = 0;
  out->grid = t.grid;
  out->block_threads = t.block_threads;
  out->lds_bytes = t.lds_bytes;
  return AM_STATUS_OK;
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
  AM_CHECK_ARG(a->rows >= 0, "fused_lm_head: negative rows");
  if (a->rows > 1) {
    // batched rows: RMSNorm + logits on the batched GEMV, then per-row argmax and the
    // decode-state update
    hipStream_t s = AsStream(stream);
    AM_CHECK_ARG(a->tokens_hist == nullptr || a->hist_stride > 0, "fused_lm_head: batched rows need hist_stride");
    if (auto st = BatchNormLogits(a, s); st != AM_STATUS_OK) return st;
    am_gfx950_argmax_args am{};
    am.x = a->logits;
    am.dtype = AM_DT_F32;
    am.rows = a->rows;
    am.n = a->w.n;
    am.out = a->token_out;
    am.workspace = a->workspace;
    am.workspace_bytes = a->workspace_bytes;
    if (auto st = am_gfx950_argmax(&am, stream); st != AM_STATUS_OK) return st;
    if (a->pos == nullptr) return AM_STATUS_OK;
    return am_gfx950_decode_advance_rows(a->token_out, a->rows, a->tokens_hist, a->hist_stride, a->pos, a->step,
                                         stream);
  }
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
