// Batched decode GEMV for gfx950: 1..16 token rows (one decode step of up to 16
// independent sequences) share a single read of the weights.
//
// The linear layers of a batched decode step are skinny GEMMs (M = batch <= 16).  A
// tile of 16 output features is the B operand of v_mfma_f32_16x16x32_bf16 (lane l:
// feature l % 16, k slice l / 16), the token rows are the A operand (rows past the
// batch are zero), so one 16-byte weight load per lane feeds one (bf16), two (INT8)
// or four (INT4) MFMAs for every row of the batch at once, and the unpack costs the
// same as for one row:
//   * INT4 word = k 8w..8w+7 (nibble j holds k 8w + {0,2,4,6,1,3,5,7}[j], value q+8):
//     (word >> 4t) & 0x000F000F | 0x43004300 is the bf16 pair (136+q_2t, 136+q_2t+1),
//     so the four shifted words are the eight bf16 of one MFMA operand in k order.
//     Each 128-k step is one quantisation group: its MFMA sum starts at -136 * sum(x)
//     (one more MFMA per 32 k, x times an all -136 operand) and is scaled by the fp16
//     group scale, staged per unit in LDS.
//   * INT8 bytes q+128 convert exactly to bf16 q; the fp32 row scale is applied once.
//   * bf16 weights are the operand as loaded.
// Products are exact (bf16 x times an integer below 256), sums are fp32.
//
// Block: 8 waves.  The prologue stages the token rows as bf16 in LDS (optionally
// RMSNorm'd; rows padded by 16 bytes so the 16-lane column reads are conflict-free).
// A unit is TPB tiles of 16 features (TPB = 2 pairs the gate and up rows of SiLU-Mul or
// the two halves of a RoPE rotation); its k steps (64 bytes of every tile row) are
// dealt to the waves round-robin, and each wave keeps R steps of loads in flight,
// running on into the block's next unit.  The waves' partial tiles are summed in LDS
// and the epilogue runs on one thread per (token row, feature), with the reference
// op-boundary roundings of the nodes it replaces.

#include <algorithm>

#include "am_kernel_common.h"
#include "am_launch_timing.h"
#include <hip/hip_ext.h>

namespace am {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBatchMaxRows = 16;
constexpr int kBWaves = 8;

enum BEpi { kBStore = 0, kBResidual = 1, kBGateUp = 2, kBQkv = 3 };

struct BatchArgs {
  const uint16_t* x;  // token rows (bf16), x_stride elements apart
  int64_t x_stride;
  const uint16_t* norm_w;
  float eps;
  const uint8_t* w;
  const void* scales;
  int32_t n, k, rows, units;
  int64_t row_bytes;
  void* out;
  int64_t out_stride;
  int32_t out_f32;
  const uint16_t* residual;
  int64_t res_stride;
  const float* cos_tab;
  const float* sin_tab;
  const int64_t* pos;  // [rows]
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int32_t hq, hkv, d;
  int64_t cap, cbs;  // cache capacity (positions), elements between rows' caches
  KvRows kv;         // K/V row addressing (contiguous rows cbs apart, or paged)
  int32_t row0;      // sequence index of token row 0 (a launch may cover a group of rows)
};

// k values per step (64 bytes of a weight row) and MFMAs per 16-byte lane slice
template <int WF> struct BFmt;
template <> struct BFmt<AM_WF_BF16> { static constexpr int ks = 32, mi = 1; };
template <> struct BFmt<AM_WF_INT8> { static constexpr int ks = 64, mi = 2; };
template <> struct BFmt<AM_WF_INT4> { static constexpr int ks = 128, mi = 4; };

__device__ __forceinline__ uint32_t pack_small_ints(float lo, float hi) {
  // small integers: the bf16 encoding is the top half of the fp32 bits
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

// B operand of MFMA i from the lane's 16-byte weight slice (k values 8i..8i+7 of it)
template <int WF>
__device__ __forceinline__ bf16x8_t w_operand(const u32x4_t& v, int i, uint32_t mask, uint32_t magic) {
  u32x4_t o;
  if constexpr (WF == AM_WF_BF16) {
    o = v;
  } else if constexpr (WF == AM_WF_INT8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t wd = v[2 * i + h];
      const float q0 = static_cast<float>(wd & 0xFFu) - 128.0f;
      const float q1 = static_cast<float>((wd >> 8) & 0xFFu) - 128.0f;
      const float q2 = static_cast<float>((wd >> 16) & 0xFFu) - 128.0f;
      const float q3 = static_cast<float>(wd >> 24) - 128.0f;
      o[2 * h] = pack_small_ints(q0, q1);
      o[2 * h + 1] = pack_small_ints(q2, q3);
    }
  } else {
    const uint32_t wd = v[i];
#pragma unroll
    for (int t = 0; t < 4; ++t) o[t] = ((wd >> (4 * t)) & mask) | magic;
  }
  return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ float bsilu(float g) {
  if (g >= 0.0f) return g / (1.0f + expf(-g));
  const float e = expf(g);
  return g * e / (1.0f + e);
}

// Block barrier for LDS traffic only: the fences are scoped to LDS, so the barrier
// waits for this wave's LDS accesses but leaves its global loads in flight
// (__syncthreads would also drain every outstanding weight load).
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }
__device__ __forceinline__ float rnd(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// first weight row of tile tt of unit u
template <int EPI, int TPB>
__device__ __forceinline__ int tile_row(const BatchArgs& p, int u, int tt) {
  if constexpr (EPI == kBGateUp) {
    return u * 16 + tt * (p.n >> 1);  // gate rows [0, F), up rows [F, 2F)
  } else if constexpr (EPI == kBQkv) {
    const int per = p.d >> 5;  // tile pairs per head: features i and i + d/2
    const int head = u / per;
    return head * p.d + (u - head * per) * 16 + tt * (p.d >> 1);
  } else {
    return (u * TPB + tt) * 16;
  }
}

// R: k steps of loads in flight per wave (per tile)
template <int WF, int EPI, bool NORM, int TPB, int R>
__global__ __launch_bounds__(kBWaves * 64) void gemv_batch_kernel(BatchArgs p) {
  constexpr int NW = kBWaves, NT = NW * 64;
  constexpr int KS = BFmt<WF>::ks, MI = BFmt<WF>::mi;
  extern __shared__ __align__(16) uint8_t bsm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = p.k, rows = p.rows, units = p.units;
  const int S = K / KS;                        // k steps
  const int XR = K + 8;                        // LDS row stride (elements)
  const int cnt = ((S + NW - 1) / NW + R - 1) / R * R;  // steps per wave and unit (padded)
  uint16_t* xs = reinterpret_cast<uint16_t*>(bsm);
  float* red = reinterpret_cast<float*>(bsm + ((static_cast<size_t>(rows) * XR * 2 + 15) & ~size_t{15}));
  // [NW][TPB][64][4]
  float* nred = red + NW * TPB * 256;                   // [NW][16]
  // INT4 group scales of a unit as fp32, double-buffered: [2][TPB][16 rows][S + 1]
  // (rows padded by one float: the 16 rows of a step read different banks)
  float* scl = nred + NW * 16;
  const int SP = S + 1, stile = TPB * 16 * SP;

  const int fl = lane & 15, g = lane >> 4;
  uint32_t mask = 0x000F000Fu, magic = 0x43004300u;  // VGPR operands (VOP3 takes no literal)
  asm volatile("" : "+v"(mask), "+v"(magic));
  const bf16x8_t neg136 = __builtin_bit_cast(bf16x8_t, u32x4_t{0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u});

  // ---- weight loads: (unit, wave step t) -> slot; step s = wave + NW * t, dead steps
  // (s >= S) re-read step S - 1 and are not accumulated ----
  // ---- prologue loads go out first (the memory counter is in order): the first
  // XB 16-byte pieces of the token rows per thread and the first gain piece, then the
  // weight ring, so staging x waits for those loads only ----
  const int pieces = K / 8;       // 16-byte pieces per token row
  const int tp = rows * pieces;   // pieces of all token rows
  constexpr int XB = 4;
  auto xsrc = [&](int e) {
    e = min(e, tp - 1);
    const int b = e / pieces;
    return reinterpret_cast<const u32x4_t*>(p.x + b * p.x_stride) + (e - b * pieces);
  };
  auto xdst = [&](int e) {  // clamped like xsrc: a duplicate writes the same piece again
    e = min(e, tp - 1);
    const int b = e / pieces;
    return reinterpret_cast<u32x4_t*>(xs + b * XR + 8 * (e - b * pieces));
  };
  u32x4_t xv[XB];
#pragma unroll
  for (int j = 0; j < XB; ++j) xv[j] = *xsrc(tid + NT * j);
  const uint4* nw = reinterpret_cast<const uint4*>(p.norm_w);
  uint4 nw0 = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (NORM) nw0 = nw[min(tid, pieces - 1)];

  // INT4 scales of a unit (TPB x 16 rows x S fp16) are loaded by the whole block as
  // coalesced 2-byte loads, up to kScl per thread, and kept in LDS; loads and stores
  // are unconditional (clamped: a duplicate rewrites the same value).
  constexpr int kScl = 4;
  const int stot = TPB * 16 * S;
  uint32_t scr[kScl];
  auto issue_scales = [&](const int (&rb)[TPB]) {
    if constexpr (WF == AM_WF_INT4) {
#pragma unroll
      for (int j = 0; j < kScl; ++j) {
        const int e = min(tid + NT * j, stot - 1);
        const int tt = e / (16 * S), rem = e - tt * 16 * S;
        const int rr = rem / S;
        const int row = min(rb[tt] + rr, p.n - 1);
        scr[j] = static_cast<const uint16_t*>(p.scales)[static_cast<int64_t>(row) * S + (rem - rr * S)];
      }
    }
  };
  auto store_scales = [&](int buf) {
    if constexpr (WF == AM_WF_INT4) {
#pragma unroll
      for (int j = 0; j < kScl; ++j) {
        const int e = min(tid + NT * j, stot - 1);
        const int tt = e / (16 * S), rem = e - tt * 16 * S;
        const int rr = rem / S;
        scl[buf * stile + (tt * 16 + rr) * SP + (rem - rr * S)] =
            static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(scr[j])));
      }
    }
  };

  // Slots refilled past the block's last unit are never read; they load the token
  // rows this block has just read (cached) instead of re-streaming weights, and stay
  // unconditional: a conditional refill makes the compiler's memory-counter waits
  // conservative at the loop head.
  u32x4_t wv[R][TPB];
  const uint8_t* tail_src = reinterpret_cast<const uint8_t*>(p.x) + (lane * 16) % (rows * K * 2);
  // lane's row pointers of the tiles of a unit (computed once per unit)
  auto row_ptrs = [&](const int (&rb)[TPB], bool tail, const uint8_t* (&wp)[TPB]) {
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt)
      wp[tt] = tail ? tail_src : p.w + static_cast<int64_t>(min(rb[tt] + fl, p.n - 1)) * p.row_bytes + 16 * g;
  };
  auto issue = [&](int r, const uint8_t* const (&wp)[TPB], int t, bool tail) {
    const int off = tail ? 0 : min(wave + NW * t, S - 1) * 64;  // wave-uniform
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt)
      wv[r][tt] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wp[tt] + off));
  };
  const int grid = gridDim.x;
  int u = blockIdx.x;
  int rb_cur[TPB];  // first weight row of each tile of unit u
#pragma unroll
  for (int tt = 0; tt < TPB; ++tt) rb_cur[tt] = tile_row<EPI, TPB>(p, u, tt);
  issue_scales(rb_cur);
  const uint8_t* wp_cur[TPB];
  row_ptrs(rb_cur, false, wp_cur);
#pragma unroll
  for (int r = 0; r < R; ++r) issue(r, wp_cur, r, false);

  // ---- prologue: token rows -> LDS (bf16), RMSNorm'd when NORM ----
  // stores are unconditional (clamped): a store under a branch would pull its load
  // into the branch, behind a wait for every weight load issued above
#pragma unroll
  for (int j = 0; j < XB; ++j) *xdst(tid + NT * j) = xv[j];
  for (int e0 = XB * NT; e0 < tp; e0 += XB * NT) {  // more than XB pieces per thread
#pragma unroll
    for (int j = 0; j < XB; ++j) xv[j] = *xsrc(e0 + tid + NT * j);
#pragma unroll
    for (int j = 0; j < XB; ++j) *xdst(e0 + tid + NT * j) = xv[j];
  }
  store_scales(0);
  if constexpr (NORM) {
    lds_sync();
    // one wave per token row: sum of squares, then 1/rms into nred[b]
    for (int b = wave; b < rows; b += NW) {
      float ss = 0.0f;
      for (int c = lane; c < pieces; c += 64) {
        const uint4 v = *reinterpret_cast<const uint4*>(xs + b * XR + 8 * c);
        const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float a0 = __uint_as_float(wd[t] << 16), a1 = __uint_as_float(wd[t] & 0xFFFF0000u);
          ss = fmaf(a0, a0, ss);
          ss = fmaf(a1, a1, ss);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) nred[b] = 1.0f / sqrtf(ss / static_cast<float>(K) + p.eps);
    }
    lds_sync();
    auto norm_piece = [&](int c, const uint4& wn) {
      const uint32_t nn[4] = {wn.x, wn.y, wn.z, wn.w};
      for (int b = 0; b < rows; ++b) {
        const float inv = nred[b];
        uint4* dst = reinterpret_cast<uint4*>(xs + b * XR + 8 * c);
        const uint4 v = *dst;
        const uint32_t xw[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float x0 = (__uint_as_float(xw[q] << 16) * inv) * __uint_as_float(nn[q] << 16);
          const float x1 = (__uint_as_float(xw[q] & 0xFFFF0000u) * inv) * __uint_as_float(nn[q] & 0xFFFF0000u);
          o[q] = static_cast<uint32_t>(f32_to_bf16_bits(x0)) | (static_cast<uint32_t>(f32_to_bf16_bits(x1)) << 16);
        }
        *dst = make_uint4(o[0], o[1], o[2], o[3]);
      }
    };
    if (tid < pieces) norm_piece(tid, nw0);  // the gain piece loaded with the rows
    for (int c = tid + NT; c < pieces; c += NT) norm_piece(c, nw[c]);
  }
  lds_sync();

  // A operand rows: lanes past the batch use zeros
  const bool xrow_ok = fl < rows;
  const uint16_t* xrow = xs + min(fl, rows - 1) * XR + g * (KS / 4);

  for (int buf = 0; u < units; u += grid, buf ^= 1) {
    const bool more = u + grid < units;  // the block has a next unit
    int rb_nxt[TPB];
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt) rb_nxt[tt] = more ? tile_row<EPI, TPB>(p, u + grid, tt) : rb_cur[tt];
    issue_scales(rb_nxt);  // next unit's scales, ahead of this unit's refills
    const uint8_t* wp_nxt[TPB];
    row_ptrs(rb_nxt, !more, wp_nxt);
    const float* sct = scl + buf * stile + fl * SP;
    f32x4_t acc[TPB];
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt) acc[tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    for (int t0 = 0; t0 < cnt; t0 += R) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int t = t0 + r;
        const int s_raw = wave + NW * t;
        const float live = s_raw < S ? 1.0f : 0.0f;  // wave-uniform: dead steps add nothing
        const int s = min(s_raw, S - 1);
        bf16x8_t xa[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
          const bf16x8_t v = *reinterpret_cast<const bf16x8_t*>(xrow + s * KS + 8 * i);
          xa[i] = xrow_ok ? v : bf16x8_t{};
        }
        // INT4: the step's MFMA sums start at -136 * sum(x) of each token row, itself an
        // MFMA of x with an all -136 operand (exact products, fp32 sums)
        f32x4_t c0 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (WF == AM_WF_INT4) {
#pragma unroll
          for (int i = 0; i < MI; ++i) c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], neg136, c0, 0, 0, 0);
        }
#pragma unroll
        for (int tt = 0; tt < TPB; ++tt) {
          f32x4_t part = c0;
#pragma unroll
          for (int i = 0; i < MI; ++i)
            part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[i], w_operand<WF>(wv[r][tt], i, mask, magic), part, 0,
                                                           0, 0);
          float sc = live;
          if constexpr (WF == AM_WF_INT4) sc *= sct[tt * 16 * SP + s];
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[tt][e] = fmaf(sc, part[e], acc[tt][e]);
        }
        // refill the slot: the next step of this unit, or the first steps of the next
        // unit; nothing past the block's last unit (those slots are never read again)
        int tn = t + R;
        const bool wrap = tn >= cnt;
        if (wrap) tn -= cnt;
        issue(r, wrap ? wp_nxt : wp_cur, tn, wrap && !more);
      }
    }

    // ---- reduce the waves' partial tiles, then the epilogue ----
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt)
      *reinterpret_cast<f32x4_t*>(red + ((wave * TPB + tt) * 64 + lane) * 4) = acc[tt];
    store_scales(buf ^ 1);  // every wave is past its last read of that buffer (unit u-1)
    lds_sync();
    if (tid < rows * 16) {
      const int b = tid >> 4, f = tid & 15;
      const int src = (f + 16 * (b >> 2)) * 4 + (b & 3);
      float v[TPB];
#pragma unroll
      for (int tt = 0; tt < TPB; ++tt) {
        float a = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) a += red[(w2 * TPB + tt) * 256 + src];
        v[tt] = a;
      }
      const int j0 = rb_cur[0] + f;
      if constexpr (WF == AM_WF_INT8) {
#pragma unroll
        for (int tt = 0; tt < TPB; ++tt) {
          const int j = min(rb_cur[tt] + f, p.n - 1);
          v[tt] *= static_cast<const float*>(p.scales)[j];
        }
      }
      if constexpr (EPI == kBStore) {
#pragma unroll
        for (int tt = 0; tt < TPB; ++tt) {
          const int j = j0 + 16 * tt;
          if (j < p.n) {
            if (p.out_f32)
              static_cast<float*>(p.out)[b * p.out_stride + j] = v[tt];
            else
              static_cast<uint16_t*>(p.out)[b * p.out_stride + j] = f32_to_bf16_bits(v[tt]);
          }
        }
      } else if constexpr (EPI == kBResidual) {
#pragma unroll
        for (int tt = 0; tt < TPB; ++tt) {
          const int j = j0 + 16 * tt;
          if (j < p.n) {
            const float h = bf(p.residual[b * p.res_stride + j]);
            static_cast<uint16_t*>(p.out)[b * p.out_stride + j] = f32_to_bf16_bits(h + rnd(v[tt]));
          }
        }
      } else if constexpr (EPI == kBGateUp) {
        const float gg = rnd(v[0]), up = rnd(v[1]);
        static_cast<uint16_t*>(p.out)[b * p.out_stride + j0] = f32_to_bf16_bits(bsilu(gg) * up);
      } else if constexpr (EPI == kBQkv) {
        const int half = p.d >> 1;
        const int head = j0 / p.d, i = j0 - head * p.d;  // i < d/2
        const float y0 = rnd(v[0]), y1 = rnd(v[1]);
        const int64_t pos = p.pos[b];
        const bool in_cache = pos >= 0 && pos < p.cap;
        const int64_t pr = in_cache ? pos : 0;  // table row (the tables hold cap positions)
        if (head < p.hq + p.hkv) {
          const float c = p.cos_tab[pr * half + i], sn = p.sin_tab[pr * half + i];
          float o0, o1;
          rope_rotate(y0, y1, c, sn, o0, o1);
          if (head < p.hq) {
            uint16_t* q = p.q_out + static_cast<int64_t>(b) * p.hq * p.d + head * p.d;
            q[i] = f32_to_bf16_bits(o0);
            q[i + half] = f32_to_bf16_bits(o1);
          } else if (in_cache) {
            const int64_t row = p.kv.WriteRow(p.row0 + b, head - p.hq, pos);
            if (row >= 0) {
              uint16_t* kc = p.k_cache + row;
              kc[i] = f32_to_bf16_bits(o0);
              kc[i + half] = f32_to_bf16_bits(o1);
            }
          }
        } else if (in_cache) {
          const int64_t row = p.kv.WriteRow(p.row0 + b, head - p.hq - p.hkv, pos);
          if (row >= 0) {
            uint16_t* vc = p.v_cache + row;
            vc[i] = f32_to_bf16_bits(y0);
            vc[i + half] = f32_to_bf16_bits(y1);
          }
        }
      }
    }
    lds_sync();
#pragma unroll
    for (int tt = 0; tt < TPB; ++tt) {
      rb_cur[tt] = rb_nxt[tt];
      wp_cur[tt] = wp_nxt[tt];
    }
  }
}

// ---- host ----
template <int WF, int EPI, bool NORM, int TPB, int R>
am_status_code LaunchBatch(const BatchArgs& a, size_t lds, hipStream_t s) {
  auto fn = gemv_batch_kernel<WF, EPI, NORM, TPB, R>;
  static thread_local size_t cached_lds = 0;
  static thread_local int cached_blocks = 0;
  if (cached_lds != lds) {
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return SetLastError(AM_STATUS_INTERNAL, "gemv_batch: could not raise the dynamic LDS limit");
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, kBWaves * 64, lds) != hipSuccess || nb < 1) nb = 1;
    cached_blocks = nb;
    cached_lds = lds;
  }
  const int64_t blocks = std::min<int64_t>(a.units, static_cast<int64_t>(DeviceCUs()) * cached_blocks);
  RecordLaunch(blocks, kBWaves * 64, static_cast<int32_t>(lds), "gemv_batch<wf=%d,epi=%d,norm=%d,tpb=%d,r=%d>", WF, EPI,
               NORM ? 1 : 0, TPB, R);
  LaunchTiming& lt = ThreadLaunchTiming();
  if (lt.start != nullptr) {
    hipExtLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(kBWaves * 64), lds, s, lt.start, lt.stop, 0,
                          a);
    lt.used = true;
  } else {
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(kBWaves * 64), lds, s, a);
  }
  AM_RETURN_IF_LAUNCH_FAILED("gemv_batch");
  return AM_STATUS_OK;
}

// Single-tile units keep 8 steps in flight per wave once a wave has that many steps
// (long rows); paired units (two loads per step) and short rows keep 4.
template <int WF, int EPI, bool NORM, int TPB>
am_status_code LaunchBatchR(const BatchArgs& a, size_t lds, hipStream_t s) {
  if constexpr (TPB == 1) {
    const int S = a.k / BFmt<WF>::ks;
    if ((S + kBWaves - 1) / kBWaves >= 8) return LaunchBatch<WF, EPI, NORM, TPB, 8>(a, lds, s);
  }
  return LaunchBatch<WF, EPI, NORM, TPB, 4>(a, lds, s);
}

template <int EPI, bool NORM, int TPB>
am_status_code DispatchBatch(int32_t fmt, const BatchArgs& a, size_t lds, hipStream_t s) {
  switch (fmt) {
    case AM_WF_BF16: return LaunchBatchR<AM_WF_BF16, EPI, NORM, TPB>(a, lds, s);
    case AM_WF_INT8: return LaunchBatchR<AM_WF_INT8, EPI, NORM, TPB>(a, lds, s);
    default: return LaunchBatchR<AM_WF_INT4, EPI, NORM, TPB>(a, lds, s);
  }
}

bool Aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// LDS of one block for `rows` token rows: the rows (bf16, padded by 16 bytes), the
// per-wave partial tiles, 1/rms per row and, for INT4, the unit's group scales.
size_t BatchLdsOf(const am_gfx950_weight& w, int64_t rows, int tpb) {
  size_t b = (static_cast<size_t>(rows) * (w.k + 8) * 2 + 15) & ~size_t{15};
  b += static_cast<size_t>(kBWaves) * tpb * 256 * 4 + kBWaves * 16 * 4;
  if (w.format == AM_WF_INT4) b += static_cast<size_t>(2) * tpb * 16 * (w.k / 128 + 1) * 4;
  return b;
}

// Most token rows (up to 16) whose block fits the 160 KB of LDS (0: not even one).
int64_t BatchRowsFit(const am_gfx950_weight& w, int tpb) {
  for (int64_t r = kBatchMaxRows; r >= 1; --r)
    if (BatchLdsOf(w, r, tpb) <= 160 * 1024) return r;
  return 0;
}

// Shape / format checks shared by every batched entry; fills the weight fields and
// returns the dynamic LDS bytes through *lds.
am_status_code PrepareBatch(const am_gfx950_weight& w, int64_t rows, const void* x, int64_t x_stride, int tpb,
                            BatchArgs* a, size_t* lds) {
  AM_CHECK_ARG(rows >= 1 && rows <= kBatchMaxRows, "batched decode: rows must be 1..16");
  AM_CHECK_ARG(w.data != nullptr && w.n > 0 && w.k > 0 && w.n < (int64_t{1} << 30) && w.k < (int64_t{1} << 30),
               "batched decode: bad weight shape");
  AM_CHECK_ARG(w.format == AM_WF_BF16 || w.format == AM_WF_INT8 || w.format == AM_WF_INT4,
               "batched decode: weights must be bf16, int8 or int4");
  AM_CHECK_ARG(w.format != AM_WF_INT4 || w.group_size == 128, "batched decode: int4 needs group_size 128");
  AM_CHECK_ARG(w.format == AM_WF_BF16 || w.scales != nullptr, "batched decode: quantized weight needs scales");
  const int64_t ks = w.format == AM_WF_BF16 ? 32 : (w.format == AM_WF_INT8 ? 64 : 128);
  AM_CHECK_ARG(w.k % ks == 0, "batched decode: in_features must be a multiple of 32 (bf16), 64 (int8), 128 (int4)");
  AM_CHECK_ARG(Aligned16(w.data) && x != nullptr && Aligned16(x) && x_stride % 8 == 0 && x_stride >= w.k,
               "batched decode: weights and token rows must be 16-byte aligned");
  const int64_t S = w.k / ks;
  if (w.format == AM_WF_INT4)
    AM_CHECK_ARG(tpb * 16 * S <= 4 * kBWaves * 64, "batched decode: int4 rows too long for the scale tile");
  AM_CHECK_ARG(BatchRowsFit(w, tpb) >= 1, "batched decode: one token row does not fit in LDS (in_features too large)");
  a->x = static_cast<const uint16_t*>(x);
  a->x_stride = x_stride;
  a->w = static_cast<const uint8_t*>(w.data);
  a->scales = w.scales;
  a->n = static_cast<int32_t>(w.n);
  a->k = static_cast<int32_t>(w.k);
  a->rows = static_cast<int32_t>(rows);
  a->row_bytes = w.format == AM_WF_BF16 ? 2 * w.k : (w.format == AM_WF_INT8 ? w.k : w.k / 2);
  *lds = BatchLdsOf(w, std::min<int64_t>(rows, BatchRowsFit(w, tpb)), tpb);
  return AM_STATUS_OK;
}

// Runs launch(args, lds) over groups of token rows small enough for one block's LDS
// (every group re-reads the weights): the k = 14336 down projection of the 8B shape
// fits 5 rows of 14336 bf16 values; shorter rows fit all 16.  off(args, g0) moves the
// group's row pointers (token rows, outputs, residuals, positions) to row g0.
template <class Launch, class Offset>
am_status_code ForRowGroups(const BatchArgs& a, const am_gfx950_weight& w, int tpb, Launch launch, Offset off) {
  const int64_t per = std::min<int64_t>(a.rows, BatchRowsFit(w, tpb));
  for (int64_t g0 = 0; g0 < a.rows; g0 += per) {
    BatchArgs ga = a;
    ga.rows = static_cast<int32_t>(std::min<int64_t>(per, a.rows - g0));
    ga.row0 = a.row0 + static_cast<int32_t>(g0);
    ga.x = a.x + g0 * a.x_stride;
    off(ga, g0);
    if (auto st = launch(ga, BatchLdsOf(w, ga.rows, tpb)); st != AM_STATUS_OK) return st;
  }
  return AM_STATUS_OK;
}

}  // namespace

// Linear rows through the batched kernel (am_gfx950_linear with 1 <= m <= 16 and bf16
// activations): out[m][n] (bf16 or fp32), optional residual added in bf16.
bool BatchLinearEligible(int32_t act, const am_gfx950_weight& w, int64_t m, const void* x) {
  if (act != AM_DT_BF16 || m < 1 || m > kBatchMaxRows) return false;
  if (w.format == AM_WF_F32 || (w.format == AM_WF_INT4 && w.group_size != 128)) return false;
  const int64_t ks = w.format == AM_WF_BF16 ? 32 : (w.format == AM_WF_INT8 ? 64 : 128);
  if (w.k % ks != 0 || !Aligned16(x) || !Aligned16(w.data)) return false;
  size_t b = static_cast<size_t>(m) * (w.k + 8) * 2 + kBWaves * 256 * 4 + kBWaves * 64 + 16;
  if (w.format == AM_WF_INT4) {
    if (16 * (w.k / 128) > 4 * kBWaves * 64) return false;
    b += static_cast<size_t>(2) * 16 * (w.k / 128 + 1) * 4;
  }
  return b <= 160 * 1024;
}

am_status_code BatchLinear(const void* x, int64_t m, const am_gfx950_weight& w, void* out, int32_t out_dtype,
                           const void* residual, hipStream_t s) {
  BatchArgs a{};
  size_t lds = 0;
  if (auto st = PrepareBatch(w, m, x, w.k, 1, &a, &lds); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(out != nullptr, "linear: null output");
  a.out = out;
  a.out_stride = w.n;
  a.out_f32 = out_dtype == AM_DT_F32 ? 1 : 0;
  a.units = static_cast<int32_t>(CeilDiv(w.n, 16));
  auto off = [&](BatchArgs& g, int64_t g0) {
    g.out = static_cast<uint8_t*>(out) + g0 * a.out_stride * (a.out_f32 ? 4 : 2);
    if (g.residual != nullptr) g.residual = a.residual + g0 * a.res_stride;
  };
  if (residual != nullptr) {
    AM_CHECK_ARG(out_dtype == AM_DT_BF16, "linear: residual needs out dtype == activation dtype");
    a.residual = static_cast<const uint16_t*>(residual);
    a.res_stride = w.n;
    return ForRowGroups(a, w, 1, [&](const BatchArgs& g, size_t l) {
      return DispatchBatch<kBResidual, false, 1>(w.format, g, l, s); }, off);
  }
  return ForRowGroups(a, w, 1, [&](const BatchArgs& g, size_t l) {
    return DispatchBatch<kBStore, false, 1>(w.format, g, l, s); }, off);
}

am_status_code BatchQkv(const am_gfx950_fused_qkv_args* q, hipStream_t s) {
  BatchArgs a{};
  size_t lds = 0;
  if (auto st = PrepareBatch(q->w_qkv, q->rows, q->h, q->w_qkv.k, 2, &a, &lds); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(q->dtype == AM_DT_BF16, "fused_qkv: batched rows need bf16 activations");
  AM_CHECK_ARG(q->head_dim % 32 == 0, "fused_qkv: batched rows need head_dim % 32 == 0");
  AM_CHECK_ARG(Aligned16(q->norm_w), "fused_qkv: norm weight must be 16-byte aligned");
  AM_CHECK_ARG(q->cache_batch_stride >= 0, "fused_qkv: negative cache batch stride");
  a.norm_w = static_cast<const uint16_t*>(q->norm_w);
  a.eps = q->eps;
  a.cos_tab = q->cos_tab;
  a.sin_tab = q->sin_tab;
  a.pos = q->pos;
  a.q_out = static_cast<uint16_t*>(q->q_out);
  a.k_cache = static_cast<uint16_t*>(q->k_cache);
  a.v_cache = static_cast<uint16_t*>(q->v_cache);
  a.hq = static_cast<int32_t>(q->hq);
  a.hkv = static_cast<int32_t>(q->hkv);
  a.d = static_cast<int32_t>(q->head_dim);
  a.cap = q->capacity;
  a.cbs = q->cache_batch_stride;
  if (auto st = MakeKvRows(q->pages, a.cbs, a.cap, q->hkv, q->head_dim, &a.kv); st != AM_STATUS_OK) return st;
  a.units = static_cast<int32_t>((q->hq + 2 * q->hkv) * (q->head_dim / 32));
  return ForRowGroups(a, q->w_qkv, 2, [&](const BatchArgs& g, size_t l) {
    return DispatchBatch<kBQkv, true, 2>(q->w_qkv.format, g, l, s); },
    [&](BatchArgs& g, int64_t g0) {
      g.q_out = a.q_out + g0 * a.hq * a.d;
      g.pos = a.pos + g0;
    });
}

am_status_code BatchLinearResidual(const am_gfx950_fused_linear_residual_args* r, hipStream_t s) {
  BatchArgs a{};
  size_t lds = 0;
  if (auto st = PrepareBatch(r->w, r->rows, r->x, r->w.k, 1, &a, &lds); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(r->dtype == AM_DT_BF16, "fused_linear_residual: batched rows need bf16 activations");
  a.out = r->h;
  a.out_stride = r->w.n;
  a.residual = static_cast<const uint16_t*>(r->h);
  a.res_stride = r->w.n;
  a.units = static_cast<int32_t>(CeilDiv(r->w.n, 16));
  return ForRowGroups(a, r->w, 1, [&](const BatchArgs& g, size_t l) {
    return DispatchBatch<kBResidual, false, 1>(r->w.format, g, l, s); },
    [&](BatchArgs& g, int64_t g0) {
      g.out = static_cast<uint16_t*>(a.out) + g0 * a.out_stride;
      g.residual = a.residual + g0 * a.res_stride;
    });
}

am_status_code BatchGateUp(const am_gfx950_fused_gate_up_args* gu, hipStream_t s) {
  BatchArgs a{};
  size_t lds = 0;
  if (auto st = PrepareBatch(gu->w_gate_up, gu->rows, gu->h, gu->w_gate_up.k, 2, &a, &lds); st != AM_STATUS_OK)
    return st;
  AM_CHECK_ARG(gu->dtype == AM_DT_BF16, "fused_gate_up: batched rows need bf16 activations");
  AM_CHECK_ARG(gu->w_gate_up.n % 32 == 0, "fused_gate_up: batched rows need ffn % 16 == 0");
  AM_CHECK_ARG(Aligned16(gu->norm_w), "fused_gate_up: norm weight must be 16-byte aligned");
  a.norm_w = static_cast<const uint16_t*>(gu->norm_w);
  a.eps = gu->eps;
  a.out = gu->act_out;
  a.out_stride = gu->w_gate_up.n / 2;
  a.units = static_cast<int32_t>(gu->w_gate_up.n / 32);
  return ForRowGroups(a, gu->w_gate_up, 2, [&](const BatchArgs& g, size_t l) {
    return DispatchBatch<kBGateUp, true, 2>(gu->w_gate_up.format, g, l, s); },
    [&](BatchArgs& g, int64_t g0) { g.out = static_cast<uint16_t*>(a.out) + g0 * a.out_stride; });
}

// RMSNorm -> lm_head logits (fp32) for rows token rows.
am_status_code BatchNormLogits(const am_gfx950_fused_lm_head_args* lm, hipStream_t s) {
  BatchArgs a{};
  size_t lds = 0;
  if (auto st = PrepareBatch(lm->w, lm->rows, lm->h, lm->w.k, 1, &a, &lds); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(lm->dtype == AM_DT_BF16, "fused_lm_head: batched rows need bf16 activations");
  AM_CHECK_ARG(lm->logits != nullptr, "fused_lm_head: batched rows need a logits buffer");
  AM_CHECK_ARG(Aligned16(lm->norm_w), "fused_lm_head: norm weight must be 16-byte aligned");
  a.norm_w = static_cast<const uint16_t*>(lm->norm_w);
  a.eps = lm->eps;
  a.out = lm->logits;
  a.out_stride = lm->w.n;
  a.out_f32 = 1;
  a.units = static_cast<int32_t>(CeilDiv(lm->w.n, 16));
  return ForRowGroups(a, lm->w, 1, [&](const BatchArgs& g, size_t l) {
    return DispatchBatch<kBStore, true, 1>(lm->w.format, g, l, s); },
    [&](BatchArgs& g, int64_t g0) { g.out = static_cast<float*>(a.out) + g0 * a.out_stride; });
}

}  // namespace am
