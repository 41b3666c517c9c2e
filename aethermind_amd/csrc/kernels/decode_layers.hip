// Persistent decode of every transformer layer of one token (batch 1) on gfx950:
// one launch runs the per-layer node sequence of model_graph_builder.cpp:133-290
// (RmsNorm -> Linear q|k|v -> RoPE -> KVCacheUpdate -> Attention -> Linear o -> Add
//  -> RmsNorm -> Linear gate|up -> SiluMul -> Linear down -> Add) for all layers.
//
// Why one launch: at batch 1 a layer is five dependent steps over ~112 MB of INT4
// weights (8B shape).  As separate kernels each step pays a launch, a ramp and a
// drain (~3.5-4.5 us); here a step boundary is a data-carrying flag exchange between
// blocks (~1.6 us for a 4096-value vector), and every block issues the weight loads of
// its next step BEFORE it waits for that step's input, so the weight stream overlaps
// the exchange.
//
// Grid: one 512-thread block per CU (the LDS request admits one block per CU, the
// grid is the CU count), all blocks resident at once.  Work split per layer:
//   P1  q|k|v rows in quads (r, r+1, r+64, r+65) of one head: two RoPE pairs whose
//       outputs are adjacent values; RMSNorm of h recomputed by every block.
//   P2  attention partials: unit = (kv head, split of the positions), online softmax
//       over the unit's positions for all q heads of the group (GQA).
//   P2b merge of the splits: one block per q head.
//   P3  o rows in pairs + residual (h kept in LDS since P1).
//   P4  RMSNorm + gate|up rows for two adjacent features + SiLU-Mul.
//   P5  down projection split-K: a block owns H/grid consecutive rows, thread t holds
//       16-byte chunk t of each of them, the x values of chunk t arrive straight into
//       its registers; + residual.
// Exchange format ("LL" words): 64-bit words = (epoch << 32) | payload, written and
// read with device-scope relaxed 64-bit atomics (single-copy atomic).  A reader polls
// until every word it needs carries the current layer's epoch: no fences, no cache
// maintenance, no counters.  Buffers alternate by layer parity, so a word is never
// rewritten while a slower block may still read its previous value (a block can only
// reach layer l+2 after every block has finished layer l).  The epoch of layer l of a
// launch is E0 + l + 1, E0 read from the workspace and advanced by L at the end.
// Every wait is bounded: a block that waits too long sets the workspace abort flag,
// every other wait sees it and returns, and the launch ends (the host reports it).
//
// Numerics match the fused per-op decode kernels: bf16 rounding at every reference
// op boundary, fp32 accumulation, INT4 dot as sum x*(136+q) - 136*sum x with exact
// products, RoPE in fp32 from the bf16 projection, fp32 softmax.

#include <algorithm>

#include "am_gemv_common.h"
#include "am_launch_timing.h"
#include <hip/hip_ext.h>

namespace am {
namespace {

constexpr int kNT = 512;  // threads per block
constexpr int kNW = kNT / 64;
constexpr int kD = 128;   // head_dim
constexpr int kMaxG = 8;  // q heads per kv head
constexpr int kGrid = 256;
constexpr int kLds = 96 * 1024;  // > half of the 160 KB LDS: one block per CU
constexpr float kOff = 136.0f;   // INT4 bf16 unpack bias (128 exponent + 8 offset)
constexpr long kSpinLimit = 1L << 18;

struct Args {
  const am_gfx950_decode_layer* layers;
  int32_t L, H, hq, hkv, F, cap;
  float eps;
  const float* cos_tab;
  const float* sin_tab;
  const int64_t* pos;
  uint16_t* h;
  uint64_t* ll;    // two parities of ll_par words
  int64_t ll_par;  // words per parity
  int32_t o_qkv, o_att, o_hm, o_h, o_a, o_part, o_flag;
  uint32_t* epoch;
  int32_t* abort_flag;
  uint64_t* timeline;  // optional: [L][grid][16] phase stamps (100 MHz), null = off
};

// Phase stamp k of (layer l, this block): thread 0 writes the 100 MHz wall clock.
__device__ __forceinline__ void stamp(const Args& a, int l, int k) {
  if (a.timeline != nullptr && threadIdx.x == 0)
    a.timeline[(static_cast<int64_t>(l) * gridDim.x + blockIdx.x) * 16 + k] = __builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ uint64_t ll_ld(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_st(uint64_t* p, uint32_t ep, uint32_t v) {
  __hip_atomic_store(p, (static_cast<uint64_t>(ep) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool aborted(const int32_t* f) {
  return __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Polls the PER words idx(j) (negative: none) of buf until each carries epoch ep;
// payloads to val.  Returns false when the launch is aborted (or this wait times out,
// which aborts it).
template <int PER, class Idx>
__device__ __forceinline__ bool ll_wait(const uint64_t* buf, Idx idx, uint32_t ep, uint32_t (&val)[PER],
                                        int32_t* abort_flag) {
  long spins = 0;
  for (;;) {
    uint64_t v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int i = idx(j);
      v[j] = i >= 0 ? ll_ld(buf + i) : (static_cast<uint64_t>(ep) << 32);
    }
    bool ok = true;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      ok &= static_cast<uint32_t>(v[j] >> 32) == ep;
      val[j] = static_cast<uint32_t>(v[j]);
    }
    if (ok) return true;
    if ((++spins & 31) == 0) {
      if (aborted(abort_flag)) return false;
      if (spins > kSpinLimit) {
        __hip_atomic_store(abort_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
      }
    }
  }
}

// Block barrier for LDS traffic only: the fences are scoped to LDS, so the barrier
// leaves outstanding global loads (the next step's weights) in flight.
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Gathers n words of buf (epoch ep) into dst[0..n) (payloads); every thread of the
// block takes part.  Returns false (block-uniformly) on abort.
__device__ __forceinline__ bool ll_gather(const uint64_t* buf, int n, uint32_t ep, uint32_t* dst, int32_t* abort_flag,
                                          int* blk_ok) {
  bool ok = true;
  for (int b0 = 0; b0 < n && ok; b0 += kNT * 8) {
    uint32_t val[8];
    auto idx = [&](int j) {
      const int i = b0 + static_cast<int>(threadIdx.x) + j * kNT;
      return i < n ? i : -1;
    };
    ok = ll_wait<8>(buf, idx, ep, val, abort_flag);
    if (ok) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (idx(j) >= 0) dst[idx(j)] = val[j];
    }
  }
  if (!ok) *blk_ok = 0;
  lds_sync();
  return *blk_ok != 0;
}

// Step outputs announced per block: after a block's exchange words of a step are
// issued, one flag word (the epoch) per block.  Consumers poll the flags of the
// blocks they depend on (one word each) and then read the data words once, still
// checking each word's epoch: a poll of the data itself would move every block's
// whole input vector through the memory system on every round.
enum FlagKind { kFlagH = 0, kFlagQkv = 1, kFlagPart = 2, kFlagAtt = 3, kFlagHm = 4, kFlagA = 5, kFlagKinds = 6 };
// one flag per 64-byte line: every block polls every producer's flag, and packed flags
// put thousands of polls per round on the same few lines
constexpr int kFlagStride = 8;

__device__ __forceinline__ void publish_flag(uint64_t* buf, int o_flag, int kind, uint32_t ep) {
  lds_sync();  // every wave of the block has issued its exchange stores
  if (threadIdx.x == 0) ll_st(buf + o_flag + (kind * kGrid + blockIdx.x) * kFlagStride, ep, 0u);
}

// Waits for the flags of producer blocks [p0, p0 + n) (n <= threads); block-uniform.
__device__ __forceinline__ bool wait_flags(const uint64_t* buf, int o_flag, int kind, int p0, int n, uint32_t ep,
                                           int32_t* abort_flag, int* blk_ok) {
  bool ok = true;
  const int t = static_cast<int>(threadIdx.x);
  if (t < n) {
    uint32_t v[1];
    auto idx = [&](int) { return o_flag + (kind * kGrid + p0 + t) * kFlagStride; };
    ok = ll_wait<1>(buf, idx, ep, v, abort_flag);
  }
  if (!ok) *blk_ok = 0;
  lds_sync();
  return *blk_ok != 0;
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16_bits(lo)) | (static_cast<uint32_t>(f32_to_bf16_bits(hi)) << 16);
}
__device__ __forceinline__ float rnd(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ uint4 ld_w(const uint8_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum over the block; every thread receives it.  red: kNW floats of LDS.
__device__ __forceinline__ float blk_sum(float v, float* red) {
  v = wave_sum(v);
  lds_sync();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  lds_sync();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < kNW; ++w) t += red[w];
  return t;
}

// Lane's x chunks (chunk c = lane + 64 j of a K = 2048*J row) from the bf16 vector in
// LDS (as u32 pairs), and the offset correction 136 * sum(x) of each chunk.
template <int J>
__device__ __forceinline__ void lane_x(const uint32_t* xs, int lane, uint32_t (&xr)[J][16], float (&corr)[J]) {
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    const uint4* src = reinterpret_cast<const uint4*>(xs + 16 * c);
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = src[q];
      xr[j][4 * q] = v.x;
      xr[j][4 * q + 1] = v.y;
      xr[j][4 * q + 2] = v.z;
      xr[j][4 * q + 3] = v.w;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) s += lo_bf(xr[j][t]) + hi_bf(xr[j][t]);
    corr[j] = kOff * s;
  }
}

// R rows x J chunks of weights (+ fp16 group scales) of one unit, in registers.
template <int R, int J>
struct Frag {
  uint4 w[R][J];
  uint32_t s[R][J];
};

// Loads rows[r] (row indices) of a K = 2048*J INT4 weight: chunk lane + 64 j.
template <int R, int J>
__device__ __forceinline__ void load_frag(Frag<R, J>& f, const uint8_t* w, const uint16_t* sc, const int (&rows)[R],
                                          int K, int lane) {
  const int rb = K / 2, ng = K / 128;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      // 32-bit offsets: every matrix of this kernel is below 2^31 bytes (host-checked)
      f.w[r][j] = ld_w(w + static_cast<uint32_t>(rows[r] * rb + 16 * c));
      f.s[r][j] = sc[static_cast<uint32_t>(rows[r] * ng + (c >> 2))];
    }
}

template <int R, int J>
__device__ __forceinline__ void dot_frag(const Frag<R, J>& f, const uint32_t (&xr)[J][16], const float (&corr)[J],
                                         float (&acc)[R], const Unpack& up) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float a = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) a = fmaf(f16_bits_to_f32(f.s[r][j]), int4_chunk_dot_bf16(f.w[r][j], xr[j], -corr[j], up), a);
    acc[r] = a;
  }
}

// RMSNorm of the H-vector held as u32 pairs in src (LDS) with gains w (global bf16):
// dst = round((x * inv) * w), inv = 1/sqrt(mean(x^2) + eps).  wv: this thread's gain
// pairs (words t + kNT i), loaded ahead.
template <int HW>
__device__ __forceinline__ void rmsnorm_lds(const uint32_t* src, uint32_t* dst, const uint32_t (&wv)[HW], int H,
                                            float eps, float* red) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < HW; ++i) {
    const int wi = static_cast<int>(threadIdx.x) + kNT * i;
    if (wi < H / 2) {
      const uint32_t x = src[wi];
      ss = fmaf(lo_bf(x), lo_bf(x), ss);
      ss = fmaf(hi_bf(x), hi_bf(x), ss);
    }
  }
  ss = blk_sum(ss, red);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
#pragma unroll
  for (int i = 0; i < HW; ++i) {
    const int wi = static_cast<int>(threadIdx.x) + kNT * i;
    if (wi < H / 2) {
      const uint32_t x = src[wi];
      dst[wi] = pack_bf16((lo_bf(x) * inv) * lo_bf(wv[i]), (hi_bf(x) * inv) * hi_bf(wv[i]));
    }
  }
  lds_sync();
}

// Step T of fold_rows: lanes 32 >> T apart exchange half of the remaining rows.
template <int RB, int T>
__device__ __forceinline__ void fold_step(float (&v)[RB], int lane, int& row) {
  constexpr int m = 32 >> T, half = RB >> (T + 1);
  if constexpr (half >= 1) {
    const bool hi = (lane & m) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = hi ? v[i] : v[i + half];
      const float keep = hi ? v[i + half] : v[i];
      v[i] = keep + __shfl_xor(send, m, 64);
    }
    if (hi) row += half;
    fold_step<RB, T + 1>(v, lane, row);
  }
}

// Fold v[RB] (per-lane partial sums of RB rows) over the wave: returns the full sum
// of row `row` in the lanes with (lane & (64/RB - 1)) == 0.
template <int RB>
__device__ __forceinline__ float fold_rows(float (&v)[RB], int lane, int& row) {
  static_assert(RB == 2 || RB == 4 || RB == 8 || RB == 16, "RB must be 2, 4, 8 or 16");
  row = 0;
  fold_step<RB, 0>(v, lane, row);
  float s = v[0];
#pragma unroll
  for (int m = 32 / RB; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
  return s;
}

// The kernel's Args, read in place from the kernel-argument segment (scalar loads)
// wherever a phase needs them.
__device__ __forceinline__ const Args& kargs() {
  return *(const Args*)__builtin_amdgcn_kernarg_segment_ptr();  // address-space conversion
}

// LDS carve-up of the 96 KB block allocation.
struct Lds {
  uint32_t *hraw, *hmid, *xs, *qs, *kvcur;
  float* sc;
  uint32_t* vt;
  float *mg, *red;
  int* blk_ok;
};
extern __shared__ __align__(16) uint8_t dl_lds[];
template <int J>
__device__ __forceinline__ Lds carve() {
  Lds m;
  m.hraw = reinterpret_cast<uint32_t*>(dl_lds);           // H bf16: h entering the layer
  m.hmid = m.hraw + 1024 * J;                             // H bf16: h after o + residual
  m.xs = m.hmid + 1024 * J;                               // H bf16: normalised / gathered x
  m.qs = m.xs + 1024 * J;                                 // G*128 bf16 q of the unit's heads
  m.kvcur = m.qs + kMaxG * 64;                            // 128 + 128 bf16: current k, v
  m.sc = reinterpret_cast<float*>(m.kvcur + 128);         // [kMaxG][64] scores
  m.vt = reinterpret_cast<uint32_t*>(m.sc + kMaxG * 64);  // [64][64] V rows (bf16 pairs)
  m.mg = reinterpret_cast<float*>(m.vt + 64 * 64);        // merge: [4][3][128]
  m.red = m.mg + 4 * 3 * 128;                             // [kNW][16]
  m.blk_ok = reinterpret_cast<int*>(m.red + kNW * 16);
  return m;
}

// Rows of gate|up unit u (features 2u, 2u+1): gate 2u, up 2u, gate 2u+1, up 2u+1.
__device__ __forceinline__ void gate_up_rows(int u, int F, int (&rows)[4]) {
  rows[0] = 2 * u;
  rows[1] = F + 2 * u;
  rows[2] = 2 * u + 1;
  rows[3] = F + 2 * u + 1;
}

// First two gate|up units of this wave (the P4 work split), issued ahead of P4 so
// that they stream while the block waits through earlier steps.
template <int J>
__device__ __forceinline__ void issue_gate_up(const Args& a, const am_gfx950_decode_layer& Ld, Frag<4, J>& fa,
                                              Frag<4, J>& fb) {
  const int nu = a.F / 2, nb = gridDim.x;
  const int upb = (nu + nb - 1) / nb;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int u0 = blockIdx.x * upb + wave, u1 = min(nu, (static_cast<int>(blockIdx.x) + 1) * upb);
  const uint8_t* wgu = static_cast<const uint8_t*>(Ld.w_gate_up.data);
  const uint16_t* sgu = static_cast<const uint16_t*>(Ld.w_gate_up.scales);
  int rows[4];
  if (u0 < u1) {
    gate_up_rows(u0, a.F, rows);
    load_frag<4, J>(fa, wgu, sgu, rows, a.H, lane);
  }
  if (u0 + kNW < u1) {
    gate_up_rows(u0 + kNW, a.F, rows);
    load_frag<4, J>(fb, wgu, sgu, rows, a.H, lane);
  }
}

// P1 of layer l: RMSNorm + q|k|v + RoPE + KV write.  False when the launch aborted.
template <int J, int G>
__device__ __forceinline__ bool phase_qkv(int l, uint32_t E0, int64_t pos, int S) {
  const Args& a = kargs();
  [[maybe_unused]] constexpr int HW = J * 2;  // h words (bf16 pairs) per thread: H/2 = 1024 J
  [[maybe_unused]] constexpr int RB = 8 * J;  // down rows per block (H / 256)
  [[maybe_unused]] const Lds sm = carve<J>();
  [[maybe_unused]] uint32_t* hraw = sm.hraw;
  [[maybe_unused]] uint32_t* hmid = sm.hmid;
  [[maybe_unused]] uint32_t* xs = sm.xs;
  [[maybe_unused]] uint32_t* qs = sm.qs;
  [[maybe_unused]] uint32_t* kvcur = sm.kvcur;
  [[maybe_unused]] float* sc = sm.sc;
  [[maybe_unused]] uint32_t* vt = sm.vt;
  [[maybe_unused]] float* mg = sm.mg;
  [[maybe_unused]] float* red = sm.red;
  [[maybe_unused]] int* blk_ok = sm.blk_ok;
  [[maybe_unused]] const int tid = threadIdx.x, lane = tid & 63;
  [[maybe_unused]] const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  [[maybe_unused]] const int blk = blockIdx.x, nb = gridDim.x;
  [[maybe_unused]] const int H = a.H, F = a.F, hq = a.hq, hkv = a.hkv;
  [[maybe_unused]] const int NQKV = (hq + 2 * hkv) * kD;
  [[maybe_unused]] const int ctx = static_cast<int>(pos) + 1;
  [[maybe_unused]] const int U = hkv * S;
  [[maybe_unused]] const float qk_scale = 1.4426950408889634f / sqrtf(static_cast<float>(kD));
  [[maybe_unused]] const Unpack up;
  const am_gfx950_decode_layer& Ld = a.layers[l];
  [[maybe_unused]] const uint8_t* wqkv = static_cast<const uint8_t*>(Ld.w_qkv.data);
  [[maybe_unused]] const uint16_t* sqkv = static_cast<const uint16_t*>(Ld.w_qkv.scales);
  [[maybe_unused]] const uint32_t ep = E0 + static_cast<uint32_t>(l) + 1u;
  [[maybe_unused]] uint64_t* cur = a.ll + (l & 1) * a.ll_par;
  [[maybe_unused]] const uint64_t* prev = a.ll + ((l + 1) & 1) * a.ll_par;
  // ================= P1: RMSNorm + q|k|v + RoPE + KV write =================
  stamp(a, l, 0);
  {
    const int nquad = NQKV / 4;
    const int qpb = (nquad + nb - 1) / nb;  // quads per block
    const int q0 = blk * qpb + wave;
    const int q1 = min(nquad, (blk + 1) * qpb);
    // prefetch: this wave's first quad, gains, cos/sin
    Frag<4, J> f;
    int rows[4] = {0, 0, 0, 0};
    int head = 0, i0 = 0;
    if (q0 < q1) {
      head = q0 / (kD / 4);
      i0 = 2 * (q0 % (kD / 4));
      const int r0 = head * kD + i0;
      rows[0] = r0;
      rows[1] = r0 + 1;
      rows[2] = r0 + kD / 2;
      rows[3] = r0 + kD / 2 + 1;
      load_frag<4, J>(f, wqkv, sqkv, rows, H, lane);
    }
    uint32_t wv[HW];
    const uint32_t* gain = reinterpret_cast<const uint32_t*>(Ld.in_norm);
#pragma unroll
    for (int i = 0; i < HW; ++i) wv[i] = gain[tid + kNT * i];
    const int64_t pc = pos < a.cap ? pos : 0;
    const float cs_c = a.cos_tab[pc * (kD / 2) + i0 + (lane >> 5)];
    const float cs_s = a.sin_tab[pc * (kD / 2) + i0 + (lane >> 5)];
    // h entering the layer
    if (l == 0) {
      const uint32_t* hg = reinterpret_cast<const uint32_t*>(a.h);
#pragma unroll
      for (int i = 0; i < HW; ++i) hraw[tid + kNT * i] = hg[tid + kNT * i];
      lds_sync();
    } else {
      if (!wait_flags(prev, a.o_flag, kFlagH, 0, nb, ep - 1u, a.abort_flag, blk_ok)) return false;
      if (!ll_gather(prev + a.o_h, H / 2, ep - 1u, hraw, a.abort_flag, blk_ok)) return false;
    }
    stamp(a, l, 1);
    rmsnorm_lds<HW>(hraw, xs, wv, H, a.eps, red);
    uint32_t xr[J][16];
    float corr[J];
    lane_x<J>(xs, lane, xr, corr);
    for (int qd = q0; qd < q1; qd += kNW) {
      if (qd != q0) {
        head = qd / (kD / 4);
        i0 = 2 * (qd % (kD / 4));
        const int r0 = head * kD + i0;
        rows[0] = r0;
        rows[1] = r0 + 1;
        rows[2] = r0 + kD / 2;
        rows[3] = r0 + kD / 2 + 1;
        load_frag<4, J>(f, wqkv, sqkv, rows, H, lane);
      }
      float acc4[4];
      dot_frag<4, J>(f, xr, corr, acc4, up);
      // pairs: (r0, r0+64) for dim i0, (r0+1, r0+65) for dim i0+1
      const float accp[2][2] = {{acc4[0], acc4[2]}, {acc4[1], acc4[3]}};
      float a0, a1;
      const int pp = reduce_pairs<2>(accp, lane, a0, a1);
      float o0 = 0.0f, o1 = 0.0f;
      if (pp >= 0) {
        const float y0 = rnd(a0), y1 = rnd(a1);
        if (head < hq + hkv) {
          const float cq = (qd == q0) ? cs_c : a.cos_tab[pc * (kD / 2) + i0 + pp];
          const float sq = (qd == q0) ? cs_s : a.sin_tab[pc * (kD / 2) + i0 + pp];
          rope_rotate(y0, y1, cq, sq, o0, o1);
        } else {
          o0 = y0;
          o1 = y1;
        }
      }
      // lane 0 holds dim i0, lane 32 dim i0 + 1
      const float p0 = __shfl(o0, 32, 64), p1 = __shfl(o1, 32, 64);
      if (lane == 0) {
        const uint32_t wlo = pack_bf16(o0, p0), whi = pack_bf16(o1, p1);
        const int r0 = head * kD + i0;
        ll_st(cur + a.o_qkv + r0 / 2, ep, wlo);
        ll_st(cur + a.o_qkv + (r0 + kD / 2) / 2, ep, whi);
        if (head >= hq && pos < a.cap) {
          const bool isk = head < hq + hkv;
          uint16_t* plane = isk ? static_cast<uint16_t*>(Ld.k_cache) : static_cast<uint16_t*>(Ld.v_cache);
          const int kh = isk ? head - hq : head - hq - hkv;
          uint32_t* dst = reinterpret_cast<uint32_t*>(plane + (static_cast<int64_t>(kh) * a.cap + pos) * kD + i0);
          dst[0] = wlo;
          dst[kD / 4] = whi;
        }
      }
    }
  }
  publish_flag(cur, a.o_flag, kFlagQkv, ep);
  return true;
}

// P2, P2b, P3 of layer l: attention partials, split merge, o projection + residual
// (its weights are prefetched first: they do not depend on attention).
template <int J, int G>
__device__ __forceinline__ bool phase_attn_o(int l, uint32_t E0, int64_t pos, int S, Frag<4, J>& fa, Frag<4, J>& fb) {
  const Args& a = kargs();
  [[maybe_unused]] constexpr int HW = J * 2;  // h words (bf16 pairs) per thread: H/2 = 1024 J
  [[maybe_unused]] constexpr int RB = 8 * J;  // down rows per block (H / 256)
  [[maybe_unused]] const Lds sm = carve<J>();
  [[maybe_unused]] uint32_t* hraw = sm.hraw;
  [[maybe_unused]] uint32_t* hmid = sm.hmid;
  [[maybe_unused]] uint32_t* xs = sm.xs;
  [[maybe_unused]] uint32_t* qs = sm.qs;
  [[maybe_unused]] uint32_t* kvcur = sm.kvcur;
  [[maybe_unused]] float* sc = sm.sc;
  [[maybe_unused]] uint32_t* vt = sm.vt;
  [[maybe_unused]] float* mg = sm.mg;
  [[maybe_unused]] float* red = sm.red;
  [[maybe_unused]] int* blk_ok = sm.blk_ok;
  [[maybe_unused]] const int tid = threadIdx.x, lane = tid & 63;
  [[maybe_unused]] const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  [[maybe_unused]] const int blk = blockIdx.x, nb = gridDim.x;
  [[maybe_unused]] const int H = a.H, F = a.F, hq = a.hq, hkv = a.hkv;
  [[maybe_unused]] const int NQKV = (hq + 2 * hkv) * kD;
  [[maybe_unused]] const int ctx = static_cast<int>(pos) + 1;
  [[maybe_unused]] const int U = hkv * S;
  [[maybe_unused]] const float qk_scale = 1.4426950408889634f / sqrtf(static_cast<float>(kD));
  [[maybe_unused]] const Unpack up;
  const am_gfx950_decode_layer& Ld = a.layers[l];
  [[maybe_unused]] const uint8_t* wqkv = static_cast<const uint8_t*>(Ld.w_qkv.data);
  [[maybe_unused]] const uint16_t* sqkv = static_cast<const uint16_t*>(Ld.w_qkv.scales);
  [[maybe_unused]] const uint32_t ep = E0 + static_cast<uint32_t>(l) + 1u;
  [[maybe_unused]] uint64_t* cur = a.ll + (l & 1) * a.ll_par;
  [[maybe_unused]] const uint64_t* prev = a.ll + ((l + 1) & 1) * a.ll_par;
  // ================= P2: attention partials (units < U) =================
  // o-proj weights of this wave first: they do not depend on attention
  stamp(a, l, 2);
  const int npair_o = H / 2;
  const int opb = (npair_o + nb - 1) / nb;
  const int u_o0 = blk * opb + wave, u_o1 = min(npair_o, (blk + 1) * opb);
  Frag<2, J> fo;
  {
    const int rows[2] = {2 * u_o0, 2 * u_o0 + 1};
    if (u_o0 < u_o1) load_frag<2, J>(fo, static_cast<const uint8_t*>(Ld.w_o.data),
                                     static_cast<const uint16_t*>(Ld.w_o.scales), rows, hq * kD, lane);
  }
  // Blocks with no attention or merge work issue their first gate|up units now (HBM
  // is nearly idle during attention); the others after their own step, so that
  // their exchange polls do not queue behind 32 MB of weight loads.
  const int mb0 = U + hq <= nb ? U : 0;
  const bool is_attn = blk < U, is_merge = blk >= mb0 && blk < mb0 + hq;
  auto attention = [&]() -> bool {
    const int g = blk / S, s = blk % S;
    const int p_begin = static_cast<int>((static_cast<int64_t>(s) * ctx) / S);
    const int p_end = static_cast<int>((static_cast<int64_t>(s + 1) * ctx) / S);
    const int slot = tid >> 3, sl = tid & 7;  // position slot, 16-dim slice
    const uint16_t* kp = static_cast<const uint16_t*>(Ld.k_cache) + static_cast<int64_t>(g) * a.cap * kD;
    const uint16_t* vp = static_cast<const uint16_t*>(Ld.v_cache) + static_cast<int64_t>(g) * a.cap * kD;
    // prefetch pass 0 (past positions come from the cache)
    // K and V slices of this thread's position (16 dims = two 16-byte pieces each)
    u32x4_t k0, k1, v0, v1;
    auto load_kv = [&](const uint16_t* kb, const uint16_t* vb) {
      const u32x4_t* ks = reinterpret_cast<const u32x4_t*>(kb + 16 * sl);
      const u32x4_t* vs = reinterpret_cast<const u32x4_t*>(vb + 16 * sl);
      k0 = ks[0];
      k1 = ks[1];
      v0 = vs[0];
      v1 = vs[1];
    };
    {
      const int p = p_begin + slot;
      const int pl = (p < p_end && p < pos) ? p : 0;
      load_kv(kp + static_cast<int64_t>(pl) * kD, vp + static_cast<int64_t>(pl) * kD);
    }
    // q of the group's heads, current k and v
    if (!wait_flags(cur, a.o_flag, kFlagQkv, 0, nb, ep, a.abort_flag, blk_ok)) return false;
    stamp(a, l, 8);
    {
      uint32_t val[2];
      const int nq = G * 64;
      auto idx = [&](int j) {
        const int i = tid + j * kNT;
        if (i < nq) return (g * G * kD) / 2 + i;
        if (i < nq + 64) return (hq * kD + g * kD) / 2 + (i - nq);
        if (i < nq + 128) return ((hq + hkv) * kD + g * kD) / 2 + (i - nq - 64);
        return -1;
      };
      const bool ok = ll_wait<2>(cur + a.o_qkv, idx, ep, val, a.abort_flag);
      if (!ok) *blk_ok = 0;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int i = tid + j * kNT;
        if (i < nq)
          qs[i] = val[j];
        else if (i < nq + 128)
          kvcur[i - nq] = val[j];
      }
      lds_sync();
      if (!*blk_ok) return false;
    }
    stamp(a, l, 9);
    // output threads: (head ho, dim) pairs, kNT / 128 heads per pass over outputs
    constexpr int KO = (G + 3) / 4;  // outputs (head, dim) per thread
    float o_run[KO];
#pragma unroll
    for (int k = 0; k < KO; ++k) o_run[k] = 0.0f;
    // running max / sum per head (red[hh], red[8 + hh]); red[16 + hh]: this pass's rescale
    if (tid < G) {
      red[tid] = -INFINITY;
      red[8 + tid] = 0.0f;
    }
    lds_sync();
    const int dim = tid & 127;
    for (int pb = p_begin; pb < p_end; pb += 64) {
      const int p = pb + slot;
      const bool valid = p < p_end;
      if (pb != p_begin) {
        const int pl = (valid && p < pos) ? p : 0;
        load_kv(kp + static_cast<int64_t>(pl) * kD, vp + static_cast<int64_t>(pl) * kD);
      }
      if (valid && p == pos)  // the current position: k, v from this token's exchange
        load_kv(reinterpret_cast<const uint16_t*>(kvcur), reinterpret_cast<const uint16_t*>(kvcur + 64));
      const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
          // q slice of head hh (16 dims) straight from LDS: keeping every head's q in
          // registers would crowd out the prefetched gate|up weights
          const u32x4_t* qv = reinterpret_cast<const u32x4_t*>(qs + hh * 64 + 8 * sl);
          const u32x4_t q0 = qv[0], q1 = qv[1];
          const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
          float sdot = 0.0f;
#pragma unroll
          for (int t = 0; t < 8; ++t) sdot = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(qw[t]), as_bf2(kw[t]), sdot, false);
          sdot = sum8(sdot);
          if (sl == 0) sc[hh * 64 + slot] = valid ? sdot * qk_scale : -INFINITY;
        }
      u32x4_t* vdst = reinterpret_cast<u32x4_t*>(vt + slot * 64 + 8 * sl);
      vdst[0] = v0;
      vdst[1] = v1;
      lds_sync();
      // softmax statistics: one wave per head, lane q = slot q; the probabilities
      // replace the scores in LDS (-inf past the unit's positions gives 0)
      if (wave < G) {
        const float sv = sc[wave * 64 + lane];
        const float mp = wave_max(sv);
        const float m_old = red[wave];
        const float mn = fmaxf(m_old, mp);
        const float pq = __builtin_amdgcn_exp2f(sv - mn);
        sc[wave * 64 + lane] = pq;
        const float lp = wave_sum(pq);
        if (lane == 0) {
          const float rs = m_old == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_old - mn);
          red[16 + wave] = rs;
          red[8 + wave] = red[8 + wave] * rs + lp;
          red[wave] = mn;
        }
      }
      lds_sync();
      // P.V: output thread (head ho, dim) over the pass's slots (all 64 hold a finite V
      // row; probabilities past the unit's positions are 0)
      const int nq4 = p_end - pb <= 32 ? 8 : 16;
#pragma unroll
      for (int k = 0; k < KO; ++k) {
        const int ho = (tid >> 7) + 4 * k;  // head within the group
        if (ho < G) {
          const float4* p4 = reinterpret_cast<const float4*>(sc + ho * 64);
          const uint16_t* vcol = reinterpret_cast<const uint16_t*>(vt) + dim;
          float os = 0.0f;
#pragma unroll 8
          for (int q4 = 0; q4 < nq4; ++q4) {
            const float4 pv = p4[q4];
            os = fmaf(pv.x, bf16_bits_to_f32(vcol[(4 * q4) * 128]), os);
            os = fmaf(pv.y, bf16_bits_to_f32(vcol[(4 * q4 + 1) * 128]), os);
            os = fmaf(pv.z, bf16_bits_to_f32(vcol[(4 * q4 + 2) * 128]), os);
            os = fmaf(pv.w, bf16_bits_to_f32(vcol[(4 * q4 + 3) * 128]), os);
          }
          o_run[k] = o_run[k] * red[16 + ho] + os;
        }
      }
      lds_sync();
    }
    // publish (m, l, o[128]) per head of the unit
    uint64_t* part = cur + a.o_part + static_cast<int64_t>(blk) * (G * (kD + 2));
#pragma unroll
    for (int k = 0; k < KO; ++k) {
      const int ho = (tid >> 7) + 4 * k;
      if (ho < G) {
        uint64_t* ph = part + ho * (kD + 2);
        if (dim == 0) {
          ll_st(ph, ep, __float_as_uint(red[ho]));
          ll_st(ph + 1, ep, __float_as_uint(red[8 + ho]));
        }
        ll_st(ph + 2 + dim, ep, __float_as_uint(o_run[k]));
      }
    }
    publish_flag(cur, a.o_flag, kFlagPart, ep);
    stamp(a, l, 10);
    return true;
  };

  // ================= P2b: merge the splits of one q head per block =================
  // merge blocks: the ones after the attention units when there are enough (they have
  // no attention stores queued ahead of their polls), else the first hq
  auto merge = [&]() -> bool {
    const int hqi = blk - mb0;
    const int g = hqi / G, hh = hqi % G;
    const int grp = tid >> 7, dim = tid & 127;
    float M = -INFINITY, Lsum = 0.0f, O = 0.0f;
    if (!wait_flags(cur, a.o_flag, kFlagPart, g * S, S, ep, a.abort_flag, blk_ok)) return false;
    stamp(a, l, 11);
    for (int s0 = grp; s0 < S; s0 += 4 * 8) {
      uint32_t val[24];
      auto idx = [&](int j) {
        const int s = s0 + 4 * (j / 3);
        if (s >= S) return -1;
        const int base = a.o_part + (g * S + s) * (G * (kD + 2)) + hh * (kD + 2);
        return base + (j % 3 == 2 ? 2 + dim : j % 3);
      };
      if (!ll_wait<24>(cur, idx, ep, val, a.abort_flag)) {
        *blk_ok = 0;
        break;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + 4 * j >= S) continue;
        const float ms = __uint_as_float(val[3 * j]), ls = __uint_as_float(val[3 * j + 1]);
        const float os = __uint_as_float(val[3 * j + 2]);
        if (ms == -INFINITY) continue;
        const float mn = fmaxf(M, ms);
        const float c0 = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - mn), c1 = __builtin_amdgcn_exp2f(ms - mn);
        Lsum = Lsum * c0 + ls * c1;
        O = O * c0 + os * c1;
        M = mn;
      }
    }
    stamp(a, l, 12);
    mg[(grp * 3 + 0) * 128 + dim] = M;
    mg[(grp * 3 + 1) * 128 + dim] = Lsum;
    mg[(grp * 3 + 2) * 128 + dim] = O;
    lds_sync();
    if (!*blk_ok) return false;
    float outv = 0.0f;
    if (tid < 128) {
      float Mm = -INFINITY;
      for (int k = 0; k < 4; ++k) Mm = fmaxf(Mm, mg[(k * 3) * 128 + dim]);
      float Ls = 0.0f, Os = 0.0f;
      for (int k = 0; k < 4; ++k) {
        const float mk = mg[(k * 3) * 128 + dim];
        if (mk == -INFINITY) continue;
        const float c = __builtin_amdgcn_exp2f(mk - Mm);
        Ls = fmaf(mg[(k * 3 + 1) * 128 + dim], c, Ls);
        Os = fmaf(mg[(k * 3 + 2) * 128 + dim], c, Os);
      }
      outv = Os / Ls;
    }
    const float nxt = __shfl_down(outv, 1, 64);
    if (tid < 128 && (dim & 1) == 0) ll_st(cur + a.o_att + (hqi * kD + dim) / 2, ep, pack_bf16(outv, nxt));
    publish_flag(cur, a.o_flag, kFlagAtt, ep);
    stamp(a, l, 13);
    return true;
  };

  // The first gate|up units are issued after the block's own attention / merge work
  // (their exchange polls must not queue behind 32 MB of weight loads), at once by
  // the other blocks (HBM is nearly idle during attention).  Disjoint branches keep
  // the prefetched registers out of the attention code's live ranges.
  if (is_merge) {
    if (is_attn && !attention()) return false;
    if (!merge()) return false;
    issue_gate_up<J>(a, Ld, fa, fb);
  } else if (is_attn) {
    if (!attention()) return false;
    issue_gate_up<J>(a, Ld, fa, fb);
  } else {
    issue_gate_up<J>(a, Ld, fa, fb);
  }

  // ================= P3: o projection + residual =================
  {
    if (!wait_flags(cur, a.o_flag, kFlagAtt, mb0, hq, ep, a.abort_flag, blk_ok)) return false;
    stamp(a, l, 14);
    if (!ll_gather(cur + a.o_att, hq * kD / 2, ep, xs, a.abort_flag, blk_ok)) return false;
    stamp(a, l, 3);
    uint32_t xr[J][16];
    float corr[J];
    lane_x<J>(xs, lane, xr, corr);
    for (int u = u_o0; u < u_o1; u += kNW) {
      if (u != u_o0) {
        const int rows[2] = {2 * u, 2 * u + 1};
        load_frag<2, J>(fo, static_cast<const uint8_t*>(Ld.w_o.data), static_cast<const uint16_t*>(Ld.w_o.scales),
                        rows, hq * kD, lane);
      }
      float acc2[2];
      dot_frag<2, J>(fo, xr, corr, acc2, up);
      const float accp[1][2] = {{acc2[0], acc2[1]}};
      float a0, a1;
      const int pp = reduce_pairs<1>(accp, lane, a0, a1);
      if (pp >= 0) {
        const uint32_t hr = hraw[u];
        ll_st(cur + a.o_hm + u, ep, pack_bf16(lo_bf(hr) + rnd(a0), hi_bf(hr) + rnd(a1)));
      }
    }
  }
  publish_flag(cur, a.o_flag, kFlagHm, ep);
  return true;
}

// P4 of layer l: RMSNorm + gate|up + SiLU-Mul.
template <int J, int G>
__device__ __forceinline__ bool phase_ffn(int l, uint32_t E0, int64_t pos, int S, Frag<4, J>& fa, Frag<4, J>& fb) {
  const Args& a = kargs();
  [[maybe_unused]] constexpr int HW = J * 2;  // h words (bf16 pairs) per thread: H/2 = 1024 J
  [[maybe_unused]] constexpr int RB = 8 * J;  // down rows per block (H / 256)
  [[maybe_unused]] const Lds sm = carve<J>();
  [[maybe_unused]] uint32_t* hraw = sm.hraw;
  [[maybe_unused]] uint32_t* hmid = sm.hmid;
  [[maybe_unused]] uint32_t* xs = sm.xs;
  [[maybe_unused]] uint32_t* qs = sm.qs;
  [[maybe_unused]] uint32_t* kvcur = sm.kvcur;
  [[maybe_unused]] float* sc = sm.sc;
  [[maybe_unused]] uint32_t* vt = sm.vt;
  [[maybe_unused]] float* mg = sm.mg;
  [[maybe_unused]] float* red = sm.red;
  [[maybe_unused]] int* blk_ok = sm.blk_ok;
  [[maybe_unused]] const int tid = threadIdx.x, lane = tid & 63;
  [[maybe_unused]] const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  [[maybe_unused]] const int blk = blockIdx.x, nb = gridDim.x;
  [[maybe_unused]] const int H = a.H, F = a.F, hq = a.hq, hkv = a.hkv;
  [[maybe_unused]] const int NQKV = (hq + 2 * hkv) * kD;
  [[maybe_unused]] const int ctx = static_cast<int>(pos) + 1;
  [[maybe_unused]] const int U = hkv * S;
  [[maybe_unused]] const float qk_scale = 1.4426950408889634f / sqrtf(static_cast<float>(kD));
  [[maybe_unused]] const Unpack up;
  const am_gfx950_decode_layer& Ld = a.layers[l];
  [[maybe_unused]] const uint8_t* wqkv = static_cast<const uint8_t*>(Ld.w_qkv.data);
  [[maybe_unused]] const uint16_t* sqkv = static_cast<const uint16_t*>(Ld.w_qkv.scales);
  [[maybe_unused]] const uint32_t ep = E0 + static_cast<uint32_t>(l) + 1u;
  [[maybe_unused]] uint64_t* cur = a.ll + (l & 1) * a.ll_par;
  [[maybe_unused]] const uint64_t* prev = a.ll + ((l + 1) & 1) * a.ll_par;
  // ================= P4: RMSNorm + gate|up + SiLU-Mul =================
  {
    const int nu = F / 2;
    const int upb = (nu + nb - 1) / nb;
    stamp(a, l, 4);
    const int u0 = blk * upb + wave, u1 = min(nu, (blk + 1) * upb);
    const uint8_t* wgu = static_cast<const uint8_t*>(Ld.w_gate_up.data);
    const uint16_t* sgu = static_cast<const uint16_t*>(Ld.w_gate_up.scales);
    auto unit_rows = [&](int u, int (&rows)[4]) { gate_up_rows(u, F, rows); };
    uint32_t wv[HW];
    const uint32_t* gain = reinterpret_cast<const uint32_t*>(Ld.post_norm);
#pragma unroll
    for (int i = 0; i < HW; ++i) wv[i] = gain[tid + kNT * i];
    if (!wait_flags(cur, a.o_flag, kFlagHm, 0, nb, ep, a.abort_flag, blk_ok)) return false;
    if (!ll_gather(cur + a.o_hm, H / 2, ep, hmid, a.abort_flag, blk_ok)) return false;
    stamp(a, l, 5);
    rmsnorm_lds<HW>(hmid, xs, wv, H, a.eps, red);
    uint32_t xr[J][16];
    float corr[J];
    lane_x<J>(xs, lane, xr, corr);
    auto finish = [&](const Frag<4, J>& f, int u) {
      float acc4[4];
      dot_frag<4, J>(f, xr, corr, acc4, up);
      const float accp[2][2] = {{acc4[0], acc4[1]}, {acc4[2], acc4[3]}};
      float a0, a1;
      const int pp = reduce_pairs<2>(accp, lane, a0, a1);
      float v = 0.0f;
      if (pp >= 0) v = silu_ref(rnd(a0)) * rnd(a1);
      const float v1 = __shfl(v, 32, 64);
      if (lane == 0) ll_st(cur + a.o_a + u, ep, pack_bf16(v, v1));
    };
    int u = u0;
    while (u < u1) {
      finish(fa, u);
      if (u + 2 * kNW < u1) {
        int rows[4];
        unit_rows(u + 2 * kNW, rows);
        load_frag<4, J>(fa, wgu, sgu, rows, H, lane);
      }
      u += kNW;
      if (u >= u1) break;
      finish(fb, u);
      if (u + 2 * kNW < u1) {
        int rows[4];
        unit_rows(u + 2 * kNW, rows);
        load_frag<4, J>(fb, wgu, sgu, rows, H, lane);
      }
      u += kNW;
    }
  }
  publish_flag(cur, a.o_flag, kFlagA, ep);
  return true;
}

// P5 of layer l: down projection (split-K) + residual.
template <int J, int G>
__device__ __forceinline__ bool phase_down(int l, uint32_t E0, int64_t pos, int S) {
  const Args& a = kargs();
  [[maybe_unused]] constexpr int HW = J * 2;  // h words (bf16 pairs) per thread: H/2 = 1024 J
  [[maybe_unused]] constexpr int RB = 8 * J;  // down rows per block (H / 256)
  [[maybe_unused]] const Lds sm = carve<J>();
  [[maybe_unused]] uint32_t* hraw = sm.hraw;
  [[maybe_unused]] uint32_t* hmid = sm.hmid;
  [[maybe_unused]] uint32_t* xs = sm.xs;
  [[maybe_unused]] uint32_t* qs = sm.qs;
  [[maybe_unused]] uint32_t* kvcur = sm.kvcur;
  [[maybe_unused]] float* sc = sm.sc;
  [[maybe_unused]] uint32_t* vt = sm.vt;
  [[maybe_unused]] float* mg = sm.mg;
  [[maybe_unused]] float* red = sm.red;
  [[maybe_unused]] int* blk_ok = sm.blk_ok;
  [[maybe_unused]] const int tid = threadIdx.x, lane = tid & 63;
  [[maybe_unused]] const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  [[maybe_unused]] const int blk = blockIdx.x, nb = gridDim.x;
  [[maybe_unused]] const int H = a.H, F = a.F, hq = a.hq, hkv = a.hkv;
  [[maybe_unused]] const int NQKV = (hq + 2 * hkv) * kD;
  [[maybe_unused]] const int ctx = static_cast<int>(pos) + 1;
  [[maybe_unused]] const int U = hkv * S;
  [[maybe_unused]] const float qk_scale = 1.4426950408889634f / sqrtf(static_cast<float>(kD));
  [[maybe_unused]] const Unpack up;
  const am_gfx950_decode_layer& Ld = a.layers[l];
  [[maybe_unused]] const uint8_t* wqkv = static_cast<const uint8_t*>(Ld.w_qkv.data);
  [[maybe_unused]] const uint16_t* sqkv = static_cast<const uint16_t*>(Ld.w_qkv.scales);
  [[maybe_unused]] const uint32_t ep = E0 + static_cast<uint32_t>(l) + 1u;
  [[maybe_unused]] uint64_t* cur = a.ll + (l & 1) * a.ll_par;
  [[maybe_unused]] const uint64_t* prev = a.ll + ((l + 1) & 1) * a.ll_par;
  // ================= P5: down projection (split-K) + residual =================
  {
    stamp(a, l, 6);
    const int CF = F / 32;  // 16-byte chunks per row
    const int rb = F / 2, ng = F / 128;
    const uint8_t* wd = static_cast<const uint8_t*>(Ld.w_down.data);
    const uint16_t* sd = static_cast<const uint16_t*>(Ld.w_down.scales);
    const int row0 = blk * RB;
    const int c = tid < CF ? tid : 0;
    uint4 w[RB];
    uint32_t s[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      w[r] = ld_w(wd + static_cast<uint32_t>((row0 + r) * rb + 16 * c));
      s[r] = sd[static_cast<uint32_t>((row0 + r) * ng + (c >> 2))];
    }
    if (!wait_flags(cur, a.o_flag, kFlagA, 0, nb, ep, a.abort_flag, blk_ok)) return false;
    uint32_t xd[16];
    auto idx = [&](int j) { return tid < CF ? 16 * tid + j : -1; };
    const bool ok = ll_wait<16>(cur + a.o_a, idx, ep, xd, a.abort_flag);
    if (!ok) *blk_ok = 0;
    stamp(a, l, 7);
    float v[RB];
    if (tid < CF) {
      float sx = 0.0f;
#pragma unroll
      for (int t = 0; t < 16; ++t) sx += lo_bf(xd[t]) + hi_bf(xd[t]);
      const float cr = kOff * sx;
#pragma unroll
      for (int r = 0; r < RB; ++r) v[r] = f16_bits_to_f32(s[r]) * int4_chunk_dot_bf16(w[r], xd, -cr, up);
    } else {
#pragma unroll
      for (int r = 0; r < RB; ++r) v[r] = 0.0f;
    }
    int row;
    const float rs = fold_rows<RB>(v, lane, row);
    if ((lane & (64 / RB - 1)) == 0) red[wave * 16 + row] = rs;
    lds_sync();
    if (!*blk_ok) return false;
    if (tid < RB / 2) {
      float d0 = 0.0f, d1 = 0.0f;
      for (int w2 = 0; w2 < kNW; ++w2) {
        d0 += red[w2 * 16 + 2 * tid];
        d1 += red[w2 * 16 + 2 * tid + 1];
      }
      const uint32_t hm = hmid[(row0 >> 1) + tid];
      const uint32_t out = pack_bf16(lo_bf(hm) + rnd(d0), hi_bf(hm) + rnd(d1));
      if (l + 1 < a.L)
        ll_st(cur + a.o_h + (row0 >> 1) + tid, ep, out);
      else
        reinterpret_cast<uint32_t*>(a.h)[(row0 >> 1) + tid] = out;
    }
    if (l + 1 < a.L) publish_flag(cur, a.o_flag, kFlagH, ep);
    lds_sync();
  }
  return true;
}

template <int J, int G>
__global__ __launch_bounds__(kNT) void decode_layers_kernel(Args a) {
  const int tid = threadIdx.x;
  const Lds sm = carve<J>();
  if (tid == 0) *sm.blk_ok = aborted(a.abort_flag) ? 0 : 1;  // one read per block: a uniform exit
  const uint32_t E0 = *a.epoch;
  const int64_t pos = *a.pos;
  lds_sync();
  if (!*sm.blk_ok) return;
  // attention split of this token: units of >= 32 positions, at most grid/hkv per kv head
  const int ctx = static_cast<int>(pos) + 1;
  int S = (ctx + 31) / 32;
  if (S > static_cast<int>(gridDim.x) / a.hkv) S = static_cast<int>(gridDim.x) / a.hkv;
  for (int l = 0; l < a.L; ++l) {
    if (!phase_qkv<J, G>(l, E0, pos, S)) return;
    Frag<4, J> fa, fb;  // first two gate|up units, issued during the attention step
    if (!phase_attn_o<J, G>(l, E0, pos, S, fa, fb)) return;
    if (!phase_ffn<J, G>(l, E0, pos, S, fa, fb)) return;
    if (!phase_down<J, G>(l, E0, pos, S)) return;
  }
  if (blockIdx.x == 0 && tid == 0) *a.epoch = E0 + static_cast<uint32_t>(a.L);
}

// ---- workspace layout (64-bit words after a 256-byte header: epoch, abort) ----
struct WsLayout {
  int64_t o_qkv, o_att, o_hm, o_h, o_a, o_part, o_flag, par;
};
WsLayout Layout(int64_t H, int64_t hq, int64_t hkv, int64_t F) {
  WsLayout w{};
  auto up64 = [](int64_t x) { return (x + 63) / 64 * 64; };
  int64_t o = 0;
  w.o_qkv = o;
  o += up64((hq + 2 * hkv) * kD / 2);
  w.o_att = o;
  o += up64(hq * kD / 2);
  w.o_hm = o;
  o += up64(H / 2);
  w.o_h = o;
  o += up64(H / 2);
  w.o_a = o;
  o += up64(F / 2);
  w.o_part = o;
  o += up64(static_cast<int64_t>(kGrid) * kMaxG * (kD + 2));
  w.o_flag = o;
  o += kFlagKinds * kGrid * kFlagStride;
  w.par = o;
  return w;
}
constexpr int64_t kWsHeader = 256;

template <int J, int G>
am_status_code Launch(const Args& k, hipStream_t s) {
  // > 64 KB of dynamic LDS needs the attribute (set once per device and kernel)
  static int attr_dev = -1;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return SetLastError(AM_STATUS_INTERNAL, "decode_layers: no device");
  if (attr_dev != dev) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_layers_kernel<J, G>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLds) != hipSuccess)
      return SetLastError(AM_STATUS_INTERNAL, "decode_layers: cannot request 96 KB of LDS");
    attr_dev = dev;
  }
  LaunchTiming& lt = ThreadLaunchTiming();
  if (lt.start != nullptr) {
    hipExtLaunchKernelGGL((decode_layers_kernel<J, G>), dim3(kGrid), dim3(kNT), static_cast<size_t>(kLds), s, lt.start,
                          lt.stop, 0, k);
    lt.used = true;
  } else {
    hipLaunchKernelGGL((decode_layers_kernel<J, G>), dim3(kGrid), dim3(kNT), static_cast<size_t>(kLds), s, k);
  }
  AM_RETURN_IF_LAUNCH_FAILED("decode_layers");
  return AM_STATUS_OK;
}

}  // namespace

extern "C" int64_t am_gfx950_decode_layers_workspace_bytes(int64_t hidden, int64_t hq, int64_t hkv, int64_t head_dim,
                                                           int64_t ffn) {
  if (hidden <= 0 || hq <= 0 || hkv <= 0 || head_dim != kD || ffn <= 0) return 0;
  return kWsHeader + 2 * Layout(hidden, hq, hkv, ffn).par * 8;
}

extern "C" am_status_code am_gfx950_decode_layers_validate(const am_gfx950_decode_layers_args* a,
                                                           const am_gfx950_decode_layer* host_layers) {
  AM_CHECK_ARG(a != nullptr, "decode_layers: null args");
  AM_CHECK_ARG(a->dtype == AM_DT_BF16, "decode_layers: bf16 activations only");
  AM_CHECK_ARG(a->head_dim == kD, "decode_layers: head_dim must be 128");
  AM_CHECK_ARG(a->hq > 0 && a->hkv > 0 && a->hq % a->hkv == 0 && (a->hq / a->hkv == 4 || a->hq / a->hkv == 8),
               "decode_layers: q heads must be 4x or 8x the kv heads");
  AM_CHECK_ARG(a->hidden == a->hq * kD, "decode_layers: hidden must equal q heads x head_dim");
  AM_CHECK_ARG(a->hidden == 2048 || a->hidden == 4096, "decode_layers: hidden must be 2048 or 4096");
  AM_CHECK_ARG(a->ffn > 0 && a->ffn % 128 == 0 && a->ffn / 32 <= kNT, "decode_layers: ffn must be a multiple of 128, <= 16384");
  AM_CHECK_ARG(a->num_layers > 0 && a->capacity > 0 && a->capacity < (int64_t{1} << 31), "decode_layers: layers/capacity");
  AM_CHECK_ARG(a->layers && a->cos_tab && a->sin_tab && a->pos && a->h && a->workspace,
               "decode_layers: null pointer argument");
  AM_CHECK_ARG(a->workspace_bytes >= am_gfx950_decode_layers_workspace_bytes(a->hidden, a->hq, a->hkv, a->head_dim, a->ffn),
               "decode_layers: workspace too small");
  AM_CHECK_ARG((reinterpret_cast<uintptr_t>(a->workspace) & 255u) == 0 && (reinterpret_cast<uintptr_t>(a->h) & 15u) == 0,
               "decode_layers: workspace must be 256-byte and h 16-byte aligned");
  if (host_layers != nullptr) {
    const int64_t H = a->hidden, F = a->ffn, QKV = (a->hq + 2 * a->hkv) * kD;
    for (int64_t l = 0; l < a->num_layers; ++l) {
      const am_gfx950_decode_layer& L = host_layers[l];
      const am_gfx950_weight* ws[4] = {&L.w_qkv, &L.w_o, &L.w_gate_up, &L.w_down};
      const int64_t n[4] = {QKV, H, 2 * F, H}, k[4] = {H, a->hq * kD, H, F};
      for (int i = 0; i < 4; ++i) {
        AM_CHECK_ARG(ws[i]->format == AM_WF_INT4 && ws[i]->group_size == 128, "decode_layers: INT4 group-128 weights only");
        AM_CHECK_ARG(ws[i]->n == n[i] && ws[i]->k == k[i], "decode_layers: weight shape mismatch");
        AM_CHECK_ARG(ws[i]->data && ws[i]->scales && (reinterpret_cast<uintptr_t>(ws[i]->data) & 15u) == 0,
                     "decode_layers: weight data/scales");
      }
      AM_CHECK_ARG(L.in_norm && L.post_norm && L.k_cache && L.v_cache, "decode_layers: null layer pointer");
      AM_CHECK_ARG((reinterpret_cast<uintptr_t>(L.in_norm) & 15u) == 0 && (reinterpret_cast<uintptr_t>(L.post_norm) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(L.k_cache) & 15u) == 0 && (reinterpret_cast<uintptr_t>(L.v_cache) & 15u) == 0,
                   "decode_layers: norm gains and cache planes must be 16-byte aligned");
    }
  }
  if (DeviceCUs() != kGrid) return SetLastError(AM_STATUS_UNIMPLEMENTED, "decode_layers: needs a 256-CU device");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_decode_layers(const am_gfx950_decode_layers_args* a, void* stream) {
  const am_status_code st = am_gfx950_decode_layers_validate(a, nullptr);
  if (st != AM_STATUS_OK) return st;
  const WsLayout w = Layout(a->hidden, a->hq, a->hkv, a->ffn);
  Args k{};
  k.layers = a->layers;
  k.L = static_cast<int32_t>(a->num_layers);
  k.H = static_cast<int32_t>(a->hidden);
  k.hq = static_cast<int32_t>(a->hq);
  k.hkv = static_cast<int32_t>(a->hkv);
  k.F = static_cast<int32_t>(a->ffn);
  k.cap = static_cast<int32_t>(a->capacity);
  k.eps = a->eps;
  k.cos_tab = a->cos_tab;
  k.sin_tab = a->sin_tab;
  k.pos = a->pos;
  k.h = static_cast<uint16_t*>(a->h);
  uint8_t* ws = static_cast<uint8_t*>(a->workspace);
  k.epoch = reinterpret_cast<uint32_t*>(ws);
  k.abort_flag = reinterpret_cast<int32_t*>(ws + 64);
  k.ll = reinterpret_cast<uint64_t*>(ws + kWsHeader);
  k.ll_par = w.par;
  k.o_qkv = static_cast<int32_t>(w.o_qkv);
  k.o_att = static_cast<int32_t>(w.o_att);
  k.o_hm = static_cast<int32_t>(w.o_hm);
  k.o_h = static_cast<int32_t>(w.o_h);
  k.o_a = static_cast<int32_t>(w.o_a);
  k.o_part = static_cast<int32_t>(w.o_part);
  k.o_flag = static_cast<int32_t>(w.o_flag);
  k.timeline = static_cast<uint64_t*>(a->timeline);
  const hipStream_t s = AsStream(stream);
  const int64_t G = a->hq / a->hkv;
  if (a->hidden == 4096) return G == 4 ? Launch<2, 4>(k, s) : Launch<2, 8>(k, s);
  return G == 4 ? Launch<1, 4>(k, s) : Launch<1, 8>(k, s);
}

extern "C" am_status_code am_gfx950_decode_layers_aborted(const void* workspace, int32_t* out) {
  AM_CHECK_ARG(workspace != nullptr && out != nullptr, "decode_layers_aborted: null argument");
  if (hipMemcpy(out, static_cast<const uint8_t*>(workspace) + 64, 4, hipMemcpyDeviceToHost) != hipSuccess)
    return SetLastError(AM_STATUS_INTERNAL, "decode_layers_aborted: copy failed");
  return AM_STATUS_OK;
}

}  // namespace am
