// Prefill GEMM on gfx950: out[M,N] = X[M,K] (bf16) @ W[N,K]^T on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16) for INT4 g128, INT8 per-channel and bf16 weights, with the
// prefill plan's fused epilogues.
//
//   * Block tile 128 x 128 (M x N), k step 64, 256 threads = 2 x 2 waves of 64 x 64
//     (4 x 4 MFMA tiles each), or 128 x 256 with 8 waves when that still gives every
//     CU a tile.
//   * Operands move global -> LDS by DMA (global_load_lds_dwordx4): no registers and no
//     LDS store instructions, so two or three k steps are in flight while one is
//     computed.  The ring holds the stages of X (128 rows x 128 B) and W (rows of 32 B
//     INT4, 64 B INT8 or 128 B bf16 per k step), plus for INT4 a four-slot ring of the
//     fp16 group scales.
//   * DMA writes a wave's 64 lanes to 1 KB of consecutive LDS, so the bank layout is
//     set by which global chunk each lane fetches: 16-byte chunk c of X row r (and of a
//     bf16 W row) sits at slot c ^ ((r >> 1) & 7) of the row, chunk c of an INT8 W row n
//     at slot c ^ ((n >> 2) & 3), chunk c of an INT4 W row n at slot c ^ ((n >> 3) & 1).
//     The 16 rows read by one MFMA operand fetch then fall into distinct banks.
//   * The weight stays in its storage format in LDS and becomes the bf16 B operand in
//     registers right before the MFMA.  INT4: one 32-bit read of 8 nibbles, one shift
//     and one AND-OR per bf16 pair (nibble q+8 in the low mantissa bits of bf16 128.0
//     reads 136+q).  INT8: one 64-bit read of 8 bytes q+128, each converted exactly
//     (integers below 256 are exact in bf16).  bf16: one 128-bit read, no conversion.
//   * The offset the stored codes carry (136 * sum(x) for INT4, 128 * sum(x) for INT8)
//     is taken out on the MFMA: the A operand times an all -136 (-128) B operand gives
//     -136 * (row sum) in exactly the accumulator layout of the output tiles.  INT4
//     scales each group's sum by its fp16 scale when the group (two k steps) completes;
//     INT8 scales the whole sum by the row's fp32 scale after the split-K merge.
//     Products are exact and accumulation is fp32.
//   * Rows past the M or N edge read row 0 and are never stored.
//   * The INT4 k loop runs one group per iteration: the group's first MFMAs start from
//     a zero accumulator, so closing a group is one fma per output and no clearing.
//   * Split-K (tiles that would leave CUs idle): split s of a tile owns a contiguous
//     range of whole groups (128 k values for INT8 and bf16).  Each split block stores
//     its fp32 accumulators with device-scope stores, waits for them, and takes a ticket;
//     the last block of the tile reads the other partials back with device-scope loads
//     and sums all of them in split order (the same order whichever block is last, so
//     results do not depend on scheduling), resets the ticket and runs the epilogue.
//   * Epilogues (the op boundaries of the reference graph, model_graph_builder.cpp:
//     133-290) go through LDS: the block writes round(acc) as a bf16 tile, then every
//     thread moves 16-byte row chunks (one load of residual, one store per chunk).
//     Store; residual (out = round(res + round(acc)), Linear then Add); column split
//     (one q|k|v weight, three outputs); SiLU-Mul (tile columns [0, BN/2) are gate
//     features u, [BN/2, BN) the up rows of the same u: act = round(silu(round(gate))
//     * round(up))); q|k|v with RoPE and the KV cache write.  Chunks that cross the N
//     edge or a split column, or outputs whose rows are not 16-byte aligned, take the
//     per-element path.

#include <algorithm>
#include <type_traits>

#include "am_gemv_common.h"
#include "am_launch_timing.h"

namespace am {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

constexpr int QBM = 128, QBK = 64;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
// Split-K partials move as 16-byte buffer loads and stores carrying the sc1 cache
// policy (bit 4 of the builtins' aux operand on gfx950): the device-coherent accesses
// the relaxed agent-scope atomics compile to, four words at a time.  The descriptor's
// last dword is the raw-buffer format word (32-bit data, no swizzle); a wave's region
// is 16 tiles x 64 lanes x 16 bytes.
constexpr int kCpolSc1 = 16;
constexpr int kRawBufferFlags = 0x00020000;
constexpr int kPartWaveBytes = 16 * 64 * 16;
constexpr int XST = QBM * QBK * 2;  // 16 KB of X per stage

// Bytes of one weight row per k step of 64, and the 16-byte chunks they make.
template <int WF> struct WRow;
template <> struct WRow<AM_WF_INT4> { static constexpr int kBytes = 32; };
template <> struct WRow<AM_WF_INT8> { static constexpr int kBytes = 64; };
template <> struct WRow<AM_WF_BF16> { static constexpr int kBytes = 128; };

// Block shapes: NWN waves along N (64 columns each) by 2 along M.
//   NWN = 2: 256 threads, 128 x 128 tile, 3 stages (INT4 62 KB of LDS and INT8 72 KB:
//            two blocks per CU; bf16 96 KB: one)
//   NWN = 4: 512 threads, 128 x 256 tile, 4 stages (3 for bf16; INT4 100 KB, INT8
//            128 KB, bf16 144 KB, one block per CU): half the X bytes per MFMA, which
//            moves most of the traffic.
template <int WF, int NWN>
struct Shape {
  static constexpr bool kI4 = WF == AM_WF_INT4;
  static constexpr int kWaves = 2 * NWN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBN = 64 * NWN;
  static constexpr int kStages = NWN == 2 ? 3 : (WF == AM_WF_BF16 ? 3 : 4);
  static constexpr int kRowB = WRow<WF>::kBytes;   // W row bytes per k step
  static constexpr int kWSt = kBN * kRowB;         // W bytes per stage
  static constexpr int kStg = XST + kWSt;
  static constexpr int kScSlot = kBN * 4;          // INT4: one dword per weight row
  static constexpr int kLds = kStages * kStg + (kI4 ? 4 * kScSlot : 0);
  static constexpr int kXi = 16 / kWaves;          // X DMA instructions per wave per step
  static constexpr int kWi = kWSt / 1024 / kWaves; // W DMA instructions per wave per step
  static constexpr int kLoads = kXi + kWi + (kI4 ? 1 : 0);  // + the INT4 scale dword
  static_assert(kWi >= 1 && kWi * kWaves * 1024 == kWSt, "W stage must be whole DMA instructions per wave");
};

// Slot of 16-byte chunk c of weight row n within the row's k-step bytes.
template <int WF>
__device__ __forceinline__ int wslot(int n, int c) {
  if constexpr (WF == AM_WF_INT4) return c ^ ((n >> 3) & 1);
  else if constexpr (WF == AM_WF_INT8) return c ^ ((n >> 2) & 3);
  else return c ^ ((n & 7) ^ ((n >> 3) & 1));
}

// X row r's 16-byte chunk c sits at slot c ^ xsw(r) of the row: 8 consecutive rows, and
// 16 rows taken as two parity classes, land in distinct LDS banks.
__device__ __forceinline__ int xsw(int r) { return (r & 7) ^ ((r >> 3) & 1); }

enum I4Epi { kI4Store = 0, kI4Residual = 1, kI4Split = 2, kI4SiluMul = 3, kI4QkvRope = 4 };

struct I4Args {
  const uint16_t* x;  // bf16 [M][K]
  const uint8_t* w;   // [N][K]: INT4 device order (K/2 bytes a row), INT8 q+128 bytes, or bf16
  const void* s;      // INT4: fp16 scales [N][K/group]; INT8: fp32 row scales [N]; bf16: unused
  int32_t M, N, K, group;  // group: the INT4 group; 128 (the split-K unit) for INT8 and bf16
  int32_t ffn;  // SiLU-Mul: rows [0, ffn) gate, [ffn, 2 ffn) up
  uint16_t* out0;
  uint16_t* out1;
  uint16_t* out2;
  int32_t c1, c2;             // split: columns [0,c1) -> out0, [c1,c2) -> out1, [c2,N) -> out2
  const uint16_t* residual;   // [M][N] bf16, may alias out0
  int32_t vec;                // 1: 16-byte output chunks (row strides and split columns % 8 == 0, aligned)
  int32_t splits;             // k splits per tile (1: none)
  float* part;                // [tiles][splits][waves][16][64] x 4 fp32 partial accumulators
  unsigned* tickets;          // [tiles], zero between launches
  // q|k|v + RoPE + KV epilogue: columns [0,c1) q -> out0 (rotated), [c1,c2) k (rotated)
  // and [c2,N) v into the cache planes at position *start + row
  const float* cos_tab;       // [cap][hd/2]
  const float* sin_tab;
  const int64_t* start;
  uint16_t* kc;
  uint16_t* vc;
  KvRows kv;
  int32_t hd, cap;
  int32_t* err;               // optional: set when a row's position is outside [0, cap)
};

// 8 bytes q+128 -> 8 exact bf16 values 0..255, in byte order
__device__ __forceinline__ bf16x8_t bytes8(uint2 v) {
  const uint32_t w[2] = {v.x, v.y};
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = w[i >> 1];
    const int sh = 16 * (i & 1);
    const float lo = static_cast<float>((word >> sh) & 0xFFu), hi = static_cast<float>((word >> (sh + 8)) & 0xFFu);
    const bf16x2_t h = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    d[i] = __builtin_bit_cast(uint32_t, h);
  }
  return __builtin_bit_cast(bf16x8_t, make_uint4(d[0], d[1], d[2], d[3]));
}

__device__ __forceinline__ bf16x8_t unpack8(uint32_t word, uint32_t mask, uint32_t magic) {
  uint32_t d[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = ((word >> (4 * i)) & mask) | magic;
  return __builtin_bit_cast(bf16x8_t, make_uint4(d[0], d[1], d[2], d[3]));
}

__device__ __forceinline__ void dma16(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds((const gvoid*)(g), (lvoid*)(l), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds((const gvoid*)(g), (lvoid*)(l), 4, 0, 0);
}

// Weight row of local tile row r.
template <int EPI, int BN>
__device__ __forceinline__ int32_t wrow(const I4Args& p, int32_t tn, int32_t r) {
  if constexpr (EPI == kI4SiluMul) return r < BN / 2 ? tn * (BN / 2) + r : p.ffn + tn * (BN / 2) + (r - BN / 2);
  const int32_t g = tn * BN + r;
  return g < p.N ? g : 0;
}

// Wait until at most AHEAD steps of this wave's DMA are in flight, then a plain
// s_barrier, as one asm statement (no memory access moves across it; a fenced barrier
// would also wait for the younger steps' DMA).
template <int LOADS>
__device__ __forceinline__ void wait_barrier(int ahead) {
  if (ahead >= 2)
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * LOADS) : "memory");
  else if (ahead == 1)
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(LOADS) : "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int WF, int EPI, int NWN>
__global__ __launch_bounds__((Shape<WF, NWN>::kThreads), NWN == 2 ? 2 : 1) void gemm_mfma_kernel(I4Args p) {
  using S = Shape<WF, NWN>;
  constexpr int BN = S::kBN, NST = S::kStages, STG = S::kStg;
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / NWN, wn = wave % NWN;

  // tile mapping: bands of 8 M-tiles, N fastest inside a band
  const int32_t tiles_m = (p.M + QBM - 1) / QBM;
  const int32_t tiles_n = EPI == kI4SiluMul ? p.ffn / (BN / 2) : (p.N + BN - 1) / BN;
  const int32_t tiles = tiles_m * tiles_n;
  const int32_t split = blockIdx.x / tiles;
  const int32_t bid = blockIdx.x - split * tiles;
  const int32_t per_band = 8 * tiles_n;
  const int32_t b0 = bid / per_band, rem = bid - b0 * per_band;
  const int32_t bands_m = min(tiles_m - b0 * 8, 8);
  const int32_t tm = b0 * 8 + rem % bands_m, tn = rem / bands_m;
  const int32_t m0 = tm * QBM;

  const int32_t ng = p.K / p.group;
  const int32_t spg = p.group / QBK;  // k steps per group
  // this split's groups [g0, g1) = k steps [k0, k0 + nk)
  const int32_t g0 = split * ng / p.splits, g1 = (split + 1) * ng / p.splits;
  const int32_t k0 = g0 * spg, nk = (g1 - g0) * spg;

  // ---- DMA sources of this lane ----
  // X: wave w moves rows [8 kXi w, 8 kXi (w + 1)), 8 rows per instruction
  const uint8_t* xsrc[S::kXi];
#pragma unroll
  for (int i = 0; i < S::kXi; ++i) {
    const int r = (wave * S::kXi + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ xsw(r);
    const int32_t gr = m0 + r < p.M ? m0 + r : 0;
    xsrc[i] = reinterpret_cast<const uint8_t*>(p.x) + (static_cast<int64_t>(gr) * p.K + 8 * c) * 2;
  }
  // INT8: the fp32 scales of this lane's four output columns, loaded ahead of every DMA
  float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if constexpr (WF == AM_WF_INT8) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
      rs[nt] = static_cast<const float*>(p.s)[wrow<EPI, BN>(p, tn, wn * 64 + nt * 16 + (lane & 15))];
  }
  // W: instruction i of wave w fills 1 KB of the stage's W rows; lane L's 16 bytes land
  // at row (1024 (w kWi + i) + 16 L) / kRowB, slot ((16 L) mod kRowB) / 16, so it fetches
  // the chunk whose slot that is (the slot map is an XOR, its own inverse)
  const int64_t wrow_bytes = static_cast<int64_t>(p.K) / QBK * S::kRowB;
  const uint8_t* wsrc[S::kWi];
#pragma unroll
  for (int i = 0; i < S::kWi; ++i) {
    const int o = (wave * S::kWi + i) * 1024 + 16 * lane;
    const int r = o / S::kRowB, slot = (o % S::kRowB) / 16;
    wsrc[i] = p.w + static_cast<int64_t>(wrow<EPI, BN>(p, tn, r)) * wrow_bytes + 16 * wslot<WF>(r, slot);
  }
  // INT4 scales: lane -> weight row (wave % NWN) * 64 + lane (waves past NWN repeat the
  // same rows); the dword holding its fp16
  const int sr = (wave % NWN) * 64 + lane;
  const int64_t sbase = S::kI4 ? static_cast<int64_t>(wrow<EPI, BN>(p, tn, sr)) * ng : 0;

  auto issue = [&](int32_t j) {  // local step j = k step k0 + j
    const int32_t ks = k0 + j;
    uint8_t* st = lds + (j % NST) * STG;
#pragma unroll
    for (int i = 0; i < S::kXi; ++i) dma16(xsrc[i] + ks * (QBK * 2), st + (wave * S::kXi + i) * 1024);
#pragma unroll
    for (int i = 0; i < S::kWi; ++i) dma16(wsrc[i] + ks * S::kRowB, st + XST + (wave * S::kWi + i) * 1024);
    if constexpr (S::kI4) {
      const int32_t g = ks / spg;
      const int64_t se = sbase + g;  // fp16 element; its dword, aligned down
      dma4(reinterpret_cast<const uint8_t*>(p.s) + ((se * 2) & ~int64_t{3}),
           lds + NST * STG + (g & 3) * S::kScSlot + (wave % NWN) * 256);
    }
  };

  f32x4_t acc[4][4], part[4][4], corr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    corr[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
  uint32_t mask = 0x000F000Fu, magic = 0x43004300u;
  asm volatile("" : "+v"(mask), "+v"(magic));
  // the code offset times -1 (INT4 -136, INT8 -128) as an all-equal B operand
  constexpr uint32_t kNeg = S::kI4 ? 0xC308C308u : 0xC300C300u;
  constexpr bool kOff = WF != AM_WF_BF16;
  const bf16x8_t bneg = __builtin_bit_cast(bf16x8_t, make_uint4(kNeg, kNeg, kNeg, kNeg));

  // LDS read offsets of this lane (within a stage)
  int aoff[4][2], boff[4][2];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int r = wm * 64 + mt * 16 + (lane & 15);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) aoff[mt][kk] = r * 128 + 16 * ((kk * 4 + (lane >> 4)) ^ xsw(r));
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = wn * 64 + nt * 16 + (lane & 15);
    const int kb = lane >> 4;  // 8-value k block of this lane's B operand
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      if constexpr (WF == AM_WF_INT4)
        boff[nt][kk] = XST + n * 32 + 16 * wslot<WF>(n, kk) + 4 * kb;
      else if constexpr (WF == AM_WF_INT8)
        boff[nt][kk] = XST + n * 64 + 16 * wslot<WF>(n, 2 * kk + (kb >> 1)) + 8 * (kb & 1);
      else
        boff[nt][kk] = XST + n * 128 + 16 * wslot<WF>(n, 4 * kk + kb);
    }
  }
  // scale of this lane's column of tile nt in group g: the half of the slot dword that
  // holds element (row * ng + g)
  int soff[4], shalf_base[4];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int n = wn * 64 + nt * 16 + (lane & 15);
    soff[nt] = NST * STG + n * 4;
    shalf_base[nt] = S::kI4 ? static_cast<int>(static_cast<int64_t>(wrow<EPI, BN>(p, tn, n)) * ng & 1) : 0;
  }

  // prologue: steps 0 .. NST-2 in flight
#pragma unroll
  for (int i = 0; i < NST - 1; ++i)
    if (i < nk) issue(i);

  const f32x4_t zero4 = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // one k step: FIRST starts the group's partial sums from zero
  auto step = [&](int32_t j, auto first_tag) {
    constexpr bool FIRST = decltype(first_tag)::value;
    // this wave's DMA for step j has landed (younger steps may still be in flight);
    // after the barrier every wave's has, and step j-1 is no longer read
    static_assert(NST <= 4, "wait_barrier keeps at most two younger steps in flight");
    wait_barrier<S::kLoads>(min(nk - 1 - j, NST - 2));
    if (j + NST - 1 < nk) issue(j + NST - 1);
    const uint8_t* st = lds + (j % NST) * STG;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      bf16x8_t af[4], bfr[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) af[mt] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(st + aoff[mt][kk]));
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        if constexpr (WF == AM_WF_INT4)
          bfr[nt] = unpack8(*reinterpret_cast<const uint32_t*>(st + boff[nt][kk]), mask, magic);
        else if constexpr (WF == AM_WF_INT8)
          bfr[nt] = bytes8(*reinterpret_cast<const uint2*>(st + boff[nt][kk]));
        else
          bfr[nt] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(st + boff[nt][kk]));
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        if constexpr (kOff)
          corr[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bneg, (FIRST && kk == 0) ? zero4 : corr[mt], 0, 0, 0);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
          part[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], (FIRST && kk == 0) ? zero4 : part[mt][nt],
                                                                 0, 0, 0);
      }
    }
  };
  int32_t j = 0;
  if constexpr (S::kI4) {
    for (int32_t g = g0; g < g1; ++g) {
      step(j++, std::true_type{});
      for (int32_t t = 1; t < spg; ++t) step(j++, std::false_type{});
      // the group closes: scale and fold into acc
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint32_t sw = *reinterpret_cast<const uint32_t*>(lds + soff[nt] + (g & 3) * S::kScSlot);
        const uint32_t bits = ((shalf_base[nt] + g) & 1) ? (sw >> 16) : (sw & 0xFFFFu);
        const float sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(sc, part[mt][nt][r] + corr[mt][r], acc[mt][nt][r]);
      }
    }
  } else {
    // one running sum over the split's k range (the row scale comes after the merge)
    step(j++, std::true_type{});
    while (j < nk) step(j++, std::false_type{});
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][nt][r] = kOff ? part[mt][nt][r] + corr[mt][r] : part[mt][nt][r];
  }

  if (p.splits > 1) {
    // partial of this split: device-scope (sc1) 16-byte buffer stores of the wave's
    // 16 KB region, acknowledged before the ticket
    float* mine = p.part + ((static_cast<int64_t>(bid) * p.splits + split) * S::kWaves + wave) * (16 * 64 * 4);
    const __amdgpu_buffer_rsrc_t rmine = __builtin_amdgcn_make_buffer_rsrc(mine, 0, kPartWaveBytes, kRawBufferFlags);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, acc[i / 4][i % 4]), rmine, (i * 64 + lane) * 16, 0,
                                             kCpolSc1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ unsigned last;
    if (tid == 0)
      last = __hip_atomic_fetch_add(&p.tickets[bid], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             static_cast<unsigned>(p.splits - 1);
    __syncthreads();
    if (!last) return;
    // the tile's sum in split order
    f32x4_t sum[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sum[i] = zero4;
    for (int sp = 0; sp < p.splits; ++sp) {
      if (sp == split) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sum[i] += acc[i / 4][i % 4];
        continue;
      }
      const float* src = p.part + ((static_cast<int64_t>(bid) * p.splits + sp) * S::kWaves + wave) * (16 * 64 * 4);
      const __amdgpu_buffer_rsrc_t rsrc =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), 0, kPartWaveBytes, kRawBufferFlags);
      u32x4_t v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (i * 64 + lane) * 16, 0, kCpolSc1);
#pragma unroll
      for (int i = 0; i < 16; ++i) sum[i] += __builtin_bit_cast(f32x4_t, v[i]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i / 4][i % 4] = sum[i];
    if (tid == 0) __hip_atomic_store(&p.tickets[bid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if constexpr (WF == AM_WF_INT8) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][nt][r] *= rs[nt];
  }
  // ---- epilogue: round(acc) as a bf16 tile in LDS (lane holds D[4*(lane/16)+r][lane%16]
  // of each 16x16 tile), then 16-byte row chunks ----
  constexpr int TS = BN + 8;  // tile row stride in bf16 (16-byte pad)
  uint16_t* T = reinterpret_cast<uint16_t*>(lds);
  __syncthreads();  // every wave is done with the ring
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        T[(wm * 64 + mt * 16 + 4 * (lane >> 4) + r) * TS + wn * 64 + nt * 16 + (lane & 15)] =
            f32_to_bf16_bits(acc[mt][nt][r]);
  __syncthreads();

  if constexpr (EPI == kI4QkvRope) {
    // A thread takes a chunk pair: 8 columns of the first half of a head and the 8
    // columns d/2 later (the RoPE partners), from the rounded tile.  q and k pairs are
    // rotated in fp32 from the bf16 values and rounded once (the RoPE node); k and v
    // go straight to the cache rows of their positions (the KVCacheUpdate node).
    const int32_t d = p.hd, half = d >> 1, hpt = d >> 4;  // chunk pairs per head
    const int64_t start = *p.start;
    constexpr int PPR = BN / 16;  // chunk pairs per tile row (BN is a multiple of d)
    for (int c = tid; c < QBM * PPR; c += S::kThreads) {
      const int row = c / PPR, pr = c % PPR;
      const int32_t gm = m0 + row;
      const int i0 = (pr % hpt) * 8;              // offset of the chunk inside its head
      const int col = (pr / hpt) * d + i0;        // tile column of the first-half chunk
      const int32_t gn = tn * BN + col;
      if (gm >= p.M || gn >= p.N) continue;
      const uint4 a1 = *reinterpret_cast<const uint4*>(T + row * TS + col);
      const uint4 a2 = *reinterpret_cast<const uint4*>(T + row * TS + col + half);
      const int64_t pos = start + gm;
      const bool ok = pos >= 0 && pos < p.cap;
      uint4 o1 = a1, o2 = a2;
      if (gn < p.c2 && ok) {
        const float4* cp = reinterpret_cast<const float4*>(p.cos_tab + pos * half + i0);
        const float4* sp = reinterpret_cast<const float4*>(p.sin_tab + pos * half + i0);
        const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
        const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        const uint32_t w1[4] = {a1.x, a1.y, a1.z, a1.w}, w2[4] = {a2.x, a2.y, a2.z, a2.w};
        uint32_t r1[4], r2[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint32_t y1[2], y2[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const float x1 = bf16_bits_to_f32(hh ? (w1[q] >> 16) : (w1[q] & 0xFFFFu));
            const float x2 = bf16_bits_to_f32(hh ? (w2[q] >> 16) : (w2[q] & 0xFFFFu));
            const float cc = cv[2 * q + hh], sn = sv[2 * q + hh];
            float r1v, r2v;
            rope_rotate(x1, x2, cc, sn, r1v, r2v);
            y1[hh] = f32_to_bf16_bits(r1v);
            y2[hh] = f32_to_bf16_bits(r2v);
          }
          r1[q] = y1[0] | (y1[1] << 16);
          r2[q] = y2[0] | (y2[1] << 16);
        }
        o1 = make_uint4(r1[0], r1[1], r1[2], r1[3]);
        o2 = make_uint4(r2[0], r2[1], r2[2], r2[3]);
      }
      if (!ok && p.err != nullptr) *p.err = 1;
      if (gn < p.c1) {
        uint16_t* dst = p.out0 + static_cast<int64_t>(gm) * p.c1 + gn;
        *reinterpret_cast<uint4*>(dst) = o1;
        *reinterpret_cast<uint4*>(dst + half) = o2;
      } else if (ok) {
        const bool isk = gn < p.c2;
        const int32_t hc = isk ? gn - p.c1 : gn - p.c2;
        const int64_t row = p.kv.WriteRow(0, hc / d, pos);
        if (row >= 0) {
          uint16_t* dst = (isk ? p.kc : p.vc) + row + i0;
          *reinterpret_cast<uint4*>(dst) = o1;
          *reinterpret_cast<uint4*>(dst + half) = o2;
        }
      }
    }
    return;
  }

  if constexpr (EPI == kI4SiluMul) {
    constexpr int CPR = BN / 16;  // 16-byte output chunks per row (BN/2 features)
    constexpr int IT = QBM * CPR / S::kThreads;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + S::kThreads * i, row = c / CPR, cc = c % CPR;
      const int32_t gm = m0 + row;
      if (gm >= p.M) continue;
      const uint16_t* gt = T + row * TS + cc * 8;
      const uint16_t* ut = gt + BN / 2;
      uint16_t* o = p.out0 + static_cast<int64_t>(gm) * p.ffn + tn * (BN / 2) + cc * 8;
      if (p.vec) {
        const uint4 gv = *reinterpret_cast<const uint4*>(gt), uv = *reinterpret_cast<const uint4*>(ut);
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
        uint32_t ow[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ow[q] = f32_to_bf16_bits(silu_ref(bf16_bits_to_f32(gw[q] & 0xFFFFu)) * bf16_bits_to_f32(uw[q] & 0xFFFFu)) |
                  (static_cast<uint32_t>(
                       f32_to_bf16_bits(silu_ref(bf16_bits_to_f32(gw[q] >> 16)) * bf16_bits_to_f32(uw[q] >> 16)))
                   << 16);
        *reinterpret_cast<uint4*>(o) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f32_to_bf16_bits(silu_ref(bf16_bits_to_f32(gt[e])) * bf16_bits_to_f32(ut[e]));
      }
    }
    return;
  }

  constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
  constexpr int IT = QBM * CPR / S::kThreads;
  // residual chunks first, all loads in flight (each thread reads only the chunks it
  // writes, so an aliased residual is read before it is overwritten)
  uint4 rres[EPI == kI4Residual ? IT : 1];
  if constexpr (EPI == kI4Residual) {
    if (p.vec) {
#pragma unroll
      for (int i = 0; i < IT; ++i) {
        const int c = tid + S::kThreads * i, row = c / CPR, cc = c % CPR;
        const int32_t gm = m0 + row, gn = tn * BN + cc * 8;
        const int64_t idx = (gm < p.M && gn + 8 <= p.N) ? static_cast<int64_t>(gm) * p.N + gn : 0;
        rres[i] = *reinterpret_cast<const uint4*>(p.residual + idx);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int c = tid + S::kThreads * i, row = c / CPR, cc = c % CPR;
    const int32_t gm = m0 + row, gn = tn * BN + cc * 8;
    if (gm >= p.M || gn >= p.N) continue;
    const uint16_t* t = T + row * TS + cc * 8;
    // destination of column gn (split: the output whose column range holds it)
    uint16_t* o = p.out0;
    int32_t col = gn, ld = p.N, lim = p.N;  // lim: end of the destination's columns
    if constexpr (EPI == kI4Split) {
      if (gn < p.c1) {
        ld = lim = p.c1;
      } else if (gn < p.c2) {
        o = p.out1;
        col = gn - p.c1;
        ld = p.c2 - p.c1;
        lim = p.c2;
      } else {
        o = p.out2;
        col = gn - p.c2;
        ld = p.N - p.c2;
      }
    }
    uint16_t* dst = o + static_cast<int64_t>(gm) * ld + col;
    if (p.vec && gn + 8 <= lim) {
      const uint4 tv = *reinterpret_cast<const uint4*>(t);
      uint4 ov = tv;
      if constexpr (EPI == kI4Residual) {
        const uint32_t tw[4] = {tv.x, tv.y, tv.z, tv.w}, rw[4] = {rres[i].x, rres[i].y, rres[i].z, rres[i].w};
        uint32_t ow[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ow[q] = f32_to_bf16_bits(bf16_bits_to_f32(rw[q] & 0xFFFFu) + bf16_bits_to_f32(tw[q] & 0xFFFFu)) |
                  (static_cast<uint32_t>(f32_to_bf16_bits(bf16_bits_to_f32(rw[q] >> 16) + bf16_bits_to_f32(tw[q] >> 16)))
                   << 16);
        ov = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
      *reinterpret_cast<uint4*>(dst) = ov;
    } else {
      // per element: the N edge, a chunk that straddles split outputs, unaligned rows
      for (int e = 0; e < 8 && gn + e < p.N; ++e) {
        int32_t ge = gn + e;
        uint16_t* de = p.out0 + static_cast<int64_t>(gm) * p.N + ge;
        if constexpr (EPI == kI4Split) {
          if (ge < p.c1) de = p.out0 + static_cast<int64_t>(gm) * p.c1 + ge;
          else if (ge < p.c2) de = p.out1 + static_cast<int64_t>(gm) * (p.c2 - p.c1) + (ge - p.c1);
          else de = p.out2 + static_cast<int64_t>(gm) * (p.N - p.c2) + (ge - p.c2);
        }
        uint16_t v = t[e];
        if constexpr (EPI == kI4Residual)
          v = f32_to_bf16_bits(bf16_bits_to_f32(p.residual[static_cast<int64_t>(gm) * p.N + ge]) + bf16_bits_to_f32(v));
        *de = v;
      }
    }
  }
}

// Tiles of a launch with NWN waves along N.
template <int EPI, int NWN>
int64_t TilesOf(const I4Args& p) {
  const int64_t tiles_m = CeilDiv(p.M, QBM);
  constexpr int64_t BN = 64 * NWN;
  return tiles_m * (EPI == kI4SiluMul ? p.ffn / (BN / 2) : CeilDiv(p.N, BN));
}

constexpr int64_t kTicketRegion = 4096;               // bytes at the start of the workspace
constexpr int64_t kMaxSplitTiles = kTicketRegion / 4;  // tiles of a launch that may split

// Blocks of a shape that one CU holds at once, by LDS (160 KB per CU): two for the
// 128-wide INT4 and INT8 tiles, one for the bf16 tile and for every 256-wide tile.
constexpr int64_t kLdsPerCu = 160 * 1024;
template <int WF, int NWN>
constexpr int BlocksPerCu() {
  return kLdsPerCu / Shape<WF, NWN>::kLds > 1 ? static_cast<int>(kLdsPerCu / Shape<WF, NWN>::kLds) : 1;
}

// Split-K count: the largest power of two <= 4 that keeps every split at >= 8 groups
// and the launch within one round of resident blocks (bpc per CU).  Measured on the
// 8B 512-row shapes with the 16-byte partial stores: q|k|v 2 splits (INT4 71 -> 58 us,
// INT8 103 -> 64 us; bf16, one block per CU, unsplit), o 4 (INT4 44 -> 39 us, INT8
// 60 -> 43 us; bf16 2), down 4 (bf16 2: 116 -> 109 us), gate/up unsplit (448 tiles
// already fill the CUs; 2 splits 206 -> 232 us).
int SplitsFor(int64_t tiles, int64_t groups, int64_t cus, int bpc) {
  if (tiles > kMaxSplitTiles) return 1;
  int s = 1;
  while (s < 4 && tiles * s * 2 <= bpc * cus && groups / (s * 2) >= 8) s *= 2;
  return s;
}

// Workspace layout: a fixed ticket region (one u32 per tile of a splitting launch),
// then the partials.  The region's size does not depend on the launch's shape, so
// launches of different shapes can share one workspace: no launch's partials land on
// another launch's tickets.
int64_t TicketBytes(int64_t) { return kTicketRegion; }
template <int NWN>
int64_t PartialBytes(int64_t tiles, int splits) {
  return splits > 1 ? tiles * splits * (2 * NWN) * (16 * 64 * 16) : 0;
}

template <int WF, int EPI, int NWN>
am_status_code LaunchMfma(I4Args p, void* ws, int64_t ws_bytes, hipStream_t s) {
  using S = Shape<WF, NWN>;
  static const bool lds_ok =
      hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_mfma_kernel<WF, EPI, NWN>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, S::kLds) == hipSuccess;
  if (!lds_ok) return SetLastError(AM_STATUS_INTERNAL, "gemm_i4: could not set the dynamic LDS size");
  const int64_t tiles = TilesOf<EPI, NWN>(p);
  int splits = ws != nullptr ? SplitsFor(tiles, p.K / p.group, DeviceCUs(), BlocksPerCu<WF, NWN>()) : 1;
  if (splits > 1 && TicketBytes(tiles) + PartialBytes<NWN>(tiles, splits) > ws_bytes) splits = 1;
  p.splits = splits;
  if (splits > 1) {
    p.tickets = static_cast<unsigned*>(ws);
    p.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + TicketBytes(tiles));
  }
  const int64_t blocks = tiles * splits;
  static const char* const names[] = {"store", "residual", "split", "silu_mul", "qkv_rope_kv"};
  const char* fmt = WF == AM_WF_INT4 ? "i4" : WF == AM_WF_INT8 ? "i8" : "bf16";
  RecordLaunch(blocks, S::kThreads, S::kLds, "gemm_%s<%s,bn=%d,splits=%d>", fmt, names[EPI], S::kBN, splits);
  hipLaunchKernelGGL((gemm_mfma_kernel<WF, EPI, NWN>), dim3(static_cast<unsigned>(blocks)), dim3(S::kThreads), S::kLds,
                     s, p);
  AM_RETURN_IF_LAUNCH_FAILED("gemm_i4");
  return AM_STATUS_OK;
}

// Tile width per shape: the 256-wide tile when it still gives every CU a block.
template <int EPI>
bool WideI4(const I4Args& p) {
  const int64_t tiles_m = CeilDiv(p.M, QBM);
  const int64_t cols = EPI == kI4SiluMul ? 2 * static_cast<int64_t>(p.ffn) : p.N;
  return (EPI != kI4SiluMul || p.ffn % 128 == 0) && tiles_m * CeilDiv(cols, 256) >= DeviceCUs();
}

template <int WF, int EPI>
am_status_code LaunchWF(const I4Args& p, void* ws, int64_t ws_bytes, hipStream_t s) {
  return WideI4<EPI>(p) ? LaunchMfma<WF, EPI, 4>(p, ws, ws_bytes, s) : LaunchMfma<WF, EPI, 2>(p, ws, ws_bytes, s);
}

// The weight format picks the kernel (p.group: the INT4 group, 128 otherwise).
template <int EPI>
am_status_code LaunchI4Any(const I4Args& p, int32_t fmt, void* ws, int64_t ws_bytes, hipStream_t s) {
  switch (fmt) {
    case AM_WF_INT4: return LaunchWF<AM_WF_INT4, EPI>(p, ws, ws_bytes, s);
    case AM_WF_INT8: return LaunchWF<AM_WF_INT8, EPI>(p, ws, ws_bytes, s);
    default: return LaunchWF<AM_WF_BF16, EPI>(p, ws, ws_bytes, s);
  }
}

// Split-K unit along k: the INT4 group, 128 values for INT8 and bf16 weights.
int32_t SplitUnit(const am_gfx950_weight& w) { return w.format == AM_WF_INT4 ? w.group_size : 2 * QBK; }

bool Aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

}  // namespace

// bf16 activations with INT4 weights (group % 64 == 0 and K % group == 0), INT8
// per-channel weights (K % 128 == 0) or bf16 weights (K % 128 == 0).
bool GemmI4Eligible(const am_gfx950_weight& w, int64_t m, const void* x) {
  bool fmt = false;
  int64_t row_bytes = 0;
  if (w.format == AM_WF_INT4) {
    fmt = w.scales != nullptr && w.group_size > 0 && w.group_size % QBK == 0 && w.k % w.group_size == 0;
    row_bytes = w.k / 2;
  } else if (w.format == AM_WF_INT8) {
    fmt = w.scales != nullptr && w.k % (2 * QBK) == 0;
    row_bytes = w.k;
  } else if (w.format == AM_WF_BF16) {
    fmt = w.k % (2 * QBK) == 0;
    row_bytes = 2 * w.k;
  }
  return fmt && m > 0 && m * w.k < (int64_t{1} << 31) && w.n * row_bytes < (int64_t{1} << 31) &&
         m * w.n < (int64_t{1} << 31) && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

// Workspace that lets the launch of this shape split K (0: it never splits).  The same
// bound serves every epilogue (the SiLU-Mul tiles are never more numerous) and every
// weight format (the most resident blocks per CU any format has for the tile width).
int64_t GemmI4WorkspaceBytes(int64_t m, int64_t n, int64_t k, int64_t group) {
  if (m <= 0 || n <= 0 || k <= 0 || group <= 0 || k % group != 0) return 0;
  const int64_t cus = DeviceCUs();
  int64_t best = 0;
  for (int nwn : {2, 4}) {
    const int64_t tiles = CeilDiv(m, QBM) * CeilDiv(n, 64 * nwn);
    const int bpc = nwn == 2 ? std::max({BlocksPerCu<AM_WF_INT4, 2>(), BlocksPerCu<AM_WF_INT8, 2>(),
                                         BlocksPerCu<AM_WF_BF16, 2>()})
                             : std::max({BlocksPerCu<AM_WF_INT4, 4>(), BlocksPerCu<AM_WF_INT8, 4>(),
                                         BlocksPerCu<AM_WF_BF16, 4>()});
    const int sp = SplitsFor(tiles, k / group, cus, bpc);
    if (sp > 1)
      best = std::max(best, TicketBytes(tiles) + (nwn == 2 ? PartialBytes<2>(tiles, sp) : PartialBytes<4>(tiles, sp)));
  }
  return best;
}

// q|k|v GEMM with the RoPE and KVCacheUpdate nodes in the epilogue (one sequence).
am_status_code GemmI4QkvRopeKv(const void* x, int64_t m, const am_gfx950_weight& w, const am_gfx950_prefill_rope_kv& r,
                               void* q_out, void* ws, int64_t ws_bytes, hipStream_t s) {
  if (!GemmI4Eligible(w, m, x)) return SetLastError(AM_STATUS_INVALID_ARGUMENT, "gemm: unsupported shape or weight");
  AM_CHECK_ARG(ws == nullptr || (Aligned16(ws) && ws_bytes >= 0), "gemm: workspace must be 16-byte aligned");
  AM_CHECK_ARG(r.head_dim == 64 || r.head_dim == 128, "prefill q|k|v RoPE: head_dim must be 64 or 128");
  AM_CHECK_ARG(r.hq > 0 && r.hkv > 0 && r.hq % r.hkv == 0 && w.n == (r.hq + 2 * r.hkv) * r.head_dim,
               "prefill q|k|v RoPE: the weight rows must be hq + 2 hkv heads");
  AM_CHECK_ARG(r.capacity > 0 && r.max_pos >= r.capacity && r.capacity * r.head_dim < (int64_t{1} << 31),
               "prefill q|k|v RoPE: bad capacity or table length");
  AM_CHECK_ARG(q_out && r.cos_tab && r.sin_tab && r.start_pos_dev && r.k_cache && r.v_cache,
               "prefill q|k|v RoPE: null pointer");
  AM_CHECK_ARG(Aligned16(q_out) && Aligned16(r.k_cache) && Aligned16(r.v_cache) && Aligned16(r.cos_tab) &&
                   Aligned16(r.sin_tab),
               "prefill q|k|v RoPE: q, the cache planes and the tables must be 16-byte aligned");
  I4Args p{};
  p.x = static_cast<const uint16_t*>(x);
  p.w = static_cast<const uint8_t*>(w.data);
  p.s = w.scales;
  p.M = static_cast<int32_t>(m);
  p.N = static_cast<int32_t>(w.n);
  p.K = static_cast<int32_t>(w.k);
  p.group = SplitUnit(w);
  p.out0 = static_cast<uint16_t*>(q_out);
  p.c1 = static_cast<int32_t>(r.hq * r.head_dim);
  p.c2 = static_cast<int32_t>((r.hq + r.hkv) * r.head_dim);
  p.vec = 1;
  p.splits = 1;
  p.cos_tab = r.cos_tab;
  p.sin_tab = r.sin_tab;
  p.start = r.start_pos_dev;
  p.kc = static_cast<uint16_t*>(r.k_cache);
  p.vc = static_cast<uint16_t*>(r.v_cache);
  p.hd = static_cast<int32_t>(r.head_dim);
  p.cap = static_cast<int32_t>(r.capacity);
  p.err = r.err_flag;
  if (auto st = MakeKvRows(r.pages, 0, r.capacity, r.hkv, r.head_dim, &p.kv); st != AM_STATUS_OK) return st;
  if (p.kv.err == nullptr) p.kv.err = r.err_flag;
  return LaunchI4Any<kI4QkvRope>(p, w.format, ws, ws_bytes, s);
}

am_status_code GemmI4(const void* x, int64_t m, const am_gfx950_weight& w, int32_t epi, void* out0, void* out1,
                      void* out2, int64_t c1, int64_t c2, const void* residual, void* ws, int64_t ws_bytes,
                      hipStream_t s) {
  if (!GemmI4Eligible(w, m, x)) return SetLastError(AM_STATUS_INVALID_ARGUMENT, "gemm: unsupported shape or weight");
  AM_CHECK_ARG(ws == nullptr || (Aligned16(ws) && ws_bytes >= 0), "gemm: workspace must be 16-byte aligned");
  I4Args p{};
  p.x = static_cast<const uint16_t*>(x);
  p.w = static_cast<const uint8_t*>(w.data);
  p.s = w.scales;
  p.M = static_cast<int32_t>(m);
  p.N = static_cast<int32_t>(w.n);
  p.K = static_cast<int32_t>(w.k);
  p.group = SplitUnit(w);
  p.out0 = static_cast<uint16_t*>(out0);
  p.out1 = static_cast<uint16_t*>(out1);
  p.out2 = static_cast<uint16_t*>(out2);
  p.c1 = static_cast<int32_t>(c1);
  p.c2 = static_cast<int32_t>(c2);
  p.residual = static_cast<const uint16_t*>(residual);
  p.splits = 1;
  // 16-byte chunks need every output row (and the residual's) to start 16-byte aligned
  bool vec = Aligned16(out0) && (!residual || Aligned16(residual));
  switch (epi) {
    case kI4Store: vec = vec && w.n % 8 == 0; break;
    case kI4Residual: vec = vec && w.n % 8 == 0; break;
    case kI4Split:
      vec = vec && c1 % 8 == 0 && c2 % 8 == 0 && w.n % 8 == 0 && (c2 == c1 || Aligned16(out1)) &&
            (c2 == w.n || Aligned16(out2));
      break;
    default: vec = vec && (w.n / 2) % 8 == 0; break;
  }
  p.vec = vec ? 1 : 0;
  switch (epi) {
    case kI4Store: return LaunchI4Any<kI4Store>(p, w.format, ws, ws_bytes, s);
    case kI4Residual:
      AM_CHECK_ARG(residual != nullptr, "gemm: residual epilogue without a residual");
      return LaunchI4Any<kI4Residual>(p, w.format, ws, ws_bytes, s);
    case kI4Split:
      AM_CHECK_ARG(0 < c1 && c1 <= c2 && c2 <= w.n && out0 && (c2 == c1 || out1) && (c2 == w.n || out2),
                   "gemm: bad column split");
      return LaunchI4Any<kI4Split>(p, w.format, ws, ws_bytes, s);
    case kI4SiluMul:
      AM_CHECK_ARG(w.n % 128 == 0, "gemm: SiLU-Mul needs 2*ffn rows with ffn a multiple of 64");
      p.ffn = static_cast<int32_t>(w.n / 2);
      return LaunchI4Any<kI4SiluMul>(p, w.format, ws, ws_bytes, s);
    default: return SetLastError(AM_STATUS_INVALID_ARGUMENT, "gemm: unknown epilogue");
  }
}

}  // namespace am
