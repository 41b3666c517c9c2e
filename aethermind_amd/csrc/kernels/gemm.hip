// Prefill GEMM for gfx950: out[M,N] = X[M,K] (bf16) @ W[N,K]^T on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16), with the weight tile dequantised into LDS.
//
//   * Block tile 128 x 128 (M x N), K step 128; 4 waves in a 2x2 arrangement, each
//     owning a 64 x 64 sub-tile = 4 x 4 MFMA tiles of 16 x 16 (64 fp32 accumulators
//     per lane).
//   * X tile and W tile are staged in LDS as bf16 rows padded by 16 bytes, so the
//     16 rows read by one MFMA operand fetch fall into distinct banks.  The tiles are
//     double-buffered: step k+1 is fetched into registers while step k runs on MFMA.
//   * Quantized weights are written to LDS as exact bf16 integers, never as q*s.
//     INT8 stores q and scales the sum by the per-row scale in the epilogue.  INT4
//     stores 136+q, which is one AND-OR per pair of nibbles: nibble n = q+8 placed in
//     the low mantissa bits of bf16 128.0 (0x4300) reads 128+n.  The 136*sum(x) this
//     adds is removed by starting each group's MFMA sum at -136*sum(x) (the row sums
//     are taken with v_dot2_f32_bf16 at staging), and the group sum is scaled by the
//     fp16 group scale when the group completes.  Products are exact and accumulation
//     is fp32.
//   * Rows past the M or N edge are loaded from row 0 and left in the tile: an MFMA
//     output element depends only on its own X row and W row, and the epilogue
//     stores no element outside the matrix.
//   * Block index -> tile mapping walks N fastest inside a band of 8 M-tiles, which
//     keeps each XCD's L2 working on neighbouring weight columns.

#include "am_kernel_common.h"
#include "am_launch_timing.h"

namespace am {
am_status_code GemvLinearRow(const void* x, int32_t act, const am_gfx950_weight& w, void* out, int32_t out_dtype,
                             const void* residual, hipStream_t s);
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int KPT = BK / 2;  // k values each staging thread moves per step (two threads per tile row)
constexpr int LDSROW = BK + 8;  // bf16 elements per padded LDS row

struct GemmArgs {
  const uint16_t* x;  // bf16 [M][K]
  const uint8_t* w;
  const void* scales;
  int64_t M, N, K;
  int32_t group;
  void* out;
  int32_t out_dtype;
  const void* residual;
};

__device__ __forceinline__ uint32_t pack_bf16_int(float lo, float hi) {
  // lo/hi are small integers: their bf16 encoding is the fp32 bits >> 16 exactly.
  return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
__device__ __forceinline__ bf16x2_t as_bf2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// Global -> register stage of one k step: the thread's X row half (KPT bf16) and W
// row half (KPT values in the weight's storage format).
template <int WF>
struct Stage {
  uint4 x[KPT / 8];
  uint4 w[WF == AM_WF_BF16 ? KPT / 8 : (WF == AM_WF_INT8 ? KPT / 16 : KPT / 32)];
};

template <int WF>
__device__ __forceinline__ void stage_load(Stage<WF>& st, const GemmArgs& p, int64_t m0, int64_t n0, int64_t k0,
                                           int lrow, int lhalf) {
  const int64_t gm = m0 + lrow, gn = n0 + lrow;
  // rows past the edge read row 0: in bounds, and their outputs are never stored
  const int64_t rm = gm < p.M ? gm : 0, rn = gn < p.N ? gn : 0;
  const uint4* xs = reinterpret_cast<const uint4*>(p.x + rm * p.K + k0 + KPT * lhalf);
#pragma unroll
  for (int i = 0; i < KPT / 8; ++i) st.x[i] = xs[i];
  constexpr int NW4 = sizeof(st.w) / sizeof(uint4);
  const uint4* ws;
  if constexpr (WF == AM_WF_BF16)
    ws = reinterpret_cast<const uint4*>(p.w + (rn * p.K + k0 + KPT * lhalf) * 2);
  else if constexpr (WF == AM_WF_INT8)
    ws = reinterpret_cast<const uint4*>(p.w + rn * p.K + k0 + KPT * lhalf);
  else
    ws = reinterpret_cast<const uint4*>(p.w + rn * (p.K / 2) + (k0 + KPT * lhalf) / 2);
#pragma unroll
  for (int i = 0; i < NW4; ++i) st.w[i] = ws[i];
}

// Stage -> LDS.  INT8 weights become bf16 q, INT4 weights bf16 136+q, and for INT4
// the tile row's sum of x over the step goes to xsum[row].
template <int WF>
__device__ __forceinline__ void stage_store(const Stage<WF>& st, uint16_t* As, uint16_t* Bs, float* xsum, int lrow,
                                            int lhalf) {
  uint4* dx = reinterpret_cast<uint4*>(As + lrow * LDSROW + KPT * lhalf);
#pragma unroll
  for (int i = 0; i < KPT / 8; ++i) dx[i] = st.x[i];
  uint4 o[KPT / 8];  // KPT bf16 values
  if constexpr (WF == AM_WF_BF16) {
#pragma unroll
    for (int i = 0; i < KPT / 8; ++i) o[i] = st.w[i];
  } else if constexpr (WF == AM_WF_INT8) {
#pragma unroll
    for (int c = 0; c < KPT / 16; ++c) {  // 16 bytes -> 16 bf16
      const uint32_t ws[4] = {st.w[c].x, st.w[c].y, st.w[c].z, st.w[c].w};
      uint32_t outw[8];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float q0 = static_cast<float>(ws[t] & 0xFFu) - 128.0f;
        const float q1 = static_cast<float>((ws[t] >> 8) & 0xFFu) - 128.0f;
        const float q2 = static_cast<float>((ws[t] >> 16) & 0xFFu) - 128.0f;
        const float q3 = static_cast<float>(ws[t] >> 24) - 128.0f;
        outw[2 * t] = pack_bf16_int(q0, q1);
        outw[2 * t + 1] = pack_bf16_int(q2, q3);
      }
      o[2 * c] = make_uint4(outw[0], outw[1], outw[2], outw[3]);
      o[2 * c + 1] = make_uint4(outw[4], outw[5], outw[6], outw[7]);
    }
  } else {  // INT4: 16 bytes = 32 nibbles; word t holds k 8t + {0,2,4,6,1,3,5,7}
    uint32_t mask = 0x000F000Fu, magic = 0x43004300u;  // kept in VGPRs: VOP3 takes no literal
    asm volatile("" : "+v"(mask), "+v"(magic));
#pragma unroll
    for (int c = 0; c < KPT / 32; ++c) {
      const uint32_t ws[4] = {st.w[c].x, st.w[c].y, st.w[c].z, st.w[c].w};
      uint32_t outw[16];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) outw[4 * t + pp] = ((ws[t] >> (4 * pp)) & mask) | magic;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[4 * c + i] = make_uint4(outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]);
    }
    uint32_t ones = 0x3F803F80u;  // bf16 pair (1, 1)
    asm volatile("" : "+v"(ones));
    float sx[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KPT / 8; ++i) {
      const uint32_t xw[4] = {st.x[i].x, st.x[i].y, st.x[i].z, st.x[i].w};
#pragma unroll
      for (int t = 0; t < 4; ++t) sx[t] = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(xw[t]), as_bf2(ones), sx[t], false);
    }
    float h = (sx[0] + sx[1]) + (sx[2] + sx[3]);
    // the row's other half sits in the neighbouring lane (quad_perm [1,0,3,2])
    h += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, h), 0xB1, 0xF, 0xF, false));
    if (lhalf == 0) xsum[lrow] = h;
  }
  uint4* dw = reinterpret_cast<uint4*>(Bs + lrow * LDSROW + KPT * lhalf);
#pragma unroll
  for (int i = 0; i < KPT / 8; ++i) dw[i] = o[i];
}

// double-buffered X and W tiles, then the double-buffered per-row x sums (INT4)
constexpr size_t kGemmTiles = 2 * (BM + BN) * LDSROW * sizeof(uint16_t);
constexpr size_t kGemmLds = kGemmTiles + 2 * BM * sizeof(float);

// G1: INT4 with group == BK, so every k step closes a group.
template <int WF, bool G1>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  extern __shared__ __align__(16) uint16_t gsm[];
  uint16_t* const As0 = gsm;
  uint16_t* const Bs0 = gsm + 2 * BM * LDSROW;
  float* const Xs0 = reinterpret_cast<float*>(gsm + 2 * (BM + BN) * LDSROW);
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // tile mapping (grouped by 8 along M)
  const int64_t tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
  const int64_t bid = blockIdx.x;
  const int64_t band = 8;
  const int64_t per_band = band * tiles_n;
  const int64_t b0 = bid / per_band;
  const int64_t rem = bid % per_band;
  const int64_t bands_m = (tiles_m - b0 * band) < band ? (tiles_m - b0 * band) : band;
  const int64_t tm = b0 * band + rem % bands_m;
  const int64_t tn = rem / bands_m;
  const int64_t m0 = tm * BM, n0 = tn * BN;

  constexpr bool Q4 = WF == AM_WF_INT4;
  f32x4_t acc[4][4];
  f32x4_t part[4][4];  // INT4: the current group's sum of x * (136 + q)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

  const int lrow = tid >> 1;   // 0..127: tile row this thread stages
  const int lhalf = tid & 1;   // which half of the k step
  const int64_t ng = Q4 ? p.K / p.group : 1;
  const int64_t nk = p.K / BK;
  // INT4 scale row of each of the lane's 4 output columns (columns past N read row 0)
  const uint16_t* scp[4] = {};
  if constexpr (Q4) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      const int64_t gn = n0 + wn * 64 + nt * 16 + (lane & 15);
      scp[nt] = static_cast<const uint16_t*>(p.scales) + (gn < p.N ? gn : 0) * ng;
    }
  }

  // Software pipeline: step k+1 is loaded into registers while step k runs on MFMA
  // from one LDS buffer; the registers then go to the other buffer.  One barrier per
  // step.
  Stage<WF> st;
  stage_load<WF>(st, p, m0, n0, 0, lrow, lhalf);
  stage_store<WF>(st, As0, Bs0, Xs0, lrow, lhalf);
  __syncthreads();
  for (int64_t ks = 0; ks < nk; ++ks) {
    const int cur = static_cast<int>(ks & 1);
    const uint16_t* As = As0 + cur * BM * LDSROW;
    const uint16_t* Bs = Bs0 + cur * BN * LDSROW;
    const int64_t k0 = ks * BK;
    const bool closes = !Q4 || G1 || (k0 + BK) % p.group == 0;
    _Float16 sh[4];
    if constexpr (Q4) {
      if (closes) {
        const int64_t g = G1 ? ks : (k0 + BK) / p.group - 1;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) sh[nt] = __builtin_bit_cast(_Float16, scp[nt][g]);
      }
    }
    const bool more = ks + 1 < nk;
    if (more) stage_load<WF>(st, p, m0, n0, k0 + BK, lrow, lhalf);
    // INT4: -136 * (row sums of x over this step), the start value of the step's sums
    f32x4_t c[4];
    if constexpr (Q4) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(Xs0 + cur * BM + wm * 64 + mt * 16 + 4 * (lane >> 4));
        c[mt] = v * -136.0f;
      }
      if constexpr (!G1) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
          for (int nt = 0; nt < 4; ++nt) part[mt][nt] += c[mt];
      }
    }
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      bf16x8_t af[4], bfr[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const uint4 v = *reinterpret_cast<const uint4*>(As + (wm * 64 + mt * 16 + (lane & 15)) * LDSROW +
                                                        kk * 32 + 8 * (lane >> 4));
        af[mt] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint4 v = *reinterpret_cast<const uint4*>(Bs + (wn * 64 + nt * 16 + (lane & 15)) * LDSROW +
                                                        kk * 32 + 8 * (lane >> 4));
        bfr[nt] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          if constexpr (Q4 && G1)
            part[mt][nt] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], kk == 0 ? c[mt] : part[mt][nt], 0, 0, 0);
          else if constexpr (Q4)
            part[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], part[mt][nt], 0, 0, 0);
          else
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], acc[mt][nt], 0, 0, 0);
        }
    }
    if (more)
      stage_store<WF>(st, As0 + (cur ^ 1) * BM * LDSROW, Bs0 + (cur ^ 1) * BN * LDSROW, Xs0 + (cur ^ 1) * BM, lrow,
                      lhalf);

    if constexpr (Q4) {
      if (closes) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const float sc = static_cast<float>(sh[nt]);
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(sc, part[mt][nt][r], acc[mt][nt][r]);
            if constexpr (!G1) part[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds D[4*(lane/16)+r][lane%16] of each 16x16 tile ----
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int64_t gn = n0 + wn * 64 + nt * 16 + (lane & 15);
    if (gn >= p.N) continue;
    float rs = 1.0f;
    if constexpr (WF == AM_WF_INT8) rs = static_cast<const float*>(p.scales)[gn];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t gm = m0 + wm * 64 + mt * 16 + 4 * (lane >> 4) + r;
        if (gm >= p.M) continue;
        float v = acc[mt][nt][r] * rs;
        const int64_t idx = gm * p.N + gn;
        if (p.out_dtype == AM_DT_F32) {
          float* o = static_cast<float*>(p.out);
          if (p.residual != nullptr) v = static_cast<const float*>(p.residual)[idx] + v;
          o[idx] = v;
        } else {
          uint16_t* o = static_cast<uint16_t*>(p.out);
          if (p.residual != nullptr)
            v = bf16_bits_to_f32(static_cast<const uint16_t*>(p.residual)[idx]) +
                bf16_bits_to_f32(f32_to_bf16_bits(v));
          o[idx] = f32_to_bf16_bits(v);
        }
      }
  }
}

}  // namespace
}  // namespace am

using namespace am;

namespace {
am_status_code ValidateLinearWeight(const am_gfx950_weight& w) {
  AM_CHECK_ARG(w.data != nullptr && w.n > 0 && w.k > 0, "linear: null weight or empty shape");
  AM_CHECK_ARG(w.format >= AM_WF_F32 && w.format <= AM_WF_INT4, "linear: unknown weight format");
  return AM_STATUS_OK;
}
}  // namespace

extern "C" int64_t am_gfx950_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int64_t group_size) {
  return GemmI4WorkspaceBytes(m, n, k, group_size);
}

extern "C" am_status_code am_gfx950_prefill_linear(const am_gfx950_prefill_linear_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "prefill_linear: null args");
  if (auto st = ValidateLinearWeight(a->w); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->m > 0 && a->x != nullptr && a->out[0] != nullptr, "prefill_linear: bad rows or pointers");
  if (!GemmI4Eligible(a->w, a->m, a->x))
    return SetLastError(AM_STATUS_UNIMPLEMENTED,
                        "prefill_linear: needs INT4 (group a multiple of 64), INT8 or bf16 weights (k a multiple of "
                        "128) and bf16 rows 16-byte aligned");
  switch (a->epilogue) {
    case AM_PREFILL_SPLIT:
      return GemmI4(a->x, a->m, a->w, 2, a->out[0], a->out[1], a->out[2], a->split[0], a->split[1], nullptr,
                    a->workspace, a->workspace_bytes, AsStream(stream));
    case AM_PREFILL_SILU_MUL:
      return GemmI4(a->x, a->m, a->w, 3, a->out[0], nullptr, nullptr, 0, 0, nullptr, a->workspace, a->workspace_bytes,
                    AsStream(stream));
    case AM_PREFILL_QKV_ROPE_KV:
      AM_CHECK_ARG(a->rope_kv != nullptr, "prefill_linear: the q|k|v RoPE epilogue needs rope_kv");
      return GemmI4QkvRopeKv(a->x, a->m, a->w, *a->rope_kv, a->out[0], a->workspace, a->workspace_bytes,
                             AsStream(stream));
    default: return SetLastError(AM_STATUS_INVALID_ARGUMENT, "prefill_linear: unknown epilogue");
  }
}

extern "C" am_status_code am_gfx950_linear(const am_gfx950_linear_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr, "linear: null args");
  if (auto st = ValidateLinearWeight(a->w); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->x_dtype == AM_DT_F32 || a->x_dtype == AM_DT_BF16, "linear: x dtype must be f32 or bf16");
  AM_CHECK_ARG(a->out_dtype == a->x_dtype || a->out_dtype == AM_DT_F32, "linear: out dtype must be x dtype or f32");
  AM_CHECK_ARG(a->m >= 0, "linear: negative rows");
  if (a->m == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->x && a->out, "linear: null pointer");
  hipStream_t s = AsStream(stream);
  const am_gfx950_weight& w = a->w;
  const bool gemm_ok = a->x_dtype == AM_DT_BF16 && w.format != AM_WF_F32 && w.k % BK == 0 &&
                       (w.format != AM_WF_INT4 || (w.group_size % BK == 0 && w.k % w.group_size == 0)) &&
                       (reinterpret_cast<uintptr_t>(a->x) & 15u) == 0;
  if (a->mode == 3 || (a->mode == 0 && a->m >= 2 && BatchLinearEligible(a->x_dtype, w, a->m, a->x)))
    return BatchLinear(a->x, a->m, w, a->out, a->out_dtype, a->residual, s);
  const bool use_gemm = a->mode == 2 || (a->mode == 0 && a->m > 8 && gemm_ok);
  if (use_gemm && a->out_dtype == AM_DT_BF16 && GemmI4Eligible(w, a->m, a->x))
    return GemmI4(a->x, a->m, w, a->residual != nullptr ? 1 : 0, a->out, nullptr, nullptr, 0, 0, a->residual,
                  a->workspace, a->workspace_bytes, s);
  if (use_gemm) {
    AM_CHECK_ARG(gemm_ok, "linear: MFMA GEMM needs bf16 activations, bf16/int8/int4 weights, K % 128 == 0");
    if (w.format >= AM_WF_INT8) AM_CHECK_ARG(w.scales != nullptr, "linear: quantized weight needs scales");
    GemmArgs g{};
    g.x = static_cast<const uint16_t*>(a->x);
    g.w = static_cast<const uint8_t*>(w.data);
    g.scales = w.scales;
    g.M = a->m;
    g.N = w.n;
    g.K = w.k;
    g.group = w.group_size;
    g.out = a->out;
    g.out_dtype = a->out_dtype;
    g.residual = a->residual;
    const int64_t tiles = CeilDiv(a->m, BM) * CeilDiv(w.n, BN);
    AM_CHECK_ARG(tiles <= 0x7FFFFFFF, "linear: too many tiles");
    const dim3 grid(static_cast<unsigned>(tiles));
    // the double-buffered tiles exceed the 64 KiB default dynamic LDS limit
    static const bool lds_ok = [] {
      const void* fns[] = {reinterpret_cast<const void*>(gemm_kernel<AM_WF_BF16, false>),
                           reinterpret_cast<const void*>(gemm_kernel<AM_WF_INT8, false>),
                           reinterpret_cast<const void*>(gemm_kernel<AM_WF_INT4, true>),
                           reinterpret_cast<const void*>(gemm_kernel<AM_WF_INT4, false>)};
      for (const void* f : fns)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kGemmLds)) !=
            hipSuccess)
          return false;
      return true;
    }();
    if (!lds_ok) return SetLastError(AM_STATUS_INTERNAL, "gemm: could not raise the dynamic LDS limit");
    RecordLaunch(tiles, 256, static_cast<int32_t>(kGemmLds), "gemm<%s,%dx%dx%d>",
                 w.format == AM_WF_BF16 ? "bf16" : w.format == AM_WF_INT8 ? "int8" : "int4", static_cast<int>(BM),
                 static_cast<int>(BN), static_cast<int>(BK));
    switch (w.format) {
      case AM_WF_BF16: hipLaunchKernelGGL((gemm_kernel<AM_WF_BF16, false>), grid, dim3(256), kGemmLds, s, g); break;
      case AM_WF_INT8: hipLaunchKernelGGL((gemm_kernel<AM_WF_INT8, false>), grid, dim3(256), kGemmLds, s, g); break;
      default:
        if (w.group_size == BK)
          hipLaunchKernelGGL((gemm_kernel<AM_WF_INT4, true>), grid, dim3(256), kGemmLds, s, g);
        else
          hipLaunchKernelGGL((gemm_kernel<AM_WF_INT4, false>), grid, dim3(256), kGemmLds, s, g);
        break;
    }
    AM_RETURN_IF_LAUNCH_FAILED("gemm");
    return AM_STATUS_OK;
  }
  // GEMV per row (decode, fp32 activations, or shapes the GEMM does not tile).
  const int64_t esz = a->x_dtype == AM_DT_F32 ? 4 : 2;
  const int64_t osz = a->out_dtype == AM_DT_F32 ? 4 : 2;
  for (int64_t r = 0; r < a->m; ++r) {
    const void* xr = static_cast<const uint8_t*>(a->x) + r * w.k * esz;
    void* orow = static_cast<uint8_t*>(a->out) + r * w.n * osz;
    const void* rr = a->residual ? static_cast<const uint8_t*>(a->residual) + r * w.n * osz : nullptr;
    if (auto st = GemvLinearRow(xr, a->x_dtype, w, orow, a->out_dtype, rr, s); st != AM_STATUS_OK) return st;
  }
  return AM_STATUS_OK;
}
