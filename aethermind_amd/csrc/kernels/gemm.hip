// Prefill GEMM for gfx950: out[M,N] = X[M,K] (bf16) @ W[N,K]^T on bf16 MFMA
// (v_mfma_f32_16x16x32_bf16), with the weight tile dequantised into LDS.
//
//   * Block tile 128 x 128 (M x N), K step 64; 4 waves in a 2x2 arrangement, each
//     owning a 64 x 64 sub-tile = 4 x 4 MFMA tiles of 16 x 16 (64 fp32 accumulators
//     per lane).
//   * X tile and W tile are staged in LDS as bf16 rows padded by 16 bytes, so the
//     16 rows read by one MFMA operand fetch fall into distinct banks.
//   * Quantized weights are written to LDS as the exact integer q (|q| <= 127 is
//     exact in bf16), never as q*s: INT4 group partial sums are kept in a second
//     accumulator set and scaled by the fp16 group scale when a group completes,
//     INT8 sums are scaled by the per-row scale in the epilogue.  Products are exact
//     and accumulation is fp32, so the only rounding is the fp32 accumulation.
//   * Block index -> tile mapping walks N fastest inside a band of 8 M-tiles, which
//     keeps each XCD's L2 working on neighbouring weight columns.

#include "am_kernel_common.h"

namespace am {
am_status_code GemvLinearRow(const void* x, int32_t act, const am_gfx950_weight& w, void* out, int32_t out_dtype,
                             const void* residual, hipStream_t s);
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

constexpr int BM = 128, BN = 128, BK = 64;
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

template <int WF>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  __shared__ __align__(16) uint16_t As[BM * LDSROW];
  __shared__ __align__(16) uint16_t Bs[BN * LDSROW];
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

  f32x4_t acc[4][4];
  f32x4_t part[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      part[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

  const int lrow = tid >> 1;   // 0..127: tile row this thread stages
  const int lhalf = tid & 1;   // which 32-k half of the 64-k step
  const int64_t ng = (WF == AM_WF_INT4) ? p.K / p.group : 1;

  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
    // ---- stage X tile: row lrow, k [k0 + 32*lhalf, +32) ----
    {
      const int64_t gm = m0 + lrow;
      uint4 v[4];
      if (gm < p.M) {
        const uint4* src = reinterpret_cast<const uint4*>(p.x + gm * p.K + k0 + 32 * lhalf);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = src[i];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = make_uint4(0, 0, 0, 0);
      }
      uint4* dst = reinterpret_cast<uint4*>(As + lrow * LDSROW + 32 * lhalf);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = v[i];
    }
    // ---- stage W tile: row n0+lrow, same k range, as bf16 integers / values ----
    {
      const int64_t gn = n0 + lrow;
      uint4 o[4];
      if (gn < p.N) {
        if constexpr (WF == AM_WF_BF16) {
          const uint4* src = reinterpret_cast<const uint4*>(p.w + (gn * p.K + k0 + 32 * lhalf) * 2);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = src[i];
        } else if constexpr (WF == AM_WF_INT8) {
          const uint4* src = reinterpret_cast<const uint4*>(p.w + gn * p.K + k0 + 32 * lhalf);
          const uint4 a = src[0], b = src[1];
          const uint32_t ws[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
          uint32_t outw[16];
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const float q0 = static_cast<float>(ws[t] & 0xFFu) - 128.0f;
            const float q1 = static_cast<float>((ws[t] >> 8) & 0xFFu) - 128.0f;
            const float q2 = static_cast<float>((ws[t] >> 16) & 0xFFu) - 128.0f;
            const float q3 = static_cast<float>(ws[t] >> 24) - 128.0f;
            outw[2 * t] = pack_bf16_int(q0, q1);
            outw[2 * t + 1] = pack_bf16_int(q2, q3);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = make_uint4(outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]);
        } else {  // INT4: 32 nibbles = 16 bytes; word t holds k 8t + {0,2,4,6,1,3,5,7}
          const uint4 a = *reinterpret_cast<const uint4*>(p.w + gn * (p.K / 2) + (k0 + 32 * lhalf) / 2);
          const uint32_t ws[4] = {a.x, a.y, a.z, a.w};
          uint32_t outw[16];
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
              const uint32_t pr = (ws[t] >> (4 * pp)) & 0x000F000Fu;
              const float lo = static_cast<float>(pr & 0xFu) - 8.0f;
              const float hi = static_cast<float>(pr >> 16) - 8.0f;
              outw[4 * t + pp] = pack_bf16_int(lo, hi);
            }
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = make_uint4(outw[4 * i], outw[4 * i + 1], outw[4 * i + 2], outw[4 * i + 3]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_uint4(0, 0, 0, 0);
      }
      uint4* dst = reinterpret_cast<uint4*>(Bs + lrow * LDSROW + 32 * lhalf);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = o[i];
    }
    __syncthreads();

    // ---- MFMA over the 64-k step (two k32 slices) ----
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8_t af[4], bfr[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const uint4 v = *reinterpret_cast<const uint4*>(As + (wm * 64 + mt * 16 + (lane & 15)) * LDSROW +
                                                        ks * 32 + 8 * (lane >> 4));
        af[mt] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const uint4 v = *reinterpret_cast<const uint4*>(Bs + (wn * 64 + nt * 16 + (lane & 15)) * LDSROW +
                                                        ks * 32 + 8 * (lane >> 4));
        bfr[nt] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          if constexpr (WF == AM_WF_INT4)
            part[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], part[mt][nt], 0, 0, 0);
          else
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfr[nt], acc[mt][nt], 0, 0, 0);
        }
    }
    __syncthreads();

    if constexpr (WF == AM_WF_INT4) {
      if ((k0 + BK) % p.group == 0) {
        const int64_t g = (k0 + BK) / p.group - 1;
        const uint16_t* sc = static_cast<const uint16_t*>(p.scales);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
          const int64_t gn = n0 + wn * 64 + nt * 16 + (lane & 15);
          const float s = gn < p.N ? static_cast<float>(__builtin_bit_cast(_Float16, sc[gn * ng + g])) : 0.0f;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[mt][nt][r] = fmaf(s, part[mt][nt][r], acc[mt][nt][r]);
            part[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
        }
      }
    }
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
  const bool use_gemm = a->mode == 2 || (a->mode == 0 && a->m > 8 && gemm_ok);
  if (use_gemm) {
    AM_CHECK_ARG(gemm_ok, "linear: MFMA GEMM needs bf16 activations, bf16/int8/int4 weights, K % 64 == 0");
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
    switch (w.format) {
      case AM_WF_BF16: hipLaunchKernelGGL(gemm_kernel<AM_WF_BF16>, grid, dim3(256), 0, s, g); break;
      case AM_WF_INT8: hipLaunchKernelGGL(gemm_kernel<AM_WF_INT8>, grid, dim3(256), 0, s, g); break;
      default: hipLaunchKernelGGL(gemm_kernel<AM_WF_INT4>, grid, dim3(256), 0, s, g); break;
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
