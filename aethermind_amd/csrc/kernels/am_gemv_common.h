// Device helpers shared by the decode GEMV kernels (gemv.hip) and the persistent
// decode-layers kernel (decode_layers.hip): INT4 unpack, the bf16 dot of one 16-byte
// weight chunk, fp16 scale bits, and the cross-lane row-sum reductions of a wave.
#pragma once

#include "am_kernel_common.h"

namespace am {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x2_t as_bf2(uint32_t u) { return __builtin_bit_cast(bf16x2_t, u); }

// Unpack constants held in VGPRs: gfx9 VOP3 encodings take no literal operands, so
// with both constants in registers each nibble pair costs one v_and_or_b32 (plus one
// shift) instead of separate and/or instructions.
struct Unpack {
  uint32_t mask, magic;
  __device__ __forceinline__ Unpack() : mask(0x000F000Fu), magic(0x43004300u) {
    asm volatile("" : "+v"(mask), "+v"(magic));
  }
};

// INT4 device word = k 8w..8w+7, nibble j holding q+8 of k 8w + {0,2,4,6,1,3,5,7}[j]:
// (word >> 4t) & 0x000F000F | 0x43004300 is the bf16 pair (136+q_2t, 136+q_2t+1).
// Returns init + sum over the 32 k of the chunk of x * (136 + q), with x as 16 bf16
// pairs in k order (xd).  Products are exact; sums are fp32.
__device__ __forceinline__ float int4_chunk_dot_bf16(const uint4 w, const uint32_t* xd, float init,
                                                     const Unpack& up) {
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  float acc = init;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const uint32_t pair = ((ws[t] >> (4 * pp)) & up.mask) | up.magic;
      acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(xd[4 * t + pp]), as_bf2(pair), acc, false);
    }
  return acc;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}

// SiLU of the reference's const-eval form (const_eval_silu_mul.cpp:18-31).
__device__ __forceinline__ float silu_ref(float g) {
  if (g >= 0.0f) return g / (1.0f + expf(-g));
  const float e = expf(g);
  return g * e / (1.0f + e);
}

// ---- cross-lane reduction of one iteration's row sums ----
// Every lane holds partial sums of the 2P rows of an iteration (P pairs).  A butterfly
// of gfx950 permlane swaps (32-lane halves, then 16-lane rows), one DPP row rotation
// and DPP adds folds all rows at once; a final swap leaves both rows of pair pp in
// one lane, so the epilogue of every pair runs in the same instruction stream.
//   v_permlane32_swap(a, b) -> {[a.lo, b.lo], [a.hi, b.hi]}
//   v_permlane16_swap(a, b) -> {[a.r0, b.r0, a.r2, b.r2], [a.r1, b.r1, a.r3, b.r3]}
__device__ __forceinline__ float swap32_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap16_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// sum over each aligned 8-lane group (every lane receives it)
__device__ __forceinline__ float sum8(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  return dpp_add<0x141>(v);  // row_half_mirror
}
__device__ __forceinline__ float sum16(float v) { return dpp_add<0x140>(sum8(v)); }  // + row_mirror

// acc[pp][rr] partial sums -> (a0, a1) = full sums of pair pp in the lane that owns it;
// returns pp for that lane, -1 elsewhere.
template <int P>
__device__ __forceinline__ int reduce_pairs(const float (&acc)[P][2], int lane, float& a0, float& a1) {
  if constexpr (P == 1) {
    float x = swap32_add(acc[0][0], acc[0][1]);  // [v0 | v1] halves
    x = swap16_add(x, x);                        // each 16-lane row: its half folded to 16 lanes
    x = sum16(x);                                // lanes 0-31: v0, 32-63: v1
    const auto w = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    a0 = __uint_as_float(w[0]);
    a1 = __uint_as_float(w[1]);
    return lane == 0 ? 0 : -1;
  } else if constexpr (P == 2) {
    const float x0 = swap32_add(acc[0][0], acc[1][0]);  // [v0 | v2]
    const float x1 = swap32_add(acc[0][1], acc[1][1]);  // [v1 | v3]
    float y = swap16_add(x0, x1);                       // rows [v0, v1, v2, v3]
    y = sum16(y);
    const auto w = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    a0 = __uint_as_float(w[0]);  // lane 0: pair 0, lane 32: pair 1
    a1 = __uint_as_float(w[1]);
    return (lane & 31) == 0 ? (lane >> 5) : -1;
  } else {
    static_assert(P == 4, "pairs per iteration: 1, 2 or 4");
    // v_k = acc[k / 2][k % 2]
    const float x0 = swap32_add(acc[0][0], acc[2][0]);  // [v0 | v4]
    const float x1 = swap32_add(acc[0][1], acc[2][1]);  // [v1 | v5]
    const float x2 = swap32_add(acc[1][0], acc[3][0]);  // [v2 | v6]
    const float x3 = swap32_add(acc[1][1], acc[3][1]);  // [v3 | v7]
    const float y0 = swap16_add(x0, x1);                // rows [v0, v1, v4, v5]
    const float y1 = swap16_add(x2, x3);                // rows [v2, v3, v6, v7]
    // fold each row to 8 lanes: low 8 lanes keep y0's row, high 8 lanes y1's
    const bool hi8 = (lane & 8) != 0;
    const float keep = hi8 ? y1 : y0, send = hi8 ? y0 : y1;
    float z = keep + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0x128, 0xF,
                                                                         0xF, false));  // row_ror:8
    z = sum8(z);  // 8-lane groups: row0 [v0|v2], row1 [v1|v3], row2 [v4|v6], row3 [v5|v7]
    const auto w = __builtin_amdgcn_permlane16_swap(__float_as_uint(z), __float_as_uint(z), false, false);
    a0 = __uint_as_float(w[0]);  // lanes 0, 8, 32, 40: pairs 0, 1, 2, 3
    a1 = __uint_as_float(w[1]);
    return ((lane & 23) == 0) ? (((lane >> 5) << 1) | ((lane >> 3) & 1)) : -1;
  }
}

}  // namespace am
