// Shared device helpers and host-side launch utilities for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "am_gfx950.h"

namespace am {

// ---- host: error reporting (defined in host/c_api.cpp) ----
am_status_code SetLastError(am_status_code code, const char* msg);

#define AM_CHECK_ARG(cond, msg)                                              \
  do {                                                                       \
    if (!(cond)) return ::am::SetLastError(AM_STATUS_INVALID_ARGUMENT, msg); \
  } while (0)

#define AM_RETURN_IF_LAUNCH_FAILED(what)                                                 \
  do {                                                                                   \
    hipError_t e_ = hipGetLastError();                                                   \
    if (e_ != hipSuccess) return ::am::SetLastError(AM_STATUS_INTERNAL, hipGetErrorString(e_)); \
  } while (0)

inline hipStream_t AsStream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t CeilDiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// KV cache row addressing, in elements from the cache (pool) base.  Contiguous
// (table == nullptr): sequence b's planes start b * cbs elements in and head g's rows
// g * cap * d after that.  Paged: the cache is a pool of blocks [hkv][1 << shift][d]
// and table[b * stride + (pos >> shift)] names the block holding position pos of
// sequence b.  Readers clamp an entry outside [0, num_blocks) into the pool (Row), so a
// bad table cannot address outside it; writers (WriteRow) skip the row instead and set
// err, so a position whose block is unassigned (-1) never overwrites another
// sequence's block.  A run of positions that starts at a multiple of 32 and stays
// inside 32 positions lies in one block (blocks are at least 32 positions), so kernels
// look up one block per 32-position step.
struct KvRows {
  const int32_t* table = nullptr;
  int32_t* err = nullptr;  // writers: set to 1 on an entry outside the pool (optional)
  int64_t cbs = 0, cap = 0;
  int64_t num_blocks = 0;
  int32_t shift = 0, stride = 0;
  int32_t hkv = 0, d = 0;

  __device__ __forceinline__ int64_t Row(int64_t b, int64_t g, int64_t pos) const {
    if (table == nullptr) return b * cbs + (g * cap + pos) * d;
    int64_t blk = table[b * stride + (pos >> shift)];
    blk = blk < 0 ? 0 : (blk >= num_blocks ? num_blocks - 1 : blk);
    return (((blk * hkv + g) << shift) + (pos & ((int64_t{1} << shift) - 1))) * d;
  }

  // The row a writer stores position pos of (b, g) to, or -1 (row skipped, err set)
  // when the table entry lies outside [0, num_blocks).
  __device__ __forceinline__ int64_t WriteRow(int64_t b, int64_t g, int64_t pos) const {
    if (table == nullptr) return b * cbs + (g * cap + pos) * d;
    const int64_t blk = table[b * stride + (pos >> shift)];
    if (blk < 0 || blk >= num_blocks) {
      if (err != nullptr) *err = 1;
      return -1;
    }
    return (((blk * hkv + g) << shift) + (pos & ((int64_t{1} << shift) - 1))) * d;
  }
};

// Host side: the KvRows of a cache (pages may be null) after checking the page table
// arguments against the logical capacity.
am_status_code MakeKvRows(const am_gfx950_kv_pages* pages, int64_t cbs, int64_t cap, int64_t hkv, int64_t d,
                          KvRows* out);

// Number of compute units of the current device (cached per device).
int DeviceCUs();

// Batched decode GEMV (gemv_batch.hip): 1..16 token rows share one weight read.
bool BatchLinearEligible(int32_t act, const am_gfx950_weight& w, int64_t m, const void* x);
am_status_code BatchLinear(const void* x, int64_t m, const am_gfx950_weight& w, void* out, int32_t out_dtype,
                           const void* residual, hipStream_t s);
am_status_code BatchQkv(const am_gfx950_fused_qkv_args* a, hipStream_t s);
am_status_code BatchLinearResidual(const am_gfx950_fused_linear_residual_args* a, hipStream_t s);
am_status_code BatchGateUp(const am_gfx950_fused_gate_up_args* a, hipStream_t s);
am_status_code BatchNormLogits(const am_gfx950_fused_lm_head_args* a, hipStream_t s);

// Prefill INT4 GEMM (gemm_i4.hip): epilogue 0 store, 1 residual, 2 column split into
// out0|out1|out2 at columns c1, c2, 3 SiLU-Mul of the gate|up halves into out0.
// ws (optional, tickets zero, left zero) lets shapes with few tiles split K.
bool GemmI4Eligible(const am_gfx950_weight& w, int64_t m, const void* x);
int64_t GemmI4WorkspaceBytes(int64_t m, int64_t n, int64_t k, int64_t group);
am_status_code GemmI4(const void* x, int64_t m, const am_gfx950_weight& w, int32_t epi, void* out0, void* out1,
                      void* out2, int64_t c1, int64_t c2, const void* residual, void* ws, int64_t ws_bytes,
                      hipStream_t s);
am_status_code GemmI4QkvRopeKv(const void* x, int64_t m, const am_gfx950_weight& w, const am_gfx950_prefill_rope_kv& r,
                               void* q_out, void* ws, int64_t ws_bytes, hipStream_t s);

// ---- device: numeric helpers ----
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// RoPE rotation of the pair (x1, x2) = (value i, value i + d/2) of a head (rope_op.cpp
// split-half form): y1 = x1 c - x2 s, y2 = x2 c + x1 s in fp32.  The fused multiply-adds
// are written out so every kernel that rotates (the RoPE node, and the q|k|v epilogues
// that replace it) rounds identically whatever the compiler would contract.
__device__ __forceinline__ void rope_rotate(float x1, float x2, float c, float s, float& y1, float& y2) {
  y1 = __builtin_fmaf(x1, c, -(x2 * s));
  y2 = __builtin_fmaf(x1, s, x2 * c);
}

// float -> bf16 round-to-nearest-even, NaN -> 0x7FC0 (the reference's conversion,
// bfloat16.cpp:20-32).
// The conversion is v_cvt_pk_bf16_f32 (RNE); only NaN needs the canonical pattern.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v) {
  const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  return v != v ? static_cast<uint16_t>(0x7FC0u) : h;
}

struct ActF32 {
  using T = float;
  static constexpr int kDtype = AM_DT_F32;
  __device__ static __forceinline__ float load(const T* p, int64_t i) { return p[i]; }
  __device__ static __forceinline__ void store(T* p, int64_t i, float v) { p[i] = v; }
  __device__ static __forceinline__ float round(float v) { return v; }
};

struct ActBF16 {
  using T = uint16_t;
  static constexpr int kDtype = AM_DT_BF16;
  __device__ static __forceinline__ float load(const T* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  __device__ static __forceinline__ void store(T* p, int64_t i, float v) { p[i] = f32_to_bf16_bits(v); }
  __device__ static __forceinline__ float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over a 256-thread block; every thread gets the result.  `red` holds >= 4 floats.
// Sum over a block of NW waves (every thread receives it); red holds NW floats.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += red[w];
  return t;
}

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Argmax tie rule (build SPEC): larger value wins; equal values -> lower index;
// NaN never wins.  (v, i) is "better" than (bv, bi)?
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float bv, int64_t bi) {
  if (v != v) return false;
  if (bi < 0) return true;
  return v > bv || (v == bv && i < bi);
}

}  // namespace am
