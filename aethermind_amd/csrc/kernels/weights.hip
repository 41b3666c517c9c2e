// Weight loader / repack kernels for gfx950: synthetic weights of the build SPEC,
// INT8 per-channel and INT4 group quantization straight into the device tile
// layout, plain (f32/bf16) packing with row concatenation/interleave, conversion of
// the logical INT4 interchange format, and the bit-exact dequantizer used by tests.

#include <cmath>

#include "am_kernel_common.h"

namespace am {
namespace {

// ---------------- synthetic generator (build SPEC) ----------------
// SplitMix64 counter stream + Box-Muller evaluated with fma/mul/add only, so the
// result bits do not depend on any math library.  Contraction is disabled so every
// product below is rounded exactly where it is written.
#pragma clang fp contract(off)

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t splitmix64_hd(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ double recip_newton(double d) {
  double r = 0.5;
  for (int i = 0; i < 6; ++i) {
    const double e = __fma_rn(-d, r, 1.0);
    r = __fma_rn(r, e, r);
  }
  return r;
}

__device__ double portable_log(double x) {
  const uint64_t b = __double_as_longlong(x);
  int e = static_cast<int>((b >> 52) & 0x7FF) - 1023;
  double m = __longlong_as_double(static_cast<long long>((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) * recip_newton(m + 1.0);
  const double s2 = s * s;
  const double c[13] = {1.0 / 3,  1.0 / 5,  1.0 / 7,  1.0 / 9,  1.0 / 11, 1.0 / 13, 1.0 / 15,
                        1.0 / 17, 1.0 / 19, 1.0 / 21, 1.0 / 23, 1.0 / 25, 1.0 / 27};
  double p = c[12];
  for (int i = 11; i >= 0; --i) p = __fma_rn(p, s2, c[i]);
  const double lnm = 2.0 * __fma_rn(s * s2, p, s);
  return __fma_rn(static_cast<double>(e), 0.6931471805599453, lnm);
}

__device__ void portable_sincos_turns(double turns, double* so, double* co) {
  const double t = turns * 4.0;
  const int q = static_cast<int>(t);
  double f = t - static_cast<double>(q);
  bool swap = false;
  if (f > 0.5) {
    f = 1.0 - f;
    swap = true;
  }
  const double a = f * 1.5707963267948966;
  const double a2 = a * a;
  const double sc[9] = {-1.0 / 6.0,           1.0 / 120.0,          -1.0 / 5040.0,
                        1.0 / 362880.0,       -1.0 / 39916800.0,    1.0 / 6227020800.0,
                        -1.0 / 1307674368000.0, 1.0 / 355687428096000.0, -1.0 / 121645100408832000.0};
  const double cc[9] = {-1.0 / 2.0,         1.0 / 24.0,           -1.0 / 720.0,
                        1.0 / 40320.0,      -1.0 / 3628800.0,     1.0 / 479001600.0,
                        -1.0 / 87178291200.0, 1.0 / 20922789888000.0, -1.0 / 6402373705728000.0};
  double ps = sc[8], pc = cc[8];
  for (int i = 7; i >= 0; --i) {
    ps = __fma_rn(ps, a2, sc[i]);
    pc = __fma_rn(pc, a2, cc[i]);
  }
  double sv = __fma_rn(a * a2, ps, a);
  double cv = __fma_rn(a2, pc, 1.0);
  if (swap) {
    const double tmp = sv;
    sv = cv;
    cv = tmp;
  }
  switch (q & 3) {
    case 0: *so = sv; *co = cv; break;
    case 1: *so = cv; *co = -sv; break;
    case 2: *so = -sv; *co = -cv; break;
    default: *so = -cv; *co = sv; break;
  }
}

__device__ double portable_sqrt(double x) {
  if (x == 0.0) return 0.0;
  const uint64_t b = __double_as_longlong(x);
  int e = static_cast<int>((b >> 52) & 0x7FF) - 1023;
  double m = __longlong_as_double(static_cast<long long>((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
  if (e & 1) {
    m = m * 2.0;
    e -= 1;
  }
  double y = __fma_rn(-0.1666666666666667, m - 1.0, 1.0);
  const double h = 0.5 * m;
  for (int i = 0; i < 6; ++i) {
    const double hy = h * y;
    y = y * __fma_rn(-hy, y, 1.5);
  }
  const double r = m * y;
  return r * __longlong_as_double(static_cast<long long>(static_cast<uint64_t>(e / 2 + 1023) << 52));
}

template <class O>
__global__ __launch_bounds__(256) void synth_kernel(uint64_t key, double stddev, int64_t offset, int64_t n,
                                                    typename O::T* out) {
  // one thread per Box-Muller pair
  const int64_t first = offset >> 1;
  const int64_t last = (offset + n - 1) >> 1;
  for (int64_t pidx = first + blockIdx.x * 256 + threadIdx.x; pidx <= last;
       pidx += static_cast<int64_t>(gridDim.x) * 256) {
    const uint64_t r = splitmix64(key + static_cast<uint64_t>(pidx));
    const double u1 = static_cast<double>((r >> 32) + 1ull) * 2.3283064365386963e-10;
    const double u2 = static_cast<double>(r & 0xFFFFFFFFull) * 2.3283064365386963e-10;
    const double rad = portable_sqrt(-2.0 * portable_log(u1));
    double sn, cs;
    portable_sincos_turns(u2, &sn, &cs);
    const int64_t i0 = 2 * pidx, i1 = 2 * pidx + 1;
    if (i0 >= offset && i0 < offset + n) O::store(out, i0 - offset, static_cast<float>(stddev * (rad * cs)));
    if (i1 >= offset && i1 < offset + n) O::store(out, i1 - offset, static_cast<float>(stddev * (rad * sn)));
  }
}

__global__ __launch_bounds__(256) void token_ids_kernel(uint64_t key, int64_t vocab, int64_t n, int64_t* out) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256) {
    const uint64_t r = splitmix64(key + static_cast<uint64_t>(i));
    out[i] = static_cast<int64_t>(((r >> 32) * static_cast<uint64_t>(vocab)) >> 32);
  }
}

#pragma clang fp contract(on)

// ---------------- quantization into device tiles ----------------
__device__ __forceinline__ float load_src(const void* src, int32_t dt, int64_t i) {
  if (dt == AM_DT_F32) return static_cast<const float*>(src)[i];
  const uint16_t b = static_cast<const uint16_t*>(src)[i];
  if (dt == AM_DT_F16) return static_cast<float>(__builtin_bit_cast(_Float16, b));  // exact
  return bf16_bits_to_f32(b);
}

__device__ __forceinline__ float block_max_256(float v, float* red) {
  v = fmaxf(v, __shfl_xor(v, 32, 64));
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  v = fmaxf(v, __shfl_xor(v, 8, 64));
  v = fmaxf(v, __shfl_xor(v, 4, 64));
  v = fmaxf(v, __shfl_xor(v, 2, 64));
  v = fmaxf(v, __shfl_xor(v, 1, 64));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One block per source row.  INT8: byte = q + 128 with q = clamp(rint(w/s), -127, 127),
// s = max|w|/127 (1 if the row is zero).
__global__ __launch_bounds__(256) void quant_int8_kernel(const void* src, int32_t sdt, int64_t k, uint8_t* dst,
                                                         float* scales, int64_t row_off, int64_t row_stride) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int64_t dr = row_off + r * row_stride;
  float amax = 0.0f;
  for (int64_t j = threadIdx.x; j < k; j += 256) amax = fmaxf(amax, fabsf(load_src(src, sdt, r * k + j)));
  amax = block_max_256(amax, red);
  const float s = amax == 0.0f ? 1.0f : amax / 127.0f;
  if (threadIdx.x == 0) scales[dr] = s;
  for (int64_t j = threadIdx.x; j < k; j += 256) {
    float q = rintf(load_src(src, sdt, r * k + j) / s);
    q = fminf(127.0f, fmaxf(-127.0f, q));
    dst[dr * k + j] = static_cast<uint8_t>(static_cast<int>(q) + 128);
  }
}

// INT4: per group s16 = fp16(max|w|/7) (RNE), q = clamp(rint(w/s), -8, 7) (0 if s == 0),
// nibble = q + 8, placed in device tile order.
__global__ __launch_bounds__(256) void quant_int4_kernel(const void* src, int32_t sdt, int64_t k, int32_t group,
                                                         uint8_t* dst, uint16_t* scales, int64_t row_off,
                                                         int64_t row_stride) {
  extern __shared__ float gsc[];  // k/group scales (fp32 value of the fp16 scale)
  const int64_t r = blockIdx.x;
  const int64_t dr = row_off + r * row_stride;
  const int64_t ng = k / group;
  for (int64_t g = threadIdx.x; g < ng; g += 256) {
    float amax = 0.0f;
    for (int j = 0; j < group; ++j) amax = fmaxf(amax, fabsf(load_src(src, sdt, r * k + g * group + j)));
    const _Float16 h = static_cast<_Float16>(amax / 7.0f);
    scales[dr * ng + g] = __builtin_bit_cast(uint16_t, h);
    gsc[g] = static_cast<float>(h);
  }
  __syncthreads();
  const int64_t words = k / 8;
  uint32_t* drow = reinterpret_cast<uint32_t*>(dst + dr * (k / 2));
  for (int64_t wi = threadIdx.x; wi < words; wi += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t kk = 8 * wi + ((j < 4) ? 2 * j : 2 * (j - 4) + 1);
      const float s = gsc[kk / group];
      float q = 0.0f;
      if (s != 0.0f) {
        q = rintf(load_src(src, sdt, r * k + kk) / s);
        q = fminf(7.0f, fmaxf(-8.0f, q));
      }
      word |= static_cast<uint32_t>(static_cast<int>(q) + 8) << (4 * j);
    }
    drow[wi] = word;
  }
}

__global__ __launch_bounds__(256) void pack_plain_kernel(const void* src, int32_t sdt, int64_t k, void* dst,
                                                         int32_t dfmt, int64_t row_off, int64_t row_stride) {
  const int64_t r = blockIdx.x;
  const int64_t dr = row_off + r * row_stride;
  for (int64_t j = threadIdx.x; j < k; j += 256) {
    const float v = load_src(src, sdt, r * k + j);
    if (dfmt == AM_WF_F32)
      static_cast<float*>(dst)[dr * k + j] = v;
    else
      static_cast<uint16_t*>(dst)[dr * k + j] =
          sdt == AM_DT_BF16 ? static_cast<const uint16_t*>(src)[r * k + j] : f32_to_bf16_bits(v);
  }
}

// logical (low nibble = even k, two's complement) -> device tile order, q+8 nibbles
__global__ __launch_bounds__(256) void pack_int4_kernel(const uint8_t* logical, uint8_t* dst, int64_t k) {
  const int64_t r = blockIdx.x;
  const int64_t words = k / 8;
  const uint8_t* lrow = logical + r * (k / 2);
  uint32_t* drow = reinterpret_cast<uint32_t*>(dst + r * (k / 2));
  for (int64_t wi = threadIdx.x; wi < words; wi += 256) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t kk = 8 * wi + ((j < 4) ? 2 * j : 2 * (j - 4) + 1);
      const uint8_t b = lrow[kk / 2];
      const uint32_t nib = (kk & 1) ? (b >> 4) : (b & 0xFu);
      word |= (nib ^ 8u) << (4 * j);
    }
    drow[wi] = word;
  }
}

__global__ __launch_bounds__(256) void dequant_kernel(const void* data, const void* scales, int32_t fmt, int64_t k,
                                                      int32_t group, float* out) {
  const int64_t r = blockIdx.x;
  for (int64_t j = threadIdx.x; j < k; j += 256) {
    float v;
    if (fmt == AM_WF_F32) {
      v = static_cast<const float*>(data)[r * k + j];
    } else if (fmt == AM_WF_BF16) {
      v = bf16_bits_to_f32(static_cast<const uint16_t*>(data)[r * k + j]);
    } else if (fmt == AM_WF_INT8) {
      const int q = static_cast<int>(static_cast<const uint8_t*>(data)[r * k + j]) - 128;
      v = static_cast<float>(q) * static_cast<const float*>(scales)[r];
    } else {
      const uint32_t word = reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(data) + r * (k / 2))[j / 8];
      const int m = static_cast<int>(j & 7);
      const int nib_idx = (m & 1) ? 4 + (m >> 1) : (m >> 1);
      const int q = static_cast<int>((word >> (4 * nib_idx)) & 0xFu) - 8;
      const uint16_t sb = static_cast<const uint16_t*>(scales)[r * (k / group) + j / group];
      v = static_cast<float>(q) * static_cast<float>(__builtin_bit_cast(_Float16, sb));
    }
    out[r * k + j] = v;
  }
}

// ---------------- GPTQ ingestion ----------------
// One thread per qweight word (input features 8i .. 8i+7 of output column j); j runs
// fastest, so the qweight, qzeros and scales reads are coalesced.
struct GptqKernelArgs {
  const int32_t* qweight;
  const int32_t* qzeros;
  const void* scales;
  const int32_t* g_idx;
  int64_t n, k, group, groups;
  int32_t sdt, zoff;
  float* out_f32;
  uint8_t* out_logical;
};

__global__ __launch_bounds__(256) void gptq_unpack_kernel(GptqKernelArgs a) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= (a.k / 8) * a.n) return;
  const int64_t i = idx / a.n, j = idx % a.n;
  const uint32_t word = static_cast<uint32_t>(a.qweight[i * a.n + j]);
  uint32_t packed = 0;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int64_t kk = 8 * i + t;
    int64_t g = a.g_idx != nullptr ? a.g_idx[kk] : kk / a.group;
    g = g < 0 ? 0 : (g >= a.groups ? a.groups - 1 : g);
    const uint32_t zw = static_cast<uint32_t>(a.qzeros[g * (a.n / 8) + j / 8]);
    const int z = static_cast<int>(((zw >> (4 * (j & 7))) + static_cast<uint32_t>(a.zoff)) & 0xFu);
    const int d = static_cast<int>((word >> (4 * t)) & 0xFu) - z;
    if (a.out_f32 != nullptr)
      a.out_f32[j * a.k + kk] = load_src(a.scales, a.sdt, g * a.n + j) * static_cast<float>(d);
    packed |= (static_cast<uint32_t>(d) & 0xFu) << (4 * t);  // k order: low nibble = even k
  }
  if (a.out_logical != nullptr) reinterpret_cast<uint32_t*>(a.out_logical + j * (a.k / 2))[i] = packed;
}

// fp16 scales [groups][n] -> [n][groups]
__global__ __launch_bounds__(256) void gptq_scales_kernel(const uint16_t* s, int64_t n, int64_t groups, uint16_t* out) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= n * groups) return;
  const int64_t g = idx / n, j = idx % n;
  out[j * groups + g] = s[g * n + j];
}

}  // namespace
}  // namespace am

using namespace am;

extern "C" am_status_code am_gfx950_weight_bytes(int64_t n, int64_t k, int32_t format, int32_t group_size,
                                                 int64_t* data_bytes, int64_t* scale_bytes) {
  AM_CHECK_ARG(n > 0 && k > 0 && data_bytes && scale_bytes, "weight_bytes: bad args");
  switch (format) {
    case AM_WF_F32: *data_bytes = n * k * 4; *scale_bytes = 0; break;
    case AM_WF_BF16: *data_bytes = n * k * 2; *scale_bytes = 0; break;
    case AM_WF_INT8: *data_bytes = n * k; *scale_bytes = n * 4; break;
    case AM_WF_INT4:
      AM_CHECK_ARG(group_size > 0 && k % group_size == 0 && k % 32 == 0, "weight_bytes: INT4 needs k % group == 0");
      *data_bytes = n * k / 2;
      *scale_bytes = n * (k / group_size) * 2;
      break;
    default: return SetLastError(AM_STATUS_INVALID_ARGUMENT, "weight_bytes: unknown format");
  }
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_synth_normal(const am_gfx950_synth_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && (a->dtype == AM_DT_F32 || a->dtype == AM_DT_BF16), "synth_normal: bad args");
  AM_CHECK_ARG(a->offset >= 0 && a->n >= 0, "synth_normal: bad range");
  if (a->n == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(a->out != nullptr, "synth_normal: null output");
  const uint64_t key = splitmix64_hd(splitmix64_hd(a->seed) ^ a->tensor_id);
  const int64_t pairs = ((a->offset + a->n - 1) >> 1) - (a->offset >> 1) + 1;
  int64_t grid = CeilDiv(pairs, 256);
  if (grid > 16384) grid = 16384;
  if (a->dtype == AM_DT_F32)
    hipLaunchKernelGGL(synth_kernel<ActF32>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, AsStream(stream), key,
                       a->stddev, a->offset, a->n, static_cast<float*>(a->out));
  else
    hipLaunchKernelGGL(synth_kernel<ActBF16>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, AsStream(stream), key,
                       a->stddev, a->offset, a->n, static_cast<uint16_t*>(a->out));
  AM_RETURN_IF_LAUNCH_FAILED("synth_normal");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_synth_token_ids(uint64_t seed, uint64_t stream_id, int64_t vocab, int64_t n,
                                                    int64_t* out, void* stream) {
  AM_CHECK_ARG(vocab > 0 && n >= 0, "synth_token_ids: bad args");
  if (n == 0) return AM_STATUS_OK;
  AM_CHECK_ARG(out != nullptr, "synth_token_ids: null output");
  const uint64_t key = splitmix64_hd(splitmix64_hd(seed) ^ (0xF00D0000ull + stream_id));
  int64_t grid = CeilDiv(n, 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(token_ids_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, AsStream(stream), key, vocab,
                     n, out);
  AM_RETURN_IF_LAUNCH_FAILED("synth_token_ids");
  return AM_STATUS_OK;
}

namespace {
am_status_code CheckQuantArgs(const am_gfx950_quantize_args* a) {
  AM_CHECK_ARG(a != nullptr && a->src != nullptr, "quantize: null args");
  AM_CHECK_ARG(a->src_dtype == AM_DT_F32 || a->src_dtype == AM_DT_BF16 || a->src_dtype == AM_DT_F16,
               "quantize: src dtype must be f32, bf16 or f16");
  AM_CHECK_ARG(a->dst.data != nullptr && a->dst.n > 0 && a->dst.k > 0, "quantize: bad destination");
  AM_CHECK_ARG(a->dst_row_offset >= 0 && a->dst_row_stride >= 1, "quantize: bad row mapping");
  AM_CHECK_ARG(a->src_rows > 0 && a->src_rows <= 0x7FFFFFFF, "quantize: src_rows must be positive");
  AM_CHECK_ARG(a->dst_row_offset + (a->src_rows - 1) * a->dst_row_stride < a->dst.n,
               "quantize: rows would land past the destination");
  return AM_STATUS_OK;
}
}  // namespace

extern "C" am_status_code am_gfx950_quantize(const am_gfx950_quantize_args* a, void* stream) {
  if (auto st = CheckQuantArgs(a); st != AM_STATUS_OK) return st;
  const int64_t rows = a->src_rows;
  const int64_t k = a->dst.k;
  hipStream_t s = AsStream(stream);
  uint8_t* dst = static_cast<uint8_t*>(const_cast<void*>(a->dst.data));
  if (a->dst.format == AM_WF_INT8) {
    AM_CHECK_ARG(a->dst.scales != nullptr, "quantize: INT8 needs scales");
    hipLaunchKernelGGL(quant_int8_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, a->src, a->src_dtype, k,
                       dst, static_cast<float*>(const_cast<void*>(a->dst.scales)), a->dst_row_offset,
                       a->dst_row_stride);
  } else if (a->dst.format == AM_WF_INT4) {
    const int32_t g = a->dst.group_size;
    AM_CHECK_ARG(g > 0 && g % 2 == 0 && k % g == 0 && k % 8 == 0, "quantize: INT4 needs k % group == 0 and k % 8 == 0");
    AM_CHECK_ARG(a->dst.scales != nullptr, "quantize: INT4 needs scales");
    AM_CHECK_ARG((k / g) * 4 <= 64 * 1024, "quantize: too many groups per row");
    hipLaunchKernelGGL(quant_int4_kernel, dim3(static_cast<unsigned>(rows)), dim3(256),
                       static_cast<size_t>((k / g) * 4), s, a->src, a->src_dtype, k, g, dst,
                       static_cast<uint16_t*>(const_cast<void*>(a->dst.scales)), a->dst_row_offset,
                       a->dst_row_stride);
  } else {
    return SetLastError(AM_STATUS_INVALID_ARGUMENT, "quantize: destination must be INT8 or INT4 (use pack_plain)");
  }
  AM_RETURN_IF_LAUNCH_FAILED("quantize");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_pack_plain(const am_gfx950_quantize_args* a, void* stream) {
  if (auto st = CheckQuantArgs(a); st != AM_STATUS_OK) return st;
  AM_CHECK_ARG(a->dst.format == AM_WF_F32 || a->dst.format == AM_WF_BF16, "pack_plain: destination must be F32 or BF16");
  const int64_t rows = a->src_rows;
  hipLaunchKernelGGL(pack_plain_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, AsStream(stream), a->src,
                     a->src_dtype, a->dst.k, const_cast<void*>(a->dst.data), a->dst.format, a->dst_row_offset,
                     a->dst_row_stride);
  AM_RETURN_IF_LAUNCH_FAILED("pack_plain");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_pack_int4(const am_gfx950_pack_int4_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && a->logical && a->scales, "pack_int4: null args");
  AM_CHECK_ARG(a->dst.format == AM_WF_INT4 && a->dst.data && a->dst.scales, "pack_int4: destination must be INT4");
  AM_CHECK_ARG(a->dst.n > 0 && a->dst.k > 0 && a->dst.k % 8 == 0 && a->dst.group_size > 0 &&
                   a->dst.k % a->dst.group_size == 0,
               "pack_int4: bad shape");
  hipStream_t s = AsStream(stream);
  hipLaunchKernelGGL(pack_int4_kernel, dim3(static_cast<unsigned>(a->dst.n)), dim3(256), 0, s, a->logical,
                     static_cast<uint8_t*>(const_cast<void*>(a->dst.data)), a->dst.k);
  AM_RETURN_IF_LAUNCH_FAILED("pack_int4");
  const int64_t sb = a->dst.n * (a->dst.k / a->dst.group_size) * 2;
  if (hipMemcpyAsync(const_cast<void*>(a->dst.scales), a->scales, static_cast<size_t>(sb), hipMemcpyDeviceToDevice, s) !=
      hipSuccess)
    return SetLastError(AM_STATUS_INTERNAL, "pack_int4: scale copy failed");
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_gptq_unpack(const am_gfx950_gptq_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && a->qweight && a->qzeros && a->scales, "gptq_unpack: null args");
  AM_CHECK_ARG(a->n > 0 && a->k > 0 && a->n % 8 == 0 && a->k % 8 == 0 && a->n < (int64_t{1} << 31) &&
                   a->k < (int64_t{1} << 31),
               "gptq_unpack: n and k must be positive multiples of 8");
  AM_CHECK_ARG(a->group_size > 0 && a->k % a->group_size == 0, "gptq_unpack: group_size must divide k");
  AM_CHECK_ARG(a->scales_dtype == AM_DT_F16 || a->scales_dtype == AM_DT_BF16 || a->scales_dtype == AM_DT_F32,
               "gptq_unpack: scales must be F16, BF16 or F32");
  AM_CHECK_ARG(a->zero_offset == 0 || a->zero_offset == 1, "gptq_unpack: zero_offset must be 0 or 1");
  const bool f32 = a->out_f32 != nullptr, logical = a->out_logical != nullptr;
  AM_CHECK_ARG(f32 != logical, "gptq_unpack: give exactly one of out_f32 and out_logical");
  if (logical)
    AM_CHECK_ARG(a->out_scales != nullptr && a->scales_dtype == AM_DT_F16,
                 "gptq_unpack: the logical INT4 output needs out_scales and F16 scales");
  am::GptqKernelArgs g{a->qweight, a->qzeros, a->scales, a->g_idx, a->n, a->k, a->group_size, a->k / a->group_size,
                       a->scales_dtype, a->zero_offset, a->out_f32, a->out_logical};
  hipStream_t s = AsStream(stream);
  const int64_t words = (a->k / 8) * a->n;
  hipLaunchKernelGGL(am::gptq_unpack_kernel, dim3(static_cast<unsigned>(CeilDiv(words, 256))), dim3(256), 0, s, g);
  AM_RETURN_IF_LAUNCH_FAILED("gptq_unpack");
  if (logical) {
    hipLaunchKernelGGL(am::gptq_scales_kernel, dim3(static_cast<unsigned>(CeilDiv(a->n * g.groups, 256))), dim3(256), 0,
                       s, static_cast<const uint16_t*>(a->scales), a->n, g.groups, a->out_scales);
    AM_RETURN_IF_LAUNCH_FAILED("gptq_unpack");
  }
  return AM_STATUS_OK;
}

extern "C" am_status_code am_gfx950_dequant(const am_gfx950_dequant_args* a, void* stream) {
  AM_CHECK_ARG(a != nullptr && a->out != nullptr, "dequant: null args");
  const am_gfx950_weight& w = a->w;
  AM_CHECK_ARG(w.data != nullptr && w.n > 0 && w.k > 0 && w.n <= 0x7FFFFFFF, "dequant: bad weight");
  AM_CHECK_ARG(w.format >= AM_WF_F32 && w.format <= AM_WF_INT4, "dequant: unknown format");
  if (w.format >= AM_WF_INT8) AM_CHECK_ARG(w.scales != nullptr, "dequant: quantized weight needs scales");
  if (w.format == AM_WF_INT4)
    AM_CHECK_ARG(w.group_size > 0 && w.k % w.group_size == 0 && w.k % 8 == 0, "dequant: bad INT4 shape");
  hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<unsigned>(w.n)), dim3(256), 0, AsStream(stream), w.data,
                     w.scales, w.format, w.k, w.group_size, a->out);
  AM_RETURN_IF_LAUNCH_FAILED("dequant");
  return AM_STATUS_OK;
}
