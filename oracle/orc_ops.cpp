// CPU ORACLE -- test infrastructure only (see oracle.h).
//
// Per-op restatements of the reference CPU semantics and of the build SPEC for the
// ops the reference left unimplemented.  Compiled with -O3 -mavx2 -mfma
// -ffp-contract=off.

#include "oracle.h"

#include <immintrin.h>

#include <cmath>
#include <cstring>
#include <vector>

namespace {

inline float hsum256(__m256 v) {
  // Same reduction tree as the reference HorizontalSumAvx2
  // (src/backend/cpu/kernels/common/cpu_simd_utils.h).
  const __m128 lo = _mm256_castps256_ps128(v);
  const __m128 hi = _mm256_extractf128_ps(v, 1);
  __m128 s = _mm_add_ps(lo, hi);
  s = _mm_hadd_ps(s, s);
  s = _mm_hadd_ps(s, s);
  return _mm_cvtss_f32(s);
}

inline float round_bf16(float v) { return orc_bf16_to_f32(orc_f32_to_bf16(v)); }

}  // namespace

extern "C" {

// ---------------- quantization (build SPEC) ----------------
// INT8: symmetric per output channel, s = max|w| / 127 (fp32), s = 1 for an all-zero
// row, q = clamp(rint(w / s), -127, 127).
int orc_quant_int8(const float* w, int64_t n, int64_t k, int8_t* q, float* scales) {
  if (n <= 0 || k <= 0) return 3;
  for (int64_t r = 0; r < n; ++r) {
    const float* row = w + r * k;
    float amax = 0.0f;
    for (int64_t j = 0; j < k; ++j) amax = std::fmax(amax, std::fabs(row[j]));
    const float s = amax == 0.0f ? 1.0f : amax / 127.0f;
    scales[r] = s;
    for (int64_t j = 0; j < k; ++j) {
      float v = std::nearbyint(row[j] / s);
      v = std::fmin(127.0f, std::fmax(-127.0f, v));
      q[r * k + j] = static_cast<int8_t>(v);
    }
  }
  return 0;
}

int orc_dequant_int8(const int8_t* q, const float* scales, int64_t n, int64_t k, float* w) {
  for (int64_t r = 0; r < n; ++r)
    for (int64_t j = 0; j < k; ++j) w[r * k + j] = static_cast<float>(q[r * k + j]) * scales[r];
  return 0;
}

// INT4: symmetric groups of `group` along K, fp16 scale s = f16(max|w| / 7),
// q = clamp(rint(w / s), -8, 7) (q = 0 when s == 0), no zero point.
// Logical packing: byte i of a row = (q[2i] & 0xF) | (q[2i+1] << 4).
int orc_quant_int4(const float* w, int64_t n, int64_t k, int64_t group, uint8_t* packed,
                   uint16_t* scales_f16) {
  if (n <= 0 || k <= 0 || group <= 0 || k % group != 0 || group % 2 != 0) return 3;
  const int64_t ng = k / group;
  std::vector<int8_t> qrow(static_cast<size_t>(k));
  for (int64_t r = 0; r < n; ++r) {
    const float* row = w + r * k;
    for (int64_t g = 0; g < ng; ++g) {
      float amax = 0.0f;
      for (int64_t j = 0; j < group; ++j) amax = std::fmax(amax, std::fabs(row[g * group + j]));
      const uint16_t s16 = orc_f32_to_f16(amax / 7.0f);
      const float s = orc_f16_to_f32(s16);
      scales_f16[r * ng + g] = s16;
      for (int64_t j = 0; j < group; ++j) {
        float v = 0.0f;
        if (s != 0.0f) {
          v = std::nearbyint(row[g * group + j] / s);
          v = std::fmin(7.0f, std::fmax(-8.0f, v));
        }
        qrow[static_cast<size_t>(g * group + j)] = static_cast<int8_t>(v);
      }
    }
    for (int64_t i = 0; i < k / 2; ++i) {
      const uint8_t lo = static_cast<uint8_t>(qrow[static_cast<size_t>(2 * i)]) & 0xFu;
      const uint8_t hi = static_cast<uint8_t>(qrow[static_cast<size_t>(2 * i + 1)]) & 0xFu;
      packed[r * (k / 2) + i] = static_cast<uint8_t>(lo | (hi << 4));
    }
  }
  return 0;
}

int orc_dequant_int4(const uint8_t* packed, const uint16_t* scales_f16, int64_t n, int64_t k,
                     int64_t group, float* w) {
  if (k % group != 0 || group % 2 != 0) return 3;
  const int64_t ng = k / group;
  for (int64_t r = 0; r < n; ++r) {
    for (int64_t j = 0; j < k; ++j) {
      const uint8_t b = packed[r * (k / 2) + j / 2];
      int nib = (j & 1) ? (b >> 4) : (b & 0xF);
      if (nib >= 8) nib -= 16;
      const float s = orc_f16_to_f32(scales_f16[r * ng + j / group]);
      w[r * k + j] = static_cast<float>(nib) * s;
    }
  }
  return 0;
}

// ---------------- ops ----------------
// Reference: src/backend/cpu/kernels/embedding/embedding_entry.cpp:32-126.
// Returns 11 (AM_STATUS_OUT_OF_RANGE) for an id outside [0, vocab).
int orc_embedding_i64(const int64_t* ids, int64_t n_tokens, const float* table, int64_t vocab,
                      int64_t hidden, float* out) {
  if (vocab <= 0 || hidden <= 0) return 3;
  for (int64_t t = 0; t < n_tokens; ++t) {
    const int64_t id = ids[t];
    if (id < 0 || id >= vocab) return 11;
    std::memcpy(out + t * hidden, table + id * hidden, sizeof(float) * static_cast<size_t>(hidden));
  }
  return 0;
}

// Reference: src/backend/cpu/kernels/rmsnorm/rmsnorm_fp32_scalar.cpp:10-31
// (double accumulation, y = x * inv_rms * w evaluated in double, rounded once).
int orc_rmsnorm_scalar(const float* x, const float* w, int64_t rows, int64_t hidden, float eps,
                       float* out) {
  if (rows < 0 || hidden <= 0 || !(eps > 0.0f)) return 3;
  for (int64_t r = 0; r < rows; ++r) {
    const float* in = x + r * hidden;
    double sum_sq = 0.0;
    for (int64_t j = 0; j < hidden; ++j) {
      const double v = static_cast<double>(in[j]);
      sum_sq += v * v;
    }
    const double mean_sq = sum_sq / static_cast<double>(hidden);
    const double inv_rms = 1.0 / std::sqrt(mean_sq + static_cast<double>(eps));
    for (int64_t j = 0; j < hidden; ++j)
      out[r * hidden + j] =
          static_cast<float>(static_cast<double>(in[j]) * inv_rms * static_cast<double>(w[j]));
  }
  return 0;
}

// Reference: src/backend/cpu/kernels/rmsnorm/rmsnorm_fp32_avx2.cpp:15-91.
int orc_rmsnorm_avx2(const float* x, const float* w, int64_t rows, int64_t hidden, float eps,
                     float* out) {
  if (rows < 0 || hidden <= 0 || !(eps > 0.0f)) return 3;
  for (int64_t r = 0; r < rows; ++r) {
    const float* input = x + r * hidden;
    float* output = out + r * hidden;
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
    int64_t j = 0;
    for (; j + 32 <= hidden; j += 32) {
      const __m256 a = _mm256_loadu_ps(input + j), b = _mm256_loadu_ps(input + j + 8);
      const __m256 c = _mm256_loadu_ps(input + j + 16), d = _mm256_loadu_ps(input + j + 24);
      s0 = _mm256_fmadd_ps(a, a, s0);
      s1 = _mm256_fmadd_ps(b, b, s1);
      s2 = _mm256_fmadd_ps(c, c, s2);
      s3 = _mm256_fmadd_ps(d, d, s3);
    }
    __m256 acc = _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3));
    for (; j + 8 <= hidden; j += 8) {
      const __m256 a = _mm256_loadu_ps(input + j);
      acc = _mm256_fmadd_ps(a, a, acc);
    }
    float sum_sq = hsum256(acc);
    for (; j < hidden; ++j) sum_sq += input[j] * input[j];
    const float mean_sq = sum_sq / static_cast<float>(hidden);
    const float inv_rms = 1.0f / std::sqrt(mean_sq + eps);
    const __m256 vinv = _mm256_set1_ps(inv_rms);
    j = 0;
    for (; j + 8 <= hidden; j += 8) {
      const __m256 a = _mm256_mul_ps(_mm256_loadu_ps(input + j), vinv);
      _mm256_storeu_ps(output + j, _mm256_mul_ps(a, _mm256_loadu_ps(w + j)));
    }
    for (; j < hidden; ++j) output[j] = input[j] * inv_rms * w[j];
  }
  return 0;
}

// Reference: src/backend/cpu/kernels/cpu_dot_product_avx2.cpp:8-40.
float orc_dot_avx2(const float* a, const float* b, int64_t n) {
  __m256 v0 = _mm256_setzero_ps(), v1 = _mm256_setzero_ps();
  __m256 v2 = _mm256_setzero_ps(), v3 = _mm256_setzero_ps();
  int64_t i = 0;
  for (; i + 32 <= n; i += 32) {
    v0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), v0);
    v1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), v1);
    v2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), v2);
    v3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), v3);
  }
  __m256 acc = _mm256_add_ps(_mm256_add_ps(v0, v1), _mm256_add_ps(v2, v3));
  for (; i + 8 <= n; i += 8)
    acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
  float result = hsum256(acc);
  for (; i < n; ++i) result += a[i] * b[i];
  return result;
}

// Reference GEMM loop (docs/designs/kernel_dev/LinearOp...v1.0.md:415-437):
// out[m,n] = sum_k x[m,k] * w[n,k], W row-major [out, in].  The oracle accumulates
// in double so it is the accuracy yardstick for the GPU's fp32 accumulation.
void orc_linear(const float* x, const float* w, int64_t m, int64_t n, int64_t k, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < n; ++c) {
    const float* wr = w + c * k;
    for (int64_t r = 0; r < m; ++r) {
      const float* xr = x + r * k;
      double acc = 0.0;
      for (int64_t j = 0; j < k; ++j) acc += static_cast<double>(xr[j]) * static_cast<double>(wr[j]);
      out[r * n + c] = static_cast<float>(acc);
    }
  }
}

// Same loop with the reference's AVX2 dot product as the inner kernel (fp32).
void orc_linear_avx2(const float* x, const float* w, int64_t m, int64_t n, int64_t k, float* out) {
  for (int64_t r = 0; r < m; ++r)
    for (int64_t c = 0; c < n; ++c) out[r * n + c] = orc_dot_avx2(x + r * k, w + c * k, k);
}

// Reference RoPE design (RoPEOp...v1.0.md:588-622): inv_freq_i = 1/theta^(2i/d) in
// double, cos/sin in double cast to float; split-half rotation in fp32.
void orc_rope_table(int64_t max_pos, int64_t head_dim, double theta, float* cos_tab,
                    float* sin_tab) {
  const int64_t half = head_dim / 2;
  for (int64_t p = 0; p < max_pos; ++p) {
    for (int64_t i = 0; i < half; ++i) {
      const double exponent = 2.0 * static_cast<double>(i) / static_cast<double>(head_dim);
      const double inv_freq = 1.0 / std::pow(theta, exponent);
      const double angle = static_cast<double>(p) * inv_freq;
      cos_tab[p * half + i] = static_cast<float>(std::cos(angle));
      sin_tab[p * half + i] = static_cast<float>(std::sin(angle));
    }
  }
}

void orc_rope(float* x, int64_t seq, int64_t heads, int64_t head_dim, const int64_t* pos,
              const float* cos_tab, const float* sin_tab) {
  const int64_t half = head_dim / 2;
  for (int64_t s = 0; s < seq; ++s) {
    const float* c = cos_tab + pos[s] * half;
    const float* sn = sin_tab + pos[s] * half;
    for (int64_t h = 0; h < heads; ++h) {
      float* v = x + (s * heads + h) * head_dim;
      for (int64_t i = 0; i < half; ++i) {
        const float x1 = v[i];
        const float x2 = v[i + half];
        v[i] = x1 * c[i] - x2 * sn[i];
        v[i + half] = x2 * c[i] + x1 * sn[i];
      }
    }
  }
}

// GQA causal scaled-dot-product attention over one layer's cache planes
// kc/vc [hkv][cap][d]; query s sits at position start_pos + s and sees keys
// [0, start_pos + s].  q head h reads kv head h / (hq / hkv).  fp64 softmax.
void orc_attention(const float* q, const float* kc, const float* vc, int64_t seq, int64_t hq,
                   int64_t hkv, int64_t head_dim, int64_t cap, int64_t start_pos, float* out) {
  const int64_t group = hq / hkv;
  const double scale = 1.0 / std::sqrt(static_cast<double>(head_dim));
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t s = 0; s < seq; ++s) {
    for (int64_t h = 0; h < hq; ++h) {
      const int64_t g = h / group;
      const int64_t n_keys = start_pos + s + 1;
      const float* qv = q + (s * hq + h) * head_dim;
      std::vector<double> sc(static_cast<size_t>(n_keys));
      double mx = -INFINITY;
      for (int64_t p = 0; p < n_keys; ++p) {
        const float* kv = kc + (g * cap + p) * head_dim;
        double d = 0.0;
        for (int64_t i = 0; i < head_dim; ++i) d += static_cast<double>(qv[i]) * kv[i];
        sc[static_cast<size_t>(p)] = d * scale;
        mx = std::fmax(mx, sc[static_cast<size_t>(p)]);
      }
      double denom = 0.0;
      for (int64_t p = 0; p < n_keys; ++p) {
        sc[static_cast<size_t>(p)] = std::exp(sc[static_cast<size_t>(p)] - mx);
        denom += sc[static_cast<size_t>(p)];
      }
      float* o = out + (s * hq + h) * head_dim;
      for (int64_t i = 0; i < head_dim; ++i) {
        double acc = 0.0;
        for (int64_t p = 0; p < n_keys; ++p)
          acc += sc[static_cast<size_t>(p)] * static_cast<double>(vc[(g * cap + p) * head_dim + i]);
        o[i] = static_cast<float>(acc / denom);
      }
    }
  }
}

// Reference: src/graph/optimization/const_eval_silu_mul.cpp:18-31.
void orc_silu_mul(const float* gate, const float* up, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    const float u = up[i];
    float silu;
    if (g >= 0.0f) {
      silu = g / (1.0f + std::exp(-g));
    } else {
      const float e = std::exp(g);
      silu = g * e / (1.0f + e);
    }
    out[i] = silu * u;
  }
}

// Build SPEC: first (lowest) index among equal maxima; NaN never selected; all-NaN
// or empty input -> 0.
int64_t orc_argmax(const float* x, int64_t n) {
  int64_t best = -1;
  for (int64_t i = 0; i < n; ++i) {
    if (std::isnan(x[i])) continue;
    if (best < 0 || x[i] > x[best]) best = i;
  }
  return best < 0 ? 0 : best;
}

void orc_round_bf16_inplace(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = round_bf16(x[i]);
}

}  // extern "C"
