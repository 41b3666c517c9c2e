// CPU ORACLE -- test infrastructure only (see oracle.h).
//
// Numeric conversions and the build's portable synthetic-data generator.
// Compiled with -ffp-contract=off: every a*b+c below is two roundings unless it is
// written as std::fma, so results are identical on any IEEE-754 host.

#include "oracle.h"

#include <cmath>
#include <cstring>

namespace {

inline uint32_t f2u(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
inline float u2f(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline uint64_t d2u(double d) {
  uint64_t u;
  std::memcpy(&u, &d, 8);
  return u;
}
inline double u2d(uint64_t u) {
  double d;
  std::memcpy(&d, &u, 8);
  return d;
}

}  // namespace

extern "C" {

// Reference: src/dtypes/bfloat16.cpp:20-32 -- RNE via rounding bias, NaN -> 0x7FC0.
uint16_t orc_f32_to_bf16(float v) {
  if (std::isnan(v)) return 0x7FC0u;
  const uint32_t x = f2u(v);
  const uint32_t bias = ((x >> 16) & 1u) + 0x7FFFu;
  return static_cast<uint16_t>((x + bias) >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return u2f(static_cast<uint32_t>(b) << 16); }

// IEEE binary16, round to nearest even, NaN -> 0x7E00 (sign kept).
uint16_t orc_f32_to_f16(float v) {
  const uint32_t x = f2u(v);
  const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;
  if (a >= 0x477FF000u) return sign | 0x7C00u;  // >= 65520 rounds to inf
  const int e = static_cast<int>(a >> 23) - 127;
  if (e < -14) {
    // subnormal half: value / 2^-24 = sig * 2^(e+1)
    if (a == 0) return sign;
    const uint32_t sig = (a & 0x7FFFFFu) | 0x800000u;
    const int sh = -(e + 1);
    if (sh > 24) return sign;
    const uint32_t q = sig >> sh;
    const uint32_t rem = sig & ((1u << sh) - 1u);
    const uint32_t halfway = 1u << (sh - 1);
    uint32_t r = q;
    if (rem > halfway || (rem == halfway && (q & 1u))) r += 1;
    return sign | static_cast<uint16_t>(r);  // r == 0x400 becomes the smallest normal
  }
  uint32_t h = (static_cast<uint32_t>(e + 15) << 10) | ((a & 0x7FFFFFu) >> 13);
  const uint32_t rem = a & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // may carry into exponent
  return sign | static_cast<uint16_t>(h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0) {
    // zero or subnormal: m * 2^-24, exact in fp32
    const float v = static_cast<float>(m) * 5.9604644775390625e-8f;
    return u2f(f2u(v) | sign);
  }
  if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

// ---- portable transcendental functions (fma/mul/add only) ----
// These are part of the synthetic-weight SPEC, not general-purpose math: the GPU
// generator evaluates the same operation sequence, so both produce the same bits.

static double recip_newton(double d) {  // d in [1.5, 2.5]
  double r = 0.5;
  for (int i = 0; i < 6; ++i) {
    const double e = std::fma(-d, r, 1.0);
    r = std::fma(r, e, r);
  }
  return r;
}

double orc_portable_log(double x) {  // x > 0, normal
  const uint64_t b = d2u(x);
  int e = static_cast<int>((b >> 52) & 0x7FF) - 1023;
  double m = u2d((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e += 1;
  }
  const double s = (m - 1.0) * recip_newton(m + 1.0);
  const double s2 = s * s;
  // 2*atanh(s) = 2*(s + s^3/3 + s^5/5 + ...)
  static const double c[] = {1.0 / 3,  1.0 / 5,  1.0 / 7,  1.0 / 9,  1.0 / 11,
                             1.0 / 13, 1.0 / 15, 1.0 / 17, 1.0 / 19, 1.0 / 21,
                             1.0 / 23, 1.0 / 25, 1.0 / 27};
  double p = c[12];
  for (int i = 11; i >= 0; --i) p = std::fma(p, s2, c[i]);
  const double lnm = 2.0 * std::fma(s * s2, p, s);
  return std::fma(static_cast<double>(e), 0.6931471805599453, lnm);
}

void orc_portable_sincos_turns(double turns, double* s_out, double* c_out) {  // turns in [0,1)
  const double t = turns * 4.0;
  int q = static_cast<int>(t);
  double f = t - static_cast<double>(q);
  bool swap = false;
  if (f > 0.5) {
    f = 1.0 - f;
    swap = true;
  }
  const double a = f * 1.5707963267948966;
  const double a2 = a * a;
  // sin: a - a^3/3! + ... ; cos: 1 - a^2/2! + ...
  static const double sc[] = {-1.0 / 6.0,
                              1.0 / 120.0,
                              -1.0 / 5040.0,
                              1.0 / 362880.0,
                              -1.0 / 39916800.0,
                              1.0 / 6227020800.0,
                              -1.0 / 1307674368000.0,
                              1.0 / 355687428096000.0,
                              -1.0 / 121645100408832000.0};
  static const double cc[] = {-1.0 / 2.0,
                              1.0 / 24.0,
                              -1.0 / 720.0,
                              1.0 / 40320.0,
                              -1.0 / 3628800.0,
                              1.0 / 479001600.0,
                              -1.0 / 87178291200.0,
                              1.0 / 20922789888000.0,
                              -1.0 / 6402373705728000.0};
  double ps = sc[8];
  double pc = cc[8];
  for (int i = 7; i >= 0; --i) {
    ps = std::fma(ps, a2, sc[i]);
    pc = std::fma(pc, a2, cc[i]);
  }
  double sv = std::fma(a * a2, ps, a);
  double cv = std::fma(a2, pc, 1.0);
  if (swap) {
    const double tmp = sv;
    sv = cv;
    cv = tmp;
  }
  switch (q & 3) {
    case 0: *s_out = sv; *c_out = cv; break;
    case 1: *s_out = cv; *c_out = -sv; break;
    case 2: *s_out = -sv; *c_out = -cv; break;
    default: *s_out = -cv; *c_out = sv; break;
  }
}

double orc_portable_sqrt(double x) {  // x >= 0, finite
  if (x == 0.0) return 0.0;
  const uint64_t b = d2u(x);
  int e = static_cast<int>((b >> 52) & 0x7FF) - 1023;
  double m = u2d((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);  // [1,2)
  if (e & 1) {
    m = m * 2.0;  // [2,4)
    e -= 1;
  }
  double y = std::fma(-0.1666666666666667, m - 1.0, 1.0);  // ~ 1/sqrt(m)
  const double h = 0.5 * m;
  for (int i = 0; i < 6; ++i) {
    const double hy = h * y;
    y = y * std::fma(-hy, y, 1.5);
  }
  const double r = m * y;
  return r * u2d(static_cast<uint64_t>(e / 2 + 1023) << 52);
}

// ---- synthetic generator (build SPEC) ----
uint64_t orc_splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t orc_tensor_key(uint64_t seed, uint64_t tensor_id) {
  return orc_splitmix64(orc_splitmix64(seed) ^ tensor_id);
}

static inline void box_muller_pair(uint64_t key, uint64_t p, double* z0, double* z1) {
  const uint64_t r = orc_splitmix64(key + p);
  const double u1 = static_cast<double>((r >> 32) + 1ull) * 2.3283064365386963e-10;  // (0,1]
  const double u2 = static_cast<double>(r & 0xFFFFFFFFull) * 2.3283064365386963e-10;  // [0,1)
  const double rad = orc_portable_sqrt(-2.0 * orc_portable_log(u1));
  double s, c;
  orc_portable_sincos_turns(u2, &s, &c);
  *z0 = rad * c;
  *z1 = rad * s;
}

void orc_synth_normal_f32(uint64_t seed, uint64_t tensor_id, double stddev, int64_t offset,
                          int64_t n, float* out) {
  const uint64_t key = orc_tensor_key(seed, tensor_id);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t idx = offset + i;
    double z0, z1;
    box_muller_pair(key, static_cast<uint64_t>(idx >> 1), &z0, &z1);
    const double z = (idx & 1) ? z1 : z0;
    out[i] = static_cast<float>(stddev * z);
  }
}

void orc_synth_normal_bf16(uint64_t seed, uint64_t tensor_id, double stddev, int64_t offset,
                           int64_t n, uint16_t* out) {
  const uint64_t key = orc_tensor_key(seed, tensor_id);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t idx = offset + i;
    double z0, z1;
    box_muller_pair(key, static_cast<uint64_t>(idx >> 1), &z0, &z1);
    const double z = (idx & 1) ? z1 : z0;
    out[i] = orc_f32_to_bf16(static_cast<float>(stddev * z));
  }
}

void orc_synth_token_ids(uint64_t seed, uint64_t stream, int64_t vocab, int64_t n, int64_t* out) {
  const uint64_t key = orc_tensor_key(seed, 0xF00D0000ull + stream);
  for (int64_t i = 0; i < n; ++i) {
    const uint64_t r = orc_splitmix64(key + static_cast<uint64_t>(i));
    out[i] = static_cast<int64_t>(((r >> 32) * static_cast<uint64_t>(vocab)) >> 32);
  }
}

}  // extern "C"
