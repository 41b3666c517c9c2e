// CPU ORACLE -- test infrastructure only.
// C entry point over the reference's own DotProductAvx2Unroll, which is compiled
// straight from /root/reference/src/backend/cpu/kernels/cpu_dot_product_avx2.cpp
// by oracle/Makefile into oracle/_ref/libref_dot.so.  Used to pin orc_dot_avx2.
#include <cstddef>

namespace aethermind {
float DotProductAvx2Unroll(const float* a, const float* b, std::size_t n) noexcept;
}

extern "C" float ref_dot_avx2(const float* a, const float* b, long n) {
  return aethermind::DotProductAvx2Unroll(a, b, static_cast<std::size_t>(n));
}
