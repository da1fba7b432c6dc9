// Division of a non-negative int32 by a runtime constant d >= 1 with one
// mul-hi, one add and one shift: the round-up multiplier method
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", 1994), valid for numerators below 2^31.
// Self-contained so host tests can compile it with a plain C++ compiler.
#pragma once

#include <stdint.h>

#if defined(__HIP__) || defined(__HIPCC__)
#define QSA_HD __host__ __device__
#else
#define QSA_HD
#endif

namespace qsa {

struct FastDiv {
  uint32_t mul;
  uint32_t shift;
  int32_t divisor;

  static FastDiv make(int32_t d) {
    FastDiv f;
    f.divisor = d;
    uint32_t l = 0;
    while (l < 31 && (1u << l) < (uint32_t)d) ++l;
    const uint64_t num = ((uint64_t)1 << 32) * (((uint64_t)1 << l) - (uint64_t)d);
    f.mul = (uint32_t)(num / (uint64_t)d + 1);
    f.shift = l;
    return f;
  }

  QSA_HD inline int32_t div(int32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t hi = __umulhi((uint32_t)n, mul);
#else
    const uint32_t hi = (uint32_t)(((uint64_t)(uint32_t)n * mul) >> 32);
#endif
    return (int32_t)((hi + (uint32_t)n) >> shift);
  }
};

}  // namespace qsa
