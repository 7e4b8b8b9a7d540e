// fast_div.hpp -- unsigned 32-bit division by a divisor fixed for a whole launch,
// as one high multiply, an add and a shift instead of a division sequence.
//
// The method is Granlund and Montgomery, "Division by Invariant Integers using
// Multiplication" (PLDI 1994), section 4: for a divisor 1 <= d <= 2^31 take
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1 (which fits 32 bits);
// then for 0 <= n < 2^31, n / d = (mulhi(m, n) + n) >> l, where the sum stays
// below 2^32 because mulhi(m, n) <= n.  The host builds the pair once per launch.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define MCKE_HD __host__ __device__
#else
#define MCKE_HD
#endif

namespace mcke_amd {

struct FastDivU32 {
  std::uint32_t m = 1;   // multiplier
  std::uint32_t l = 0;   // shift

  // d in [1, 2^31]; the caller checks the range.
  static FastDivU32 make(std::uint32_t d) {
    FastDivU32 f;
    std::uint32_t l = 0;
    while ((std::uint64_t{1} << l) < d) ++l;
    f.l = l;
    f.m = static_cast<std::uint32_t>(
        ((std::uint64_t{1} << 32) * ((std::uint64_t{1} << l) - d)) / d + 1);
    return f;
  }

  // n / d for 0 <= n < 2^31.
  MCKE_HD std::uint32_t div(std::uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const std::uint32_t t = __umulhi(m, n);
#else
    const std::uint32_t t = static_cast<std::uint32_t>((static_cast<std::uint64_t>(m) * n) >> 32);
#endif
    return (t + n) >> l;
  }
};

}  // namespace mcke_amd
