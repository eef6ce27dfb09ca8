// fastdiv.hpp -- unsigned 32-bit division by a divisor fixed for a launch,
// as a multiply-high, an add and two shifts (Granlund and Montgomery,
// "Division by Invariant Integers using Multiplication", PLDI 1994, Fig. 4.1):
//   l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
//   q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0),  t = mulhi(m, n),
// exact for every 0 <= n < 2^32 and 1 <= d < 2^32.  The divisor is prepared
// on the host; the kernels divide with fastdiv().  Plain C++ (no HIP types),
// so host tests compile it with g++.
#pragma once

#include <stdint.h>

#if defined(__HIP__) || defined(__HIPCC__)
#define MIMIR_HD __host__ __device__
#else
#define MIMIR_HD
#endif

namespace mimir {

struct FastDiv {
    uint32_t d;   // the divisor
    uint32_t m;   // the multiplier
    uint32_t s1;  // min(l, 1)
    uint32_t s2;  // max(l - 1, 0)
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while (l < 32 && (uint64_t(1) << l) < d) ++l;  // ceil(log2 d); d = 0 is the caller's error
    const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / (d ? d : 1) + 1;
    return FastDiv{d, static_cast<uint32_t>(m), l < 1 ? l : 1u, l > 1 ? l - 1 : 0u};
}

MIMIR_HD inline uint32_t fastdiv(uint32_t n, const FastDiv& f) {
    const uint32_t t = static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> 32);
    return (t + ((n - t) >> f.s1)) >> f.s2;
}

MIMIR_HD inline uint32_t fastmod(uint32_t n, const FastDiv& f) { return n - fastdiv(n, f) * f.d; }

}  // namespace mimir
