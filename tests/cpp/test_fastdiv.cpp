// Host check of fastdiv.hpp against the hardware division: every divisor up
// to 2^16 and sampled ones above, each with the dividends where a wrong
// multiplier or shift shows (0, 1, multiples of d and their neighbours, the
// top of the range) plus pseudo-random ones.
#include <cstdint>
#include <cstdio>
#include <initializer_list>

#include "../../mimir-framework_amd/csrc/fastdiv.hpp"

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint32_t next32() {  // splitmix64
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return static_cast<uint32_t>(z ^ (z >> 31));
}

static long failures = 0, checks = 0;
static void check(uint32_t n, const mimir::FastDiv& f) {
    ++checks;
    if (mimir::fastdiv(n, f) != n / f.d || mimir::fastmod(n, f) != n % f.d) {
        if (failures++ < 10) std::printf("mismatch: %u / %u\n", n, f.d);
    }
}

static void divisor(uint32_t d) {
    const mimir::FastDiv f = mimir::make_fastdiv(d);
    const uint32_t edges[] = {0u, 1u, 2u, d - 1u, d, d + 1u, 2u * d - 1u, 2u * d, 0x7fffffffu, 0x80000000u,
                              0xfffffffeu, 0xffffffffu};
    for (uint32_t n : edges) check(n, f);
    const uint32_t q = 0xffffffffu / d;
    for (uint32_t k : {q, q - 1u, q / 2u, q / 3u + 1u})
        for (int64_t delta = -1; delta <= 1; ++delta) check(static_cast<uint32_t>(int64_t(k) * d + delta), f);
    for (int i = 0; i < 64; ++i) check(next32(), f);
}

int main() {
    for (uint32_t d = 1; d <= 65536; ++d) divisor(d);
    for (int i = 0; i < 200000; ++i) divisor(next32() | 1u);
    for (uint32_t s = 16; s < 32; ++s) {
        divisor(1u << s);
        divisor((1u << s) - 1u);
        divisor((1u << s) + 1u);
    }
    divisor(0xffffffffu);
    std::printf("%ld checks, %ld failures\n", checks, failures);
    return failures ? 1 : 0;
}
