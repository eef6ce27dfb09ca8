// Host check of the launch-size limits every kernel launch goes through
// (dispatch_fits / grid_for, mimir-framework_amd/csrc/rows.hpp): at most
// 2^31 - 1 workgroups per grid dimension, and fewer than 2^32 work-items
// (workgroups x threads), which the dispatch packet holds in 32 bits.
#include <cstdio>
#include <initializer_list>

#include "../../mimir-framework_amd/csrc/rows.hpp"

static int failures = 0;

static void expect(bool got, bool want, const char* what, long long a, long long b) {
    if (got != want) {
        std::printf("FAIL %s(%lld, %lld): got %d want %d\n", what, a, b, got, want);
        ++failures;
    }
}

int main() {
    using mimir::dispatch_fits;
    using mimir::grid_for;
    const long long big = 0x7fffffffLL;
    // Workgroup-count limit (threads = 1 leaves only that one).
    expect(dispatch_fits(big, 1), true, "dispatch_fits", big, 1);
    expect(dispatch_fits(big + 1, 1), false, "dispatch_fits", big + 1, 1);
    expect(dispatch_fits(0, 256), false, "dispatch_fits", 0, 256);
    expect(dispatch_fits(-1, 256), false, "dispatch_fits", -1, 256);
    // Work-item limit: blocks * threads < 2^32.
    for (long long t : {64LL, 256LL, 512LL, 1024LL}) {
        const long long last = 0xffffffffLL / t;  // the largest grid of t-thread workgroups
        expect(dispatch_fits(last, t), true, "dispatch_fits", last, t);
        expect(dispatch_fits(last + 1, t), false, "dispatch_fits", last + 1, t);
    }
    expect(dispatch_fits(big, 2), true, "dispatch_fits", big, 2);    // 2^32 - 2 work-items
    expect(dispatch_fits(big, 3), false, "dispatch_fits", big, 3);
    // grid_for rounds units up to whole workgroups before the check.
    unsigned b = 0;
    expect(grid_for(1, 4, 256, &b) && b == 1, true, "grid_for", 1, 4);
    expect(grid_for(4097, 4096, 1024, &b) && b == 2, true, "grid_for", 4097, 4096);
    expect(grid_for(0, 4, 256, &b), false, "grid_for", 0, 4);
    const long long units = (0xffffffffLL / 1024) * 4;  // 4 rows per 1024-thread workgroup
    expect(grid_for(units, 4, 1024, &b) && b == 0xffffffffLL / 1024, true, "grid_for", units, 4);
    expect(grid_for(units + 1, 4, 1024, &b), false, "grid_for", units + 1, 4);
    std::printf("dispatch limits: %d failures\n", failures);
    return failures ? 1 : 0;
}
