// Host-side check of FastDiv (prologue_kernels.h), the multiply-shift
// division of the prologue's row addressing: every divisor 1 .. 70000 and
// the divisors next to powers of two up to 2^30, against n / d for the
// numerators at and around every multiple boundary reached by a stride
// sweep, 0, 1 and 2^31 - 1.  Built and run by tests/test_geometry.py;
// prints "ok <cases>".
#include <cstdint>
#include <cstdio>
#include <vector>

#include "prologue_kernels.h"

static bool check(uint32_t d, uint32_t n, long long* cases) {
    ++*cases;
    const mft::FastDiv f = mft::FastDiv::make(d);
    if (f.div(n) != n / d) {
        std::printf("BAD d=%u n=%u got %u want %u\n", d, n, f.div(n), n / d);
        return false;
    }
    return true;
}

int main() {
    std::vector<uint32_t> ds;
    for (uint32_t d = 1; d <= 70000; ++d) ds.push_back(d);
    for (int l = 17; l <= 30; ++l)
        for (int k = -3; k <= 3; ++k) ds.push_back((uint32_t)((1u << l) + k));
    long long cases = 0;
    const uint32_t top = 0x7FFFFFFFu;
    for (uint32_t d : ds) {
        const uint32_t ns[] = {0u, 1u, d - 1, d, d + 1, top, top - 1, top - d, top / d * d, top / d * d - 1};
        for (uint32_t n : ns)
            if (n <= top && !check(d, n, &cases)) return 1;
        // multiples of d spread over [0, 2^31), and their neighbours
        const uint64_t step = (uint64_t)top / 97 / d * d + d;
        for (uint64_t n = d; n <= top; n += step)
            for (int k = -1; k <= 1; ++k)
                if (n + k <= top && !check(d, (uint32_t)(n + k), &cases)) return 1;
    }
    std::printf("ok %lld\n", cases);
    return 0;
}
