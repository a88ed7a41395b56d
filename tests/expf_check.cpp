// Compares leo::glibc_expf_nonpositive (the device restatement of glibc's expf)
// with the host's expf for every float in [lo, 0] (walked by bit pattern), and
// for the special inputs. Prints the first mismatch and exits non-zero on any.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "glibc_expf.h"

static uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
static float from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

int main(int argc, char** argv) {
    const uint32_t stride = argc > 1 ? static_cast<uint32_t>(std::strtoul(argv[1], nullptr, 10)) : 1u;
    const float lo = -0x1.9fe368p6f;  // below this both return +0
    uint64_t checked = 0;
    // -0.0 up to the most negative input of the domain: patterns 0x80000000 .. bits(lo)
    for (uint64_t u = 0x80000000u; u <= bits(lo); u += stride) {
        const float x = from_bits(static_cast<uint32_t>(u));
        const float want = expf(x), got = leo::glibc_expf_nonpositive(x);
        if (bits(want) != bits(got)) {
            std::printf("mismatch at x=%a: glibc %a, restatement %a\n", x, want, got);
            return 1;
        }
        ++checked;
    }
    const float specials[] = {0.0f, -0.0f, -1.0f, -0x1p-149f, -88.72283f, -87.33655f, -103.0f, -103.972077f,
                              lo, std::nextafter(lo, 0.0f), std::nextafter(lo, -1.0f), -200.0f, -INFINITY};
    for (float x : specials) {
        const float want = expf(x), got = leo::glibc_expf_nonpositive(x);
        if (bits(want) != bits(got)) {
            std::printf("mismatch at special x=%a: glibc %a, restatement %a\n", x, want, got);
            return 1;
        }
    }
    std::printf("checked %llu inputs\n", static_cast<unsigned long long>(checked));
    return 0;
}
