// Division by a runtime divisor fixed for a launch (synapse count, block size),
// as a multiply and a shift. Plain C++ so that the host test compiles the same
// code the kernels run.
#ifndef LEO_FAST_DIV_H
#define LEO_FAST_DIV_H

#include <stdint.h>

#if defined(__HIPCC__)
#define LEO_HOST_DEVICE __host__ __device__
#else
#define LEO_HOST_DEVICE
#endif

namespace leo {

// x / d for every x < 2^31 by one 32x32->64-bit multiply and a shift: with
// l = ceil(log2 d) and m = ceil(2^(31+l) / d) < 2^32, the error
// e = m*d - 2^(31+l) is below d <= 2^l, so x*m / 2^(31+l) = x/d + x*e/(d*2^(31+l))
// exceeds x/d by less than 1/d and its floor is floor(x/d).
struct FastDiv {
    uint32_t d, m, shift;
};

inline FastDiv make_fast_div(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const unsigned long long m = ((1ull << (31 + l)) + d - 1) / d;
    return FastDiv{d, static_cast<uint32_t>(m), 31 + l};
}

LEO_HOST_DEVICE inline uint32_t fast_div(uint32_t x, const FastDiv& f) {
    return static_cast<uint32_t>((static_cast<unsigned long long>(x) * f.m) >> f.shift);
}

}  // namespace leo

#endif
