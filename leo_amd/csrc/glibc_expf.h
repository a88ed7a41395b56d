// Bit-exact restatement of glibc's expf (the FMA build that glibc >= 2.27
// dispatches on x86_64 CPUs with FMA). Rust's f32::exp -- and so Leo's CPU
// softmax (runtime.rs:1169-1188) -- calls this function, so the device
// softmax must reproduce it bit for bit.
//
// Algorithm: ARM optimized-routines math/expf.c (MIT / Apache-2.0), as
// shipped in glibc sysdeps/ieee754/flt-32/e_expf.c with e_exp2f_data.c:
//   x*N/ln2 = k + r, r in [-1/2, 1/2], N = 32
//   exp(x) = 2^(k/N) * 2^(r/N) ~= s * (C0*r^3 + C1*r^2 + C2*r + 1)
// evaluated in double precision, with the FMA contractions the FMA build
// uses. Table entries are tab[i] = bits(2^(i/32)) - (i << 47).
//
// Domain: the softmax only evaluates x = logit - max <= 0. Inputs below
// log(2^-150) return +0 exactly as glibc does; x > 0 is not supported here.
// tests/test_glibc_expf.py checks this function against the host glibc over
// the whole domain [-103.97, 0].
#ifndef LEO_GLIBC_EXPF_H
#define LEO_GLIBC_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define LEO_HD __host__ __device__
#else
#define LEO_HD
#include <cmath>
#endif

namespace leo {

// 2^(i/32) table (glibc e_exp2f_data.c, N = 32).
static constexpr uint64_t kExp2fTab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

LEO_HD inline double expf_bits_to_double(uint64_t u) {
    union {
        uint64_t u;
        double d;
    } v;
    v.u = u;
    return v.d;
}
LEO_HD inline uint64_t expf_double_to_bits(double d) {
    union {
        uint64_t u;
        double d;
    } v;
    v.d = d;
    return v.u;
}

LEO_HD inline float glibc_expf_nonpositive(float x) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    if (x < -0x1.9fe368p6f) return 0.0f;  // below log(2^-150): underflow to +0
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    const uint64_t ki = expf_double_to_bits(kd);
    kd -= kShift;
    const double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = kExp2fTab[ki % 32];
    t += ki << 47;
    const double s = expf_bits_to_double(t);
    double z = __builtin_fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

}  // namespace leo

#endif
