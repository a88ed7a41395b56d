// Checks leo::fast_div (leo_amd/csrc/fast_div.h) against integer division for
// every divisor up to 5000, powers of two and their neighbours, and random
// divisors, each at the edge dividends (0, d-1, d, k*d-1, k*d, 2^31-1) and at
// random ones below 2^31. Exits non-zero on the first mismatch.
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "fast_div.h"

int main() {
    std::vector<uint32_t> divisors;
    for (uint32_t d = 1; d <= 5000; ++d) divisors.push_back(d);
    for (uint32_t k = 1; k < 31; ++k)
        for (int e = -1; e <= 1; ++e) divisors.push_back((1u << k) + e);
    divisors.push_back(0x7fffffffu);
    std::mt19937_64 rng(7);
    for (int i = 0; i < 3000; ++i) divisors.push_back(1 + static_cast<uint32_t>(rng() % 0x7fffffffu));
    uint64_t checked = 0;
    for (uint32_t d : divisors) {
        const leo::FastDiv f = leo::make_fast_div(d);
        std::vector<uint64_t> xs = {0, 1, d - 1ull, d, d + 1ull, 0x7ffffffeull, 0x7fffffffull};
        for (uint64_t k : {2ull, 3ull, 0x7fffffffull / d})
            for (uint64_t r : {0ull, d - 1ull}) xs.push_back(k * d + r);
        for (int i = 0; i < 300; ++i) xs.push_back(rng() % 0x80000000ull);
        for (uint64_t x : xs) {
            if (x >= 0x80000000ull) continue;
            const uint32_t got = leo::fast_div(static_cast<uint32_t>(x), f);
            const uint32_t want = static_cast<uint32_t>(x / d);
            ++checked;
            if (got != want) {
                std::printf("mismatch: %llu / %u = %u, fast_div gives %u\n", static_cast<unsigned long long>(x), d, want, got);
                return 1;
            }
        }
    }
    std::printf("checked %llu divisions\n", static_cast<unsigned long long>(checked));
    return 0;
}
