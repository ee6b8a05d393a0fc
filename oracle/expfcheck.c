/* Exhaustive comparison of ws_expf (weightstream_amd/csrc/ws_expf.h) with the
 * host libm expf over every 32-bit pattern in [lo, hi). Test infrastructure:
 * called by tests/test_oracle_expf.py. Also folds glibc's results into an
 * order-independent checksum that the GPU test compares its device results
 * against. */
#include <math.h>
#include <stdint.h>
#include "../weightstream_amd/csrc/ws_expf.h"

/* Returns the number of mismatching inputs; NaN results compare equal. */
uint64_t ws_expf_mismatches(uint64_t lo, uint64_t hi) {
    uint64_t mism = 0;
#pragma omp parallel for reduction(+ : mism) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        float x = ws_u2f((uint32_t)u);
        float a = expf(x), b = ws_expf(x);
        if (ws_f2u(a) != ws_f2u(b) && !(a != a && b != b)) mism++;
    }
    return mism;
}

/* sum over u in [lo,hi) of mix(u, bits(expf(u))) mod 2^64, NaNs canonical */
static inline uint64_t mix(uint64_t u, uint32_t r) {
    uint64_t z = (u << 32) ^ r;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
uint64_t glibc_expf_checksum(uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
#pragma omp parallel for reduction(+ : acc) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        float r = expf(ws_u2f((uint32_t)u));
        uint32_t b = (r != r) ? 0x7fc00000u : ws_f2u(r);
        acc += mix((uint64_t)u, b);
    }
    return acc;
}
