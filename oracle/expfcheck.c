/* Exhaustive comparison of ws_expf (weightstream_amd/csrc/ws_expf.h) with the
 * host libm expf over every 32-bit pattern in [lo, hi). Test infrastructure:
 * called by tests/test_oracle_expf.py and tests/test_gpu_route.py (glibc's
 * results, raw or folded into a digest, are what the device ws_expf is
 * compared against). */
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

/* glibc expf bits for the 32-bit patterns [lo, lo+n) (NaNs canonical). */
void glibc_expf_bits(uint32_t lo, uint32_t n, uint32_t *out) {
#pragma omp parallel for schedule(static, 1 << 16)
    for (long long i = 0; i < (long long)n; i++) {
        float r = expf(ws_u2f(lo + (uint32_t)i));
        out[i] = (r != r) ? 0x7fc00000u : ws_f2u(r);
    }
}

/* sum over u in [lo,hi) of (bits(expf(u)) ^ (u * 0x9E3779B1)) * (2u+1) mod
 * 2^64, NaNs canonical: an order-independent digest that a GPU can compute
 * with wrapping int64 arithmetic. */
uint64_t glibc_expf_digest(uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
#pragma omp parallel for reduction(+ : acc) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        float r = expf(ws_u2f((uint32_t)u));
        uint32_t b = (r != r) ? 0x7fc00000u : ws_f2u(r);
        acc += (uint64_t)(b ^ (uint32_t)((uint32_t)u * 0x9E3779B1u)) * (2 * (uint64_t)u + 1);
    }
    return acc;
}

/* ---- logf (weightstream_amd/csrc/ws_logf.h) and the sqrtsoftplus score ---- */
#include "../weightstream_amd/csrc/ws_logf.h"

/* glibc sqrt(softplus(x)) in weightstream-ref num.rs:82-88 order */
static float ref_sqrtsoftplus(float x) {
    float sp = x > 20.0f ? x : logf(1.0f + expf(x));
    return sqrtf(sp);
}

/* fn 0: logf; fn 1: sqrtsoftplus score. Host library result for x. */
static float ref_fn(int fn, float x) { return fn == 0 ? logf(x) : ref_sqrtsoftplus(x); }

/* Mismatches of ws_logf (fn 0) or sqrtf(ws_softplus) (fn 1) against glibc over
 * the 32-bit patterns [lo, hi); NaN results compare equal. */
uint64_t ws_math_mismatches(int fn, uint64_t lo, uint64_t hi) {
    uint64_t mism = 0;
#pragma omp parallel for reduction(+ : mism) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        float x = ws_u2f((uint32_t)u);
        float a = ref_fn(fn, x);
        float b = fn == 0 ? ws_logf(x) : sqrtf(ws_softplus(x));
        if (ws_f2u(a) != ws_f2u(b) && !(a != a && b != b)) mism++;
    }
    return mism;
}

/* Digest of the host library's fn results, as glibc_expf_digest. */
uint64_t glibc_math_digest(int fn, uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
#pragma omp parallel for reduction(+ : acc) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++) {
        float r = ref_fn(fn, ws_u2f((uint32_t)u));
        uint32_t b = (r != r) ? 0x7fc00000u : ws_f2u(r);
        acc += (uint64_t)(b ^ (uint32_t)((uint32_t)u * 0x9E3779B1u)) * (2 * (uint64_t)u + 1);
    }
    return acc;
}

/* Host library results for [lo, lo+n) (NaNs canonical). */
void glibc_math_bits(int fn, uint32_t lo, uint32_t n, uint32_t *out) {
#pragma omp parallel for schedule(static, 1 << 16)
    for (long long i = 0; i < (long long)n; i++) {
        float r = ref_fn(fn, ws_u2f(lo + (uint32_t)i));
        out[i] = (r != r) ? 0x7fc00000u : ws_f2u(r);
    }
}
