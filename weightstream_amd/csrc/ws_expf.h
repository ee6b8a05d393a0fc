/* ws_expf: single-precision exp, bit-identical to glibc's expf, usable from
 * host C/C++ and from HIP device code.
 *
 * Why: MoE routing must select the same experts, with the same weights, as
 * the CPU reference (weightstream-ref num.rs:71 `sigmoid = 1/(1+exp(-x))`,
 * Rust f32::exp lowers to the platform libm expf). The GPU math library's
 * expf differs from glibc's by 1 ulp on some inputs, which can reorder two
 * near-tied experts. Evaluating the same algorithm in double precision on
 * both sides removes that.
 *
 * Algorithm: the published table-driven method of the Arm optimized-routines
 * project (Szabolcs Nagy, 2017), which glibc >= 2.27 uses for expf:
 *   x*N/ln2 = k + r, |r| <= 1/2, N = 32;
 *   exp(x) = 2^(k/N) * 2^(r/N), 2^(r/N) ~= 1 + C2 r + C1 r^2 + C0 r^3.
 * The 32-entry table holds bits(2^(i/32)) - (i << 52)/32, computed from
 * exp2l (correctly rounded), except entry 31: glibc's entry is not the
 * correctly rounded 2^(31/32); an exhaustive scan over every float input
 * accepts exactly the entries +12..+40 ulp above it (and no others at or
 * below +11), so entry 31 is set to +16 ulp. Every float input is checked
 * against the host glibc expf by an exhaustive test of this repository
 * (tests/test_oracle_expf.py), for host and device builds alike.
 *
 * WS_EXPF_FMA selects the fused evaluation order that glibc's x86-64 FMA
 * variant (selected at run time on CPUs with FMA) uses; the exhaustive test
 * decides which one matches the host library.
 */
#ifndef WS_EXPF_H
#define WS_EXPF_H

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define WS_HD __host__ __device__ __forceinline__
#else
#define WS_HD static inline
#endif

#if defined(__HIPCC__)
#define WS_CONST_TABLE __constant__ static const
#else
#define WS_CONST_TABLE static const
#endif

WS_CONST_TABLE uint64_t ws_exp2f_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4550ull,
};

WS_HD uint32_t ws_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
WS_HD float ws_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
WS_HD uint64_t ws_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
WS_HD double ws_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

#if defined(__clang__)
#define WS_NO_CONTRACT _Pragma("clang fp contract(off)")
#else
#define WS_NO_CONTRACT
#endif

#ifndef WS_EXPF_FMA
#define WS_EXPF_FMA 1
#endif

/* Split in two so that a caller may fetch the table entry its own way (the
 * GPU routing kernel keeps the table in lane registers): ws_expf_reduce
 * handles the special inputs (returns 1 with the result in *out) or computes
 * k and r; ws_expf_finish evaluates 2^(k/N) * 2^(r/N) given the table entry
 * ws_exp2f_tab[k % 32]. */
WS_HD int ws_expf_reduce(float x, uint64_t *ki_out, double *r_out, float *out) {
WS_NO_CONTRACT
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    uint32_t ux = ws_f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= (ws_f2u(88.0f) >> 20)) {
        if (ux == 0xff800000u) { *out = 0.0f; return 1; }                 /* -inf */
        if (abstop >= (0x7f800000u >> 20)) { *out = x + x; return 1; }      /* +inf, nan */
        if (x > 0x1.62e42ep6f) { *out = ws_u2f(0x7f800000u); return 1; }   /* overflow */
        if (x < -0x1.9fe368p6f) { *out = 0.0f; return 1; }                 /* underflow */
    }
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki = ws_d2u(kd);
    kd -= shift;
    *r_out = z - kd;
    *ki_out = ki;
    return 0;
}

WS_HD float ws_expf_finish(uint64_t ki, double r, uint64_t tab) {
WS_NO_CONTRACT
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint64_t t = tab + (ki << (52 - 5));
    double s = ws_u2d(t);
#if WS_EXPF_FMA
    double zz = __builtin_fma(c0, r, c1);
    double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(zz, r2, y);
#else
    double zz = c0 * r + c1;
    double r2 = r * r;
    double y = c2 * r + 1.0;
    y = zz * r2 + y;
#endif
    y = y * s;
    return (float)y;
}

WS_HD float ws_expf(float x) {
    uint64_t ki;
    double r;
    float out;
    if (ws_expf_reduce(x, &ki, &r, &out)) return out;
    return ws_expf_finish(ki, r, ws_exp2f_tab[ki % 32]);
}

/* sigmoid and silu in the reference's exact operation order
 * (weightstream-ref num.rs:71-79): 1/(1+exp(-x)), x*sigmoid(x). */
WS_HD float ws_sigmoid(float x) {
WS_NO_CONTRACT
    return 1.0f / (1.0f + ws_expf(-x));
}
WS_HD float ws_silu(float x) {
WS_NO_CONTRACT
    return x * ws_sigmoid(x);
}

#endif
