/* ws_logf: single-precision natural log, bit-identical to glibc's logf,
 * usable from host C/C++ and from HIP device code.
 *
 * Why: the sqrtsoftplus router score of weightstream-ref (num.rs:82-88,
 * moe.rs:38-42) is sqrt(ln(1 + exp(x))); Rust's f32::ln lowers to the
 * platform libm logf. The GPU math library's logf can differ from glibc's by
 * an ulp, which can reorder two near-tied experts. Evaluating the same
 * algorithm in double precision on both sides removes that.
 *
 * Algorithm: the published table-driven method of the Arm optimized-routines
 * project (Szabolcs Nagy, 2017), which glibc >= 2.28 uses for logf:
 *   x = 2^k z, z in [OFF, 2 OFF), OFF = 0x3f330000 (about 0.7);
 *   log(x) = k ln2 + log(c) + log1p(z/c - 1), with 1/c and log(c) from a
 *   16-entry table indexed by the top 4 mantissa bits of z, and log1p(r)
 *   ~= r + A2 r^2 + A1 r^3 + A0 r^4 in double.
 * The table and polynomial are that project's published data. Every float
 * input is checked against the host glibc logf by an exhaustive test of this
 * repository (tests/test_oracle_expf.py), for the host build, and by a device
 * digest over every input (tests/test_gpu_route.py).
 *
 * WS_LOGF_FMA selects the fused evaluation order of glibc's x86-64 FMA
 * variant; on this image both orders equal glibc on all 2^32 inputs.
 */
#ifndef WS_LOGF_H
#define WS_LOGF_H

#include "ws_expf.h"

/* {1/c, log(c)} per 1/16 of the reduced mantissa range */
WS_CONST_TABLE double ws_logf_tab[16][2] = {
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2},
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2},  {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3},
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3},
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4},
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0},
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5},  {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4},
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3}, {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3},
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2}, {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2},
};

#ifndef WS_LOGF_FMA
#define WS_LOGF_FMA 1
#endif

/* Split in two like ws_expf: ws_logf_reduce handles the special inputs
 * (returns 1 with the result in *out) or computes the table index *i, the
 * exponent *k and the reduced z; ws_logf_finish evaluates the result given
 * the table entry {invc, logc} of index *i. */
WS_HD int ws_logf_reduce(float x, int *i_out, int *k_out, double *z_out, float *out) {
WS_NO_CONTRACT
    uint32_t ix = ws_f2u(x);
    if (ix == 0x3f800000u) { *out = 0.0f; return 1; }  /* log(1) = +0 */
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        /* x < 2^-126, inf or nan */
        if (ix * 2 == 0) { *out = ws_u2f(0xff800000u); return 1; }             /* -inf */
        if (ix == 0x7f800000u) { *out = x; return 1; }                         /* +inf */
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) { *out = ws_u2f(0x7fc00000u); return 1; }
        /* subnormal: normalise */
        ix = ws_f2u(x * 0x1p23f);
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - 0x3f330000u;
    *i_out = (int)((tmp >> 19) & 15);
    *k_out = (int32_t)tmp >> 23;
    *z_out = (double)ws_u2f(ix - (tmp & 0xff800000u));
    return 0;
}

WS_HD float ws_logf_finish(int k, double z, double invc, double logc) {
WS_NO_CONTRACT
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2,
                 a2 = -0x1.ffffef20a4123p-2;
    const double ln2 = 0x1.62e42fefa39efp-1;
#if WS_LOGF_FMA
    double r = __builtin_fma(z, invc, -1.0);
    double y0 = __builtin_fma((double)k, ln2, logc);
    double r2 = r * r;
    double y = __builtin_fma(a1, r, a2);
    y = __builtin_fma(a0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
#else
    double r = z * invc - 1.0;
    double y0 = logc + (double)k * ln2;
    double r2 = r * r;
    double y = a1 * r + a2;
    y = a0 * r2 + y;
    y = y * r2 + (y0 + r);
#endif
    return (float)y;
}

WS_HD float ws_logf(float x) {
    int i, k;
    double z;
    float out;
    if (ws_logf_reduce(x, &i, &k, &z, &out)) return out;
    return ws_logf_finish(k, z, ws_logf_tab[i][0], ws_logf_tab[i][1]);
}

/* num.rs:82-88 softplus (torch's threshold 20) and the sqrtsoftplus score
 * of moe.rs:38-42: sqrt(softplus(x)). sqrt is IEEE (correctly rounded). */
WS_HD float ws_softplus(float x) {
WS_NO_CONTRACT
    return x > 20.0f ? x : ws_logf(1.0f + ws_expf(x));
}

#endif
