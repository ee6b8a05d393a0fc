/* CPU oracle for weightstream's quantized-matmul / MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of the reference CPU path,
 * loaded by tests/, smoke() and bench.py's cpu_baseline leg as the checker.
 * The HIP library never links, loads or calls it.
 *
 * Reference paths are relative to the weightstream repository root.
 * Built with -O2 -ffp-contract=off (see Makefile): every a*b+c below is a
 * rounded multiply followed by a rounded add, as in Rust.
 *
 * Pinning (how each group is checked beyond restating it; the tests named
 * are in tests/test_oracle_*.py):
 *  - quant primitives: the reference's known-answer tests (quant.rs:221-356)
 *    plus exhaustive enumeration of all 256 e4m3 codes, all 16 e2m1 codes,
 *    and a closed-form RNE definition checked on 2^24 random f32 inputs.
 *  - activation snaps: actquant.rs:180-223 KATs + the power-of-two grid
 *    identity (snap(x) == emit->decode(x)) on random data.
 *  - fp8/fp4 GEMV: actquant.rs:225-270 (GEMV == dense dequant dot) plus an
 *    f64 brute-force dot bounded by the f32 summation error bound.
 *  - f32-scale generalisation: f64 brute force of the dequantised product
 *    within the f32 summation bound; reduces to the UE8M0 path when all
 *    scales are powers of two (checked bit-exact). The quantisers are
 *    checked block by block against a numpy recomputation of the amax over
 *    the block (ragged last row block included), the scale fl32(amax/448)
 *    bit for bit and torch's e4m3 cast of the f32 quotient; a UE8M0-rounded
 *    scale, a reciprocal multiply, a missing floor and a last-row amax are
 *    each shown to fail that check (tests/test_oracle_f32s.py).
 *  - num: expf against the exhaustive glibc check of ws_expf, sigmoid /
 *    softplus closed forms at special points.
 *  - routing: a brute-force O(E^2) rank-count selection with the explicit
 *    (value desc, index asc, total order on -0/+0) rule, with injected ties.
 *  - experts/moe: closed form of the reference GPU test
 *    (weightstream-gpu/src/tests.rs:837-1020: all-0x11 fp4 weights), the
 *    routing-weight-before-w2 property (moe.rs:272-298), and linearity of
 *    the routed sum in the per-expert outputs.
 *  - dispatch: invariants (permutation, counts, 32-aligned monotone offsets,
 *    route_pos[order[i]] == i) and a hand-worked example.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Rust f32::clamp: NaN passes through. */
static inline float rclamp(float v, float lo, float hi) {
    if (v < lo) return lo;
    if (v > hi) return hi;
    return v;
}

/* ------------------------------------------------------------------ */
/* quant.rs                                                            */
/* ------------------------------------------------------------------ */

/* quant.rs:11-13 FP4_TABLE */
static const float FP4_TABLE[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

float or_fp4_value(uint8_t nibble) { return FP4_TABLE[nibble & 0x0F]; }

/* quant.rs:75-79 pow2i: f32::exp2 of an integer is exact (0 below 2^-149,
 * inf above 2^127), which ldexpf reproduces. */
float or_pow2i(int32_t e) { return ldexpf(1.0f, e); }

/* quant.rs:24-39 */
float or_e4m3_to_f32(uint8_t b) {
    float sign = (b & 0x80) ? -1.0f : 1.0f;
    uint8_t exp = (b >> 3) & 0x0F;
    uint8_t mant = b & 0x07;
    if (exp == 0x0F && mant == 0x07) return NAN;
    if (exp == 0) return sign * (float)mant * (1.0f / 512.0f);
    return sign * or_pow2i((int32_t)exp - 7) * (1.0f + (float)mant / 8.0f);
}

/* quant.rs:41-48 */
float or_e8m0_to_f32(uint8_t b) {
    if (b == 0xFF) return NAN;
    return or_pow2i((int32_t)b - 127);
}

/* quant.rs:60-73 */
int32_t or_log2_ceil(float x) {
    uint32_t bits = f2u(x);
    int32_t exp = (int32_t)((bits >> 23) & 0xFF) - 127;
    uint32_t mant = bits & 0x7FFFFF;
    return mant != 0 ? exp + 1 : exp;
}

/* quant.rs:81-87 */
float or_ue8m0_round_scale(float amax, float fp_max) {
    return or_pow2i(or_log2_ceil(amax / fp_max));
}

/* quant.rs:89-101 */
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
uint16_t or_f32_to_bf16(float v) {
    uint32_t bits = f2u(v);
    uint32_t round = ((bits >> 16) & 1) + 0x7FFF;
    return (uint16_t)((bits + round) >> 16);
}

/* quant.rs:103-137: RNE, saturating at +-448, NaN -> 0x7F with sign. */
uint8_t or_f32_to_e4m3(float v) {
    uint32_t bits = f2u(v);
    uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
    if (isnan(v)) return sign | 0x7F;
    float a = fabsf(v);
    if (a >= 448.0f) return sign | 0x7E;
    if (a < or_pow2i(-6)) {
        float q = a * 512.0f;
        int32_t m = (int32_t)nearbyintf(q);
        if (m == 8) return sign | 0x38;
        return sign | (uint8_t)m;
    }
    int32_t e = (int32_t)((bits >> 23) & 0xFF) - 127;
    float q = a * or_pow2i(3 - e);
    int32_t m8 = (int32_t)nearbyintf(q);
    int32_t exp_field, mant;
    if (m8 == 16) { exp_field = e + 8; mant = 0; }
    else { exp_field = e + 7; mant = m8 - 8; }
    return sign | (uint8_t)(exp_field << 3) | (uint8_t)mant;
}

/* quant.rs:139-163: thresholds encode RNE on the e2m1 grid. */
uint8_t or_f32_to_e2m1(float v) {
    uint8_t sign = (f2u(v) >> 31) ? 0x8 : 0x0;
    float a = fabsf(v);
    uint8_t code;
    if (a <= 0.25f) code = 0;
    else if (a < 0.75f) code = 1;
    else if (a <= 1.25f) code = 2;
    else if (a < 1.75f) code = 3;
    else if (a <= 2.5f) code = 4;
    else if (a < 3.5f) code = 5;
    else if (a <= 5.0f) code = 6;
    else code = 7;
    return sign | code;
}

/* quant.rs:165-170 */
uint8_t or_pack_fp4(uint8_t even, uint8_t odd) { return (uint8_t)((even & 0x0F) | (odd << 4)); }

/* quant.rs:172-187 */
void or_dequant_fp8_blockwise(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, float *out) {
    size_t sb_cols = (cols + 31) / 32;
    for (size_t r = 0; r < rows; r++)
        for (size_t c = 0; c < cols; c++) {
            float sc = or_e8m0_to_f32(s[(r / 32) * sb_cols + c / 32]);
            out[r * cols + c] = or_e4m3_to_f32(w[r * cols + c]) * sc;
        }
}

/* quant.rs:189-215 */
void or_dequant_fp4_packed(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, float *out) {
    size_t kbn = (cols + 31) / 32;
    for (size_t r = 0; r < rows; r++)
        for (size_t kb = 0; kb < kbn; kb++) {
            float sc = or_e8m0_to_f32(s[r * kbn + kb]);
            for (size_t j = 0; j < 32; j++) {
                size_t c = kb * 32 + j;
                if (c >= cols) break;
                uint8_t byte = w[r * (cols / 2) + c / 2];
                float v = (c % 2 == 0) ? FP4_TABLE[byte & 0x0F] : FP4_TABLE[byte >> 4];
                out[r * cols + c] = v * sc;
            }
        }
}

/* ------------------------------------------------------------------ */
/* actquant.rs                                                         */
/* ------------------------------------------------------------------ */

/* actquant.rs:19-45 */
void or_fp8_snap(float *x, size_t n, size_t block) {
    for (size_t g0 = 0; g0 + block <= n; g0 += block) {
        float amax = 0.0f;
        for (size_t i = 0; i < block; i++) {
            float a = fabsf(x[g0 + i]);
            if (a > amax) amax = a;
        }
        if (amax < 1e-4f) amax = 1e-4f;
        float s = or_pow2i(or_log2_ceil(amax / 448.0f));
        for (size_t i = 0; i < block; i++) {
            float q = rclamp(x[g0 + i] / s, -448.0f, 448.0f);
            x[g0 + i] = or_e4m3_to_f32(or_f32_to_e4m3(q)) * s;
        }
    }
}

/* actquant.rs:59-79 */
void or_fp4_snap_e8m0(float *x, size_t n, size_t block) {
    for (size_t g0 = 0; g0 + block <= n; g0 += block) {
        float amax = 0.0f;
        for (size_t i = 0; i < block; i++) {
            float a = fabsf(x[g0 + i]);
            if (a > amax) amax = a;
        }
        float fl = 6.0f * or_pow2i(-126);
        if (amax < fl) amax = fl;
        float s = or_pow2i(or_log2_ceil(amax / 6.0f));
        for (size_t i = 0; i < block; i++) {
            float q = rclamp(x[g0 + i] / s, -6.0f, 6.0f);
            x[g0 + i] = FP4_TABLE[or_f32_to_e2m1(q) & 0x0F] * s;
        }
    }
}

/* actquant.rs:81-103 */
void or_fp4_snap_e4m3(float *x, size_t n, size_t block) {
    for (size_t g0 = 0; g0 + block <= n; g0 += block) {
        float amax = 0.0f;
        for (size_t i = 0; i < block; i++) {
            float a = fabsf(x[g0 + i]);
            if (a > amax) amax = a;
        }
        float fl = 6.0f * or_pow2i(-9);
        if (amax < fl) amax = fl;
        float s = or_e4m3_to_f32(or_f32_to_e4m3(amax / 6.0f));
        for (size_t i = 0; i < block; i++) {
            float q = rclamp(x[g0 + i] / s, -6.0f, 6.0f);
            x[g0 + i] = FP4_TABLE[or_f32_to_e2m1(q) & 0x0F] * s;
        }
    }
}

/* Storage form of actquant.rs:21-45 (the bytes act_quant_fp8_emit writes,
 * weightstream-cuda/kernels/actquant.cu:47-85): q = e4m3(clamp(x/s)), scale
 * byte = log2_ceil(amax/448) + 127. */
void or_fp8_act_emit(const float *x, size_t n, uint8_t *q, uint8_t *s) {
    for (size_t g = 0; g * 32 < n; g++) {
        const float *v = x + g * 32;
        float amax = 0.0f;
        for (size_t i = 0; i < 32; i++) {
            float a = fabsf(v[i]);
            if (a > amax) amax = a;
        }
        if (amax < 1e-4f) amax = 1e-4f;
        int32_t e = or_log2_ceil(amax / 448.0f);
        float sc = or_pow2i(e);
        s[g] = (uint8_t)(e + 127);
        for (size_t i = 0; i < 32; i++)
            q[g * 32 + i] = or_f32_to_e4m3(rclamp(v[i] / sc, -448.0f, 448.0f));
    }
}

/* actquant.rs:110-138: per 32-K block, blk += qa*(w*s_b) in K order; acc += blk. */
/* Threads for the row loops of the GEMVs (1 = the reference's scalar loop).
 * Rows are independent and each keeps its sequential sum, so the results do
 * not depend on the count; only the timing baseline uses more than one. */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

void or_fp8_gemv(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, const float *x, float *y) {
    size_t kbn = cols / 32;
    float *qa = (float *)malloc(cols * sizeof(float));
    memcpy(qa, x, cols * sizeof(float));
    or_fp8_snap(qa, cols, 32);
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t n = 0; n < rows; n++) {
        const uint8_t *row = w + n * cols;
        size_t srow = (n / 32) * kbn;
        float acc = 0.0f;
        for (size_t kb = 0; kb < kbn; kb++) {
            float s_b = or_e8m0_to_f32(s[srow + kb]);
            float blk = 0.0f;
            for (size_t j = 0; j < 32; j++) {
                size_t c = kb * 32 + j;
                blk += qa[c] * (or_e4m3_to_f32(row[c]) * s_b);
            }
            acc += blk;
        }
        y[n] = acc;
    }
    free(qa);
}

/* actquant.rs:140-173 */
void or_fp4_gemv(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, const float *x, float *y) {
    size_t kbn = cols / 32, half = cols / 2;
    float *qa = (float *)malloc(cols * sizeof(float));
    memcpy(qa, x, cols * sizeof(float));
    or_fp8_snap(qa, cols, 32);
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t n = 0; n < rows; n++) {
        const uint8_t *row = w + n * half;
        float acc = 0.0f;
        for (size_t kb = 0; kb < kbn; kb++) {
            float s_b = or_e8m0_to_f32(s[n * kbn + kb]);
            float blk = 0.0f;
            for (size_t j = 0; j < 32; j++) {
                size_t c = kb * 32 + j;
                uint8_t byte = row[c / 2];
                float v = (c % 2 == 0) ? FP4_TABLE[byte & 0x0F] : FP4_TABLE[byte >> 4];
                blk += qa[c] * (v * s_b);
            }
            acc += blk;
        }
        y[n] = acc;
    }
    free(qa);
}

/* The GEMV arithmetic above for M rows of already-quantised activations:
 * qa = e4m3(aq)*e8m0(as) is exactly what fp8_act_values produces
 * (actquant.rs:47-57), so this equals fp8_gemv/fp4_gemv row by row. */
void or_gemm_q(const uint8_t *aq, const uint8_t *as, size_t M,
               const uint8_t *w, const uint8_t *ws, size_t N, size_t K, int w_fp4, float *y) {
    size_t kbn = K / 32;
    float *qa = (float *)malloc(K * sizeof(float));
    for (size_t m = 0; m < M; m++) {
        for (size_t c = 0; c < K; c++)
            qa[c] = or_e4m3_to_f32(aq[m * K + c]) * or_e8m0_to_f32(as[m * kbn + c / 32]);
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
        for (size_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (size_t kb = 0; kb < kbn; kb++) {
                float blk = 0.0f;
                if (w_fp4) {
                    float s_b = or_e8m0_to_f32(ws[n * kbn + kb]);
                    const uint8_t *row = w + n * (K / 2);
                    for (size_t j = 0; j < 32; j++) {
                        size_t c = kb * 32 + j;
                        uint8_t byte = row[c / 2];
                        float v = (c % 2 == 0) ? FP4_TABLE[byte & 0x0F] : FP4_TABLE[byte >> 4];
                        blk += qa[c] * (v * s_b);
                    }
                } else {
                    float s_b = or_e8m0_to_f32(ws[(n / 32) * kbn + kb]);
                    const uint8_t *row = w + n * K;
                    for (size_t j = 0; j < 32; j++) {
                        size_t c = kb * 32 + j;
                        blk += qa[c] * (or_e4m3_to_f32(row[c]) * s_b);
                    }
                }
                acc += blk;
            }
            y[m * N + n] = acc;
        }
    }
    free(qa);
}

/* ------------------------------------------------------------------ */
/* f32-scale generalisation (BASELINE.json configs 1-2 scheme)         */
/* Not in the reference: 1xB activation / BxB weight blocks with f32    */
/* scale = amax/448 (amax floored at 1e-4 as in actquant.rs:36-38).    */
/* The GEMM keeps fp8_gemv's structure (actquant.rs:114-138): a        */
/* sequential e4m3 x e4m3 block dot, scale-corrected once per block,   */
/* accumulated in K order.                                             */
/* ------------------------------------------------------------------ */
void or_act_quant_f32s(const float *x, size_t M, size_t K, size_t block, uint8_t *q, float *s) {
    size_t kbn = K / block;
    for (size_t m = 0; m < M; m++)
        for (size_t kb = 0; kb < kbn; kb++) {
            const float *v = x + m * K + kb * block;
            float amax = 0.0f;
            for (size_t i = 0; i < block; i++) {
                float a = fabsf(v[i]);
                if (a > amax) amax = a;
            }
            if (amax < 1e-4f) amax = 1e-4f;
            float sc = amax / 448.0f;
            s[m * kbn + kb] = sc;
            for (size_t i = 0; i < block; i++)
                q[m * K + kb * block + i] = or_f32_to_e4m3(rclamp(v[i] / sc, -448.0f, 448.0f));
        }
}

void or_weight_quant_fp8_f32s(const float *w, size_t N, size_t K, size_t block, uint8_t *q, float *s) {
    size_t nbn = (N + block - 1) / block, kbn = K / block;
    for (size_t nb = 0; nb < nbn; nb++)
        for (size_t kb = 0; kb < kbn; kb++) {
            size_t r1 = (nb + 1) * block < N ? (nb + 1) * block : N;
            float amax = 0.0f;
            for (size_t r = nb * block; r < r1; r++)
                for (size_t c = kb * block; c < (kb + 1) * block; c++) {
                    float a = fabsf(w[r * K + c]);
                    if (a > amax) amax = a;
                }
            if (amax < 1e-4f) amax = 1e-4f;
            float sc = amax / 448.0f;
            s[nb * kbn + kb] = sc;
            for (size_t r = nb * block; r < r1; r++)
                for (size_t c = kb * block; c < (kb + 1) * block; c++)
                    q[r * K + c] = or_f32_to_e4m3(rclamp(w[r * K + c] / sc, -448.0f, 448.0f));
        }
}

void or_gemm_f32s(const uint8_t *aq, const float *as, size_t M,
                  const uint8_t *w, const float *ws, size_t N, size_t K, size_t block, float *y) {
    size_t kbn = K / block;
    /* outputs are independent sequential sums: threads change no bits */
#pragma omp parallel for collapse(2) num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (size_t kb = 0; kb < kbn; kb++) {
                float blk = 0.0f;
                for (size_t j = 0; j < block; j++) {
                    size_t c = kb * block + j;
                    blk += or_e4m3_to_f32(aq[m * K + c]) * or_e4m3_to_f32(w[n * K + c]);
                }
                acc += blk * (as[m * kbn + kb] * ws[(n / block) * kbn + kb]);
            }
            y[m * N + n] = acc;
        }
}

/* ------------------------------------------------------------------ */
/* weight encoders (store.rs:357-422) with a true per-block amax: the   */
/* FP8 encoder takes the amax over the whole 32x32 block (store.rs's    */
/* test encoder keeps the last row's scale, a self-consistent quirk     */
/* that is deliberately not reproduced).                               */
/* ------------------------------------------------------------------ */
void or_weight_quant_fp8(const float *w, size_t rows, size_t cols, uint8_t *q, uint8_t *s) {
    size_t s_cols = (cols + 31) / 32;
    for (size_t rb = 0; rb * 32 < rows; rb++)
        for (size_t kb = 0; kb < s_cols; kb++) {
            size_t r1 = (rb + 1) * 32 < rows ? (rb + 1) * 32 : rows;
            size_t c1 = (kb + 1) * 32 < cols ? (kb + 1) * 32 : cols;
            float amax = 1e-4f;
            for (size_t r = rb * 32; r < r1; r++)
                for (size_t c = kb * 32; c < c1; c++) {
                    float a = fabsf(w[r * cols + c]);
                    if (a > amax) amax = a;   /* f32::max */
                }
            int32_t e = or_log2_ceil(amax / 448.0f);
            float sc = or_pow2i(e);
            s[rb * s_cols + kb] = (uint8_t)(e + 127);
            for (size_t r = rb * 32; r < r1; r++)
                for (size_t c = kb * 32; c < c1; c++)
                    q[r * cols + c] = or_f32_to_e4m3(rclamp(w[r * cols + c] / sc, -448.0f, 448.0f));
        }
}

void or_weight_quant_fp4(const float *w, size_t rows, size_t cols, uint8_t *q, uint8_t *s) {
    size_t s_cols = (cols + 31) / 32;
    memset(q, 0, rows * cols / 2);
    for (size_t r = 0; r < rows; r++)
        for (size_t kb = 0; kb < s_cols; kb++) {
            size_t c1 = (kb + 1) * 32 < cols ? (kb + 1) * 32 : cols;
            float amax = 6.0f * or_pow2i(-126);
            for (size_t c = kb * 32; c < c1; c++) {
                float a = fabsf(w[r * cols + c]);
                if (a > amax) amax = a;
            }
            int32_t e = or_log2_ceil(amax / 6.0f);
            float sc = or_pow2i(e);
            s[r * s_cols + kb] = (uint8_t)(e + 127);
            for (size_t c = kb * 32; c < c1; c++) {
                uint8_t code = or_f32_to_e2m1(rclamp(w[r * cols + c] / sc, -6.0f, 6.0f));
                size_t idx = r * (cols / 2) + c / 2;
                if (c % 2 == 0) q[idx] = (uint8_t)((q[idx] & 0xF0) | (code & 0x0F));
                else q[idx] = (uint8_t)((q[idx] & 0x0F) | (code << 4));
            }
        }
}

/* ------------------------------------------------------------------ */
/* num.rs                                                              */
/* ------------------------------------------------------------------ */

/* Rust f32::exp lowers to the platform libm expf (glibc here). */
float or_expf(float x) { return expf(x); }

/* num.rs:7-16 */
float or_dot(const float *a, const float *b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* num.rs:18-28 */
void or_gemv_f32(const float *w, size_t n, size_t k, const float *x, float *y) {
    for (size_t r = 0; r < n; r++) y[r] = or_dot(w + r * k, x, k);
}

/* num.rs:46-62 */
void or_softmax(float *x, size_t n) {
    float m = -INFINITY;
    for (size_t i = 0; i < n; i++) if (x[i] > m) m = x[i];
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) { x[i] = expf(x[i] - m); s += x[i]; }
    for (size_t i = 0; i < n; i++) x[i] /= s;
}

/* num.rs:70-88 */
float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
float or_silu(float x) { return x * or_sigmoid(x); }
float or_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

/* ------------------------------------------------------------------ */
/* moe.rs                                                              */
/* ------------------------------------------------------------------ */

/* moe.rs:24-42 */
void or_score(float *s, size_t n, int score_func, float gate_temp) {
    if (gate_temp != 1.0f)
        for (size_t i = 0; i < n; i++) s[i] /= gate_temp;
    if (score_func == OR_SCORE_SOFTMAX) {
        or_softmax(s, n);
    } else if (score_func == OR_SCORE_SIGMOID) {
        for (size_t i = 0; i < n; i++) s[i] = or_sigmoid(s[i]);
    } else {
        for (size_t i = 0; i < n; i++) s[i] = sqrtf(or_softplus(s[i]));
    }
}

/* Rust f32::total_cmp as a signed integer key. */
static inline int32_t total_key(float v) {
    int32_t b = (int32_t)f2u(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

static const int32_t *g_keys;
static int cmp_route(const void *pa, const void *pb) {
    int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
    /* moe.rs:50: biased[b].total_cmp(&biased[a]).then(a.cmp(&b)) */
    if (g_keys[a] != g_keys[b]) return g_keys[b] > g_keys[a] ? 1 : -1;
    return (a > b) - (a < b);
}

/* moe.rs:45-69 */
void or_route(const float *scores, const float *bias, size_t n, size_t top_k,
              int norm_topk_prob, float route_scale, int32_t *idx, float *w) {
    int32_t *order = (int32_t *)malloc(n * sizeof(int32_t));
    int32_t *keys = (int32_t *)malloc(n * sizeof(int32_t));
    for (size_t i = 0; i < n; i++) {
        order[i] = (int32_t)i;
        keys[i] = total_key(scores[i] + bias[i]);
    }
    g_keys = keys;
    qsort(order, n, sizeof(int32_t), cmp_route);
    for (size_t k = 0; k < top_k; k++) {
        idx[k] = order[k];
        w[k] = scores[order[k]];
    }
    if (norm_topk_prob && top_k > 1) {
        float sum = -0.0f;   /* Rust's f32 Sum folds from -0.0 */
        for (size_t k = 0; k < top_k; k++) sum += w[k];
        for (size_t k = 0; k < top_k; k++) w[k] /= sum + 1e-20f;
    }
    for (size_t k = 0; k < top_k; k++) w[k] *= route_scale;
    free(order);
    free(keys);
}

/* moe.rs:187-202 (asymmetric clamps; limit <= 0 disables them) */
static void swiglu(const float *gate, const float *up, size_t n, float limit, float rw,
                   int apply_rw, float *h) {
    for (size_t i = 0; i < n; i++) {
        float u = limit > 0.0f ? rclamp(up[i], -limit, limit) : up[i];
        float g = limit > 0.0f ? fminf(gate[i], limit) : gate[i];
        h[i] = apply_rw ? or_silu(g) * u * rw : or_silu(g) * u;
    }
}

/* moe.rs:162-208 */
void or_expert_fp4(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, float rw, float limit, float *y) {
    float *g = (float *)malloc(inter * sizeof(float));
    float *u = (float *)malloc(inter * sizeof(float));
    float *h = (float *)malloc(inter * sizeof(float));
    or_fp4_gemv(w1, s1, inter, dim, x, g);
    or_fp4_gemv(w3, s3, inter, dim, x, u);
    swiglu(g, u, inter, limit, rw, 1, h);
    or_fp4_gemv(w2, s2, dim, inter, h, y);
    free(g); free(u); free(h);
}

/* The hidden state of or_expert_fp4 before its FP8 re-quantisation (the
 * input or_fp4_gemv snaps for the down projection): moe.rs:162-200. */
void or_expert_hidden_fp4(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                          const uint8_t *s3, size_t dim, size_t inter, const float *x, float rw,
                          float limit, float *h) {
    float *g = (float *)malloc(inter * sizeof(float));
    float *u = (float *)malloc(inter * sizeof(float));
    or_fp4_gemv(w1, s1, inter, dim, x, g);
    or_fp4_gemv(w3, s3, inter, dim, x, u);
    swiglu(g, u, inter, limit, rw, 1, h);
    free(g); free(u);
}

/* moe.rs:210-250 */
void or_shared_fp8(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, float limit, float *y) {
    float *g = (float *)malloc(inter * sizeof(float));
    float *u = (float *)malloc(inter * sizeof(float));
    float *h = (float *)malloc(inter * sizeof(float));
    or_fp8_gemv(w1, s1, inter, dim, x, g);
    or_fp8_gemv(w3, s3, inter, dim, x, u);
    swiglu(g, u, inter, limit, 1.0f, 0, h);
    or_fp8_gemv(w2, s2, dim, inter, h, y);
    free(g); free(u); free(h);
}

/* moe.rs:75-84: y = sum of expert outputs in ascending expert id. */
void or_moe_routed(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, const int32_t *idx, const float *w, size_t top_k,
                   float limit, float *y) {
    size_t fp4_mat = inter * dim / 2, sc_up = inter * (dim / 32), sc_dn = dim * (inter / 32);
    int32_t *ord = (int32_t *)malloc(top_k * sizeof(int32_t));
    for (size_t k = 0; k < top_k; k++) ord[k] = (int32_t)k;
    for (size_t i = 1; i < top_k; i++) {          /* stable sort by expert id */
        int32_t v = ord[i];
        size_t j = i;
        while (j > 0 && idx[ord[j - 1]] > idx[v]) { ord[j] = ord[j - 1]; j--; }
        ord[j] = v;
    }
    float *h = (float *)malloc(dim * sizeof(float));
    for (size_t d = 0; d < dim; d++) y[d] = 0.0f;
    for (size_t k = 0; k < top_k; k++) {
        size_t e = (size_t)idx[ord[k]];
        or_expert_fp4(w1 + e * fp4_mat, s1 + e * sc_up, w3 + e * fp4_mat, s3 + e * sc_up,
                      w2 + e * fp4_mat, s2 + e * sc_dn, dim, inter, x, w[ord[k]], limit, h);
        for (size_t d = 0; d < dim; d++) y[d] += h[d];
    }
    free(h);
    free(ord);
}

/* ------------------------------------------------------------------ */
/* Grouped dispatch: the contract of moe_dispatch_kernel               */
/* (weightstream-cuda/kernels/tilelang/moe_dispatch.cu:17-153): routes  */
/* with expert >= 0 are counted per expert, each expert's segment is    */
/* padded to a multiple of 32 and placed by an exclusive scan in        */
/* ascending expert order; inside a segment routes keep ascending route */
/* index. order[slot] = route (or -1 pad), layout_w[slot] = its weight  */
/* (0 pad), route_pos[route] = slot (-1 if dropped), tile_expert[t] =   */
/* expert of 32-row tile t (-1 past the used tiles), psum = offset +    */
/* count, num_tiles = used tiles. Slots at or beyond tiles*32 are not   */
/* written (the kernel bounds-checks the same way).                    */
/* ------------------------------------------------------------------ */
void or_dispatch(const int32_t *topk_idx, const float *topk_w, size_t routes, size_t n_experts,
                 size_t tiles, int32_t *order, float *layout_w, int32_t *route_pos,
                 int32_t *tile_expert, int32_t *count, int32_t *offset, int32_t *psum,
                 int32_t *num_tiles) {
    size_t cap = tiles * 32;
    for (size_t e = 0; e < n_experts; e++) count[e] = 0;
    for (size_t r = 0; r < routes; r++)
        if (topk_idx[r] >= 0) count[topk_idx[r]]++;
    int32_t run = 0;
    for (size_t e = 0; e < n_experts; e++) {
        int32_t padded = (count[e] + 31) / 32 * 32;
        offset[e] = run;
        psum[e] = run + count[e];
        run += padded;
    }
    *num_tiles = run / 32;
    for (size_t t = 0; t < tiles; t++) tile_expert[t] = -1;
    for (size_t e = 0; e < n_experts; e++) {
        int32_t padded = (count[e] + 31) / 32 * 32;
        for (int32_t i = count[e]; i < padded; i++) {
            size_t slot = (size_t)(offset[e] + i);
            if (slot < cap) { order[slot] = -1; layout_w[slot] = 0.0f; }
        }
        for (int32_t t = 0; t < padded / 32; t++) {
            size_t tt = (size_t)(offset[e] / 32 + t);
            if (tt < tiles) tile_expert[tt] = (int32_t)e;
        }
    }
    int32_t *fill = (int32_t *)calloc(n_experts, sizeof(int32_t));
    for (size_t r = 0; r < routes; r++) {
        int32_t e = topk_idx[r];
        if (e < 0) { route_pos[r] = -1; continue; }
        int32_t slot = offset[e] + fill[e]++;
        if ((size_t)slot < cap) { order[slot] = (int32_t)r; layout_w[slot] = topk_w[r]; }
        route_pos[r] = slot;
    }
    free(fill);
}

/* Test infrastructure: the reference's byte for the 32-bit pattern u, for
 * the exhaustive device checks of ws_math_probe: fn 2 the e4m3 encoding of
 * x (quant.rs:103-137), fn 3 the UE8M0 scale byte of a block whose largest
 * magnitude is |x| (or_fp8_act_emit's rule: the `a > amax` scan from 0, so
 * NaN counts as 0; floor 1e-4; log2_ceil(amax / 448) + 127), fn 4 the f32
 * bits of the value of x's e4m3 byte (NaN canonical). */
static uint32_t or_probe_byte(int fn, uint32_t u) {
    const float x = u2f(u);
    if (fn == 2) return or_f32_to_e4m3(x);
    if (fn == 4) {  /* the value of the e4m3 byte of x (NaN canonical) */
        const float d = or_e4m3_to_f32(or_f32_to_e4m3(x));
        return isnan(d) ? 0x7FC00000u : f2u(d);
    }
    float a = fabsf(x), amax = 0.0f;
    if (a > amax) amax = a;
    if (amax < 1e-4f) amax = 1e-4f;
    return (uint32_t)(uint8_t)(or_log2_ceil(amax / 448.0f) + 127);
}

/* sum over u in [lo, hi) of (byte(u) ^ (u * 0x9E3779B1)) * (2u + 1) mod 2^64
 * (the digest the GPU test computes with wrapping int64 arithmetic) */
uint64_t or_probe_digest(int fn, uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
#pragma omp parallel for reduction(+ : acc) schedule(static, 1 << 16)
    for (long long u = (long long)lo; u < (long long)hi; u++)
        acc += (uint64_t)(or_probe_byte(fn, (uint32_t)u) ^ (uint32_t)((uint32_t)u * 0x9E3779B1u)) *
               (2 * (uint64_t)u + 1);
    return acc;
}

/* the bytes for the patterns [lo, lo + n) */
void or_probe_bytes(int fn, uint32_t lo, uint32_t n, uint32_t *out) {
#pragma omp parallel for schedule(static, 1 << 16)
    for (long long i = 0; i < (long long)n; i++) out[i] = or_probe_byte(fn, lo + (uint32_t)i);
}
