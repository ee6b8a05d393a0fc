// Block-scaled GEMM on CDNA4 scaled MFMA: C[M,N] = A[M,K] . B[N,K]^T.
//
// Replaces fp8_gemm.cu:9 (M=1 decode), fp8_gemm_tile.cu:28 (M-batch),
// fp4_expert_gemm.cu:9 / fp4_gemm_tile.cu:21 and the TileLang gemm_mxfp8
// kernels (launch.rs:344-377, 717-804). CPU semantics: weightstream-ref
// actquant.rs:110-173 (per-32 block dot, scale-corrected, f32 accumulate).
//
// Design (gfx950):
//  - one v_mfma_scale_f32_16x16x128_f8f6f4 per 16x16 output fragment and
//    128-K step. The hardware applies the UE8M0 scales per lane, i.e. per
//    (row, 32-K block), which is exactly the reference's activation (1x32) and
//    FP4 weight (1x32) granularity; FP8 32x32 weight scales are broadcast to
//    the 32 rows of their block. The f32-scale scheme runs the MFMA with unit
//    scales and applies sa*sb once per 128-K step in f32.
//  - fragment layout (measured on gfx950): lane l holds row/col l % 16; with
//    g = l / 16, an FP8 lane holds K [16g, 16g+16) and [64+16g, 64+16g+16) of
//    the 128-K step, an FP4 lane holds K [32g, 32g+32) (low nibble = even K),
//    and the lane's UE8M0 byte scales K block [32g, 32g+32) of its row in
//    both cases. The four lanes of a row therefore read 128 contiguous FP8
//    bytes (64 FP4 bytes) per step with 16-byte loads; no LDS staging.
//  - a workgroup is GM x GK waves: GM waves along M share the weight
//    fragments through L1/L2; GK waves split K and are reduced through LDS in
//    wave order (deterministic).
//  - the weight operand is streamed with non-temporal loads: each weight byte
//    is used by exactly one workgroup.
#include "ws_internal.hpp"

#include <stdlib.h>

namespace ws {

enum ScaleMode { kUe8m0 = 0, kF32s = 1 };
enum OutMode { kOutF32 = 0, kOutBf16 = 1 };

// Operand registers of U consecutive 128-K steps of one wave.
template <int WM, int WN, int U>
struct GemmStage {
    uint4 a[U][WM][2];
    uint4 b[U][WN][2];
    uint32_t sa[U][WM], sb[U][WN];
};

template <int WM, int WN, int GM, int GK, bool BFP4, int SMODE, int OMODE, int U, bool EXACT>
__global__ __launch_bounds__(64 * GM * GK) void gemm_kernel(const uint8_t *__restrict__ A,
                                                            const void *__restrict__ SA,
                                                            const uint8_t *__restrict__ B,
                                                            const void *__restrict__ SB,
                                                            void *__restrict__ C, int M, int N,
                                                            int K) {
    constexpr int kTileM = 16 * WM * GM;
    constexpr int kTileN = 16 * WN;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int wm = w % GM, wk = w / GM;
    const int r = lane & 15, kb = lane >> 4;
    const int m_base = blockIdx.y * kTileM + wm * 16 * WM;
    const int n_base = blockIdx.x * kTileN;
    const int ksteps = K / 128;
    const int k0 = wk * ksteps / GK, k1 = (wk + 1) * ksteps / GK;
    const int kbn = K / 32;  // UE8M0 scale columns
    const int kb128 = K / 128;

    // per-fragment row / column this lane loads (clamped; stores are guarded)
    const uint8_t *arow[WM];
    const uint8_t *brow[WN];
    const uint8_t *sarow[WM];
    const uint8_t *sbrow[WN];
    int col_of[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        int row = min(m_base + i * 16 + r, M - 1);
        // exact: contiguous K [32g, 32g+32); native FP8 MFMA: split halves
        arow[i] = A + (size_t)row * K + (EXACT ? kb * 32 : kb * 16);
        if (SMODE == kUe8m0) sarow[i] = (const uint8_t *)SA + (size_t)row * kbn;
    }
#pragma unroll
    for (int j = 0; j < WN; j++) {
        int col = min(n_base + j * 16 + r, N - 1);
        col_of[j] = col;
        brow[j] = BFP4 ? B + (size_t)col * (K / 2) + kb * 16
                       : B + (size_t)col * K + (EXACT ? kb * 32 : kb * 16);
        if (SMODE == kUe8m0)
            sbrow[j] = (const uint8_t *)SB + (size_t)(BFP4 ? col : col / 32) * kbn;
    }

    v4f acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // f32-scale mode: the activation scales of the 4 D rows of each fragment
    // and the weight scale of the lane's column, per 128-K step.
    const float *saf = (const float *)SA;
    const float *sbf = (const float *)SB;

    // steps past k1 re-load step k1-1 and are not used: unconditional loads
    // keep a whole stage in flight behind one wait
    auto load = [&](GemmStage<WM, WN, U> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            int ks = min(ks0 + u, k1 - 1);
#pragma unroll
            for (int i = 0; i < WM; i++) {
                const uint8_t *p = arow[i] + (size_t)ks * 128;
                st.a[u][i][0] = ldg16(p);
                st.a[u][i][1] = ldg16(p + (EXACT ? 16 : 64));
                if (SMODE == kUe8m0)
                    st.sa[u][i] = *(const uint32_t *)(sarow[i] + ks * 4) >> (8 * kb);
            }
#pragma unroll
            for (int j = 0; j < WN; j++) {
                if (BFP4) {
                    st.b[u][j][0] = ldg16_stream(brow[j] + (size_t)ks * 64);
                } else {
                    const uint8_t *p = brow[j] + (size_t)ks * 128;
                    st.b[u][j][0] = ldg16_stream(p);
                    st.b[u][j][1] = ldg16_stream(p + (EXACT ? 16 : 64));
                }
                if (SMODE == kUe8m0)
                    st.sb[u][j] = *(const uint32_t *)(sbrow[j] + ks * 4) >> (8 * kb);
            }
        }
    };

    auto compute = [&](const GemmStage<WM, WN, U> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            int ks = ks0 + u;
            if (ks >= k1) continue;
            if (EXACT) {
                v8bf bq[WN][4];
#pragma unroll
                for (int j = 0; j < WN; j++) {
                    float sbv_f = SMODE == kUe8m0 ? e8m0_to_f32(st.sb[u][j] & 0xFF) : 1.0f;
                    if (BFP4) cvt_fp4x32(st.b[u][j][0], sbv_f, bq[j]);
                    else cvt_fp8x32(st.b[u][j][0], st.b[u][j][1], sbv_f, bq[j]);
                }
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    v8bf aq[4];
                    float sav_f = SMODE == kUe8m0 ? e8m0_to_f32(st.sa[u][i] & 0xFF) : 1.0f;
                    cvt_fp8x32(st.a[u][i][0], st.a[u][i][1], sav_f, aq);
#pragma unroll
                    for (int j = 0; j < WN; j++) {
                        if (SMODE == kUe8m0) {
                            acc[i][j] = mfma_bf16_k128(aq, bq[j], acc[i][j]);
                        } else {
                            v4f t = mfma_bf16_k128(aq, bq[j], v4f{0.f, 0.f, 0.f, 0.f});
                            float sb = sbf[(size_t)(col_of[j] / 128) * kb128 + ks];
#pragma unroll
                            for (int v = 0; v < 4; v++) {
                                int row = min(m_base + i * 16 + 4 * kb + v, M - 1);
                                float sc = saf[(size_t)row * kb128 + ks] * sb;
                                acc[i][j][v] = acc[i][j][v] + t[v] * sc;
                            }
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    v8i a = frag_from(st.a[u][i][0], st.a[u][i][1]);
#pragma unroll
                    for (int j = 0; j < WN; j++) {
                        v8i b = BFP4 ? frag_from4(st.b[u][j][0])
                                     : frag_from(st.b[u][j][0], st.b[u][j][1]);
                        if (SMODE == kUe8m0) {
                            acc[i][j] = BFP4 ? mfma_scaled<kFmtFp8, kFmtFp4>(
                                                   a, b, acc[i][j], (int)st.sa[u][i],
                                                   (int)st.sb[u][j])
                                             : mfma_scaled<kFmtFp8, kFmtFp8>(
                                                   a, b, acc[i][j], (int)st.sa[u][i],
                                                   (int)st.sb[u][j]);
                        } else {
                            v4f t = mfma_scaled<kFmtFp8, kFmtFp8>(
                                a, b, v4f{0.f, 0.f, 0.f, 0.f}, kScaleOne, kScaleOne);
                            float sb = sbf[(size_t)(col_of[j] / 128) * kb128 + ks];
#pragma unroll
                            for (int v = 0; v < 4; v++) {
                                int row = min(m_base + i * 16 + 4 * kb + v, M - 1);
                                float sc = saf[(size_t)row * kb128 + ks] * sb;
                                acc[i][j][v] = acc[i][j][v] + t[v] * sc;
                            }
                        }
                    }
                }
            }
        }
    };

    // two register stages: the loads of stage n+1 are in flight while stage n
    // is converted and multiplied, so a wave waits on memory once, not once per
    // batch of U steps
    GemmStage<WM, WN, U> s0, s1;
    load(s0, k0);
    for (int ks0 = k0; ks0 < k1; ks0 += 2 * U) {
        if (ks0 + U < k1) load(s1, ks0 + U);
        compute(s0, ks0);
        if (ks0 + 2 * U < k1) load(s0, ks0 + 2 * U);
        if (ks0 + U < k1) compute(s1, ks0 + U);
    }

    if (GK > 1) {
        // ordered reduction of the K-split partials through LDS
        __shared__ float red[GK > 1 ? (GK - 1) * GM * WM * WN * 4 * 64 : 1];
        if (wk > 0) {
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        red[((((wk - 1) * GM + wm) * WM + i) * WN + j) * 256 + v * 64 + lane] =
                            acc[i][j][v];
        }
        __syncthreads();
        if (wk > 0) return;
#pragma unroll
        for (int s = 1; s < GK; s++)
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[i][j][v] =
                            acc[i][j][v] +
                            red[((((s - 1) * GM + wm) * WM + i) * WN + j) * 256 + v * 64 + lane];
    }

#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) {
            int col = n_base + j * 16 + r;
            if (col >= N) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                int row = m_base + i * 16 + 4 * kb + v;
                if (row >= M) continue;
                if (OMODE == kOutF32)
                    ((float *)C)[(size_t)row * N + col] = acc[i][j][v];
                else
                    ((uint16_t *)C)[(size_t)row * N + col] = f32_to_bf16(acc[i][j][v]);
            }
        }
}

// ---- K-parallel GEMM: one workgroup per 16 output columns -----------------
// HBM-bound shapes (M <= a few hundred, e.g. M=128, K=4096): the weight matrix
// must cross HBM exactly once, so a workgroup owns a 16-column strip of B for
// all K and up to 16*MF*GMH rows of A. Its GMH x GK waves split the rows in
// GMH halves and K in GK parts; a wave streams its K part in double-buffered
// register stages of U 128-K steps (clamped, unconditional loads: one wait per
// stage). The GK partial sums meet in LDS and are added in wave order
// (deterministic). f32-scale mode stages the activation scales of the
// workgroup's rows in LDS once, transposed to [step][row].
template <int MF, int U>
struct KpStage {
    uint4 a[U][MF][2];
    uint32_t sa[U][MF];
    uint4 b[U][2];
    uint32_t sb[U];
    float sbf[U];
};

constexpr int kKpMaxSaPerThread = 4;  // f32 A scales staged per thread (float4 each)

template <int MF, int GMH, int GK, bool BFP4, int SMODE, int OMODE, int U, bool EXACT>
__global__ __launch_bounds__(64 * GMH * GK) void gemm_kp_kernel(const uint8_t *A, const void *SA,
                                                                const uint8_t *__restrict__ B,
                                                                const void *__restrict__ SB,
                                                                void *__restrict__ C, int M,
                                                                int N, int K) {
    constexpr int kRows = 16 * MF * GMH;
    constexpr int kThreads = 64 * GMH * GK;
    extern __shared__ __align__(16) float kp_lds[];
    float *part = kp_lds;                      // [GK][kRows][16]
    float *sa_l = kp_lds + GK * kRows * 16;    // [ksteps][kRows] (f32-scale mode)
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wk = w % GK, wm = w / GK;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int mb = blockIdx.y * kRows;           // workgroup's first row
    const int ml = wm * 16 * MF;                 // wave's first row within the workgroup
    const int ksteps = K / 128;
    const int k0 = wk * ksteps / GK, k1 = (wk + 1) * ksteps / GK;
    const int kbn = K / 32, kb128 = K / 128;

    // f32 activation scales of the workgroup's rows: loads first
    float4 sav[kKpMaxSaPerThread];
    const int nsa = kRows * ksteps;  // <= kThreads * 4 * kKpMaxSaPerThread (checked on the host)
    if (SMODE == kF32s) {
        const float *saf = (const float *)SA;
#pragma unroll
        for (int j = 0; j < kKpMaxSaPerThread; j++) {
            // element e = row_local * ksteps + ks, four at a time (ksteps % 4 == 0)
            const int e = min((j * kThreads + t) * 4, nsa - 4);
            const int rl = e / ksteps, ks = e % ksteps;
            const int row = min(mb + rl, M - 1);
            sav[j] = *(const float4 *)(saf + (size_t)row * kb128 + ks);
        }
        mem_order();
    }

    const uint8_t *arow[MF];
    const uint8_t *sarow[MF];
#pragma unroll
    for (int i = 0; i < MF; i++) {
        const int row = min(mb + ml + 16 * i + r, M - 1);
        arow[i] = A + (size_t)row * K + (EXACT ? g * 32 : g * 16);
        sarow[i] = (const uint8_t *)SA + (size_t)row * kbn;
    }
    const int col = n0 + r;
    const uint8_t *brow = BFP4 ? B + (size_t)col * (K / 2) + g * 16
                               : B + (size_t)col * K + (EXACT ? g * 32 : g * 16);
    const uint8_t *sbrow = (const uint8_t *)SB + (size_t)(BFP4 ? col : col / 32) * kbn;
    const float *sbf_row = (const float *)SB + (size_t)(n0 / 128) * kb128;

    auto load = [&](KpStage<MF, U> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int ks = max(min(ks0 + u, k1 - 1), 0);
#pragma unroll
            for (int i = 0; i < MF; i++) {
                const uint8_t *p = arow[i] + (size_t)ks * 128;
                st.a[u][i][0] = ldg16(p);
                st.a[u][i][1] = ldg16(p + (EXACT ? 16 : 64));
                if (SMODE == kUe8m0) st.sa[u][i] = *(const uint32_t *)(sarow[i] + ks * 4) >> (8 * g);
            }
            if (BFP4) {
                st.b[u][0] = ldg16_stream(brow + (size_t)ks * 64);
            } else {
                const uint8_t *p = brow + (size_t)ks * 128;
                st.b[u][0] = ldg16_stream(p);
                st.b[u][1] = ldg16_stream(p + (EXACT ? 16 : 64));
            }
            if (SMODE == kUe8m0) st.sb[u] = *(const uint32_t *)(sbrow + ks * 4) >> (8 * g);
            else st.sbf[u] = sbf_row[ks];
        }
    };

    v4f acc[MF];
#pragma unroll
    for (int i = 0; i < MF; i++) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const KpStage<MF, U> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int ks = ks0 + u;
            if (ks >= k1) continue;  // uniform
            if (EXACT) {
                v8bf bq[4];
                const float sbv = SMODE == kUe8m0 ? e8m0_to_f32(st.sb[u] & 0xFF) : 1.0f;
                if (BFP4) cvt_fp4x32(st.b[u][0], sbv, bq);
                else cvt_fp8x32(st.b[u][0], st.b[u][1], sbv, bq);
#pragma unroll
                for (int i = 0; i < MF; i++) {
                    v8bf aq[4];
                    const float sav_f = SMODE == kUe8m0 ? e8m0_to_f32(st.sa[u][i] & 0xFF) : 1.0f;
                    cvt_fp8x32(st.a[u][i][0], st.a[u][i][1], sav_f, aq);
                    if (SMODE == kUe8m0) {
                        acc[i] = mfma_bf16_k128(aq, bq, acc[i]);
                    } else {
                        const v4f p = mfma_bf16_k128(aq, bq, v4f{0.f, 0.f, 0.f, 0.f});
                        const float4 sa4 = *(const float4 *)(sa_l + ks * kRows + ml + 16 * i + 4 * g);
                        const float sa_v[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[i][v] = acc[i][v] + p[v] * (sa_v[v] * st.sbf[u]);
                    }
                }
            } else {
                const v8i b = BFP4 ? frag_from4(st.b[u][0]) : frag_from(st.b[u][0], st.b[u][1]);
#pragma unroll
                for (int i = 0; i < MF; i++) {
                    const v8i a = frag_from(st.a[u][i][0], st.a[u][i][1]);
                    if (SMODE == kUe8m0) {
                        acc[i] = BFP4 ? mfma_scaled<kFmtFp8, kFmtFp4>(a, b, acc[i], (int)st.sa[u][i],
                                                                      (int)st.sb[u])
                                      : mfma_scaled<kFmtFp8, kFmtFp8>(a, b, acc[i], (int)st.sa[u][i],
                                                                      (int)st.sb[u]);
                    } else {
                        const v4f p = mfma_scaled<kFmtFp8, kFmtFp8>(a, b, v4f{0.f, 0.f, 0.f, 0.f},
                                                                    kScaleOne, kScaleOne);
                        const float4 sa4 = *(const float4 *)(sa_l + ks * kRows + ml + 16 * i + 4 * g);
                        const float sa_v[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[i][v] = acc[i][v] + p[v] * (sa_v[v] * st.sbf[u]);
                    }
                }
            }
        }
    };

    KpStage<MF, U> s0, s1;
    load(s0, k0);
    mem_order();
    load(s1, k0 + U);
    mem_order();
    if (SMODE == kF32s) {
#pragma unroll
        for (int j = 0; j < kKpMaxSaPerThread; j++) {
            const int e = (j * kThreads + t) * 4;
            if (e >= nsa) continue;
            const int rl = e / ksteps, ks = e % ksteps;
            const float v[4] = {sav[j].x, sav[j].y, sav[j].z, sav[j].w};
#pragma unroll
            for (int c = 0; c < 4; c++) sa_l[(ks + c) * kRows + rl] = v[c];
        }
        lds_barrier();
    }

    // steady state: both stages reloaded unconditionally (straight-line body)
    const int nst = (k1 - k0 + U - 1) / U;
    int i = 0, ks0 = k0;
    for (; i + 3 < nst; i += 2, ks0 += 2 * U) {
        compute(s0, ks0);
        load(s0, ks0 + 2 * U);
        compute(s1, ks0 + U);
        load(s1, ks0 + 3 * U);
    }
    const int rest = nst - i;
    if (rest == 3) {
        compute(s0, ks0);
        load(s0, ks0 + 2 * U);
        compute(s1, ks0 + U);
        compute(s0, ks0 + 2 * U);
    } else {
        if (rest >= 1) compute(s0, ks0);
        if (rest == 2) compute(s1, ks0 + U);
    }

    // D[m][n]: lane -> row 4g+v of fragment i, column r
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
        for (int v = 0; v < 4; v++) part[(wk * kRows + ml + 16 * f + 4 * g + v) * 16 + r] = acc[f][v];
    __syncthreads();
    for (int o = t; o < kRows * 16; o += kThreads) {
        const int rl = o >> 4, c = o & 15;
        const int row = mb + rl;
        if (row >= M) continue;
        float sum = part[rl * 16 + c];
#pragma unroll
        for (int q = 1; q < GK; q++) sum = sum + part[(q * kRows + rl) * 16 + c];
        if (OMODE == kOutF32) ((float *)C)[(size_t)row * N + n0 + c] = sum;
        else ((uint16_t *)C)[(size_t)row * N + n0 + c] = f32_to_bf16(sum);
    }
}

template <int MF, int GMH, int GK, bool BFP4, int SMODE, int OMODE, int U>
static int launch_kp(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                     int m, int n, int k, hipStream_t stream) {
    constexpr int rows = 16 * MF * GMH, threads = 64 * GMH * GK;
    const int ksteps = k / 128;
    if (SMODE == kF32s && (rows * ksteps > threads * 4 * kKpMaxSaPerThread || ksteps % 4 ||
                           ((uintptr_t)sa & 15)))
        return -1;  // caller falls back to the general kernel
    size_t lds = (size_t)GK * rows * 16 * 4 + (SMODE == kF32s ? (size_t)ksteps * rows * 4 : 0);
    dim3 grid((unsigned)(n / 16), (unsigned)((m + rows - 1) / rows));
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_kp_kernel<MF, GMH, GK, BFP4, SMODE, OMODE, U, false>), grid,
                           dim3(threads), lds, stream, a, sa, b, sb, out, m, n, k);
    else
        hipLaunchKernelGGL((gemm_kp_kernel<MF, GMH, GK, BFP4, SMODE, OMODE, U, true>), grid,
                           dim3(threads), lds, stream, a, sa, b, sb, out, m, n, k);
    return launch_status();
}

// ---- split-K GEMM with the A block in LDS ---------------------------------
// For M-batch shapes every CU would otherwise pull all of A through L2 (the
// L2->CU rate, ~14 TB/s for the whole chip, bounds a 16-column strip kernel at
// M=128, K=4096 near 9 us). Here a workgroup owns a 128 x 64 output tile and a
// K range of at most 8 steps (1024 K): its A block (128 x <=1024 e4m3 + scales)
// is copied into LDS once by direct global->LDS loads, and its 64 columns of W
// stream from HBM in two register stages of four 128-K steps. The 8 waves own
// 32 x 32 sub-tiles (2 x 2 MFMA fragments), so every A and W fragment feeds two
// MFMA tiles. With S > 1 K ranges the splits write f32 partials to the
// workspace and sk_reduce_kernel adds them in split order (deterministic).
// Workgroups are numbered so that the S splits of a tile share an XCD
// (dispatch goes round-robin over the 8 XCDs).
constexpr int kSkBM = 128, kSkBN = 64, kSkU = 4, kSkMaxSteps = 2 * kSkU;
constexpr int kSkThreads = 512;

template <bool BFP4>
struct SkStage {
    uint4 b[kSkU][2][BFP4 ? 1 : 2];  // W: 2 column fragments
    uint32_t sb[kSkU][2];            // UE8M0 weight scale of the lane's K block
    float sbf[kSkU];                 // f32 weight scale (128-block; uniform)
};

// Copy rows of `row_bytes` (row i at src(i)) into an LDS image with a row
// pitch of `pitch` bytes (>= row_bytes; the padding spreads rows over the LDS
// banks), `total` = rows * pitch, with direct loads of PIECE bytes per lane
// (16 or 4). Padding bytes get a copy of the row's last piece.
template <int PIECE, class Src>
__device__ __forceinline__ void sk_dma(Src src, int row_bytes, int pitch, int total, uint8_t *lds,
                                       int w, int lane) {
    const int per = 64 * PIECE;
    const int n = (total + per - 1) / per;
    for (int c = w; c < n; c += kSkThreads / 64) {
        const int o = min(c * per + lane * PIECE, total - PIECE);
        const int row = o / pitch, col = min(o - row * pitch, row_bytes - PIECE);
        const void *gp = (const void *)(src(row) + col);
        auto *lp = (__attribute__((address_space(3))) void *)(lds + c * per);
        if constexpr (PIECE == 16) __builtin_amdgcn_global_load_lds(gp, lp, 16, 0, 0);
        else __builtin_amdgcn_global_load_lds(gp, lp, 4, 0, 0);
    }
}

template <bool BFP4, int SMODE, int OMODE, bool EXACT>
__global__ __launch_bounds__(kSkThreads) void gemm_sk_kernel(
    const uint8_t *A, const void *SA, const uint8_t *B, const void *SB,
    void *__restrict__ C, int M, int N, int K, int S, int ntn, int tiles,
    float *__restrict__ part) {
    extern __shared__ __align__(16) uint8_t sk_lds[];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r = lane & 15, g = lane >> 4;
    // XCD-aware numbering: ids x, x+8, x+16, ... hold the tiles t = x (mod 8)
    const int id = blockIdx.x, xcd = id & 7, q = id >> 3;
    const int tile = xcd + 8 * (q / S), s = q % S;
    if (tile >= tiles) return;  // whole workgroup
    const int mb = tile / ntn, nt = tile % ntn;
    const int m0 = mb * kSkBM, n0 = nt * kSkBN;
    const int ksteps = K / 128, kbn = K / 32, kb128 = K / 128;
    const int ka = s * ksteps / S, kz = (s + 1) * ksteps / S, nks = kz - ka;  // nks <= 8
    const int kr = nks * 128;                           // A bytes per row
    const int kp = kr + 16;                             // LDS row pitch (bank spread)
    uint8_t *a_l = sk_lds;                              // [128][kp] e4m3
    uint8_t *as_l = sk_lds + (size_t)kSkBM * kp;        // UE8M0 [128][nks*4] or f32 [128][nks]
    const int wm = w & 3, wn = w >> 2;

    // W columns n0 + 32 wn + 16 j + r, steps [ka, kz)
    const uint8_t *brow[2];
    const uint8_t *sbrow[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int col = min(n0 + 32 * wn + 16 * j + r, N - 1);
        brow[j] = BFP4 ? B + (size_t)col * (K / 2) + g * 16
                       : B + (size_t)col * K + (EXACT ? g * 32 : g * 16);
        sbrow[j] = (const uint8_t *)SB + (size_t)(BFP4 ? col : col / 32) * kbn;
    }
    const float *sbf_row = (const float *)SB + (size_t)(n0 / 128) * kb128;
    auto load = [&](SkStage<BFP4> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < kSkU; u++) {
            const int ks = max(min(ks0 + u, kz - 1), 0);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                if (BFP4) {
                    st.b[u][j][0] = ldg16_stream(brow[j] + (size_t)ks * 64);
                } else {
                    const uint8_t *p = brow[j] + (size_t)ks * 128;
                    st.b[u][j][0] = ldg16_stream(p);
                    st.b[u][j][BFP4 ? 0 : 1] = ldg16_stream(p + (EXACT ? 16 : 64));
                }
                if (SMODE == kUe8m0) st.sb[u][j] = *(const uint32_t *)(sbrow[j] + ks * 4) >> (8 * g);
            }
            if (SMODE == kF32s) st.sbf[u] = sbf_row[ks];
        }
    };
    // 1. the A block and its scales into LDS (rows past M repeat row M-1), issued
    //    first so that a wait for W stage 0 also covers them
    sk_dma<16>([&](int i) { return A + (size_t)min(m0 + i, M - 1) * K + (size_t)ka * 128; }, kr,
               kp, kSkBM * kp, a_l, w, lane);
    if (SMODE == kUe8m0)
        sk_dma<4>([&](int i) {
            return (const uint8_t *)SA + (size_t)min(m0 + i, M - 1) * kbn + ka * 4; },
                  nks * 4, nks * 4, kSkBM * nks * 4, as_l, w, lane);
    else
        sk_dma<4>([&](int i) {
            return (const uint8_t *)((const float *)SA + (size_t)min(m0 + i, M - 1) * kb128 + ka); },
                  nks * 4, nks * 4, kSkBM * nks * 4, as_l, w, lane);
    mem_order();
    // 2. the two W stages
    SkStage<BFP4> s0, s1;
    load(s0, ka);
    mem_order();
    load(s1, ka + kSkU);
    mem_order();
    // wait until at most stage 1's weight loads are outstanding (a lower bound
    // on the loads stage 1 issues: its scale loads only make the wait
    // stricter): this wave's LDS copies and stage 0 have landed
    constexpr int kStage1Loads = kSkU * 2 * (BFP4 ? 1 : 2);
    __builtin_amdgcn_s_waitcnt((kStage1Loads & 15) | ((kStage1Loads >> 4) << 14) | (7 << 4) |
                               (15 << 8));
    raw_barrier();

    // 3. multiply
    v4f acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const SkStage<BFP4> &st, int ks0) {
#pragma unroll
        for (int u = 0; u < kSkU; u++) {
            const int ks = ks0 + u;
            if (ks >= kz) continue;  // uniform
            const int kl = ks - ka;
            if (EXACT) {
                v8bf bq[2][4];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float sbv = SMODE == kUe8m0 ? e8m0_to_f32(st.sb[u][j] & 0xFF) : 1.0f;
                    if (BFP4) cvt_fp4x32(st.b[u][j][0], sbv, bq[j]);
                    else cvt_fp8x32(st.b[u][j][0], st.b[u][j][BFP4 ? 0 : 1], sbv, bq[j]);
                }
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int ml = 32 * wm + 16 * i + r;
                    const uint8_t *ap = a_l + ml * kp + kl * 128 + g * 32;
                    const float sav = SMODE == kUe8m0 ? e8m0_to_f32(as_l[ml * nks * 4 + kl * 4 + g])
                                                      : 1.0f;
                    v8bf aq[4];
                    cvt_fp8x32(*(const uint4 *)ap, *(const uint4 *)(ap + 16), sav, aq);
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        if (SMODE == kUe8m0) {
                            acc[i][j] = mfma_bf16_k128(aq, bq[j], acc[i][j]);
                        } else {
                            const v4f pr = mfma_bf16_k128(aq, bq[j], v4f{0.f, 0.f, 0.f, 0.f});
                            const float *sar = (const float *)as_l + (32 * wm + 16 * i + 4 * g) * nks + kl;
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                acc[i][j][v] = acc[i][j][v] + pr[v] * (sar[v * nks] * st.sbf[u]);
                        }
                    }
                }
            } else {
                v8i bf[2];
#pragma unroll
                for (int j = 0; j < 2; j++)
                    bf[j] = BFP4 ? frag_from4(st.b[u][j][0])
                                 : frag_from(st.b[u][j][0], st.b[u][j][BFP4 ? 0 : 1]);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int ml = 32 * wm + 16 * i + r;
                    const uint8_t *ap = a_l + ml * kp + kl * 128 + g * 16;
                    const v8i af = frag_from(*(const uint4 *)ap, *(const uint4 *)(ap + 64));
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        if (SMODE == kUe8m0) {
                            const int sa = as_l[ml * nks * 4 + kl * 4 + g];
                            acc[i][j] = BFP4 ? mfma_scaled<kFmtFp8, kFmtFp4>(af, bf[j], acc[i][j], sa,
                                                                             (int)st.sb[u][j])
                                             : mfma_scaled<kFmtFp8, kFmtFp8>(af, bf[j], acc[i][j], sa,
                                                                             (int)st.sb[u][j]);
                        } else {
                            const v4f pr = mfma_scaled<kFmtFp8, kFmtFp8>(
                                af, bf[j], v4f{0.f, 0.f, 0.f, 0.f}, kScaleOne, kScaleOne);
                            const float *sar = (const float *)as_l + (32 * wm + 16 * i + 4 * g) * nks + kl;
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                acc[i][j][v] = acc[i][j][v] + pr[v] * (sar[v * nks] * st.sbf[u]);
                        }
                    }
                }
            }
        }
    };
    compute(s0, ka);
    compute(s1, ka + kSkU);

    // 4. store: C directly (one split) or the split's partial
    auto store_c = [&](int row, int col, float v) {
        if (OMODE == kOutF32) ((float *)C)[(size_t)row * N + col] = v;
        else ((uint16_t *)C)[(size_t)row * N + col] = f32_to_bf16(v);
    };
    const size_t mpad = (size_t)((M + kSkBM - 1) / kSkBM) * kSkBM;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + 32 * wn + 16 * j + r;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + 32 * wm + 16 * i + 4 * g + v;
                if (S == 1) {
                    if (row < M && col < N) store_c(row, col, acc[i][j][v]);
                } else if (col < N) {
                    part[((size_t)s * mpad + row) * N + col] = acc[i][j][v];
                }
            }
        }
}

// Sum of the S partials of every output in split order (deterministic);
// the kernel boundary after gemm_sk_kernel makes them visible.
template <int OMODE>
__global__ __launch_bounds__(256) void sk_reduce_kernel(const float *__restrict__ part,
                                                        void *__restrict__ C, int M, int N, int S,
                                                        size_t mpad) {
    const size_t o = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const size_t total = (size_t)M * N;
    if (o >= total) return;
    const size_t plane = mpad * N;
    float4 acc = *(const float4 *)(part + o);
    for (int q = 1; q < S; q++) {
        const float4 v = *(const float4 *)(part + (size_t)q * plane + o);
        acc.x = acc.x + v.x;
        acc.y = acc.y + v.y;
        acc.z = acc.z + v.z;
        acc.w = acc.w + v.w;
    }
    if (OMODE == kOutF32) {
        *(float4 *)((float *)C + o) = acc;
    } else {
        uint16_t *c = (uint16_t *)C + o;
        *(uint2 *)c = uint2{(uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16),
                            (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16)};
    }
}

// Workspace for the split-K kernel, per device (ws_set_gemm_workspace).
struct SkWorkspace {
    uint8_t *ptr;
    size_t bytes;
};
static SkWorkspace g_sk_ws[64];

static SkWorkspace &sk_ws() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    return g_sk_ws[dev];
}

// Splits for (M, N, K): every split at most 8 steps, enough workgroups to
// cover the CUs; 0 when the split-K kernel does not apply.
static int sk_splits(int M, int N, int K, size_t ws_bytes) {
    const int ksteps = K / 128;
    const int tiles = ((M + kSkBM - 1) / kSkBM) * ((N + kSkBN - 1) / kSkBN);
    int S = (ksteps + kSkMaxSteps - 1) / kSkMaxSteps;
    const int want = (cu_count() + tiles - 1) / tiles;
    if (want > S) S = want;
    if (S > ksteps) S = ksteps;
    const size_t mpad = (size_t)((M + kSkBM - 1) / kSkBM) * kSkBM;
    if (S > 1 && (size_t)S * mpad * N * 4 > ws_bytes) return 0;
    return S;
}

template <bool BFP4, int SMODE, int OMODE>
static int launch_sk(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                     int m, int n, int k, hipStream_t stream) {
    SkWorkspace &wsp = sk_ws();
    if (!wsp.ptr) return -1;
    const int S = sk_splits(m, n, k, wsp.bytes);
    if (S <= 0) return -1;
    const int ksteps = k / 128;
    const int nks_max = (ksteps + S - 1) / S;
    const int ntn = (n + kSkBN - 1) / kSkBN;
    const int tiles = ((m + kSkBM - 1) / kSkBM) * ntn;
    const size_t lds = (size_t)kSkBM * (nks_max * 128 + 16) + (size_t)kSkBM * nks_max * 4;
    const unsigned grid = (unsigned)(8 * ((tiles + 7) / 8) * S);
    float *part = (float *)wsp.ptr;
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_sk_kernel<BFP4, SMODE, OMODE, false>), dim3(grid),
                           dim3(kSkThreads), lds, stream, a, sa, b, sb, out, m, n, k, S, ntn,
                           tiles, part);
    else
        hipLaunchKernelGGL((gemm_sk_kernel<BFP4, SMODE, OMODE, true>), dim3(grid),
                           dim3(kSkThreads), lds, stream, a, sa, b, sb, out, m, n, k, S, ntn,
                           tiles, part);
    int rc = launch_status();
    if (rc || S == 1) return rc;
    const size_t mpad = (size_t)((m + kSkBM - 1) / kSkBM) * kSkBM;
    const size_t quads = ((size_t)m * n + 3) / 4;
    hipLaunchKernelGGL((sk_reduce_kernel<OMODE>), dim3((unsigned)((quads + 255) / 256)), dim3(256),
                       0, stream, part, out, m, n, S, mpad);
    return launch_status();
}

// General kernel configurations, used where the K-parallel kernel does not
// stage a shape (f32 scales with K > 8192 or unaligned scale rows), or when
// WS_GEMM_CFG forces one (0: 16 x 16 tiles, 1: 64 x 16 tiles) for measurements.
template <int WM, int WN, int GM, int GK, bool BFP4, int SMODE, int OMODE, int U>
static int launch_cfg(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                      int m, int n, int k, hipStream_t stream) {
    constexpr int tm = 16 * WM * GM, tn = 16 * WN;
    dim3 grid((n + tn - 1) / tn, (m + tm - 1) / tm);
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_kernel<WM, WN, GM, GK, BFP4, SMODE, OMODE, U, false>), grid,
                           dim3(64 * GM * GK), 0, stream, a, sa, b, sb, out, m, n, k);
    else
        hipLaunchKernelGGL((gemm_kernel<WM, WN, GM, GK, BFP4, SMODE, OMODE, U, true>), grid,
                           dim3(64 * GM * GK), 0, stream, a, sa, b, sb, out, m, n, k);
    return launch_status();
}

static int forced_cfg() {
    const char *e = getenv("WS_GEMM_CFG");
    return e ? atoi(e) : -1;
}

template <bool BFP4, int SMODE, int OMODE>
static int gemm_dispatch(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb,
                         void *out, int64_t m, int64_t n, int64_t k, hipStream_t stream) {
    if (!a || !sa || !b || !sb || !out) return WS_ERR_INVALID_ARG;
    if (m <= 0 || n <= 0 || k <= 0) return WS_ERR_INVALID_ARG;
    if (k % 128 || n % 16 || m > (1 << 24) || n > (1 << 24) || k > (1 << 24)) return WS_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)b) & 15 || ((uintptr_t)sa | (uintptr_t)sb) & 3)
        return WS_ERR_INVALID_ARG;
    int M = (int)m, N = (int)n, K = (int)k;
    int cfg = forced_cfg();
    if (cfg < 0) {
        // K-parallel strips (one workgroup per 16 columns); -1: shape outside
        // what they stage, use the general kernel
        // split-K unless the 16-column strips alone fill the chip in one round
        // (measured at M=128, K=4096: strips win at N=4096, split-K at N=2048
        // and N=12288)
        const int strips = N / 16, cus = cu_count();
        const bool strips_fit = strips >= cus * 3 / 4 && strips <= cus * 3 / 2;
        int rc = (M > 16 && !strips_fit)
                     ? launch_sk<BFP4, SMODE, OMODE>(a, sa, b, sb, out, M, N, K, stream)
                     : -1;
        if (rc >= 0) return rc;
        if (M <= 16) rc = launch_kp<1, 1, 8, BFP4, SMODE, OMODE, 2>(a, sa, b, sb, out, M, N, K, stream);
        else if (M <= 32) rc = launch_kp<2, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream);
        else if (M <= 64) rc = launch_kp<4, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream);
        else rc = launch_kp<4, 2, 4, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream);
        if (rc >= 0) return rc;
        cfg = (M <= 16) ? 0 : 1;
    }
    switch (cfg) {
        case 0:  // 16 x 16 tile, K split over 8 waves
            return launch_cfg<1, 1, 1, 8, BFP4, SMODE, OMODE, 4>(a, sa, b, sb, out, M, N, K, stream);
        case 1:  // 64 x 16 tile, K split over 4 (16 waves)
            return launch_cfg<1, 1, 4, 4, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream);
        default:
            return WS_ERR_INVALID_ARG;
    }
}

}  // namespace ws

using namespace ws;

extern "C" {

size_t ws_gemm_workspace_size(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 128) return 0;
    const int64_t ksteps = k / 128;
    int64_t S = (ksteps + kSkMaxSteps - 1) / kSkMaxSteps;
    const int64_t tiles = ((m + kSkBM - 1) / kSkBM) * ((n + kSkBN - 1) / kSkBN);
    const int64_t want = (cu_count() + tiles - 1) / tiles;
    if (want > S) S = want;
    if (S > ksteps) S = ksteps;
    const int64_t mpad = (m + kSkBM - 1) / kSkBM * kSkBM;
    return (size_t)(S > 1 ? S : 1) * mpad * n * 4;
}

int ws_set_gemm_workspace(void *workspace, size_t bytes, ws_stream_t stream) {
    (void)stream;
    SkWorkspace &wsp = sk_ws();
    if (!workspace || bytes == 0) {
        wsp.ptr = nullptr;
        wsp.bytes = 0;
        return workspace ? WS_ERR_INVALID_ARG : WS_OK;
    }
    if ((uintptr_t)workspace & 255) return WS_ERR_INVALID_ARG;
    wsp.ptr = (uint8_t *)workspace;
    wsp.bytes = bytes;
    return WS_OK;
}

int ws_fp8_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp8_gemm_tile(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp8_gemm_bf16(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     uint16_t *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutBf16>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp8_gemm_f32s(const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                     void *out, int out_bf16, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    if (out_bf16)
        return gemm_dispatch<false, kF32s, kOutBf16>(a, sa, b, sb, out, m, n, k, stream);
    return gemm_dispatch<false, kF32s, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp4_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<true, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp4_gemm_tile(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<true, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

}  // extern "C"
