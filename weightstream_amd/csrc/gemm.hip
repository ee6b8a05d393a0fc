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
#include "ws_gate.hpp"
#include "ws_kp.hpp"

#include <stdlib.h>

#include <mutex>

namespace ws {

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
                    st.b[u][j][0] = ldg16(brow[j] + (size_t)ks * 64);
                } else {
                    const uint8_t *p = brow[j] + (size_t)ks * 128;
                    st.b[u][j][0] = ldg16(p);
                    st.b[u][j][1] = ldg16(p + (EXACT ? 16 : 64));
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

template <int MF, int NF, int GMH, int GK, bool BFP4, int SMODE, int OMODE, int U, bool EXACT,
          bool AF32 = false, bool ALDS = false>
__global__ __launch_bounds__(64 * GMH * GK) void gemm_kp_kernel(const uint8_t *A, const void *SA,
                                                                const uint8_t *__restrict__ B,
                                                                const void *__restrict__ SB,
                                                                void *__restrict__ C, int M,
                                                                int N, int K, int S,
                                                                float *__restrict__ part_out,
                                                                int sb_div, const float *aux,
                                                                float limit, int jstride) {
    kp_body<MF, NF, GMH, GK, BFP4, SMODE, OMODE, U, EXACT, AF32, ALDS>(
        blockIdx.x, blockIdx.y, blockIdx.z, A, SA, B, SB, C, M, N, K, S, part_out, sb_div, aux,
        limit, jstride);
}

// out = the S partial planes [S][M][N] summed in plane order (deterministic)
template <int OMODE>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float *__restrict__ part,
                                                          void *__restrict__ C, int64_t mn,
                                                          int S) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= mn) return;  // mn % 4 == 0 (N % 16 == 0)
    float4 acc = *(const float4 *)(part + i);
    for (int z = 1; z < S; z++) {
        const float4 v = *(const float4 *)(part + (size_t)z * mn + i);
        acc.x = acc.x + v.x;
        acc.y = acc.y + v.y;
        acc.z = acc.z + v.z;
        acc.w = acc.w + v.w;
    }
    if (OMODE == kOutF32) {
        *(float4 *)((float *)C + i) = acc;
    } else {
        uint16_t *o = (uint16_t *)C + i;
        *(uint2 *)o = uint2{(uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16),
                            (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16)};
    }
}

template <int MF, int NF, int GMH, int GK, bool BFP4, int SMODE, int OMODE, int U>
static int launch_kp(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                     int m, int n, int k, hipStream_t stream, int S = 1, float *part = nullptr,
                     int sb_div = 32, const float *aux = nullptr) {
    constexpr int rows = 16 * MF * GMH, threads = 64 * GMH * GK;
    if (n % (16 * NF)) return -1;
    const int ksteps = k / 128;
    constexpr bool stage = SMODE == kF32s || rows > 16;
    if (stage && rows * ksteps > threads * kKpMaxSaWords)
        return -1;  // caller falls back to the general kernel
    // blocks of 32 or 64 rows read A through LDS (kp_body's ALDS)
    constexpr bool alds = MF >= 2 && GMH == 1 && U == 1;
    const size_t lds = kp_head_bytes<MF, NF, GMH, GK, alds>() + (size_t)ksteps * rows * 4;
    if (lds > 160 * 1024) return -1;
    if (S < 1 || (S > 1 && !part)) return -1;
    if (S > 1 && (OMODE == kOutAcc || OMODE == kOutAcc2)) return -1;  // the reduction writes
    dim3 grid((unsigned)(n / (16 * NF)), (unsigned)((m + rows - 1) / rows), (unsigned)S);
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_kp_kernel<MF, NF, GMH, GK, BFP4, SMODE, OMODE, U, false, false, alds>),
                           grid, dim3(threads), lds, stream, a, sa, b, sb, out, m, n, k, S, part,
                           sb_div, aux, 0.0f, 16);
    else
        hipLaunchKernelGGL((gemm_kp_kernel<MF, NF, GMH, GK, BFP4, SMODE, OMODE, U, true, false, alds>),
                           grid, dim3(threads), lds, stream, a, sa, b, sb, out, m, n, k, S, part,
                           sb_div, aux, 0.0f, 16);
    int rc = launch_status();
    if (rc || S == 1) return rc;
    const int64_t mn = (int64_t)m * n;
    hipLaunchKernelGGL((split_reduce_kernel<OMODE>), dim3((unsigned)((mn / 4 + 255) / 256)),
                       dim3(256), 0, stream, part, out, mn, S);
    return launch_status();
}

// The fused GEMVs (M <= 16, FP8 weights with 32 x 32 UE8M0 scales, f32
// activations quantised in the kernel): the 16-column-strip kernel with
// 8 K waves and no K split, so every output is the same sum, bit for bit,
// as ws_emit8 followed by ws_fp8_gemm (whose kernel this is for M <= 16 and
// K <= 8192). OMODE kOutAcc / kOutAcc2 write n columns; kOutSwiglu writes
// h [m][n] from the gate rows [0, n) and up rows [n, 2n) of the weights.
int kp_gemv_fused(int omode, const float *x, const uint8_t *w, const uint8_t *sw, float *out,
                  const float *aux, float limit, int64_t m, int64_t n, int64_t k,
                  hipStream_t stream) {
    if (!x || !w || !sw || !out || (omode == kOutAcc2 && !aux)) return WS_ERR_INVALID_ARG;
    if (m <= 0 || m > 16 || n <= 0 || k <= 0) return WS_ERR_INVALID_ARG;
    if (k % 128 || n % 16 || k > 8192 || n > (1 << 24)) return WS_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out | (uintptr_t)aux) & 15 ||
        (uintptr_t)sw & 3)
        return WS_ERR_INVALID_ARG;
    const int nf = omode == kOutSwiglu ? 2 : 1;
    const size_t lds = (size_t)8 * 16 * 16 * nf * 4 + (size_t)m * (k + 16) + (size_t)m * (k / 32);
    if (lds > 160 * 1024) return WS_ERR_SHAPE;
    const dim3 grid((unsigned)(n / 16)), block(512);
    const bool ex = math_mode() == WS_MATH_EXACT;
    const int M = (int)m, N = (int)n, K = (int)k;
#define WS_KPF(OM, NFV, E)                                                                     \
    hipLaunchKernelGGL((gemm_kp_kernel<1, NFV, 1, 8, false, kUe8m0, OM, 1, E, true>), grid, block, \
                       lds, stream, (const uint8_t *)x, (const void *)nullptr, w, (const void *)sw, \
                       (void *)out, M, N, K, 1, (float *)nullptr, 32, aux, limit, N)
    switch (omode) {
        case kOutAcc: if (ex) WS_KPF(kOutAcc, 1, true); else WS_KPF(kOutAcc, 1, false); break;
        case kOutAcc2: if (ex) WS_KPF(kOutAcc2, 1, true); else WS_KPF(kOutAcc2, 1, false); break;
        case kOutSwiglu: if (ex) WS_KPF(kOutSwiglu, 2, true); else WS_KPF(kOutSwiglu, 2, false); break;
        default: return WS_ERR_INVALID_ARG;
    }
#undef WS_KPF
    return launch_status();
}

// The gate logits and the shared expert's gate/up GEMV + SwiGLU in one
// launch: both read h and neither reads the other's output. The logits are a
// latency-bound sequential chain per expert (two waves on each of the first
// ceil(E / 4) x m workgroups); the GEMV is a weight stream over the next
// inter / 16 workgroups. Each part is the same code, and gives the same bits,
// as its own kernel (gate_logits_pc_kernel<4, 1, f32>; the kOutSwiglu GEMV).
template <bool EXACT>
__global__ __launch_bounds__(512) void gate_w13_kernel(const float *h, const float *gw,
                                                       float *logits, int m, int dim,
                                                       int n_experts, const uint8_t *w13,
                                                       const uint8_t *s13, float *hs, int inter,
                                                       float limit) {
    const int gx = (n_experts + 3) / 4, n_gate = gx * m;
    const int b = blockIdx.x;
    if (b < n_gate) {
        gate_pc_body<4, 1, false>(b % gx, b / gx, h, gw, logits, m, dim, n_experts);
        return;
    }
    kp_body<1, 2, 1, 8, false, kUe8m0, kOutSwiglu, 1, EXACT, true>(
        b - n_gate, 0, 0, (const uint8_t *)h, nullptr, w13, s13, hs, m, inter, dim, 1, nullptr, 32,
        nullptr, limit, inter);
}

int gate_w13_launch(const float *h, const float *gw, float *logits, const uint8_t *w13,
                    const uint8_t *s13, float *hs, int64_t m, int64_t dim, int64_t n_experts,
                    int64_t inter, float limit, hipStream_t stream) {
    if (!h || !gw || !logits || !w13 || !s13 || !hs) return WS_ERR_INVALID_ARG;
    if (m <= 0 || m > 8 || dim <= 0 || n_experts <= 0 || inter <= 0) return WS_ERR_INVALID_ARG;
    if (dim % kGC || dim > 8192 || inter % 16 || inter > (1 << 20) || n_experts > (1 << 16))
        return WS_ERR_SHAPE;
    if (((uintptr_t)h | (uintptr_t)w13 | (uintptr_t)hs) & 15 || (uintptr_t)s13 & 3)
        return WS_ERR_INVALID_ARG;
    using G = GateGeom<4, 1, false>;
    const size_t gate_lds = (size_t)kGS * G::kStage + (size_t)2 * 4 * kPcPitch * 4;
    const size_t kp_lds = (size_t)8 * 16 * 32 * 4 + (size_t)m * (dim + 16) + (size_t)m * (dim / 32);
    const size_t lds = gate_lds > kp_lds ? gate_lds : kp_lds;
    const unsigned grid = (unsigned)((n_experts + 3) / 4 * m + inter / 16);
    if (math_mode() == WS_MATH_EXACT)
        hipLaunchKernelGGL(gate_w13_kernel<true>, dim3(grid), dim3(512), lds, stream, h, gw, logits,
                           (int)m, (int)dim, (int)n_experts, w13, s13, hs, (int)inter, limit);
    else
        hipLaunchKernelGGL(gate_w13_kernel<false>, dim3(grid), dim3(512), lds, stream, h, gw,
                           logits, (int)m, (int)dim, (int)n_experts, w13, s13, hs, (int)inter,
                           limit);
    return launch_status();
}

// K splits for a 16-column-strip GEMM of at most 16 rows: enough to give
// every CU a workgroup when the strips alone leave most of the chip idle and
// each wave would otherwise chain more than 8 steps of 128 K (K > 8192),
// each split at least one step per wave (8 waves); 1 when no split pays or
// the workspace is too small. Measured at M=1: N=1280, K=15360 10.2 against
// 15.2 us; at K=5120 (N = 512, 1280) the reduction launch costs more than
// the split gains (7.3 against 6.9 us).
static int strip_splits(int M, int N, int K, size_t ws_bytes) {
    const int wgs = N / 16, ksteps = K / 128;
    if (ksteps <= 8 * 8) return 1;
    int S = cu_count() / (wgs > 0 ? wgs : 1);
    if (S > ksteps / 8) S = ksteps / 8;
    if (S < 2) return 1;
    if ((size_t)S * M * N * 4 > ws_bytes) return 1;
    return S;
}

// ---- A-resident GEMM: a 32-row block of A in LDS, K split over 8 waves ----
// For M of a few hundred with K <= 4096 (M = 128: the projection shapes). A
// workgroup owns 32 rows x 16*NF columns and the whole K. Its 32 rows of A
// (one contiguous block of M x K row-major e4m3) and their scales are copied
// once into LDS by direct global->LDS loads (rows padded to K + 16 bytes, so
// the 16 rows one read touches fall on distinct banks); the weight rows are
// streamed into registers in double-buffered stages (each weight byte is read
// once). Wave w multiplies K part w of the tile; the 8 partial tiles meet in
// LDS (reusing the A image) and are added in wave order (deterministic).
// Every A element is converted once per workgroup, and nothing is re-read
// from HBM: A is 0.5 MB, the weights cross HBM once.
constexpr int kAlRows = 32, kAlWaves = 8;

__host__ __device__ constexpr size_t al_a_bytes(int K) {
    return ((size_t)kAlRows * (K + 16) + 1023) / 1024 * 1024;
}
// scales of the 32 rows: K / 32 bytes per row in both scale modes (K/32
// UE8M0 bytes, or K/128 f32), padded to whole 1 KB pieces
__host__ __device__ constexpr size_t al_s_bytes(int K) {
    return ((size_t)kAlRows * (K / 32) + 1023) / 1024 * 1024;
}

template <int NF>
struct AlStage {
    uint4 b[NF][2];
    uint32_t sb[NF];
    float sbf;
};

template <int NF, int SMODE, int OMODE, bool EXACT>
__global__ __launch_bounds__(64 * kAlWaves) void gemm_al_kernel(const uint8_t *A, const void *SA,
                                                                const uint8_t *B, const void *SB,
                                                                void *__restrict__ C, int M, int N,
                                                                int K) {
    constexpr int kCols = 16 * NF;
    extern __shared__ __align__(16) uint8_t al_lds[];
    uint8_t *a_l = al_lds;
    uint8_t *s_l = al_lds + al_a_bytes(K);
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * kCols, mb = blockIdx.y * kAlRows;
    const int ksteps = K / 128, kbn = K / 32, kb128 = K / 128;
    const int k0 = w * ksteps / kAlWaves, k1 = (w + 1) * ksteps / kAlWaves;
    const int pitch = K + 16;

    // 1. the A block and its scales into LDS (rows past M repeat row M-1;
    // a piece that would cross the image's end repeats its last 16 bytes).
    // Every workgroup of a row block copies the same bytes at the same time:
    // each starts at its own piece, so that they do not all queue on the
    // same L2 channel.
    {
        const int total = kAlRows * pitch, nq = (total + 1023) / 1024;
        const int rot = (int)((blockIdx.x * 41u) % (unsigned)nq);
        for (int c0 = w; c0 < nq; c0 += kAlWaves) {
            const int c = c0 + rot < nq ? c0 + rot : c0 + rot - nq;
            const int o = min(c * 1024 + lane * 16, total - 16);
            const int row = o / pitch, col = min(o - row * pitch, K - 16);
            __builtin_amdgcn_global_load_lds(
                (const void *)(A + (size_t)min(mb + row, M - 1) * K + col),
                (__attribute__((address_space(3))) void *)(a_l + c * 1024), 16, 0, 0);
        }
        const int stot = kAlRows * kbn, nsq = (stot + 1023) / 1024;
        const int srot = (int)(blockIdx.x % (unsigned)nsq);
        for (int c0 = w; c0 < nsq; c0 += kAlWaves) {
            const int c = c0 + srot < nsq ? c0 + srot : c0 + srot - nsq;
            const int o = min(c * 1024 + lane * 16, stot - 16);
            const int row = o / kbn, col = o - row * kbn;
            __builtin_amdgcn_global_load_lds(
                (const void *)((const uint8_t *)SA + (size_t)min(mb + row, M - 1) * kbn + col),
                (__attribute__((address_space(3))) void *)(s_l + c * 1024), 16, 0, 0);
        }
    }
    // the A copies are older than every weight load below: loads complete in
    // issue order, so waiting for "all but the weight loads" waits for them
    mem_order();

    // 2. the wave's weight rows: 16 B at K offset 32g (+16) (exact) or 16g
    // (+64) (native) of each 128-K step
    const uint8_t *brow[NF];
    const uint8_t *sbrow[NF];
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const int col = n0 + 16 * j + r;
        brow[j] = B + (size_t)col * K + (EXACT ? g * 32 : g * 16);
        sbrow[j] = (const uint8_t *)SB + (size_t)(col / 32) * kbn;
    }
    const float *sbf_row = (const float *)SB + (size_t)(n0 / 128) * kb128;
    auto load = [&](AlStage<NF> &st, int ks0) {
        const int ks = max(min(ks0, k1 - 1), 0);
#pragma unroll
        for (int j = 0; j < NF; j++) {
            const uint8_t *p = brow[j] + (size_t)ks * 128;
            st.b[j][0] = ldg16(p);
            st.b[j][1] = ldg16(p + (EXACT ? 16 : 64));
            if (SMODE == kUe8m0) st.sb[j] = *(const uint32_t *)(sbrow[j] + ks * 4) >> (8 * g);
        }
        if (SMODE == kF32s) st.sbf = sbf_row[ks];
    };
    constexpr int kStageLoads = 2 * NF + (SMODE == kUe8m0 ? NF : 1);

    v4f acc[2][NF];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NF; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    const uint32_t a_base = lds_addr(a_l), s_base = lds_addr(s_l);
    auto compute = [&](const AlStage<NF> &st, int ks) {
        if (ks >= k1) return;  // uniform
        // the wave's two A fragments of this step, and their scales
        u32x4v alo[2], ahi[2];
        uint32_t saw[2];
        float saf[2][4];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int rl = 16 * i + r;
            const uint32_t ap = a_base + rl * pitch + ks * 128 + (EXACT ? g * 32 : g * 16);
            alo[i] = lds_read_b128(ap);
            ahi[i] = lds_read_b128(ap + (EXACT ? 16 : 64));
            if (SMODE == kUe8m0) {
                saw[i] = lds_read_b32(s_base + rl * kbn + ks * 4);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    saf[i][v] = __uint_as_float(
                        lds_read_b32(s_base + ((16 * i + 4 * g + v) * kb128 + ks) * 4));
            }
        }
        lds_wait_all();
#pragma unroll
        for (int i = 0; i < 2; i++) {
            lds_ready(alo[i]);
            lds_ready(ahi[i]);
            if (SMODE == kUe8m0) lds_ready(saw[i]);
            else {
#pragma unroll
                for (int v = 0; v < 4; v++) lds_ready(saf[i][v]);
            }
        }
        if (EXACT) {
            v8bf bq[NF][4];
#pragma unroll
            for (int j = 0; j < NF; j++)
                cvt_fp8x32(st.b[j][0], st.b[j][1],
                           SMODE == kUe8m0 ? e8m0_to_f32(st.sb[j] & 0xFF) : 1.0f, bq[j]);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                v8bf aq[4];
                cvt_fp8x32(uint4{alo[i][0], alo[i][1], alo[i][2], alo[i][3]},
                           uint4{ahi[i][0], ahi[i][1], ahi[i][2], ahi[i][3]},
                           SMODE == kUe8m0 ? e8m0_to_f32((saw[i] >> (8 * g)) & 0xFF) : 1.0f, aq);
#pragma unroll
                for (int j = 0; j < NF; j++) {
                    if (SMODE == kUe8m0) {
                        acc[i][j] = mfma_bf16_k128(aq, bq[j], acc[i][j]);
                    } else {
                        const v4f p = mfma_bf16_k128(aq, bq[j], v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            acc[i][j][v] = acc[i][j][v] + p[v] * (saf[i][v] * st.sbf);
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const v8i a = frag_from(uint4{alo[i][0], alo[i][1], alo[i][2], alo[i][3]},
                                        uint4{ahi[i][0], ahi[i][1], ahi[i][2], ahi[i][3]});
#pragma unroll
                for (int j = 0; j < NF; j++) {
                    const v8i b = frag_from(st.b[j][0], st.b[j][1]);
                    if (SMODE == kUe8m0) {
                        acc[i][j] = mfma_scaled<kFmtFp8, kFmtFp8>(
                            a, b, acc[i][j], (int)((saw[i] >> (8 * g)) & 0xFF),
                            (int)(st.sb[j] & 0xFF));
                    } else {
                        const v4f p = mfma_scaled<kFmtFp8, kFmtFp8>(
                            a, b, v4f{0.f, 0.f, 0.f, 0.f}, kScaleOne, kScaleOne);
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            acc[i][j][v] = acc[i][j][v] + p[v] * (saf[i][v] * st.sbf);
                    }
                }
            }
        }
    };

    AlStage<NF> s0, s1;
    load(s0, k0);
    mem_order();
    load(s1, k0 + 1);
    mem_order();
    wait_vm<2 * kStageLoads>();  // this wave's A / scale copies have landed
    raw_barrier();               // ... and every wave's

    const int nst = k1 - k0;
    int i = 0, ks = k0;
    for (; i + 3 < nst; i += 2, ks += 2) {
        compute(s0, ks);
        load(s0, ks + 2);
        compute(s1, ks + 1);
        load(s1, ks + 3);
    }
    const int rest = nst - i;
    if (rest == 3) {
        compute(s0, ks);
        load(s0, ks + 2);
        compute(s1, ks + 1);
        compute(s0, ks + 2);
    } else {
        if (rest >= 1) compute(s0, ks);
        if (rest == 2) compute(s1, ks + 1);
    }

    // the K parts meet in LDS (the A image is no longer read), in wave order
    __syncthreads();
    float *part = (float *)al_lds;  // [8][32][kCols]
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int j = 0; j < NF; j++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                part[(w * kAlRows + 16 * f + 4 * g + v) * kCols + 16 * j + r] = acc[f][j][v];
    __syncthreads();
    for (int o = t; o < kAlRows * kCols; o += 64 * kAlWaves) {
        const int rl = o / kCols, c = o % kCols;
        const int row = mb + rl;
        if (row >= M) continue;
        float sum = part[rl * kCols + c];
#pragma unroll
        for (int q = 1; q < kAlWaves; q++) sum = sum + part[(q * kAlRows + rl) * kCols + c];
        if (OMODE == kOutF32) ((float *)C)[(size_t)row * N + n0 + c] = sum;
        else ((uint16_t *)C)[(size_t)row * N + n0 + c] = f32_to_bf16(sum);
    }
}

template <int NF, int SMODE, int OMODE>
static int launch_al(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                     int m, int n, int k, hipStream_t stream) {
    if (n % (16 * NF) || k % 512 || k > 4096) return -1;
    const size_t lds = al_a_bytes(k) + al_s_bytes(k);
    if ((size_t)kAlWaves * kAlRows * 16 * NF * 4 > lds) return -1;  // the partials reuse it
    dim3 grid((unsigned)(n / (16 * NF)), (unsigned)((m + kAlRows - 1) / kAlRows));
    const bool exact = math_mode() != WS_MATH_NATIVE;
    if (exact)
        hipLaunchKernelGGL((gemm_al_kernel<NF, SMODE, OMODE, true>), grid, dim3(64 * kAlWaves), lds,
                           stream, a, sa, b, sb, out, m, n, k);
    else
        hipLaunchKernelGGL((gemm_al_kernel<NF, SMODE, OMODE, false>), grid, dim3(64 * kAlWaves), lds,
                           stream, a, sa, b, sb, out, m, n, k);
    return launch_status();
}

// ---- pipelined split-K GEMM (A and W streamed through an LDS ring) -------
// A workgroup (4 waves, 2 x 2 over the tile) owns a 128 x BN output tile and
// a range of at most kPMaxSteps 128-K steps. Every step's A block (128 x 128
// e4m3) and weight block (BN x 128 e4m3, or BN x 64 packed e2m1) are copied
// into one of NS LDS stages by direct global->LDS loads, NS-1 steps ahead of
// the math, so the weight stream does not wait for the multiply. The scales of
// the whole K range are copied once, before the first stage. Each wave
// converts its 64 x BN/2 share of a step to bf16 and runs bf16 MFMAs (exact
// mode) or feeds the bytes to the scaled MFMA (native mode).
// LDS rows are 128 B (64 B for e2m1) with their 16-B chunks permuted by the
// row index, so the 16 rows read by one instruction hit distinct banks.
constexpr int kPM = 128, kPMaxSteps = 16;

// BN = 64 or 128: 4 waves (2 x 2, wave tile 64 x BN/2); BN = 256: 8 waves
// (2 x 4, wave tile 64 x 64), two per SIMD, so one wave's conversions overlap
// another's MFMAs.
template <int BN, bool BFP4, int SMODE>
struct PipeGeom {
    static constexpr int kWaves = BN == 256 ? 8 : 4;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kWN = kWaves / 2;                 // waves along N
    static constexpr int kA = kPM * 128;               // A bytes per step
    static constexpr int kW = BN * (BFP4 ? 64 : 128);  // weight bytes per step
    static constexpr int kStage = kA + kW;
    static constexpr int kAL = kA / 1024 / kWaves;     // 16-B direct loads per wave and step
    static constexpr int kWL = kW / 1024 / kWaves;
    static constexpr int kLoads = kAL + kWL;
    static constexpr int kNJ = BN / kWN / 16;          // 16-column fragments per wave
    // scale words per step: one per A row, then one per weight scale row
    static constexpr int kSW = SMODE == kF32s ? (BN + 127) / 128 : (BFP4 ? BN : BN / 32);
    static constexpr int kScaleBytes = ((kPM + kSW) * kPMaxSteps + 63) / 64 * 256;
    static constexpr int kNSFit = (160 * 1024 - kScaleBytes) / kStage;
    static constexpr int NS = kNSFit > 6 ? 6 : kNSFit;  // LDS stages
    static constexpr int kLds = NS * kStage + kScaleBytes;
};

// chunk permutation: 128-B rows (8 chunks) and 64-B rows (4 chunks)
__device__ __forceinline__ int sw8(int row, int c) { return c ^ ((row >> 1) & 7); }
__device__ __forceinline__ int sw4(int row, int c) { return c ^ ((row >> 2) & 3); }

template <int BN, bool BFP4, int SMODE, int OMODE, bool EXACT>
__global__ __launch_bounds__(BN == 256 ? 512 : 256) void gemm_pipe_kernel(
    const uint8_t *A, const void *SA, const uint8_t *B, const void *SB, void *__restrict__ C,
    int M, int N, int K, int S, int ntn, float *__restrict__ part) {
    using G = PipeGeom<BN, BFP4, SMODE>;
    constexpr int NS = G::NS;
    extern __shared__ __align__(16) uint8_t p_lds[];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int tile = blockIdx.x / S, s = blockIdx.x % S;
    const int mb = tile / ntn, nt = tile % ntn;
    const int m0 = mb * kPM, n0 = nt * BN;
    const int ksteps = K / 128, kbn = K / 32, kb128 = K / 128;
    const int ka = s * ksteps / S, kz = (s + 1) * ksteps / S, n = kz - ka;  // n <= kPMaxSteps
    const int wm = w & 1, wn = w >> 1;
    uint8_t *const sc_lds = p_lds + NS * G::kStage;

    // ---- 1. scales of steps [ka, kz): word (row * n + j) for A row `row`,
    // word ((kPM + q) * n + j) for weight scale row q (a 32-column block of
    // FP8 weights, one FP4 weight row, or a 128-column f32 block). A lane
    // copies one word; consecutive lanes walk a row's steps, so an
    // instruction touches few cache lines.
    {
        const int words = (kPM + G::kSW) * n;
        const int ninstr = (words + 63) / 64;
        for (int c = w; c < ninstr; c += G::kWaves) {
            const int o = min(c * 64 + lane, words - 1);
            const int q = o / n, j = o - q * n;
            const uint8_t *src;
            if (q < kPM) {
                const int row = min(m0 + q, M - 1);
                src = SMODE == kF32s ? (const uint8_t *)((const float *)SA + (size_t)row * kb128 + ka + j)
                                     : (const uint8_t *)SA + (size_t)row * kbn + (ka + j) * 4;
            } else if (SMODE == kF32s) {
                const int wrow = min(n0 / 128 + q - kPM, (N + 127) / 128 - 1);
                src = (const uint8_t *)((const float *)SB + (size_t)wrow * kb128 + ka + j);
            } else {
                const int wq = q - kPM;
                const int wrow = BFP4 ? min(n0 + wq, N - 1) : min(n0 / 32 + wq, (N + 31) / 32 - 1);
                src = (const uint8_t *)SB + (size_t)wrow * kbn + (ka + j) * 4;
            }
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (__attribute__((address_space(3))) void *)(sc_lds + c * 256),
                                             4, 0, 0);
        }
    }

    // ---- 2. direct loads of one step into stage buffer `buf`; a lane's
    // source rows are fixed, only the K offset moves
    const uint8_t *asrc[G::kAL];
#pragma unroll
    for (int j = 0; j < G::kAL; j++) {
        const int o = (w * G::kAL + j) * 1024 + lane * 16;
        const int row = o >> 7, c = (o >> 4) & 7;
        asrc[j] = A + (size_t)min(m0 + row, M - 1) * K + sw8(row, c) * 16;
    }
    const uint8_t *wsrc[G::kWL];
#pragma unroll
    for (int j = 0; j < G::kWL; j++) {
        const int o = (w * G::kWL + j) * 1024 + lane * 16;
        if (BFP4) {
            const int row = o >> 6, c = (o >> 4) & 3;
            wsrc[j] = B + (size_t)min(n0 + row, N - 1) * (K / 2) + sw4(row, c) * 16;
        } else {
            const int row = o >> 7, c = (o >> 4) & 7;
            wsrc[j] = B + (size_t)min(n0 + row, N - 1) * K + sw8(row, c) * 16;
        }
    }
    auto issue = [&](int buf, int ks) {
        uint8_t *base = p_lds + buf * G::kStage;
#pragma unroll
        for (int j = 0; j < G::kAL; j++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(asrc[j] + (size_t)ks * 128),
                (__attribute__((address_space(3))) void *)(base + (w * G::kAL + j) * 1024), 16, 0, 0);
#pragma unroll
        for (int j = 0; j < G::kWL; j++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(wsrc[j] + (size_t)ks * (BFP4 ? 64 : 128)),
                (__attribute__((address_space(3))) void *)(base + G::kA + (w * G::kWL + j) * 1024),
                16, 0, 0);
    };

    // ---- 3. registers of one step (LDS reads as asm: see lds_read_b128)
    struct Raw {
        u32x4v a[4][2];
        u32x4v b[G::kNJ][BFP4 ? 1 : 2];
        uint32_t sa[4][SMODE == kF32s ? 4 : 1], sb[G::kNJ];
    };
    auto fetch = [&](int buf, int i, Raw &x) {
        const uint32_t base = lds_addr(p_lds) + buf * G::kStage;
        const uint32_t wl = base + G::kA;
        const uint32_t sl = lds_addr(sc_lds);
        const int c0 = EXACT ? 2 * g : g, c1 = EXACT ? 2 * g + 1 : 4 + g;
#pragma unroll
        for (int f = 0; f < 4; f++) {
            const int row = 64 * wm + 16 * f + r;
            x.a[f][0] = lds_read_b128(base + row * 128 + sw8(row, c0) * 16);
            x.a[f][1] = lds_read_b128(base + row * 128 + sw8(row, c1) * 16);
            if (SMODE == kUe8m0) {
                x.sa[f][0] = lds_read_b32(sl + (row * n + i) * 4);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    x.sa[f][v] = lds_read_b32(sl + ((64 * wm + 16 * f + 4 * g + v) * n + i) * 4);
            }
        }
#pragma unroll
        for (int j = 0; j < G::kNJ; j++) {
            const int col = (BN / G::kWN) * wn + 16 * j + r;
            if (BFP4) {
                x.b[j][0] = lds_read_b128(wl + col * 64 + sw4(col, g) * 16);
            } else {
                x.b[j][0] = lds_read_b128(wl + col * 128 + sw8(col, c0) * 16);
                x.b[j][BFP4 ? 0 : 1] = lds_read_b128(wl + col * 128 + sw8(col, c1) * 16);
            }
            const int q = SMODE == kF32s ? col / 128 : (BFP4 ? col : col / 32);
            x.sb[j] = lds_read_b32(sl + ((kPM + q) * n + i) * 4);
        }
    };
    auto settle = [&](Raw &x) {
        lds_wait_all();
#pragma unroll
        for (int f = 0; f < 4; f++) {
            lds_ready(x.a[f][0]);
            lds_ready(x.a[f][1]);
#pragma unroll
            for (int v = 0; v < (SMODE == kF32s ? 4 : 1); v++) lds_ready(x.sa[f][v]);
        }
#pragma unroll
        for (int j = 0; j < G::kNJ; j++) {
            lds_ready(x.b[j][0]);
            if (!BFP4) lds_ready(x.b[j][BFP4 ? 0 : 1]);
            lds_ready(x.sb[j]);
        }
    };
    auto u4 = [](const u32x4v &v) { return uint4{v[0], v[1], v[2], v[3]}; };

    v4f acc[4][G::kNJ];
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int j = 0; j < G::kNJ; j++) acc[f][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // f32 scales: acc += P * (sa[row] * sb) once per step
    auto scale_add = [&](v4f &a, const v4f &p, const Raw &x, int f, int j) {
        const float sbf = __uint_as_float(x.sb[j]);
#pragma unroll
        for (int v = 0; v < 4; v++) a[v] = a[v] + p[v] * (__uint_as_float(x.sa[f][v]) * sbf);
    };
    auto math = [&](const Raw &x) {
        if (EXACT) {
            v8bf aq[4][4];
#pragma unroll
            for (int f = 0; f < 4; f++)
                cvt_fp8x32(u4(x.a[f][0]), u4(x.a[f][1]),
                           SMODE == kUe8m0 ? e8m0_to_f32((x.sa[f][0] >> (8 * g)) & 0xFF) : 1.0f, aq[f]);
#pragma unroll
            for (int j = 0; j < G::kNJ; j++) {
                v8bf bq[4];
                const float sb = SMODE == kUe8m0 ? e8m0_to_f32((x.sb[j] >> (8 * g)) & 0xFF) : 1.0f;
                if (BFP4) cvt_fp4x32(u4(x.b[j][0]), sb, bq);
                else cvt_fp8x32(u4(x.b[j][0]), u4(x.b[j][BFP4 ? 0 : 1]), sb, bq);
#pragma unroll
                for (int f = 0; f < 4; f++) {
                    if (SMODE == kUe8m0) acc[f][j] = mfma_bf16_k128(aq[f], bq, acc[f][j]);
                    else scale_add(acc[f][j], mfma_bf16_k128(aq[f], bq, v4f{0.f, 0.f, 0.f, 0.f}), x, f, j);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < G::kNJ; j++) {
                const v8i bf = BFP4 ? frag_from4(u4(x.b[j][0]))
                                    : frag_from(u4(x.b[j][0]), u4(x.b[j][BFP4 ? 0 : 1]));
#pragma unroll
                for (int f = 0; f < 4; f++) {
                    const v8i af = frag_from(u4(x.a[f][0]), u4(x.a[f][1]));
                    if (SMODE == kUe8m0) {
                        const int sa = (x.sa[f][0] >> (8 * g)) & 0xFF, sb = (x.sb[j] >> (8 * g)) & 0xFF;
                        acc[f][j] = BFP4 ? mfma_scaled<kFmtFp8, kFmtFp4>(af, bf, acc[f][j], sa, sb)
                                         : mfma_scaled<kFmtFp8, kFmtFp8>(af, bf, acc[f][j], sa, sb);
                    } else {
                        scale_add(acc[f][j],
                                  mfma_scaled<kFmtFp8, kFmtFp8>(af, bf, v4f{0.f, 0.f, 0.f, 0.f},
                                                                kScaleOne, kScaleOne),
                                  x, f, j);
                    }
                }
            }
        }
    };

    // ---- 4. pipeline: NS-1 steps ahead, one refill per step
#pragma unroll
    for (int p = 0; p < NS - 1; p++)
        if (p < n) issue(p, ka + p);
    for (int i = 0; i < n; i++) {
        // this wave's copies of step i (and the older scale copies) have
        // landed once at most min(n-1-i, NS-2) newer steps are in flight
        mem_order();
        wait_newer<G::kLoads, NS - 2>(min(n - 1 - i, NS - 2));
        raw_barrier();  // every wave's copies of step i are in LDS; step i-1's buffer is free
        Raw x;
        fetch(i % NS, i, x);
        if (i + NS - 1 < n) issue((i + NS - 1) % NS, ka + i + NS - 1);
        settle(x);
        math(x);
    }

    // ---- 5. store: C directly (one split), or the split's partial in
    // fragment order (one 1-KB float4 row per fragment: coalesced)
    if (S > 1) {
        float4 *pp = (float4 *)part + (((size_t)s * gridDim.x / S + tile) * G::kWaves + w) * (4 * G::kNJ * 64);
#pragma unroll
        for (int f = 0; f < 4; f++)
#pragma unroll
            for (int j = 0; j < G::kNJ; j++)
                pp[(f * G::kNJ + j) * 64 + lane] = float4{acc[f][j][0], acc[f][j][1], acc[f][j][2], acc[f][j][3]};
        return;
    }
#pragma unroll
    for (int f = 0; f < 4; f++)
#pragma unroll
        for (int j = 0; j < G::kNJ; j++) {
            const int col = n0 + (BN / G::kWN) * wn + 16 * j + r;
            if (col >= N) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int row = m0 + 64 * wm + 16 * f + 4 * g + v;
                if (row < M) {
                    if (OMODE == kOutF32) ((float *)C)[(size_t)row * N + col] = acc[f][j][v];
                    else ((uint16_t *)C)[(size_t)row * N + col] = f32_to_bf16(acc[f][j][v]);
                }
            }
        }
}

// Sum of the S partials of every output in split order (deterministic);
// the kernel boundary after gemm_pipe_kernel makes them visible. Partials are
// in the GEMM's fragment order: [split][tile][wave][f][j][lane] float4, the
// float4 holding rows 4g..4g+3 (g = lane / 16) of column lane % 16.
template <int BN, int OMODE>
__global__ __launch_bounds__(256) void pipe_reduce_kernel(const float4 *__restrict__ part,
                                                          void *__restrict__ C, int M, int N, int S,
                                                          int tiles, int ntn) {
    constexpr int NW = BN == 256 ? 8 : 4, WN = NW / 2, NJ = BN / WN / 16;
    const size_t q = (size_t)blockIdx.x * 256 + threadIdx.x;  // float4 index within a split
    const size_t plane = (size_t)tiles * NW * 4 * NJ * 64;
    if (q >= plane) return;
    // loads in groups of four, all issued before the adds (planes past S-1
    // repeat the last one and are not added); the sum runs in split order
    float4 acc = float4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = part[(size_t)min(s0 + u, S - 1) * plane + q];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (s0 + u >= S) break;
            if (s0 + u == 0) {
                acc = v[u];
            } else {
                acc.x = acc.x + v[u].x;
                acc.y = acc.y + v[u].y;
                acc.z = acc.z + v[u].z;
                acc.w = acc.w + v[u].w;
            }
        }
    }
    const int lane = (int)(q & 63);
    size_t rest = q >> 6;
    const int j = (int)(rest % NJ);
    rest /= NJ;
    const int f = (int)(rest & 3);
    rest >>= 2;
    const int w = (int)(rest % NW);
    const int tile = (int)(rest / NW);
    const int mb = tile / ntn, nt = tile % ntn;
    const int col = nt * BN + (BN / WN) * (w >> 1) + 16 * j + (lane & 15);
    if (col >= N) return;
    const int row0 = mb * 128 + 64 * (w & 1) + 16 * f + 4 * (lane >> 4);
    const float v[4] = {acc.x, acc.y, acc.z, acc.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int row = row0 + e;
        if (row >= M) break;
        if (OMODE == kOutF32) ((float *)C)[(size_t)row * N + col] = v[e];
        else ((uint16_t *)C)[(size_t)row * N + col] = f32_to_bf16(v[e]);
    }
}

// Workspaces for the split-K kernels, one per (device, stream)
// (ws_set_gemm_workspace): GEMMs on different streams never share partials.
struct SkWorkspace {
    uint8_t *ptr;
    size_t bytes;
};
struct SkEntry {
    int dev;
    hipStream_t stream;
    SkWorkspace ws;
};
constexpr int kMaxSkEntries = 256;
static std::mutex g_sk_mu;
static SkEntry g_sk[kMaxSkEntries];
static int g_sk_n = 0;

static int current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    return dev;
}

// the workspace registered for `stream` on the current device (none: {0, 0})
static SkWorkspace sk_ws(hipStream_t stream) {
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(g_sk_mu);
    for (int i = 0; i < g_sk_n; i++)
        if (g_sk[i].dev == dev && g_sk[i].stream == stream) return g_sk[i].ws;
    return SkWorkspace{nullptr, 0};
}

static int sk_set(hipStream_t stream, uint8_t *ptr, size_t bytes) {
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(g_sk_mu);
    for (int i = 0; i < g_sk_n; i++) {
        if (g_sk[i].dev == dev && g_sk[i].stream == stream) {
            if (ptr) {
                g_sk[i].ws = SkWorkspace{ptr, bytes};
            } else {
                g_sk[i] = g_sk[--g_sk_n];
            }
            return WS_OK;
        }
    }
    if (!ptr) return WS_OK;
    if (g_sk_n == kMaxSkEntries) return WS_ERR_SHAPE;
    g_sk[g_sk_n++] = SkEntry{dev, stream, SkWorkspace{ptr, bytes}};
    return WS_OK;
}

// Splits for the pipelined kernel: K ranges of at most kPMaxSteps steps, and
// as many as keep every CU busy with one workgroup; 0 when the workspace is
// too small.
static int pipe_splits(int M, int N, int K, int BN, size_t ws_bytes) {
    const int ksteps = K / 128;
    const int tiles = ((M + kPM - 1) / kPM) * ((N + BN - 1) / BN);
    int S = cu_count() / tiles;
    const int smin = (ksteps + kPMaxSteps - 1) / kPMaxSteps;
    if (S < smin) S = smin;
    if (S > ksteps) S = ksteps;
    // partials: S planes of tiles x (128 x BN) floats
    if (S > 1 && (size_t)S * tiles * kPM * BN * 4 > ws_bytes) return 0;
    return S;
}

// Tile width of the pipelined kernel for (M, N): 256 columns when that still
// gives every eighth CU a tile, else 64.
static int pipe_bn(int M, int N) {
    const int mt = (M + kPM - 1) / kPM;
    // measured at M=128, K=4096: 256 wins at N=12288, 64 at N=4096 and 2048
    // (fewer partial bytes per split than 128)
    return mt * ((N + 255) / 256) * 8 >= cu_count() ? 256 : 64;
}

template <int BN, bool BFP4, int SMODE, int OMODE>
static int launch_pipe(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                       int m, int n, int k, hipStream_t stream, const SkWorkspace &wsp) {
    using G = PipeGeom<BN, BFP4, SMODE>;
    const int S = pipe_splits(m, n, k, BN, wsp.ptr ? wsp.bytes : 0);
    if (S <= 0) return -1;
    const int ntn = (n + BN - 1) / BN;
    const int tiles = ((m + kPM - 1) / kPM) * ntn;
    float *part = (float *)wsp.ptr;
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_pipe_kernel<BN, BFP4, SMODE, OMODE, false>), dim3(tiles * S),
                           dim3(G::kThreads), G::kLds, stream, a, sa, b, sb, out, m, n, k, S, ntn, part);
    else
        hipLaunchKernelGGL((gemm_pipe_kernel<BN, BFP4, SMODE, OMODE, true>), dim3(tiles * S),
                           dim3(G::kThreads), G::kLds, stream, a, sa, b, sb, out, m, n, k, S, ntn, part);
    int rc = launch_status();
    if (rc || S == 1) return rc;
    const size_t quads = (size_t)tiles * G::kWaves * 4 * G::kNJ * 64;
    hipLaunchKernelGGL((pipe_reduce_kernel<BN, OMODE>), dim3((unsigned)((quads + 255) / 256)),
                       dim3(256), 0, stream, (const float4 *)part, out, m, n, S, tiles, ntn);
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

template <bool BFP4, int SMODE, int OMODE>
// OMODE kOutAcc (C += A.B^T) and kOutAcc2 (C = C + (aux + A.B^T)) run on the
// kernels with those epilogues (line, column strips), never split over K.
static int gemm_dispatch(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb,
                         void *out, int64_t m, int64_t n, int64_t k, hipStream_t stream,
                         int sb_div = 32, const float *aux = nullptr) {
    constexpr bool kAccOut = OMODE == kOutAcc || OMODE == kOutAcc2;
    if (OMODE == kOutAcc2 && !aux) return WS_ERR_INVALID_ARG;
    if (!a || !sa || !b || !sb || !out) return WS_ERR_INVALID_ARG;
    if (m <= 0 || n <= 0 || k <= 0) return WS_ERR_INVALID_ARG;
    if (k % 128 || n % 16 || m > (1 << 24) || n > (1 << 24) || k > (1 << 24)) return WS_ERR_SHAPE;
    if (((uintptr_t)a | (uintptr_t)b) & 15 || ((uintptr_t)sa | (uintptr_t)sb) & 3)
        return WS_ERR_INVALID_ARG;
    int M = (int)m, N = (int)n, K = (int)k;
    const SkWorkspace wsp = sk_ws(stream);
    if (sb_div != 32) {
        // weight scales per row (the reference's packed scale table): the
        // column-strip kernel only
        int rc;
        if (M <= 16) {
            const int S = kAccOut ? 1 : strip_splits(M, N, K, wsp.ptr ? wsp.bytes : 0);
            rc = launch_kp<1, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, S,
                                                               (float *)wsp.ptr, sb_div, aux);
        } else if (M <= 32) {
            rc = launch_kp<2, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1,
                                                               nullptr, sb_div, aux);
        } else if (M <= 64) {
            rc = launch_kp<4, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1,
                                                               nullptr, sb_div, aux);
        } else {
            rc = launch_kp<4, 1, 2, 4, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1,
                                                               nullptr, sb_div, aux);
        }
        return rc < 0 ? WS_ERR_SHAPE : rc;
    }
    int cfg = -1;
    {
        int rc = -1;
        // 1. 32-column strips when they give the chip one round of workgroups:
        // 64-row blocks (M=128, N=4096) or 32-row blocks (M=128, N=2048;
        // M=64, N=4096). Measured at K=4096: 16.4 us (kp) and 10.0 us (A in
        // LDS; kp 11.3) against 19.7 and 15.7 for the split-K kernel.
        // (measured at M=128: for K = 5120, or N = 5120 with K = 2048-2304,
        // the split-K pipeline is faster: 17.8 against 27.8 us at N=2304,
        // K=5120; 16.5 against 22.0 at N=5120, K=2304)
        if (M > 16 && N % 32 == 0 && K <= 4096 && N <= 4096) {
            const long cus = cu_count();
            const long wg64 = (long)(N / 32) * ((M + 63) / 64), wg32 = (long)(N / 32) * ((M + 31) / 32);
            if (wg64 * 4 >= cus * 3 && wg64 * 2 <= cus * 3) {
                // 64 x 32 tiles: the line kernel (whole-line LDS stages of
                // 512 K, XCD-paired row blocks) when K allows its stages;
                // measured at M=128, N=4096, K=4096: 13.8 against 16.6 us
                if (!BFP4 && K % 512 == 0 && M > 64)
                    rc = line_gemm(SMODE, OMODE, a, sa, b, sb, out, M, N, K, stream, 0, aux);
                if (rc < 0)
                    rc = launch_kp<4, 2, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream,
                                                                       1, nullptr, 32, aux);
            } else if (wg32 * 4 >= cus * 3 && wg32 * 2 <= cus * 3) {
                // 32-row blocks: the line kernel with 32 x 32 tiles (M=128,
                // N=2048, K=4096: 9.95 against 10.9 us for the A-resident
                // kernel), else the A-resident kernel (K <= 4096), else kp
                if (!BFP4 && K % 512 == 0)
                    rc = line_gemm(SMODE, OMODE, a, sa, b, sb, out, M, N, K, stream, 2, aux);
                if (!BFP4 && !kAccOut && rc < 0)
                    rc = launch_al<2, SMODE, OMODE>(a, sa, b, sb, out, M, N, K, stream);
                if (rc < 0)
                    rc = launch_kp<2, 2, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream,
                                                                       1, nullptr, 32, aux);
            }
        }
        if (rc >= 0) return rc;
        // 2. whole 128-row blocks, 48-column tiles filling the chip once: the
        // line kernel (M=128, N=12288, K=4096: 29.2 against 31.5 us for the
        // split-K pipeline and its reduction, graph replays)
        if (!BFP4 && M > 64 && M <= 128 && N % 48 == 0 && K % 256 == 0) {
            const long wg = N / 48, cus = cu_count();
            if (wg * 4 >= cus * 3 && wg * 2 <= cus * 3)
                rc = line_gemm(SMODE, OMODE, a, sa, b, sb, out, M, N, K, stream, 4, aux);
        }
        if (rc >= 0) return rc;
        // 3. the line kernel at the other shapes it stages (K a multiple of
        // 512; K > 4096, N > 4096 or few tiles): 32 x 32 tiles when they fit
        // one round of workgroups, else 64 x 32. Cold weights, against the
        // kernels below with a split-K workspace registered: M=64 all engine
        // projection shapes faster (N=25600, K=5120 86.6 -> 57.8 us; N=5120,
        // K=2048 15.6 -> 8.5; N=4096, K=8192 19.8 -> 14.9); M=128 faster with
        // one round of tiles or K <= 4096 (N=512, K=5120 17.3 -> 9.7; N=8192,
        // K=2048 23.0 -> 15.6), slower otherwise (N=4608, K=5120 23.0 ->
        // 28.4; N=1280, K=15360 21.7 -> 23.6), so those keep the split-K
        // pipeline. At 32 rows only the 32 x 32 tiles, with 64 or more.
        if (!BFP4 && M > 16 && M <= 128 && N % 32 == 0 && K % 512 == 0) {
            const long cus = cu_count();
            const long w2 = (long)((M + 31) / 32) * (N / 32);  // 32 x 32 tiles
            const long w0 = (long)((M + 63) / 64) * (N / 32);  // 64 x 32 tiles
            int lc = -1;
            if (M <= 32) lc = w2 >= 64 ? 2 : -1;
            else lc = w2 <= cus ? 2 : 0;
            if (M > 64 && lc >= 0 && (K > 8192 || ((lc == 2 ? w2 : w0) > cus && K > 4096)))
                lc = -1;
            if (lc >= 0) rc = line_gemm(SMODE, OMODE, a, sa, b, sb, out, M, N, K, stream, lc, aux);
        }
        if (rc >= 0) return rc;
        // 4. M > 64: the pipelined split-K kernel (128-row tiles)
        if (M > 64 && !kAccOut) {
            const int bn = pipe_bn(M, N);
            rc = bn == 256   ? launch_pipe<256, BFP4, SMODE, OMODE>(a, sa, b, sb, out, M, N, K, stream, wsp)
                 : bn == 128 ? launch_pipe<128, BFP4, SMODE, OMODE>(a, sa, b, sb, out, M, N, K, stream, wsp)
                             : launch_pipe<64, BFP4, SMODE, OMODE>(a, sa, b, sb, out, M, N, K, stream, wsp);
        }
        if (rc >= 0) return rc;
        // 5. 16-column strips (no split-K workspace, or shapes the others
        // do not stage)
        if (M <= 16) {
            const int S = kAccOut ? 1 : strip_splits(M, N, K, wsp.ptr ? wsp.bytes : 0);
            rc = launch_kp<1, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, S,
                                                               (float *)wsp.ptr, 32, aux);
        }
        else if (M <= 32) rc = launch_kp<2, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1, nullptr, 32, aux);
        else if (M <= 64) rc = launch_kp<4, 1, 1, 8, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1, nullptr, 32, aux);
        else rc = launch_kp<4, 1, 2, 4, BFP4, SMODE, OMODE, 1>(a, sa, b, sb, out, M, N, K, stream, 1, nullptr, 32, aux);
        if (rc >= 0) return rc;
        if (kAccOut) return WS_ERR_SHAPE;
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

// C = C + (aux + A.B^T), UE8M0 32 x 32 weight scales (the engine's
// acc_f32 pair after a GEMM, in the GEMM's epilogue: the same bits)
int fp8_gemm_acc2(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                  float *c, const float *aux, int64_t m, int64_t n, int64_t k, hipStream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutAcc2>(a, sa, b, sb, c, m, n, k, stream, 32, aux);
}

}  // namespace ws

using namespace ws;

extern "C" {

size_t ws_gemm_workspace_size(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || k % 128 || m > (1 << 24) || n > (1 << 24) || k > (1 << 24))
        return 0;
    size_t best = 0;
    for (int bn : {64, 128, 256}) {
        const int S = pipe_splits((int)m, (int)n, (int)k, bn, (size_t)-1);
        const size_t tiles = (size_t)((m + kPM - 1) / kPM) * ((n + bn - 1) / bn);
        const size_t need = S > 1 ? (size_t)S * tiles * kPM * bn * 4 : 0;
        if (need > best) best = need;
    }
    if (m <= 16) {  // the split 16-column strips
        const size_t need = (size_t)strip_splits((int)m, (int)n, (int)k, (size_t)-1) * m * n * 4;
        if (need > best) best = need;
    }
    return best;
}

int ws_set_gemm_workspace(void *workspace, size_t bytes, ws_stream_t stream) {
    if (!workspace || bytes == 0) {
        sk_set(stream, nullptr, 0);
        return workspace ? WS_ERR_INVALID_ARG : WS_OK;
    }
    if ((uintptr_t)workspace & 255) return WS_ERR_INVALID_ARG;
    return sk_set(stream, (uint8_t *)workspace, bytes);
}

int ws_fp8_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream);
}

int ws_fp8_gemm_acc(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                    float *c, int64_t m, int64_t n, int64_t k, ws_stream_t stream) {
    return gemm_dispatch<false, kUe8m0, kOutAcc>(a, sa, b, sb, c, m, n, k, stream);
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

// launch.rs:325-339 TlGemm: (N, K) of each hard-coded TileLang GEMM
// (engine.rs:3387-3398; WoA from its kernel's strides)
static const int kTlShapes[][2] = {{1280, 5120}, {8192, 1280}, {512, 5120},  {2048, 4096},
                                   {5120, 2048}, {2304, 5120}, {4608, 5120}, {5120, 2304},
                                   {25600, 5120}, {1280, 15360}};

int ws_tl_gemm_shape(int kind, int64_t *n, int64_t *k) {
    if (kind < 0 || kind >= (int)(sizeof(kTlShapes) / sizeof(kTlShapes[0])) || !n || !k)
        return WS_ERR_INVALID_ARG;
    *n = kTlShapes[kind][0];
    *k = kTlShapes[kind][1];
    return WS_OK;
}

int ws_fp8_gemm_tl(int kind, const uint8_t *a, const uint32_t *sa, const uint8_t *b,
                   const uint32_t *sb, float *out, int64_t m, ws_stream_t stream) {
    int64_t n, k;
    int rc = ws_tl_gemm_shape(kind, &n, &k);
    if (rc) return rc;
    // the packed activation words are the UE8M0 bytes [m, k/32] as they lie
    // in memory; the weight table holds each row's K/32 scale bytes
    return gemm_dispatch<false, kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream, 1);
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
