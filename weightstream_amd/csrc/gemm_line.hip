// FP8 block-scaled GEMM for blocks of 32 or 64 rows with K a multiple of 512
// (M = 128, K = 4096, N = 4096 and 2048): the "line"
// kernel.
//
// Reference semantics: weightstream-cuda/kernels/fp8_gemm_tile.cu:28-92 and
// weightstream-ref actquant.rs:110-140 (y = sum over K blocks of the
// dequantised products, f32 accumulation).
//
// Design, from measurements of the load pattern on gfx950 (256 workgroups,
// loads only, wall-clock stamps per workgroup):
//  - both operands stream into LDS by direct global->LDS loads in whole
//    128-byte lines: a stage holds KS = 128 * KQ bytes of every A row and
//    every weight row of the tile (512 or 256 contiguous bytes per row, the
//    16-byte pieces XOR-permuted so fragment reads spread over the banks);
//  - the workgroup owns its tile for the whole K, so no split-K partials are
//    written (8 MB of partials at M = 128, N = 4096 added ~4 us to the kernel
//    end, more than the re-read of A they save);
//  - the row blocks that share a weight column block run on one XCD (the
//    hardware deals workgroups to the 8 XCDs round-robin), so the second
//    read of those weights hits that XCD's L2: the weight stream of a 64 x 32
//    tile set took 3.8 instead of 8.4 us;
//  - the K steps of a stage go to different waves (wave q of a row half
//    takes sub-step q), so every A and weight value is converted once per
//    workgroup; the waves' partial tiles meet in LDS at the end and are added
//    in wave order (deterministic);
//  - scales ride in the same stages (4-byte direct loads), so one wait count
//    covers a stage.
#include "ws_internal.hpp"
#include "ws_kp.hpp"

namespace ws {

template <int MT, int NT, int WMH>
struct LineGeom {
    static constexpr int kWaves = 4;
    static constexpr int KQ = kWaves / WMH;        // 128-K sub-steps per stage
    static constexpr int KS = 128 * KQ;            // bytes of a row per stage
    static constexpr int MF = MT / WMH / 16;       // 16-row fragments per wave
    static constexpr int NJ = NT / 16;             // 16-column fragments
    static constexpr int kA = MT * KS, kW = NT * KS;
    static constexpr int kScA = 1024, kScW = 1024;  // scale words of a stage
    static constexpr int kStage = kA + kW + kScA + kScW;
    static constexpr int AL = kA / 1024 / kWaves;  // 16-byte direct loads per wave and stage
    static constexpr int WL = kW / 1024 / kWaves;
    static constexpr int L = AL + WL + 2;          // + one A-scale and one W-scale load
    static constexpr int kRed = kWaves * MF * NJ * 1024;
    static constexpr int lds_bytes(int D) { return D * kStage > kRed ? D * kStage : kRed; }
    static_assert(kA % (1024 * kWaves) == 0 && kW % (1024 * kWaves) == 0, "whole loads per wave");
    static_assert(MT * KQ <= 256, "A scale words of a stage: one load per wave");
};

// piece c (16 bytes) of row `row` sits at piece c ^ (row & 15) of the LDS row
__device__ __forceinline__ int ln_sw(int row, int c) { return c ^ (row & 15); }

template <int MT, int NT, int WMH, int D, int SMODE, int OMODE, bool EXACT>
__global__ __launch_bounds__(256) void gemm_line_kernel(const uint8_t *A, const void *SA,
                                                        const uint8_t *B, const void *SB,
                                                        void *__restrict__ C, int M, int N, int K,
                                                        int nrb, int xcd_map, const float *aux) {
    using G = LineGeom<MT, NT, WMH>;
    constexpr int KQ = G::KQ, KS = G::KS, MF = G::MF, NJ = G::NJ;
    extern __shared__ __align__(16) uint8_t ln_lds[];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int wm = w / KQ, q = w % KQ;
    // workgroup -> tile: with xcd_map, the row blocks of a column block are
    // consecutive in the per-XCD order (hardware XCD = blockIdx.x % 8)
    int b = blockIdx.x;
    if (xcd_map) b = (b & 7) * (gridDim.x >> 3) + (b >> 3);
    const int rb = b % nrb, cb = b / nrb;
    const int m0 = rb * MT, n0 = cb * NT;
    const int ns = K / KS;                      // stages
    const int kbn = K / 32, kb128 = K / 128;
    const int wsr0 = SMODE == kF32s ? n0 / 128 : n0 / 32;              // first weight scale row
    const int wsrl = SMODE == kF32s ? (N - 1) / 128 : (N - 1) / 32;   // last one

    // ---- direct loads of stage s into slot `slot` (lane sources fixed but
    // for the K offset)
    const uint8_t *asrc[G::AL];
#pragma unroll
    for (int j = 0; j < G::AL; j++) {
        const int o = (w * G::AL + j) * 1024 + lane * 16;
        const int row = o / KS, pc = (o % KS) / 16;
        asrc[j] = A + (size_t)min(m0 + row, M - 1) * K + ln_sw(row, pc) * 16;
    }
    const uint8_t *wsrc[G::WL];
#pragma unroll
    for (int j = 0; j < G::WL; j++) {
        const int o = (w * G::WL + j) * 1024 + lane * 16;
        const int row = o / KS, pc = (o % KS) / 16;
        wsrc[j] = B + (size_t)min(n0 + row, N - 1) * K + ln_sw(row, pc) * 16;
    }
    // scale words: A word e = row * KQ + sub-step, W word e = local scale
    // row * KQ + sub-step; a wave loads words [64 w, 64 w + 64) of each
    const int ea = min(w * 64 + lane, MT * KQ - 1);
    const int arow = min(m0 + ea / KQ, M - 1), aq = ea % KQ;
    const int ew = w * 64 + lane;
    const int wrow = min(wsr0 + (ew / KQ), wsrl), wq = ew % KQ;
    auto issue = [&](int slot, int s) {
        uint8_t *base = ln_lds + slot * G::kStage;
#pragma unroll
        for (int j = 0; j < G::AL; j++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(asrc[j] + (size_t)s * KS),
                (__attribute__((address_space(3))) void *)(base + (w * G::AL + j) * 1024), 16, 0, 0);
#pragma unroll
        for (int j = 0; j < G::WL; j++)
            __builtin_amdgcn_global_load_lds(
                (const void *)(wsrc[j] + (size_t)s * KS),
                (__attribute__((address_space(3))) void *)(base + G::kA + (w * G::WL + j) * 1024),
                16, 0, 0);
        const int step_a = s * KQ + aq, step_w = s * KQ + wq;
        const void *sa_src = SMODE == kF32s
                                 ? (const void *)((const float *)SA + (size_t)arow * kb128 + step_a)
                                 : (const void *)((const uint8_t *)SA + (size_t)arow * kbn + step_a * 4);
        const void *sw_src = SMODE == kF32s
                                 ? (const void *)((const float *)SB + (size_t)wrow * kb128 + step_w)
                                 : (const void *)((const uint8_t *)SB + (size_t)wrow * kbn + step_w * 4);
        __builtin_amdgcn_global_load_lds(
            sa_src, (__attribute__((address_space(3))) void *)(base + G::kA + G::kW + w * 256), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(
            sw_src, (__attribute__((address_space(3))) void *)(base + G::kA + G::kW + G::kScA + w * 256),
            4, 0, 0);
    };

    // ---- registers of a wave's sub-step (LDS reads as asm: lds_read_b128)
    struct Raw {
        u32x4v a[MF][2];
        u32x4v b[NJ][2];
        uint32_t sa[MF][SMODE == kF32s ? 4 : 1], sb[NJ];
    };
    auto fetch = [&](int slot, Raw &x) {
        const uint32_t base = lds_addr(ln_lds) + slot * G::kStage;
        const uint32_t wl = base + G::kA;
        const uint32_t sal = base + G::kA + G::kW, swl = sal + G::kScA;
        const int c0 = 8 * q + (EXACT ? 2 * g : g), c1 = 8 * q + (EXACT ? 2 * g + 1 : 4 + g);
#pragma unroll
        for (int f = 0; f < MF; f++) {
            const int row = wm * (MT / WMH) + 16 * f + r;
            x.a[f][0] = lds_read_b128(base + row * KS + ln_sw(row, c0) * 16);
            x.a[f][1] = lds_read_b128(base + row * KS + ln_sw(row, c1) * 16);
            if (SMODE == kUe8m0) {
                x.sa[f][0] = lds_read_b32(sal + (row * KQ + q) * 4);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    x.sa[f][v] = lds_read_b32(sal + ((wm * (MT / WMH) + 16 * f + 4 * g + v) * KQ + q) * 4);
            }
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int col = 16 * j + r;
            x.b[j][0] = lds_read_b128(wl + col * KS + ln_sw(col, c0) * 16);
            x.b[j][1] = lds_read_b128(wl + col * KS + ln_sw(col, c1) * 16);
            const int sr = (SMODE == kF32s ? (n0 + col) / 128 : (n0 + col) / 32) - wsr0;
            x.sb[j] = lds_read_b32(swl + (sr * KQ + q) * 4);
        }
    };
    auto settle = [&](Raw &x) {
        lds_wait_all();
#pragma unroll
        for (int f = 0; f < MF; f++) {
            lds_ready(x.a[f][0]);
            lds_ready(x.a[f][1]);
#pragma unroll
            for (int v = 0; v < (SMODE == kF32s ? 4 : 1); v++) lds_ready(x.sa[f][v]);
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            lds_ready(x.b[j][0]);
            lds_ready(x.b[j][1]);
            lds_ready(x.sb[j]);
        }
    };
    auto u4 = [](const u32x4v &v) { return uint4{v[0], v[1], v[2], v[3]}; };

    v4f acc[MF][NJ];
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[f][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // f32 scales: acc += P * (sa[row] * sb) once per 128-K step, one fused
    // multiply-add (the GEMM tolerance covers the accumulation order anyway)
    auto scale_add = [&](v4f &a, const v4f &p, const Raw &x, int f, int j) {
        const float sbf = __uint_as_float(x.sb[j]);
#pragma unroll
        for (int v = 0; v < 4; v++) a[v] = __builtin_fmaf(p[v], __uint_as_float(x.sa[f][v]) * sbf, a[v]);
    };
    auto math = [&](const Raw &x) {
        if (EXACT) {
            v8bf aq8[MF][4];
#pragma unroll
            for (int f = 0; f < MF; f++)
                cvt_fp8x32(u4(x.a[f][0]), u4(x.a[f][1]),
                           SMODE == kUe8m0 ? e8m0_to_f32((x.sa[f][0] >> (8 * g)) & 0xFF) : 1.0f, aq8[f]);
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                v8bf bq[4];
                const float sb = SMODE == kUe8m0 ? e8m0_to_f32((x.sb[j] >> (8 * g)) & 0xFF) : 1.0f;
                cvt_fp8x32(u4(x.b[j][0]), u4(x.b[j][1]), sb, bq);
#pragma unroll
                for (int f = 0; f < MF; f++) {
                    if (SMODE == kUe8m0) acc[f][j] = mfma_bf16_k128(aq8[f], bq, acc[f][j]);
                    else scale_add(acc[f][j], mfma_bf16_k128(aq8[f], bq, v4f{0.f, 0.f, 0.f, 0.f}), x, f, j);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const v8i bf = frag_from(u4(x.b[j][0]), u4(x.b[j][1]));
#pragma unroll
                for (int f = 0; f < MF; f++) {
                    const v8i af = frag_from(u4(x.a[f][0]), u4(x.a[f][1]));
                    if (SMODE == kUe8m0) {
                        const int sa = (x.sa[f][0] >> (8 * g)) & 0xFF, sb = (x.sb[j] >> (8 * g)) & 0xFF;
                        acc[f][j] = mfma_scaled<kFmtFp8, kFmtFp8>(af, bf, acc[f][j], sa, sb);
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

    // ---- pipeline: D-1 stages ahead, one refill per stage
#pragma unroll
    for (int p = 0; p < D - 1; p++)
        if (p < ns) issue(p, p);
    for (int i = 0; i < ns; i++) {
        // this wave's loads of stage i have landed once at most
        // min(ns-1-i, D-2) newer stages are in flight
        mem_order();
        wait_newer<G::L, D - 2>(min(ns - 1 - i, D - 2));
        raw_barrier();  // every wave's loads of stage i are in LDS; stage i-1's slot is free
        Raw x;
        fetch(i % D, x);
        if (i + D - 1 < ns) issue((i + D - 1) % D, i + D - 1);
        settle(x);
        math(x);
    }


    // ---- the KQ partial tiles of each row half meet in LDS, added in
    // sub-step order
    __syncthreads();
    float4 *red = (float4 *)ln_lds;
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
            red[((w * MF + f) * NJ + j) * 64 + lane] =
                float4{acc[f][j][0], acc[f][j][1], acc[f][j][2], acc[f][j][3]};
    __syncthreads();
    constexpr int items = WMH * MF * NJ * 64;
    for (int it = t; it < items; it += 256) {
        const int ln = it & 63;
        int rest = it >> 6;
        const int j = rest % NJ;
        rest /= NJ;
        const int f = rest % MF;
        const int h = rest / MF;
        float4 s = red[(((h * KQ) * MF + f) * NJ + j) * 64 + ln];
#pragma unroll
        for (int qq = 1; qq < KQ; qq++) {
            const float4 v = red[(((h * KQ + qq) * MF + f) * NJ + j) * 64 + ln];
            s.x = s.x + v.x;
            s.y = s.y + v.y;
            s.z = s.z + v.z;
            s.w = s.w + v.w;
        }
        const int col = n0 + 16 * j + (ln & 15);
        const int row0 = m0 + h * (MT / WMH) + 16 * f + 4 * (ln >> 4);
        const float o4[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const int row = row0 + v;
            if (row >= M) break;
            const size_t at = (size_t)row * N + col;
            if (OMODE == kOutF32) ((float *)C)[at] = o4[v];
            else if (OMODE == kOutBf16) ((uint16_t *)C)[at] = f32_to_bf16(o4[v]);
            else if (OMODE == kOutAcc) ((float *)C)[at] = ((float *)C)[at] + o4[v];
            else ((float *)C)[at] = ((float *)C)[at] + (aux[at] + o4[v]);
        }
    }
}

template <int MT, int NT, int WMH, int D, int SMODE, int OMODE>
static int launch_line_cfg(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb,
                           void *out, int m, int n, int k, hipStream_t stream, const float *aux) {
    using G = LineGeom<MT, NT, WMH>;
    static_assert(G::lds_bytes(D) <= 160 * 1024, "stages must fit the LDS");
    if (n % NT || k % G::KS) return -1;
    const int nrb = (m + MT - 1) / MT;
    const int grid = nrb * (n / NT);
    const int xcd = (grid % 8 == 0 && (grid / 8) % nrb == 0) ? 1 : 0;
    if (math_mode() == WS_MATH_NATIVE)
        hipLaunchKernelGGL((gemm_line_kernel<MT, NT, WMH, D, SMODE, OMODE, false>), dim3(grid),
                           dim3(256), G::lds_bytes(D), stream, a, sa, b, sb, out, m, n, k, nrb, xcd,
                           aux);
    else
        hipLaunchKernelGGL((gemm_line_kernel<MT, NT, WMH, D, SMODE, OMODE, true>), dim3(grid),
                           dim3(256), G::lds_bytes(D), stream, a, sa, b, sb, out, m, n, k, nrb, xcd,
                           aux);
    return launch_status();
}


// The line kernel for (m, n, k) in tiling cfg when the shape fits it, else
// -1 (the caller runs another kernel).
template <int SMODE, int OMODE>
static int launch_line(const uint8_t *a, const void *sa, const uint8_t *b, const void *sb, void *out,
                       int m, int n, int k, hipStream_t stream, int cfg, const float *aux) {
    switch (cfg) {
        // 64 x 32 tiles, 4 waves on the 4 sub-steps of 512-K stages, 3 stages
        case 0: return launch_line_cfg<64, 32, 1, 3, SMODE, OMODE>(a, sa, b, sb, out, m, n, k, stream, aux);
        // 32 x 32 tiles (four row blocks per column block on one XCD), 3 stages
        case 2: return launch_line_cfg<32, 32, 1, 3, SMODE, OMODE>(a, sa, b, sb, out, m, n, k, stream, aux);
        // 128 x 48 tiles (two 64-row halves x two K sub-steps of 256-K
        // stages), 3 stages: wide N (M=128, N=12288)
        case 4: return launch_line_cfg<128, 48, 2, 3, SMODE, OMODE>(a, sa, b, sb, out, m, n, k, stream, aux);
        default: return -1;
    }
}

int line_gemm(int smode, int omode, const uint8_t *a, const void *sa, const uint8_t *b,
              const void *sb, void *out, int m, int n, int k, hipStream_t stream, int cfg,
              const float *aux) {
    if (smode == kUe8m0) {
        switch (omode) {
            case kOutF32: return launch_line<kUe8m0, kOutF32>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
            case kOutBf16: return launch_line<kUe8m0, kOutBf16>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
            case kOutAcc: return launch_line<kUe8m0, kOutAcc>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
            case kOutAcc2: return launch_line<kUe8m0, kOutAcc2>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
            default: return -1;
        }
    }
    switch (omode) {
        case kOutF32: return launch_line<kF32s, kOutF32>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
        case kOutBf16: return launch_line<kF32s, kOutBf16>(a, sa, b, sb, out, m, n, k, stream, cfg, aux);
        default: return -1;
    }
}

}  // namespace ws
