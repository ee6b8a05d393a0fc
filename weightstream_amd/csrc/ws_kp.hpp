// The 16-column-strip GEMM/GEMV body (gemm.hip's gemm_kp_kernel) as a
// device function, so that other launches (the fused decode steps) can run
// it on some of their workgroups.
#pragma once

#include "ws_internal.hpp"

namespace ws {

enum ScaleMode { kUe8m0 = 0, kF32s = 1 };
// kOutAcc: C += sum; kOutAcc2: C = C + (aux + sum); kOutSwiglu: fragment 0
// is a gate column, fragment 1 the up column jstride rows further, and C gets
// silu(min(g, L)) * clamp(u, -L, L) (the three used by the fused GEMV paths,
// one K split only)
enum OutMode { kOutF32 = 0, kOutBf16 = 1, kOutAcc = 2, kOutAcc2 = 3, kOutSwiglu = 4 };
static_assert(kOutAcc == kGemvAcc && kOutAcc2 == kGemvAcc2 && kOutSwiglu == kGemvSwiglu, "");

// ---- K-parallel GEMM: one workgroup per 16 output columns -----------------
// HBM-bound shapes (M <= a few hundred, e.g. M=128, K=4096): the weight matrix
// must cross HBM exactly once, so a workgroup owns a 16*NF-column strip of B
// for all K and up to 16*MF*GMH rows of A. Its GMH x GK waves split the rows in
// GMH halves and K in GK parts; a wave streams its K part in double-buffered
// register stages of U 128-K steps (clamped, unconditional loads: one wait per
// stage). The GK partial sums meet in LDS and are added in wave order
// (deterministic). The activation scales of the workgroup's rows (f32, or a
// step's four UE8M0 bytes) are staged in LDS once, transposed to [step][row].
template <int MF, int NF, int U>
struct KpStage {
    uint4 a[U][MF][2];
    uint32_t sa[U][MF];
    uint4 b[U][NF][2];
    uint32_t sb[U][NF];
    float sbf[U];
};

constexpr int kKpMaxSaWords = 16;  // activation scale words staged per thread

//
// AF32: A is f32 (M <= 16 rows); the workgroup quantises it per 1x32 block
// (the act_quant rule, quant_fp8_block32: the bytes ws_emit8 writes) into
// LDS, rows K + 16 bytes apart, while its first weight stages are in flight,
// and the waves read their A fragments and scale words from there.
//
// ALDS (blocks of 32 or 64 rows, one step per stage): a wave's A rows go
// through two LDS buffers of its own by direct global->LDS loads, one
// instruction per 8 whole 128-byte rows, instead of into registers in the
// MFMA layout (whose 16-byte pieces cover half of each row's line per
// instruction). Measured on the load pattern of a 64 x 32 tile at K=4096:
// 8.1 against 11.4 us to deliver A and the weights. The 16-byte pieces of a
// row are XOR-permuted by (row >> 1) & 7, so fragment reads hit distinct
// banks; every LDS access of the multiply is an asm read ordered by explicit
// waits, so the compiler adds no wait for the direct loads of the newer stage.
__device__ __forceinline__ int kp_sw8(int row, int c) { return c ^ ((row >> 1) & 7); }

template <int MF, int NF, int GMH, int GK, bool ALDS>
__host__ __device__ constexpr size_t kp_head_bytes() {
    // the A buffers (ALDS) and, after the multiply, the GK partial tiles
    return ALDS && (size_t)GK * GMH * 2 * 16 * MF * 128 > (size_t)GK * 16 * MF * GMH * 16 * NF * 4
               ? (size_t)GK * GMH * 2 * 16 * MF * 128
               : (size_t)GK * 16 * MF * GMH * 16 * NF * 4;
}

template <int MF, int NF, int GMH, int GK, bool BFP4, int SMODE, int OMODE, int U, bool EXACT,
          bool AF32 = false, bool ALDS = false>
__device__ __forceinline__ void kp_body(int bx, int by, int bz, const uint8_t *A, const void *SA,
                                        const uint8_t *__restrict__ B, const void *__restrict__ SB,
                                        void *__restrict__ C, int M, int N, int K, int S,
                                        float *__restrict__ part_out, int sb_div, const float *aux,
                                        float limit, int jstride) {
    constexpr int kRows = 16 * MF * GMH;
    constexpr int kCols = 16 * NF;
    static_assert(!AF32 || (MF == 1 && GMH == 1 && SMODE == kUe8m0 && !BFP4), "AF32: a GEMV");
    static_assert(OMODE != kOutSwiglu || NF == 2, "SwiGLU pairs two fragments");
    static_assert(!ALDS || (!AF32 && U == 1 && MF >= 2), "ALDS: blocks of rows, one step per stage");
    // UE8M0 activation scales: staged in LDS for blocks of rows; a single
    // 16-row fragment (GEMV) loads its word per step instead (no prologue)
    constexpr bool kStageSa = !AF32 && (SMODE == kF32s || kRows > 16);
    constexpr int kThreads = 64 * GMH * GK;
    extern __shared__ __align__(16) float kp_lds[];
    float *part = kp_lds;                         // [GK][kRows][kCols]
    float *sa_l = (float *)((uint8_t *)kp_lds + kp_head_bytes<MF, NF, GMH, GK, ALDS>());  // [ksteps][kRows]
    uint8_t *a_l = (uint8_t *)sa_l;               // AF32: [M][K + 16] e4m3
    const int a_pitch = K + 16;
    uint8_t *as_l = a_l + (size_t)M * a_pitch;    // AF32: [M][K / 32] UE8M0
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int wk = w % GK, wm = w / GK;
    const int r = lane & 15, g = lane >> 4;
    const int n0 = bx * (OMODE == kOutSwiglu ? 16 : kCols);
    const int mb = by * kRows;                   // workgroup's first row
    const int ml = wm * 16 * MF;                 // wave's first row within the workgroup
    const int ksteps = K / 128;
    // K split S ways over bz (S > 1: f32 partial planes, added in
    // split order by split_reduce_kernel), then over the GK waves
    const int kz0 = bz * ksteps / S, kzn = (bz + 1) * ksteps / S - kz0;
    const int k0 = kz0 + wk * kzn / GK, k1 = kz0 + (wk + 1) * kzn / GK;
    const int kbn = K / 32, kb128 = K / 128;
    constexpr int kWRows = 16 * MF;  // A rows of a wave
    // ALDS: this wave's two A buffers
    uint8_t *ring = (uint8_t *)kp_lds + (size_t)w * 2 * kWRows * 128;

    // activation scales of the workgroup's rows, one 32-bit word per (row,
    // step): the f32 scale, or the step's four UE8M0 bytes. Loaded first
    // and staged in LDS as [step][row].
    // four steps per 16-byte load when the rows allow it, else word by word
    uint32_t sav[kKpMaxSaWords];
    const int nsa = kRows * ksteps;  // <= kThreads * kKpMaxSaWords (checked on the host)
    const bool quad = (ksteps % 4) == 0 && (((uintptr_t)SA & 15) == 0);
    if (kStageSa) {
        if (quad) {
#pragma unroll
            for (int j = 0; j < kKpMaxSaWords / 4; j++) {
                // words e..e+3 = row_local * ksteps + ks .. +3
                const int e = min((j * kThreads + t) * 4, nsa - 4);
                const int rl = e / ksteps, ks = e % ksteps;
                const int row = min(mb + rl, M - 1);
                const uint4 v = SMODE == kF32s
                                    ? *(const uint4 *)((const uint32_t *)SA + (size_t)row * kb128 + ks)
                                    : *(const uint4 *)((const uint8_t *)SA + (size_t)row * kbn + ks * 4);
                sav[4 * j] = v.x;
                sav[4 * j + 1] = v.y;
                sav[4 * j + 2] = v.z;
                sav[4 * j + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kKpMaxSaWords; j++) {
                const int e = min(j * kThreads + t, nsa - 1);
                const int rl = e / ksteps, ks = e % ksteps;
                const int row = min(mb + rl, M - 1);
                sav[j] = SMODE == kF32s ? *((const uint32_t *)SA + (size_t)row * kb128 + ks)
                                        : *(const uint32_t *)((const uint8_t *)SA + (size_t)row * kbn + ks * 4);
            }
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
    // ALDS: instruction q of a step loads wave rows 8q + lane / 8, piece
    // kp_sw8(row, lane % 8)
    const uint8_t *asrc[ALDS ? 2 * MF : 1];
    if (ALDS) {
#pragma unroll
        for (int q = 0; q < 2 * MF; q++) {
            const int rl = 8 * q + (lane >> 3);
            asrc[q] = A + (size_t)min(mb + ml + rl, M - 1) * K + kp_sw8(rl, lane & 7) * 16;
        }
    }
    const uint8_t *brow[NF];
    const uint8_t *sbrow[NF];
#pragma unroll
    for (int j = 0; j < NF; j++) {
        const int col = n0 + (OMODE == kOutSwiglu ? j * jstride : 16 * j) + r;
        brow[j] = BFP4 ? B + (size_t)col * (K / 2) + g * 16
                       : B + (size_t)col * K + (EXACT ? g * 32 : g * 16);
        // FP8 weight scales: one row per 32-row block, or per row (sb_div 1)
        sbrow[j] = (const uint8_t *)SB + (size_t)(BFP4 ? col : col / sb_div) * kbn;
    }
    const float *sbf_row = (const float *)SB + (size_t)(n0 / 128) * kb128;

    auto load = [&](KpStage<MF, NF, U> &st, int ks0, int buf) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int ks = max(min(ks0 + u, k1 - 1), 0);
            if (ALDS) {
#pragma unroll
                for (int q = 0; q < 2 * MF; q++)
                    __builtin_amdgcn_global_load_lds(
                        (const void *)(asrc[q] + (size_t)ks * 128),
                        (__attribute__((address_space(3))) void *)(ring + buf * kWRows * 128 + q * 1024),
                        16, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < MF; i++) {
                if (AF32 || ALDS) break;  // A is read from LDS at use
                const uint8_t *p = arow[i] + (size_t)ks * 128;
                st.a[u][i][0] = ldg16(p);
                st.a[u][i][1] = ldg16(p + (EXACT ? 16 : 64));
                if (!kStageSa) st.sa[u][i] = *(const uint32_t *)(sarow[i] + ks * 4) >> (8 * g);
            }
#pragma unroll
            for (int j = 0; j < NF; j++) {
                if (BFP4) {
                    st.b[u][j][0] = ldg16(brow[j] + (size_t)ks * 64);
                } else {
                    const uint8_t *p = brow[j] + (size_t)ks * 128;
                    st.b[u][j][0] = ldg16(p);
                    st.b[u][j][1] = ldg16(p + (EXACT ? 16 : 64));
                }
                if (SMODE == kUe8m0) st.sb[u][j] = *(const uint32_t *)(sbrow[j] + ks * 4) >> (8 * g);
            }
            if (SMODE == kF32s) st.sbf[u] = sbf_row[ks];
        }
    };

    v4f acc[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; i++)
#pragma unroll
        for (int j = 0; j < NF; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // ALDS: VMEM instructions of one stage that precede nothing of the
    // older stage (the direct A loads, the weight pieces, their UE8M0 words;
    // a wave-uniform f32 scale load may go to the scalar unit): waiting
    // until at most that many are in flight leaves the older stage landed
    constexpr int kStageVm = 2 * MF + NF * (BFP4 ? 1 : 2) + (SMODE == kUe8m0 ? NF : 0);
    // A fragment i of buffer `buf` (ALDS): the two pieces a lane holds
    auto a_lds = [&](int buf, int i, uint4 &lo, uint4 &hi) {
        const int rl = 16 * i + r;
        const int pa = EXACT ? 2 * g : g, pb = EXACT ? 2 * g + 1 : g + 4;
        const uint32_t base = lds_addr(ring + buf * kWRows * 128 + rl * 128);
        u32x4v x = lds_read_b128(base + kp_sw8(rl, pa) * 16);
        u32x4v y = lds_read_b128(base + kp_sw8(rl, pb) * 16);
        lds_wait_all();
        lds_ready(x);
        lds_ready(y);
        lo = uint4{x[0], x[1], x[2], x[3]};
        hi = uint4{y[0], y[1], y[2], y[3]};
    };
    // LDS scale words (kStageSa) as asm reads under ALDS
    auto sa_word = [&](int idx) -> uint32_t {
        if (!ALDS) return ((const uint32_t *)sa_l)[idx];
        uint32_t v = lds_read_b32(lds_addr(sa_l + idx));
        lds_wait_all();
        lds_ready(v);
        return v;
    };
    auto sa_quad = [&](int idx) -> float4 {
        if (!ALDS) return *(const float4 *)(sa_l + idx);
        u32x4v v = lds_read_b128(lds_addr(sa_l + idx));
        lds_wait_all();
        lds_ready(v);
        return float4{__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3])};
    };
    auto compute = [&](const KpStage<MF, NF, U> &st, int ks0, int buf, bool newer) {
        if (ALDS) {
            if (newer) wait_vm<kStageVm>();
            else wait_vm<0>();
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int ks = ks0 + u;
            if (ks >= k1) continue;  // uniform
            if (EXACT) {
                v8bf bq[NF][4];
#pragma unroll
                for (int j = 0; j < NF; j++) {
                    const float sbv = SMODE == kUe8m0 ? e8m0_to_f32(st.sb[u][j] & 0xFF) : 1.0f;
                    if (BFP4) cvt_fp4x32(st.b[u][j][0], sbv, bq[j]);
                    else cvt_fp8x32(st.b[u][j][0], st.b[u][j][1], sbv, bq[j]);
                }
#pragma unroll
                for (int i = 0; i < MF; i++) {
                    v8bf aq[4];
                    uint4 a0, a1;
                    uint32_t saw;
                    if (AF32) {
                        const int rl = min(r, M - 1);
                        const uint8_t *ap = a_l + rl * a_pitch + ks * 128 + g * 32;
                        a0 = *(const uint4 *)ap;
                        a1 = *(const uint4 *)(ap + 16);
                        saw = *(const uint32_t *)(as_l + rl * (K / 32) + ks * 4) >> (8 * g);
                    } else {
                        if (ALDS) {
                            a_lds(buf, i, a0, a1);
                        } else {
                            a0 = st.a[u][i][0];
                            a1 = st.a[u][i][1];
                        }
                        saw = !kStageSa ? st.sa[u][i] : sa_word(ks * kRows + ml + 16 * i + r) >> (8 * g);
                    }
                    const float sav_f = SMODE == kUe8m0 ? e8m0_to_f32(saw & 0xFF) : 1.0f;
                    cvt_fp8x32(a0, a1, sav_f, aq);
#pragma unroll
                    for (int j = 0; j < NF; j++) {
                        if (SMODE == kUe8m0) {
                            acc[i][j] = mfma_bf16_k128(aq, bq[j], acc[i][j]);
                        } else {
                            const v4f p = mfma_bf16_k128(aq, bq[j], v4f{0.f, 0.f, 0.f, 0.f});
                            const float4 sa4 = sa_quad(ks * kRows + ml + 16 * i + 4 * g);
                            const float sa_v[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                acc[i][j][v] = acc[i][j][v] + p[v] * (sa_v[v] * st.sbf[u]);
                        }
                    }
                }
            } else {
                v8i b[NF];
#pragma unroll
                for (int j = 0; j < NF; j++)
                    b[j] = BFP4 ? frag_from4(st.b[u][j][0]) : frag_from(st.b[u][j][0], st.b[u][j][1]);
#pragma unroll
                for (int i = 0; i < MF; i++) {
                    v8i a;
                    int sai;
                    if (AF32) {
                        const int rl = min(r, M - 1);
                        const uint8_t *ap = a_l + rl * a_pitch + ks * 128 + g * 16;
                        a = frag_from(*(const uint4 *)ap, *(const uint4 *)(ap + 64));
                        sai = (int)((*(const uint32_t *)(as_l + rl * (K / 32) + ks * 4) >> (8 * g)) & 0xFF);
                    } else {
                        if (ALDS) {
                            uint4 lo, hi;
                            a_lds(buf, i, lo, hi);
                            a = frag_from(lo, hi);
                        } else {
                            a = frag_from(st.a[u][i][0], st.a[u][i][1]);
                        }
                        sai = SMODE != kUe8m0 ? 0
                              : !kStageSa     ? (int)(st.sa[u][i] & 0xFF)
                                              : (int)((sa_word(ks * kRows + ml + 16 * i + r) >> (8 * g)) & 0xFF);
                    }
#pragma unroll
                    for (int j = 0; j < NF; j++) {
                        if (SMODE == kUe8m0) {
                            acc[i][j] = BFP4 ? mfma_scaled<kFmtFp8, kFmtFp4>(a, b[j], acc[i][j], sai,
                                                                             (int)(st.sb[u][j] & 0xFF))
                                             : mfma_scaled<kFmtFp8, kFmtFp8>(a, b[j], acc[i][j], sai,
                                                                             (int)(st.sb[u][j] & 0xFF));
                        } else {
                            const v4f p = mfma_scaled<kFmtFp8, kFmtFp8>(a, b[j], v4f{0.f, 0.f, 0.f, 0.f},
                                                                        kScaleOne, kScaleOne);
                            const float4 sa4 = sa_quad(ks * kRows + ml + 16 * i + 4 * g);
                            const float sa_v[4] = {sa4.x, sa4.y, sa4.z, sa4.w};
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                acc[i][j][v] = acc[i][j][v] + p[v] * (sa_v[v] * st.sbf[u]);
                        }
                    }
                }
            }
        }
    };

    // AF32: the activation is read in rounds of kXR float4 per thread, the
    // first round before the weight stages: loads return in issue order, so
    // a wait for activation values issued after the weights would wait for
    // the weights too (measured at M=1, K=8192: 12.9 against 8.2 us for the
    // GEMV of pre-quantised bytes; 11.0 us this way)
    constexpr int kXR = 4;
    const float4 *X = (const float4 *)A;
    const int n4 = AF32 ? M * K / 4 : 0;
    float4 xr[AF32 ? kXR : 1];
    if (AF32) {
#pragma unroll
        for (int j = 0; j < kXR; j++) {
            const int i = j * kThreads + t;
            xr[j] = i < n4 ? X[i] : float4{0.f, 0.f, 0.f, 0.f};
        }
    }
    mem_order();
    KpStage<MF, NF, U> s0, s1;
    load(s0, k0, 0);
    mem_order();
    load(s1, k0 + U, 1);
    mem_order();
    if (AF32) {
        // four values per lane, a 1x32 block per 8 lanes; every lane of a
        // block takes part in its maximum (dead blocks quantise zeros and
        // store nothing; M K % 32 == 0)
        for (int base = 0; base < n4; base += kXR * kThreads) {
            if (base > 0) {
#pragma unroll
                for (int j = 0; j < kXR; j++) {
                    const int i = base + j * kThreads + t;
                    xr[j] = i < n4 ? X[i] : float4{0.f, 0.f, 0.f, 0.f};
                }
            }
#pragma unroll
            for (int j = 0; j < kXR; j++) {
                const int i = base + j * kThreads + t;
                uint32_t sbyte;
                const uint32_t q = quant_fp8_block32_x4(xr[j], &sbyte);
                if (i < n4) {
                    const int row = (4 * i) / K, col = 4 * i - row * K;
                    *(uint32_t *)(a_l + row * a_pitch + col) = q;
                    if ((t & 7) == 0) as_l[row * (K / 32) + col / 32] = (uint8_t)sbyte;
                }
            }
        }
        lds_barrier();
    }
    if (kStageSa) {
        uint32_t *sa_w = (uint32_t *)sa_l;
#pragma unroll
        for (int j = 0; j < kKpMaxSaWords; j++) {
            const int e = quad ? ((j / 4) * kThreads + t) * 4 + j % 4 : j * kThreads + t;
            if (e >= nsa) continue;
            const int rl = e / ksteps, ks = e % ksteps;
            if (ALDS) lds_write_b32(lds_addr(sa_w + ks * kRows + rl), sav[j]);
            else sa_w[ks * kRows + rl] = sav[j];
        }
        if (ALDS) {
            lds_wait_all();
            raw_barrier();
        } else {
            lds_barrier();
        }
    }

    // steady state: both stages reloaded unconditionally (straight-line body)
    const int nst = (k1 - k0 + U - 1) / U;
    int i = 0, ks0 = k0;
    for (; i + 3 < nst; i += 2, ks0 += 2 * U) {
        compute(s0, ks0, 0, true);
        mem_order();
        load(s0, ks0 + 2 * U, 0);
        mem_order();
        compute(s1, ks0 + U, 1, true);
        mem_order();
        load(s1, ks0 + 3 * U, 1);
        mem_order();
    }
    const int rest = nst - i;
    if (rest == 3) {
        compute(s0, ks0, 0, true);
        mem_order();
        load(s0, ks0 + 2 * U, 0);
        mem_order();
        compute(s1, ks0 + U, 1, true);
        compute(s0, ks0 + 2 * U, 0, false);
    } else {
        if (rest >= 1) compute(s0, ks0, 0, rest == 2);
        if (rest == 2) compute(s1, ks0 + U, 1, false);
    }
    // ALDS: the partial tiles reuse the A buffers of other waves
    if (ALDS) __syncthreads();

    // D[m][n]: lane -> row 4g+v of fragment i, column 16j + r
#pragma unroll
    for (int f = 0; f < MF; f++)
#pragma unroll
        for (int j = 0; j < NF; j++)
#pragma unroll
            for (int v = 0; v < 4; v++)
                part[(wk * kRows + ml + 16 * f + 4 * g + v) * kCols + 16 * j + r] = acc[f][j][v];
    __syncthreads();
    auto wave_sum = [&](int rl, int c) {
        float sum = part[rl * kCols + c];
#pragma unroll
        for (int q = 1; q < GK; q++) sum = sum + part[(q * kRows + rl) * kCols + c];
        return sum;
    };
    if (OMODE == kOutSwiglu) {
        // C [M][N]: N = the intermediate width (jstride)
        for (int o = t; o < kRows * 16; o += kThreads) {
            const int rl = o / 16, c = o % 16;
            const int row = mb + rl;
            if (row >= M) continue;
            float gv = wave_sum(rl, c), uv = wave_sum(rl, c + 16);
            if (limit > 0.0f) {
                uv = rclamp(uv, -limit, limit);
                gv = fminf(gv, limit);
            }
            ((float *)C)[(size_t)row * N + n0 + c] = ws_silu(gv) * uv;
        }
        return;
    }
    for (int o = t; o < kRows * kCols; o += kThreads) {
        const int rl = o / kCols, c = o % kCols;
        const int row = mb + rl;
        if (row >= M) continue;
        const float sum = wave_sum(rl, c);
        const size_t at = (size_t)row * N + n0 + c;
        if (S > 1) part_out[((size_t)bz * M + row) * N + n0 + c] = sum;
        else if (OMODE == kOutF32) ((float *)C)[at] = sum;
        else if (OMODE == kOutBf16) ((uint16_t *)C)[at] = f32_to_bf16(sum);
        else if (OMODE == kOutAcc) ((float *)C)[at] = ((float *)C)[at] + sum;
        else ((float *)C)[at] = ((float *)C)[at] + (aux[at] + sum);
    }
}

}  // namespace ws
