// Routed FP4 experts for one token (M = 1 decode).
//
// Replaces the reference's device-side grouped decode chain
// moe_local_slots -> expert_glu -> expert_quant -> expert_reduce
// (weightstream-cuda/kernels/moe_grouped.cu:23-224, launch.rs:89-206) with two
// kernels. CPU semantics: weightstream-ref moe.rs:75-84 (experts summed in
// ascending id) and :162-208 (gate/up, asymmetric swiglu clamps, routing
// weight before the FP8 re-quantisation and the down projection).
//
// M = 1 is HBM-bound: the two kernels stream 8 x 3 x 4.45 MB of packed FP4
// weights + UE8M0 scales once. Each wave owns 16 weight rows and walks K in
// 128-wide steps with one 16-byte load per lane per step; the token sits in
// LDS and feeds the MFMA's other operand (every column of the 16x16 MFMA
// output is the same token). Exact mode dequantises the weights to bf16 in
// registers (v_cvt_scalef32_pk_bf16_fp4 applies the UE8M0 scale) and keeps
// the token as exact bf16 in LDS; native mode feeds the scaled FP4 x FP8 MFMA.
//
//  glu_quant: 8 streaming waves per workgroup. A wave streams one packed
//    16-row band of w1 or w3 (double-buffered 8 KB register stages) and,
//    while its first stages are in flight, quantises 1/8 of the token into
//    LDS; the waves meet at an LDS-only barrier. At the BASELINE shape a workgroup owns two 32-row tiles
//    and every wave walks the whole K (256 workgroups: one resident round);
//    smaller problems give a workgroup one tile with K split in halves. The
//    epilogue applies SwiGLU x routing weight and quantises each 32-value
//    tile (one FP8 1x32 block) straight to e4m3 + UE8M0.
//  reduce: grid (dim/16), 8 streaming waves over (expert, K part) units for
//    16 output rows; each also decodes 1/8 of the picks' hidden states into
//    LDS; per-expert results meet in LDS and are added in ascending
//    expert id, one f32 add per expert like the reference's acc_f32 chain.
#include <mutex>

#include "ws_internal.hpp"
#include "ws_kp.hpp"
#include "ws_pack.hpp"
#include "ws_route.hpp"

namespace ws {

constexpr int kGluKParts = 2;       // glu: (w1|w3) x (rows 0-15|16-31) x K half,
constexpr int kGluStreamWaves = 4 * kGluKParts;
constexpr int kDecThreads = 64 * kGluStreamWaves;
constexpr int kRedWaves = 8;        // reduce: 8 streaming waves over (expert, K part) units
constexpr int kRedThreads = 64 * kRedWaves;
constexpr int kMaxTopkDec = 16;
constexpr int kMaxPickBytes = 32768;  // top_k * inter: the picks in LDS as bf16
constexpr int kRedShareRounds = kMaxPickBytes / kRedWaves / 1024;

// The picks as the whole wave sees them: lane j < top_k holds pick j (its
// expert id and its rank among the valid picks ordered by (expert id, slot)).
// One vector load and top_k lane reads; no memory round trip per pick.
struct WavePicks {
    int e;     // expert id of the lane's pick (-1 for lanes >= top_k)
    int rank;  // rank of the lane's pick, -1 if invalid (outside [0, E))
    int nv;    // number of valid picks
};

// from lane j's pick (expert id e_lane for lanes < top_k)
__device__ __forceinline__ WavePicks wave_picks_of(int e_lane, int top_k, int n_experts,
                                                   int lane) {
    WavePicks wp;
    wp.e = lane < top_k ? e_lane : -1;
    const bool valid = lane < top_k && wp.e >= 0 && wp.e < n_experts;
    int rank = 0;
    for (int i = 0; i < top_k; i++) {
        const int ei = __builtin_amdgcn_readlane(wp.e, i);
        const bool vi = ei >= 0 && ei < n_experts;
        rank += (vi && (ei < wp.e || (ei == wp.e && i < lane))) ? 1 : 0;
    }
    wp.rank = valid ? rank : -1;
    wp.nv = __popcll(__ballot(valid));
    return wp;
}

// The valid picks in summation order (ascending expert id, then slot), as
// the down kernel walks them: lane r < nv holds the gate-output slot of the
// pick of rank r (its row of hq / hs) and its expert's row in the slab.
struct RankedPicks {
    int slot;
    int e;
    int nv;
};


// from moe_local_slots' lists (moe_grouped.cu:23-58: slots already in
// ascending expert id): slot local[r], slab row gate_idx[slot] - e_start.
// A row outside [0, e_len) (which moe_local_slots never produces) is dropped
// instead of read out of bounds.
__device__ __forceinline__ RankedPicks ranked_from_local(const int32_t *local,
                                                         const int32_t *local_count,
                                                         const int32_t *gate_idx, int e_start,
                                                         int e_len, int top_k, int lane) {
    const int cnt = min(*local_count, top_k);
    int slot = 0, e = -1;
    if (lane < cnt) {
        slot = local[lane];
        e = (slot >= 0 && slot < top_k) ? gate_idx[slot] - e_start : -1;
    }
    const bool valid = lane < cnt && e >= 0 && e < e_len;
    const unsigned long long vm = __ballot(valid);
    const int nr = __popcll(vm & ((1ull << lane) - 1));
    RankedPicks rp{0, 0, (int)__popcll(vm)};
    for (int i = 0; i < cnt; i++) {
        if (((vm >> i) & 1) && __builtin_amdgcn_readlane(nr, i) == lane) {
            rp.slot = __builtin_amdgcn_readlane(slot, i);
            rp.e = __builtin_amdgcn_readlane(e, i);
        }
    }
    return rp;
}

// Multiply one register stage of a packed 16-row FP4 band with the operand in
// LDS: EXACT -> bf16 values (x_lds); native -> e4m3 bytes + UE8M0 scales
// (xq_lds, xs_lds). Returns the updated 16x16 accumulator (row i of the band
// in D[i][*]).
template <bool EXACT, int U>
__device__ __forceinline__ v4f fp4_compute(const Fp4StageU<U> &st, v4f acc, const uint8_t *xq_lds,
                                           const uint8_t *xs_lds, const __bf16 *x_lds, int kb,
                                           int ks0, int kend) {
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int ks = ks0 + u;
        if (ks >= kend) continue;  // uniform
        const uint32_t sw = stage_scale(st, u);
        if (EXACT) {
            v8bf wq[4], xb[4];
            cvt_fp4x32(st.w[u], e8m0_to_f32(sw), wq);
            const v8bf *xp = (const v8bf *)(x_lds + ks * 128 + kb * 32);
#pragma unroll
            for (int j = 0; j < 4; j++) xb[j] = xp[j];
            acc = mfma_bf16_k128(wq, xb, acc);
        } else {
            const uint8_t *xp = xq_lds + ks * 128 + kb * 16;
            v8i b = frag_from(*(const uint4 *)xp, *(const uint4 *)(xp + 64));
            acc = mfma_scaled<kFmtFp4, kFmtFp8>(frag_from4(st.w[u]), b, acc, (int)sw,
                                                (int)xs_lds[ks * 4 + kb]);
        }
    }
    return acc;
}

// Stream band steps [k0, k1) (k0 % U == 0) given the first two stages already
// in flight (s0 = k0.., s1 = k0+U..): one stage is multiplied while the
// other's loads are outstanding. The steady-state loop reloads both stages
// unconditionally, so its body is straight-line and each wait covers only the
// stage about to be used; the last two or three stages are the tail.
// `between` runs after each reload (the wave waits on memory there): the
// decode kernel's routing wave finishes its top-k rounds in those gaps.
struct NoHook {
    __device__ __forceinline__ void operator()() const {}
};

template <bool EXACT, int U, class Hook = NoHook>
__device__ __forceinline__ v4f fp4_stream(const Fp4Band &b, Fp4StageU<U> &s0, Fp4StageU<U> &s1,
                                          const uint8_t *xq_lds, const uint8_t *xs_lds,
                                          const __bf16 *x_lds, int kb, int k0, int k1,
                                          Hook between = Hook{}) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    const int nst = (k1 - k0 + U - 1) / U;
    int i = 0, ks0 = k0;
    for (; i + 3 < nst; i += 2, ks0 += 2 * U) {
        acc = fp4_compute<EXACT, U>(s0, acc, xq_lds, xs_lds, x_lds, kb, ks0, k1);
        fp4_load(s0, b, ks0 + 2 * U, k1);
        between();
        acc = fp4_compute<EXACT, U>(s1, acc, xq_lds, xs_lds, x_lds, kb, ks0 + U, k1);
        fp4_load(s1, b, ks0 + 3 * U, k1);
        between();
    }
    const int rest = nst - i;
    if (rest == 3) {
        acc = fp4_compute<EXACT, U>(s0, acc, xq_lds, xs_lds, x_lds, kb, ks0, k1);
        fp4_load(s0, b, ks0 + 2 * U, k1);
        acc = fp4_compute<EXACT, U>(s1, acc, xq_lds, xs_lds, x_lds, kb, ks0 + U, k1);
        acc = fp4_compute<EXACT, U>(s0, acc, xq_lds, xs_lds, x_lds, kb, ks0 + 2 * U, k1);
    } else {
        if (rest >= 1) acc = fp4_compute<EXACT, U>(s0, acc, xq_lds, xs_lds, x_lds, kb, ks0, k1);
        if (rest == 2) acc = fp4_compute<EXACT, U>(s1, acc, xq_lds, xs_lds, x_lds, kb, ks0 + U, k1);
    }
    return acc;
}

// 128-K steps per register stage of the decode streams (two stages in
// flight per wave)
constexpr int kUD = 4;

// K range [k0, k1) of part `part` of `parts`, in whole decode stages
__device__ __forceinline__ void k_part(int ksteps, int part, int parts, int &k0, int &k1) {
    const int stages = (ksteps + kUD - 1) / kUD;
    k0 = min(ksteps, part * stages / parts * kUD);
    k1 = min(ksteps, (part + 1) * stages / parts * kUD);
}

// ---- operand preparation in LDS ------------------------------------------
// Every streaming wave converts a share of the operand all waves multiply (the
// token, or the picks' hidden states) into LDS. It issues the share's loads
// before its weight loads, converts while the weight stages are in flight,
// and the waves meet at an LDS-only barrier that leaves those loads in flight.

// ---- the token, split over the streaming waves ----------------------------
// Each of the `parts` streaming waves converts its share of the token into
// LDS. It issues the share's loads before its weight loads (loads return in
// order, so the conversion waits for the token bytes only) and converts while
// its weight stages are in flight. All rounds of a share are loaded up front
// (straight-line code: a wait for them never covers a weight load): 4 rounds
// of 256 f32 values (dim <= 8192) or 2 rounds of 1 KB e4m3 (dim <= 16384).
constexpr int kXRF = 4, kXRQ = 2;
constexpr int kMaxDimF32 = kGluStreamWaves * kXRF * 256;
constexpr int kMaxDimFp8 = kGluStreamWaves * kXRQ * 1024;

// e4m3 bytes + their UE8M0 scale bytes, 16 bytes per lane and round
template <int R>
struct Fp8Share {
    uint4 q[R];
    uint32_t s[R];
};

struct TokenRegs {
    float4 f[kXRF];   // f32 token: 4 values of one 1x32 block per lane and round
    Fp8Share<kXRQ> b; // e4m3 token
};

// f32 token, blocks [b0, b1) of 32 values: round r covers 8 blocks, a block
// is 8 lanes x 4 values. Loads are clamped into the share (or block 0).
__device__ __forceinline__ void tok_load_f32(TokenRegs &tr, const float *x, int b0, int b1,
                                             int lane) {
#pragma unroll
    for (int j = 0; j < kXRF; j++) {
        const int blk = max(min(b0 + j * 8 + (lane >> 3), b1 - 1), 0);
        tr.f[j] = *(const float4 *)(x + (size_t)blk * 32 + (lane & 7) * 4);
    }
}

// FP8 1x32 quantisation of the loaded rounds (the act_quant_fp8_emit rule,
// weightstream-ref actquant.rs:21-45) into LDS: exact bf16 values (EXACT) or
// e4m3 bytes + UE8M0 scales.
template <bool EXACT>
__device__ __forceinline__ void tok_quant_f32(const TokenRegs &tr, int b0, int b1, int lane,
                                              __bf16 *x_l, uint8_t *xq_l, uint8_t *xs_l) {
#pragma unroll
    for (int j = 0; j < kXRF; j++) {
        if (j * 8 >= b1 - b0) break;  // uniform
        const int blk = b0 + j * 8 + (lane >> 3);
        const float4 v = tr.f[j];
        float amax = fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                           fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
        amax = max8_lanes(amax);
        if (!(amax >= 1e-4f)) amax = 1e-4f;
        const int e = log2_ceil_div448(amax);
        const float inv = block_inv_scale(e), sc = __builtin_ldexpf(1.0f, e);
        const float f[4] = {v.x, v.y, v.z, v.w};
        const int i = blk * 32 + (lane & 7) * 4;
        if (EXACT) {
            // the dequantised values (e4m3 value x 2^e), each with at most 4
            // significant bits, so exact in bf16
            float d[4];
#pragma unroll
            for (int c = 0; c < 4; c++) d[c] = e4m3_round_value(rclamp(f[c] * inv, -448.0f, 448.0f)) * sc;
            // (an infinite block: sc = inf, so every value is NaN, as the
            // reference's decoded scale byte 0xFF is)
            if (blk >= b1) continue;
            *(uint2 *)(x_l + i) =
                uint2{(__float_as_uint(d[0]) >> 16) | (__float_as_uint(d[1]) & 0xFFFF0000u),
                      (__float_as_uint(d[2]) >> 16) | (__float_as_uint(d[3]) & 0xFFFF0000u)};
        } else {
            uint32_t q[4];
#pragma unroll
            for (int c = 0; c < 4; c++) q[c] = block_byte(f[c], inv);
            if (blk >= b1) continue;
            *(uint32_t *)(xq_l + i) = q[0] | (q[1] << 8) | (q[2] << 16) | (q[3] << 24);
            if ((lane & 7) == 0) xs_l[blk] = (uint8_t)(e + 127);
        }
    }
}

// e4m3 bytes [c0, c1) (16-byte multiples, c1 - c0 <= R KB) with one scale
// byte per 32: 16 bytes per lane and round.
template <int R>
__device__ __forceinline__ void share_load_fp8(Fp8Share<R> &tr, const uint8_t *q, const uint8_t *s,
                                               int c0, int c1, int lane) {
#pragma unroll
    for (int j = 0; j < R; j++) {
        const int i = max(min(c0 + j * 1024 + lane * 16, c1 - 16), 0);
        tr.q[j] = *(const uint4 *)(q + i);
        tr.s[j] = s[i / 32];
    }
}

// As share_load_fp8 over the concatenation of the picks' rows in rank order:
// byte i of it is byte i % inter of hq row rp.slot of rank i / inter.
template <int R>
__device__ __forceinline__ void share_load_ranked(Fp8Share<R> &tr, const uint8_t *q,
                                                  const uint8_t *s, const RankedPicks &rp,
                                                  int inter, int c0, int c1, int lane) {
#pragma unroll
    for (int j = 0; j < R; j++) {
        const int i = max(min(c0 + j * 1024 + lane * 16, c1 - 16), 0);
        const int r = i / inter, off = i - r * inter;
        const int row = max(__shfl(rp.slot, r, 64), 0);
        const size_t a = (size_t)row * inter + off;
        tr.q[j] = *(const uint4 *)(q + a);
        tr.s[j] = s[a / 32];
    }
}

// ... into LDS: exact bf16 values (EXACT) or the bytes and scales as they are.
// With slot_rank (lane s: the rank of row s, -1 to drop it) the source is the
// rows in slot order, each stored at its rank's row.
template <bool EXACT, int R>
__device__ __forceinline__ void share_store_fp8(const Fp8Share<R> &tr, int c0, int c1, int lane,
                                                __bf16 *x_l, uint8_t *xq_l, uint8_t *xs_l,
                                                int inter = 0, int slot_rank = 0,
                                                bool remap = false) {
#pragma unroll
    for (int j = 0; j < R; j++) {
        const int src = c0 + j * 1024 + lane * 16;
        int i = src;
        bool keep = src < c1;
        if (remap) {
            // every lane takes part in the shuffle
            const int sr = min(src, c1 - 1) / inter;
            const int rk = __shfl(slot_rank, min(sr, 63), 64);
            keep = keep && rk >= 0;
            i = rk * inter + (src - sr * inter);
        }
        if (!keep) continue;
        if (EXACT) {
            const float f = e8m0_to_f32(tr.s[j]);
            const uint32_t wd[4] = {tr.q[j].x, tr.q[j].y, tr.q[j].z, tr.q[j].w};
#pragma unroll
            for (int c = 0; c < 2; c++) {
                u32x4v o = pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * c], f, false),
                               __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * c], f, true),
                               __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * c + 1], f, false),
                               __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wd[2 * c + 1], f, true));
                *(u32x4v *)(x_l + i + 8 * c) = o;
            }
        } else {
            *(u32x4v *)(xq_l + i) = u32x4v{tr.q[j].x, tr.q[j].y, tr.q[j].z, tr.q[j].w};
            if ((i & 31) == 0) xs_l[i / 32] = (uint8_t)tr.s[j];
        }
    }
}

// Routing computed inside the gate/up kernel (moe_select fused in): the
// waves of every workgroup score the token's logits (a column of 64 experts
// each), wave 0 runs the top-k rounds (WaveTopk, the rounds of wave_select),
// and workgroup (0, 0) publishes the picks for the down kernel and the
// caller.
struct RouteArgs {
    const float *logits, *bias;
    int score_func;
    float gate_temp;
    int norm;
    float route_scale;
    int32_t *idx_out;
    float *w_out;
};

// Where the picks come from when the kernel does not route (CPL == 0):
//  - the top-k output (local == nullptr): workgroup row y is pick (slot) y,
//    expert idx[y], routing weight w[y];
//  - the reference's local-slot lists (moe_local_slots, moe_grouped.cu:23):
//    row y < *local_count is slot local[y] of the gate output, local expert
//    row local_experts[y], weight w[slot]; rows beyond the count do nothing.
// Either way h of a pick is written to row `slot` of the output, as the
// reference's expert_glu / expert_quant write h_slots / q_slots.
struct PickSrc {
    const int32_t *idx;
    const float *w;
    const int32_t *local, *local_experts, *local_count;
};

// CPL > 0: route in the kernel (CPL candidates per lane, E <= 64 CPL);
// CPL == 0: picks from `ps`. HF32: write h in f32 to hf [slot, inter]
// (expert_glu) instead of its FP8 1x32 quantisation to hq / hs.
template <bool EXACT, bool XF32, int CPL, bool HF32 = false>
__device__ __forceinline__ void glu_body(
    int bx, int by, const uint8_t *xq, const uint8_t *xs, const float *xf, const PickSrc &ps,
    const RouteArgs &ra, const uint8_t *__restrict__ w1, const uint8_t *__restrict__ s1,
    const uint8_t *__restrict__ w3, const uint8_t *__restrict__ s3, uint8_t *__restrict__ hq,
    uint8_t *__restrict__ hs, float *__restrict__ hf, int dim, int inter, int n_experts,
    int top_k, float limit, int tpw) {
    extern __shared__ __align__(16) uint8_t lds[];
    // EXACT: bf16 token (2*dim bytes); native: e4m3 token + scales
    __bf16 *x_l = (__bf16 *)lds;
    uint8_t *xq_l = lds;
    uint8_t *xs_l = lds + dim;
    __shared__ float gu[kGluKParts][2][32];
    int slot = by;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int ksteps = dim / 128;

    // waves -> (matrix, 16-row half of a 32-row tile, sub): with tpw == 2
    // the workgroup owns tiles 2x, 2x+1 and `sub` picks the tile (a wave
    // streams the whole K); with tpw == 1 it owns tile x and `sub` picks the
    // K half. Every wave also converts 1/8 of the token into LDS; its token
    // loads go out first (they do not depend on the routing).
    const int mat = (w >> 1) & 1, half = w & 1, sub = w >> 2;
    const int kparts = tpw == 2 ? 1 : kGluKParts;
    // token share: blocks [tb0, tb1) (f32) or bytes [tc0, tc1) (e4m3)
    const int nblk = dim / 32;
    const int tb0 = w * nblk / kGluStreamWaves, tb1 = (w + 1) * nblk / kGluStreamWaves;
    const int tc0 = tb0 * 32, tc1 = tb1 * 32;
    // the routing inputs first (the weight loads wait for the routing), then
    // the token share
    RouteIn<(CPL > 0 ? CPL : 1)> rin;
    if constexpr (CPL > 0) route_load<CPL>(rin, ra.logits, ra.bias, n_experts, lane);
    mem_order();
    TokenRegs tr;
    if (XF32) tok_load_f32(tr, xf, tb0, tb1, lane);
    else share_load_fp8(tr.b, xq, xs, tc0, tc1, lane);
    mem_order();

    // the slot's expert: with the routing in the kernel, the top-k rounds
    // up to this slot's run before the weight loads go out and the rest
    // while they are in flight (the same rounds in the same order)
    // (wave 0 alone runs the rounds, so that they do not share its SIMD with
    // another wave's copy; the scores come to it and the picks go to the
    // other waves through LDS)
    int e;
    float rw;
    WaveTopk<(CPL > 0 ? CPL : 1)> tk;
    __shared__ int e_l;
    __shared__ int pk_l[kMaxTopkDec];
    __shared__ float pw_l[kMaxTopkDec];
    if constexpr (CPL > 0) {
        // the scores column by column over the waves (expert lane + 64 c on
        // wave c % 8), through LDS to wave 0
        __shared__ float sc_l[CPL][64];
        for (int c = w; c < CPL; c += kGluStreamWaves) {
            float v[1] = {0.0f}, o[1];
#pragma unroll
            for (int j = 0; j < CPL; j++) v[0] = j == c ? rin.v[j] : v[0];  // no indexed load
            wave_scores_of<1>(v, ra.score_func, ra.gate_temp, lane, o);
            sc_l[c][lane] = o[0];
        }
        lds_barrier();
        if (w == 0) {
            float sc[CPL];
#pragma unroll
            for (int c = 0; c < CPL; c++) sc[c] = sc_l[c][lane];
            tk.init(sc, rin.b, n_experts, lane);
            e = 0;
            for (int k = 0; k <= slot; k++) e = tk.round(k, lane);
            if (lane == 0) e_l = e;
        }
        lds_barrier();
        e = e_l;
    } else if (ps.local) {
        const int i = slot;
        if (i >= *ps.local_count) return;  // whole workgroup
        slot = ps.local[i];
        e = ps.local_experts[i];
        rw = ps.w[slot];
    } else {
        e = ps.idx[slot];
        rw = ps.w[slot];
    }
    // whole workgroup: a pick another rank owns (or a row outside the slab)
    if (e < 0 || e >= n_experts) return;

    const int tile = bx * tpw + (tpw == 2 ? sub : 0);
    int k0, k1;
    k_part(ksteps, tpw == 2 ? 0 : sub, kparts, k0, k1);
    const size_t wmat = (size_t)inter * (dim / 2);
    const size_t smat = (size_t)packed_fp4_scale_bytes(inter, dim);
    const Fp4Band band = fp4_band((mat ? w3 : w1) + (size_t)e * wmat,
                                  (mat ? s3 : s1) + (size_t)e * smat, tile * 2 + half, dim, lane);
    Fp4StageU<kUD> st0, st1;
    fp4_load(st0, band, k0, k1);
    mem_order();
    fp4_load(st1, band, k0 + kUD, k1);
    mem_order();

    if (XF32) tok_quant_f32<EXACT>(tr, tb0, tb1, lane, x_l, xq_l, xs_l);
    else share_store_fp8<EXACT>(tr.b, tc0, tc1, lane, x_l, xq_l, xs_l);
    lds_barrier();

    {
        // the routing weight needs every pick: wave 0 runs the rounds after
        // this slot's in the gaps of its weight stream (the other waves do
        // not wait for them) and the rest after it; the weight is used in the
        // epilogue only
        int kn = slot + 1;
        auto rounds = [&]() {
            if constexpr (CPL > 0) {
                if (w == 0 && kn < top_k) {  // uniform
                    tk.round(kn, lane);
                    kn++;
                }
            }
        };
        v4f acc = fp4_stream<EXACT>(band, st0, st1, xq_l, xs_l, x_l, lane >> 4, k0, k1, rounds);
        if constexpr (CPL > 0) {
            if (w == 0) {
                for (; kn < top_k; kn++) tk.round(kn, lane);
                const int pk = tk.pick;
                const float pw = tk.weight(top_k, ra.norm, ra.route_scale);
                if (lane < top_k) {
                    pk_l[lane] = pk;
                    pw_l[lane] = pw;
                    if (bx == 0 && slot == 0) {
                        ra.idx_out[lane] = pk;
                        ra.w_out[lane] = pw;
                    }
                }
            }
        }
        // D[i][j]: i = weight row 4*(lane/16)+v, j = lane%16 (all columns equal)
        if ((lane & 15) == 0) {
#pragma unroll
            for (int v = 0; v < 4; v++) gu[sub][mat][half * 16 + 4 * (lane >> 4) + v] = acc[v];
        }
    }
    __syncthreads();
    if constexpr (CPL > 0) rw = pw_l[slot];
    if (w >= tpw) return;
    // wave w finishes tile bx * tpw + w; lanes 0-31 own its 32 values,
    // lanes 32-63 mirror them so the half-wave reduction stays uniform, and do
    // not store. K halves (tpw == 1) are added in fixed order.
    const int otile = bx * tpw + w;
    const int n = lane & 31;
    float g = gu[w][0][n], u = gu[w][1][n];
    for (int q = 1; q < kparts; q++) {
        g = g + gu[q][0][n];
        u = u + gu[q][1][n];
    }
    if (limit > 0.0f) {
        u = rclamp(u, -limit, limit);
        g = fminf(g, limit);
    }
    float h = ws_silu(g) * u * rw;
    if constexpr (HF32) {
        if (lane < 32) hf[(size_t)slot * inter + otile * 32 + n] = h;
    } else {
        uint32_t sb;
        uint32_t qb = quant_fp8_block32(h, &sb);
        if (lane < 32) {
            hq[(size_t)slot * inter + otile * 32 + n] = (uint8_t)qb;
            if (n == 0) hs[(size_t)slot * (inter / 32) + otile] = (uint8_t)sb;
        }
    }
}

template <bool EXACT, bool XF32, int CPL, bool HF32 = false>
__global__ __launch_bounds__(kDecThreads) void expert_glu_quant_kernel(
    const uint8_t *xq, const uint8_t *xs, const float *xf, PickSrc ps, RouteArgs ra,
    const uint8_t *__restrict__ w1, const uint8_t *__restrict__ s1,
    const uint8_t *__restrict__ w3, const uint8_t *__restrict__ s3, uint8_t *__restrict__ hq,
    uint8_t *__restrict__ hs, float *__restrict__ hf, int dim, int inter, int n_experts,
    int top_k, float limit, int tpw) {
    glu_body<EXACT, XF32, CPL, HF32>(blockIdx.x, blockIdx.y, xq, xs, xf, ps, ra, w1, s1, w3, s3,
                                     hq, hs, hf, dim, inter, n_experts, top_k, limit, tpw);
}

// The routed gate/up kernel with the shared expert's down GEMV on extra
// workgroups (rows top_k.. of the grid): ys [sdim] = emit8(hsf) . w2s^T, the
// 16-column-strip GEMV with the f32 activation quantised in the kernel (the
// same sums as ws_fp8_gemm of ws_emit8's bytes). Its weight stream joins the
// routed one; neither part reads the other's output.
struct SharedDown {
    const float *hsf;
    const uint8_t *w2, *s2;
    float *ys;
    int dim, inter;
};

template <bool EXACT, int CPL>
__global__ __launch_bounds__(kDecThreads) void glu_shared_down_kernel(
    const float *xf, RouteArgs ra, const uint8_t *__restrict__ w1,
    const uint8_t *__restrict__ s1, const uint8_t *__restrict__ w3,
    const uint8_t *__restrict__ s3, uint8_t *__restrict__ hq, uint8_t *__restrict__ hs, int dim,
    int inter, int n_experts, int top_k, float limit, int tpw, SharedDown sd) {
    if ((int)blockIdx.y < top_k) {
        glu_body<EXACT, true, CPL, false>(blockIdx.x, blockIdx.y, nullptr, nullptr, xf, PickSrc{},
                                          ra, w1, s1, w3, s3, hq, hs, nullptr, dim, inter,
                                          n_experts, top_k, limit, tpw);
        return;
    }
    const int b = (blockIdx.y - top_k) * gridDim.x + blockIdx.x;
    if (b >= sd.dim / 16) return;  // whole workgroup
    kp_body<1, 1, 1, 8, false, kUe8m0, kOutF32, 1, EXACT, true>(
        b, 0, 0, (const uint8_t *)sd.hsf, nullptr, sd.w2, sd.s2, sd.ys, 1, sd.dim, sd.inter, 1,
        nullptr, 32, nullptr, 0.0f, 16);
}

// Picks of the down kernel: the top-k output (local == nullptr; picks outside
// [0, E) skipped) or moe_local_slots' lists with the global ids in idx.
struct ReducePicks {
    const int32_t *idx;
    const int32_t *local, *local_count;
    int e_start;
};

template <bool EXACT>
__global__ __launch_bounds__(kRedThreads) void expert_reduce_kernel(
    const uint8_t *hq, const uint8_t *hs, ReducePicks pk,
    const uint8_t *__restrict__ w2, const uint8_t *__restrict__ s2, float *__restrict__ y, int dim,
    int inter, int n_experts, int top_k, float *hres, const float *ys) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float part[kMaxTopkDec][kRedWaves][16];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int row0 = blockIdx.x * 16;
    // the picks' hidden states: every wave converts 1/8 of them into LDS, in
    // rank order (ascending expert id). From the top-k output the rows are
    // loaded in slot order before the picks are ranked (no dependence on the
    // ranking) and stored at their ranks' rows; from local-slot lists, in
    // rank order after it.
    const bool by_slot = pk.local == nullptr;
    // the picks first: loads return in issue order, so the ranking then
    // waits for them only. Both loads go out unconditionally (the idx
    // clamped into its top_k entries, hq's top_k rows exist either way), so
    // that the ranking's wait counts the younger hq loads out.
    const int e_ld = pk.idx[min(lane, top_k - 1)];
    mem_order();
    Fp8Share<kRedShareRounds> hr;
    const int tot_s = top_k * inter;
    const int c0s = w * (tot_s / kRedWaves), c1s = c0s + tot_s / kRedWaves;
    share_load_fp8(hr, hq, hs, c0s, c1s, lane);
    mem_order();
    const int e_lane = (by_slot && lane < top_k) ? e_ld : -1;
    // every wave ranks the (<= 16) picks itself: no barrier before the loads
    WavePicks wp{};
    RankedPicks rp;
    if (by_slot) {
        wp = wave_picks_of(e_lane, top_k, n_experts, lane);
        rp = RankedPicks{0, 0, wp.nv};
        for (int i = 0; i < top_k; i++) {
            if (__builtin_amdgcn_readlane(wp.rank, i) == lane) {
                rp.slot = i;
                rp.e = __builtin_amdgcn_readlane(wp.e, i);
            }
        }
    } else {
        rp = ranked_from_local(pk.local, pk.local_count, pk.idx, pk.e_start, n_experts, top_k,
                               lane);
    }
    const int nv = rp.nv;
    const int tot = nv * inter;
    const int c0 = w * (tot / kRedWaves), c1 = c0 + tot / kRedWaves;
    if (!by_slot) share_load_ranked(hr, hq, hs, rp, inter, c0, c1, lane);
    mem_order();

    // work units (pick, K part): a wave streams 16 rows of one expert's w2
    // over 1/ksplit of inter; with 8 picks every wave owns one whole expert.
    // A wave without a unit streams nothing (its clamped loads re-read one
    // 1 KB step).
    const int ksteps = inter / 128;
    int ksplit = kRedWaves / (nv > 0 ? nv : 1);
    ksplit = ksplit < 1 ? 1 : ksplit;
    const int stages = (ksteps + kUD - 1) / kUD;
    if (ksplit > stages) ksplit = stages;
    const int nunits = nv * ksplit;
    const size_t wmat = (size_t)dim * (inter / 2);
    const size_t smat = (size_t)packed_fp4_scale_bytes(dim, inter);
    const bool has = w < nunits;
    int p = has ? w / ksplit : 0, ksp = has ? w % ksplit : 0, k0 = 0, k1 = 0;
    if (has) k_part(ksteps, ksp, ksplit, k0, k1);
    const int e0 = __builtin_amdgcn_readlane(rp.e, p);
    Fp4Band band = fp4_band(w2 + (size_t)e0 * wmat, s2 + (size_t)e0 * smat, blockIdx.x, inter,
                            lane);
    Fp4StageU<kUD> s0, s1;
    fp4_load(s0, band, k0, k1);
    mem_order();
    fp4_load(s1, band, k0 + kUD, k1);
    mem_order();

    // EXACT: picks as bf16 (2 * top_k * inter bytes); native: e4m3 + scales
    __bf16 *h_l = (__bf16 *)lds;
    uint8_t *hq_l = lds;
    uint8_t *hs_l = lds + (size_t)top_k * inter;
    if (by_slot)
        share_store_fp8<EXACT>(hr, c0s, c1s, lane, h_l, hq_l, hs_l, inter, wp.rank, true);
    else
        share_store_fp8<EXACT>(hr, c0, c1, lane, h_l, hq_l, hs_l);
    lds_barrier();

    if (has) {
        v4f acc = fp4_stream<EXACT>(band, s0, s1, hq_l + (size_t)p * inter,
                                    hs_l + (size_t)p * (inter / 32), h_l + (size_t)p * inter,
                                    lane >> 4, k0, k1);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int v = 0; v < 4; v++) part[p][ksp][4 * (lane >> 4) + v] = acc[v];
        }
    }
    // more units than waves (more than 8 picks)
    for (int unit = w + kRedWaves; unit < nunits; unit += kRedWaves) {
        p = unit / ksplit;
        ksp = unit % ksplit;
        k_part(ksteps, ksp, ksplit, k0, k1);
        const int e = __builtin_amdgcn_readlane(rp.e, p);
        band = fp4_band(w2 + (size_t)e * wmat, s2 + (size_t)e * smat, blockIdx.x, inter, lane);
        fp4_load(s0, band, k0, k1);
        fp4_load(s1, band, k0 + kUD, k1);
        v4f acc = fp4_stream<EXACT>(band, s0, s1, hq_l + (size_t)p * inter,
                                    hs_l + (size_t)p * (inter / 32), h_l + (size_t)p * inter,
                                    lane >> 4, k0, k1);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int v = 0; v < 4; v++) part[p][ksp][4 * (lane >> 4) + v] = acc[v];
        }
    }
    __syncthreads();
    if (t < 16) {
        // one f32 add per expert, ascending expert id (moe.rs:76-84)
        float acc = 0.0f;
        for (int q = 0; q < nv; q++) {
            float pe = part[q][0][t];
            for (int r = 1; r < ksplit; r++) pe = pe + part[q][r][t];
            acc = acc + pe;
        }
        y[row0 + t] = acc;
        // with hres: the block's residual add h = h + (y + ys) (acc_f32 twice)
        if (hres) hres[row0 + t] = hres[row0 + t] + (acc + ys[row0 + t]);
    }
}

static int check_decode_shapes(int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k) {
    if (dim <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0) return WS_ERR_INVALID_ARG;
    if (dim % 128 || inter % 128 || top_k > kMaxTopkDec) return WS_ERR_SHAPE;
    // LDS holds the token and the picks as bf16 (2 bytes per value)
    // the gate/up kernel holds a wave's share of the token in registers
    if (dim > kMaxDimFp8 || top_k * inter > kMaxPickBytes || n_experts > (1 << 20)) return WS_ERR_SHAPE;
    return WS_OK;
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace ws

using namespace ws;

namespace ws {

static int glu_launch(const uint8_t *xq, const uint8_t *xs, const float *xf, const PickSrc &ps,
                      const RouteArgs *ra, const uint8_t *w1, const uint8_t *s1,
                      const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs, float *hf,
                      int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                      float swiglu_limit, hipStream_t stream) {
    // two tiles per workgroup when that still gives every CU a workgroup:
    // one resident round of 8-wave workgroups, each wave streaming whole K rows
    const int tpw = (inter / 32) * top_k >= 512 ? 2 : 1;
    dim3 grid((unsigned)(inter / 32 / tpw), (unsigned)top_k);
    const bool exact = math_mode() == WS_MATH_EXACT;
    size_t lds = exact ? (size_t)dim * 2 : (size_t)dim + dim / 32;
    const RouteArgs none{};
#define WS_GLU(EX, XF, CPL, RA, HF)                                                              \
    hipLaunchKernelGGL((expert_glu_quant_kernel<EX, XF, CPL, HF>), grid, dim3(kDecThreads), lds,  \
                       stream, xq, xs, xf, ps, RA, w1, s1, w3, s3, hq, hs, hf, (int)dim,          \
                       (int)inter, (int)n_experts, (int)top_k, swiglu_limit, tpw)
    if (ra) {  // routed in the kernel (f32 token)
        const int cpl = n_experts <= 128 ? 2 : n_experts <= 256 ? 4 : n_experts <= 384 ? 6
                      : n_experts <= 512 ? 8 : 16;
#define WS_GLU_R(EX)                                                  \
        switch (cpl) {                                                \
            case 2: WS_GLU(EX, true, 2, *ra, false); break;           \
            case 4: WS_GLU(EX, true, 4, *ra, false); break;           \
            case 6: WS_GLU(EX, true, 6, *ra, false); break;           \
            case 8: WS_GLU(EX, true, 8, *ra, false); break;           \
            default: WS_GLU(EX, true, 16, *ra, false); break;         \
        }
        if (exact) { WS_GLU_R(true) } else { WS_GLU_R(false) }
#undef WS_GLU_R
    } else if (hf) {  // expert_glu: e4m3 token in, f32 h out
        if (exact) WS_GLU(true, false, 0, none, true); else WS_GLU(false, false, 0, none, true);
    } else if (exact) {
        if (xf) WS_GLU(true, true, 0, none, false); else WS_GLU(true, false, 0, none, false);
    } else {
        if (xf) WS_GLU(false, true, 0, none, false); else WS_GLU(false, false, 0, none, false);
    }
#undef WS_GLU
    return launch_status();
}

static int reduce_launch(const uint8_t *hq, const uint8_t *hs, const ReducePicks &pk,
                         const uint8_t *w2, const uint8_t *s2, float *y, int64_t dim,
                         int64_t inter, int64_t n_experts, int64_t top_k, hipStream_t stream,
                         float *hres = nullptr, const float *ys = nullptr) {
    const bool exact = math_mode() == WS_MATH_EXACT;
    size_t lds = exact ? (size_t)top_k * inter * 2
                       : (size_t)top_k * inter + (size_t)top_k * (inter / 32);
    dim3 grid((unsigned)(dim / 16));
    if (exact)
        hipLaunchKernelGGL(expert_reduce_kernel<true>, grid, dim3(kRedThreads), lds, stream, hq,
                           hs, pk, w2, s2, y, (int)dim, (int)inter, (int)n_experts, (int)top_k,
                           hres, ys);
    else
        hipLaunchKernelGGL(expert_reduce_kernel<false>, grid, dim3(kRedThreads), lds, stream, hq,
                           hs, pk, w2, s2, y, (int)dim, (int)inter, (int)n_experts, (int)top_k,
                           hres, ys);
    return launch_status();
}

// moe_local_slots (moe_grouped.cu:23-58): one wave; lane s < top_k holds gate
// slot s; the picks in [e_start, e_start + e_len) are ranked by (expert id,
// slot), the order of the reference's stable insertion sort.
__global__ __launch_bounds__(64) void local_slots_kernel(const int32_t *gate_idx,
                                                         int32_t *local_slots,
                                                         int32_t *local_experts,
                                                         int32_t *local_count, int top_k,
                                                         int e_start, int e_len) {
    const int lane = threadIdx.x;
    const int e = lane < top_k ? gate_idx[lane] : 0;
    const bool in = lane < top_k && e >= e_start && e - e_start < e_len;
    int rank = 0;
    for (int i = 0; i < top_k; i++) {
        const int ei = __builtin_amdgcn_readlane(e, i);
        const bool vi = ei >= e_start && ei - e_start < e_len;
        rank += (vi && (ei < e || (ei == e && i < lane))) ? 1 : 0;
    }
    if (in) {
        local_slots[rank] = lane;
        local_experts[rank] = e - e_start;
    }
    const int n = __popcll(__ballot(in));
    if (lane == 0) *local_count = n;
}

// moe_dispatch_ids (moe_grouped.cu:226-236): local expert row or -1, int64
__global__ __launch_bounds__(64) void dispatch_ids_kernel(const int32_t *gate_idx,
                                                          int64_t *dispatch_idx, int top_k,
                                                          int e_start, int e_len) {
    const int s = blockIdx.x * 64 + threadIdx.x;
    if (s >= top_k) return;
    const int e = gate_idx[s];
    dispatch_idx[s] = (e >= e_start && e - e_start < e_len) ? (int64_t)(e - e_start) : -1;
}

// expert_quant (moe_grouped.cu:128-162): the FP8 1x32 emit of each local
// slot's h row; one 32-lane group per 1x32 block.
__global__ __launch_bounds__(256) void expert_quant_kernel(const float *h, const int32_t *local,
                                                           const int32_t *local_count,
                                                           uint8_t *q, uint8_t *sc, int n,
                                                           int top_k) {
    const int i = blockIdx.y;
    if (i >= min(*local_count, top_k)) return;
    const int slot = local[i];
    if (slot < 0 || slot >= top_k) return;
    const int c = blockIdx.x * 256 + threadIdx.x;
    const bool live = c < n;
    const size_t at = (size_t)slot * n + min(c, n - 1);
    uint32_t sb;
    const uint32_t qb = quant_fp8_block32(h[at], &sb);
    if (live) {
        q[at] = (uint8_t)qb;
        if ((c & 31) == 0) sc[at / 32] = (uint8_t)sb;
    }
}

}  // namespace ws

extern "C" {

int ws_moe_local_slots(const int32_t *gate_idx, int32_t *local_slots, int32_t *local_experts,
                       int32_t *local_count, int64_t top_k, int64_t e_start, int64_t e_len,
                       ws_stream_t stream) {
    if (!gate_idx || !local_slots || !local_experts || !local_count) return WS_ERR_INVALID_ARG;
    if (top_k <= 0 || e_start < 0 || e_len <= 0) return WS_ERR_INVALID_ARG;
    if (top_k > kMaxTopkDec || e_start + e_len > (1 << 30)) return WS_ERR_SHAPE;
    hipLaunchKernelGGL(local_slots_kernel, dim3(1), dim3(64), 0, stream, gate_idx, local_slots,
                       local_experts, local_count, (int)top_k, (int)e_start, (int)e_len);
    return launch_status();
}

int ws_moe_dispatch_ids(const int32_t *gate_idx, int64_t *dispatch_idx, int64_t top_k,
                        int64_t e_start, int64_t e_len, ws_stream_t stream) {
    if (!gate_idx || !dispatch_idx || top_k <= 0 || e_start < 0 || e_len <= 0)
        return WS_ERR_INVALID_ARG;
    if (top_k > (1 << 24) || e_start + e_len > (1 << 30)) return WS_ERR_SHAPE;
    hipLaunchKernelGGL(dispatch_ids_kernel, dim3((unsigned)((top_k + 63) / 64)), dim3(64), 0,
                       stream, gate_idx, dispatch_idx, (int)top_k, (int)e_start, (int)e_len);
    return launch_status();
}

int ws_expert_glu(const uint8_t *act_x, const uint8_t *act_x_s, const uint8_t *w1,
                  const uint8_t *w1_s, const uint8_t *w3, const uint8_t *w3_s,
                  const float *route_w, const int32_t *local_slots,
                  const int32_t *local_experts, const int32_t *local_count, float *h_slots,
                  int64_t n, int64_t k, int64_t top_k, int64_t e_len, ws_stream_t stream) {
    if (!act_x || !act_x_s || !w1 || !w1_s || !w3 || !w3_s || !route_w || !local_slots ||
        !local_experts || !local_count || !h_slots)
        return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(k, n, e_len, top_k);
    if (rc) return rc;
    if (!aligned16(act_x) || !aligned16(w1) || !aligned16(w3) || ((uintptr_t)w1_s & 7) ||
        ((uintptr_t)w3_s & 7) || ((uintptr_t)h_slots & 3))
        return WS_ERR_INVALID_ARG;
    const PickSrc ps{nullptr, route_w, local_slots, local_experts, local_count};
    return glu_launch(act_x, act_x_s, nullptr, ps, nullptr, w1, w1_s, w3, w3_s, nullptr, nullptr,
                      h_slots, k, n, e_len, top_k, 10.0f, stream);
}

int ws_expert_quant(const float *h_slots, const int32_t *local_slots, const int32_t *local_count,
                    uint8_t *q_slots, uint8_t *s_slots, int64_t n, int64_t top_k,
                    ws_stream_t stream) {
    if (!h_slots || !local_slots || !local_count || !q_slots || !s_slots)
        return WS_ERR_INVALID_ARG;
    if (n <= 0 || top_k <= 0) return WS_ERR_INVALID_ARG;
    if (n % 32 || top_k > kMaxTopkDec || n > (1 << 24)) return WS_ERR_SHAPE;
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)top_k);
    hipLaunchKernelGGL(expert_quant_kernel, grid, dim3(256), 0, stream, h_slots, local_slots,
                       local_count, q_slots, s_slots, (int)n, (int)top_k);
    return launch_status();
}

int ws_expert_glu_quant(const uint8_t *xq, const uint8_t *xs, const int32_t *topk_idx,
                        const float *topk_w, const uint8_t *w1, const uint8_t *s1,
                        const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                        int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                        float swiglu_limit, ws_stream_t stream) {
    if (!xq || !xs || !topk_idx || !topk_w || !w1 || !s1 || !w3 || !s3 || !hq || !hs)
        return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (!aligned16(xq) || !aligned16(w1) || !aligned16(w3) || ((uintptr_t)s1 & 7) ||
        ((uintptr_t)s3 & 7))
        return WS_ERR_INVALID_ARG;
    const PickSrc ps{topk_idx, topk_w, nullptr, nullptr, nullptr};
    return glu_launch(xq, xs, nullptr, ps, nullptr, w1, s1, w3, s3, hq, hs, nullptr, dim, inter,
                      n_experts, top_k, swiglu_limit, stream);
}

int ws_expert_glu_quant_x(const float *x, const int32_t *topk_idx, const float *topk_w,
                          const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                          const uint8_t *s3, uint8_t *hq, uint8_t *hs, int64_t dim, int64_t inter,
                          int64_t n_experts, int64_t top_k, float swiglu_limit,
                          ws_stream_t stream) {
    if (!x || !topk_idx || !topk_w || !w1 || !s1 || !w3 || !s3 || !hq || !hs)
        return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (dim > kMaxDimF32) return WS_ERR_SHAPE;
    if (((uintptr_t)x & 15) || !aligned16(w1) || !aligned16(w3) || ((uintptr_t)s1 & 7) ||
        ((uintptr_t)s3 & 7))
        return WS_ERR_INVALID_ARG;
    const PickSrc ps{topk_idx, topk_w, nullptr, nullptr, nullptr};
    return glu_launch(nullptr, nullptr, x, ps, nullptr, w1, s1, w3, s3, hq, hs, nullptr, dim,
                      inter, n_experts, top_k, swiglu_limit, stream);
}

int ws_expert_glu_quant_route(const float *logits, const float *bias, int score_func,
                              float gate_temp, int norm_topk_prob, float route_scale,
                              const float *x, const uint8_t *w1, const uint8_t *s1,
                              const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                              int32_t *topk_idx, float *topk_w, int64_t dim, int64_t inter,
                              int64_t n_experts, int64_t top_k, float swiglu_limit,
                              ws_stream_t stream) {
    if (!logits || !bias || !x || !w1 || !s1 || !w3 || !s3 || !hq || !hs || !topk_idx || !topk_w)
        return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExperts || top_k > kMaxTopk || top_k > n_experts) return WS_ERR_SHAPE;
    if (score_func != WS_SCORE_SIGMOID && score_func != WS_SCORE_SQRTSOFTPLUS)
        return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (dim > kMaxDimF32) return WS_ERR_SHAPE;
    if (((uintptr_t)x & 15) || !aligned16(w1) || !aligned16(w3) || ((uintptr_t)s1 & 7) ||
        ((uintptr_t)s3 & 7))
        return WS_ERR_INVALID_ARG;
    const RouteArgs ra{logits, bias, score_func, gate_temp, norm_topk_prob, route_scale,
                       topk_idx, topk_w};
    return glu_launch(nullptr, nullptr, x, PickSrc{}, &ra, w1, s1, w3, s3, hq, hs, nullptr, dim,
                      inter, n_experts, top_k, swiglu_limit, stream);
}

int ws_expert_reduce(const uint8_t *act_slots, const uint8_t *act_s_slots, const uint8_t *w2,
                     const uint8_t *w2_s, const int32_t *gate_idx, const int32_t *local_slots,
                     const int32_t *local_count, float *y, int64_t dim, int64_t inter,
                     int64_t top_k, int64_t e_start, int64_t e_len, ws_stream_t stream) {
    if (!act_slots || !act_s_slots || !w2 || !w2_s || !gate_idx || !local_slots || !local_count ||
        !y)
        return WS_ERR_INVALID_ARG;
    if (e_start < 0) return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, e_len, top_k);
    if (rc) return rc;
    if (!aligned16(act_slots) || !aligned16(w2) || ((uintptr_t)w2_s & 7))
        return WS_ERR_INVALID_ARG;
    const ReducePicks pk{gate_idx, local_slots, local_count, (int)e_start};
    return reduce_launch(act_slots, act_s_slots, pk, w2, w2_s, y, dim, inter, e_len, top_k,
                         stream);
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t ws_moe_decode_workspace_size(int64_t dim, int64_t inter, int64_t top_k) {
    if (dim <= 0 || inter <= 0 || top_k <= 0) return 0;
    // hq, hs; for dim > kMaxDimF32 also the e4m3 token and its scales
    size_t n = align256(top_k * inter) + align256(top_k * (inter / 32));
    if (dim > kMaxDimF32) n += align256(dim) + align256(dim / 32);
    return n;
}

int ws_moe_decode(const float *x, const int32_t *topk_idx, const float *topk_w, const uint8_t *w1,
                  const uint8_t *s1, const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                  const uint8_t *s2, float *y, int64_t dim, int64_t inter, int64_t n_experts,
                  int64_t top_k, float swiglu_limit, void *workspace, size_t workspace_bytes,
                  ws_stream_t stream) {
    if (!x || !workspace) return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (workspace_bytes < ws_moe_decode_workspace_size(dim, inter, top_k) || !aligned16(workspace))
        return WS_ERR_INVALID_ARG;
    if (((uintptr_t)x & 15) || !aligned16(w1) || !aligned16(w3) || !aligned16(w2) ||
        ((uintptr_t)s1 & 7) || ((uintptr_t)s3 & 7) || ((uintptr_t)s2 & 7) || !topk_idx ||
        !topk_w || !w1 || !s1 || !w3 || !s3 || !w2 || !s2 || !y)
        return WS_ERR_INVALID_ARG;
    uint8_t *hq = (uint8_t *)workspace;
    uint8_t *hs = hq + align256(top_k * inter);
    if (dim <= kMaxDimF32) {
        // the gate/up kernel quantises x itself (the act_quant_fp8_emit rule)
        rc = glu_launch(nullptr, nullptr, x, PickSrc{topk_idx, topk_w, nullptr, nullptr, nullptr},
                        nullptr, w1, s1, w3, s3, hq, hs, nullptr, dim, inter, n_experts, top_k,
                        swiglu_limit, stream);
    } else {
        uint8_t *xq = hs + align256(top_k * (inter / 32));
        uint8_t *xs = xq + align256(dim);
        rc = ws_emit8(x, xq, xs, dim, stream);
        if (rc) return rc;
        rc = glu_launch(xq, xs, nullptr, PickSrc{topk_idx, topk_w, nullptr, nullptr, nullptr},
                        nullptr, w1, s1, w3, s3, hq, hs, nullptr, dim, inter, n_experts, top_k,
                        swiglu_limit, stream);
    }
    if (rc) return rc;
    return reduce_launch(hq, hs, ReducePicks{topk_idx, nullptr, nullptr, 0}, w2, s2, y, dim, inter,
                         n_experts, top_k, stream);
}

// ---- allocation-free decode step -------------------------------------------
// Device scratch of ws_moe_decode_route_noalloc: the picks' hidden states
// (hq, hs) and, for dim > 8192, the quantised token, laid out as the
// ws_moe_decode workspace. Its largest use under check_decode_shapes is
// 32768 + 1024 + 16384 + 512 bytes.
constexpr size_t kDecodeScratchBytes = 64 << 10;
static __device__ __align__(256) uint8_t scratch[kDecodeScratchBytes];

// The device address of this device's copy of `scratch`, looked up once per
// device with that device current (the array's name in host code is only a
// host-side handle, not a device address). nullptr if the lookup fails.
static uint8_t *decode_scratch() {
    static std::mutex mu;
    static uint8_t *ptrs[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        ptrs[dev] = (uint8_t *)p;
    }
    return ptrs[dev];
}

int ws_moe_decode_route_noalloc(const float *logits, const float *bias, int score_func,
                                float gate_temp, int norm_topk_prob, float route_scale,
                                const float *x, const uint8_t *w1, const uint8_t *s1,
                                const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                                const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                                int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                                float swiglu_limit, ws_stream_t stream) {
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    const size_t need = ws_moe_decode_workspace_size(dim, inter, top_k);
    if (need == 0) return WS_ERR_INVALID_ARG;
    if (need > kDecodeScratchBytes) return WS_ERR_SHAPE;
    uint8_t *ws = decode_scratch();
    if (!ws) return WS_ERR_NO_DEVICE;
    // every byte of the scratch that a kernel reads was written by an earlier
    // kernel of the same call (hq / hs of the valid picks, the quantised
    // token): nothing has to start at zero
    return ws_moe_decode_route(logits, bias, score_func, gate_temp, norm_topk_prob, route_scale, x,
                               w1, s1, w3, s3, w2, s2, y, topk_idx, topk_w, dim, inter, n_experts,
                               top_k, swiglu_limit, ws, kDecodeScratchBytes, stream);
}

int ws_moe_decode_route(const float *logits, const float *bias, int score_func, float gate_temp,
                        int norm_topk_prob, float route_scale, const float *x, const uint8_t *w1,
                        const uint8_t *s1, const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                        const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                        int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                        float swiglu_limit, void *workspace, size_t workspace_bytes,
                        ws_stream_t stream) {
    if (!logits || !bias || !topk_idx || !topk_w) return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExperts || top_k > kMaxTopk || top_k > n_experts) return WS_ERR_SHAPE;
    if (score_func < WS_SCORE_SOFTMAX || score_func > WS_SCORE_SQRTSOFTPLUS) return WS_ERR_INVALID_ARG;
    if (score_func == WS_SCORE_SOFTMAX || dim > kMaxDimF32) {
        // the sequential softmax sum, or a token too wide for the fused
        // quantisation: route first, then the two expert kernels
        int rc = ws_moe_topk(logits, bias, nullptr, topk_idx, topk_w, 1, n_experts, top_k,
                             score_func, gate_temp, norm_topk_prob, route_scale, stream);
        if (rc) return rc;
        return ws_moe_decode(x, topk_idx, topk_w, w1, s1, w3, s3, w2, s2, y, dim, inter, n_experts,
                             top_k, swiglu_limit, workspace, workspace_bytes, stream);
    }
    if (!x || !workspace) return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (workspace_bytes < ws_moe_decode_workspace_size(dim, inter, top_k) || !aligned16(workspace))
        return WS_ERR_INVALID_ARG;
    if (((uintptr_t)x & 15) || !aligned16(w1) || !aligned16(w3) || !aligned16(w2) ||
        ((uintptr_t)s1 & 7) || ((uintptr_t)s3 & 7) || ((uintptr_t)s2 & 7) || !w1 || !s1 || !w3 ||
        !s3 || !w2 || !s2 || !y)
        return WS_ERR_INVALID_ARG;
    uint8_t *hq = (uint8_t *)workspace;
    uint8_t *hs = hq + align256(top_k * inter);
    const RouteArgs ra{logits, bias, score_func, gate_temp, norm_topk_prob, route_scale,
                       topk_idx, topk_w};
    rc = glu_launch(nullptr, nullptr, x, PickSrc{}, &ra, w1, s1, w3, s3, hq, hs, nullptr, dim,
                    inter, n_experts, top_k, swiglu_limit, stream);
    if (rc) return rc;
    return reduce_launch(hq, hs, ReducePicks{topk_idx, nullptr, nullptr, 0}, w2, s2, y, dim, inter,
                         n_experts, top_k, stream);
}

int ws_moe_decode_route_shared(const float *logits, const float *bias, int score_func,
                               float gate_temp, int norm_topk_prob, float route_scale,
                               const float *x, const uint8_t *w1, const uint8_t *s1,
                               const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                               const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                               int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                               float swiglu_limit, const float *hs_shared, const uint8_t *w2_shared,
                               const uint8_t *s2_shared, int64_t shared_inter, float *ys,
                               float *h, void *workspace, size_t workspace_bytes,
                               ws_stream_t stream) {
    if (!hs_shared || !w2_shared || !s2_shared || !ys || !h) return WS_ERR_INVALID_ARG;
    if (shared_inter <= 0 || shared_inter % 128) return WS_ERR_SHAPE;
    if (((uintptr_t)hs_shared | (uintptr_t)w2_shared | (uintptr_t)ys | (uintptr_t)h) & 15 ||
        ((uintptr_t)s2_shared & 3))
        return WS_ERR_INVALID_ARG;
    const bool fused_path = logits && bias && score_func != WS_SCORE_SOFTMAX &&
                            score_func >= WS_SCORE_SOFTMAX && score_func <= WS_SCORE_SQRTSOFTPLUS &&
                            dim <= kMaxDimF32 && shared_inter <= 8192 && n_experts <= kMaxExperts &&
                            top_k <= kMaxTopk && top_k <= n_experts;
    if (!fused_path) {
        // the same results through the separate launches
        int rc = ws_moe_decode_route(logits, bias, score_func, gate_temp, norm_topk_prob,
                                     route_scale, x, w1, s1, w3, s3, w2, s2, y, topk_idx, topk_w,
                                     dim, inter, n_experts, top_k, swiglu_limit, workspace,
                                     workspace_bytes, stream);
        if (rc) return rc;
        return ws_shared_expert_down_acc(hs_shared, w2_shared, s2_shared, y, h, 1, dim,
                                         shared_inter, stream);
    }
    if (!x || !workspace || !topk_idx || !topk_w) return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (dim % 16) return WS_ERR_SHAPE;
    if (workspace_bytes < ws_moe_decode_workspace_size(dim, inter, top_k) || !aligned16(workspace))
        return WS_ERR_INVALID_ARG;
    if (((uintptr_t)x & 15) || !aligned16(w1) || !aligned16(w3) || !aligned16(w2) ||
        ((uintptr_t)s1 & 7) || ((uintptr_t)s3 & 7) || ((uintptr_t)s2 & 7) || !w1 || !s1 || !w3 ||
        !s3 || !w2 || !s2 || !y)
        return WS_ERR_INVALID_ARG;
    uint8_t *hq = (uint8_t *)workspace;
    uint8_t *hs = hq + align256(top_k * inter);
    const RouteArgs ra{logits, bias, score_func, gate_temp, norm_topk_prob, route_scale,
                       topk_idx, topk_w};
    const SharedDown sd{hs_shared, w2_shared, s2_shared, ys, (int)dim, (int)shared_inter};
    // the routed grid of glu_launch, plus rows of workgroups for the shared
    // down GEMV (one per 16 output columns)
    const int tpw = (inter / 32) * top_k >= 512 ? 2 : 1;
    const int gx = (int)(inter / 32 / tpw);
    const int kp_rows = (int)((dim / 16 + gx - 1) / gx);
    dim3 grid((unsigned)gx, (unsigned)(top_k + kp_rows));
    const bool exact = math_mode() == WS_MATH_EXACT;
    const size_t glu_lds = exact ? (size_t)dim * 2 : (size_t)dim + dim / 32;
    const size_t kp_lds = (size_t)8 * 16 * 16 * 4 + (size_t)(shared_inter + 16) +
                          (size_t)(shared_inter / 32);
    const size_t lds = glu_lds > kp_lds ? glu_lds : kp_lds;
    const int cpl = n_experts <= 128 ? 2 : n_experts <= 256 ? 4 : n_experts <= 384 ? 6
                  : n_experts <= 512 ? 8 : 16;
#define WS_GSD(EX, CPL)                                                                         \
    hipLaunchKernelGGL((glu_shared_down_kernel<EX, CPL>), grid, dim3(kDecThreads), lds, stream, x, \
                       ra, w1, s1, w3, s3, hq, hs, (int)dim, (int)inter, (int)n_experts,          \
                       (int)top_k, swiglu_limit, tpw, sd)
#define WS_GSD_R(EX)                          \
    switch (cpl) {                            \
        case 2: WS_GSD(EX, 2); break;         \
        case 4: WS_GSD(EX, 4); break;         \
        case 6: WS_GSD(EX, 6); break;         \
        case 8: WS_GSD(EX, 8); break;         \
        default: WS_GSD(EX, 16); break;       \
    }
    if (exact) { WS_GSD_R(true) } else { WS_GSD_R(false) }
#undef WS_GSD_R
#undef WS_GSD
    rc = launch_status();
    if (rc) return rc;
    return reduce_launch(hq, hs, ReducePicks{topk_idx, nullptr, nullptr, 0}, w2, s2, y, dim, inter,
                         n_experts, top_k, stream, h, ys);
}

}  // extern "C"
