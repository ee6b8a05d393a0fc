// Wave-level MoE routing shared by the routing kernels and the fused decode
// kernel: scores (weightstream-ref num.rs:71-88 on the exact expf) and the
// top-k selection with routing weights (moe.rs:47-66), all in registers.
#pragma once

#include "ws_device.hpp"

namespace ws {

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 16;

__device__ __forceinline__ float score_fn(float v, int score_func, float gate_temp) {
    if (gate_temp != 1.0f) v = v / gate_temp;
    if (score_func == WS_SCORE_SIGMOID) return ws_sigmoid(v);
    if (score_func == WS_SCORE_SQRTSOFTPLUS) {
        return sqrtf(ws_softplus(v));
    }
    return v;  // softmax handled by the caller, identity for given scores
}

// f32 total order (Rust f32::total_cmp) as an unsigned key: larger = greater.
__device__ __forceinline__ uint32_t total_key_u(float v) {
    int32_t b = (int32_t)__float_as_uint(v);
    int32_t k = b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return (uint32_t)k ^ 0x80000000u;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint64_t o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Wave max with DPP lane moves (no LDS permutes): quad swaps, half-row and
// row mirrors, then row broadcasts 15 and 31 carry the maximum to lane 63.
#define WS_DPP_MAX(v, ctrl, rmask)                                                           \
    do {                                                                                    \
        uint32_t o_ = (uint32_t)__builtin_amdgcn_update_dpp((int)(v), (int)(v), ctrl, rmask, \
                                                            0xf, false);                    \
        v = o_ > v ? o_ : v;                                                                \
    } while (0)

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    WS_DPP_MAX(v, 0xB1, 0xf);   // quad_perm [1,0,3,2]
    WS_DPP_MAX(v, 0x4E, 0xf);   // quad_perm [2,3,0,1]
    WS_DPP_MAX(v, 0x141, 0xf);  // row_half_mirror
    WS_DPP_MAX(v, 0x140, 0xf);  // row_mirror
    WS_DPP_MAX(v, 0x142, 0xa);  // row_bcast:15 -> rows 1, 3
    WS_DPP_MAX(v, 0x143, 0xc);  // row_bcast:31 -> rows 2, 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
#undef WS_DPP_MAX

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The routing inputs of experts lane + 64 c (c < CPL): logits and bias,
// loaded together so that their latencies overlap.
template <int CPL>
struct RouteIn {
    float v[CPL], b[CPL];
};

template <int CPL>
__device__ __forceinline__ void route_load(RouteIn<CPL> &in, const float *lg, const float *bias,
                                           int n_experts, int lane) {
#pragma unroll
    for (int c = 0; c < CPL; c++) in.v[c] = lg[min(lane + 64 * c, n_experts - 1)];
#pragma unroll
    for (int c = 0; c < CPL; c++) in.b[c] = bias[min(lane + 64 * c, n_experts - 1)];
}

// Scores of experts lane + 64 c (c < CPL) from their logits: sigmoid,
// sqrtsoftplus or identity (softmax needs the whole row; not handled here),
// after dividing by gate_temp. The exp table sits in lane registers.
template <int CPL>
__device__ __forceinline__ void wave_scores_of(const float lg[CPL], int score_func,
                                               float gate_temp, int lane, float sc[CPL]) {
    float v[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) v[c] = lg[c];
    const uint64_t tab = ws_lane_exp2f_tab(lane);
    if (gate_temp != 1.0f) {
#pragma unroll
        for (int c = 0; c < CPL; c++) v[c] = v[c] / gate_temp;
    }
    if (score_func == WS_SCORE_SIGMOID) {
#pragma unroll
        for (int c = 0; c < CPL; c++) sc[c] = ws_sigmoid_lanes(v[c], tab);
    } else if (score_func == WS_SCORE_SQRTSOFTPLUS) {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const float ex = ws_expf_lanes(v[c], tab);
            sc[c] = sqrtf(v[c] > 20.0f ? v[c] : ws_logf(1.0f + ex));
        }
    } else {
#pragma unroll
        for (int c = 0; c < CPL; c++) sc[c] = v[c];
    }
}

// ... from logits lg[E]
template <int CPL>
__device__ __forceinline__ void wave_scores(const float *lg, int n_experts, int score_func,
                                            float gate_temp, int lane, float sc[CPL]) {
    float v[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) v[c] = lg[min(lane + 64 * c, n_experts - 1)];
    wave_scores_of<CPL>(v, score_func, gate_temp, lane, sc);
}

// Top-k of score + bias (f32 total order, ties to the lower index) over
// experts lane + 64 c; lane k < top_k gets pick k and its weight: the score,
// normalised by the top-k-order sum + 1e-20 (norm 1: moe.rs:61, only when
// top_k > 1; norm 2: moe_select's unconditional normalisation, moe.cu:84-88),
// times route_scale. Each lane keeps CPL 64-bit keys (score+bias key, then
// the complemented index), sorted once in descending order, so a lane's
// largest remaining key is its first; a round is a 32-bit DPP wave max of
// the lanes' first score halves and a ballot (only an exact score tie across
// lanes takes the 64-bit wave max), and the winning lane shifts its keys.
// bv[c]: the bias of expert lane + 64 c.
template <int CPL>
struct WaveTopk {
    uint64_t cand[CPL];
    float sc[CPL];
    int pick;  // lane k: pick k, once round k has run
    float ws;  // lane k: its score

    __device__ __forceinline__ void init(const float s[CPL], const float bv[CPL], int n_experts,
                                         int lane) {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int e = lane + 64 * c;
            cand[c] = e < n_experts
                          ? ((uint64_t)total_key_u(s[c] + bv[c]) << 32) | (uint32_t)(~(uint32_t)e)
                          : 0ull;
            sc[c] = s[c];
        }
        // odd-even transposition sort, descending (keys are distinct)
#pragma unroll
        for (int p = 0; p < CPL; p++)
#pragma unroll
            for (int c = p & 1; c + 1 < CPL; c += 2) {
                const bool sw = cand[c + 1] > cand[c];
                const uint64_t a = cand[c], b = cand[c + 1];
                const float x = sc[c], y = sc[c + 1];
                cand[c] = sw ? b : a;
                cand[c + 1] = sw ? a : b;
                sc[c] = sw ? y : x;
                sc[c + 1] = sw ? x : y;
            }
        pick = 0;
        ws = 0.0f;
    }

    // round k: the largest remaining key; returns its expert id (uniform)
    __device__ __forceinline__ int round(int k, int lane) {
        // the lane's largest remaining key is its first (keys are distinct:
        // the low half is the complemented expert id)
        const uint64_t best = cand[0];
        const float sb = sc[0];
        const uint32_t hk = (uint32_t)(best >> 32);
        const uint32_t wk = wave_max_u32(hk);
        uint64_t bal = __ballot(hk == wk);
        if (__popcll(bal) > 1) {
            // equal scores on several lanes: the larger full key (lower index)
            const uint64_t full = wave_max_u64(hk == wk ? best : 0ull);
            bal = __ballot(hk == wk && best == full);
        }
        const int win = __ffsll((long long)bal) - 1;
        const int e = (int)~(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)best, win);
        const float w = readlane_f(sb, win);
        if (lane == k) {
            pick = e;
            ws = w;
        }
        // the winning lane drops its first key (constant indices only: a
        // select between array elements by a run-time index would become an
        // indexed load of a private-memory copy of the array)
        const bool drop = lane == win;
#pragma unroll
        for (int c = 0; c + 1 < CPL; c++) {
            cand[c] = drop ? cand[c + 1] : cand[c];
            sc[c] = drop ? sc[c + 1] : sc[c];
        }
        cand[CPL - 1] = drop ? 0ull : cand[CPL - 1];
        return e;
    }

    // lane k's weight after all top_k rounds
    __device__ __forceinline__ float weight(int top_k, int norm, float route_scale) const {
        float wout = ws;
        if ((norm == 1 && top_k > 1) || norm == 2) {
            float s = -0.0f;
            for (int k = 0; k < top_k; k++) s = s + readlane_f(ws, k);
            wout = ws / (s + 1e-20f);
        }
        return wout * route_scale;
    }
};

template <int CPL>
__device__ __forceinline__ void wave_select_of(const float sc[CPL], const float bv[CPL],
                                               int n_experts, int top_k, int norm,
                                               float route_scale, int lane, int &my_pick,
                                               float &my_w) {
    WaveTopk<CPL> tk;
    tk.init(sc, bv, n_experts, lane);
    for (int k = 0; k < top_k; k++) tk.round(k, lane);
    my_pick = tk.pick;
    my_w = tk.weight(top_k, norm, route_scale);
}

template <int CPL>
__device__ __forceinline__ void wave_select(const float sc[CPL], const float *bias, int n_experts,
                                            int top_k, int norm, float route_scale, int lane,
                                            int &my_pick, float &my_w) {
    float bv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) bv[c] = bias[min(lane + 64 * c, n_experts - 1)];
    wave_select_of<CPL>(sc, bv, n_experts, top_k, norm, route_scale, lane, my_pick, my_w);
}

}  // namespace ws
