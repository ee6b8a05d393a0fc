// MoE routing: gate logits, score function, top-k and routing weights.
//
// Reference GPU kernels: weightstream-cuda/kernels/moe.cu (moe_gate :18,
// moe_select :48, moe_route :100, moe_gate_m :160), launched by
// launch.rs:998-1093. CPU semantics (the parity target): weightstream-ref
// moe.rs:20-69 and num.rs:8-88.
//
// Bit-exactness with the CPU path:
//  - gate logits follow num::gemv: one sequential f32 dot per (token, expert);
//    a lane owns one expert and walks d = 0..dim-1 in order, multiply then add
//    (compiled without contraction);
//  - sigmoid / softmax use ws_expf, equal to glibc expf on every input;
//  - top-k orders by f32 total order of score+bias, ties to the lower index
//    (moe.rs:50 `total_cmp(..).then(a.cmp(&b))`);
//  - the weight normaliser is the sequential sum in top-k order plus 1e-20
//    (moe.rs:61-66), then * route_scale.
// sqrtsoftplus uses ws_logf and sqrtf: ws_logf equals glibc logf on every
// input (ws_logf.h), sqrtf is correctly rounded, so the scores are the CPU's
// bits.
#include <type_traits>
#include <utility>

#include "ws_internal.hpp"
#include "ws_route.hpp"
#include "ws_gate.hpp"

namespace ws {

constexpr int kScoreIdentity = 3;  // scores given (moe_select)

// ---- gate logits ----------------------------------------------------------
// grid (ceil(E/64), M), 64 threads: lane = expert. Each lane streams its own
// weight row with 16-byte loads (consecutive iterations reuse the cache line).
template <bool BF16>
__global__ __launch_bounds__(64) void gate_logits_kernel(const float *__restrict__ x,
                                                         const void *__restrict__ gw,
                                                         float *__restrict__ logits, int dim,
                                                         int n_experts) {
    int e = blockIdx.x * 64 + threadIdx.x;
    int m = blockIdx.y;
    __shared__ float xs[4096];
    const float *xr = x + (size_t)m * dim;
    float s = 0.0f;
    for (int d0 = 0; d0 < dim; d0 += 4096) {
        int len = min(4096, dim - d0);
        __syncthreads();
        for (int i = threadIdx.x; i < len; i += 64) xs[i] = xr[d0 + i];
        __syncthreads();
        if (e < n_experts) {
            if (BF16) {
                const uint16_t *w = (const uint16_t *)gw + (size_t)e * dim + d0;
                int i = 0;
                for (; i + 8 <= len; i += 8) {
                    uint4 q = *(const uint4 *)(w + i);
                    uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int t = 0; t < 4; t++) {
                        s = s + xs[i + 2 * t] * __uint_as_float(wd[t] << 16);
                        s = s + xs[i + 2 * t + 1] * __uint_as_float(wd[t] & 0xFFFF0000u);
                    }
                }
                for (; i < len; i++) s = s + xs[i] * __uint_as_float((uint32_t)w[i] << 16);
            } else {
                const float *w = (const float *)gw + (size_t)e * dim + d0;
                int i = 0;
                for (; i + 4 <= len; i += 4) {
                    float4 q = *(const float4 *)(w + i);
                    s = s + xs[i] * q.x;
                    s = s + xs[i + 1] * q.y;
                    s = s + xs[i + 2] * q.z;
                    s = s + xs[i + 3] * q.w;
                }
                for (; i < len; i++) s = s + xs[i] * w[i];
            }
        }
    }
    if (e < n_experts) logits[(size_t)m * n_experts + e] = s;
}

// ---- gate logits, pipelined (dim % 256 == 0) --------------------------------
// (kGC, kGS, GateGeom: ws_gate.hpp)
// One wave computes a block of TM tokens x TE experts, one lane per (token,
// expert) chain; every chain is the sequential dot of num::gemv above
// (multiply then add, d = 0..dim-1), so the logits are the same bits. The
// block's token rows and weight rows are streamed through a kGS-stage LDS ring
// of kGC-element chunks by direct global->LDS loads, kGS-1 chunks ahead of the
// chains, which read them back from LDS: the sequential adds never wait on
// global memory. Small blocks (4 experts for one token) spread the weight
// stream over many CUs. Rows of 1 KB (tokens, f32 weights) sit 1040 bytes
// apart in a stage, so rows read at one position fall on distinct banks and
// every read is the row's base plus a constant (no address arithmetic in the
// chains' loop); bf16 weight rows (512 bytes, two per direct load) keep their
// 16-byte pieces permuted by the row index instead.
template <int TE, int TM, bool BF16>
struct PipeGeom {
    using G = GateGeom<TE, TM, BF16>;
    static_assert(G::kXRow == 1024, "one token row chunk per direct load");
    static constexpr int kXP = G::kXRow + 16;                  // token row pitch
    static constexpr int kWP = BF16 ? G::kWRow : G::kWRow + 16;  // weight row pitch
    static constexpr int kXs = TM * kXP;
    static constexpr int kStage = kXs + TE * kWP;
};

template <int OFF>
__device__ __forceinline__ u32x4v lds_read_b128_at(uint32_t a) {
    u32x4v v;
    __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF));
    return v;
}

template <class F, int... I>
__device__ __forceinline__ void unroll_seq(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}

template <int TE, int TM, bool BF16>
__global__ __launch_bounds__(64) void gate_logits_pipe_kernel(const float *x, const void *gw,
                                                              float *__restrict__ logits,
                                                              int m_rows, int dim, int n_experts) {
    using G = GateGeom<TE, TM, BF16>;
    using P = PipeGeom<TE, TM, BF16>;
    extern __shared__ __align__(16) uint8_t g_lds[];
    const int lane = threadIdx.x;
    const int e0 = blockIdx.x * TE, m0 = blockIdx.y * TM;
    const int nc = dim / kGC;
    constexpr int kEB = BF16 ? 2 : 4;

    // a lane's direct-load sources: fixed rows, the chunk offset moves
    // direct load j: token row j, f32 weight row j - TM, or bf16 weight rows
    // 2 (j - TM) and 2 (j - TM) + 1; its LDS offset in the stage is dst(j)
    const uint8_t *src[G::kLoads];
#pragma unroll
    for (int j = 0; j < G::kLoads; j++) {
        const int o = j * 1024 + lane * 16;
        if (o < G::kX) {
            src[j] = (const uint8_t *)(x + (size_t)min(m0 + j, m_rows - 1) * dim) + lane * 16;
        } else {
            const int oo = o - G::kX;
            const int row = oo / G::kWRow, c = (oo % G::kWRow) / 16;
            src[j] = (const uint8_t *)gw + (size_t)min(e0 + row, n_experts - 1) * dim * kEB +
                     (BF16 ? (c ^ (row & 15)) : c) * 16;
        }
    }
    auto dst = [](int j) {
        return j * 1024 < G::kX ? j * P::kXP
                                : P::kXs + (BF16 ? (j * 1024 - G::kX) : (j - TM) * P::kWP);
    };
    auto issue = [&](int buf, int chunk) {
        uint8_t *base = g_lds + buf * P::kStage;
#pragma unroll
        for (int j = 0; j < G::kLoads; j++) {
            const int off = j * 1024 < G::kX ? chunk * G::kXRow : chunk * G::kWRow;
            __builtin_amdgcn_global_load_lds(
                (const void *)(src[j] + off),
                (__attribute__((address_space(3))) void *)(base + dst(j)), 16, 0, 0);
        }
    };

    const int tm = min(lane / TE, TM - 1), te = lane % TE;
    float s = 0.0f;
    // 16 elements at a time (a group): 4 pieces of the token row and 4
    // (f32) or 2 (bf16) of the weight row; the next group's reads are issued
    // before a group's adds, so LDS latency overlaps the chain
    constexpr int kWP = BF16 ? 2 : 4;        // weight pieces per group
    constexpr int kRd = 4 + kWP;             // LDS reads per group
    constexpr int kNG = kGC / 16;            // groups per chunk
    auto reads = [&](auto gc, uint32_t xb, uint32_t wb, u32x4v *xr, u32x4v *wr) {
        constexpr int grp = decltype(gc)::value;
        xr[0] = lds_read_b128_at<(grp * 4 + 0) * 16>(xb);
        xr[1] = lds_read_b128_at<(grp * 4 + 1) * 16>(xb);
        xr[2] = lds_read_b128_at<(grp * 4 + 2) * 16>(xb);
        xr[3] = lds_read_b128_at<(grp * 4 + 3) * 16>(xb);
        if constexpr (BF16) {
#pragma unroll
            for (int k = 0; k < kWP; k++)
                wr[k] = lds_read_b128(wb + ((grp * kWP + k) ^ (te & 15)) * 16);
        } else {
            wr[0] = lds_read_b128_at<(grp * 4 + 0) * 16>(wb);
            wr[1] = lds_read_b128_at<(grp * 4 + 1) * 16>(wb);
            wr[2] = lds_read_b128_at<(grp * 4 + 2) * 16>(wb);
            wr[3] = lds_read_b128_at<(grp * 4 + 3) * 16>(wb);
        }
    };
#pragma unroll
    for (int p = 0; p < kGS - 1; p++)
        if (p < nc) issue(p, p);
    for (int i = 0; i < nc; i++) {
        mem_order();
        wait_newer<G::kLoads, kGS - 2>(min(nc - 1 - i, kGS - 2));
        raw_barrier();  // chunk i is in LDS; chunk i-1's buffer is free
        if (i + kGS - 1 < nc) issue((i + kGS - 1) % kGS, i + kGS - 1);
        const uint32_t xb = lds_addr(g_lds) + (i % kGS) * P::kStage + tm * P::kXP;
        const uint32_t wb = lds_addr(g_lds) + (i % kGS) * P::kStage + P::kXs + te * P::kWP;
        u32x4v xv[2][4], wv[2][4];
        reads(std::integral_constant<int, 0>{}, xb, wb, xv[0], wv[0]);
        unroll_seq([&](auto gc) {
            constexpr int grp = decltype(gc)::value;
            constexpr int cur = grp & 1;
            if constexpr (grp + 1 < kNG) {
                reads(std::integral_constant<int, grp + 1>{}, xb, wb, xv[cur ^ 1], wv[cur ^ 1]);
                lds_wait<kRd>();
            } else {
                lds_wait<0>();
            }
#pragma unroll
            for (int k = 0; k < 4; k++) lds_ready(xv[cur][k]);
#pragma unroll
            for (int k = 0; k < kWP; k++) lds_ready(wv[cur][k]);
            // the 16 products first (independent), then the 16 dependent adds
            float pr[16];
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const float xe = __uint_as_float(xv[cur][j / 4][j % 4]);
                float we;
                if (BF16) {
                    const uint32_t word = wv[cur][j / 8][(j % 8) / 2];
                    we = __uint_as_float((j & 1) ? (word & 0xFFFF0000u) : (word << 16));
                } else {
                    we = __uint_as_float(wv[cur][j / 4][j % 4]);
                }
                pr[j] = xe * we;
            }
#pragma unroll
            for (int j = 0; j < 16; j++) s = s + pr[j];
        }, std::make_integer_sequence<int, kNG>{});
    }
    if (lane < TE * TM && m0 + tm < m_rows && e0 + te < n_experts)
        logits[(size_t)(m0 + tm) * n_experts + e0 + te] = s;
}

template <int TE, int TM>
static void gate_pipe_launch(const float *x, const void *gw, int bf16, float *logits, int64_t m,
                             int64_t dim, int64_t n_experts, hipStream_t stream) {
    dim3 g((unsigned)((n_experts + TE - 1) / TE), (unsigned)((m + TM - 1) / TM));
    if (bf16)
        hipLaunchKernelGGL((gate_logits_pipe_kernel<TE, TM, true>), g, dim3(64),
                           (kGS * PipeGeom<TE, TM, true>::kStage), stream, x, gw, logits, (int)m,
                           (int)dim, (int)n_experts);
    else
        hipLaunchKernelGGL((gate_logits_pipe_kernel<TE, TM, false>), g, dim3(64),
                           (kGS * PipeGeom<TE, TM, false>::kStage), stream, x, gw, logits, (int)m,
                           (int)dim, (int)n_experts);
}

template <int TE, int TM, bool BF16>
__global__ __launch_bounds__(128) void gate_logits_pc_kernel(const float *x, const void *gw,
                                                             float *__restrict__ logits,
                                                             int m_rows, int dim, int n_experts) {
    gate_pc_body<TE, TM, BF16>(blockIdx.x, blockIdx.y, x, gw, logits, m_rows, dim, n_experts);
}

template <int TE, int TM>
static void gate_pc_launch(const float *x, const void *gw, int bf16, float *logits, int64_t m,
                           int64_t dim, int64_t n_experts, hipStream_t stream) {
    dim3 g((unsigned)((n_experts + TE - 1) / TE), (unsigned)((m + TM - 1) / TM));
    const size_t prod = (size_t)2 * TE * TM * kPcPitch * 4;
    if (bf16)
        hipLaunchKernelGGL((gate_logits_pc_kernel<TE, TM, true>), g, dim3(128),
                           (kGS * GateGeom<TE, TM, true>::kStage + prod), stream, x, gw, logits,
                           (int)m, (int)dim, (int)n_experts);
    else
        hipLaunchKernelGGL((gate_logits_pc_kernel<TE, TM, false>), g, dim3(128),
                           (kGS * GateGeom<TE, TM, false>::kStage + prod), stream, x, gw, logits,
                           (int)m, (int)dim, (int)n_experts);
}

// One wave per token row (wave_scores + wave_select of ws_route.hpp); the
// softmax path keeps the reference's sequential sum (one lane, LDS).
template <int CPL>
__global__ __launch_bounds__(64) void topk_kernel(
    const float *__restrict__ logits, const float *__restrict__ bias, float *__restrict__ scores_out,
    int32_t *__restrict__ out_idx, float *__restrict__ out_w, int n_experts, int top_k,
    int score_func, float gate_temp, int norm, float route_scale) {
    __shared__ float sm[kMaxExperts];
    __shared__ float ssum;
    const int m = blockIdx.x;
    const int lane = threadIdx.x;
    const float *lg = logits + (size_t)m * n_experts;

    float sc[CPL];
    if (score_func == WS_SCORE_SOFTMAX) {
        // num.rs:46-62: max, exp(x - max) in place with a sequential sum, divide
        for (int e = lane; e < n_experts; e += 64) sm[e] = score_fn(lg[e], score_func, gate_temp);
        __syncthreads();
        if (lane == 0) {
            float mx = -__builtin_inff();
            for (int e = 0; e < n_experts; e++)
                if (sm[e] > mx) mx = sm[e];
            float s = 0.0f;
            for (int e = 0; e < n_experts; e++) {
                sm[e] = ws_expf(sm[e] - mx);
                s = s + sm[e];
            }
            ssum = s;
        }
        __syncthreads();
        const float s = ssum;
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int e = lane + 64 * c;
            sc[c] = e < n_experts ? sm[e] / s : 0.0f;
        }
    } else {
        wave_scores<CPL>(lg, n_experts, score_func, gate_temp, lane, sc);
    }
    if (scores_out) {
#pragma unroll
        for (int c = 0; c < CPL; c++) {
            const int e = lane + 64 * c;
            if (e < n_experts) scores_out[(size_t)m * n_experts + e] = sc[c];
        }
    }
    int my_pick;
    float my_w;
    wave_select<CPL>(sc, bias, n_experts, top_k, norm, route_scale, lane, my_pick, my_w);
    if (lane < top_k) {
        out_idx[(size_t)m * top_k + lane] = my_pick;
        out_w[(size_t)m * top_k + lane] = my_w;
    }
}

// Fused single-workgroup gate + select for one token (moe.cu:100 moe_route).
__global__ __launch_bounds__(1024) void route_fused_kernel(const float *__restrict__ x,
                                                           const uint16_t *__restrict__ gw,
                                                           const float *__restrict__ bias,
                                                           float *__restrict__ out_w,
                                                           int32_t *__restrict__ out_idx, int dim,
                                                           int n_experts, int top_k,
                                                           float route_scale) {
    __shared__ float sc[kMaxExperts];
    __shared__ int32_t picked[kMaxTopk];
    __shared__ uint64_t wave_best[16];
    const int t = threadIdx.x;
    if (t < n_experts) {
        const uint16_t *w = gw + (size_t)t * dim;
        float s = 0.0f;
        for (int d = 0; d < dim; d++) s = s + x[d] * __uint_as_float((uint32_t)w[d] << 16);
        sc[t] = score_fn(s, WS_SCORE_SQRTSOFTPLUS, 1.0f);
    }
    __syncthreads();
    uint64_t cand = t < n_experts
                        ? ((uint64_t)total_key_u(sc[t] + bias[t]) << 32) | (uint32_t)(~(uint32_t)t)
                        : 0ull;
    const int nw = (blockDim.x + 63) / 64;
    for (int k = 0; k < top_k; k++) {
        uint64_t best = wave_max_u64(cand);
        if ((t & 63) == 0) wave_best[t >> 6] = best;
        __syncthreads();
        best = wave_best[0];
        for (int wv = 1; wv < nw; wv++) best = wave_best[wv] > best ? wave_best[wv] : best;
        int e = (int)(~(uint32_t)best);
        if (t == 0) picked[k] = e;
        if (t == e) cand = 0ull;
        __syncthreads();
    }
    if (t == 0) {
        float w[kMaxTopk];
        float s = 0.0f;
        for (int k = 0; k < top_k; k++) {
            w[k] = sc[picked[k]];
            s = s + w[k];
        }
        for (int k = 0; k < top_k; k++) {
            out_idx[k] = picked[k];
            out_w[k] = w[k] / (s + 1e-20f) * route_scale;
        }
    }
}

// Score-only pass (moe_gate / moe_gate_m write scores, no selection).
__global__ __launch_bounds__(256) void score_kernel(float *__restrict__ v, int64_t n, int score_func) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) v[i] = score_fn(v[i], score_func, 1.0f);
}

// Device math over the 32-bit patterns lo .. lo+n-1 (exhaustive host/device
// agreement checks): fn 0 logf, fn 1 the sqrtsoftplus score of score_fn
// (each also evaluates the wave-lane variant the top-k kernels use,
// wave_scores_of, and reports a difference as 0x7fbadbad); fn 2 the e4m3
// byte of x (f32_to_e4m3), fn 3 the UE8M0 scale byte of the activation
// quantisation for a block whose largest magnitude is |x|, fn 4 x rounded
// to the e4m3 grid (e4m3_round_value: the value of the e4m3 byte of x).
__global__ __launch_bounds__(256) void math_probe_kernel(int fn, uint32_t lo, uint32_t n,
                                                         uint32_t *out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const float x = __uint_as_float(lo + min(i, n - 1));
    uint32_t a, b;
    if (fn == 0) {
        a = b = __float_as_uint(ws_logf(x));
    } else if (fn == 2) {
        a = b = f32_to_e4m3(x);
    } else if (fn == 4) {
        a = b = __float_as_uint(e4m3_round_value(x));
    } else if (fn == 3) {
        float amax = __builtin_fabsf(x);
        if (!(amax >= 1e-4f)) amax = 1e-4f;
        a = b = (uint32_t)(log2_ceil_div448(amax) + 127) & 0xFF;
    } else {
        a = __float_as_uint(score_fn(x, WS_SCORE_SQRTSOFTPLUS, 1.0f));
        float v[1] = {x}, o[1];
        wave_scores_of<1>(v, WS_SCORE_SQRTSOFTPLUS, 1.0f, threadIdx.x & 63, o);
        b = __float_as_uint(o[0]);
    }
    if (i < n) out[i] = a == b ? a : 0x7fbadbadu;
}

static int gate_logits_launch(const float *x, const void *gw, int bf16, float *logits, int64_t m,
                              int64_t dim, int64_t n_experts, hipStream_t stream) {
    if (!x || !gw || !logits) return WS_ERR_INVALID_ARG;
    if (m <= 0 || dim <= 0 || n_experts <= 0) return WS_ERR_INVALID_ARG;
    if (dim % 8 || m > 65535 || n_experts > (1 << 20)) return WS_ERR_SHAPE;
    if (dim % kGC == 0 && m <= (1 << 20)) {
        // one token: 4 experts per wave (the weight stream spread over many
        // CUs); a few tokens: 16 x 4 blocks; more: 8 x 8
        // few tokens: the chain latency is the bound, so a dedicated add wave
        // per 4 chains (16 us at m = 1 against 31 for the single-wave kernel);
        // many tokens: 64 chains per wave (throughput)
        if (m <= 8) gate_pc_launch<4, 1>(x, gw, bf16, logits, m, dim, n_experts, stream);
        else gate_pipe_launch<8, 8>(x, gw, bf16, logits, m, dim, n_experts, stream);
        return launch_status();
    }
    dim3 grid((unsigned)((n_experts + 63) / 64), (unsigned)m);
    if (bf16)
        hipLaunchKernelGGL(gate_logits_kernel<true>, grid, dim3(64), 0, stream, x, gw, logits,
                           (int)dim, (int)n_experts);
    else
        hipLaunchKernelGGL(gate_logits_kernel<false>, grid, dim3(64), 0, stream, x, gw, logits,
                           (int)dim, (int)n_experts);
    return launch_status();
}

static int topk_launch(const float *logits, const float *bias, float *scores_out, int32_t *idx,
                       float *w, int64_t m, int64_t n_experts, int64_t top_k, int score_func,
                       float gate_temp, int norm, float route_scale, hipStream_t stream) {
    if (!logits || !bias || !idx || !w) return WS_ERR_INVALID_ARG;
    if (m <= 0 || n_experts <= 0 || top_k <= 0) return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExperts || top_k > kMaxTopk || top_k > n_experts || m > (1 << 30))
        return WS_ERR_SHAPE;
    if (score_func < 0 || score_func > kScoreIdentity) return WS_ERR_INVALID_ARG;
#define WS_TOPK(C)                                                                            \
    hipLaunchKernelGGL(topk_kernel<C>, dim3((unsigned)m), dim3(64), 0, stream, logits, bias,      \
                       scores_out, idx, w, (int)n_experts, (int)top_k, score_func, gate_temp,    \
                       norm, route_scale)
    if (n_experts <= 128) WS_TOPK(2);
    else if (n_experts <= 256) WS_TOPK(4);
    else if (n_experts <= 384) WS_TOPK(6);
    else if (n_experts <= 512) WS_TOPK(8);
    else WS_TOPK(16);
#undef WS_TOPK
    return launch_status();
}

}  // namespace ws

using namespace ws;

extern "C" {

int ws_math_probe(int fn, uint32_t lo, uint32_t n, uint32_t *out, ws_stream_t stream) {
    if (!out || n == 0 || fn < 0 || fn > 4) return WS_ERR_INVALID_ARG;
    hipLaunchKernelGGL(math_probe_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, fn, lo, n,
                       out);
    return launch_status();
}

int ws_moe_gate_logits(const float *x, const void *gate_w, int w_bf16, float *logits, int64_t m,
                       int64_t dim, int64_t n_experts, ws_stream_t stream) {
    return gate_logits_launch(x, gate_w, w_bf16, logits, m, dim, n_experts, stream);
}

int ws_moe_topk(const float *logits, const float *bias, float *scores_out, int32_t *out_idx,
                float *out_w, int64_t m, int64_t n_experts, int64_t top_k, int score_func,
                float gate_temp, int norm_topk_prob, float route_scale, ws_stream_t stream) {
    if (score_func == kScoreIdentity) return WS_ERR_INVALID_ARG;
    return topk_launch(logits, bias, scores_out, out_idx, out_w, m, n_experts, top_k, score_func,
                       gate_temp, norm_topk_prob, route_scale, stream);
}

int ws_moe_gate_m(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                  int64_t m, int64_t dim, int64_t n_experts, ws_stream_t stream) {
    (void)bias;
    int rc = gate_logits_launch(x, gate_w, 1, scores, m, dim, n_experts, stream);
    if (rc) return rc;
    int64_t n = m * n_experts;
    hipLaunchKernelGGL(score_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, scores,
                       n, WS_SCORE_SQRTSOFTPLUS);
    return launch_status();
}

int ws_moe_gate(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                int64_t dim, int64_t n_experts, ws_stream_t stream) {
    return ws_moe_gate_m(x, gate_w, bias, scores, 1, dim, n_experts, stream);
}

int ws_moe_select(const float *scores, const float *bias, float *out_w, int32_t *out_idx,
                  int64_t n_experts, int64_t top_k, float route_scale, ws_stream_t stream) {
    return topk_launch(scores, bias, nullptr, out_idx, out_w, 1, n_experts, top_k, kScoreIdentity,
                       1.0f, 2, route_scale, stream);
}

int ws_moe_route(const float *x, const uint16_t *gate_w, const float *bias, float *out_w,
                 int32_t *out_idx, int64_t dim, int64_t n_experts, int64_t top_k,
                 float route_scale, ws_stream_t stream) {
    if (!x || !gate_w || !bias || !out_w || !out_idx) return WS_ERR_INVALID_ARG;
    if (dim <= 0 || n_experts <= 0 || top_k <= 0) return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExperts || top_k > kMaxTopk || top_k > n_experts) return WS_ERR_SHAPE;
    unsigned threads = (unsigned)((n_experts + 63) / 64 * 64);
    hipLaunchKernelGGL(route_fused_kernel, dim3(1), dim3(threads), 0, stream, x, gate_w, bias, out_w,
                       out_idx, (int)dim, (int)n_experts, (int)top_k, route_scale);
    return launch_status();
}

}  // extern "C"
