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
//  glu_quant: grid (inter/32, top_k), 16 waves: a wave streams 16 rows of w1 or
//    w3 of the 32-row tile over a quarter of K (8 KB at the BASELINE shape, all
//    loads in flight at once); the quarters are added in LDS in fixed order,
//    then the epilogue applies SwiGLU x routing weight and quantises the 32
//    values (one FP8 1x32 block) straight to e4m3 + UE8M0.
//  reduce: grid (dim/16), 16 waves over (expert, K part) units for 16 output
//    rows; per-expert results meet in LDS and are added in ascending expert id,
//    one f32 add per expert like the reference's acc_f32 chain.
#include "ws_internal.hpp"

namespace ws {

constexpr int kDecThreads = 1024;  // 16 waves: K is split across waves
constexpr int kGluKSplit = 4;      // glu: 4 (matrix, half) units x 4 K parts
constexpr int kRedKSplitMax = 16;
constexpr int kMaxTopkDec = 16;
constexpr int kU = 8;  // K steps in flight per wave

// rank of pick `slot` among valid picks ordered by (expert id, slot)
__device__ __forceinline__ int pick_rank(const int32_t *idx, int top_k, int n_experts, int slot) {
    int e = idx[slot];
    int rank = 0;
    for (int j = 0; j < top_k; j++) {
        int f = idx[j];
        if (f < 0 || f >= n_experts) continue;
        if (f < e || (f == e && j < slot)) rank++;
    }
    return rank;
}

// Stream a 16-row FP4 weight tile against the token held in LDS and return the
// 16x16 MFMA accumulator (all columns equal). w_rows / s_rows point at row 0
// of the tile and its scale row; row strides k/2 bytes and k/32 bytes.
// EXACT: the token is bf16 in LDS (x_lds, k values), the weights are
// dequantised to bf16 in registers, bf16 MFMA. Native: the token is e4m3 +
// UE8M0 in LDS (xq_lds, xs_lds) and feeds the scaled FP4 x FP8 MFMA.
template <bool EXACT>
__device__ __forceinline__ v4f stream_fp4_rows(const uint8_t *__restrict__ w_rows,
                                               const uint8_t *__restrict__ s_rows,
                                               const uint8_t *xq_lds, const uint8_t *xs_lds,
                                               const __bf16 *x_lds, int k, int kstep0,
                                               int ksteps, int lane) {
    const int r = lane & 15, kb = lane >> 4;
    const uint8_t *wp = w_rows + (size_t)r * (k / 2) + kb * 16;
    const uint8_t *sp = s_rows + (size_t)r * (k / 32);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int ks0 = kstep0; ks0 < ksteps; ks0 += kU) {
        uint4 wf[kU];
        uint32_t ws_[kU];
#pragma unroll
        for (int u = 0; u < kU; u++) {
            int ks = ks0 + u;
            if (ks < ksteps) {
                wf[u] = ldg16_stream(wp + (size_t)ks * 64);
                ws_[u] = *(const uint32_t *)(sp + ks * 4) >> (8 * kb);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
            int ks = ks0 + u;
            if (ks >= ksteps) continue;
            if (EXACT) {
                v8bf wq[4], xb[4];
                cvt_fp4x32(wf[u], e8m0_to_f32(ws_[u] & 0xFF), wq);
                const v8bf *xp = (const v8bf *)(x_lds + ks * 128 + kb * 32);
#pragma unroll
                for (int j = 0; j < 4; j++) xb[j] = xp[j];
                acc = mfma_bf16_k128(wq, xb, acc);
            } else {
                const uint8_t *xp = xq_lds + ks * 128 + kb * 16;
                v8i b = frag_from(*(const uint4 *)xp, *(const uint4 *)(xp + 64));
                int sx = xs_lds[ks * 4 + kb];
                acc = mfma_scaled<kFmtFp4, kFmtFp8>(frag_from4(wf[u]), b, acc, (int)ws_[u], sx);
            }
        }
    }
    return acc;
}

// n e4m3 values + their UE8M0 scales (global) -> exact bf16 values in LDS.
// n % 8 == 0; every thread converts 8 values (one 8-byte chunk of one block).
__device__ __forceinline__ void fp8_to_bf16_lds(const uint8_t *q, const uint8_t *s, __bf16 *dst,
                                                int n, int t, int nthreads) {
    for (int i = t * 8; i < n; i += nthreads * 8) {
        uint2 v = *(const uint2 *)(q + i);
        float sc = e8m0_to_f32(s[i / 32]);
        u32x4v o = pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, sc, false),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.x, sc, true),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, sc, false),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v.y, sc, true));
        *(u32x4v *)(dst + i) = o;
    }
}

template <bool EXACT>
__global__ __launch_bounds__(kDecThreads) void expert_glu_quant_kernel(
    const uint8_t *__restrict__ xq, const uint8_t *__restrict__ xs, const int32_t *__restrict__ idx,
    const float *__restrict__ topk_w, const uint8_t *__restrict__ w1, const uint8_t *__restrict__ s1,
    const uint8_t *__restrict__ w3, const uint8_t *__restrict__ s3, uint8_t *__restrict__ hq,
    uint8_t *__restrict__ hs, int dim, int inter, int n_experts, int top_k, float limit) {
    extern __shared__ __align__(16) uint8_t lds[];
    // EXACT: bf16 token (2*dim bytes); native: e4m3 token + scales
    __bf16 *x_l = (__bf16 *)lds;
    uint8_t *xq_l = lds;
    uint8_t *xs_l = lds + dim;
    __shared__ float part[kGluKSplit][2][32];
    const int slot = blockIdx.y;
    const int e = idx[slot];
    if (e < 0 || e >= n_experts) return;  // whole workgroup
    const int tile = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;

    if (EXACT) {
        fp8_to_bf16_lds(xq, xs, x_l, dim, t, kDecThreads);
    } else {
        for (int i = t * 16; i < dim; i += kDecThreads * 16)
            *(uint4 *)(xq_l + i) = *(const uint4 *)(xq + i);
        for (int i = t; i < dim / 32; i += kDecThreads) xs_l[i] = xs[i];
    }
    __syncthreads();

    // wave -> (matrix, 16-row half of the tile, K quarter)
    const int unit = w & 3, ksp = w >> 2;
    const int mat = unit >> 1, half = unit & 1;
    const int ksteps = dim / 128;
    const int k0 = ksp * ksteps / kGluKSplit, k1 = (ksp + 1) * ksteps / kGluKSplit;
    const int row0 = tile * 32 + half * 16;
    const size_t wmat = (size_t)inter * (dim / 2), smat = (size_t)inter * (dim / 32);
    const uint8_t *W = (mat ? w3 : w1) + (size_t)e * wmat + (size_t)row0 * (dim / 2);
    const uint8_t *S = (mat ? s3 : s1) + (size_t)e * smat + (size_t)row0 * (dim / 32);
    v4f acc = stream_fp4_rows<EXACT>(W, S, xq_l, xs_l, x_l, dim, k0, k1, lane);
    // D[i][j]: i = weight row 4*(lane/16)+v, j = lane%16 (all columns equal)
    if ((lane & 15) == 0) {
#pragma unroll
        for (int v = 0; v < 4; v++) part[ksp][mat][half * 16 + 4 * (lane >> 4) + v] = acc[v];
    }
    __syncthreads();
    if (w != 0) return;
    // lanes 0-31 own the tile's 32 values; lanes 32-63 mirror them so the
    // half-wave reduction stays uniform, and do not store
    const int n = lane & 31;
    float g = part[0][0][n], u = part[0][1][n];
#pragma unroll
    for (int q = 1; q < kGluKSplit; q++) {
        g = g + part[q][0][n];
        u = u + part[q][1][n];
    }
    if (limit > 0.0f) {
        u = rclamp(u, -limit, limit);
        g = fminf(g, limit);
    }
    const float rw = topk_w[slot];
    float h = ws_silu(g) * u * rw;
    uint32_t sb;
    uint32_t qb = quant_fp8_block32(h, &sb);
    if (lane < 32) {
        const int rank = pick_rank(idx, top_k, n_experts, slot);
        hq[(size_t)rank * inter + tile * 32 + n] = (uint8_t)qb;
        if (n == 0) hs[(size_t)rank * (inter / 32) + tile] = (uint8_t)sb;
    }
}

template <bool EXACT>
__global__ __launch_bounds__(kDecThreads) void expert_reduce_kernel(
    const uint8_t *__restrict__ hq, const uint8_t *__restrict__ hs, const int32_t *__restrict__ idx,
    const uint8_t *__restrict__ w2, const uint8_t *__restrict__ s2, float *__restrict__ y, int dim,
    int inter, int n_experts, int top_k) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int32_t sorted_e[kMaxTopkDec];
    __shared__ int32_t n_valid;
    __shared__ float part[kMaxTopkDec][kRedKSplitMax][16];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int row0 = blockIdx.x * 16;
    if (t == 0) {
        int cnt = 0;
        for (int s = 0; s < top_k; s++) {
            int e = idx[s];
            if (e < 0 || e >= n_experts) continue;
            sorted_e[pick_rank(idx, top_k, n_experts, s)] = e;
            cnt++;
        }
        n_valid = cnt;
    }
    // EXACT: picks as bf16 (2 * top_k * inter bytes); native: e4m3 + scales
    __bf16 *h_l = (__bf16 *)lds;
    uint8_t *hq_l = lds;
    uint8_t *hs_l = lds + (size_t)top_k * inter;
    __syncthreads();
    const int nv = n_valid;
    if (EXACT) {
        fp8_to_bf16_lds(hq, hs, h_l, nv * inter, t, kDecThreads);
    } else {
        for (int i = t * 16; i < nv * inter; i += kDecThreads * 16)
            *(uint4 *)(hq_l + i) = *(const uint4 *)(hq + i);
        for (int i = t; i < nv * (inter / 32); i += kDecThreads) hs_l[i] = hs[i];
    }
    __syncthreads();

    // work units (pick, K part): every wave streams 16 rows of one expert's
    // w2 over 1/ksplit of inter
    const int ksteps = inter / 128;
    int ksplit = (kDecThreads / 64) / (nv > 0 ? nv : 1);
    ksplit = ksplit < 1 ? 1 : (ksplit > kRedKSplitMax ? kRedKSplitMax : ksplit);
    if (ksplit > ksteps) ksplit = ksteps;
    const size_t wmat = (size_t)dim * (inter / 2), smat = (size_t)dim * (inter / 32);
    for (int unit = w; unit < nv * ksplit; unit += kDecThreads / 64) {
        const int p = unit / ksplit, ksp = unit % ksplit;
        const int e = sorted_e[p];
        const uint8_t *W = w2 + (size_t)e * wmat + (size_t)row0 * (inter / 2);
        const uint8_t *S = s2 + (size_t)e * smat + (size_t)row0 * (inter / 32);
        v4f acc = stream_fp4_rows<EXACT>(W, S, hq_l + (size_t)p * inter,
                                         hs_l + (size_t)p * (inter / 32),
                                         h_l + (size_t)p * inter, inter, ksp * ksteps / ksplit,
                                         (ksp + 1) * ksteps / ksplit, lane);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int v = 0; v < 4; v++) part[p][ksp][4 * (lane >> 4) + v] = acc[v];
        }
    }
    __syncthreads();
    if (t < 16) {
        // one f32 add per expert, ascending expert id (moe.rs:76-84)
        float acc = 0.0f;
        for (int p = 0; p < nv; p++) {
            float pe = part[p][0][t];
            for (int q = 1; q < ksplit; q++) pe = pe + part[p][q][t];
            acc = acc + pe;
        }
        y[row0 + t] = acc;
    }
}

static int check_decode_shapes(int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k) {
    if (dim <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0) return WS_ERR_INVALID_ARG;
    if (dim % 128 || inter % 128 || top_k > kMaxTopkDec) return WS_ERR_SHAPE;
    // LDS holds the token / the picks as bf16 (2 bytes per value)
    if (dim > 32768 || inter > 32768 || top_k * inter > 32768 || n_experts > (1 << 20))
        return WS_ERR_SHAPE;
    return WS_OK;
}

static inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace ws

using namespace ws;

extern "C" {

int ws_expert_glu_quant(const uint8_t *xq, const uint8_t *xs, const int32_t *topk_idx,
                        const float *topk_w, const uint8_t *w1, const uint8_t *s1,
                        const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                        int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                        float swiglu_limit, ws_stream_t stream) {
    if (!xq || !xs || !topk_idx || !topk_w || !w1 || !s1 || !w3 || !s3 || !hq || !hs)
        return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (!aligned16(xq) || !aligned16(w1) || !aligned16(w3) || ((uintptr_t)s1 & 3) ||
        ((uintptr_t)s3 & 3))
        return WS_ERR_INVALID_ARG;
    dim3 grid((unsigned)(inter / 32), (unsigned)top_k);
    const bool exact = math_mode() == WS_MATH_EXACT;
    size_t lds = exact ? (size_t)dim * 2 : (size_t)dim + dim / 32;
    if (exact)
        hipLaunchKernelGGL(expert_glu_quant_kernel<true>, grid, dim3(kDecThreads), lds, stream, xq,
                           xs, topk_idx, topk_w, w1, s1, w3, s3, hq, hs, (int)dim, (int)inter,
                           (int)n_experts, (int)top_k, swiglu_limit);
    else
        hipLaunchKernelGGL(expert_glu_quant_kernel<false>, grid, dim3(kDecThreads), lds, stream, xq,
                           xs, topk_idx, topk_w, w1, s1, w3, s3, hq, hs, (int)dim, (int)inter,
                           (int)n_experts, (int)top_k, swiglu_limit);
    return launch_status();
}

int ws_expert_reduce(const uint8_t *hq, const uint8_t *hs, const int32_t *topk_idx,
                     const uint8_t *w2, const uint8_t *s2, float *y, int64_t dim, int64_t inter,
                     int64_t n_experts, int64_t top_k, ws_stream_t stream) {
    if (!hq || !hs || !topk_idx || !w2 || !s2 || !y) return WS_ERR_INVALID_ARG;
    int rc = check_decode_shapes(dim, inter, n_experts, top_k);
    if (rc) return rc;
    if (!aligned16(hq) || !aligned16(w2) || ((uintptr_t)s2 & 3)) return WS_ERR_INVALID_ARG;
    const bool exact = math_mode() == WS_MATH_EXACT;
    size_t lds = exact ? (size_t)top_k * inter * 2 : (size_t)top_k * inter + (size_t)top_k * (inter / 32);
    if (exact)
        hipLaunchKernelGGL(expert_reduce_kernel<true>, dim3((unsigned)(dim / 16)), dim3(kDecThreads),
                           lds, stream, hq, hs, topk_idx, w2, s2, y, (int)dim, (int)inter,
                           (int)n_experts, (int)top_k);
    else
        hipLaunchKernelGGL(expert_reduce_kernel<false>, dim3((unsigned)(dim / 16)),
                           dim3(kDecThreads), lds, stream, hq, hs, topk_idx, w2, s2, y, (int)dim,
                           (int)inter, (int)n_experts, (int)top_k);
    return launch_status();
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

size_t ws_moe_decode_workspace_size(int64_t dim, int64_t inter, int64_t top_k) {
    if (dim <= 0 || inter <= 0 || top_k <= 0) return 0;
    return align256(dim) + align256(dim / 32) + align256(top_k * inter) +
           align256(top_k * (inter / 32));
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
    uint8_t *p = (uint8_t *)workspace;
    uint8_t *xq = p;
    p += align256(dim);
    uint8_t *xs = p;
    p += align256(dim / 32);
    uint8_t *hq = p;
    p += align256(top_k * inter);
    uint8_t *hs = p;
    rc = ws_emit8(x, xq, xs, dim, stream);
    if (rc) return rc;
    rc = ws_expert_glu_quant(xq, xs, topk_idx, topk_w, w1, s1, w3, s3, hq, hs, dim, inter,
                             n_experts, top_k, swiglu_limit, stream);
    if (rc) return rc;
    return ws_expert_reduce(hq, hs, topk_idx, w2, s2, y, dim, inter, n_experts, top_k, stream);
}

}  // extern "C"
