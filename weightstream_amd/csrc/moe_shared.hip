// Shared FP8 expert and the f32 accumulate of the MoE block.
//
// Reference: weightstream-ref moe.rs:210-250 (shared_expert_hidden: FP8
// gate/up, SwiGLU with routing weight 1, FP8 down, each activation quantised
// per 1x32 by fp8_gemv), the engine's moe_shared_step (engine.rs:4063) which
// runs it as emit8 + fp8 GEMMs + swiglu on the device, and acc_f32
// (gemv.cu:63, launch.rs:1175) that adds it to the routed sum.
//
// The shared expert is three FP8 block-scaled GEMMs (ws_fp8_gemm) around two
// small kernels: the token quantisation (ws_emit8) and a fused SwiGLU +
// 1x32 FP8 quantisation of the hidden state, so h never round-trips as f32.
#include "ws_internal.hpp"

namespace ws {

// h = silu(min(g, L)) * clamp(u, -L, L) (moe.rs:187-201 with weight 1; L <= 0
// disables both clamps), then the 1x32 FP8 quantisation of actquant.rs:21-45.
// One thread per element of h [rows, inter]; gate and up rows are `ld`
// floats apart (inter for separate buffers, 2 * inter for the fused w13
// output); a 32-lane half-wave is one scale block.
__global__ __launch_bounds__(256) void swiglu_emit8_kernel(const float *__restrict__ gate,
                                                           const float *__restrict__ up,
                                                           uint8_t *__restrict__ hq,
                                                           uint8_t *__restrict__ hs, int64_t n,
                                                           int inter, int ld, float limit) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool live = i < n;  // n % 32 == 0: a half-wave is all live or all dead
    float h = 0.0f;
    if (live) {
        const int64_t o = (i / inter) * ld + i % inter;
        float g = gate[o], u = up[o];
        if (limit > 0.0f) {
            u = rclamp(u, -limit, limit);
            g = fminf(g, limit);
        }
        h = ws_silu(g) * u;
    }
    uint32_t sb;
    const uint32_t qb = quant_fp8_block32(h, &sb);
    if (!live) return;
    hq[i] = (uint8_t)qb;
    if ((threadIdx.x & 31) == 0) hs[i / 32] = (uint8_t)sb;
}

__global__ __launch_bounds__(256) void acc_f32_kernel(const float *__restrict__ x,
                                                      float *__restrict__ y, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 4 <= n) {
        const float4 a = *(const float4 *)(x + i);
        float4 b = *(const float4 *)(y + i);
        b.x = b.x + a.x;
        b.y = b.y + a.y;
        b.z = b.z + a.z;
        b.w = b.w + a.w;
        *(float4 *)(y + i) = b;
    } else {
        for (int64_t j = i; j < n; j++) y[j] = y[j] + x[j];
    }
}

// h = h + (yr + ys), the two acc_f32 adds of the block in their order
// (yr += ys, then h += yr) without writing yr
__global__ __launch_bounds__(256) void acc2_f32_kernel(const float *__restrict__ ys,
                                                       const float *__restrict__ yr,
                                                       float *__restrict__ h, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = h[i] + (yr[i] + ys[i]);
}

struct SharedLayout {
    size_t xq, xs, g, u, hq, hs, y, total;
};

static size_t al256(size_t v) { return (v + 255) / 256 * 256; }

static SharedLayout shared_layout(int64_t m, int64_t dim, int64_t inter) {
    SharedLayout l;
    size_t o = 0;
    l.xq = o; o += al256((size_t)m * dim);
    l.xs = o; o += al256((size_t)m * (dim / 32));
    l.g = o; o += al256((size_t)m * inter * 4);
    l.u = o; o += al256((size_t)m * inter * 4);
    l.hq = o; o += al256((size_t)m * inter);
    l.hs = o; o += al256((size_t)m * (inter / 32));
    l.y = o; o += al256((size_t)m * dim * 4);
    l.total = o;
    return l;
}

}  // namespace ws

using namespace ws;

extern "C" {

int ws_acc_f32(const float *x, float *y, int64_t n, ws_stream_t stream) {
    if (!x || !y) return WS_ERR_INVALID_ARG;
    if (n <= 0) return WS_ERR_SHAPE;
    if (((uintptr_t)x | (uintptr_t)y) & 15) return WS_ERR_INVALID_ARG;
    const int64_t quads = (n + 3) / 4;
    hipLaunchKernelGGL(acc_f32_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, stream,
                       x, y, n);
    return launch_status();
}

size_t ws_shared_expert_workspace_size(int64_t m, int64_t dim, int64_t inter) {
    if (m <= 0 || dim <= 0 || inter <= 0) return 0;
    return shared_layout(m, dim, inter).total;
}

int ws_shared_expert_fp8(const float *x, const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                         const uint8_t *s3, const uint8_t *w2, const uint8_t *s2, float *y,
                         int64_t m, int64_t dim, int64_t inter, float swiglu_limit,
                         void *workspace, size_t workspace_bytes, ws_stream_t stream) {
    if (!x || !w1 || !s1 || !w3 || !s3 || !w2 || !s2 || !y || !workspace)
        return WS_ERR_INVALID_ARG;
    if (m <= 0 || dim <= 0 || inter <= 0 || dim % 128 || inter % 128) return WS_ERR_SHAPE;
    const SharedLayout l = shared_layout(m, dim, inter);
    if (workspace_bytes < l.total || ((uintptr_t)workspace & 255)) return WS_ERR_INVALID_ARG;
    uint8_t *ws = (uint8_t *)workspace;
    uint8_t *xq = ws + l.xq, *xs = ws + l.xs, *hq = ws + l.hq, *hs = ws + l.hs;
    float *g = (float *)(ws + l.g), *u = (float *)(ws + l.u);
    int rc = ws_emit8(x, xq, xs, m * dim, stream);
    if (rc) return rc;
    rc = ws_fp8_gemm(xq, xs, w1, s1, g, m, inter, dim, stream);
    if (rc) return rc;
    rc = ws_fp8_gemm(xq, xs, w3, s3, u, m, inter, dim, stream);
    if (rc) return rc;
    const int64_t n = m * inter;
    hipLaunchKernelGGL(swiglu_emit8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       g, u, hq, hs, n, (int)inter, (int)inter, swiglu_limit);
    rc = launch_status();
    if (rc) return rc;
    return ws_fp8_gemm(hq, hs, w2, s2, y, m, dim, inter, stream);
}

int ws_shared_expert_fp8_w13(const float *x, const uint8_t *w13, const uint8_t *s13,
                             const uint8_t *w2, const uint8_t *s2, float *y, int64_t m,
                             int64_t dim, int64_t inter, float swiglu_limit, void *workspace,
                             size_t workspace_bytes, ws_stream_t stream) {
    if (!x || !w13 || !s13 || !w2 || !s2 || !y || !workspace) return WS_ERR_INVALID_ARG;
    if (m <= 0 || dim <= 0 || inter <= 0 || dim % 128 || inter % 128) return WS_ERR_SHAPE;
    const SharedLayout l = shared_layout(m, dim, inter);
    if (workspace_bytes < l.total || ((uintptr_t)workspace & 255)) return WS_ERR_INVALID_ARG;
    uint8_t *ws = (uint8_t *)workspace;
    uint8_t *xq = ws + l.xq, *xs = ws + l.xs, *hq = ws + l.hq, *hs = ws + l.hs;
    // gate|up rows [m, 2 * inter] span the two adjacent f32 regions
    float *gu = (float *)(ws + l.g);
    int rc = ws_emit8(x, xq, xs, m * dim, stream);
    if (rc) return rc;
    rc = ws_fp8_gemm(xq, xs, w13, s13, gu, m, 2 * inter, dim, stream);
    if (rc) return rc;
    const int64_t n = m * inter;
    hipLaunchKernelGGL(swiglu_emit8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       gu, gu + inter, hq, hs, n, (int)inter, (int)(2 * inter), swiglu_limit);
    rc = launch_status();
    if (rc) return rc;
    return ws_fp8_gemm(hq, hs, w2, s2, y, m, dim, inter, stream);
}

// emit8 + fp8_gemm + acc_f32 in one launch (m <= 16)
int ws_fp8_gemv_acc(const float *x, const uint8_t *w, const uint8_t *sw, float *h, int64_t m,
                    int64_t n, int64_t k, ws_stream_t stream) {
    return kp_gemv_fused(kGemvAcc, x, w, sw, h, nullptr, 0.0f, m, n, k, stream);
}

int ws_shared_expert_fp8_w13_acc(const float *x, const uint8_t *w13, const uint8_t *s13,
                                 const uint8_t *w2, const uint8_t *s2, const float *yr, float *h,
                                 int64_t m, int64_t dim, int64_t inter, float swiglu_limit,
                                 void *workspace, size_t workspace_bytes, ws_stream_t stream) {
    if (!x || !w13 || !s13 || !w2 || !s2 || !yr || !h || !workspace) return WS_ERR_INVALID_ARG;
    if (m <= 0 || dim <= 0 || inter <= 0 || dim % 128 || inter % 128) return WS_ERR_SHAPE;
    const SharedLayout l = shared_layout(m, dim, inter);
    if (workspace_bytes < l.total || ((uintptr_t)workspace & 255)) return WS_ERR_INVALID_ARG;
    uint8_t *ws = (uint8_t *)workspace;
    if (m <= 2 && dim <= 8192 && inter <= 8192) {
        // gate/up GEMV + SwiGLU -> h_s (f32), then the down GEMV that
        // quantises h_s and adds into h. Every workgroup quantises the whole
        // activation itself, so this pays for few rows only (block at m = 8:
        // 184.7 us/layer this way against 167 unfused)
        float *hf = (float *)(ws + l.g);
        int rc = kp_gemv_fused(kGemvSwiglu, x, w13, s13, hf, nullptr, swiglu_limit, m, inter, dim,
                               stream);
        if (rc) return rc;
        return kp_gemv_fused(kGemvAcc2, hf, w2, s2, h, yr, 0.0f, m, dim, inter, stream);
    }
    // ws_shared_expert_fp8_w13, its down GEMM adding into h in the epilogue
    // (h = h + (yr + ys): the acc_f32 pair's bits); x may be h (x is
    // quantised first)
    uint8_t *xq = ws + l.xq, *xs = ws + l.xs, *hq = ws + l.hq, *hs = ws + l.hs;
    float *gu = (float *)(ws + l.g);
    int rc = ws_emit8(x, xq, xs, m * dim, stream);
    if (rc) return rc;
    rc = ws_fp8_gemm(xq, xs, w13, s13, gu, m, 2 * inter, dim, stream);
    if (rc) return rc;
    const int64_t n = m * inter;
    hipLaunchKernelGGL(swiglu_emit8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       gu, gu + inter, hq, hs, n, (int)inter, (int)(2 * inter), swiglu_limit);
    rc = launch_status();
    if (rc) return rc;
    rc = fp8_gemm_acc2(hq, hs, w2, s2, h, yr, m, dim, inter, stream);
    if (rc != WS_ERR_SHAPE) return rc;
    // shapes the accumulating kernels do not take: the GEMM, then the adds
    float *ys = (float *)(ws + l.y);
    rc = ws_fp8_gemm(hq, hs, w2, s2, ys, m, dim, inter, stream);
    if (rc) return rc;
    const int64_t nd = m * dim;
    hipLaunchKernelGGL(acc2_f32_kernel, dim3((unsigned)((nd + 255) / 256)), dim3(256), 0, stream,
                       ys, yr, h, nd);
    return launch_status();
}

int ws_moe_gate_shared_w13(const float *h, const float *gate_w, float *logits,
                           const uint8_t *w13, const uint8_t *s13, float *hs, int64_t m,
                           int64_t dim, int64_t n_experts, int64_t inter, float swiglu_limit,
                           ws_stream_t stream) {
    return gate_w13_launch(h, gate_w, logits, w13, s13, hs, m, dim, n_experts, inter, swiglu_limit,
                           stream);
}

int ws_shared_expert_down_acc(const float *hs, const uint8_t *w2, const uint8_t *s2,
                              const float *yr, float *h, int64_t m, int64_t dim, int64_t inter,
                              ws_stream_t stream) {
    if (!yr) return WS_ERR_INVALID_ARG;
    return kp_gemv_fused(kGemvAcc2, hs, w2, s2, h, yr, 0.0f, m, dim, inter, stream);
}

}  // extern "C"
