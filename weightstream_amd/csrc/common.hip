// Runtime entry points and activation quantisation kernels.
//
// Reference: weightstream-cuda/kernels/actquant.cu (act_quant_ue8m0_snap :9,
// act_quant_fp8_emit :47, pack_scale_words :87), launched by
// weightstream-gpu/src/launch.rs:296-326; CPU semantics weightstream-ref
// actquant.rs:21-57.
#include "ws_internal.hpp"

#include <atomic>

namespace ws {

// One thread per element; each 32-lane half of a wave is one 1x32 block.
template <int MODE>  // 0: emit bytes, 1: snap in place
__global__ __launch_bounds__(256) void act_quant_kernel(float *xio, const float *xin, uint8_t *q,
                                                        uint8_t *s, int64_t n,
                                                        int64_t packed_offset) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    bool live = i < n;  // n % 32 == 0, so a half-wave is all live or all dead
    float x = live ? (MODE == 1 ? xio[i] : xin[i]) : 0.0f;
    uint32_t sb;
    uint32_t qb = quant_fp8_block32(x, &sb);
    if (!live) return;
    if (MODE == 1) {
        float sc = __builtin_ldexpf(1.0f, (int)sb - 127);
        xio[i] = e4m3_to_f32(qb) * sc;
    } else {
        q[i] = (uint8_t)qb;
        if ((threadIdx.x & 31) == 0) {
            s[i / 32] = (uint8_t)sb;
            if (packed_offset > 0) s[packed_offset + i / 32] = (uint8_t)sb;
        }
    }
}

__global__ __launch_bounds__(256) void pack_scale_words_kernel(const uint8_t *src, uint32_t *dst,
                                                               int64_t words) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= words) return;
    const uint8_t *p = src + i * 4;
    dst[i] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
             ((uint32_t)p[3] << 24);
}

// f32-scale activation quant: one wave per 1x128 block, two values per lane.
__global__ __launch_bounds__(256) void act_quant_f32s_kernel(const float *x, uint8_t *q, float *s,
                                                             int64_t blocks) {
    int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= blocks) return;  // whole wave exits together
    int l = threadIdx.x & 63;
    const float *v = x + b * 128;
    float x0 = v[l], x1 = v[l + 64];
    float amax = fmaxf(__builtin_fabsf(x0), __builtin_fabsf(x1));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if (!(amax >= 1e-4f)) amax = 1e-4f;  // an all-NaN block too, as the reference's `a > amax` scan
    float sc = amax / 448.0f;
    // inf / inf (a block holding an infinity) is the host's invalid-operation
    // NaN, sign bit set on x86: byte 0xFF, as block_byte
    const bool inf_blk = sc == __builtin_inff();
    const uint32_t q0 = f32_to_e4m3(rclamp(x0 / sc, -448.0f, 448.0f));
    const uint32_t q1 = f32_to_e4m3(rclamp(x1 / sc, -448.0f, 448.0f));
    q[b * 128 + l] = (uint8_t)(inf_blk && __builtin_fabsf(x0) == sc ? 0xFFu : q0);
    q[b * 128 + l + 64] = (uint8_t)(inf_blk && __builtin_fabsf(x1) == sc ? 0xFFu : q1);
    if (l == 0) s[b] = sc;
}

// ---- weight encoders (weightstream-ref store.rs:357-422) -------------------
// e2m1 code with the RNE thresholds of quant.rs:139-163.
__device__ __forceinline__ uint32_t f32_to_e2m1(float v) {
    uint32_t sign = (__float_as_uint(v) >> 31) ? 8u : 0u;
    float a = __builtin_fabsf(v);
    uint32_t c = a <= 0.25f ? 0 : a < 0.75f ? 1 : a <= 1.25f ? 2 : a < 1.75f ? 3
               : a <= 2.5f ? 4 : a < 3.5f ? 5 : a <= 5.0f ? 6 : 7;
    return sign | c;
}

// FP4: one scale per row per 32 columns; a half-wave owns one block, adjacent
// lanes pair into one byte (even column in the low nibble).
__global__ __launch_bounds__(256) void weight_quant_fp4_kernel(const float *w, uint8_t *q,
                                                               uint8_t *s, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    bool live = i < n;
    float v = live ? w[i] : 0.0f;
    float amax = half_wave_max(__builtin_fabsf(v));
    const float floor_ = 6.0f * __builtin_ldexpf(1.0f, -126);
    if (amax < floor_) amax = floor_;
    int e = log2_ceil(amax / 6.0f);
    float sc = __builtin_ldexpf(1.0f, e);
    uint32_t code = f32_to_e2m1(rclamp(v / sc, -6.0f, 6.0f));
    uint32_t hi = __shfl_xor(code, 1, 64);
    if (!live) return;
    if ((threadIdx.x & 1) == 0) q[i / 2] = (uint8_t)((code & 0xF) | (hi << 4));
    if ((threadIdx.x & 31) == 0) s[i / 32] = (uint8_t)(e + 127);
}

// FP8: one scale per 32x32 block; a workgroup of 256 threads owns one block
// (4 values per thread), amax over the whole block.
__global__ __launch_bounds__(256) void weight_quant_fp8_kernel(const float *w, uint8_t *q,
                                                               uint8_t *s, int rows, int cols) {
    __shared__ float wmax[4];
    const int rb = blockIdx.y, cb = blockIdx.x, t = threadIdx.x;
    const int c = cb * 32 + (t & 31);
    float v[4];
    float amax = 1e-4f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int r = rb * 32 + (t >> 5) + 8 * j;
        v[j] = (r < rows) ? w[(size_t)r * cols + c] : 0.0f;
        amax = fmaxf(amax, __builtin_fabsf(v[j]));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((t & 63) == 0) wmax[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int e = log2_ceil(amax / 448.0f);
    float sc = __builtin_ldexpf(1.0f, e);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        int r = rb * 32 + (t >> 5) + 8 * j;
        // an infinity over inf is the host's negative NaN (byte 0xFF), as block_byte
        const uint32_t b = f32_to_e4m3(rclamp(v[j] / sc, -448.0f, 448.0f));
        if (r < rows)
            q[(size_t)r * cols + c] =
                (uint8_t)(sc == __builtin_inff() && __builtin_fabsf(v[j]) == sc ? 0xFFu : b);
    }
    if (t == 0) s[(size_t)rb * (cols / 32) + cb] = (uint8_t)(e + 127);
}

// ws_expf on inputs lo .. lo+n-1; the lane-table variant (ws_expf_lanes) is
// evaluated beside it and any difference is reported as 0x7fbadbad.
__global__ __launch_bounds__(256) void expf_probe_kernel(uint32_t lo, uint32_t n, uint32_t *out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const float x = __uint_as_float(lo + min(i, n - 1));
    const uint32_t a = __float_as_uint(ws_expf(x));
    const uint32_t b = __float_as_uint(ws_expf_lanes(x, ws_lane_exp2f_tab(threadIdx.x & 63)));
    if (i < n) out[i] = a == b ? a : 0x7fbadbadu;
}

// ---- swiglu_limit10 (moe.cu:143), elementwise in moe.rs:187-201 order ----
__global__ __launch_bounds__(256) void swiglu_kernel(const float *gate, const float *up, float *out,
                                                     int64_t n, float rw) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float u = rclamp(up[i], -10.0f, 10.0f);
    float g = fminf(gate[i], 10.0f);
    out[i] = ws_silu(g) * u * rw;
}

int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
        n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace ws

using namespace ws;

extern "C" {

int ws_built_with_hip(void) { return 1; }

int ws_get_math_mode(void) { return math_mode(); }

const char *ws_error_string(int code) {
    switch (code) {
        case WS_OK: return "ok";
        case WS_ERR_INVALID_ARG: return "weightstream-hip: invalid argument";
        case WS_ERR_SHAPE: return "weightstream-hip: unsupported shape";
        case WS_ERR_NO_DEVICE: return "weightstream-hip: no gfx950 device";
        default: return hipGetErrorString((hipError_t)code);
    }
}

int ws_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) return (int)e;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return WS_ERR_NO_DEVICE;
    return WS_OK;
}

int ws_expf_probe(uint32_t lo, uint32_t n, uint32_t *out, ws_stream_t stream) {
    if (!out || n == 0) return WS_ERR_INVALID_ARG;
    hipLaunchKernelGGL(expf_probe_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, lo, n, out);
    return launch_status();
}

static int act_quant_launch(int mode, float *xio, const float *x, uint8_t *q, uint8_t *s,
                            int64_t n, int64_t packed, ws_stream_t stream) {
    if (n <= 0 || n % 32) return WS_ERR_SHAPE;
    dim3 grid((unsigned)((n + 255) / 256));
    if (mode == 1)
        hipLaunchKernelGGL(act_quant_kernel<1>, grid, dim3(256), 0, stream, xio, x, q, s, n, packed);
    else
        hipLaunchKernelGGL(act_quant_kernel<0>, grid, dim3(256), 0, stream, xio, x, q, s, n, packed);
    return launch_status();
}

int ws_snap8(float *x, int64_t n, ws_stream_t stream) {
    if (!x) return WS_ERR_INVALID_ARG;
    return act_quant_launch(1, x, nullptr, nullptr, nullptr, n, 0, stream);
}

int ws_emit8(const float *x, uint8_t *q, uint8_t *s, int64_t n, ws_stream_t stream) {
    if (!x || !q || !s) return WS_ERR_INVALID_ARG;
    return act_quant_launch(0, nullptr, x, q, s, n, 0, stream);
}

int ws_emit8_packed(const float *x, uint8_t *q, uint8_t *s, int64_t n, ws_stream_t stream) {
    if (!x || !q || !s) return WS_ERR_INVALID_ARG;
    int64_t raw = n / 32;
    int64_t packed = (raw + 15) / 16 * 16;
    return act_quant_launch(0, nullptr, x, q, s, n, packed, stream);
}

int ws_pack_scales(const uint8_t *src, uint32_t *dst, int64_t n, ws_stream_t stream) {
    if (!src || !dst) return WS_ERR_INVALID_ARG;
    if (n <= 0 || n % 128) return WS_ERR_SHAPE;
    int64_t words = n / 128;
    hipLaunchKernelGGL(pack_scale_words_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                       stream, src, dst, words);
    return launch_status();
}

int ws_act_quant_f32s(const float *x, uint8_t *q, float *s, int64_t m, int64_t k,
                      ws_stream_t stream) {
    if (!x || !q || !s) return WS_ERR_INVALID_ARG;
    if (m <= 0 || k <= 0 || k % 128) return WS_ERR_SHAPE;
    int64_t blocks = m * (k / 128);
    hipLaunchKernelGGL(act_quant_f32s_kernel, dim3((unsigned)((blocks + 3) / 4)), dim3(256), 0,
                       stream, x, q, s, blocks);
    return launch_status();
}

int ws_weight_quant_fp4(const float *w, uint8_t *q, uint8_t *s, int64_t rows, int64_t cols,
                        ws_stream_t stream) {
    if (!w || !q || !s) return WS_ERR_INVALID_ARG;
    if (rows <= 0 || cols <= 0 || cols % 32) return WS_ERR_SHAPE;
    int64_t n = rows * cols;
    hipLaunchKernelGGL(weight_quant_fp4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       stream, w, q, s, n);
    return launch_status();
}

int ws_weight_quant_fp8(const float *w, uint8_t *q, uint8_t *s, int64_t rows, int64_t cols,
                        ws_stream_t stream) {
    if (!w || !q || !s) return WS_ERR_INVALID_ARG;
    if (rows <= 0 || cols <= 0 || cols % 32 || rows > (1 << 24) || cols > (1 << 24))
        return WS_ERR_SHAPE;
    dim3 grid((unsigned)(cols / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(weight_quant_fp8_kernel, grid, dim3(256), 0, stream, w, q, s, (int)rows,
                       (int)cols);
    return launch_status();
}

int ws_swiglu(const float *gate, const float *up, float *out, int64_t n, float rw,
              ws_stream_t stream) {
    if (!gate || !up || !out) return WS_ERR_INVALID_ARG;
    if (n <= 0) return WS_ERR_SHAPE;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, gate,
                       up, out, n, rw);
    return launch_status();
}

}  // extern "C"
