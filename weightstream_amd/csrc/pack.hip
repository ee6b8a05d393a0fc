// Upload-time relayout of FP4 weight matrices into the fragment-major layout
// of ws_pack.hpp (the counterpart of weightstream-gpu engine.rs:842-884
// pack_expert_scales / tile_major_expert).
#include "ws_internal.hpp"
#include "ws_pack.hpp"

namespace ws {

// one thread per 16-byte chunk (row r, K [32c, 32c+32)) and its scale byte
__global__ __launch_bounds__(256) void prepack_fp4_kernel(const uint8_t *__restrict__ w,
                                                          const uint8_t *__restrict__ s,
                                                          uint8_t *__restrict__ pw,
                                                          uint8_t *__restrict__ ps, int64_t rows,
                                                          int cols) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int cpr = cols / 32;  // 32-value chunks per row
    if (i >= rows * cpr) return;
    const int64_t r = i / cpr;
    const int c = (int)(i % cpr);
    const int ks = c / 4, g = c % 4, ksn = cols / 128, ks8 = (ksn + 7) / 8;
    const int64_t rt = r / 16;
    const int lane = (int)(r % 16) + 16 * g;
    const uint4 v = *(const uint4 *)(w + r * (cols / 2) + (int64_t)c * 16);
    *(uint4 *)(pw + ((rt * ksn + ks) * 64 + lane) * 16) = v;
    ps[((rt * ks8 + ks / 8) * 64 + lane) * 8 + ks % 8] = s[r * cpr + c];
}

__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t *p, int64_t n, uint8_t v) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace ws

using namespace ws;

extern "C" {

size_t ws_packed_fp4_scale_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 128) return 0;
    return (size_t)packed_fp4_scale_bytes(rows, cols);
}

int ws_prepack_fp4(const uint8_t *w, const uint8_t *s, int64_t rows, int64_t cols, uint8_t *pw,
                   uint8_t *ps, ws_stream_t stream) {
    if (!w || !s || !pw || !ps || rows <= 0 || cols <= 0) return WS_ERR_INVALID_ARG;
    if (rows % 16 || cols % 128 || cols > (1 << 24)) return WS_ERR_SHAPE;
    if (((uintptr_t)w | (uintptr_t)pw) & 15) return WS_ERR_INVALID_ARG;
    const int64_t n = rows * (cols / 32);
    // the padding bytes of every lane's last 8-step scale group are never
    // read; fill them anyway so the packed buffer is deterministic
    const int64_t sb = packed_fp4_scale_bytes(rows, cols);
    if ((cols / 128) % 8) {
        hipLaunchKernelGGL(fill_u8_kernel, dim3((unsigned)((sb + 255) / 256)), dim3(256), 0, stream,
                           ps, sb, (uint8_t)127);
        int rc = launch_status();
        if (rc) return rc;
    }
    hipLaunchKernelGGL(prepack_fp4_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       w, s, pw, ps, rows, (int)cols);
    return launch_status();
}

}  // extern "C"
