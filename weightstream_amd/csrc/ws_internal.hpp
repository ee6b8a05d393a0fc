// Host-side helpers shared by the translation units of libweightstream_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/ws_hip.h"
#include "ws_device.hpp"

namespace ws {

// Status of the launch just issued: a configuration error is reported at
// launch, anything asynchronous surfaces on the caller's next sync.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? WS_OK : (int)e;
}

// Math mode of this library build (math_mode.hip: WS_MATH_EXACT in
// libweightstream_hip.so, WS_MATH_NATIVE in libweightstream_hip_native.so).
int math_mode();

// Compute units of the current device (queried once per device).
int cu_count();

// Fused GEMVs (gemm.hip): f32 activations x [m <= 16][k] quantised per 1x32
// in the kernel, FP8 weights w [n or 2n][k] with 32 x 32 UE8M0 scales sw.
// kGemvAcc: out[m][n] += x.w^T; kGemvAcc2: out = out + (aux + x.w^T);
// kGemvSwiglu: out[m][n] = silu(min(g, L)) * clamp(u, -L, L) with g from
// weight rows [0, n) and u from rows [n, 2n). Bits equal to ws_emit8 then
// ws_fp8_gemm then the f32 adds / swiglu_emit8's h.
constexpr int kGemvAcc = 2, kGemvAcc2 = 3, kGemvSwiglu = 4;
int kp_gemv_fused(int omode, const float *x, const uint8_t *w, const uint8_t *sw, float *out,
                  const float *aux, float limit, int64_t m, int64_t n, int64_t k,
                  hipStream_t stream);

// gemm.hip: the f32 gate logits [m][E] of h (m <= 8, dim % 256 == 0) and
// hs = SwiGLU of the shared gate/up GEMV (kGemvSwiglu) in one launch.
int gate_w13_launch(const float *h, const float *gw, float *logits, const uint8_t *w13,
                    const uint8_t *s13, float *hs, int64_t m, int64_t dim, int64_t n_experts,
                    int64_t inter, float limit, hipStream_t stream);

// gemm_line.hip: the FP8 GEMM for row blocks of 33-128 rows with whole-K
// tiles (configuration cfg); -1 when the shape does not fit that tiling.
int line_gemm(int smode, int omode, const uint8_t *a, const void *sa, const uint8_t *b,
              const void *sb, void *out, int m, int n, int k, hipStream_t stream, int cfg,
              const float *aux = nullptr);
// C = C + (aux + A.B^T) with UE8M0 32 x 32 weight scales (gemm.hip)
int fp8_gemm_acc2(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                  float *c, const float *aux, int64_t m, int64_t n, int64_t k, hipStream_t stream);

}  // namespace ws
