// C++ host mirror of weightstream-gpu's launch.rs over the C ABI in ws_hip.h.
//
// Same names and argument order as weightstream-gpu/src/launch.rs; the `&Cuda`
// handle becomes an optional stream argument (the `*_on` variants), and a
// failed launch throws weightstream_hip::Error where launch.rs panics through
// `.unwrap()`. Header-only; link against libweightstream_hip.so.
#pragma once

#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>

#include "ws_hip.h"

namespace weightstream_hip {

struct Error : std::runtime_error {
    int code;
    Error(const char *fn, int c)
        : std::runtime_error(std::string(fn) + ": " + ws_error_string(c)), code(c) {}
};

inline void check(const char *fn, int code) {
    if (code != WS_OK) throw Error(fn, code);
}

// weightstream_cuda::gpu::Cuda::global() (gpu.rs:93): one process-wide handle
// holding the main and aux streams. Streams are created by the caller (the
// engine owns them); the handle only validates the device once.
class Hip {
  public:
    ws_stream_t stream = nullptr;
    ws_stream_t aux_stream = nullptr;
    static Hip &global() {
        static std::once_flag once;
        static Hip inst;
        std::call_once(once, [] { check("ws_init", ws_init()); });
        return inst;
    }
};

inline bool built_with_hip() { return ws_built_with_hip() != 0; }

namespace launch {

using U8 = const uint8_t *;
using F32 = float *;

// actquant.cu (launch.rs:296-326)
inline void snap8(float *x, int64_t n, ws_stream_t s = nullptr) { check("snap8", ws_snap8(x, n, s)); }
inline void emit8(const float *x, uint8_t *q, uint8_t *sc, int64_t n, ws_stream_t s = nullptr) {
    check("emit8", ws_emit8(x, q, sc, n, s));
}
inline void emit8_packed(const float *x, uint8_t *q, uint8_t *sc, int64_t n,
                         ws_stream_t s = nullptr) {
    check("emit8_packed", ws_emit8_packed(x, q, sc, n, s));
}
inline void pack_scales(U8 src, uint32_t *dst, int64_t n, ws_stream_t s = nullptr) {
    check("pack_scales", ws_pack_scales(src, dst, n, s));
}

// GEMMs (launch.rs:344-377, 717-804)
inline void fp8_gemm(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                     ws_stream_t s = nullptr) {
    check("fp8_gemm", ws_fp8_gemm(a, sa, b, sb, out, m, n, k, s));
}
inline void fp8_gemm_on(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                        ws_stream_t s) {
    fp8_gemm(a, sa, b, sb, out, m, n, k, s);
}
inline void fp8_gemm_tile(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                          ws_stream_t s = nullptr) {
    check("fp8_gemm_tile", ws_fp8_gemm_tile(a, sa, b, sb, out, m, n, k, s));
}
inline void fp4_gemm(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                     ws_stream_t s = nullptr) {
    check("fp4_gemm", ws_fp4_gemm(a, sa, b, sb, out, m, n, k, s));
}
inline void fp4_gemm_tile(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                          ws_stream_t s = nullptr) {
    check("fp4_gemm_tile", ws_fp4_gemm_tile(a, sa, b, sb, out, m, n, k, s));
}

// routing (launch.rs:998-1100)
inline void moe_gate(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                     int64_t dim, int64_t n_experts, ws_stream_t s = nullptr) {
    check("moe_gate", ws_moe_gate(x, gate_w, bias, scores, dim, n_experts, s));
}
inline void moe_gate_m(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                       int64_t m, int64_t dim, int64_t n_experts, ws_stream_t s = nullptr) {
    check("moe_gate_m", ws_moe_gate_m(x, gate_w, bias, scores, m, dim, n_experts, s));
}
inline void moe_select(const float *scores, const float *bias, float *out_w, int32_t *out_i,
                       int64_t n_experts, int64_t top_k, float route_scale,
                       ws_stream_t s = nullptr) {
    check("moe_select", ws_moe_select(scores, bias, out_w, out_i, n_experts, top_k, route_scale, s));
}
inline void moe_route(const float *x, const uint16_t *gate_w, const float *bias, float *out_w,
                      int32_t *out_i, int64_t dim, int64_t n_experts, int64_t top_k,
                      float route_scale, ws_stream_t s = nullptr) {
    check("moe_route",
          ws_moe_route(x, gate_w, bias, out_w, out_i, dim, n_experts, top_k, route_scale, s));
}
inline void swiglu(const float *gate, const float *up, float *out, int64_t n, float rw,
                   ws_stream_t s = nullptr) {
    check("swiglu", ws_swiglu(gate, up, out, n, rw, s));
}

// routed experts, decode (launch.rs:89-206)
inline void expert_glu_quant(U8 act_x, U8 act_x_s, const int32_t *topk_idx, const float *topk_w,
                             U8 w1, U8 w1_s, U8 w3, U8 w3_s, uint8_t *q_slots, uint8_t *s_slots,
                             int64_t n, int64_t k, int64_t n_experts, int64_t top_k,
                             float swiglu_limit = 10.0f, ws_stream_t s = nullptr) {
    check("expert_glu_quant",
          ws_expert_glu_quant(act_x, act_x_s, topk_idx, topk_w, w1, w1_s, w3, w3_s, q_slots,
                              s_slots, k, n, n_experts, top_k, swiglu_limit, s));
}
inline void expert_reduce(U8 act_slots, U8 act_s_slots, U8 w2, U8 w2_s, const int32_t *gate_idx,
                          float *y, int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                          ws_stream_t s = nullptr) {
    check("expert_reduce", ws_expert_reduce(act_slots, act_s_slots, gate_idx, w2, w2_s, y, dim,
                                            inter, n_experts, top_k, s));
}

}  // namespace launch
}  // namespace weightstream_hip
