// C++ host mirror of weightstream-gpu's launch.rs over the C ABI in ws_hip.h.
//
// Same names and argument order as weightstream-gpu/src/launch.rs; the `&Cuda`
// handle becomes a trailing stream argument (the `*_on` variants take it
// explicitly), and a failed launch throws weightstream_hip::Error where
// launch.rs panics through `.unwrap()`. Arguments that launch.rs does not have
// come last (slab extents that bound indices the reference trusts; the
// runtime (N, K) that replaces the TlMoe enum's hard-coded shapes).
// Header-only; link against libweightstream_hip.so (EXACT math) or
// libweightstream_hip_native.so (the same ABI with the CDNA4 scaled MFMAs).
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

// lib.rs:11-13 built_with_cuda()
inline bool built_with_hip() { return ws_built_with_hip() != 0; }

namespace launch {

using U8 = const uint8_t *;
using F32 = float *;
using I32 = int32_t *;

// ---- actquant.cu (launch.rs:296-326) ----------------------------------------
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

// ---- GEMMs (launch.rs:325-377, 717-804) ---------------------------------------
enum class TlGemm : int {
    Qa = WS_TL_QA,
    Qb = WS_TL_QB,
    Wkv = WS_TL_WKV,
    WoA = WS_TL_WO_A,
    WoB = WS_TL_WO_B,
    SharedW13 = WS_TL_SHARED_W13,
    SharedW13Fused = WS_TL_SHARED_W13_FUSED,
    SharedW2 = WS_TL_SHARED_W2,
    EngramWkv = WS_TL_ENGRAM_WKV,
    DrafterMainProj = WS_TL_DRAFTER_MAIN_PROJ,
};
inline void fp8_gemm_tl_on(TlGemm kind, U8 a, const uint32_t *sa, U8 b, const uint32_t *sb,
                           F32 out, int64_t m, ws_stream_t s) {
    check("fp8_gemm_tl", ws_fp8_gemm_tl((int)kind, a, sa, b, sb, out, m, s));
}
inline void fp8_gemm_tl(TlGemm kind, U8 a, const uint32_t *sa, U8 b, const uint32_t *sb, F32 out,
                        int64_t m) {
    fp8_gemm_tl_on(kind, a, sa, b, sb, out, m, Hip::global().stream);
}
inline void fp8_gemm_on(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                        ws_stream_t s) {
    check("fp8_gemm", ws_fp8_gemm(a, sa, b, sb, out, m, n, k, s));
}
inline void fp8_gemm(U8 a, U8 sa, U8 b, U8 sb, F32 out, int64_t m, int64_t n, int64_t k,
                     ws_stream_t s = nullptr) {
    fp8_gemm_on(a, sa, b, sb, out, m, n, k, s);
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
// split-K workspace of `s` (no counterpart: the reference has no split-K)
inline void set_gemm_workspace(void *ws, size_t bytes, ws_stream_t s = nullptr) {
    check("set_gemm_workspace", ws_set_gemm_workspace(ws, bytes, s));
}

// ---- routing (launch.rs:998-1100) ---------------------------------------------
inline void moe_gate(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                     int64_t dim, int64_t n_experts, ws_stream_t s = nullptr) {
    check("moe_gate", ws_moe_gate(x, gate_w, bias, scores, dim, n_experts, s));
}
inline void moe_gate_m(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                       int64_t m, int64_t dim, int64_t n_experts, ws_stream_t s = nullptr) {
    check("moe_gate_m", ws_moe_gate_m(x, gate_w, bias, scores, m, dim, n_experts, s));
}
inline void moe_select(const float *scores, const float *bias, float *out_w, I32 out_i,
                       int64_t n_experts, int64_t top_k, float route_scale,
                       ws_stream_t s = nullptr) {
    check("moe_select", ws_moe_select(scores, bias, out_w, out_i, n_experts, top_k, route_scale, s));
}
inline void moe_route(const float *x, const uint16_t *gate_w, const float *bias, float *out_w,
                      I32 out_i, int64_t dim, int64_t n_experts, int64_t top_k, float route_scale,
                      ws_stream_t s = nullptr) {
    check("moe_route",
          ws_moe_route(x, gate_w, bias, out_w, out_i, dim, n_experts, top_k, route_scale, s));
}
inline void swiglu(const float *gate, const float *up, float *out, int64_t n, float rw,
                   ws_stream_t s = nullptr) {
    check("swiglu", ws_swiglu(gate, up, out, n, rw, s));
}
// gemv.cu:63 (launch.rs:1175)
inline void acc_f32(const float *x, float *y, int64_t n, ws_stream_t s = nullptr) {
    check("acc_f32", ws_acc_f32(x, y, n, s));
}

// ---- routed experts, decode (launch.rs:87-206) ---------------------------------
inline void moe_local_slots(const int32_t *gate_idx, I32 local_slots, I32 local_experts,
                            I32 local_count, int64_t top_k, int64_t e_start, int64_t e_len,
                            ws_stream_t s = nullptr) {
    check("moe_local_slots", ws_moe_local_slots(gate_idx, local_slots, local_experts, local_count,
                                                top_k, e_start, e_len, s));
}
inline void expert_glu(U8 act_x, U8 act_x_s, U8 w1, U8 w1_s, U8 w3, U8 w3_s,
                       const float *route_w, const int32_t *local_slots,
                       const int32_t *local_experts, const int32_t *local_count, F32 h_slots,
                       int64_t n, int64_t k, int64_t top_k, int64_t e_len,
                       ws_stream_t s = nullptr) {
    check("expert_glu", ws_expert_glu(act_x, act_x_s, w1, w1_s, w3, w3_s, route_w, local_slots,
                                      local_experts, local_count, h_slots, n, k, top_k, e_len, s));
}
inline void expert_quant(const float *h_slots, const int32_t *local_slots,
                         const int32_t *local_count, uint8_t *q_slots, uint8_t *s_slots,
                         int64_t n, int64_t top_k, ws_stream_t s = nullptr) {
    check("expert_quant",
          ws_expert_quant(h_slots, local_slots, local_count, q_slots, s_slots, n, top_k, s));
}
inline void expert_reduce(U8 act_slots, U8 act_s_slots, U8 w2, U8 w2_s, const int32_t *gate_idx,
                          const int32_t *local_slots, const int32_t *local_count, F32 y,
                          int64_t dim, int64_t inter, int64_t top_k, int64_t e_start,
                          int64_t e_len, ws_stream_t s = nullptr) {
    check("expert_reduce", ws_expert_reduce(act_slots, act_s_slots, w2, w2_s, gate_idx,
                                            local_slots, local_count, y, dim, inter, top_k,
                                            e_start, e_len, s));
}
// expert_glu + expert_quant fused over the top-k output (rows by slot)
inline void expert_glu_quant(U8 act_x, U8 act_x_s, const int32_t *topk_idx, const float *topk_w,
                             U8 w1, U8 w1_s, U8 w3, U8 w3_s, uint8_t *q_slots, uint8_t *s_slots,
                             int64_t n, int64_t k, int64_t n_experts, int64_t top_k,
                             float swiglu_limit = 10.0f, ws_stream_t s = nullptr) {
    check("expert_glu_quant",
          ws_expert_glu_quant(act_x, act_x_s, topk_idx, topk_w, w1, w1_s, w3, w3_s, q_slots,
                              s_slots, k, n, n_experts, top_k, swiglu_limit, s));
}

// ---- routed experts, M tokens (launch.rs:430-703) -------------------------------
inline void moe_dispatch_ids(const int32_t *gate_idx, int64_t *dispatch_idx, int64_t top_k,
                             int64_t e_start, int64_t e_len, ws_stream_t s = nullptr) {
    check("moe_dispatch_ids", ws_moe_dispatch_ids(gate_idx, dispatch_idx, top_k, e_start, e_len, s));
}
inline void moe_dispatch_tl(const int64_t *topk_idx, const float *topk_weights, I32 order,
                            F32 layout_weights, I32 route_pos, I32 tile_expert, I32 expert_count,
                            I32 expert_offset, I32 expert_psum, I32 num_tiles, int64_t rows,
                            int64_t top_k, int64_t tiles, int64_t n_experts,
                            ws_stream_t s = nullptr) {
    check("moe_dispatch_tl",
          ws_moe_dispatch_tl(topk_idx, topk_weights, order, layout_weights, route_pos,
                             tile_expert, expert_count, expert_offset, expert_psum, num_tiles,
                             rows, top_k, tiles, n_experts, s));
}
enum class TlMoe : int { GateUp = WS_TL_MOE_GATE_UP, Down = WS_TL_MOE_DOWN };
// launch.rs:542: the stream follows top_k as there; n, k and n_experts (the
// slab's shape, which the reference reads from its tensor map) trail it
inline void moe_grouped_tl_cached_on(TlMoe kind, U8 a, U8 sfa, U8 weights, U8 sfb,
                                     const int32_t *order, const int32_t *tile_expert, F32 out,
                                     int64_t tiles, int64_t tokens, int64_t top_k, ws_stream_t s,
                                     int64_t n, int64_t k, int64_t n_experts) {
    check("moe_grouped_tl", ws_moe_grouped_tl((int)kind, a, sfa, weights, sfb, order, tile_expert,
                                              out, tiles, tokens, top_k, n, k, n_experts, s));
}
inline void moe_grouped_tl_cached(TlMoe kind, U8 a, U8 sfa, U8 weights, U8 sfb,
                                  const int32_t *order, const int32_t *tile_expert, F32 out,
                                  int64_t tiles, int64_t tokens, int64_t top_k, int64_t n,
                                  int64_t k, int64_t n_experts) {
    moe_grouped_tl_cached_on(kind, a, sfa, weights, sfb, order, tile_expert, out, tiles, tokens,
                             top_k, Hip::global().stream, n, k, n_experts);
}
// launch.rs:478 moe_grouped_tl: the weights as a packed slab (no tensor map)
inline void moe_grouped_tl(TlMoe kind, U8 a, U8 sfa, U8 weights, U8 sfb, const int32_t *order,
                           const int32_t *tile_expert, F32 out, int64_t tiles, int64_t tokens,
                           int64_t top_k, int64_t n, int64_t k, int64_t n_experts) {
    moe_grouped_tl_cached(kind, a, sfa, weights, sfb, order, tile_expert, out, tiles, tokens,
                          top_k, n, k, n_experts);
}
inline void moe_swiglu_route(const float *gate, const float *up, const float *weights, F32 out,
                             int64_t inter, int64_t rows, ws_stream_t s = nullptr) {
    check("moe_swiglu_route", ws_moe_swiglu_route(gate, up, weights, out, inter, rows, s));
}
inline void moe_combine_f32(const float *y, const int32_t *route_pos, F32 out, int64_t dim,
                            int64_t top_k, int64_t rows, int64_t tiles,
                            ws_stream_t s = nullptr) {
    check("moe_combine_f32", ws_moe_combine_f32(y, route_pos, out, dim, top_k, rows, tiles, s));
}

}  // namespace launch
}  // namespace weightstream_hip
