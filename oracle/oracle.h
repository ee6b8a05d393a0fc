/* CPU oracle for weightstream's quantized-matmul / MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * CPU path (weightstream-core quant.rs, weightstream-ref actquant.rs, num.rs,
 * moe.rs) used as the parity checker for the HIP library. Only tests/, the
 * smoke() entry and bench.py's cpu_baseline leg may load it. The product
 * (libweightstream_hip.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates. Arithmetic is
 * f32 in the reference's order; the library is compiled with
 * -ffp-contract=off so no multiply-add is fused (Rust never fuses).
 *
 * Pinning status of each group is stated in oracle.c beside the group.
 */
#ifndef WS_ORACLE_H
#define WS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- core quant primitives (weightstream-core/src/quant.rs) ---- */
float    or_e4m3_to_f32(uint8_t b);
uint8_t  or_f32_to_e4m3(float v);
uint8_t  or_f32_to_e2m1(float v);
float    or_e8m0_to_f32(uint8_t b);
int32_t  or_log2_ceil(float x);
float    or_pow2i(int32_t e);
float    or_ue8m0_round_scale(float amax, float fp_max);
uint16_t or_f32_to_bf16(float v);
float    or_bf16_to_f32(uint16_t b);
float    or_fp4_value(uint8_t nibble);
uint8_t  or_pack_fp4(uint8_t even, uint8_t odd);
void     or_dequant_fp8_blockwise(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, float *out);
void     or_dequant_fp4_packed(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, float *out);

/* ---- activation quant (weightstream-ref/src/actquant.rs) ---- */
void or_fp8_snap(float *x, size_t n, size_t block);
void or_fp4_snap_e8m0(float *x, size_t n, size_t block);
void or_fp4_snap_e4m3(float *x, size_t n, size_t block);
/* Storage form of the same quantisation: e4m3 bytes + UE8M0 scale bytes per
 * 1x32 block (the format act_quant_fp8_emit writes, actquant.cu:47). */
void or_fp8_act_emit(const float *x, size_t n, uint8_t *q, uint8_t *s);

/* ---- GEMV/GEMM, reference scale format (actquant.rs:114-173) ---- */
/* y[rows] = W[rows,cols](e4m3, 32x32 UE8M0) . x (f32, quantised inside) */
/* threads for the GEMV row loops (default 1; results are the same for any count) */
void or_set_threads(int n);
/* exhaustive device checks (ws_math_probe fn 2, 3): reference bytes and their digest */
uint64_t or_probe_digest(int fn, uint64_t lo, uint64_t hi);
void or_probe_bytes(int fn, uint32_t lo, uint32_t n, uint32_t *out);
void or_fp8_gemv(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, const float *x, float *y);
/* y[rows] = W[rows,cols/2](packed e2m1, 1x32 UE8M0) . x */
void or_fp4_gemv(const uint8_t *w, const uint8_t *s, size_t rows, size_t cols, const float *x, float *y);
/* Same arithmetic with already-quantised activations (q,sa) for M rows:
 * Y[m, n] for m < M. `w_fp4` selects the weight format. */
void or_gemm_q(const uint8_t *aq, const uint8_t *as, size_t M,
               const uint8_t *w, const uint8_t *ws, size_t N, size_t K, int w_fp4, float *y);

/* ---- BASELINE generalisation: f32 scales, 1xB activation / BxB weight ---- */
void or_act_quant_f32s(const float *x, size_t M, size_t K, size_t block, uint8_t *q, float *s);
void or_weight_quant_fp8_f32s(const float *w, size_t N, size_t K, size_t block, uint8_t *q, float *s);
void or_gemm_f32s(const uint8_t *aq, const float *as, size_t M,
                  const uint8_t *w, const float *ws, size_t N, size_t K, size_t block, float *y);

/* ---- weight encoders (weightstream-ref/src/store.rs:357-422) ---- */
void or_weight_quant_fp8(const float *w, size_t rows, size_t cols, uint8_t *q, uint8_t *s);
void or_weight_quant_fp4(const float *w, size_t rows, size_t cols, uint8_t *q, uint8_t *s);

/* ---- numerics (weightstream-ref/src/num.rs) ---- */
float or_dot(const float *a, const float *b, size_t n);
void  or_gemv_f32(const float *w, size_t n, size_t k, const float *x, float *y);
float or_sigmoid(float x);
float or_silu(float x);
float or_softplus(float x);
void  or_softmax(float *x, size_t n);
float or_expf(float x);

/* ---- MoE (weightstream-ref/src/moe.rs) ---- */
enum { OR_SCORE_SOFTMAX = 0, OR_SCORE_SIGMOID = 1, OR_SCORE_SQRTSOFTPLUS = 2 };
/* scores[E] from logits[E]: gate_temp division then the score function */
void or_score(float *s, size_t n, int score_func, float gate_temp);
/* top-k on scores+bias (total_cmp desc, index asc), weights from the
 * unbiased scores, /(sum+1e-20) if norm && k>1, * route_scale */
void or_route(const float *scores, const float *bias, size_t n, size_t top_k,
              int norm_topk_prob, float route_scale, int32_t *idx, float *w);
/* one routed expert: fp4 gate/up, swiglu_limit clamps, *rw, fp4 down */
void or_expert_fp4(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, float rw, float limit, float *y);
/* shared expert: fp8 gate/up/down, no routing weight */
void or_expert_hidden_fp4(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                          const uint8_t *s3, size_t dim, size_t inter, const float *x, float rw,
                          float limit, float *h);
void or_shared_fp8(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, float limit, float *y);
/* routed sum for one token: experts in ascending id, slabs [E, ...] */
void or_moe_routed(const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, size_t dim, size_t inter,
                   const float *x, const int32_t *idx, const float *w, size_t top_k,
                   float limit, float *y);

/* ---- grouped dispatch (kernels/tilelang/moe_dispatch.cu semantics) ---- */
void or_dispatch(const int32_t *topk_idx, const float *topk_w, size_t routes, size_t n_experts,
                 size_t tiles, int32_t *order, float *layout_w, int32_t *route_pos,
                 int32_t *tile_expert, int32_t *count, int32_t *offset, int32_t *psum,
                 int32_t *num_tiles);

#ifdef __cplusplus
}
#endif
#endif
