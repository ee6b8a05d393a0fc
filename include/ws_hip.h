/* weightstream-hip: C ABI of the MI355X (gfx950) quantized-matmul / MoE hot
 * path. Drop-in replacement for the kernel launches that weightstream-gpu's
 * launch.rs issues on weightstream-cuda today.
 *
 * Conventions (those of launch.rs, weightstream-gpu/src/launch.rs:1-33):
 *  - every pointer is a device pointer the caller owns; kernels never allocate
 *    (the fused MoE drivers take a caller workspace, sized by *_workspace_size);
 *  - every call is stream-ordered and asynchronous on `stream` (NULL = the
 *    default stream), like the `*_on` variants of launch.rs;
 *  - outputs are written in full, never accumulated into;
 *  - the return value is 0 on success, a hipError_t (1..999) if the launch
 *    failed, or one of the WS_ERR_* codes below if the arguments are rejected
 *    before anything is launched. launch.rs panics (`.unwrap()`) on failure;
 *    the host mirrors (include/ws_hip.hpp, weightstream_amd/launch.py) throw.
 *
 * Formats (weightstream-core/src/quant.rs:1-215): e4m3fn bytes; packed e2m1,
 * low nibble = even K; UE8M0 scale bytes 2^(b-127). Activations carry one
 * UE8M0 scale per 1x32 K block ([M, K/32]); FP8 weights one per 32x32 block
 * ([ceil(N/32), K/32]); FP4 weights one per row per 32 K ([N, K/32]).
 * Shapes: K must be a multiple of 128 and N a multiple of 16.
 */
#ifndef WS_HIP_H
#define WS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *ws_stream_t;

#define WS_OK 0
#define WS_ERR_INVALID_ARG 1001   /* null pointer or non-positive size */
#define WS_ERR_SHAPE 1002         /* shape outside what the kernels support */
#define WS_ERR_NO_DEVICE 1003     /* no gfx950 device */

/* Math modes of the GEMM-type kernels, fixed when the library is built (no
 * call changes the numerics of another). EXACT (libweightstream_hip.so):
 * FP8/FP4 operands are dequantised exactly to bf16 in registers and
 * multiplied with f32-accumulating bf16 MFMAs -- the reference's
 * dequantise-then-f32-accumulate product, rounding aside. NATIVE
 * (libweightstream_hip_native.so, same ABI): the CDNA4 FP8 / MXFP4 scaled
 * MFMAs, faster but their internal accumulation keeps about 13 bits
 * (relative error up to ~2^-12 of the sum of |products| per 128-K step). */
#define WS_MATH_EXACT 0
#define WS_MATH_NATIVE 1

/* Score functions of weightstream-ref moe.rs:29-42. */
#define WS_SCORE_SOFTMAX 0
#define WS_SCORE_SIGMOID 1
#define WS_SCORE_SQRTSOFTPLUS 2

/* ---------------------------------------------------------------------
 * Runtime. Replaces weightstream_cuda::gpu::Cuda::global() (gpu.rs:42-187):
 * code objects are linked in, so init only validates the device.
 * ------------------------------------------------------------------- */
/* Checks that the current device is gfx950. lib.rs:11-13 built_with_cuda(). */
int ws_init(void);
int ws_built_with_hip(void);
const char *ws_error_string(int code);
/* The math mode this library was built with (no reference counterpart:
 * weightstream-cuda has one precision). */
int ws_get_math_mode(void);
/* Device ws_expf over the 32-bit patterns [lo, lo+n): out[i] = bits(expf(x)).
 * Test hook for the exhaustive host/device expf agreement check. */
int ws_expf_probe(uint32_t lo, uint32_t n, uint32_t *out, ws_stream_t stream);
/* Device math over the 32-bit patterns [lo, lo+n): fn 0 out[i] =
 * bits(ws_logf(x)), fn 1 bits of the sqrtsoftplus score sqrt(softplus(x))
 * (num.rs:82-88, moe.rs:38-42), fn 2 the e4m3 byte of x (quant.rs:103-137),
 * fn 3 the UE8M0 scale byte of the FP8 activation quantisation of a block
 * whose largest magnitude is |x| (actquant.rs:21-45), fn 4 the f32 bits of
 * the value of x's e4m3 byte. Test hook for the
 * exhaustive host/device agreement checks; 0x7fbadbad marks an input where
 * the routing kernels' wave variant disagrees. */
int ws_math_probe(int fn, uint32_t lo, uint32_t n, uint32_t *out, ws_stream_t stream);

/* ---------------------------------------------------------------------
 * Activation quantisation (weightstream-cuda/kernels/actquant.cu).
 * ------------------------------------------------------------------- */
/* launch.rs:296-301 snap8 -> act_quant_ue8m0_snap: in-place FP8 snap of
 * f32 x[n], n % 32 == 0 (weightstream-ref actquant.rs:21 fp8_snap). */
int ws_snap8(float *x, int64_t n, ws_stream_t stream);
/* launch.rs:303-308 emit8 -> act_quant_fp8_emit: x[n] -> q[n] e4m3 and
 * s[n/32] UE8M0. Bit-exact with weightstream-ref's fp8 act quant. */
int ws_emit8(const float *x, uint8_t *q, uint8_t *s, int64_t n, ws_stream_t stream);
/* launch.rs:310-318 emit8_packed: as emit8, and also writes the scales again
 * at s + round_up(n/32, 16) (the packed-scale tail of the reference). */
int ws_emit8_packed(const float *x, uint8_t *q, uint8_t *s, int64_t n, ws_stream_t stream);
/* launch.rs:320-326 pack_scales -> pack_scale_words: four UE8M0 bytes per
 * little-endian u32 word, n/128 words. */
int ws_pack_scales(const uint8_t *src, uint32_t *dst, int64_t n, ws_stream_t stream);

/* Weight encoders (weightstream-ref store.rs:357-422, with the amax taken
 * over the whole block): f32 w[rows, cols] ->
 *  fp4: packed e2m1 q[rows, cols/2] + UE8M0 s[rows, cols/32] (amax floor
 *       6*2^-126, scale 2^log2_ceil(amax/6), clamp +-6);
 *  fp8: e4m3 q[rows, cols] + UE8M0 s[ceil(rows/32), cols/32] per 32x32 block
 *       (amax floor 1e-4, scale 2^log2_ceil(amax/448), clamp +-448). */
int ws_weight_quant_fp4(const float *w, uint8_t *q, uint8_t *s, int64_t rows, int64_t cols,
                        ws_stream_t stream);
int ws_weight_quant_fp8(const float *w, uint8_t *q, uint8_t *s, int64_t rows, int64_t cols,
                        ws_stream_t stream);

/* ---------------------------------------------------------------------
 * Block-scaled GEMM: C[M,N] = A[M,K] . B[N,K]^T, f32 accumulate.
 * One MFMA kernel family covers the reference's fp8_gemm (M=1 decode),
 * fp8_gemm_tile (M-batch) and the TileLang gemm_mxfp8 kernels.
 * ------------------------------------------------------------------- */
/* Split-K workspace of the FP8/FP4 GEMMs (no counterpart in the reference,
 * whose kernels keep the whole K of a tile in one block), registered per
 * (device, stream): GEMMs issued on `stream` (NULL = the default stream) of
 * the current device use the workspace registered for that stream, so GEMMs
 * on different streams never share one. With a workspace, GEMMs with M > 64
 * (and M <= 16 with few column strips and K > 8192) split K across
 * workgroups and a second kernel adds the f32 partials in split order
 * (deterministic); without one they use the single-pass kernels. Calls on one
 * stream are ordered by the stream, so they may share its workspace.
 * ws_gemm_workspace_size gives the bytes a shape needs; a smaller workspace
 * makes that shape use the single-pass kernel. Workspace NULL unregisters the
 * stream's; 256-byte aligned. The caller keeps the buffer alive while it is
 * registered. */
size_t ws_gemm_workspace_size(int64_t m, int64_t n, int64_t k);
int ws_set_gemm_workspace(void *workspace, size_t bytes, ws_stream_t stream);
/* launch.rs:717-742 fp8_gemm(_on) (fp8_gemm.cu:9): A e4m3 + sa[M,K/32],
 * B e4m3 + sb[ceil(N/32),K/32], C f32 [M,N]. */
int ws_fp8_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* No single reference counterpart: launch.rs:717-742 fp8_gemm (the
 * engine's gemm_q8 of wo_b, engine.rs:4008-4017) followed by launch.rs:1175
 * acc_f32 into the residual, in one launch: c += A.B^T with the add in the
 * GEMM's epilogue (c[i] + sum). Same operands as ws_fp8_gemm. It runs the
 * line and column-strip kernels only, never split over K: its bits are
 * those of ws_fp8_gemm + ws_acc_f32 wherever ws_fp8_gemm runs those too
 * (m <= 64, or K a multiple of 512 with m <= 128 and one round of tiles;
 * not where it splits K over a registered workspace or runs the split-K
 * pipeline's single pass). */
int ws_fp8_gemm_acc(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                    float *c, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* launch.rs:744-767 fp8_gemm_tile (fp8_gemm_tile.cu:28): same contract. */
int ws_fp8_gemm_tile(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* launch.rs:341-377 fp8_gemm_tl(_on) (TileLang gemm_mxfp8_kernel): the
 * shape comes from the TlGemm kind (WS_TL_*: (N, K) of engine.rs:3387-3398),
 * a e4m3 [m, K], sa the activation's packed scale words [m, K/128] (the
 * packed-word half that ws_emit8_packed writes at s + round_up(m*K/32, 16):
 * four UE8M0 bytes per word, so its bytes are the [m, K/32] scales), b e4m3
 * [N, K], sb the weight's upload-time packed table [N, K/128]
 * (engine.rs:842-853 pack_weight_scales: row r holds the words of its
 * 32-row block), out f32 [m, N]. */
#define WS_TL_QA 0                 /* (1280, 5120) */
#define WS_TL_QB 1                 /* (8192, 1280) */
#define WS_TL_WKV 2                /* (512, 5120) */
#define WS_TL_WO_A 3               /* (2048, 4096) */
#define WS_TL_WO_B 4               /* (5120, 2048) */
#define WS_TL_SHARED_W13 5         /* (2304, 5120) */
#define WS_TL_SHARED_W13_FUSED 6   /* (4608, 5120) */
#define WS_TL_SHARED_W2 7          /* (5120, 2304) */
#define WS_TL_ENGRAM_WKV 8         /* (25600, 5120) */
#define WS_TL_DRAFTER_MAIN_PROJ 9  /* (1280, 15360) */
int ws_tl_gemm_shape(int kind, int64_t *n, int64_t *k);
int ws_fp8_gemm_tl(int kind, const uint8_t *a, const uint32_t *sa, const uint8_t *b,
                   const uint32_t *sb, float *out, int64_t m, ws_stream_t stream);
/* fp8_gemm with bf16 output (RNE, quant.rs:95-101) instead of f32 (no
 * reference counterpart: BASELINE config 2's bf16-out GEMM). */
int ws_fp8_gemm_bf16(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     uint16_t *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* f32-scale block scheme (no reference counterpart; generalises fp8_gemm to
 * the 1xB activation / BxB weight f32 scales of DeepSeek-style checkpoints,
 * block = 128): sa f32 [M,K/128], sb f32 [ceil(N/128),K/128]. out_bf16 selects
 * bf16 (uint16_t*) instead of f32 output. */
int ws_fp8_gemm_f32s(const uint8_t *a, const float *sa, const uint8_t *b, const float *sb,
                     void *out, int out_bf16, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* Activation quantisation for the f32-scale scheme: per 1x128 block,
 * s = max(amax,1e-4)/448, q = e4m3(clamp(x/s, +-448)). */
int ws_act_quant_f32s(const float *x, uint8_t *q, float *s, int64_t m, int64_t k,
                      ws_stream_t stream);
/* launch.rs:769-779 fp4_gemm (fp4_expert_gemm.cu:9): A e4m3 + sa[M,K/32],
 * B packed e2m1 [N,K/2] + sb[N,K/32], C f32 [M,N]. */
int ws_fp4_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream);
/* launch.rs:781-804 fp4_gemm_tile (fp4_gemm_tile.cu:21): same contract. */
int ws_fp4_gemm_tile(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                     float *out, int64_t m, int64_t n, int64_t k, ws_stream_t stream);

/* ---------------------------------------------------------------------
 * MoE routing (weightstream-cuda/kernels/moe.cu; CPU: weightstream-ref
 * moe.rs:20-69). Selection and weights are bit-exact with the CPU path for
 * softmax and sigmoid (a shared expf, sequential-order dots and sums).
 * ------------------------------------------------------------------- */
/* Gate logits, num::gemv order (num.rs:18-28: one sequential dot per expert):
 * logits[M,E] = x[M,dim] . W[E,dim]^T, W f32 (w_bf16 = 0) or bf16. */
int ws_moe_gate_logits(const float *x, const void *gate_w, int w_bf16, float *logits,
                       int64_t m, int64_t dim, int64_t n_experts, ws_stream_t stream);
/* Scores + top-k + weights for M rows (moe.rs:24-69): scores = score_func(
 * logits / gate_temp); top-k of scores+bias by (value desc, index asc) under
 * f32 total order; weights = scores of the picks, / (sum + 1e-20) when
 * norm_topk_prob && top_k > 1, * route_scale. scores_out may be NULL.
 * E <= 1024, top_k <= 16. */
int ws_moe_topk(const float *logits, const float *bias, float *scores_out, int32_t *out_idx,
                float *out_w, int64_t m, int64_t n_experts, int64_t top_k, int score_func,
                float gate_temp, int norm_topk_prob, float route_scale, ws_stream_t stream);
/* launch.rs:998-1018 moe_gate (moe.cu:18): bf16 gate, sqrtsoftplus scores[E]
 * for one token (bias unused, as in the reference kernel). */
int ws_moe_gate(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                int64_t dim, int64_t n_experts, ws_stream_t stream);
/* launch.rs:1020-1041 moe_gate_m (moe.cu:160): M rows, scores[M,E]. */
int ws_moe_gate_m(const float *x, const uint16_t *gate_w, const float *bias, float *scores,
                  int64_t m, int64_t dim, int64_t n_experts, ws_stream_t stream);
/* launch.rs:1043-1066 moe_select (moe.cu:48): top-k of scores+bias, weights
 * normalised by (sum + 1e-20) and * route_scale. scores is not modified
 * (the reference kernel overwrites taken entries; callers must not rely on
 * either). */
int ws_moe_select(const float *scores, const float *bias, float *out_w, int32_t *out_idx,
                  int64_t n_experts, int64_t top_k, float route_scale, ws_stream_t stream);
/* launch.rs:1068-1093 moe_route (moe.cu:100): gate + select fused. */
int ws_moe_route(const float *x, const uint16_t *gate_w, const float *bias, float *out_w,
                 int32_t *out_idx, int64_t dim, int64_t n_experts, int64_t top_k,
                 float route_scale, ws_stream_t stream);
/* launch.rs:1095-1100 swiglu (moe.cu:143 swiglu_limit10):
 * out = silu(min(g,10)) * clamp(u,-10,10) * rw, in moe.rs:187-201's order. */
int ws_swiglu(const float *gate, const float *up, float *out, int64_t n, float rw,
              ws_stream_t stream);
/* launch.rs:1175-1179 acc_f32 (gemv.cu:63): y[i] += x[i] for i < n (both
 * 16-byte aligned). */
int ws_acc_f32(const float *x, float *y, int64_t n, ws_stream_t stream);
/* The shared FP8 expert of the MoE block: weightstream-ref moe.rs:210-250
 * (shared_expert_hidden), run on the device as the engine's moe_shared_step
 * (engine.rs:4063) does with emit8 + fp8_gemm + swiglu launches.
 * x [m, dim] f32; w1, w3 e4m3 [inter, dim] with UE8M0 [inter/32, dim/32];
 * w2 e4m3 [dim, inter] with UE8M0 [dim/32, inter/32]; y [m, dim] f32 (written,
 * not accumulated). h = silu(min(g, L)) * clamp(u, -L, L) with L =
 * swiglu_limit (<= 0: no clamps), quantised per 1x32 before the down GEMM.
 * dim and inter multiples of 128. The workspace (256-byte aligned, at least
 * ws_shared_expert_workspace_size bytes) holds the quantised token, g, u and
 * the quantised hidden state; the GEMMs use the registered split-K workspace
 * (ws_set_gemm_workspace) when there is one. */
size_t ws_shared_expert_workspace_size(int64_t m, int64_t dim, int64_t inter);
int ws_shared_expert_fp8(const float *x, const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                         const uint8_t *s3, const uint8_t *w2, const uint8_t *s2, float *y,
                         int64_t m, int64_t dim, int64_t inter, float swiglu_limit,
                         void *workspace, size_t workspace_bytes, ws_stream_t stream);
/* The shared expert with w1 and w3 fused row-wise into one FP8 matrix
 * w13 [2 * inter, dim] (rows 0..inter-1 = w1, inter.. = w3; UE8M0 scales
 * [2 * inter / 32, dim / 32]), as the engine loads it
 * (engine.rs:1520-1530 load_q8_combined_rows) and runs it (engine.rs:4067
 * moe_shared_step: one GEMM of N = 2 * inter, gate = its first inter
 * columns, up = the rest). Same workspace as ws_shared_expert_fp8. */
int ws_shared_expert_fp8_w13(const float *x, const uint8_t *w13, const uint8_t *s13,
                             const uint8_t *w2, const uint8_t *s2, float *y, int64_t m,
                             int64_t dim, int64_t inter, float swiglu_limit, void *workspace,
                             size_t workspace_bytes, ws_stream_t stream);

/* Fused block steps. No single reference counterpart: each replaces a
 * sequence of the reference's launches with one or two, same bits.
 *
 * ws_fp8_gemv_acc: h[m, n] += emit8(x) . w^T, i.e. launch.rs emit8 +
 * gemm_q8 (fp8_gemm, engine.rs:4000-4018 for wo_b) + acc_f32
 * (launch.rs:1175) in one launch: x [m, k] f32 is quantised per 1x32 inside
 * the kernel. w e4m3 [n, k] with UE8M0 [n/32, k/32]. m <= 16, k <= 8192,
 * k % 128 == 0, n % 16 == 0; x and h 16-byte aligned and not overlapping.
 * Every workgroup quantises all of x, so it pays for one or two rows (the
 * config-5 block at m = 8 is faster with the three separate launches). */
int ws_fp8_gemv_acc(const float *x, const uint8_t *w, const uint8_t *sw, float *h, int64_t m,
                    int64_t n, int64_t k, ws_stream_t stream);
/* ws_shared_expert_fp8_w13_acc: h = h + (yr + shared(x)), i.e.
 * ws_shared_expert_fp8_w13 into y, then acc_f32(y, yr) (engine.rs:4532:
 * y_moe += expert_y) and the residual add of y_moe into h, without writing
 * yr. For m <= 2 (dim, inter <= 8192) two launches: the gate/up GEMV with
 * the SwiGLU in its epilogue (h_s kept in f32 in the workspace), then the
 * down GEMV that quantises h_s per 1x32 and adds into h. Larger m: the
 * unfused sequence and one add kernel (each workgroup of the fused GEMVs
 * quantises the whole activation, which stops paying beyond a few rows).
 * Workspace as ws_shared_expert_fp8.
 * x may be h itself (it is read before h is written). */
int ws_shared_expert_fp8_w13_acc(const float *x, const uint8_t *w13, const uint8_t *s13,
                                 const uint8_t *w2, const uint8_t *s2, const float *yr, float *h,
                                 int64_t m, int64_t dim, int64_t inter, float swiglu_limit,
                                 void *workspace, size_t workspace_bytes, ws_stream_t stream);
/* The same split at the routed experts, for a decode step (m <= 8):
 * ws_moe_gate_shared_w13 computes, in one launch, the f32 gate logits
 * [m, n_experts] of h (ws_moe_gate_logits with f32 gate_w [n_experts, dim],
 * dim % 256 == 0, dim <= 8192: the same bits) and the shared expert's
 * hs [m, inter] = silu(min(g, L)) * clamp(u, -L, L) of g/u = emit8(h) . w13^T
 * (f32, not quantised); the two read h only. After the routed experts have
 * written yr, ws_shared_expert_down_acc quantises hs per 1x32 and does
 * h = h + (yr + emit8(hs) . w2^T). Together: the bits of
 * ws_moe_gate_logits + ws_shared_expert_fp8_w13_acc. hs is the caller's
 * f32 [m, inter] buffer (16-byte aligned). */
int ws_moe_gate_shared_w13(const float *h, const float *gate_w, float *logits,
                           const uint8_t *w13, const uint8_t *s13, float *hs, int64_t m,
                           int64_t dim, int64_t n_experts, int64_t inter, float swiglu_limit,
                           ws_stream_t stream);
int ws_shared_expert_down_acc(const float *hs, const uint8_t *w2, const uint8_t *s2,
                              const float *yr, float *h, int64_t m, int64_t dim, int64_t inter,
                              ws_stream_t stream);

/* ---------------------------------------------------------------------
 * Packed FP4 expert weights. The routed-expert entry points below read FP4
 * weight slabs in a fragment-major layout: 16-row bands, each 128-K step of a
 * band one contiguous 1 KB (MFMA lane order), scales grouped per lane and 8
 * steps. ws_prepack_fp4 converts the on-disk layout (packed e2m1 [rows,
 * cols/2], UE8M0 [rows, cols/32]; quant.rs:189-215) at upload, as the
 * reference engine re-tiles its expert slabs (engine.rs:842-884
 * pack_expert_scales / tile_major_expert, launch.rs:383-428 tensor maps).
 * rows % 16 == 0, cols % 128 == 0. Weight bytes keep their size
 * (rows*cols/2); scales take ws_packed_fp4_scale_bytes(rows, cols) bytes.
 * An expert slab [E, rows, cols] is E packed matrices back to back: pack
 * each expert (or pass rows = E*rows when every expert has `rows` % 16 == 0:
 * bands never straddle experts).
 * ------------------------------------------------------------------- */
size_t ws_packed_fp4_scale_bytes(int64_t rows, int64_t cols);
int ws_prepack_fp4(const uint8_t *w, const uint8_t *s, int64_t rows, int64_t cols, uint8_t *pw,
                   uint8_t *ps, ws_stream_t stream);

/* ---------------------------------------------------------------------
 * Routed experts, M = 1 decode (moe.rs:75-84,162-208; moe_grouped.cu:23-236).
 * Expert slabs (packed, see ws_prepack_fp4): w1/w3 [E, inter, dim] and
 * w2 [E, dim, inter]. The hidden state of a pick is stored in row `slot` of
 * hq [top_k, inter] / hs [top_k, inter/32] (slot = the pick's position in
 * the gate output), as the reference's expert_quant writes q_slots; the down
 * projection sums the picks in ascending expert id (then slot).
 * Shapes: dim % 128 == 0, inter % 128 == 0, dim <= 16384, top_k <= 16,
 * top_k * inter <= 32768; WS_ERR_SHAPE otherwise.
 * ------------------------------------------------------------------- */
/* launch.rs:89-112 moe_local_slots (moe_grouped.cu:23): the gate's picks
 * gate_idx[top_k] (global expert ids) that fall in [e_start, e_start+e_len),
 * sorted by ascending expert id (stable): local_slots[i] = their slot,
 * local_experts[i] = id - e_start, *local_count = how many. */
int ws_moe_local_slots(const int32_t *gate_idx, int32_t *local_slots, int32_t *local_experts,
                       int32_t *local_count, int64_t top_k, int64_t e_start, int64_t e_len,
                       ws_stream_t stream);
/* launch.rs:658-670 moe_dispatch_ids (moe_grouped.cu:226): dispatch_idx[s] =
 * gate_idx[s] - e_start if it falls in [e_start, e_start+e_len), else -1
 * (int64, the input of ws_moe_dispatch_tl). */
int ws_moe_dispatch_ids(const int32_t *gate_idx, int64_t *dispatch_idx, int64_t top_k,
                        int64_t e_start, int64_t e_len, ws_stream_t stream);
/* launch.rs:114-145 expert_glu (moe_grouped.cu:61): for local pick i <
 * *local_count, h_slots[local_slots[i], 0..n) = silu(min(w1.x, 10)) *
 * clamp(w3.x, -10, 10) * route_w[local_slots[i]] with w1/w3 = the slab rows of
 * local expert local_experts[i]; act_x / act_x_s the e4m3 token [k] and its
 * UE8M0 scales [k/32]. n = inter, k = dim. Trailing e_len (no counterpart:
 * the reference trusts local_experts) is the slab's expert count; a pick
 * outside it is skipped instead of read out of bounds. */
int ws_expert_glu(const uint8_t *act_x, const uint8_t *act_x_s, const uint8_t *w1,
                  const uint8_t *w1_s, const uint8_t *w3, const uint8_t *w3_s,
                  const float *route_w, const int32_t *local_slots,
                  const int32_t *local_experts, const int32_t *local_count, float *h_slots,
                  int64_t n, int64_t k, int64_t top_k, int64_t e_len, ws_stream_t stream);
/* launch.rs:147-166 expert_quant (moe_grouped.cu:128): the FP8 1x32 emit
 * (act_quant_fp8_emit) of each local slot's h row into q_slots [top_k, n] and
 * s_slots [top_k, n/32]. */
int ws_expert_quant(const float *h_slots, const int32_t *local_slots, const int32_t *local_count,
                    uint8_t *q_slots, uint8_t *s_slots, int64_t n, int64_t top_k,
                    ws_stream_t stream);
/* Fused expert_glu + expert_quant for the picks of the top-k output
 * (topk_idx / topk_w [top_k], top-k order; picks outside [0, E) are skipped,
 * as moe_local_slots drops another rank's experts): for each pick p
 * h = silu(min(w1.x,L)) * clamp(w3.x,+-L) * w_p, quantised FP8 1x32 into
 * row p of hq / hs. x is the quantised token (xq[dim], xs[dim/32], as
 * ws_emit8 writes). */
int ws_expert_glu_quant(const uint8_t *xq, const uint8_t *xs, const int32_t *topk_idx,
                        const float *topk_w, const uint8_t *w1, const uint8_t *s1,
                        const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                        int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                        float swiglu_limit, ws_stream_t stream);
/* As ws_expert_glu_quant with the activation quantisation (act_quant_fp8_emit,
 * actquant.cu:47) fused in: x is the f32 token [dim], dim <= 8192. */
int ws_expert_glu_quant_x(const float *x, const int32_t *topk_idx, const float *topk_w,
                          const uint8_t *w1, const uint8_t *s1, const uint8_t *w3,
                          const uint8_t *s3, uint8_t *hq, uint8_t *hs, int64_t dim, int64_t inter,
                          int64_t n_experts, int64_t top_k, float swiglu_limit,
                          ws_stream_t stream);
/* moe_select (launch.rs:1043, moe.cu:48) fused into ws_expert_glu_quant_x:
 * the gate/up kernel of ws_moe_decode_route on its own. Every workgroup
 * routes the token from logits[E] (+ bias, score_func sigmoid or
 * sqrtsoftplus, gate_temp, norm_topk_prob, route_scale as ws_moe_topk) and
 * writes hq/hs [top_k, inter] (+ [top_k, inter/32]) by pick slot; the picks
 * land in topk_idx / topk_w [top_k]. dim <= 8192, E <= 1024; softmax scores
 * are rejected (WS_ERR_INVALID_ARG: they need the sequential sum). */
int ws_expert_glu_quant_route(const float *logits, const float *bias, int score_func,
                              float gate_temp, int norm_topk_prob, float route_scale,
                              const float *x, const uint8_t *w1, const uint8_t *s1,
                              const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                              int32_t *topk_idx, float *topk_w, int64_t dim, int64_t inter,
                              int64_t n_experts, int64_t top_k, float swiglu_limit,
                              ws_stream_t stream);
/* launch.rs:178-206 expert_reduce (moe_grouped.cu:165): y[dim] = sum over the
 * local picks in local_slots order (ascending expert id) of w2_e . h_slot,
 * one f32 add per expert; e = gate_idx[slot] - e_start indexes the slab.
 * act_slots / act_s_slots are the e4m3 / UE8M0 rows by slot. Trailing e_len
 * as ws_expert_glu. */
int ws_expert_reduce(const uint8_t *act_slots, const uint8_t *act_s_slots, const uint8_t *w2,
                     const uint8_t *w2_s, const int32_t *gate_idx, const int32_t *local_slots,
                     const int32_t *local_count, float *y, int64_t dim, int64_t inter,
                     int64_t top_k, int64_t e_start, int64_t e_len, ws_stream_t stream);
/* Whole routed MoE for one token from f32 x: glu_quant_x -> reduce (two
 * kernels; hq/hs of the picks live in the workspace; for dim > 8192 the
 * token is quantised into the workspace by a third kernel first).
 * workspace >= ws_moe_decode_workspace_size(dim, inter, top_k) bytes. */
size_t ws_moe_decode_workspace_size(int64_t dim, int64_t inter, int64_t top_k);
int ws_moe_decode(const float *x, const int32_t *topk_idx, const float *topk_w,
                  const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                  const uint8_t *w2, const uint8_t *s2, float *y, int64_t dim, int64_t inter,
                  int64_t n_experts, int64_t top_k, float swiglu_limit, void *workspace,
                  size_t workspace_bytes, ws_stream_t stream);

/* moe_select (launch.rs:1043, moe.cu:48) fused with the routed MoE for one
 * token: top-k of the scores of logits[E] (score_func, gate_temp) + bias,
 * weights normalised as ws_moe_topk's norm_topk_prob says and scaled by
 * route_scale, written to topk_idx / topk_w [top_k] (top-k order, identical to
 * ws_moe_topk's), then ws_moe_decode's y. The gate/up kernel computes the
 * routing itself, so the step is two kernels. Softmax scores (a sequential
 * sum over E) and dim > 8192 run ws_moe_topk then ws_moe_decode. Workspace as
 * ws_moe_decode. */
int ws_moe_decode_route(const float *logits, const float *bias, int score_func, float gate_temp,
                        int norm_topk_prob, float route_scale, const float *x, const uint8_t *w1,
                        const uint8_t *s1, const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                        const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                        int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                        float swiglu_limit, void *workspace, size_t workspace_bytes,
                        ws_stream_t stream);
/* ws_moe_decode_route with the block's shared down projection and residual
 * add folded in (no single reference counterpart; it replaces
 * ws_moe_decode_route + ws_shared_expert_down_acc, the same bits): the
 * shared expert's down GEMV ys [dim] = emit8(hs_shared) . w2_shared^T runs on
 * extra workgroups of the routed gate/up launch (its weight stream joins the
 * routed one), and the routed down kernel ends with h = h + (y + ys). y is
 * written as by ws_moe_decode_route; hs_shared [shared_inter] is the f32
 * SwiGLU state ws_moe_gate_shared_w13 wrote; w2_shared e4m3 [dim,
 * shared_inter] with UE8M0 [dim/32, shared_inter/32]; ys [dim] f32 scratch
 * (16-byte aligned) of the caller. shared_inter % 128 == 0, <= 8192. Softmax
 * scores or dim > 8192 take the two separate calls. */
int ws_moe_decode_route_shared(const float *logits, const float *bias, int score_func,
                               float gate_temp, int norm_topk_prob, float route_scale,
                               const float *x, const uint8_t *w1, const uint8_t *s1,
                               const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                               const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                               int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                               float swiglu_limit, const float *hs_shared, const uint8_t *w2_shared,
                               const uint8_t *s2_shared, int64_t shared_inter, float *ys,
                               float *h, void *workspace, size_t workspace_bytes,
                               ws_stream_t stream);

/* ws_moe_decode_route with no workspace argument and no allocation. No
 * counterpart in the reference: for callers that cannot call hipMalloc or
 * hold a workspace (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). The workspace is a fixed device array
 * inside the library, 64 KiB per GPU, held until the process ends; it
 * covers every shape ws_moe_decode_route accepts (WS_ERR_SHAPE beyond).
 * Every call on one GPU shares that GPU's array: calls that may overlap on
 * one GPU (different streams, no ordering between them) race and must not be
 * issued; calls ordered on one stream are safe. Same results as
 * ws_moe_decode_route. */
int ws_moe_decode_route_noalloc(const float *logits, const float *bias, int score_func,
                                float gate_temp, int norm_topk_prob, float route_scale,
                                const float *x, const uint8_t *w1, const uint8_t *s1,
                                const uint8_t *w3, const uint8_t *s3, const uint8_t *w2,
                                const uint8_t *s2, float *y, int32_t *topk_idx, float *topk_w,
                                int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                                float swiglu_limit, ws_stream_t stream);

/* ---------------------------------------------------------------------
 * Routed experts, M tokens (grouped prefill / batched decode). Replaces the
 * TileLang pipeline of engine.rs:4125-4243 (moe_dispatch_tl launch.rs:430,
 * moe_grouped_tl(_cached)(_on) :478-580, moe_swiglu_route :673,
 * moe_combine_f32 :689). Routes r = token * top_k + j. Expert slabs are
 * packed (ws_prepack_fp4). Shapes: dim and inter multiples of 128, dim <=
 * 8192 (a 32-slot tile of x, or above 4096 a 16-slot half of it, is staged
 * in LDS), inter <= 4096; WS_ERR_SHAPE otherwise.
 * ------------------------------------------------------------------- */
/* Dispatch (moe_dispatch.cu:17): per-expert counts, 32-padded offsets in
 * ascending expert id (exclusive scan), psum = offset + count, order[slot] =
 * route or -1 (padding), layout_w[slot] = route weight or 0, route_pos[route]
 * = slot (-1 for an expert id outside [0,E)), tile_expert[t] = expert of
 * 32-slot tile t or -1, num_tiles[0] = used tiles. Inside an expert the routes
 * keep ascending route index. Slots >= tiles*32 are not written. This entry
 * takes int32 ids (as ws_moe_topk writes them); ws_moe_dispatch_tl below is
 * the reference's int64 form. */
int ws_moe_dispatch(const int32_t *topk_idx, const float *topk_w, int32_t *order,
                    float *layout_w, int32_t *route_pos, int32_t *tile_expert,
                    int32_t *expert_count, int32_t *expert_offset, int32_t *expert_psum,
                    int32_t *num_tiles, int64_t rows, int64_t top_k, int64_t tiles,
                    int64_t n_experts, ws_stream_t stream);
/* launch.rs:430-468 moe_dispatch_tl: the same with the int64 local ids that
 * ws_moe_dispatch_ids writes (-1 = not this rank's), in launch.rs's argument
 * order. Trailing n_experts (the TileLang kernel hard-codes its expert
 * count) bounds the ids. */
int ws_moe_dispatch_tl(const int64_t *topk_idx, const float *topk_weights, int32_t *order,
                       float *layout_weights, int32_t *route_pos, int32_t *tile_expert,
                       int32_t *expert_count, int32_t *expert_offset, int32_t *expert_psum,
                       int32_t *num_tiles, int64_t rows, int64_t top_k, int64_t tiles,
                       int64_t n_experts, ws_stream_t stream);
/* launch.rs:470-580 moe_grouped_tl(_cached)(_on) (TileLang
 * moe_grouped_fp8_fp4_gemm_kernel): out[slot, 0..n) f32 = A row . w_e^T for
 * every slot of every used tile (tile_expert[t] >= 0; e = tile_expert[t]),
 * K = k. kind GATE_UP: the A row of a slot is token order[slot] / top_k of
 * a [tokens, k] (one of w1 or w3 per call, as the engine issues them);
 * DOWN: the A row is row `slot` of a [tiles*32, k]. a is e4m3 with UE8M0
 * scales sfa [rows, k/32] (the packed-word half written by ws_emit8_packed
 * holds the same bytes, so either may be passed). weights / sfb are a packed
 * expert slab [n_experts, n, k] (ws_prepack_fp4) in place of the TMA
 * tensor map and its scale table. Rows of padding slots (order[slot] < 0)
 * are not written. The TlMoe enum's hard-coded shapes become n, k (k <=
 * 4096: the 32 x k A tile is staged in LDS) and the expert count n_experts. */
#define WS_TL_MOE_GATE_UP 0
#define WS_TL_MOE_DOWN 1
int ws_moe_grouped_tl(int kind, const uint8_t *a, const uint8_t *sfa, const uint8_t *weights,
                      const uint8_t *sfb, const int32_t *order, const int32_t *tile_expert,
                      float *out, int64_t tiles, int64_t tokens, int64_t top_k, int64_t n,
                      int64_t k, int64_t n_experts, ws_stream_t stream);
/* launch.rs:672-687 moe_swiglu_route (moe_grouped.cu:239): out[row, n] =
 * silu(min(gate,10)) * clamp(up,-10,10) * weights[row], or 0 where
 * weights[row] == 0; rows = tiles * 32 slots. out may alias gate. */
int ws_moe_swiglu_route(const float *gate, const float *up, const float *weights, float *out,
                        int64_t inter, int64_t rows, ws_stream_t stream);
/* Grouped gate/up (moe_grouped_tl GateUp) fused with moe_swiglu_route and the
 * FP8 emit: for every used tile, the 32 slots' tokens (xq [rows, dim] e4m3,
 * xs [rows, dim/32]) against the expert's w1/w3 rows; h = silu(min(g,L)) *
 * clamp(u,+-L) * layout_w[slot] quantised per 1x32 to hq [tiles*32, inter] +
 * hs [tiles*32, inter/32]; padding slots get h = 0. */
int ws_moe_grouped_glu_quant(const uint8_t *xq, const uint8_t *xs, const int32_t *order,
                             const float *layout_w, const int32_t *tile_expert,
                             const int32_t *num_tiles, const uint8_t *w1, const uint8_t *s1,
                             const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                             int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                             int64_t tiles, float swiglu_limit, ws_stream_t stream);
/* Grouped down (moe_grouped_tl Down): out [tiles*32, dim] f32 = hq . w2_e^T
 * for every used tile. */
int ws_moe_grouped_down(const uint8_t *hq, const uint8_t *hs, const int32_t *tile_expert,
                        const int32_t *num_tiles, const uint8_t *w2, const uint8_t *s2,
                        float *out, int64_t dim, int64_t inter, int64_t n_experts, int64_t tiles,
                        ws_stream_t stream);
/* launch.rs:689-703 moe_combine_f32 (moe_grouped.cu:260): out[row] = sum of
 * y[route_pos[row, j]] over the row's routes (slots outside [0, tiles*32)
 * skipped), added in ascending slot order, i.e. ascending expert id: the
 * reference CPU order of moe.rs:76-84 (the reference kernel adds in top-k
 * order). Trailing tiles (no counterpart) bounds the slots. */
int ws_moe_combine_f32(const float *y, const int32_t *route_pos, float *out, int64_t dim,
                       int64_t top_k, int64_t rows, int64_t tiles, ws_stream_t stream);
/* Whole routed MoE for `rows` tokens from f32 x [rows, dim] and routing
 * (topk_idx/topk_w [rows, top_k]): emit8 -> dispatch -> grouped glu_quant ->
 * grouped down -> combine into y [rows, dim]. tiles = ceil(rows*top_k/32) +
 * min(rows*top_k, E) (engine.rs:4131). workspace >=
 * ws_moe_prefill_workspace_size(rows, dim, inter, top_k, n_experts). */
size_t ws_moe_prefill_workspace_size(int64_t rows, int64_t dim, int64_t inter, int64_t top_k,
                                     int64_t n_experts);
int ws_moe_prefill(const float *x, const int32_t *topk_idx, const float *topk_w,
                   const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, float *y, int64_t rows, int64_t dim,
                   int64_t inter, int64_t n_experts, int64_t top_k, float swiglu_limit,
                   void *workspace, size_t workspace_bytes, ws_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
