// Grouped (M-token) routed-expert MoE: dispatch, grouped gate/up + SwiGLU +
// FP8 re-quantisation, grouped down projection, ordered combine.
//
// Replaces the reference's TileLang pipeline moe_dispatch_kernel ->
// moe_grouped_fp8_fp4_gemm_kernel (gate/up) -> moe_swiglu_route ->
// emit8_packed -> moe_grouped_fp8_fp4_gemm_kernel (down) -> moe_combine_f32
// (weightstream-cuda/kernels/tilelang/moe_dispatch.cu:17, moe_gate_up.cu,
// moe_down.cu, moe_grouped.cu:239,260; launch.rs:430-689; engine.rs:4125-4243).
// The TileLang kernels hard-code 96 local experts, 512 routes, K=5120/2304;
// these kernels take E <= 1024 experts, any route count and any dim/inter that
// are multiples of 128. CPU semantics: weightstream-ref moe.rs:75-84,162-208
// per token.
//
// Layout: routes r = token * top_k + j. The dispatch places each expert's
// routes contiguously (ascending route index), padded to 32-slot tiles, the
// experts in ascending id. A tile is 32 slots of one expert, so its weight
// rows are streamed once for up to 32 tokens; the grouped kernels gather the
// tokens' FP8 rows (L2-resident) as the MFMA's A operand and stream the
// expert's FP4 rows as B. Tiles past the used count exit at once, so the grid
// is sized from the host-known upper bound and nothing is read back.
// Because slots ascend with expert id, the combine sums each token's expert
// outputs in ascending expert id, the reference CPU order.
#include "ws_internal.hpp"
#include "ws_pack.hpp"

namespace ws {

constexpr int kDispThreads = 1024;
constexpr int kMaxExpertsG = 1024;
constexpr int kTile = 32;
constexpr int kDispHeld = 4;  // route chunks the dispatch keeps in registers
constexpr int kEsGroup = 2;   // tiles of one expert whose weights the stationary body streams once

// The expert-stationary body streams a group's weights once for its (up to
// kEsGroup) tiles. It is taken when at least a sixth of the nt tiles share a
// group with another (ng groups; skewed routing), or when there are at least
// 96 tiles: measured with 384 experts (dim 4096, inter 2048) at M=132 and
// Zipf(0.25) (237-248 tiles) 620 against 670 us, at M=64 (~140 tiles) 383
// against 416 us; at M=8 (~51 tiles, one per expert) the two are even.
__host__ __device__ constexpr bool es_pays(int nt, int ng) {
    return 6 * (nt - ng) >= nt || nt >= 96;
}

// ---- dispatch (one workgroup) -------------------------------------------
// An expert id as the dispatch sees it: ids outside [0, E) (a pick another
// rank owns, -1 from moe_dispatch_ids) all become -1.
__device__ __forceinline__ int id_of(int32_t v, int n_experts) {
    return v >= 0 && v < n_experts ? v : -1;
}
__device__ __forceinline__ int id_of(int64_t v, int n_experts) {
    return v >= 0 && v < n_experts ? (int)v : -1;
}

template <typename IdxT>
__global__ __launch_bounds__(kDispThreads) void dispatch_kernel(
    const IdxT *__restrict__ idx, const float *__restrict__ wts, int32_t *__restrict__ order,
    float *__restrict__ layout_w, int32_t *__restrict__ route_pos,
    int32_t *__restrict__ tile_expert, int32_t *__restrict__ count_out,
    int32_t *__restrict__ offset_out, int32_t *__restrict__ psum_out,
    int32_t *__restrict__ num_tiles_out, int routes, int tiles, int n_experts,
    const float *__restrict__ xf, uint8_t *__restrict__ xq, uint8_t *__restrict__ xs, int64_t nx,
    uint16_t *__restrict__ xbf, int32_t *__restrict__ select_out) {
    if (blockIdx.x > 0) {
        // workgroups 1..: the tokens' FP8 1x32 quantisation (the act_quant
        // rule, a 32-lane half-wave per block; nx % 32 == 0), independent of
        // the dispatch and run beside it in the same launch; with xbf also
        // the exact bf16 of each quantised value (byte times block scale)
        const int64_t i = (int64_t)(blockIdx.x - 1) * kDispThreads + threadIdx.x;
        const bool live = i < nx;
        uint32_t sb;
        const uint32_t qb = quant_fp8_block32(live ? xf[i] : 0.0f, &sb);
        if (live) {
            xq[i] = (uint8_t)qb;
            if ((threadIdx.x & 31) == 0) xs[i / 32] = (uint8_t)sb;
            if (xbf)
                xbf[i] = (uint16_t)__builtin_bit_cast(
                    uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(qb, e8m0_to_f32(sb), false));
        }
        return;
    }
    __shared__ int32_t base[kMaxExpertsG];
    __shared__ int32_t wcnt[kDispThreads / 64][kMaxExpertsG];
    __shared__ int32_t scan[kMaxExpertsG];
    __shared__ int32_t wsum[kDispThreads / 64];
    __shared__ int32_t gsum[kDispThreads / 64];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    base[t] = 0;
    // the first kDispHeld chunks of routes are loaded once, up front (one
    // memory round trip), and kept in registers with their ranks for pass 2
    int e_h[kDispHeld], rk_h[kDispHeld];
    float w_h[kDispHeld];
#pragma unroll
    for (int h = 0; h < kDispHeld; h++) {
        const int r = h * kDispThreads + t;
        e_h[h] = r < routes ? id_of(idx[r], n_experts) : -1;
        w_h[h] = r < routes ? wts[r] : 0.0f;
        rk_h[h] = 0;
    }
    __syncthreads();
    // pass 1: stable rank of every route inside its expert (chunk by chunk,
    // in route order)
    auto rank_chunk = [&](int e) {
        const bool valid = e >= 0;
#pragma unroll
        for (int ww = 0; ww < kDispThreads / 64; ww++) wcnt[ww][t] = 0;
        __syncthreads();
        // the wave's lanes with the same expert: the AND over the id's bits
        // (n_experts <= 1024: 10 bits, and the sign for -1) of the ballot of
        // lanes that agree with this lane on that bit
        uint64_t same = ~0ull;
#pragma unroll
        for (int b = 0; b < 11; b++) {
            const int bit = b < 10 ? (e >> b) & 1 : e < 0;
            const uint64_t m = __ballot(bit);
            same &= bit ? m : ~m;
        }
        const int cnt = __popcll(same);
        const int inrank = __popcll(same & ((1ull << lane) - 1));
        if (valid && inrank == 0) wcnt[w][e] = cnt;
        __syncthreads();
        if (t < n_experts) {
            int run = base[t];
#pragma unroll
            for (int ww = 0; ww < kDispThreads / 64; ww++) {
                int v = wcnt[ww][t];
                wcnt[ww][t] = run;
                run += v;
            }
            base[t] = run;
        }
        __syncthreads();
        const int rank = valid ? wcnt[w][e] + inrank : -1;
        __syncthreads();
        return rank;
    };
#pragma unroll
    for (int h = 0; h < kDispHeld; h++)
        if (h * kDispThreads < routes) rk_h[h] = rank_chunk(e_h[h]);  // uniform
    for (int c0 = kDispHeld * kDispThreads; c0 < routes; c0 += kDispThreads) {
        const int r = c0 + t;
        const int rank = rank_chunk(r < routes ? id_of(idx[r], n_experts) : -1);
        if (rank >= 0) route_pos[r] = rank;
    }
    // exclusive scan of the 32-padded counts over experts
    const int count = t < n_experts ? base[t] : 0;
    const int padded = (count + kTile - 1) / kTile * kTile;
    int v = padded;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    int wbase = 0;
    for (int ww = 0; ww < w; ww++) wbase += wsum[ww];
    int total = 0;
    for (int ww = 0; ww < kDispThreads / 64; ww++) total += wsum[ww];
    const int offset = wbase + v - padded;
    scan[t] = offset;
    const int used = total / kTile;
    const int cap = tiles * kTile;
    if (t < n_experts) {
        count_out[t] = count;
        offset_out[t] = offset;
        psum_out[t] = offset + count;
    }
    if (t == 0) *num_tiles_out = used;
    if (select_out) {  // the prefill's choice of body (es_pays over the used tiles)
        int g = (padded / kTile + kEsGroup - 1) / kEsGroup;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) g += __shfl_xor(g, off, 64);
        if (lane == 0) gsum[w] = g;
        __syncthreads();
        if (t == 0) {
            int ng = 0;
            for (int ww = 0; ww < kDispThreads / 64; ww++) ng += gsum[ww];
            *select_out = es_pays(used, ng) ? 1 : 0;
        }
    }
    __syncthreads();
    // every used slot starts as padding (coalesced stores); pass 2
    // overwrites the slots that hold routes, after the barrier (which waits
    // for these stores to complete)
    for (int slot = t; slot < min(used * kTile, cap); slot += kDispThreads) {
        order[slot] = -1;
        layout_w[slot] = 0.0f;
    }
    if (t < n_experts)
        for (int tt = 0; tt < padded / kTile; tt++) {
            const int ti = offset / kTile + tt;
            if (ti < tiles) tile_expert[ti] = t;
        }
    for (int ti = used + t; ti < tiles; ti += kDispThreads) tile_expert[ti] = -1;
    __syncthreads();
    // pass 2: slots
    auto place = [&](int r, int e, int rank, float wr) {
        if (e < 0) {
            route_pos[r] = -1;
            return;
        }
        const int slot = scan[e] + rank;
        if (slot < cap) {
            order[slot] = r;
            layout_w[slot] = wr;
        }
        route_pos[r] = slot;
    };
#pragma unroll
    for (int h = 0; h < kDispHeld; h++) {
        const int r = h * kDispThreads + t;
        if (r < routes) place(r, e_h[h], rk_h[h], w_h[h]);
    }
    for (int r = kDispHeld * kDispThreads + t; r < routes; r += kDispThreads) {
        const int e = id_of(idx[r], n_experts);
        place(r, e, e >= 0 ? route_pos[r] : 0, wts[r]);
    }
}

// ---- grouped expert GEMM streaming ----------------------------------------
// Work unit = (ROWS-slot A block of a 32-slot tile, block of output columns).
// The grid has one workgroup per CU; workgroup i takes the contiguous units
// [i*U/G, (i+1)*U/G) of the U = used_tiles x (32/ROWS) x column_blocks units
// (the used tile count is read on the device, so every workgroup gets an
// equal share). Within a unit each wave streams one packed 16-row FP4 band of
// the tile's expert over its K range as a sequence of 8-step chunks held in
// two register stages: chunk q of the workgroup's run (unit q / nch, chunk
// q % nch) sits in stage q & 1, and chunk q + 2 is loaded as soon as chunk q
// is multiplied, so the weight stream runs on across chunks and units. The
// A block (ROWS token rows of x for gate/up, 32 slot rows of hq for down;
// FP8 + UE8M0) sits in LDS, copied with direct global->LDS loads whenever
// the workgroup moves to a new block. ROWS is 32, or 16 when a 32-row block
// of the K bytes would not fit in LDS (gate/up at dim > 4096; the 16-row
// halves of a tile then stream the weights once each).
constexpr int kGThreads = 512;  // 8 waves
constexpr int kGCols = 32;      // gate/up columns (intermediate rows) per unit

// A block of `rows` A rows into LDS, a_l[rows][K + 16] (the 16-byte pad
// spreads the rows of an MFMA fragment over the LDS banks) and their UE8M0
// bytes as_l[rows][K/32], with direct global->LDS loads
// (global_load_lds_dwordx4 / _dword: no VGPR staging). One instruction fills a
// contiguous 1 KB (256 B) of the LDS image; lane l moves the 16 (4) bytes at
// image offset o, which belong to row o / pitch (pad bytes repeat the row's
// last piece). Row i of A starts at arow(i), its scales at srow(i). Completion
// is awaited by the caller (vmcnt) before the barrier.
template <class ARow, class SRow>
__device__ __forceinline__ void g_dma_tile(ARow arow, SRow srow, int rows, int K, int w, int lane,
                                           uint8_t *a_l, uint8_t *as_l) {
    const int pitch = K + 16, total = rows * pitch;
    const int nq = (total + 1023) / 1024;  // the last piece overhangs into the image's slack
    for (int c = w; c < nq; c += kGThreads / 64) {
        const int o = min(c * 1024 + lane * 16, total - 16);
        const int row = o / pitch, col = min(o - row * pitch, K - 16);
        __builtin_amdgcn_global_load_lds((const void *)(arow(row) + col),
                                         (__attribute__((address_space(3))) void *)(a_l + c * 1024),
                                         16, 0, 0);
    }
    const int ks = K / 32, nsq = (rows * ks + 255) / 256;
    for (int c = w; c < nsq; c += kGThreads / 64) {
        const int o = min(c * 256 + lane * 4, rows * ks - 4);
        const int row = o / ks, col = o - row * ks;
        __builtin_amdgcn_global_load_lds((const void *)(srow(row) + col),
                                         (__attribute__((address_space(3))) void *)(as_l + c * 256),
                                         4, 0, 0);
    }
}

// Bytes of the A image (rounded up to whole 1 KB pieces) and of the whole
// LDS block (scales padded to whole 256-byte pieces)
__host__ __device__ constexpr size_t g_a_lds(int rows, int K) {
    return ((size_t)rows * (K + 16) + 1023) / 1024 * 1024;
}
__host__ __device__ constexpr size_t g_tile_lds(int rows, int K) {
    return g_a_lds(rows, K) + ((size_t)rows * (K / 32) + 255) / 256 * 256;
}

// The A block as exact bf16 (the e4m3 bytes times their UE8M0 scales, each
// value converted once when the block is staged instead of once per weight
// band that meets it): abf[rows][K] with a row pitch of 2K + 16 bytes (the
// pad spreads an MFMA fragment's 16 rows over the LDS banks).
__host__ __device__ constexpr size_t g_abf_lds(int rows, int K) {
    return (size_t)rows * (2 * K + 16);
}
// K bound of the bf16 block: 32 rows of it fit the 160 KB of LDS
constexpr int kAbfMaxK = 2304;

// Stage `rows` A rows (FP8 + UE8M0 per 1x32) into abf. Thread t converts
// 16-byte pieces t, t + kGThreads, ...: four pieces' loads are issued before
// their conversions. Row i of A starts at arow(i), its scales at srow(i).
// The caller orders the LDS writes before the reads with a barrier.
template <class ARow, class SRow>
__device__ __forceinline__ void g_stage_abf(ARow arow, SRow srow, int rows, int K, int t,
                                            uint8_t *abf) {
    const int per_row = K / 16, n = rows * per_row, pitch = 2 * K + 16;
    for (int i0 = t; i0 < n; i0 += 4 * kGThreads) {
        uint4 q[4];
        uint32_t sb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = min(i0 + j * kGThreads, n - 1);
            const int row = i / per_row, c = i - row * per_row;
            q[j] = *(const uint4 *)(arow(row) + c * 16);
            sb[j] = srow(row)[c >> 1];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = i0 + j * kGThreads;
            if (i >= n) break;
            const int row = i / per_row, c = i - row * per_row;
            const float sc = e8m0_to_f32(sb[j]);
            const uint32_t wq[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
            u32x4v o[2];
#pragma unroll
            for (int h = 0; h < 2; h++)
                o[h] = pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wq[2 * h], sc, false),
                           __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wq[2 * h], sc, true),
                           __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wq[2 * h + 1], sc, false),
                           __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wq[2 * h + 1], sc, true));
            u32x4v *dst = (u32x4v *)(abf + (size_t)row * pitch + c * 32);
            dst[0] = o[0];
            dst[1] = o[1];
        }
    }
}

// g_compute2 (EXACT) against a bf16 A block: the same MFMAs in the same
// order on the same bf16 operands, so the same sums bit for bit.
template <int NF>
__device__ __forceinline__ void g_compute2_abf(const Fp4Stage &s0, const Fp4Stage &s1,
                                               v4f acc[2][2], const uint8_t *abf, int K, int ks0,
                                               int kend, int lane) {
    const int r = lane & 15, g = lane >> 4, pitch = 2 * K + 16;
#pragma unroll
    for (int u = 0; u < kU; u++) {
        const int ks = ks0 + u;
        if (ks >= kend) continue;  // uniform
        const float f0 = e8m0_to_f32(stage_scale(s0, u)), f1 = e8m0_to_f32(stage_scale(s1, u));
        const uint32_t q0[4] = {s0.w[u].x, s0.w[u].y, s0.w[u].z, s0.w[u].w};
        const uint32_t q1[4] = {s1.w[u].x, s1.w[u].y, s1.w[u].z, s1.w[u].w};
        v8bf a[NF][4];
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const v8bf *ap = (const v8bf *)(abf + (size_t)(i * 16 + r) * pitch + ks * 256 + g * 64);
#pragma unroll
            for (int j = 0; j < 4; j++) a[i][j] = ap[j];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const v8bf b0 = __builtin_bit_cast(
                v8bf, pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 0),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 1),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 2),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 3)));
            const v8bf b1 = __builtin_bit_cast(
                v8bf, pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 0),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 1),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 2),
                          __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 3)));
#pragma unroll
            for (int i = 0; i < NF; i++) {
                acc[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][j], b0, acc[0][i], 0, 0, 0);
                acc[1][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i][j], b1, acc[1][i], 0, 0, 0);
            }
        }
    }
}

// g_compute (EXACT) against a bf16 A block, the same sums bit for bit.
template <int NF>
__device__ __forceinline__ void g_compute_abf(const Fp4Stage &st, v4f acc[NF], const uint8_t *abf,
                                              int K, int ks0, int kend, int lane) {
    const int r = lane & 15, g = lane >> 4, pitch = 2 * K + 16;
#pragma unroll
    for (int u = 0; u < kU; u++) {
        const int ks = ks0 + u;
        if (ks >= kend) continue;  // uniform
        v8bf bq[4];
        cvt_fp4x32(st.w[u], e8m0_to_f32(stage_scale(st, u)), bq);
#pragma unroll
        for (int i = 0; i < NF; i++) {
            const v8bf *ap = (const v8bf *)(abf + (size_t)(i * 16 + r) * pitch + ks * 256 + g * 64);
            const v8bf aq[4] = {ap[0], ap[1], ap[2], ap[3]};
            acc[i] = mfma_bf16_k128(aq, bq, acc[i]);
        }
    }
}

// Steps [ks0, kend) (at most kU) of a band, held in one stage, times the NF
// 16-slot A fragments in LDS (row stride K + 16 bytes, scales
// as_l[slot][K/32]). D[m][n]: slot 4*(lane/16)+v of fragment i, band row
// lane%16.
template <bool EXACT, int NF>
__device__ __forceinline__ void g_compute(const Fp4Stage &st, v4f acc[NF], const uint8_t *a_l,
                                          const uint8_t *as_l, int K, int ks0, int kend,
                                          int lane) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int u = 0; u < kU; u++) {
        const int ks = ks0 + u;
        if (ks >= kend) continue;  // uniform
        const uint32_t sbyte = stage_scale(st, u);
        if (EXACT) {
            v8bf bq[4];
            cvt_fp4x32(st.w[u], e8m0_to_f32(sbyte), bq);
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int slot = i * 16 + r;
                const uint8_t *ap = a_l + slot * (K + 16) + ks * 128 + g * 32;
                v8bf aq[4];
                cvt_fp8x32(*(const uint4 *)ap, *(const uint4 *)(ap + 16),
                           e8m0_to_f32(as_l[slot * (K / 32) + ks * 4 + g]), aq);
                acc[i] = mfma_bf16_k128(aq, bq, acc[i]);
            }
        } else {
            const v8i b = frag_from4(st.w[u]);
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int slot = i * 16 + r;
                const uint8_t *ap = a_l + slot * (K + 16) + ks * 128 + g * 16;
                acc[i] = mfma_scaled<kFmtFp8, kFmtFp4>(
                    frag_from(*(const uint4 *)ap, *(const uint4 *)(ap + 64)), b, acc[i],
                    (int)as_l[slot * (K / 32) + ks * 4 + g], (int)sbyte);
            }
        }
    }
}

// The same for two bands (s0, s1) against the same A fragments: each A
// fragment is converted once for both. Per band the MFMA sequence is that of
// g_compute (the same sums, bit for bit).
// (NF <= 2 fragments of acc[band][fragment] are used)
template <bool EXACT, int NF>
__device__ __forceinline__ void g_compute2(const Fp4Stage &s0, const Fp4Stage &s1,
                                           v4f acc[2][2], const uint8_t *a_l,
                                           const uint8_t *as_l, int K, int ks0, int kend,
                                           int lane) {
    const int r = lane & 15, g = lane >> 4;
#pragma unroll
    for (int u = 0; u < kU; u++) {
        const int ks = ks0 + u;
        if (ks >= kend) continue;  // uniform
        const uint32_t sb0 = stage_scale(s0, u), sb1 = stage_scale(s1, u);
        if (EXACT) {
            // one 8-value group j of the weights and of each A fragment at a
            // time (few registers live); per band and fragment the MFMAs run
            // in group order, as in mfma_bf16_k128
            const float f0 = e8m0_to_f32(sb0), f1 = e8m0_to_f32(sb1);
            const uint32_t q0[4] = {s0.w[u].x, s0.w[u].y, s0.w[u].z, s0.w[u].w};
            const uint32_t q1[4] = {s1.w[u].x, s1.w[u].y, s1.w[u].z, s1.w[u].w};
            uint4 alo[NF], ahi[NF];
            float sa[NF];
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int slot = i * 16 + r;
                const uint8_t *ap = a_l + slot * (K + 16) + ks * 128 + g * 32;
                alo[i] = *(const uint4 *)ap;
                ahi[i] = *(const uint4 *)(ap + 16);
                sa[i] = e8m0_to_f32(as_l[slot * (K / 32) + ks * 4 + g]);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const v8bf b0 = __builtin_bit_cast(
                    v8bf, pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 0),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 1),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 2),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q0[j], f0, 3)));
                const v8bf b1 = __builtin_bit_cast(
                    v8bf, pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 0),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 1),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 2),
                              __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q1[j], f1, 3)));
#pragma unroll
                for (int i = 0; i < NF; i++) {
                    const uint32_t wa[8] = {alo[i].x, alo[i].y, alo[i].z, alo[i].w,
                                            ahi[i].x, ahi[i].y, ahi[i].z, ahi[i].w};
                    const v8bf aj = __builtin_bit_cast(
                        v8bf, pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[2 * j], sa[i], false),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[2 * j], sa[i], true),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[2 * j + 1], sa[i], false),
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wa[2 * j + 1], sa[i], true)));
                    acc[0][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aj, b0, acc[0][i], 0, 0, 0);
                    acc[1][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aj, b1, acc[1][i], 0, 0, 0);
                }
            }
        } else {
            const v8i b0 = frag_from4(s0.w[u]), b1 = frag_from4(s1.w[u]);
#pragma unroll
            for (int i = 0; i < NF; i++) {
                const int slot = i * 16 + r;
                const uint8_t *ap = a_l + slot * (K + 16) + ks * 128 + g * 16;
                const v8i a = frag_from(*(const uint4 *)ap, *(const uint4 *)(ap + 64));
                const int sa = (int)as_l[slot * (K / 32) + ks * 4 + g];
                acc[0][i] = mfma_scaled<kFmtFp8, kFmtFp4>(a, b0, acc[0][i], sa, (int)sb0);
                acc[1][i] = mfma_scaled<kFmtFp8, kFmtFp4>(a, b1, acc[1][i], sa, (int)sb1);
            }
        }
    }
}

struct Fp4Pair {
    Fp4Stage h[2];
};

__device__ __forceinline__ int g_expert(const int32_t *tile_expert, int tile, int n_experts) {
    const int e = tile_expert[tile];
    return e < 0 ? 0 : (e >= n_experts ? n_experts - 1 : e);
}

// Logical workgroup index, XCD-major: the hardware deals workgroup b to XCD
// b % 8, so logical workgroups [j G/8, (j+1) G/8) all sit on XCD j. Units are
// shared out in contiguous runs by logical index, so the workgroups that take
// the tiles of one expert side by side (same column blocks at about the same
// time) share one L2: the expert's weights come from HBM once per XCD, not
// once per tile. Identity when G is not a multiple of 8.
__device__ __forceinline__ int g_logical_wg() {
    const int b = blockIdx.x, G = gridDim.x;
    return (G & 7) ? b : (b & 7) * (G >> 3) + (b >> 3);
}

// The workgroup's units [u0, u1) of the nb A blocks (H per tile) x NT column
// blocks; false when it has none. With the dispatch's per-expert offsets and
// counts, the units go out as expert runs: each block's NT column blocks are
// cut into k = G / nb runs of NT / k, one per workgroup, ordered (expert,
// column run, block) and dealt XCD-major. The workgroups that take one
// expert's blocks then sit side by side on one XCD and stream the same
// weight columns at the same time: the first read comes from HBM, the
// others from that XCD's L2 (tile-major order, below, streams an expert's
// weights once per tile, far apart in time). Each workgroup also keeps one A
// block. Runs are used for nb <= G / 2 blocks (measured: with one run per
// block, M=132 over ~240 experts, the contiguous share below ran 7% faster)
// while the longest run is within 1.5x of the even share.
// Otherwise (or without the offsets) workgroup i takes the contiguous units
// [i U / G, (i+1) U / G) of the U = nb NT, by logical index.
__device__ __forceinline__ bool g_share_units(int &u0, int &u1, int nb, int NT, int H,
                                              const int32_t *tile_expert, const int32_t *exp_off,
                                              const int32_t *exp_cnt, int n_experts) {
    const int G = gridDim.x, b = blockIdx.x;
    const long units = (long)nb * NT;
    const int k = nb > 0 ? min(NT, G / nb) : 0;
    const long mean = (units + G - 1) / G;
    if (exp_off && exp_cnt && (G & 7) == 0 && k >= 2 && 2L * ((NT + k - 1) / k) <= 3 * mean) {
        const int runs = nb * k, per = (runs + 7) >> 3;
        const int slot = b >> 3, i = (b & 7) * per + slot;
        if (slot >= per || i >= runs) return false;
        const int e = g_expert(tile_expert, (i / k) / H, n_experts);
        const int t0 = exp_off[e] / kTile;
        const int nbe = (exp_cnt[e] + kTile - 1) / kTile * H;  // the expert's blocks
        const int v = i - k * t0 * H;
        const int c = v / nbe, blk = t0 * H + v % nbe;
        u0 = blk * NT + c * NT / k;
        u1 = blk * NT + (c + 1) * NT / k;
        return u0 < u1;
    }
    const int lwg = g_logical_wg();
    u0 = (int)((long)lwg * units / G);
    u1 = (int)((long)(lwg + 1) * units / G);
    return u0 < u1;
}

// The experts of the tiles [tb0, tb0 + n) a workgroup's run touches, copied
// to LDS before the weight stream starts (no global load between its chunks).
constexpr int kExpCache = 64;
__device__ __forceinline__ bool g_cache_experts(int *tab, const int32_t *tile_expert, int tb0,
                                                int n, int n_experts, int t) {
    if (n > kExpCache) return false;  // uniform over the workgroup
    if (t < n) tab[t] = g_expert(tile_expert, tb0 + t, n_experts);
    return true;
}

// The chunk stream of one wave over the units [u0, u1): chunk q is unit
// u0 + q / nch, chunk q % nch, i.e. steps [k0 + 8c, min(k0 + 8c + 8, k1))
// of the wave's K range [k0, k1) (empty past k1; nch is the same for every
// wave of the workgroup, so all of them pass unit boundaries, and the
// barriers there, together). Loads past the last chunk repeat it.
struct ChunkStream {
    int u0, total, nch, k0, k1;
    __device__ __forceinline__ int unit(int q) const { return u0 + min(q, total - 1) / nch; }
    __device__ __forceinline__ int cb(int q) const { return k0 + (min(q, total - 1) % nch) * kU; }
    __device__ __forceinline__ int ce(int q) const { return min(cb(q) + kU, k1); }
};

// ---- grouped gate/up + SwiGLU + FP8 re-quantisation -----------------------
// Unit = (A block, 32 * CB intermediate columns nt), K part w>>2 (k_part8
// halves rounded to 8-step stages). CB == 1: wave w streams matrix (w>>1)&1
// (w1|w3), 16-row band w&1 of the unit. CB == 2: matrix w&1, both 16-row
// bands of 32-column block (w>>1)&1, each A fragment converted once for the
// two (half the A conversions per column; wider units, so for many tiles).
// The K parts meet in LDS (gu: part 0 stores, part 1 adds); then a half-wave
// per (slot row, 32-column block) applies SwiGLU, the routing weight and the
// FP8 1x32 quantisation (one block = 32 columns).
struct GluArgs {
    const uint8_t *xq, *xs;
    const int32_t *order;
    const float *layout_w;
    const int32_t *tile_expert, *num_tiles, *exp_off, *exp_cnt;
    const uint8_t *w1, *s1, *w3, *s3;
    uint8_t *hq, *hs;
    int dim, inter, n_experts, top_k;
    float limit;
};

template <bool EXACT, int ROWS, int CB>
__device__ __forceinline__ void grouped_glu_body(const GluArgs &ga, uint8_t *g_lds) {
    const uint8_t *xq = ga.xq, *xs = ga.xs;
    const int32_t *__restrict__ order = ga.order;
    const float *__restrict__ layout_w = ga.layout_w;
    const int32_t *__restrict__ tile_expert = ga.tile_expert;
    const int32_t *__restrict__ num_tiles = ga.num_tiles;
    const int32_t *__restrict__ exp_off = ga.exp_off;
    const int32_t *__restrict__ exp_cnt = ga.exp_cnt;
    const uint8_t *__restrict__ w1 = ga.w1, *__restrict__ s1 = ga.s1;
    const uint8_t *__restrict__ w3 = ga.w3, *__restrict__ s3 = ga.s3;
    uint8_t *__restrict__ hq = ga.hq;
    uint8_t *__restrict__ hs = ga.hs;
    const int dim = ga.dim, inter = ga.inter, n_experts = ga.n_experts, top_k = ga.top_k;
    const float limit = ga.limit;
    constexpr int NF = ROWS / 16, H = kTile / ROWS;
    uint8_t *a_l = g_lds;                              // [ROWS][dim + 16]
    uint8_t *as_l = g_lds + g_a_lds(ROWS, dim);        // [ROWS][dim/32] (+ padding)
    constexpr int UC = kGCols * CB;                   // columns per unit
    __shared__ float gu[2][ROWS][UC + 1];             // [matrix][slot row][column]
    __shared__ float rw_l[ROWS];  // routing weight of each slot of the block (0: padding)
    __shared__ int pad_l[ROWS];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const uint64_t tab = ws_lane_exp2f_tab(lane);
    const int r = lane & 15, g = lane >> 4;
    const int mat = CB == 2 ? (w & 1) : ((w >> 1) & 1), sub = CB == 2 ? ((w >> 1) & 1) : (w & 1);
    const int kpart = w >> 2;
    ChunkStream cs;
    k_part8(dim / 128, kpart, 2, cs.k0, cs.k1);
    cs.nch = ((dim / 128 + kU - 1) / kU + 1) / 2;  // chunks of the longer K part
    const int NT = inter / UC;
    int u1;
    if (!g_share_units(cs.u0, u1, *num_tiles * H, NT, H, tile_expert, exp_off, exp_cnt,
                       n_experts))
        return;  // whole workgroup
    cs.total = (u1 - cs.u0) * cs.nch;
    const size_t wmat = (size_t)inter * (dim / 2);
    const size_t smat = (size_t)packed_fp4_scale_bytes(inter, dim);
    const uint8_t *wm = mat ? w3 : w1;
    const uint8_t *sm = mat ? s3 : s1;
    // band h of the wave in unit u, and its first column within the unit
    __shared__ int exp_l[kExpCache];
    const int tb0 = cs.u0 / (H * NT);
    const bool cached = g_cache_experts(exp_l, tile_expert, tb0, (u1 - 1) / (H * NT) - tb0 + 1,
                                        n_experts, t);
    if (cached) lds_barrier();
    auto band_of = [&](int u, int h) {
        const int tb = u / (H * NT);
        const int e = cached ? exp_l[tb - tb0] : g_expert(tile_expert, tb, n_experts);
        return fp4_band(wm + (size_t)e * wmat, sm + (size_t)e * smat,
                        (u % NT) * 2 * CB + sub * CB + h, dim, lane);
    };
    auto load_q = [&](Fp4Pair &st, int q) {
        const int u = cs.unit(q);
#pragma unroll
        for (int h = 0; h < CB; h++) fp4_load(st.h[h], band_of(u, h), cs.cb(q), cs.ce(q));
    };
    Fp4Pair st0, st1;
    load_q(st0, 0);
    mem_order();
    load_q(st1, 1);
    mem_order();
    int cur_blk = -1;
    bool low_only = false;  // the block's slots 16.. are all padding (a 32-row block)
    v4f acc[2][2];  // [band][16-row fragment]
    auto step = [&](Fp4Pair &st, int q) {
        const int u = cs.unit(q), c = q % cs.nch;
        const int blk = u / NT, nt = u % NT;
        const int slot0 = (blk / H) * kTile + (blk % H) * ROWS;
        if (c == 0) {
            if (blk != cur_blk) {  // uniform: stage the block's token rows in LDS
                int my_tok = 0;
                bool padded = true;
                if (lane < ROWS) {
                    const int route = order[slot0 + lane];
                    my_tok = route >= 0 ? route / top_k : 0;
                    padded = route < 0;
                    if (w == 0) {
                        pad_l[lane] = route < 0;
                        rw_l[lane] = layout_w[slot0 + lane];
                    }
                }
                // only the rows that hold routes are copied and multiplied
                low_only = NF == 2 && (__ballot(!padded) >> 16) == 0;
                g_dma_tile([&](int i) { return xq + (size_t)__shfl(my_tok, i, 64) * dim; },
                           [&](int i) { return xs + (size_t)__shfl(my_tok, i, 64) * (dim / 32); },
                           low_only ? 16 : ROWS, dim, w, lane, a_l, as_l);
                __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed
                lds_barrier();
                cur_blk = blk;
            }
#pragma unroll
            for (int h = 0; h < 2; h++) acc[h][0] = acc[h][1] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        // uniform; with low_only the upper fragment's sums stay 0 (padding slots)
        if (CB == 2) {
            if (low_only)
                g_compute2<EXACT, 1>(st.h[0], st.h[1], acc, a_l, as_l, dim, cs.cb(q), cs.ce(q), lane);
            else
                g_compute2<EXACT, NF>(st.h[0], st.h[1], acc, a_l, as_l, dim, cs.cb(q), cs.ce(q), lane);
        } else {
            if (low_only)
                g_compute<EXACT, 1>(st.h[0], acc[0], a_l, as_l, dim, cs.cb(q), cs.ce(q), lane);
            else
                g_compute<EXACT, NF>(st.h[0], acc[0], a_l, as_l, dim, cs.cb(q), cs.ce(q), lane);
        }
        load_q(st, q + 2);
        if (c == cs.nch - 1) {  // the unit's K parts are complete: epilogue
            // K part 0 stores, part 1 adds (the sum p0 + p1)
#pragma unroll
            for (int kp = 0; kp < 2; kp++) {
                if (kpart == kp) {  // uniform
#pragma unroll
                    for (int h = 0; h < CB; h++)
#pragma unroll
                        for (int i = 0; i < NF; i++)
#pragma unroll
                            for (int v = 0; v < 4; v++) {
                                float &o = gu[mat][i * 16 + 4 * g + v][(sub * CB + h) * 16 + r];
                                o = kp == 0 ? acc[h][i][v] : o + acc[h][i][v];
                            }
                }
                lds_barrier();
            }
            // a half-wave per (slot row, 32-column block): one FP8 block
            const int col = t & 31;
            for (int it = t >> 5; it < CB * ROWS; it += kGThreads / 32) {
                const int srow = it / CB, cbk = it % CB;
                const int slot = slot0 + srow;
                const bool pad = pad_l[srow] != 0;
                float gv = gu[0][srow][cbk * 32 + col];
                float uv = gu[1][srow][cbk * 32 + col];
                if (limit > 0.0f) {
                    uv = rclamp(uv, -limit, limit);
                    gv = fminf(gv, limit);
                }
                // a padding row (uniform over the half-wave) is a block of
                // zeros: no silu, the zero block's bytes
                uint32_t sbyte = zero_block_scale_byte(), qb = 0;
                if (!pad) {
                    const float h = ws_silu_lanes(gv, tab) * uv * rw_l[srow];
                    qb = quant_fp8_block32(h, &sbyte);
                }
                hq[(size_t)slot * inter + nt * UC + cbk * 32 + col] = (uint8_t)qb;
                if (col == 0) hs[(size_t)slot * (inter / 32) + nt * CB + cbk] = (uint8_t)sbyte;
            }
            lds_barrier();
        }
    };
    int q = 0;
    for (; q + 1 < cs.total; q += 2) {
        step(st0, q);
        step(st1, q + 1);
    }
    if (q < cs.total) step(st0, q);
}

template <bool EXACT, int ROWS, int CB>
__global__ __launch_bounds__(kGThreads) void grouped_glu_quant_kernel(GluArgs ga) {
    extern __shared__ __align__(16) uint8_t g_lds[];
    grouped_glu_body<EXACT, ROWS, CB>(ga, g_lds);
}

// ---- grouped down ---------------------------------------------------------
// Unit = (tile, 128 * CB output columns nt); wave w owns the CB 16-column
// bands from nt*128*CB + 16*CB*w over the whole K = inter (chunk stream of
// 8-step chunks; with CB == 2 each A fragment is converted once for both
// bands), so each output is one wave's sum and is written straight from
// registers. f32 out[slot, dim]. With CB == 2 and dim % 256 == 128 the last
// unit's upper waves have no band (clamped loads, no stores).
//
// GATHER (the gate/up form of moe_grouped_tl): the A rows are the tokens of
// the tile's routes, row order[slot] / top_k of hq (< tokens), instead of the
// slot rows. num_tiles == nullptr: the used tiles are counted from
// tile_expert (the dispatch puts them first, the rest hold -1), as a caller
// of the reference's grouped GEMM passes no count.
// ABF (EXACT, inter <= kAbfMaxK): the A block is staged as bf16 (g_stage_abf)
// and the waves convert only their weights.
struct DownArgs {
    const uint8_t *hq, *hs;
    const int32_t *tile_expert, *num_tiles, *exp_off, *exp_cnt, *order;
    const uint8_t *w2, *s2;
    float *out;
    int dim, inter, n_experts, tiles, top_k, tokens;
};

template <bool EXACT, int CB, bool GATHER = false, bool ABF = false>
__device__ __forceinline__ void grouped_down_body(const DownArgs &da, uint8_t *g_lds) {
    const uint8_t *hq = da.hq, *hs = da.hs;
    const int32_t *__restrict__ tile_expert = da.tile_expert;
    const int32_t *__restrict__ num_tiles = da.num_tiles;
    const int32_t *__restrict__ exp_off = da.exp_off;
    const int32_t *__restrict__ exp_cnt = da.exp_cnt;
    const int32_t *__restrict__ order = da.order;
    const uint8_t *__restrict__ w2 = da.w2, *__restrict__ s2 = da.s2;
    float *__restrict__ out = da.out;
    const int dim = da.dim, inter = da.inter, n_experts = da.n_experts, tiles = da.tiles,
              top_k = da.top_k, tokens = da.tokens;
    static_assert(!ABF || EXACT, "the bf16 A block serves the exact math");
    uint8_t *a_l = g_lds;                                // [32][inter + 16] (ABF: abf)
    uint8_t *as_l = g_lds + g_a_lds(kTile, inter);      // [32][inter/32] (+ padding)
    __shared__ int row_l[kTile];                         // ABF: the A row of each slot
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int r = lane & 15, g = lane >> 4;
    ChunkStream cs;
    cs.k0 = 0;
    cs.k1 = inter / 128;
    cs.nch = (cs.k1 + kU - 1) / kU;
    const int NT = (dim + 128 * CB - 1) / (128 * CB), nbands = dim / 16;
    int used;
    if (num_tiles) {
        used = *num_tiles;
    } else {
        used = 0;
        for (int c = 0; c < tiles; c += 64) {
            const bool u = c + lane < tiles && tile_expert[min(c + lane, tiles - 1)] >= 0;
            used += __popcll(__ballot(u));
        }
    }
    int u1;
    if (!g_share_units(cs.u0, u1, used, NT, 1, tile_expert, exp_off, exp_cnt, n_experts))
        return;  // whole workgroup
    cs.total = (u1 - cs.u0) * cs.nch;
    const size_t wmat = (size_t)dim * (inter / 2);
    const size_t smat = (size_t)packed_fp4_scale_bytes(dim, inter);
    __shared__ int exp_l[kExpCache];
    const int tb0 = cs.u0 / NT;
    const bool cached =
        g_cache_experts(exp_l, tile_expert, tb0, (u1 - 1) / NT - tb0 + 1, n_experts, t);
    if (cached) lds_barrier();
    auto band_of = [&](int u, int h) {
        const int tb = u / NT;
        const int e = cached ? exp_l[tb - tb0] : g_expert(tile_expert, tb, n_experts);
        return fp4_band(w2 + (size_t)e * wmat, s2 + (size_t)e * smat,
                        min((u % NT) * 8 * CB + w * CB + h, nbands - 1), inter, lane);
    };
    auto load_q = [&](Fp4Pair &st, int q) {
        const int u = cs.unit(q);
#pragma unroll
        for (int h = 0; h < CB; h++) fp4_load(st.h[h], band_of(u, h), cs.cb(q), cs.ce(q));
    };
    Fp4Pair s0, s1;
    load_q(s0, 0);
    mem_order();
    load_q(s1, 1);
    mem_order();
    int cur_tile = -1;
    // with `order`: the tile's slots that hold routes (bit i: slot i); only
    // those rows are written, and a tile whose slots 16.. are all padding
    // copies and multiplies 16 rows. Without it every slot counts.
    uint32_t real = 0xFFFFFFFFu;
    v4f acc[2][2];  // [band][16-row fragment]
    auto step = [&](Fp4Pair &st, int q) {
        const int u = cs.unit(q), c = q % cs.nch;
        const int tile = u / NT, nt = u % NT;
        const int slot0 = tile * kTile;
        if (c == 0) {
            if (tile != cur_tile) {  // uniform: stage the tile's hq rows in LDS
                int my_row = 0;
                if (order) {
                    const int route = order[slot0 + min(lane, kTile - 1)];
                    const bool has = lane < kTile && route >= 0;
                    real = (uint32_t)__ballot(has);
                    if (GATHER) my_row = has ? min(route / top_k, tokens - 1) : 0;
                }
                if (ABF && w == 0 && lane < kTile) row_l[lane] = GATHER ? my_row : slot0 + lane;
                lds_barrier();       // every wave is done with the previous tile
                if (ABF)
                    g_stage_abf([&](int i) { return hq + (size_t)row_l[i] * inter; },
                                [&](int i) { return hs + (size_t)row_l[i] * (inter / 32); },
                                (real >> 16) == 0 ? 16 : kTile, inter, t, a_l);
                else if (GATHER)
                    g_dma_tile([&](int i) { return hq + (size_t)__shfl(my_row, i, 64) * inter; },
                               [&](int i) {
                                   return hs + (size_t)__shfl(my_row, i, 64) * (inter / 32);
                               },
                               (real >> 16) == 0 ? 16 : kTile, inter, w, lane, a_l, as_l);
                else
                    g_dma_tile([&](int i) { return hq + (size_t)(slot0 + i) * inter; },
                               [&](int i) { return hs + (size_t)(slot0 + i) * (inter / 32); },
                               (real >> 16) == 0 ? 16 : kTile, inter, w, lane, a_l, as_l);
                if (!ABF) __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed
                lds_barrier();
                cur_tile = tile;
            }
#pragma unroll
            for (int h = 0; h < 2; h++) acc[h][0] = acc[h][1] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        const bool lo16 = (real >> 16) == 0;  // uniform
        if (ABF && CB == 2) {
            if (lo16)
                g_compute2_abf<1>(st.h[0], st.h[1], acc, a_l, inter, cs.cb(q), cs.ce(q), lane);
            else
                g_compute2_abf<2>(st.h[0], st.h[1], acc, a_l, inter, cs.cb(q), cs.ce(q), lane);
        } else if (ABF) {
            if (lo16)
                g_compute_abf<1>(st.h[0], acc[0], a_l, inter, cs.cb(q), cs.ce(q), lane);
            else
                g_compute_abf<2>(st.h[0], acc[0], a_l, inter, cs.cb(q), cs.ce(q), lane);
        } else if (CB == 2) {
            if (lo16)
                g_compute2<EXACT, 1>(st.h[0], st.h[1], acc, a_l, as_l, inter, cs.cb(q), cs.ce(q), lane);
            else
                g_compute2<EXACT, 2>(st.h[0], st.h[1], acc, a_l, as_l, inter, cs.cb(q), cs.ce(q), lane);
        } else {
            if (lo16)
                g_compute<EXACT, 1>(st.h[0], acc[0], a_l, as_l, inter, cs.cb(q), cs.ce(q), lane);
            else
                g_compute<EXACT, 2>(st.h[0], acc[0], a_l, as_l, inter, cs.cb(q), cs.ce(q), lane);
        }
        load_q(st, q + 2);
        const int b0 = nt * 8 * CB + w * CB;
        if (c == cs.nch - 1 && b0 < nbands) {  // uniform
#pragma unroll
            for (int h = 0; h < CB; h++) {
                const int col = (b0 + h) * 16 + r;
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        const int row = i * 16 + 4 * g + v;
                        if ((real >> row) & 1) out[(size_t)(slot0 + row) * dim + col] = acc[h][i][v];
                    }
            }
        }
    };
    int q = 0;
    for (; q + 1 < cs.total; q += 2) {
        step(s0, q);
        step(s1, q + 1);
    }
    if (q < cs.total) step(s0, q);
}

template <bool EXACT, int CB, bool GATHER = false, bool ABF = false>
__global__ __launch_bounds__(kGThreads) void grouped_down_kernel(DownArgs da) {
    extern __shared__ __align__(16) uint8_t g_lds[];
    grouped_down_body<EXACT, CB, GATHER, ABF>(da, g_lds);
}

// ---- expert-stationary grouped GEMM (exact math, ws_moe_prefill) --------
// The tile-streaming kernels above read an expert's weights once per tile.
// Here a workgroup takes a unit = (group, column block): a group is a run of
// up to kTG consecutive tiles of one expert, and every weight byte of the
// column block is loaded and converted once and multiplied into all the
// group's tiles. The A rows arrive as exact bf16 (the e4m3 bytes times their
// UE8M0 scales, written once by the step before) through direct global->LDS
// loads into a ring of kRing 128-K steps, so the waves convert only weights.
// Eight waves, two per SIMD; wave w owns two 16-row bands over the whole K:
// gate/up the w1 and the w3 bands of intermediate columns 16w .. 16w + 15
// of a 128-column block (a row's FP8 1x32 block spans wave w and its partner
// w ^ 1, which trade their maxima through LDS), down output columns
// 32w .. 32w + 31 of a 256-column block. The workgroup's steps form one
// stream across its units: the loads of step q + kAhead are issued while
// step q is multiplied, with one workgroup barrier per two steps (at an even
// step each wave waits for its copies of steps q and q + 1, then the
// barrier; the ring slot the next issues fill, that of step
// q + kAhead - kRing <= q - 2, was read before the last barrier). A step
// issues two weight loads and one copy per tile of its group, and every
// fourth step a block of scale words; the waves keep the tile counts of the
// steps in flight, so the count of newer loads (vmcnt) says when a step's
// copies have landed. Every global access goes through a buffer
// descriptor sized to its array (out-of-range reads return zeros, writes are
// dropped). Units go out sorted by group size and dealt to the workgroups in
// snake order, which evens out the work per workgroup.
namespace es {
constexpr int kTG = kEsGroup;                 // tiles per group
constexpr int kRing = 8;                      // ring slots (LDS and registers), one 128-K step each
constexpr int kRowB = 256;                    // bytes of one A row per step (128 bf16)
constexpr int kSlotB = kTG * kTile * kRowB;   // 16 KB per ring slot
constexpr int kMaxGroups = 1024;
constexpr int kThreads = 512;                 // 8 waves: two per SIMD
static_assert(kThreads == kGThreads, "the select kernels run both bodies in one workgroup");
constexpr size_t kLds = (size_t)kRing * kSlotB;
constexpr size_t kLdsAll = kLds + 2 * kMaxGroups * sizeof(int);  // ring + group table
}  // namespace es

typedef __amdgpu_buffer_rsrc_t es_rsrc;
typedef unsigned int es_u2 __attribute__((ext_vector_type(2)));
// raw buffer of `bytes` bytes at p (gfx9 descriptor word 3)
__device__ __forceinline__ es_rsrc es_buf(const void *p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(uint32_t)min(bytes, (size_t)0xFFFFFFFFu),
                                             0x00020000);
}
__device__ __forceinline__ void es_dma(es_rsrc r, uint32_t off, uint32_t lds, int bytes) {
    auto *l = (__attribute__((address_space(3))) void *)(uintptr_t)lds;
    if (bytes == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, off, 0, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, off, 0, 0, 0);
}
template <int N>
__device__ __forceinline__ void es_vmcnt() {
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// s_waitcnt vmcnt(n) for a wave-uniform run-time n in [LO, HI]
template <int LO, int HI>
__device__ __forceinline__ void es_wait_vm(int n) {
    if constexpr (LO == HI) {
        es_vmcnt<LO>();
    } else {
        constexpr int MID = (LO + HI) / 2;
        if (n <= MID) es_wait_vm<LO, MID>(n);
        else es_wait_vm<MID + 1, HI>(n);
    }
}
// An LDS word, complete when the statement ends (no ordinary LDS access, so
// the compiler does not wait for the stream's direct-to-LDS copies).
__device__ __forceinline__ int es_lds_word(const int *p) {
    int v;
    __asm__ volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}
// One 16-row A fragment of one tile and step, 4 x 16 bytes: reads at a[jj]
// + OFF, complete when the statement ends.
template <int OFF>
__device__ __forceinline__ void es_lds_frag(const uint32_t a[4], u32x4v o[4]) {
    __asm__ volatile(
        "ds_read_b128 %0, %4 offset:%8\n\tds_read_b128 %1, %5 offset:%8\n\t"
        "ds_read_b128 %2, %6 offset:%8\n\tds_read_b128 %3, %7 offset:%8\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3])
        : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "n"(OFF)
        : "memory");
}

struct EsArgs {
    const uint8_t *abf;        // A rows, bf16: gate/up xbf [a_rows][K], down hbf [a_rows][K]
    const int32_t *order;      // [slots] route index or -1
    const float *layout_w;     // [slots] routing weight
    const int32_t *tile_expert, *num_tiles, *exp_off, *exp_cnt;
    const uint8_t *wa, *sa, *wb, *sb;  // gate/up: w1 | s1, w3 | s3; down: w2 | s2 (wb unused)
    uint8_t *hbf;              // gate/up out: bf16 h [slots][N]
    float *out;                // down out: f32 [slots][N]
    int K, N, n_experts, top_k, a_rows, slots;
    float limit;
};

struct EsStep {  // one wave's weight loads of one step: two bands
    u32x4v q[2];
};
// two LDS words at a and a + 64 written / read; complete when the statement
// ends
__device__ __forceinline__ void es_lds_put2(uint32_t a, float v0, float v1) {
    __asm__ volatile("ds_write_b32 %0, %1\n\tds_write_b32 %0, %2 offset:64\n\ts_waitcnt lgkmcnt(0)"
                     :
                     : "v"(a), "v"(v0), "v"(v1)
                     : "memory");
}
__device__ __forceinline__ void es_lds_get2(uint32_t a, float &v0, float &v1) {
    __asm__ volatile(
        "ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:64\n\ts_waitcnt lgkmcnt(0)"
        : "=&v"(v0), "=&v"(v1)
        : "v"(a)
        : "memory");
}


// MODE 0: gate/up + SwiGLU + routing weight + FP8 1x32 re-quantisation of h,
// written as the exact bf16 of the quantised values (the down step's A).
// MODE 1: down, f32 out for the slots that hold routes.
template <int MODE>
__device__ __forceinline__ void es_body(const EsArgs &a, uint8_t *g_lds) {
    using namespace es;
    constexpr int kAhead = 6;  // steps issued ahead of the one multiplied
    constexpr int NW = kThreads / 64;
    // g_lds: the A ring (kLds bytes), then the group table
    int *grp_l = (int *)(g_lds + kLds);   // [kMaxGroups] tile | T << 16 | expert << 19
    int *nrl_l = grp_l + kMaxGroups;      // [kMaxGroups] slots with routes of tile j: byte j
    __shared__ int cnt_l[NW][kTG + 1];
    __shared__ float am_l[NW][kTG * kTile];          // gate/up: per-row maxima of a wave's 16 columns
    const int t = threadIdx.x, lane = t & 63;
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int NS = a.K / 128;                            // steps per unit
    const int NCG = MODE == 0 ? a.N / 128 : a.N / 256;  // column blocks per group
    const int nt = min(*a.num_tiles, min(kMaxGroups, a.slots / kTile));

    // ---- the groups, sorted by size (largest first), then by tile
    constexpr int PL = kMaxGroups / kThreads;  // tiles per lane
    int gk[PL], gt[PL], gn[PL];
#pragma unroll
    for (int h = 0; h < PL; h++) {
        const int tt = (w * PL + h) * 64 + lane;
        gk[h] = -1;
        gt[h] = gn[h] = 0;
        if (tt < nt) {
            const int e = g_expert(a.tile_expert, tt, a.n_experts);
            const int off = a.exp_off[e], cnt = a.exp_cnt[e];
            const int rel = tt - off / kTile;
            const int ntile = (cnt + kTile - 1) / kTile;
            if (rel >= 0 && rel % kTG == 0) {
                gt[h] = max(1, min(kTG, min(ntile - rel, nt - tt)));
                gk[h] = tt | (gt[h] << 16) | (e << 19);
                // an expert's routes fill its slots in order from its offset
#pragma unroll
                for (int j = 0; j < kTG; j++)
                    gn[h] |= min(max(cnt - ((tt + j) * kTile - off), 0), kTile) << (8 * j);
            }
        }
    }
    uint64_t bal[PL][kTG + 1];
#pragma unroll
    for (int T = 1; T <= kTG; T++) {
        int c = 0;
#pragma unroll
        for (int h = 0; h < PL; h++) {
            bal[h][T] = __ballot(gt[h] == T);
            c += __popcll(bal[h][T]);
        }
        if (lane == 0) cnt_l[w][T] = c;
    }
    lds_barrier();
    int cls = 0, mine[kTG + 1];
#pragma unroll
    for (int T = kTG; T >= 1; T--) {  // classes in size order, waves in order within one
        int off = cls;
        for (int ww = 0; ww < NW; ww++) {
            if (ww == w) mine[T] = off;
            off += cnt_l[ww][T];
        }
        cls = off;
    }
    const int ng = cls;
    const uint64_t below = (1ull << lane) - 1;
#pragma unroll
    for (int T = 1; T <= kTG; T++) {
        int pos = mine[T];
#pragma unroll
        for (int h = 0; h < PL; h++) {
            if (gt[h] == T) {
                grp_l[pos + __popcll(bal[h][T] & below)] = gk[h];
                nrl_l[pos + __popcll(bal[h][T] & below)] = gn[h];
            }
            pos += __popcll(bal[h][T]);
        }
    }
    lds_barrier();

    // ---- this workgroup's units: unit k of the sorted order goes to round
    // k / G, position p = k % G in even rounds and G - 1 - k % G in odd ones;
    // position p is workgroup (p % (G / 8)) * 8 + p / (G / 8), so the column
    // blocks of a group (consecutive positions) run on one XCD (the hardware
    // deals workgroup b to XCD b % 8) and read the group's A rows from that
    // XCD's L2
    const int G = gridDim.x, b = blockIdx.x;
    const int pb = (G % 8 == 0) ? (b % 8) * (G / 8) + b / 8 : b;
    const int U = ng * NCG;
    auto unit_k = [&](int ri) { return ri * G + ((ri & 1) ? G - 1 - pb : pb); };
    const int n_units = U / G + (unit_k(U / G) < U ? 1 : 0);
    if (n_units == 0) return;  // whole workgroup
    const int total = n_units * NS;
    const size_t wmat = (size_t)a.N * (a.K / 2);
    const size_t smat = (size_t)packed_fp4_scale_bytes(a.N, a.K);
    const uint32_t ring = lds_addr(g_lds);
    const es_rsrc abuf = es_buf(a.abf, (size_t)a.a_rows * a.K * 2);

    // ---- issue side: the unit whose steps are being loaded
    int ri_i = 0, s_i = 0, Ti = 1;
    int cmask = 1;            // bit j: this wave copies rows of tile j (some hold routes)
    es_rsrc wr[2], sr[2];     // the unit's expert matrices (gate/up: w1, w3; down: w2)
    uint32_t bo[2], so[2];    // this lane's byte offsets of step 0 per band (weights, scales)
    uint32_t ao[kTG];         // this lane's A row offset per tile (rows 4w .. 4w + 3)
    // gate/up: the route of row 4w + g of each tile of the next unit to open,
    // loaded one unit ahead (a vector load; the unit's first issue uses it)
    const es_rsrc ordbuf = es_buf(a.order, (size_t)a.slots * 4);
    int on[kTG];
    auto pre_order = [&](int ri) {
        if (MODE != 0) return;
        const int k = unit_k(min(ri, n_units - 1));
        const int v = __builtin_amdgcn_readfirstlane(es_lds_word(&grp_l[k / NCG]));
        const int t0 = v & 0xFFFF, T = (v >> 16) & 7;
#pragma unroll
        for (int j = 0; j < kTG; j++)
            on[j] = (int)__builtin_amdgcn_raw_buffer_load_b32(
                ordbuf, (uint32_t)(((t0 + min(j, T - 1)) * kTile + 4 * w + g) * 4), 0, 0);
    };
    auto open_issue = [&]() {
        const int k = unit_k(ri_i);
        const int v = __builtin_amdgcn_readfirstlane(es_lds_word(&grp_l[k / NCG]));
        const int cg = k % NCG, t0 = v & 0xFFFF, e = v >> 19;
        Ti = (v >> 16) & 7;
        // a tile's routes fill its rows from row 0, so rows 4w .. 4w + 3 of
        // a tile with at most 4w routes are padding: their LDS rows keep
        // whatever they held, which reaches no output (a padding row's
        // results are neither stored nor part of a block maximum, and an
        // MFMA output column depends on its own A row only)
        const int nri = __builtin_amdgcn_readfirstlane(es_lds_word(&nrl_l[k / NCG]));
        cmask = 0;
#pragma unroll
        for (int j = 0; j < kTG; j++)
            if (j < Ti && ((nri >> (8 * j)) & 0xFF) > 4 * w) cmask |= 1 << j;
#pragma unroll
        for (int m = 0; m < 2; m++) {
            wr[m] = es_buf((m == 0 || MODE == 1 ? a.wa : a.wb) + (size_t)e * wmat, wmat);
            sr[m] = es_buf((m == 0 || MODE == 1 ? a.sa : a.sb) + (size_t)e * smat, smat);
        }
        const int ks8 = (NS + 7) / 8;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int rt = MODE == 0 ? cg * 8 + w : cg * 16 + 2 * w + h;
            bo[h] = (uint32_t)(((size_t)rt * NS * 64 + lane) * 16);
            so[h] = (uint32_t)(((size_t)rt * ks8 * 64 + lane) * 8);
        }
        // row 4w + g of each tile; a row's 16-byte pieces are stored
        // XOR-permuted by the row (bank spread)
        const int row = 4 * w + g;
#pragma unroll
        for (int j = 0; j < kTG; j++) {
            const int tj = t0 + min(j, Ti - 1);
            uint32_t arow;
            if (MODE == 0) {
                const int route = on[j];
                arow = route >= 0 ? (uint32_t)(route / a.top_k) : 0u;
            } else {
                arow = (uint32_t)(tj * kTile + row);
            }
            ao[j] = arow * (uint32_t)a.K * 2u + ((r ^ (row & 15)) << 4);
        }
        pre_order(ri_i + 1);
    };
    int nT[kRing];  // this wave's copies of the step in each ring slot
    // the loads of the next step of the stream (its unit opened) into
    // register slot x and ring slot `slot`: 2 + popcount(cmask) per wave. Past the end
    // of the stream (real == false) the last step's loads are repeated and
    // not used, so that every step has the same loads in flight after it.
    auto issue = [&](EsStep &x, int slot, bool real) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int m = MODE == 0 ? h : 0;
            x.q[h] = __builtin_bit_cast(
                u32x4v, __builtin_amdgcn_raw_buffer_load_b128(wr[m], bo[h] + (uint32_t)s_i * 1024u, 0, 0));
        }
        const uint32_t lb = ring + slot * kSlotB + 4 * w * kRowB;
#pragma unroll
        for (int j = 0; j < kTG; j++)
            if ((cmask >> j) & 1)  // uniform: tiles the group has, rows with routes
                es_dma(abuf, ao[j] + (uint32_t)s_i * kRowB, lb + j * kTile * kRowB, 16);
        nT[slot] = __builtin_popcount(cmask);
        if (real && ++s_i == NS) {
            s_i = 0;
            ri_i++;
        }
    };

    // ---- compute side: the unit being multiplied
    int ri_c = 0, s_c = 0, Tc = 1, t0c = 0, cgc = 0, lo16 = 0, nrc = 0;
    // gate/up: the routing weights of the lane's rows r and 16 + r of each
    // tile, loaded when the unit opens (used at its end)
    const es_rsrc lwbuf = es_buf(a.layout_w, (size_t)a.slots * 4);
    float rwf[kTG][2];
    auto open_compute = [&]() {
        const int k = unit_k(ri_c);
        const int v = __builtin_amdgcn_readfirstlane(es_lds_word(&grp_l[k / NCG]));
        nrc = __builtin_amdgcn_readfirstlane(es_lds_word(&nrl_l[k / NCG]));
        cgc = k % NCG;
        t0c = v & 0xFFFF;
        Tc = (v >> 16) & 7;
        lo16 = 0;  // bit j: tile j's slots 16.. are padding
#pragma unroll
        for (int j = 0; j < kTG; j++)
            if (((nrc >> (8 * j)) & 0xFF) <= 16) lo16 |= 1 << j;
        if (MODE == 0)
#pragma unroll
            for (int j = 0; j < kTG; j++) {
                const int slot0 = min(t0c + j, a.slots / kTile - 1) * kTile;
#pragma unroll
                for (int i = 0; i < 2; i++)
                    rwf[j][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                        lwbuf, (uint32_t)(slot0 + 16 * i + r) * 4u, 0, 0));
            }
    };
    // [tile][band][16-row fragment]: the weights are the MFMA's first
    // operand, so lane (r, g) holds columns 4g .. 4g + 3 of the band for
    // row r of the fragment (four adjacent columns of one row)
    v4f acc[kTG][2][2];
    const uint64_t tab = ws_lane_exp2f_tab(lane);

    // The scale bytes of four steps (one per step and lane: a word) sit in
    // sw[b][band] for the 4-step block b of the 8-step iteration. Block b's
    // word is loaded at the end of step 4b + 3 of the iteration before (after
    // that step's multiply, the last read of the old word), five steps before
    // its first use; the issue side then points two steps into that block.
    uint32_t sw[2][2];
    auto load_scales = [&](int b, int back) {
        const int s0 = max(s_i - back, 0);  // the block's first step (0 past the end)
#pragma unroll
        for (int h = 0; h < 2; h++)
            sw[b][h] = __builtin_amdgcn_raw_buffer_load_b32(
                sr[MODE == 0 ? h : 0], so[h] + (uint32_t)(s0 >> 3) * 512u + (uint32_t)(s0 & 4), 0, 0);
    };
    auto multiply = [&](const EsStep &x, uint32_t sbase, int u) {
        __asm__ volatile("" : "+s"(sbase));  // opaque: the slot's addresses are formed per step
        if (s_c == 0) {
#pragma unroll
            for (int j = 0; j < kTG; j++)
#pragma unroll
                for (int h = 0; h < 2; h++) acc[j][h][0] = acc[j][h][1] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        v8bf bq[2][4];
#pragma unroll
        for (int h = 0; h < 2; h++)
            cvt_fp4x32(uint4{x.q[h][0], x.q[h][1], x.q[h][2], x.q[h][3]},
                       e8m0_to_f32((sw[u >> 2][h] >> (8 * (u & 3))) & 0xFF), bq[h]);
#pragma unroll
        for (int j = 0; j < kTG; j++) {
            if (j >= Tc) continue;  // uniform
            uint32_t ad[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++)
                ad[jj] = sbase + (j * kTile + r) * kRowB + (((4 * g + jj) ^ r) << 4);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                if (i == 1 && ((lo16 >> j) & 1)) continue;  // uniform: rows 16.. are padding
                u32x4v av[4];
                if (i == 0) es_lds_frag<0>(ad, av);
                else es_lds_frag<4096>(ad, av);
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    const v8bf am = __builtin_bit_cast(v8bf, av[jj]);
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        acc[j][h][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[h][jj], am,
                                                                               acc[j][h][i], 0, 0, 0);
                }
            }
        }
    };

    const es_rsrc obuf = MODE == 0 ? es_buf(a.hbf, (size_t)a.slots * a.N * 2)
                                   : es_buf(a.out, (size_t)a.slots * a.N * 4);
    auto epilogue = [&]() {
        if (MODE == 1) {
            // f32 out of the slots that hold routes: four adjacent columns
            // per lane and row, straight from the accumulators
#pragma unroll
            for (int j = 0; j < kTG; j++) {
                if (j >= Tc) continue;  // uniform
                const int slot0 = min(t0c + j, a.slots / kTile - 1) * kTile;
                const int nr = (nrc >> (8 * j)) & 0xFF;
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const int row = 16 * i + r;
                    if (row >= nr) continue;
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        __builtin_amdgcn_raw_buffer_store_b128(
                            __builtin_bit_cast(u32x4v, acc[j][h][i]), obuf,
                            (uint32_t)((slot0 + row) * a.N + cgc * 256 + 32 * w + 16 * h + 4 * g) * 4u,
                            0, 0);
                }
            }
            return;
        }
        // gate/up: h = silu(gate) * up * routing weight for this wave's 16
        // columns; a row's FP8 1x32 block spans this wave (lanes g = 0..3 of
        // the row's r) and its partner (w ^ 1), which meet in LDS (both
        // tiles' maxima across one barrier)
        const int col = cgc * 128 + 16 * w + 4 * g;
        float hv[kTG][2][4], m[kTG][2];  // [j][i][v]: tile j, row 16 i + r, column col + v
#pragma unroll
        for (int j = 0; j < kTG; j++) {
            const int nr = (nrc >> (8 * j)) & 0xFF;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int row = 16 * i + r;
                const float rw = rwf[j][i];
                m[j][i] = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; v++) hv[j][i][v] = 0.0f;
                // uniform: a tile the group lacks, rows 16.. of padding
                if (j >= Tc || (i == 1 && ((lo16 >> j) & 1))) continue;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    float gv = acc[j][0][i][v], uv = acc[j][1][i][v];
                    if (a.limit > 0.0f) {
                        uv = rclamp(uv, -a.limit, a.limit);
                        gv = fminf(gv, a.limit);
                    }
                    const float hh = ws_silu_lanes(gv, tab) * uv * rw;
                    hv[j][i][v] = row < nr ? hh : 0.0f;
                    m[j][i] = fmaxf(m[j][i], __builtin_fabsf(hv[j][i][v]));
                }
                m[j][i] = fmaxf(m[j][i], __shfl_xor(m[j][i], 16, 64));
                m[j][i] = fmaxf(m[j][i], __shfl_xor(m[j][i], 32, 64));
            }
        }
        // the row maxima of the wave's 16 columns: am_l[w][j * 32 + row]
        const uint32_t base = lds_addr(&am_l[0][0]) + (uint32_t)r * 4u;
        static_assert(kTG == 2, "two tiles per group");
        if (g == 0) {
            es_lds_put2(base + (uint32_t)w * kTG * kTile * 4u, m[0][0], m[0][1]);
            es_lds_put2(base + (uint32_t)(w * kTG + 1) * kTile * 4u, m[1][0], m[1][1]);
        }
        raw_barrier();  // the partner's maxima
        float mp[kTG][2];
        es_lds_get2(base + (uint32_t)(w ^ 1) * kTG * kTile * 4u, mp[0][0], mp[0][1]);
        es_lds_get2(base + (uint32_t)((w ^ 1) * kTG + 1) * kTile * 4u, mp[1][0], mp[1][1]);
#pragma unroll
        for (int j = 0; j < kTG; j++) {
            if (j >= Tc) continue;  // uniform
            const int slot0 = min(t0c + j, a.slots / kTile - 1) * kTile;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int row = 16 * i + r;
                // the rule of quant_fp8_block32 on the 1x32 block
                float mm = fmaxf(m[j][i], mp[j][i]);
                if (!(mm >= 1e-4f)) mm = 1e-4f;
                const int ex = log2_ceil_div448(mm);
                const float inv = block_inv_scale(ex), sc = e8m0_to_f32((uint32_t)(ex + 127) & 0xFF);
                uint32_t hb[2];  // the bf16 of the four quantised values, two per word
#pragma unroll
                for (int p = 0; p < 2; p++)
                    hb[p] = __builtin_bit_cast(
                        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(
                                      block_byte(hv[j][i][2 * p], inv) |
                                          (block_byte(hv[j][i][2 * p + 1], inv) << 8),
                                      sc, false));
                __builtin_amdgcn_raw_buffer_store_b64(
                    (es_u2){hb[0], hb[1]}, obuf, (uint32_t)((slot0 + row) * a.N + col) * 2u, 0, 0);
            }
        }
    };

    // ---- the stream, unrolled by the ring (static register slots); NS is a
    // multiple of kRing, so units end on the last step of an iteration. Every
    // step issues one step (past the end a repeat), and steps 3 and 7 of an
    // iteration load a block of scale words, so when steps q and q + 1 are
    // waited for, the loads of steps q + 2 .. q + kAhead - 1 and the scale
    // loads at the ends of steps q - 5 .. q - 1 are newer.
    static_assert(kAhead == 6, "the scale blocks are loaded five steps ahead");
    EsStep st[kRing];
    pre_order(0);
    open_compute();
#pragma unroll
    for (int u = 0; u < kAhead; u++) {
        if (s_i == 0) open_issue();
        issue(st[u], u, true);
    }
    load_scales(0, 6);  // steps 0 .. 3
    load_scales(1, 2);  // steps 4 .. 7
    auto step = [&](EsStep &x, EsStep &next, int u, int q) {
        if ((u & 1) == 0) {
            // steps q and q + 1 have landed: at most the newer loads are in
            // flight (four steps of 2 loads and 0 .. T copies, and two or one
            // scale blocks of two words)
            const int n = 8 + nT[(u + 2) % kRing] + nT[(u + 3) % kRing] + nT[(u + 4) % kRing] +
                          nT[(u + 5) % kRing] + ((u & 3) == 0 ? 4 : 2);
            es_wait_vm<8 + 2, 8 + 4 * kTG + 4>(n);
            raw_barrier();  // every wave's copies of both steps are in LDS
        }
        const bool real = q + kAhead < total;
        if (real && s_i == 0) open_issue();
        issue(next, (u + kAhead) % kRing, real);
        multiply(x, ring + u * kSlotB, u);
        if ((u & 3) == 3) load_scales(u >> 2, 2);  // the block five steps on
        s_c++;
    };
    static_assert(kRing == 8 && kAhead <= kRing - 2, "eight ring slots, slot q - 2 the newest reused");
    for (int q = 0; q < total; q += kRing) {
        step(st[0], st[(0 + kAhead) % kRing], 0, q);
        step(st[1], st[(1 + kAhead) % kRing], 1, q + 1);
        step(st[2], st[(2 + kAhead) % kRing], 2, q + 2);
        step(st[3], st[(3 + kAhead) % kRing], 3, q + 3);
        step(st[4], st[(4 + kAhead) % kRing], 4, q + 4);
        step(st[5], st[(5 + kAhead) % kRing], 5, q + 5);
        step(st[6], st[(6 + kAhead) % kRing], 6, q + 6);
        step(st[7], st[(7 + kAhead) % kRing], 7, q + 7);
        if (s_c == NS) {
            epilogue();
            s_c = 0;
            ri_c++;
            if (ri_c < n_units) open_compute();
        }
    }
    // the repeated loads of the last steps end here
    es_vmcnt<0>();
#pragma unroll
    for (int u = 0; u < kRing; u++)
#pragma unroll
        for (int h = 0; h < 2; h++) __asm__ volatile("" ::"v"(st[u].q[h]));
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
        for (int h = 0; h < 2; h++) __asm__ volatile("" ::"v"(sw[b][h]));
}

// One launch per half of the prefill that runs the expert-stationary body
// when the dispatch found that its groups pay (*select, es_pays) and the
// tile-streaming body otherwise; every workgroup takes the same branch.
template <int ROWS, int CB>
__global__ __launch_bounds__(kGThreads) void glu_select_kernel(const int32_t *select, EsArgs ea,
                                                              GluArgs ga) {
    extern __shared__ __align__(16) uint8_t g_lds[];
    if (__builtin_amdgcn_readfirstlane(*select)) es_body<0>(ea, g_lds);
    else grouped_glu_body<true, ROWS, CB>(ga, g_lds);
}

template <int CB, bool ABF>
__global__ __launch_bounds__(kGThreads) void down_select_kernel(const int32_t *select, EsArgs ea,
                                                               DownArgs da) {
    extern __shared__ __align__(16) uint8_t g_lds[];
    if (__builtin_amdgcn_readfirstlane(*select)) es_body<1>(ea, g_lds);
    else grouped_down_body<true, CB, false, ABF>(da, g_lds);
}

// The expert-stationary pair serves exact math, dim a multiple of 256 (whole
// 256-column down blocks), K steps (dim / 128, inter / 128) in whole rounds of
// the ring and at most kMaxGroups tiles.
static bool es_fits(int64_t dim, int64_t inter, int64_t tiles) {
    return math_mode() == WS_MATH_EXACT && dim % 256 == 0 && inter % 128 == 0 &&
           (dim / 128) % es::kRing == 0 && (inter / 128) % es::kRing == 0 &&
           tiles <= es::kMaxGroups;
}

// ---- combine: y[row] = sum of its routes' outputs in ascending slot order --
// V columns per thread (V = 4: 16-byte loads, dim % 4 == 0)
template <int V>
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ down,
                                                      const int32_t *__restrict__ route_pos,
                                                      float *__restrict__ y, int dim, int top_k,
                                                      int cap) {
    __shared__ int32_t slots[16];
    __shared__ int32_t ns;
    const int row = blockIdx.y;
    if (threadIdx.x < 64) {
        // lane j holds route j's slot; the slots of a row are distinct, so a
        // slot's place in ascending order is the number of smaller ones
        const int j = threadIdx.x;
        const int s = j < top_k ? route_pos[(size_t)row * top_k + j] : -1;
        const bool ok = s >= 0 && s < cap;
        int place = 0;
        for (int l = 0; l < top_k; l++) {
            const int sl = __shfl(s, l, 64);
            place += (sl >= 0 && sl < cap && sl < s);
        }
        const int n = __popcll(__ballot(ok));
        if (ok) slots[place] = s;
        if (j == 0) ns = n;
    }
    __syncthreads();
    const int d = (blockIdx.x * 256 + threadIdx.x) * V;
    if (d >= dim) return;
    if constexpr (V == 4) {
        float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 0; i < ns; i++) {
            const float4 v = *(const float4 *)(down + (size_t)slots[i] * dim + d);
            acc.x = acc.x + v.x;
            acc.y = acc.y + v.y;
            acc.z = acc.z + v.z;
            acc.w = acc.w + v.w;
        }
        *(float4 *)(y + (size_t)row * dim + d) = acc;
    } else {
        float acc = 0.0f;
        for (int i = 0; i < ns; i++) acc = acc + down[(size_t)slots[i] * dim + d];
        y[(size_t)row * dim + d] = acc;
    }
}

// moe_swiglu_route (moe_grouped.cu:239-256): out = silu(min(g,10)) *
// clamp(u,-10,10) * w[row], 0 where w[row] == 0 (padding slots); silu in
// weightstream-ref num.rs:71-79 order on the exact expf.
__global__ __launch_bounds__(256) void swiglu_route_kernel(const float *__restrict__ gate,
                                                           const float *__restrict__ up,
                                                           const float *__restrict__ lw,
                                                           float *out, int inter) {
    const int row = blockIdx.y;
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= inter) return;
    const size_t i = (size_t)row * inter + n;
    const float wr = lw[row];
    if (wr == 0.0f) {
        out[i] = 0.0f;
        return;
    }
    const float g = fminf(gate[i], 10.0f);
    const float u = rclamp(up[i], -10.0f, 10.0f);
    out[i] = ws_silu(g) * u * wr;
}

static inline bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }
static inline bool al4(const void *p) { return ((uintptr_t)p & 3) == 0; }
static inline bool al8(const void *p) { return ((uintptr_t)p & 7) == 0; }
static size_t a256(size_t v) { return (v + 255) & ~(size_t)255; }

// Two bands per wave (wider units, each A fragment converted once for both)
// when the tile capacity is large; one band per wave (twice the units) for
// few tiles, where the unit count limits the spread over the CUs. Measured
// with 384 experts: M=132 prefill 294 -> 266 us and M=64 279 -> 270 us wide;
// M=8 (66 tiles) 167 us narrow against 179 wide.
constexpr int64_t kWideTiles = 192;
static inline bool wide_units(int64_t tiles) { return tiles >= kWideTiles; }

static int64_t tiles_for(int64_t routes, int64_t n_experts) {
    return (routes + kTile - 1) / kTile + (routes < n_experts ? routes : n_experts);
}

}  // namespace ws

using namespace ws;

extern "C" {

// The dispatch on workgroup 0; with nx > 0 workgroups 1.. quantise the nx
// token values xf into xq / xs (ws_emit8) in the same launch.
static int dispatch_launch(const int32_t *topk_idx, const float *topk_w, int32_t *order,
                           float *layout_w, int32_t *route_pos, int32_t *tile_expert,
                           int32_t *expert_count, int32_t *expert_offset, int32_t *expert_psum,
                           int32_t *num_tiles, int64_t rows, int64_t top_k, int64_t tiles,
                           int64_t n_experts, const float *xf, uint8_t *xq, uint8_t *xs,
                           int64_t nx, ws_stream_t stream, uint16_t *xbf = nullptr,
                           int32_t *select = nullptr) {
    const int64_t qblocks = (nx + kDispThreads - 1) / kDispThreads;
    hipLaunchKernelGGL(dispatch_kernel<int32_t>, dim3((unsigned)(1 + qblocks)), dim3(kDispThreads),
                       0, stream, topk_idx, topk_w, order, layout_w, route_pos, tile_expert,
                       expert_count, expert_offset, expert_psum, num_tiles, (int)(rows * top_k),
                       (int)tiles, (int)n_experts, xf, xq, xs, nx, xbf, select);
    return launch_status();
}

int ws_moe_dispatch_tl(const int64_t *topk_idx, const float *topk_weights, int32_t *order,
                       float *layout_weights, int32_t *route_pos, int32_t *tile_expert,
                       int32_t *expert_count, int32_t *expert_offset, int32_t *expert_psum,
                       int32_t *num_tiles, int64_t rows, int64_t top_k, int64_t tiles,
                       int64_t n_experts, ws_stream_t stream) {
    if (!topk_idx || !topk_weights || !order || !layout_weights || !route_pos || !tile_expert ||
        !expert_count || !expert_offset || !expert_psum || !num_tiles)
        return WS_ERR_INVALID_ARG;
    if (rows <= 0 || top_k <= 0 || tiles <= 0 || n_experts <= 0) return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExpertsG || rows * top_k > (1 << 26) || tiles > (1 << 24))
        return WS_ERR_SHAPE;
    hipLaunchKernelGGL(dispatch_kernel<int64_t>, dim3(1), dim3(kDispThreads), 0, stream, topk_idx,
                       topk_weights, order, layout_weights, route_pos, tile_expert, expert_count,
                       expert_offset, expert_psum, num_tiles, (int)(rows * top_k), (int)tiles,
                       (int)n_experts, nullptr, nullptr, nullptr, (int64_t)0, nullptr, nullptr);
    return launch_status();
}

int ws_moe_dispatch(const int32_t *topk_idx, const float *topk_w, int32_t *order,
                    float *layout_w, int32_t *route_pos, int32_t *tile_expert,
                    int32_t *expert_count, int32_t *expert_offset, int32_t *expert_psum,
                    int32_t *num_tiles, int64_t rows, int64_t top_k, int64_t tiles,
                    int64_t n_experts, ws_stream_t stream) {
    if (!topk_idx || !topk_w || !order || !layout_w || !route_pos || !tile_expert ||
        !expert_count || !expert_offset || !expert_psum || !num_tiles)
        return WS_ERR_INVALID_ARG;
    if (rows <= 0 || top_k <= 0 || tiles <= 0 || n_experts <= 0) return WS_ERR_INVALID_ARG;
    if (n_experts > kMaxExpertsG || rows * top_k > (1 << 26) || tiles > (1 << 24))
        return WS_ERR_SHAPE;
    return dispatch_launch(topk_idx, topk_w, order, layout_w, route_pos, tile_expert, expert_count,
                           expert_offset, expert_psum, num_tiles, rows, top_k, tiles, n_experts,
                           nullptr, nullptr, nullptr, 0, stream);
}

// exp_off / exp_cnt (the dispatch's per-expert slot offsets and counts, or
// nullptr): deal the units as expert runs (g_share_units).
static int grouped_glu_launch(const uint8_t *xq, const uint8_t *xs, const int32_t *order,
                              const float *layout_w, const int32_t *tile_expert,
                              const int32_t *num_tiles, const int32_t *exp_off,
                              const int32_t *exp_cnt, const uint8_t *w1, const uint8_t *s1,
                              const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                              int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                              int64_t tiles, float swiglu_limit, ws_stream_t stream) {
    if (!xq || !xs || !order || !layout_w || !tile_expert || !num_tiles || !w1 || !s1 || !w3 ||
        !s3 || !hq || !hs)
        return WS_ERR_INVALID_ARG;
    if (dim <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0 || tiles <= 0)
        return WS_ERR_INVALID_ARG;
    if (dim % 128 || inter % 128 || tiles > 65535 || dim > (1 << 20) || inter > (1 << 20))
        return WS_ERR_SHAPE;
    if (!al16(xq) || !al16(w1) || !al16(w3) || !al4(xs) || !al8(s1) || !al8(s3))
        return WS_ERR_INVALID_ARG;
    // the A block (ROWS x dim bytes) lives in LDS: 32 rows up to dim 4096,
    // 16-row halves of each tile up to 8192
    if (dim > 8192) return WS_ERR_SHAPE;
    const GluArgs ga{xq, xs, order, layout_w, tile_expert, num_tiles, exp_off, exp_cnt, w1, s1,
                     w3, s3, hq, hs, (int)dim, (int)inter, (int)n_experts, (int)top_k,
                     swiglu_limit};
    dim3 grid((unsigned)cu_count());
#define WS_GLU(E, R, CB)                                                                      \
    hipLaunchKernelGGL((grouped_glu_quant_kernel<E, R, CB>), grid, dim3(kGThreads),          \
                       g_tile_lds(R, (int)dim), stream, ga)
#define WS_GLU_CB(E, R)                       \
    if (wide_units(tiles)) WS_GLU(E, R, 2);   \
    else WS_GLU(E, R, 1);
    const bool exact = math_mode() == WS_MATH_EXACT;
    if (dim <= 4096) {
        if (exact) { WS_GLU_CB(true, 32) } else { WS_GLU_CB(false, 32) }
    } else {
        if (exact) { WS_GLU_CB(true, 16) } else { WS_GLU_CB(false, 16) }
    }
#undef WS_GLU_CB
#undef WS_GLU
    return launch_status();
}

int ws_moe_grouped_glu_quant(const uint8_t *xq, const uint8_t *xs, const int32_t *order,
                             const float *layout_w, const int32_t *tile_expert,
                             const int32_t *num_tiles, const uint8_t *w1, const uint8_t *s1,
                             const uint8_t *w3, const uint8_t *s3, uint8_t *hq, uint8_t *hs,
                             int64_t dim, int64_t inter, int64_t n_experts, int64_t top_k,
                             int64_t tiles, float swiglu_limit, ws_stream_t stream) {
    return grouped_glu_launch(xq, xs, order, layout_w, tile_expert, num_tiles, nullptr, nullptr,
                              w1, s1, w3, s3, hq, hs, dim, inter, n_experts, top_k, tiles,
                              swiglu_limit, stream);
}

static int grouped_down_launch(const uint8_t *hq, const uint8_t *hs, const int32_t *tile_expert,
                               const int32_t *num_tiles, const int32_t *exp_off,
                               const int32_t *exp_cnt, const int32_t *order, const uint8_t *w2,
                               const uint8_t *s2, float *out, int64_t dim, int64_t inter,
                               int64_t n_experts, int64_t tiles, ws_stream_t stream);

int ws_moe_grouped_down(const uint8_t *hq, const uint8_t *hs, const int32_t *tile_expert,
                        const int32_t *num_tiles, const uint8_t *w2, const uint8_t *s2,
                        float *out, int64_t dim, int64_t inter, int64_t n_experts, int64_t tiles,
                        ws_stream_t stream) {
    if (!hq || !hs || !tile_expert || !num_tiles || !w2 || !s2 || !out) return WS_ERR_INVALID_ARG;
    if (dim <= 0 || inter <= 0 || n_experts <= 0 || tiles <= 0) return WS_ERR_INVALID_ARG;
    if (dim % 128 || inter % 128 || tiles > 65535) return WS_ERR_SHAPE;
    if (!al16(hq) || !al16(w2) || !al4(hs) || !al8(s2)) return WS_ERR_INVALID_ARG;
    if (inter > 4096) return WS_ERR_SHAPE;  // the 32 x inter hq tile lives in LDS
    return grouped_down_launch(hq, hs, tile_expert, num_tiles, nullptr, nullptr, nullptr, w2, s2,
                               out, dim, inter, n_experts, tiles, stream);
}

// order == nullptr: every slot of a used tile is computed and written.
// gather: A rows are the routes' tokens (order[slot] / top_k) of hq.
static int grouped_gemm_launch(const uint8_t *hq, const uint8_t *hs, const int32_t *tile_expert,
                               const int32_t *num_tiles, const int32_t *exp_off,
                               const int32_t *exp_cnt, const int32_t *order, const uint8_t *w2,
                               const uint8_t *s2, float *out, int64_t dim, int64_t inter,
                               int64_t n_experts, int64_t tiles, bool gather, int64_t top_k,
                               int64_t tokens, ws_stream_t stream) {
    const bool abf = math_mode() == WS_MATH_EXACT && inter <= kAbfMaxK;
    const size_t lds = abf ? g_abf_lds(kTile, (int)inter) : g_tile_lds(kTile, (int)inter);
    const DownArgs da{hq, hs, tile_expert, num_tiles, exp_off, exp_cnt, order, w2, s2, out,
                      (int)dim, (int)inter, (int)n_experts, (int)tiles, (int)top_k,
                      (int)tokens};
    dim3 grid((unsigned)cu_count());
#define WS_DOWN(E, CB, G, A)                                                                   \
    hipLaunchKernelGGL((grouped_down_kernel<E, CB, G, A>), grid, dim3(kGThreads), lds, stream,  \
                       da)
    const bool wide = wide_units(tiles);
    if (abf) {
        if (gather) { if (wide) WS_DOWN(true, 2, true, true); else WS_DOWN(true, 1, true, true); }
        else if (wide) WS_DOWN(true, 2, false, true); else WS_DOWN(true, 1, false, true);
    } else if (math_mode() == WS_MATH_EXACT) {
        if (gather) { if (wide) WS_DOWN(true, 2, true, false); else WS_DOWN(true, 1, true, false); }
        else if (wide) WS_DOWN(true, 2, false, false); else WS_DOWN(true, 1, false, false);
    } else {
        if (gather) { if (wide) WS_DOWN(false, 2, true, false); else WS_DOWN(false, 1, true, false); }
        else if (wide) WS_DOWN(false, 2, false, false); else WS_DOWN(false, 1, false, false);
    }
#undef WS_DOWN
    return launch_status();
}

static int grouped_down_launch(const uint8_t *hq, const uint8_t *hs, const int32_t *tile_expert,
                               const int32_t *num_tiles, const int32_t *exp_off,
                               const int32_t *exp_cnt, const int32_t *order, const uint8_t *w2,
                               const uint8_t *s2, float *out, int64_t dim, int64_t inter,
                               int64_t n_experts, int64_t tiles, ws_stream_t stream) {
    return grouped_gemm_launch(hq, hs, tile_expert, num_tiles, exp_off, exp_cnt, order, w2, s2,
                               out, dim, inter, n_experts, tiles, false, 1, 1, stream);
}

int ws_moe_grouped_tl(int kind, const uint8_t *a, const uint8_t *sfa, const uint8_t *weights,
                      const uint8_t *sfb, const int32_t *order, const int32_t *tile_expert,
                      float *out, int64_t tiles, int64_t tokens, int64_t top_k, int64_t n,
                      int64_t k, int64_t n_experts, ws_stream_t stream) {
    if (!a || !sfa || !weights || !sfb || !order || !tile_expert || !out)
        return WS_ERR_INVALID_ARG;
    if (kind != WS_TL_MOE_GATE_UP && kind != WS_TL_MOE_DOWN) return WS_ERR_INVALID_ARG;
    if (tiles <= 0 || tokens <= 0 || top_k <= 0 || n <= 0 || k <= 0 || n_experts <= 0)
        return WS_ERR_INVALID_ARG;
    if (n % 128 || k % 128 || tiles > 65535 || k > 4096 || n > (1 << 20)) return WS_ERR_SHAPE;
    if (!al16(a) || !al16(weights) || !al4(sfa) || !al8(sfb)) return WS_ERR_INVALID_ARG;
    return grouped_gemm_launch(a, sfa, tile_expert, nullptr, nullptr, nullptr, order, weights,
                               sfb, out, n, k,
                               n_experts, tiles, kind == WS_TL_MOE_GATE_UP, top_k, tokens, stream);
}

int ws_moe_swiglu_route(const float *gate, const float *up, const float *weights, float *out,
                        int64_t inter, int64_t rows, ws_stream_t stream) {
    if (!gate || !up || !weights || !out || inter <= 0 || rows <= 0) return WS_ERR_INVALID_ARG;
    if (rows > 65535 || inter > (1 << 24)) return WS_ERR_SHAPE;
    hipLaunchKernelGGL(swiglu_route_kernel, dim3((unsigned)((inter + 255) / 256), (unsigned)rows),
                       dim3(256), 0, stream, gate, up, weights, out, (int)inter);
    return launch_status();
}

int ws_moe_combine_f32(const float *y, const int32_t *route_pos, float *out, int64_t dim,
                       int64_t top_k, int64_t rows, int64_t tiles, ws_stream_t stream) {
    if (!y || !route_pos || !out) return WS_ERR_INVALID_ARG;
    if (rows <= 0 || dim <= 0 || top_k <= 0 || tiles <= 0) return WS_ERR_INVALID_ARG;
    if (top_k > 16 || rows > 65535) return WS_ERR_SHAPE;
    if (dim % 4 == 0 && al16(y) && al16(out))
        hipLaunchKernelGGL(combine_kernel<4>,
                           dim3((unsigned)((dim / 4 + 255) / 256), (unsigned)rows), dim3(256), 0,
                           stream, y, route_pos, out, (int)dim, (int)top_k, (int)(tiles * kTile));
    else
        hipLaunchKernelGGL(combine_kernel<1>, dim3((unsigned)((dim + 255) / 256), (unsigned)rows),
                           dim3(256), 0, stream, y, route_pos, out, (int)dim, (int)top_k,
                           (int)(tiles * kTile));
    return launch_status();
}

size_t ws_moe_prefill_workspace_size(int64_t rows, int64_t dim, int64_t inter, int64_t top_k,
                                     int64_t n_experts) {
    if (rows <= 0 || dim <= 0 || inter <= 0 || top_k <= 0 || n_experts <= 0) return 0;
    const int64_t routes = rows * top_k, tiles = tiles_for(routes, n_experts);
    const int64_t slots = tiles * kTile;
    return a256(rows * dim) + a256(rows * (dim / 32)) + a256(slots * 4) * 2 + a256(routes * 4) +
           a256(tiles * 4) + a256(n_experts * 4) * 3 + a256(4) + a256(slots * inter) +
           a256(slots * (inter / 32)) + a256(slots * dim * 4) + a256(rows * dim * 2) +
           a256(slots * inter * 2);
}

int ws_moe_prefill(const float *x, const int32_t *topk_idx, const float *topk_w,
                   const uint8_t *w1, const uint8_t *s1, const uint8_t *w3, const uint8_t *s3,
                   const uint8_t *w2, const uint8_t *s2, float *y, int64_t rows, int64_t dim,
                   int64_t inter, int64_t n_experts, int64_t top_k, float swiglu_limit,
                   void *workspace, size_t workspace_bytes, ws_stream_t stream) {
    if (!x || !topk_idx || !topk_w || !y || !workspace) return WS_ERR_INVALID_ARG;
    if (rows <= 0 || dim <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0)
        return WS_ERR_INVALID_ARG;
    // every stage's shape limit, checked before the first launch
    if (dim % 128 || inter % 128 || dim > 8192 || inter > 4096) return WS_ERR_SHAPE;
    if (!w2 || !s2 || !al16(w2) || !al8(s2)) return WS_ERR_INVALID_ARG;
    if (workspace_bytes < ws_moe_prefill_workspace_size(rows, dim, inter, top_k, n_experts) ||
        !al16(workspace))
        return WS_ERR_INVALID_ARG;
    const int64_t routes = rows * top_k, tiles = tiles_for(routes, n_experts);
    const int64_t slots = tiles * kTile;
    uint8_t *p = (uint8_t *)workspace;
    auto take = [&](size_t bytes) {
        uint8_t *q = p;
        p += a256(bytes);
        return q;
    };
    uint8_t *xq = take(rows * dim);
    uint8_t *xs = take(rows * (dim / 32));
    int32_t *order = (int32_t *)take(slots * 4);
    float *layout_w = (float *)take(slots * 4);
    int32_t *route_pos = (int32_t *)take(routes * 4);
    int32_t *tile_expert = (int32_t *)take(tiles * 4);
    int32_t *cnt = (int32_t *)take(n_experts * 4);
    int32_t *off = (int32_t *)take(n_experts * 4);
    int32_t *psum = (int32_t *)take(n_experts * 4);
    int32_t *ntiles = (int32_t *)take(4);  // [0] used tiles; [1] the stationary choice
    int32_t *sel = ntiles + 1;             // (a256: the slot holds 256 bytes)
    uint8_t *hq = take(slots * inter);
    uint8_t *hs = take(slots * (inter / 32));
    float *down = (float *)take(slots * dim * 4);
    uint16_t *xbf = (uint16_t *)take(rows * dim * 2);
    uint16_t *hbf = (uint16_t *)take(slots * inter * 2);
    // the dispatch and the tokens' quantisation in one launch
    if (n_experts > kMaxExpertsG || routes > (1 << 26) || tiles > (1 << 24)) return WS_ERR_SHAPE;
    const bool stationary = es_fits(dim, inter, tiles);
    int rc = dispatch_launch(topk_idx, topk_w, order, layout_w, route_pos, tile_expert, cnt, off,
                             psum, ntiles, rows, top_k, tiles, n_experts, x, xq, xs, rows * dim,
                             stream, stationary ? xbf : nullptr, stationary ? sel : nullptr);
    if (rc) return rc;
    if (stationary) {
        // both halves run the body the dispatch chose on the device (*sel)
        const dim3 grid((unsigned)cu_count());
        const EsArgs ea{(const uint8_t *)xbf, order, layout_w, tile_expert, ntiles, off, cnt,
                        w1, s1, w3, s3, (uint8_t *)hbf, nullptr, (int)dim, (int)inter,
                        (int)n_experts, (int)top_k, (int)rows, (int)slots, swiglu_limit};
        const GluArgs ga{xq, xs, order, layout_w, tile_expert, ntiles, off, cnt, w1, s1, w3, s3,
                         hq, hs, (int)dim, (int)inter, (int)n_experts, (int)top_k,
                         swiglu_limit};
        const bool wide = wide_units(tiles);
        const int grows = dim <= 4096 ? 32 : 16;
        const size_t glds = std::max(es::kLdsAll, g_tile_lds(grows, (int)dim));
        if (grows == 32) {
            if (wide) hipLaunchKernelGGL((glu_select_kernel<32, 2>), grid, dim3(kGThreads), glds, stream, sel, ea, ga);
            else hipLaunchKernelGGL((glu_select_kernel<32, 1>), grid, dim3(kGThreads), glds, stream, sel, ea, ga);
        } else {
            if (wide) hipLaunchKernelGGL((glu_select_kernel<16, 2>), grid, dim3(kGThreads), glds, stream, sel, ea, ga);
            else hipLaunchKernelGGL((glu_select_kernel<16, 1>), grid, dim3(kGThreads), glds, stream, sel, ea, ga);
        }
        if ((rc = launch_status())) return rc;
        const EsArgs eb{(const uint8_t *)hbf, order, layout_w, tile_expert, ntiles, off, cnt,
                        w2, s2, nullptr, nullptr, nullptr, down, (int)inter, (int)dim,
                        (int)n_experts, (int)top_k, (int)slots, (int)slots, 0.0f};
        const DownArgs da{hq, hs, tile_expert, ntiles, off, cnt, order, w2, s2, down, (int)dim,
                          (int)inter, (int)n_experts, (int)tiles, 1, 1};
        const bool abf = inter <= kAbfMaxK;
        const size_t dlds = std::max(es::kLdsAll, abf ? g_abf_lds(kTile, (int)inter)
                                                      : g_tile_lds(kTile, (int)inter));
        if (abf) {
            if (wide) hipLaunchKernelGGL((down_select_kernel<2, true>), grid, dim3(kGThreads), dlds, stream, sel, eb, da);
            else hipLaunchKernelGGL((down_select_kernel<1, true>), grid, dim3(kGThreads), dlds, stream, sel, eb, da);
        } else {
            if (wide) hipLaunchKernelGGL((down_select_kernel<2, false>), grid, dim3(kGThreads), dlds, stream, sel, eb, da);
            else hipLaunchKernelGGL((down_select_kernel<1, false>), grid, dim3(kGThreads), dlds, stream, sel, eb, da);
        }
        if ((rc = launch_status())) return rc;
        return ws_moe_combine_f32(down, route_pos, y, dim, top_k, rows, tiles, stream);
    }
    rc = grouped_glu_launch(xq, xs, order, layout_w, tile_expert, ntiles, off, cnt, w1, s1, w3, s3,
                            hq, hs, dim, inter, n_experts, top_k, tiles, swiglu_limit, stream);
    if (rc) return rc;
    // only the slots that hold routes are multiplied and written (the
    // combine reads those)
    rc = grouped_down_launch(hq, hs, tile_expert, ntiles, off, cnt, order, w2, s2, down, dim, inter,
                             n_experts, tiles, stream);
    if (rc) return rc;
    return ws_moe_combine_f32(down, route_pos, y, dim, top_k, rows, tiles, stream);
}

}  // extern "C"
