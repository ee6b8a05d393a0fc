// Gate logits, producer/consumer form, as a device function (used by the
// gate kernel of moe_route.hip and by the gate + shared gate/up launch of
// gemm.hip).
#pragma once

#include "ws_device.hpp"

namespace ws {

// Chunks of kGC elements of the token and weight rows, a kGS-stage LDS ring.
constexpr int kGC = 256, kGS = 4;

template <int TE, int TM, bool BF16>
struct GateGeom {
    static constexpr int kXRow = kGC * 4;                // bytes of a token row chunk
    static constexpr int kWRow = kGC * (BF16 ? 2 : 4);   // bytes of a weight row chunk
    static constexpr int kX = TM * kXRow;
    static constexpr int kW = TE * kWRow;
    static constexpr int kStage = kX + kW;
    static constexpr int kLoads = kStage / 1024;         // 16-B direct loads per chunk
    static_assert(kStage % 1024 == 0 && TE * TM <= 64 && (kGS - 2) * kLoads < 64, "gate block");
};


// ---- gate logits, producer/consumer (dim % 256 == 0) ----------------------
// The same sequential chains as gate_logits_pipe_kernel, split over two
// waves so that the chain wave issues almost nothing but its adds: wave 0
// (producer) streams the token and weight rows through the LDS ring and
// writes the products x[d] * w[d] of every chain for a 256-element chunk into
// one of two LDS product buffers, 64 / C products per instruction (lane ->
// chain, element); wave 1 (consumer, lane = chain) adds a chunk's products in
// order, d = 0..dim-1, while the producer fills the other buffer. One
// workgroup barrier per chunk hands the buffers over. The products and adds
// are the same f32 operations in the same order as num::gemv, so the logits
// are the same bits.
constexpr int kPcPitch = kGC + 4;  // floats per product row (16-byte pad: no bank conflicts)

// Workgroup (bx, by) of the gate grid (ceil(E / TE), ceil(m / TM)); waves 0
// and 1 of the workgroup (threads 0-127) do the work, any others return.
template <int TE, int TM, bool BF16>
__device__ __forceinline__ void gate_pc_body(int bx, int by, const float *x, const void *gw,
                                             float *__restrict__ logits, int m_rows, int dim,
                                             int n_experts) {
    using G = GateGeom<TE, TM, BF16>;
    constexpr int C = TE * TM;  // chains of the workgroup (<= 16)
    static_assert(C <= 16 && 64 % C == 0, "chains per workgroup");
    extern __shared__ __align__(16) uint8_t g_lds[];
    float *prod = (float *)(g_lds + kGS * G::kStage);  // [2][C][kPcPitch]
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (wv > 1) return;
    const int e0 = bx * TE, m0 = by * TM;
    const int nc = dim / kGC;
    constexpr int kEB = BF16 ? 2 : 4;

    if (wv == 0) {
        // ---- producer ----
        const uint8_t *src[G::kLoads];
#pragma unroll
        for (int j = 0; j < G::kLoads; j++) {
            const int o = j * 1024 + lane * 16;
            if (o < G::kX) {
                const int row = o / G::kXRow, c = (o % G::kXRow) / 16;
                src[j] = (const uint8_t *)(x + (size_t)min(m0 + row, m_rows - 1) * dim) +
                         (c ^ (row & 15)) * 16;
            } else {
                const int oo = o - G::kX;
                const int row = oo / G::kWRow, c = (oo % G::kWRow) / 16;
                src[j] = (const uint8_t *)gw + (size_t)min(e0 + row, n_experts - 1) * dim * kEB +
                         (c ^ (row & 15)) * 16;
            }
        }
        auto issue = [&](int buf, int chunk) {
            uint8_t *base = g_lds + buf * G::kStage;
#pragma unroll
            for (int j = 0; j < G::kLoads; j++) {
                const int off = j * 1024 < G::kX ? chunk * G::kXRow : chunk * G::kWRow;
                __builtin_amdgcn_global_load_lds(
                    (const void *)(src[j] + off),
                    (__attribute__((address_space(3))) void *)(base + j * 1024), 16, 0, 0);
            }
        };
        // lane -> chain ch (token tm, expert te) and element offset dk
        const int ch = lane % C, dk = lane / C;
        const int tm = ch / TE, te = ch % TE;
#pragma unroll
        for (int p = 0; p < kGS - 1; p++)
            if (p < nc) issue(p, p);
        for (int i = 0; i < nc; i++) {
            mem_order();
            wait_newer<G::kLoads, kGS - 2>(min(nc - 1 - i, kGS - 2));
            if (i + kGS - 1 < nc) issue((i + kGS - 1) % kGS, i + kGS - 1);
            const uint32_t xb = lds_addr(g_lds) + (i % kGS) * G::kStage + tm * G::kXRow;
            const uint32_t wb = lds_addr(g_lds) + (i % kGS) * G::kStage + G::kX + te * G::kWRow;
            const uint32_t pb = lds_addr(prod + (size_t)(i & 1) * C * kPcPitch + ch * kPcPitch);
            // products of elements d = dk, dk + 64/C, ... of the chunk
            constexpr int kStep = 64 / C, kN = kGC / kStep;
            constexpr int kB = 8;  // reads in flight
#pragma unroll
            for (int q0 = 0; q0 < kN; q0 += kB) {
                uint32_t xr[kB], wr[kB];
#pragma unroll
                for (int q = 0; q < kB; q++) {
                    const int d = (q0 + q) * kStep + dk;
                    xr[q] = lds_read_b32(xb + ((d / 4) ^ (tm & 15)) * 16 + (d % 4) * 4);
                    if (BF16)
                        wr[q] = lds_read_b32(wb + ((d / 8) ^ (te & 15)) * 16 + ((d % 8) / 2) * 4);
                    else
                        wr[q] = lds_read_b32(wb + ((d / 4) ^ (te & 15)) * 16 + (d % 4) * 4);
                }
                lds_wait_all();
#pragma unroll
                for (int q = 0; q < kB; q++) {
                    lds_ready(xr[q]);
                    lds_ready(wr[q]);
                    const int d = (q0 + q) * kStep + dk;
                    const float we = BF16 ? __uint_as_float((d & 1) ? (wr[q] & 0xFFFF0000u) : (wr[q] << 16))
                                          : __uint_as_float(wr[q]);
                    lds_write_b32(pb + d * 4, __float_as_uint(__uint_as_float(xr[q]) * we));
                }
            }
            lds_wait_all();
            raw_barrier();  // products of chunk i are written (the consumer reads them)
        }
        raw_barrier();  // the consumer's last chunk
    } else {
        // ---- consumer: lane = chain ----
        const int ch = min(lane, C - 1);
        float s = 0.0f;
        raw_barrier();  // products of chunk 0
        for (int i = 0; i < nc; i++) {
            const uint32_t pb = lds_addr(prod + (size_t)(i & 1) * C * kPcPitch + ch * kPcPitch);
            u32x4v pv[2][4];
            auto reads = [&](int grp, u32x4v *r) {
#pragma unroll
                for (int k = 0; k < 4; k++) r[k] = lds_read_b128(pb + (grp * 16 + k * 4) * 4);
            };
            reads(0, pv[0]);
#pragma unroll
            for (int grp = 0; grp < kGC / 16; grp++) {
                const int cur = grp & 1;
                if (grp + 1 < kGC / 16) {
                    reads(grp + 1, pv[cur ^ 1]);
                    lds_wait<4>();
                } else {
                    lds_wait<0>();
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    lds_ready(pv[cur][k]);
#pragma unroll
                    for (int j = 0; j < 4; j++) s = s + __uint_as_float(pv[cur][k][j]);
                }
            }
            raw_barrier();  // chunk i consumed; chunk i + 1's products are written
        }
        const int tm = ch / TE, te = ch % TE;
        if (lane < C && m0 + tm < m_rows && e0 + te < n_experts)
            logits[(size_t)(m0 + tm) * n_experts + e0 + te] = s;
    }
}


}  // namespace ws
