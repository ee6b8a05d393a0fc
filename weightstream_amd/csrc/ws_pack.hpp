// Fragment-major ("packed") layout of FP4 weight matrices, and the streaming
// primitives of the kernels that read it.
//
// A [R, K] e2m1 matrix (R % 16 == 0, K % 128 == 0) with one UE8M0 scale per
// row and 32 K is stored as 16-row bands; band rt, 128-K step ks and MFMA lane
// l (row 16rt + l%16, K [128ks + 32(l/16), +32)) own 16 weight bytes at
//     ((rt * KS + ks) * 64 + l) * 16,          KS = K / 128,
// so a wave reads one contiguous 1 KB per step and walks a band's K as one
// contiguous run. The scale bytes of 8 consecutive steps of a lane are
// contiguous:
//     (((rt * KS8 + ks / 8) * 64 + l) * 8 + ks % 8,   KS8 = ceil(KS / 8).
// Expert slabs [E, R, K] concatenate E packed matrices. ws_prepack_fp4 builds
// the layout from the on-disk one (weightstream-core quant.rs:189-215) at
// upload, as the reference engine re-tiles its expert slabs
// (weightstream-gpu engine.rs:868 tile_major_expert).
#pragma once

#include "ws_device.hpp"

namespace ws {

constexpr int kU = 8;  // 128-K steps per register stage

__host__ __device__ constexpr int64_t packed_fp4_scale_bytes(int64_t rows, int64_t cols) {
    return (rows / 16) * ((cols / 128 + 7) / 8) * 64 * 8;
}

struct Fp4Band {
    const uint8_t *w;  // this lane's 16 bytes of step 0
    const uint8_t *s;  // this lane's scale byte of step 0 (8-step group 0)
    int ks_total;
};

// Band `rt` of a packed [R, K] matrix at (w, s), for lane `lane`.
__device__ __forceinline__ Fp4Band fp4_band(const uint8_t *w, const uint8_t *s, int rt, int k,
                                           int lane) {
    const int ks = k / 128, ks8 = (ks + 7) / 8;
    return Fp4Band{w + ((size_t)rt * ks * 64 + lane) * 16, s + ((size_t)rt * ks8 * 64 + lane) * 8,
                   ks};
}

// U steps of a band in registers (U = 8: a whole scale group; U = 4: half
// of one, its four scale bytes in s.x)
template <int U>
struct Fp4StageU {
    static_assert(U == 8 || U == 4, "stages of 8 or 4 steps");
    uint4 w[U];
    uint2 s;  // scale bytes of the U steps
};
using Fp4Stage = Fp4StageU<kU>;

// Steps [ks0, ks0 + U) of the band; steps at or past `kend` re-load step
// max(kend - 1, 0) (never used), keeping the loads unconditional so that one
// counter wait covers a whole stage. An empty range (kend == 0, or a stage past
// the end) thus still reads inside the band. ks0 % U == 0, kend <= ks_total.
template <int U>
__device__ __forceinline__ void fp4_load(Fp4StageU<U> &st, const Fp4Band &b, int ks0, int kend) {
    const int last = kend > 0 ? kend - 1 : 0;
#pragma unroll
    for (int u = 0; u < U; u++) {
        int ks = min(ks0 + u, last);
        st.w[u] = ldg16_stream(b.w + (size_t)ks * 1024);
    }
    const int sk = min(ks0, last);
    if (U == 8) st.s = *(const uint2 *)(b.s + (size_t)(sk / 8) * 512);
    else st.s.x = *(const uint32_t *)(b.s + (size_t)(sk / 8) * 512 + (sk & 4));
}

// K range [k0, k1) of part `part` of `parts` over `ksteps` 128-K steps, in
// whole 8-step stages (so every stage starts on an 8-step scale group).
__device__ __forceinline__ void k_part8(int ksteps, int part, int parts, int &k0, int &k1) {
    const int stages = (ksteps + kU - 1) / kU;
    k0 = min(ksteps, part * stages / parts * kU);
    k1 = min(ksteps, (part + 1) * stages / parts * kU);
}

template <int U>
__device__ __forceinline__ uint32_t stage_scale(const Fp4StageU<U> &st, int u) {
    return ((u < 4 ? st.s.x : st.s.y) >> (8 * (u & 3))) & 0xFF;
}

}  // namespace ws
