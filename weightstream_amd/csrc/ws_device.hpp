// Device helpers shared by the gfx950 kernels: the reference's FP8/FP4/UE8M0
// encodings, the per-32 activation quantiser, wave reductions and the
// CDNA4 scaled-MFMA wrapper.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ws_expf.h"
#include "ws_logf.h"

namespace ws {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// MFMA operand format codes of v_mfma_scale_f32_*_f8f6f4 (cbsz / blgp).
constexpr int kFmtFp8 = 0;   // e4m3
constexpr int kFmtFp4 = 4;   // e2m1
constexpr int kScaleOne = 127;  // UE8M0 byte of 1.0

// UE8M0 byte -> f32 (weightstream-core quant.rs:41-48): 2^(b-127) built from
// bits, exact for every byte including b=0 (2^-127, subnormal).
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
    uint32_t bits = b ? (b << 23) : 0x00400000u;   // selects, no branch
    bits = (b == 0xFF) ? 0x7FC00000u : bits;
    return __uint_as_float(bits);
}

// quant.rs:60-73 log2_ceil via the exponent field.
__device__ __forceinline__ int log2_ceil(float x) {
    uint32_t bits = __float_as_uint(x);
    int e = (int)((bits >> 23) & 0xFF) - 127;
    return (bits & 0x7FFFFF) ? e + 1 : e;
}

// e4m3fn decode (quant.rs:24-39): sign * 2^(E-7) * (1 + M/8), subnormal M/512.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    uint32_t e = (b >> 3) & 0xF, m = b & 7;
    float mag;
    if (e == 0xF && m == 7) return __builtin_nanf("");
    if (e == 0) mag = (float)m * (1.0f / 512.0f);
    else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
    return (b & 0x80) ? -mag : mag;
}

// f32 -> e4m3 byte exactly as weightstream-core quant.rs:103-137 computes it:
// RNE, saturating at +-448, NaN -> 0x7F|sign. In the subnormal range a value
// rounding up to 2^-6 returns 0x38, as the reference does (quant.rs:120-122);
// inputs reaching that branch are in [15/1024, 2^-6).
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
    // branch-free: both the normal-range and the subnormal encoding are
    // computed and selected (the exponent arithmetic of the unused one may
    // be garbage); equal to the reference rule on all 2^32 inputs (device
    // digest against the oracle, tests/test_gpu_route.py)
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 24) & 0x80;
    const float a = __builtin_fabsf(v);
    const int e = (int)((bits >> 23) & 0xFF) - 127;
    // normal range: 3 mantissa bits, rounded to nearest even
    const float q = fminf(a * __builtin_ldexpf(1.0f, min(3 - e, 126)), 32.0f);
    const int m8 = (int)__builtin_rintf(q);
    const bool up = m8 == 16;
    const uint32_t cn = ((uint32_t)(up ? e + 8 : e + 7) << 3) | (uint32_t)(up ? 0 : m8 - 8);
    // below 2^-6: multiples of 2^-9 (a result of 2^-6 encodes as 0x38)
    const int m = (int)__builtin_rintf(fminf(a, 1.0f) * 512.0f);
    const uint32_t cs = m == 8 ? 0x38u : (uint32_t)m;
    uint32_t c = a < 0.015625f ? cs : cn;
    c = a >= 448.0f ? 0x7Eu : c;
    c = (v != v) ? 0x7Fu : c;
    return sign | c;
}

// Rust f32::clamp (NaN passes through).
__device__ __forceinline__ float rclamp(float v, float lo, float hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// bf16 RNE of quant.rs:95-101.
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    uint32_t bits = __float_as_uint(v);
    uint32_t round = ((bits >> 16) & 1) + 0x7FFF;
    return (uint16_t)((bits + round) >> 16);
}

// Compiler-only barrier: memory accesses are not moved across it, so loads
// issued before it leave the wave first (load counters then return them in
// issue order and a wait for them does not cover later loads).
__device__ __forceinline__ void mem_order() { __asm__ volatile("" ::: "memory"); }

// Workgroup barrier with no memory-model fences: the caller has already waited
// (s_waitcnt) for whatever other waves will read, e.g. its own direct
// global->LDS copies; global loads issued before it stay in flight. The
// compiler-only barriers keep memory accesses on their side of it.
__device__ __forceinline__ void raw_barrier() {
    mem_order();
    __builtin_amdgcn_s_barrier();
    mem_order();
}

// LDS reads the compiler does not see as memory accesses. After direct
// global->LDS loads into other buffers are issued, the compiler would make an
// ordinary LDS read wait for all of them (it cannot tell the buffers apart);
// these reads are ordered by the caller instead: issue them, then
// lds_wait_all() and lds_ready() on every result before use.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
__device__ __forceinline__ u32x4v lds_read_b128(uint32_t a) {
    u32x4v v;
    __asm__ volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a));
    return v;
}
__device__ __forceinline__ uint32_t lds_read_b32(uint32_t a) {
    uint32_t v;
    __asm__ volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(a));
    return v;
}
// LDS store the compiler does not see (so it adds no wait for outstanding
// direct global->LDS loads); ordered by the caller with lds_wait_all().
__device__ __forceinline__ void lds_write_b32(uint32_t a, uint32_t v) {
    __asm__ volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_wait_all() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// Wait until at most N of this wave's LDS reads (lds_read_*) are in flight;
// LDS reads complete in issue order.
template <int N>
__device__ __forceinline__ void lds_wait() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N) : "memory");
}
template <class T>
__device__ __forceinline__ void lds_ready(T &v) { __asm__ volatile("" : "+v"(v)); }

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maximum).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until at most `newer` steps' loads (L per step) of this wave are in
// flight; newer <= KMAX.
template <int L, int KMAX>
__device__ __forceinline__ void wait_newer(int newer) {
    if constexpr (KMAX > 0) {
        if (newer >= KMAX) wait_vm<KMAX * L>();
        else wait_newer<L, KMAX - 1>(newer);
    } else {
        wait_vm<0>();
    }
}

// Barrier that orders LDS only: global loads issued before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ws_expf with the 32-entry table held in lane registers: lane l holds
// ws_exp2f_tab[l % 32] (ws_lane_exp2f_tab) and the entry is fetched with a
// lane permute instead of a memory load, from the lane's own half-wave. Same
// arithmetic as ws_expf. Every lane of the half-wave must take part.
__device__ __forceinline__ uint64_t ws_lane_exp2f_tab(int lane) { return ws_exp2f_tab[lane & 31]; }

__device__ __forceinline__ float ws_expf_lanes(float x, uint64_t tab) {
    uint64_t ki = 0;
    double r = 0.0;
    float out = 0.0f;
    const int special = ws_expf_reduce(x, &ki, &r, &out);
    const int j = (int)(__lane_id() & 32) | (int)(ki & 31);
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)tab, j, 64);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(tab >> 32), j, 64);
    const float v = ws_expf_finish(ki, r, ((uint64_t)hi << 32) | lo);
    return special ? out : v;
}

// num.rs:71 sigmoid, 1/(1+exp(-x)), on ws_expf_lanes
__device__ __forceinline__ float ws_sigmoid_lanes(float x, uint64_t tab) {
WS_NO_CONTRACT
    return 1.0f / (1.0f + ws_expf_lanes(-x, tab));
}

// num.rs:79 silu, x * sigmoid(x), on ws_expf_lanes
__device__ __forceinline__ float ws_silu_lanes(float x, uint64_t tab) {
WS_NO_CONTRACT
    return x * ws_sigmoid_lanes(x, tab);
}

// Max over the 32 lanes of each half-wave (lanes 0-31 and 32-63 reduce
// separately). Max is exact, so the order does not matter.
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// e4m3_to_f32(f32_to_e4m3(v)) without the byte: v rounded to the e4m3 grid
// (3 mantissa bits, RNE; multiples of 2^-9 below 2^-6, where a value rounding
// up to 2^-6 gives 1.0 as the encoder's 0x38 decodes; 448 at and above 448;
// NaN -> the decoder's NaN). Equal to the composition on all 2^32 inputs
// (device digest against the oracle, tests/test_gpu_route.py).
__device__ __forceinline__ float e4m3_round_value(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = bits & 0x80000000u;
    const float a = __builtin_fabsf(v);
    const int e = (int)((bits >> 23) & 0xFF) - 127;
    const float m8 = __builtin_rintf(fminf(a * __builtin_ldexpf(1.0f, min(3 - e, 126)), 32.0f));
    const float vn = __builtin_ldexpf(m8, max(e - 3, -126));  // m8 2^(e-3), exact
    const float ms = __builtin_rintf(fminf(a, 1.0f) * 512.0f);
    const float vs = ms == 8.0f ? 1.0f : ms * 0.001953125f;  // m 2^-9, exact
    float r = a < 0.015625f ? vs : vn;
    r = a >= 448.0f ? 448.0f : r;
    const float sr = __uint_as_float(__float_as_uint(r) | sign);
    return (v != v) ? __builtin_nanf("") : sr;
}

// log2_ceil(amax / 448) from the bits of amax (amax >= 1e-4, or inf/NaN):
// with amax = M 2^E, M in [1, 2), the correctly rounded quotient is exactly
// 2^(E-8) when M == 1.75, just above it when M > 1.75 and in
// [2^(E-9), 2^(E-8)) when M < 1.75, so the ceiling is E - 8 + (M > 1.75);
// inf / 448 = inf (128) and NaN / 448 = NaN (129). Equal to the division
// form for every input (device digest against the oracle,
// tests/test_gpu_route.py).
__device__ __forceinline__ int log2_ceil_div448(float amax) {
    const uint32_t b = __float_as_uint(amax);
    const int ef = (int)((b >> 23) & 0xFF);
    const uint32_t mant = b & 0x7FFFFF;
    return ef == 255 ? (mant ? 129 : 128) : ef - 135 + (mant > 0x600000u ? 1 : 0);
}

// Max over each aligned group of 8 lanes by DPP moves (half-row mirror,
// then quad swaps 2 and 1): every lane ends with the maximum of its group.
__device__ __forceinline__ float max8_lanes(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));
    return v;
}

// x / 2^e for a block scale exponent e, as x * 2^-e. For a finite block
// maximum the rule yields e in [-22, 120], where 2^-e is an exact normal f32
// and the product is the quotient, rounded the same way. A block holding an
// infinity has e = 128: the reference divides by 2^128 = inf, which sends a
// finite x to a signed zero (so does the factor 0 below) and an infinity to
// the invalid-operation NaN, whose sign bit the host (x86) sets: its byte is
// 0xFF, whatever the infinity's sign (block_byte). A NaN x stays that NaN.
__device__ __forceinline__ float block_inv_scale(int e) {
    return e >= 128 ? 0.0f : __builtin_ldexpf(1.0f, -e);
}
__device__ __forceinline__ uint32_t block_byte(float x, float inv) {
    const uint32_t b = f32_to_e4m3(rclamp(x * inv, -448.0f, 448.0f));
    return (inv == 0.0f && __builtin_fabsf(x) == __builtin_inff()) ? 0xFFu : b;
}

// FP8 activation quantisation of one 1x32 block held one value per lane in a
// 32-lane group (weightstream-ref actquant.rs:21-45 / act_quant_fp8_emit,
// actquant.cu:47): amax floored at 1e-4, scale 2^log2_ceil(amax/448),
// q = e4m3(clamp(x/s, +-448)). Returns the e4m3 byte; *scale_byte gets the
// UE8M0 byte. fmaxf drops NaN like the reference's `a > amax` scan.
__device__ __forceinline__ uint32_t quant_fp8_block32(float x, uint32_t *scale_byte) {
    float amax = half_wave_max(__builtin_fabsf(x));
    if (!(amax >= 1e-4f)) amax = 1e-4f;  // an all-NaN block too, as the reference's scan
    int e = log2_ceil_div448(amax);
    *scale_byte = (uint32_t)(e + 127) & 0xFF;
    return block_byte(x, block_inv_scale(e));
}

// The scale byte quant_fp8_block32 gives a block of zeros (the 1e-4 floor)
__device__ __forceinline__ uint32_t zero_block_scale_byte() {
    return (uint32_t)(log2_ceil_div448(1e-4f) + 127) & 0xFF;
}

// The same block quantisation with four consecutive values per lane, a block
// being 8 lanes (a lane-group of 8 aligned lanes): the bytes of
// quant_fp8_block32, packed low value first. The block maximum is
// order-free.
__device__ __forceinline__ uint32_t quant_fp8_block32_x4(float4 v, uint32_t *scale_byte) {
    float amax = fmaxf(fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
                       fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)));
    amax = max8_lanes(amax);
    if (!(amax >= 1e-4f)) amax = 1e-4f;  // an all-NaN block too, as the reference's scan
    const int e = log2_ceil_div448(amax);
    *scale_byte = (uint32_t)(e + 127) & 0xFF;
    const float inv = block_inv_scale(e);
    return block_byte(v.x, inv) | (block_byte(v.y, inv) << 8) | (block_byte(v.z, inv) << 16) |
           (block_byte(v.w, inv) << 24);
}

// Scaled MFMA, 16x16 output, K = 128: D += (A * 2^sa) (B * 2^sb).
// Operand layout (measured on gfx950): lane l supplies row (A) / column (B)
// l % 16. With g = l / 16, an FP8 operand lane holds K [16g, 16g+16) in its
// bytes 0-15 and K [64+16g, 64+16g+16) in bytes 16-31; an FP4 operand lane
// holds K [32g, 32g+32) in bytes 0-15, low nibble first. The UE8M0 byte of
// lane l scales K block [32g, 32g+32) of its row/column, for either format.
// D: lane l, element v holds row 4*(l/16)+v, column l%16.
template <int FMT_A, int FMT_B>
__device__ __forceinline__ v4f mfma_scaled(const v8i &a, const v8i &b, v4f c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, 0, sa, 0, sb);
}

// 16-byte global load that bypasses nothing special; kept in one place so the
// load flavour of every streaming kernel can be changed together.
__device__ __forceinline__ uint4 ldg16(const uint8_t *p) {
    return *reinterpret_cast<const uint4 *>(p);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ldg16_stream(const uint8_t *p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return uint4{v[0], v[1], v[2], v[3]};
}

__device__ __forceinline__ v8i frag_from(uint4 lo, uint4 hi) {
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
    return r;
}

__device__ __forceinline__ v8i frag_from4(uint4 lo) {
    v8i r;
    r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
    r[4] = 0; r[5] = 0; r[6] = 0; r[7] = 0;
    return r;
}

// ---- exact math: dequantise to bf16, accumulate with bf16 MFMA -----------
// The FP8/FP4 scaled MFMAs of gfx950 sum their products at reduced internal
// precision (measured: about 2^-11 of sum|p| per instruction, against 2^-24
// for an f32 sum), while v_mfma_f32_16x16x32_bf16 accumulates in f32
// (measured: 2e-7 of sum|p|). Every e4m3 / e2m1 value times a UE8M0 scale is
// exactly representable in bf16 (4 and 2 significant bits, f32 exponent
// range), so converting with v_cvt_scalef32_pk_bf16_{fp8,fp4} and running bf16
// MFMAs computes the reference's dequantise-then-f32-accumulate product.
// A lane's 32 K-values [32g, 32g+32) of one 128-K step feed 4 MFMAs of K=32,
// 8 values each; operand A and B use the same assignment, so the dot product
// covers every K exactly once.

__device__ __forceinline__ u32x4v pk4(v2bf a, v2bf b, v2bf c, v2bf d) {
    return u32x4v{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                  __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
}

// 32 e4m3 bytes (K 0-15 in lo, 16-31 in hi) * scale -> 4 x 8 bf16
__device__ __forceinline__ void cvt_fp8x32(uint4 lo, uint4 hi, float s, v8bf out[4]) {
    const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        u32x4v v = pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j], s, false),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j], s, true),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j + 1], s, false),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j + 1], s, true));
        out[j] = __builtin_bit_cast(v8bf, v);
    }
}

// 16 packed e2m1 bytes (32 values, low nibble first) * scale -> 4 x 8 bf16
__device__ __forceinline__ void cvt_fp4x32(uint4 q, float s, v8bf out[4]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
        u32x4v v = pk4(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], s, 0),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], s, 1),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], s, 2),
                       __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], s, 3));
        out[j] = __builtin_bit_cast(v8bf, v);
    }
}

__device__ __forceinline__ v4f mfma_bf16_k128(const v8bf a[4], const v8bf b[4], v4f c) {
#pragma unroll
    for (int j = 0; j < 4; j++) c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], b[j], c, 0, 0, 0);
    return c;
}

}  // namespace ws
