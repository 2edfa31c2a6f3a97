// quant_primitives.hpp — gfx950 device primitives of the W4A16 G128 path.
//
// Same names and meaning as the reference's include/quant_primitives.cuh,
// written for CDNA4: v_dot4_i32_i8 (sdot4) instead of __dp4a, DPP row
// operations instead of warp shuffles, wave64 lanes.  HIP device code only.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qwen {

// ---- cross-lane helpers (DPP within a 16-lane row, ds_swizzle across 32) --
// DPP controls (GFX9 encoding): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
// ds_swizzle bit-mode: and_mask=0x1F, xor_mask=0x10 -> lane ^ 16 within 32 lanes.
__device__ __forceinline__ float swz_xor16_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// All-reduce (sum) over aligned groups of SEG lanes; every lane of the group
// ends with the total.  SEG in {1,2,4,8,16,32,64}.
template <int SEG>
__device__ __forceinline__ float seg_sum(float v) {
    if constexpr (SEG >= 2) v += dpp_f32<0xB1>(v);
    if constexpr (SEG >= 4) v += dpp_f32<0x4E>(v);
    if constexpr (SEG >= 8) v += dpp_f32<0x141>(v);
    if constexpr (SEG >= 16) v += dpp_f32<0x140>(v);
    if constexpr (SEG >= 32) v += swz_xor16_f32(v);
    if constexpr (SEG >= 64) v += __shfl_xor(v, 32);
    return v;
}

template <int SEG>
__device__ __forceinline__ float seg_max(float v) {
    if constexpr (SEG >= 2) v = fmaxf(v, dpp_f32<0xB1>(v));
    if constexpr (SEG >= 4) v = fmaxf(v, dpp_f32<0x4E>(v));
    if constexpr (SEG >= 8) v = fmaxf(v, dpp_f32<0x141>(v));
    if constexpr (SEG >= 16) v = fmaxf(v, dpp_f32<0x140>(v));
    if constexpr (SEG >= 32) v = fmaxf(v, swz_xor16_f32(v));
    if constexpr (SEG >= 64) v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

// Max over aligned groups of SEG <= 16 lanes of values that are >= +0 and
// not NaN: their bit patterns order as unsigned integers, so each step is one
// DPP-fused integer max (no NaN canonicalization).
template <int SEG>
__device__ __forceinline__ float seg_max_nonneg(float v) {
    static_assert(SEG <= 16, "DPP row");
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    if constexpr (SEG >= 2) u = max(u, static_cast<uint32_t>(dpp_i32<0xB1>(static_cast<int>(u))));
    if constexpr (SEG >= 4) u = max(u, static_cast<uint32_t>(dpp_i32<0x4E>(static_cast<int>(u))));
    if constexpr (SEG >= 8) u = max(u, static_cast<uint32_t>(dpp_i32<0x141>(static_cast<int>(u))));
    if constexpr (SEG >= 16) u = max(u, static_cast<uint32_t>(dpp_i32<0x140>(static_cast<int>(u))));
    return __builtin_bit_cast(float, u);
}

// ---- integer dot primitives ---------------------------------------------
// compute_q8_sum8 (reference quant_primitives.cuh:13-17): -8 * sum of the
// 8 signed bytes of (x_lo, x_hi).
__device__ __forceinline__ int32_t compute_q8_sum8(int32_t x_lo, int32_t x_hi) {
    int32_t s = __builtin_amdgcn_sdot4(0x01010101, x_hi, 0, false);
    s = __builtin_amdgcn_sdot4(0x01010101, x_lo, s, false);
    return -8 * s;
}

// dp4a_w4_q8_oct (reference quant_primitives.cuh:28-32): sum_j (q_j-8)*x_j
// over one packed word = sdot4(w_hi, x_hi, sdot4(w_lo, x_lo, sum8)).
// Nibbles are 0..15, so they are valid signed int8 lanes of sdot4.
__device__ __forceinline__ int32_t dp4a_w4_q8_oct(uint32_t packed, int32_t x_lo, int32_t x_hi, int32_t x_sum8) {
    int32_t w_lo = static_cast<int32_t>(packed & 0x0F0F0F0Fu);
    int32_t w_hi = static_cast<int32_t>((packed >> 4) & 0x0F0F0F0Fu);
    return __builtin_amdgcn_sdot4(w_hi, x_hi, __builtin_amdgcn_sdot4(w_lo, x_lo, x_sum8, false), false);
}

// ---- Q8_1 quantization of one 128-element group --------------------------
// 16 consecutive lanes hold 8 values each (lane l: elements 8l..8l+7).
// d = max(max|x|/127, 1e-8) (IEEE division), inv_d = 1/d (IEEE),
// q = clamp(roundf(x*inv_d), +-127) with roundf = half away from zero, as the
// reference CPU golden (tests/test_kernels.cu:311-326).  The caller's 16-lane
// group must be a DPP row (lane index multiple of 16).
struct Q8Group {
    int32_t x_lo, x_hi;  // packed q8 of the lane's 8 elements
    int32_t sum8;        // -8 * sum of those 8 values
    float d;             // group scale (same in all 16 lanes)
};

__device__ __forceinline__ Q8Group quantize_group128_q8_1(const float vals[8]) {
#pragma clang fp contract(off)
    float max_abs = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) max_abs = fmaxf(max_abs, fabsf(vals[j]));
    max_abs = seg_max_nonneg<16>(max_abs);  // fmaxf from +0 never yields NaN or -0
    float d = fmaxf(max_abs / 127.0f, 1e-8f);
    float inv_d = 1.0f / d;
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // roundf (half away from zero) as trunc(y + copysign(0.5 - 2^-25, y)):
        // equal to roundf for every |y| < 2^23 (checked exhaustively on the
        // host); the product is rounded on its own, never fused into the add.
        // No clamp to +-127 is needed: |vals[j]| <= max_abs and rounding is
        // monotonic, and max_abs * inv_d rounds to at most 127 for every
        // positive finite max_abs (checked exhaustively on the host); NaN
        // converts to 0 as before.
        const float y = vals[j] * inv_d;
        const int v = static_cast<int>(y + __builtin_copysignf(0.49999997f, y));
        b[j] = static_cast<uint32_t>(v) & 0xFFu;
    }
    Q8Group g;
    g.x_lo = static_cast<int32_t>(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24));
    g.x_hi = static_cast<int32_t>(b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
    g.sum8 = compute_q8_sum8(g.x_lo, g.x_hi);
    g.d = d;
    return g;
}

// quantize_group128_fp16_to_q8_1 (reference quant_primitives.cuh:37-89): the
// reference's entry point, same parameters and meaning.  The 16 lanes of a
// 128-element group (an aligned DPP row, all 16 active) each pass their 8
// values; lane `sub_lane` (0..15) of group `group_idx` stores its 8 q8 bytes
// at out_q8[128*group_idx + 8*sub_lane] (one 8-byte store) and its sum8 at
// out_sum8[16*group_idx + sub_lane]; sub_lane 0 stores the scale d at
// out_scale[group_idx].  A nullptr output is skipped.  Rounding is the CPU
// golden's (half away from zero), see quantize_group128_q8_1.
__device__ __forceinline__ void quantize_group128_fp16_to_q8_1(const float vals[8], int group_idx, int sub_lane,
                                                               int8_t* out_q8, float* out_scale, int32_t* out_sum8) {
    const Q8Group g = quantize_group128_q8_1(vals);
    if (out_q8 != nullptr)
        *reinterpret_cast<int2*>(out_q8 + static_cast<size_t>(group_idx) * 128 + sub_lane * 8) = make_int2(g.x_lo, g.x_hi);
    if (out_sum8 != nullptr) out_sum8[static_cast<size_t>(group_idx) * 16 + sub_lane] = g.sum8;
    if (out_scale != nullptr && sub_lane == 0) out_scale[group_idx] = g.d;
}

// ---- int4 -> fp16 dequantization -------------------------------------------
// unpack_w4_to_half2_quad (reference quant_primitives.cuh:92-115): the 8
// elements of a packed word in K order, (q-8)*scale with one fp16 RNE
// multiply.  (q-8) is formed exactly with the 0x6400 (1024.0) bias.
typedef _Float16 qe_half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 qe_half8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ qe_half8_t unpack_w4_to_half8(uint32_t packed, _Float16 scale) {
    // bytes (q0|q4<<4, 0x64, q1|q5<<4, 0x64) and (q2|q6<<4, 0x64, q3|q7<<4, 0x64):
    // masking the high nibble of the even bytes gives 0x6400|q as fp16 pairs
    const uint32_t x01 = __builtin_amdgcn_perm(0x64646464u, packed, 0x04010400u);
    const uint32_t x23 = __builtin_amdgcn_perm(0x64646464u, packed, 0x04030402u);
    const uint32_t u01 = x01 & 0xFF0FFF0Fu;
    const uint32_t u23 = x23 & 0xFF0FFF0Fu;
    const uint32_t u45 = ((x01 >> 4) & 0x000F000Fu) | 0x64006400u;
    const uint32_t u67 = ((x23 >> 4) & 0x000F000Fu) | 0x64006400u;
    const qe_half2_t b = {(_Float16)1032.0f, (_Float16)1032.0f};
    const qe_half2_t s = {scale, scale};
    qe_half2_t h01 = (__builtin_bit_cast(qe_half2_t, u01) - b) * s;
    qe_half2_t h23 = (__builtin_bit_cast(qe_half2_t, u23) - b) * s;
    qe_half2_t h45 = (__builtin_bit_cast(qe_half2_t, u45) - b) * s;
    qe_half2_t h67 = (__builtin_bit_cast(qe_half2_t, u67) - b) * s;
    return qe_half8_t{h01[0], h01[1], h23[0], h23[1], h45[0], h45[1], h67[0], h67[1]};
}

// unpack_w4_to_half2_quad (reference quant_primitives.cuh:92-115): the
// reference's entry point, same parameters and meaning: out_h2[i] holds
// elements (2i, 2i+1) of the word in K order, each (q-8)*scale rounded once
// to fp16 (RNE).  Same arithmetic as unpack_w4_to_half8.
__device__ __forceinline__ void unpack_w4_to_half2_quad(uint32_t packed, half scale, half2 out_h2[4]) {
    const qe_half8_t h = unpack_w4_to_half8(packed, __builtin_bit_cast(_Float16, scale));
#pragma unroll
    for (int i = 0; i < 4; ++i) out_h2[i] = __builtin_bit_cast(half2, qe_half2_t{h[2 * i], h[2 * i + 1]});
}

}  // namespace qwen
