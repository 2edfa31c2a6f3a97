// RMSNorm arithmetic shared by every kernel that normalizes an activation
// (rmsnorm_q8_1, rmsnorm_fp16 and the GEMV prologues that fuse RMSNorm), so
// that all of them produce the same inverse RMS for the same input, bit for
// bit, whatever their block size (reference: src/kernels/rmsnorm_rope.cu:
// 75-138 and :156-233; inv_rms = 1/sqrt(mean(x^2) + eps) in fp32, rounded to
// fp16 before the two fp16 multiplies).
//
// The sum of squares has one fixed order:
//   * unit u (elements 8u..8u+7): s_u = x0*x0, then s_u = fma(xe, xe, s_u)
//     for e = 1..7;
//   * lane l of wave 0 adds s_l, s_{l+64}, s_{l+128}, ... in that order;
//   * the 64 lane sums meet through the xor butterfly of seg_sum<64>.
// Kernels store their units' s_u in LDS and call rms_inv_f16 or
// rms_inv_f16_each_wave.
#pragma once

#include "qe_common.hpp"

namespace qe {

__device__ __forceinline__ float rms_unit_sq(uint4 raw) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = h2f(static_cast<uint16_t>(w[j] & 0xFFFFu));
        v[2 * j + 1] = h2f(static_cast<uint16_t>(w[j] >> 16));
    }
    float s = v[0] * v[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) s = __builtin_fmaf(v[e], v[e], s);
    return s;
}

// fp16(1 / sqrt(total / H + eps)) from the unit sums s_units[0..U) (U = H / 8)
// in LDS.  Every thread of the block must call it (two barriers); the first
// one makes the callers' stores of s_units visible.
__device__ __forceinline__ _Float16 rms_inv_f16(const float* s_units, int U, int H, float eps, float* s_total) {
    __syncthreads();
    if (threadIdx.x < 64) {
        float p = 0.0f;
        for (int u = threadIdx.x; u < U; u += 64) p += s_units[u];
        p = qwen::seg_sum<64>(p);
        if (threadIdx.x == 0) *s_total = p;
    }
    __syncthreads();
    const float inv_rms = 1.0f / sqrtf(*s_total / static_cast<float>(H) + eps);
    return static_cast<_Float16>(inv_rms);
}

// The same value with one barrier: every wave sums the units itself in the
// order above (lane l: s_l, s_{l+64}, ...; then the butterfly), so all waves
// hold the wave-0 result bit for bit and nothing is broadcast through LDS.
// The caller must not overwrite s_units afterwards without a barrier.
__device__ __forceinline__ _Float16 rms_inv_f16_each_wave(const float* s_units, int U, int H, float eps) {
    __syncthreads();
    const int l = threadIdx.x & 63;
    float p = 0.0f;
    for (int u = l; u < U; u += 64) p += s_units[u];
    p = qwen::seg_sum<64>(p);
    const float inv_rms = 1.0f / sqrtf(p / static_cast<float>(H) + eps);
    return static_cast<_Float16>(inv_rms);
}

}  // namespace qe
