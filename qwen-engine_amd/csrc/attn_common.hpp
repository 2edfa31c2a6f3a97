// Split-K flash-decode combine arithmetic shared by the stand-alone combine
// kernel (attention.hip) and the O-projection GEMV that folds the combine into
// its activation staging (gemv.hip).  Both compile these exact expressions, so
// the two paths give bit-identical results.
//
// Reference: src/kernels/attention_gqa.cu:230-310 (stage 2: merge of the 16
// split partials, then the Q8_1 epilogue, one group per head).
#pragma once
#include "qe_common.hpp"

namespace qe {

constexpr int kFlashSplits = 16;  // FLASH_DECODE_SPLITS, include/config.cuh:29

// Split weights w_s = exp(m_s - m) / sum_t d_t exp(m_t - m) over the splits
// that hold positions (d_s > 0); m is their largest max.  With no positions
// at all every weight is 0.  m_s is in natural-log units; exp uses exp2.
__device__ __forceinline__ void flash_split_weights(const float (&ms)[kFlashSplits], const float (&ds)[kFlashSplits],
                                                    float (&wt)[kFlashSplits]) {
    float mg = -INFINITY;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s)
        if (ds[s] > 0.0f) mg = fmaxf(mg, ms[s]);
    constexpr float kLog2e = 1.4426950408889634f;
    float es[kFlashSplits];
    float dg = 0.0f;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s) {
        es[s] = ds[s] > 0.0f ? __builtin_amdgcn_exp2f((ms[s] - mg) * kLog2e) : 0.0f;
        dg += ds[s] * es[s];
    }
    const float inv = dg > 0.0f ? 1.0f / dg : 0.0f;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s) wt[s] = es[s] * inv;
}

// One output element: sum_s w_s * o_s over the non-empty splits (the
// partials of empty splits are never read as numbers).
__device__ __forceinline__ float flash_combine(const float (&ds)[kFlashSplits], const float (&wt)[kFlashSplits],
                                               const float (&os)[kFlashSplits]) {
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s) acc += ds[s] > 0.0f ? wt[s] * os[s] : 0.0f;
    return acc;
}

// Q8_1 of one attention value: d = max(max|acc| over the head / 127, 1e-8),
// q = clamp(rint(acc / d), -127, 127) (attention_gqa.cu:263-310; rint here,
// where the activation quantizer rounds half away from zero).
__device__ __forceinline__ float flash_q8_scale(float head_max_abs) { return fmaxf(head_max_abs / 127.0f, 1e-8f); }
__device__ __forceinline__ int flash_q8_value(float acc, float d) {
    const int v = static_cast<int>(rintf(acc / d));
    return max(-127, min(127, v));
}

}  // namespace qe
