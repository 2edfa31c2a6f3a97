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

// Positions per split for a context of seq_len positions: the reference's
// ceil(seq_len / 16), but at least kFlashMinSplit, so that short contexts
// fill fewer splits (one round of loads per block either way) and the
// combine reads fewer partials.  Splits past the context hold no positions.
// (64 measured best for configs[4] decode: 32 and 128 were 3-5 % slower)
constexpr int kFlashMinSplit = 64;
__host__ __device__ __forceinline__ int flash_split_len(int seq_len) {
    const int per = (seq_len + kFlashSplits - 1) / kFlashSplits;
    return per > kFlashMinSplit ? per : kFlashMinSplit;
}
__host__ __device__ __forceinline__ int flash_live_splits(int seq_len) {
    const int per = flash_split_len(seq_len);
    return (seq_len + per - 1) / per;
}

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
// partials of empty splits are never read as numbers).  Product and sum are
// rounded separately (no fused multiply-add), so that skipping splits known
// to be empty (flash_combine_live) gives the same bits: acc starts at +0 and
// adding +0 never changes it.
__device__ __forceinline__ float flash_combine(const float (&ds)[kFlashSplits], const float (&wt)[kFlashSplits],
                                               const float (&os)[kFlashSplits]) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s) acc += ds[s] > 0.0f ? wt[s] * os[s] : 0.0f;
    return acc;
}

// The same over the first `live` splits only (block-uniform); every split
// from `live` on holds no positions.
__device__ __forceinline__ float flash_combine_live(const float (&ds)[kFlashSplits], const float (&wt)[kFlashSplits],
                                                    const float (&os)[kFlashSplits], int live) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s)
        if (s < live) acc += ds[s] > 0.0f ? wt[s] * os[s] : 0.0f;
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
