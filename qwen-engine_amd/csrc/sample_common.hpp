// Sampling primitives shared by the sampling kernels and the LM-head GEMV
// epilogue: (value, index) reductions with the reference's tie rule and the
// Philox-4x32-10 / Gumbel noise of src/kernels/sampling.cu:13-105.
#pragma once

#include "qe_common.hpp"

namespace qe {

struct Best {
    float v;
    int32_t i;
};

// larger value wins; equal values keep the lower index; NaN never compares greater
__device__ __forceinline__ Best better(Best a, Best b) {
    return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ __forceinline__ Best wave_best(Best b) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        Best o{__shfl_xor(b.v, m), __shfl_xor(b.i, m)};
        b = better(b, o);
    }
    return b;
}

// Philox-4x32-10 with counter (subsequence, offset, 0, 0) and key = seed;
// only the first output word is used (sampling.cu:13-53).
__device__ __forceinline__ uint32_t philox_word0(uint64_t seed, uint32_t subsequence, uint32_t offset) {
    uint32_t c0 = subsequence, c1 = offset, c2 = 0u, c3 = 0u;
    uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c0), lo0 = 0xD2511F53u * c0;
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c2), lo1 = 0xCD9E8D57u * c2;
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// value compared by sample_stage1_kernel: logit, or logit / T + Gumbel(u)
// with u = clamp((float(word) + 1) / 4294967298, 1e-7, 1 - 1e-7)
__device__ __forceinline__ float sample_value(float logit, float temperature, uint64_t seed, uint32_t index,
                                              uint32_t seq_pos) {
    if (!(temperature > 1e-5f)) return logit;
    const float u0 = (static_cast<float>(philox_word0(seed, index, seq_pos)) + 1.0f) / 4294967298.0f;
    const float u = fminf(fmaxf(u0, 1e-7f), 1.0f - 1e-7f);
    return logit / temperature + -logf(-logf(u));
}

}  // namespace qe
