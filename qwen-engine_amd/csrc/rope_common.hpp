// NeoX rotary embedding arithmetic shared by the bias+RoPE+KV-append kernel
// and the QKV GEMV epilogue, so the two paths round identically
// (reference: src/kernels/rmsnorm_rope.cu:320-423).
#pragma once

#include "qe_common.hpp"

namespace qe {

// angle pos * theta^(-2i/rot) of rotation pair i
__device__ __forceinline__ void rope_sincos(int pos, int i, int rot, float rope_theta, float& sn, float& cs) {
    const float inv_freq = exp2f(-2.0f * static_cast<float>(i) / static_cast<float>(rot) * log2f(rope_theta));
    sincosf(static_cast<float>(pos) * inv_freq, &sn, &cs);
}

// element e of a pair (x0 = first half, x1 = second half): x = own value, y = partner
__device__ __forceinline__ float rope_rotate(float x, float y, bool first_half, float sn, float cs) {
    return first_half ? x * cs - y * sn : y * sn + x * cs;  // (x0 c - x1 s, x0 s + x1 c)
}

}  // namespace qe
