// Sampling (greedy argmax or Gumbel-max at a temperature) + sequence advance for gfx950.
//
// Reference: src/kernels/sampling.cu:60-232.  Per thread a strict '>' scan
// from (-1e30, index 0); reductions keep the larger value and, on equal
// values, the lower index.  NaN never compares greater, so it never wins.
// Stage 1: 256 blocks x 256 threads write (value, index) partials; stage 2:
// one block reduces them and advances the device control block.
#include "sample_common.hpp"

namespace qe {
namespace {

// 256 threads -> one (value, index) per block, written by thread 0.
__device__ __forceinline__ Best block_best(Best b) {
    __shared__ float s_v[4];
    __shared__ int32_t s_i[4];
    b = wave_best(b);
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = b.v;
        s_i[threadIdx.x >> 6] = b.i;
    }
    __syncthreads();
    Best r{s_v[0], s_i[0]};
    for (int w = 1; w < 4; ++w) r = better(r, Best{s_v[w], s_i[w]});
    return r;
}

// Stage 1: per thread a strict '>' scan in index order (sample_stage1_kernel,
// sampling.cu:60-105), the compared value being the logit or, with
// temperature > 1e-5, logit / T plus the Gumbel noise of that index.
__global__ __launch_bounds__(256) void argmax_stage1_kernel(const uint16_t* __restrict__ logits, int n,
                                                            float* __restrict__ val, int32_t* __restrict__ idx,
                                                            const qe_device_control_block* ctl) {
    float temp = 0.0f;
    uint64_t seed = 0;
    uint32_t seq_pos = 0;
    if (ctl != nullptr) {
        temp = ctl->temperature;
        seed = ctl->rng_seed;
        seq_pos = static_cast<uint32_t>(ctl->seq_pos);
    }
    Best b{-1e30f, 0};
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const float v = sample_value(h2f(logits[i]), temp, seed, static_cast<uint32_t>(i), seq_pos);
        if (v > b.v) {
            b.v = v;
            b.i = i;
        }
    }
    b = block_best(b);
    if (threadIdx.x == 0) {
        val[blockIdx.x] = b.v;
        idx[blockIdx.x] = b.i;
    }
}

// Stage 2: one block reduces nparts partials (sampling.cu:111-205) and
// advances the control block: token_id, seq_pos + 1, rng_seed + golden ratio.
__global__ __launch_bounds__(256) void argmax_stage2_advance_kernel(const float* __restrict__ val,
                                                                    const int32_t* __restrict__ idx, int nparts,
                                                                    qe_device_control_block* d_control,
                                                                    int32_t* d_pinned) {
    Best b{-1e30f, 0};
    for (int i = threadIdx.x; i < nparts; i += 256) b = better(b, Best{val[i], idx[i]});
    b = block_best(b);
    if (threadIdx.x == 0) {
        if (d_control) {
            d_control->token_id = b.i;
            d_control->seq_pos += 1;
            d_control->rng_seed += 0x9E3779B97F4A7C15ull;
        }
        if (d_pinned) *d_pinned = b.i;
    }
}

}  // namespace
}  // namespace qe

using namespace qe;

// Second stage of the fused LM-head + sampling launches (gemv.hip).
namespace qe {
int launch_sample_stage2(const float* val, const int32_t* idx, int nparts, qe_device_control_block* d_control,
                         int32_t* d_pinned, hipStream_t stream) {
    argmax_stage2_advance_kernel<<<1, 256, 0, stream>>>(val, idx, nparts, d_control, d_pinned);
    return QE_OK;
}
}  // namespace qe

extern "C" int qe_launch_sample_and_advance(const uint16_t* logits, float* sample_scratch_val,
                                            int32_t* sample_scratch_idx, qe_device_control_block* d_control,
                                            int32_t* d_mapped_pinned_token, hipStream_t stream, int vocab_size) {
    QE_REQUIRE(logits && sample_scratch_val && sample_scratch_idx, "sample_and_advance: NULL pointer");
    QE_REQUIRE(vocab_size > 0, "sample_and_advance: vocab_size=%d", vocab_size);
    constexpr int kParts = 256;
    argmax_stage1_kernel<<<kParts, 256, 0, stream>>>(logits, vocab_size, sample_scratch_val, sample_scratch_idx,
                                                     d_control);
    argmax_stage2_advance_kernel<<<1, 256, 0, stream>>>(sample_scratch_val, sample_scratch_idx, kParts, d_control,
                                                        d_mapped_pinned_token);
    return check_launch("sample_and_advance");
}
