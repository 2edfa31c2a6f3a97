// Q8_1 activation quantizers and RMSNorm for gfx950.
//
// Reference behaviour: src/kernels/rmsnorm_rope.cu:75-314 (RMSNorm, fused
// RMSNorm+Q8_1, standalone fp16->Q8_1) with the rounding of the CPU golden
// (tests/test_kernels.cu:311-326).  These kernels move a few KB and are
// launch-latency bound; they are written to finish in one wave of blocks.
#include "qe_common.hpp"
#include "rms_common.hpp"

namespace qe {
namespace {

constexpr int kGroup = 128;

// One 16-lane DPP row per 128-element group; 16 groups per 256-thread block.
__global__ __launch_bounds__(256) void quantize_fp16_to_q8_1_kernel(
    const uint16_t* __restrict__ x, int8_t* __restrict__ q8, float* __restrict__ scale,
    int32_t* __restrict__ sum8, int num_groups) {
    const int group = blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    if (group >= num_groups) return;  // whole 16-lane rows drop out together
    const uint4 raw = *reinterpret_cast<const uint4*>(x + static_cast<size_t>(group) * kGroup + sub * 8);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float vals[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        vals[2 * j] = h2f(static_cast<uint16_t>(w[j] & 0xFFFFu));
        vals[2 * j + 1] = h2f(static_cast<uint16_t>(w[j] >> 16));
    }
    const qwen::Q8Group g = qwen::quantize_group128_q8_1(vals);
    if (q8) *reinterpret_cast<int2*>(q8 + static_cast<size_t>(group) * kGroup + sub * 8) = make_int2(g.x_lo, g.x_hi);
    if (sum8) sum8[group * 16 + sub] = g.sum8;
    if (scale && sub == 0) scale[group] = g.d;
}

// inv_rms = 1/sqrt(mean(x^2) + eps) in fp32 with the shared summation order
// (rms_common.hpp); the normalized value is fp16(fp16(x * fp16(inv_rms)) *
// gamma), the two fp16 multiplies of rmsnorm_rope.cu:130-136 / :214-227.
// s_units: H / 8 floats of LDS.
__device__ __forceinline__ _Float16 inv_rms_f16(const uint16_t* __restrict__ xr, int H, float eps, float* s_units,
                                                float* s_total) {
    for (int i = threadIdx.x; i < H / 8; i += blockDim.x)
        s_units[i] = rms_unit_sq(*reinterpret_cast<const uint4*>(xr + i * 8));
    return rms_inv_f16(s_units, H / 8, H, eps, s_total);
}

__device__ __forceinline__ uint4 norm8(uint4 xv, uint4 gv, _Float16 h) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        qwen::qe_half2_t xx = __builtin_bit_cast(qwen::qe_half2_t, xw[j]);
        qwen::qe_half2_t gg = __builtin_bit_cast(qwen::qe_half2_t, gw[j]);
        qwen::qe_half2_t hh = {h, h};
        qwen::qe_half2_t n = xx * hh;  // rounded to fp16
        n = n * gg;                    // rounded to fp16
        o[j] = __builtin_bit_cast(uint32_t, n);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ __launch_bounds__(256) void rmsnorm_fp16_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, uint16_t* __restrict__ out, int H, float eps) {
    extern __shared__ __align__(16) float s_units[];  // H / 8
    __shared__ float s_total;
    const uint16_t* xr = x + static_cast<size_t>(blockIdx.x) * H;
    uint16_t* orow = out + static_cast<size_t>(blockIdx.x) * H;
    const _Float16 h = inv_rms_f16(xr, H, eps, s_units, &s_total);
    for (int i = threadIdx.x; i < H / 8; i += blockDim.x) {
        const uint4 xv = *reinterpret_cast<const uint4*>(xr + i * 8);
        const uint4 gv = *reinterpret_cast<const uint4*>(gamma + i * 8);
        *reinterpret_cast<uint4*>(orow + i * 8) = norm8(xv, gv, h);
    }
}

// One token: RMSNorm into LDS (and optionally HBM), then Q8_1 of the
// fp16-rounded normalized values.  Dynamic LDS: H fp16 (2H bytes, at most
// 128 KiB).  The unit sums of squares (H / 8 floats) use the same LDS: they
// are dead once rms_inv_f16 returns (its second barrier follows the last
// read), before the first normalized value is stored.
__global__ __launch_bounds__(256) void rmsnorm_q8_1_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma, uint16_t* out_opt,
    int8_t* __restrict__ q8, float* __restrict__ scale, int32_t* __restrict__ sum8, int H, float eps) {
    extern __shared__ __align__(16) uint16_t s_norm[];
    __shared__ float s_total;
    float* s_units = reinterpret_cast<float*>(s_norm);
    const _Float16 h = inv_rms_f16(x, H, eps, s_units, &s_total);
    for (int i = threadIdx.x; i < H / 8; i += blockDim.x) {
        const uint4 xv = *reinterpret_cast<const uint4*>(x + i * 8);
        const uint4 gv = *reinterpret_cast<const uint4*>(gamma + i * 8);
        const uint4 n = norm8(xv, gv, h);
        *reinterpret_cast<uint4*>(s_norm + i * 8) = n;
        if (out_opt) *reinterpret_cast<uint4*>(out_opt + i * 8) = n;
    }
    __syncthreads();
    const int G = H / kGroup;
    const int sub = threadIdx.x & 15;
    for (int group = threadIdx.x >> 4; group < G; group += 16) {
        const uint4 raw = *reinterpret_cast<const uint4*>(s_norm + group * kGroup + sub * 8);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        float vals[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vals[2 * j] = h2f(static_cast<uint16_t>(w[j] & 0xFFFFu));
            vals[2 * j + 1] = h2f(static_cast<uint16_t>(w[j] >> 16));
        }
        const qwen::Q8Group g = qwen::quantize_group128_q8_1(vals);
        if (q8) *reinterpret_cast<int2*>(q8 + group * kGroup + sub * 8) = make_int2(g.x_lo, g.x_hi);
        if (sum8) sum8[group * 16 + sub] = g.sum8;
        if (scale && sub == 0) scale[group] = g.d;
    }
}

constexpr float kRmsEps = 1e-6f;  // RMS_NORM_EPS, include/config.cuh:20

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_launch_quantize_fp16_to_q8_1(const uint16_t* input_x, int8_t* out_q8, float* out_scale,
                                               int32_t* out_sum8, int num_elements, hipStream_t stream) {
    QE_REQUIRE(input_x != nullptr, "quantize_fp16_to_q8_1: input_x is NULL");
    QE_REQUIRE(num_elements >= 0 && num_elements % kGroup == 0,
               "quantize_fp16_to_q8_1: num_elements=%d must be a multiple of 128", num_elements);
    QE_REQUIRE(aligned(input_x, 16) && aligned(out_q8, 8) && aligned(out_scale, 4) && aligned(out_sum8, 4),
               "quantize_fp16_to_q8_1: input must be 16-byte aligned, q8 8-byte aligned");
    const int G = num_elements / kGroup;
    if (G == 0) return QE_OK;
    quantize_fp16_to_q8_1_kernel<<<(G + 15) / 16, 256, 0, stream>>>(input_x, out_q8, out_scale, out_sum8, G);
    return check_launch("quantize_fp16_to_q8_1");
}

extern "C" int qe_launch_rmsnorm_q8_1(const uint16_t* input, const uint16_t* gamma, uint16_t* output_fp16_opt,
                                      int8_t* out_q8, float* out_scale, int32_t* out_sum8,
                                      hipStream_t stream, int hidden_size) {
    QE_REQUIRE(input && gamma, "rmsnorm_q8_1: input/gamma is NULL");
    QE_REQUIRE(hidden_size > 0 && hidden_size % kGroup == 0 && hidden_size <= 65536,
               "rmsnorm_q8_1: hidden_size=%d must be a positive multiple of 128 (<= 65536)", hidden_size);
    QE_REQUIRE(aligned(input, 16) && aligned(gamma, 16) && aligned(output_fp16_opt, 16) && aligned(out_q8, 8),
               "rmsnorm_q8_1: input, gamma and output must be 16-byte aligned");
    rmsnorm_q8_1_kernel<<<1, 256, hidden_size * sizeof(uint16_t), stream>>>(
        input, gamma, output_fp16_opt, out_q8, out_scale, out_sum8, hidden_size, kRmsEps);
    return check_launch("rmsnorm_q8_1");
}

extern "C" int qe_launch_rmsnorm_fp16(const uint16_t* input, const uint16_t* gamma, uint16_t* output,
                                      int num_tokens, hipStream_t stream, int hidden_size) {
    QE_REQUIRE(input && gamma && output, "rmsnorm_fp16: NULL pointer");
    QE_REQUIRE(hidden_size > 0 && hidden_size % 8 == 0 && hidden_size <= 65536,
               "rmsnorm_fp16: hidden_size=%d must be a positive multiple of 8 (<= 65536)", hidden_size);
    QE_REQUIRE(aligned(input, 16) && aligned(gamma, 16) && aligned(output, 16),
               "rmsnorm_fp16: buffers must be 16-byte aligned");
    if (num_tokens <= 0) return QE_OK;
    rmsnorm_fp16_kernel<<<num_tokens, 256, hidden_size / 8 * sizeof(float), stream>>>(input, gamma, output,
                                                                                       hidden_size, kRmsEps);
    return check_launch("rmsnorm_fp16");
}
