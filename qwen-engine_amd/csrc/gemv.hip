// W4A8 / W4A16 group-128 decode GEMV family for gfx950.
//
// Math (bit-for-bit on the integer stage) of src/kernels/gemv_w4a16.cu:
//   per 32-element chunk: dot = sum of 4 dp4a_w4_q8_oct (sum8-seeded),
//   acc += float(dot) * (float(w_scale) * x_scale),  y = fp16(acc [+ res]).
//
// Layout of the work (MI355X-first, not the reference's 8-lane sub-warps):
//   * A "segment" of LPR lanes (LPR in 8..64, a power of two inside one
//     wave64) owns one output row (two for SwiGLU).  Lane l of the segment
//     owns the 32-element chunks c = l + i*LPR, i < NCH, of every row.
//   * Each lane keeps the Q8_1 activation of its chunks in VGPRs for the
//     whole kernel (13 dwords per chunk), so the weight stream is the only
//     per-row memory traffic: one 16-byte global_load_dwordx4 per chunk,
//     fully coalesced (16*LPR contiguous bytes per segment per load).
//   * Partial sums are reduced inside the segment with DPP row operations
//     (quad_perm, row_half_mirror, row_mirror) and ds_swizzle for 32 lanes.
//   * Blocks are 256 threads; the grid is capped at 8 blocks per CU and
//     loops over row sets, so x is staged once per block.
// Shapes the fast kernel does not cover (unaligned weights, K > 16384)
// go to a generic wave-per-row kernel with x staged in LDS.
#include "qe_common.hpp"

namespace qe {
namespace {

constexpr int kPlain = 0;
constexpr int kQKV = 1;
constexpr int kSwiglu = 2;

struct GemvParams {
    const uint32_t* qw[3];
    const uint16_t* sc[3];
    uint16_t* out[3];
    int row_begin[3];  // first virtual row of each matrix (QKV mode)
    const uint16_t* residual;
    const int8_t* q8;
    const float* xs;
    const int32_t* s8;
    const uint16_t* x16;  // fp16 activation (W4A16 entry points)
    int n_out;            // output rows (SwiGLU: intermediate features)
    int K;
};

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// fp16 x -> Q8_1 in LDS, 16 lanes per group, whole block (256 threads).
__device__ __forceinline__ void quantize_x_to_lds(const uint16_t* __restrict__ x, int K, int8_t* s_q8,
                                                  int32_t* s_s8, float* s_xs) {
    const int G = K >> 7;
    const int sub = threadIdx.x & 15;
    for (int g = threadIdx.x >> 4; g < G; g += (blockDim.x >> 4)) {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + g * 128 + sub * 8);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
        float vals[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vals[2 * j] = h2f(static_cast<uint16_t>(w[j] & 0xFFFFu));
            vals[2 * j + 1] = h2f(static_cast<uint16_t>(w[j] >> 16));
        }
        const qwen::Q8Group q = qwen::quantize_group128_q8_1(vals);
        *reinterpret_cast<int2*>(s_q8 + g * 128 + sub * 8) = make_int2(q.x_lo, q.x_hi);
        s_s8[g * 16 + sub] = q.sum8;
        if (sub == 0) s_xs[g] = q.d;
    }
}

__device__ __forceinline__ int32_t chunk_dot(const u32x4 w, const int4 xa, const int4 xb, const int4 s8) {
    return qwen::dp4a_w4_q8_oct(w.x, xa.x, xa.y, s8.x) + qwen::dp4a_w4_q8_oct(w.y, xa.z, xa.w, s8.y) +
           qwen::dp4a_w4_q8_oct(w.z, xb.x, xb.y, s8.z) + qwen::dp4a_w4_q8_oct(w.w, xb.z, xb.w, s8.w);
}

template <int LPR, int NCH, int MODE, bool F16IN>
__global__ __launch_bounds__(256) void gemv_w4_kernel(GemvParams p) {
    constexpr int SEGS = 256 / LPR;
    const int K = p.K;
    const int KC = K >> 5;
    const int G = K >> 7;
    const int seg = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;

    // ---- activation slice of this lane, kept in VGPRs --------------------
    const int8_t* q8 = p.q8;
    const int32_t* s8 = p.s8;
    const float* xs = p.xs;
    if constexpr (F16IN) {
        extern __shared__ __align__(16) uint8_t s_mem[];
        int8_t* s_q8 = reinterpret_cast<int8_t*>(s_mem);
        int32_t* s_s8 = reinterpret_cast<int32_t*>(s_mem + K);
        float* s_xs = reinterpret_cast<float*>(s_mem + K + (K >> 3) * 4);
        quantize_x_to_lds(p.x16, K, s_q8, s_s8, s_xs);
        __syncthreads();
        q8 = s_q8;
        s8 = s_s8;
        xs = s_xs;
    }
    int4 xa[NCH], xb[NCH], xsum[NCH];
    float xd[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = l + i * LPR;
        if (c < KC) {
            xa[i] = *reinterpret_cast<const int4*>(q8 + c * 32);
            xb[i] = *reinterpret_cast<const int4*>(q8 + c * 32 + 16);
            xsum[i] = *reinterpret_cast<const int4*>(s8 + c * 4);
            xd[i] = xs[c >> 2];
        } else {
            xa[i] = xb[i] = xsum[i] = make_int4(0, 0, 0, 0);
            xd[i] = 0.0f;
        }
    }

    const int stride = SEGS * gridDim.x;
    for (int r = blockIdx.x * SEGS + seg; r < p.n_out; r += stride) {
        if constexpr (MODE == kSwiglu) {
            const size_t rg = static_cast<size_t>(2 * r);
            const u32x4* wg = reinterpret_cast<const u32x4*>(p.qw[0] + rg * (K >> 3));
            const u32x4* wu = reinterpret_cast<const u32x4*>(p.qw[0] + (rg + 1) * (K >> 3));
            const uint16_t* sg = p.sc[0] + rg * G;
            const uint16_t* su = p.sc[0] + (rg + 1) * G;
            u32x4 w0[NCH], w1[NCH];
            uint16_t h0[NCH], h1[NCH];
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int c = min(l + i * LPR, KC - 1);  // clamped: no branches around the loads
                w0[i] = __builtin_nontemporal_load(wg + c);
                w1[i] = __builtin_nontemporal_load(wu + c);
                h0[i] = sg[c >> 2];
                h1[i] = su[c >> 2];
            }
            float ag = 0.0f, au = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; ++i) {  // out-of-range chunks have a zero x slice
                ag += static_cast<float>(chunk_dot(w0[i], xa[i], xb[i], xsum[i])) * (h2f(h0[i]) * xd[i]);
                au += static_cast<float>(chunk_dot(w1[i], xa[i], xb[i], xsum[i])) * (h2f(h1[i]) * xd[i]);
            }
            ag = qwen::seg_sum<LPR>(ag);
            au = qwen::seg_sum<LPR>(au);
            if (l == 0) p.out[0][r] = f2h(silu_mul(ag, au));
        } else {
            int m = 0;
            int row = r;
            if constexpr (MODE == kQKV) {
                m = (r >= p.row_begin[1]) + (r >= p.row_begin[2]);
                row = r - p.row_begin[m];
            }
            const u32x4* wr = reinterpret_cast<const u32x4*>(p.qw[m] + static_cast<size_t>(row) * (K >> 3));
            const uint16_t* sr = p.sc[m] + static_cast<size_t>(row) * G;
            u32x4 w0[NCH];
            uint16_t h0[NCH];
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int c = min(l + i * LPR, KC - 1);
                w0[i] = __builtin_nontemporal_load(wr + c);
                h0[i] = sr[c >> 2];
            }
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; ++i)
                acc += static_cast<float>(chunk_dot(w0[i], xa[i], xb[i], xsum[i])) * (h2f(h0[i]) * xd[i]);
            acc = qwen::seg_sum<LPR>(acc);
            if (l == 0) {
                if (MODE == kPlain && p.residual != nullptr) acc += h2f(p.residual[row]);
                p.out[m][row] = f2h(acc);
            }
        }
    }
}

// Generic kernel: one wave per output row (pair), dword weight loads, Q8_1
// staged in LDS with scalar copies.  Covers any K % 128 == 0 up to the LDS
// limit and any 4-byte weight alignment (the reference's uint32 fallback,
// src/kernels/gemv_w4a16.cu:264-630).
template <int MODE, bool F16IN>
__global__ __launch_bounds__(256) void gemv_w4_generic_kernel(GemvParams p) {
    extern __shared__ __align__(16) uint8_t s_mem[];
    const int K = p.K;
    const int G = K >> 7;
    const int KW = K >> 3;
    int8_t* s_q8 = reinterpret_cast<int8_t*>(s_mem);
    int32_t* s_s8 = reinterpret_cast<int32_t*>(s_mem + K);
    float* s_xs = reinterpret_cast<float*>(s_mem + K + KW * 4);
    if constexpr (F16IN) {
        const int sub = threadIdx.x & 15;
        for (int g = threadIdx.x >> 4; g < G; g += 16) {
            float vals[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) vals[j] = h2f(p.x16[g * 128 + sub * 8 + j]);
            const qwen::Q8Group q = qwen::quantize_group128_q8_1(vals);
            reinterpret_cast<int32_t*>(s_q8)[(g * 128 + sub * 8) / 4] = q.x_lo;
            reinterpret_cast<int32_t*>(s_q8)[(g * 128 + sub * 8) / 4 + 1] = q.x_hi;
            s_s8[g * 16 + sub] = q.sum8;
            if (sub == 0) s_xs[g] = q.d;
        }
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) s_q8[i] = p.q8[i];
        for (int i = threadIdx.x; i < KW; i += blockDim.x) s_s8[i] = p.s8[i];
        for (int i = threadIdx.x; i < G; i += blockDim.x) s_xs[i] = p.xs[i];
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int stride = 4 * gridDim.x;
    const int32_t* xq = reinterpret_cast<const int32_t*>(s_q8);
    for (int r = blockIdx.x * 4 + wave; r < p.n_out; r += stride) {
        const int nrows = (MODE == kSwiglu) ? 2 : 1;
        float acc[2] = {0.0f, 0.0f};
        int m = 0;
        int row = r;
        if constexpr (MODE == kQKV) {
            m = (r >= p.row_begin[1]) + (r >= p.row_begin[2]);
            row = r - p.row_begin[m];
        }
        for (int k = 0; k < nrows; ++k) {
            const size_t rr = (MODE == kSwiglu) ? static_cast<size_t>(2 * r + k) : static_cast<size_t>(row);
            const uint32_t* wr = p.qw[m] + rr * KW;
            const uint16_t* sr = p.sc[m] + rr * G;
            float a = 0.0f;
            for (int w = l; w < KW; w += 64) {
                const int32_t d = qwen::dp4a_w4_q8_oct(wr[w], xq[2 * w], xq[2 * w + 1], s_s8[w]);
                a += static_cast<float>(d) * (h2f(sr[w >> 4]) * s_xs[w >> 4]);
            }
            acc[k] = qwen::seg_sum<64>(a);
        }
        if (l == 0) {
            if constexpr (MODE == kSwiglu) {
                p.out[0][r] = f2h(silu_mul(acc[0], acc[1]));
            } else {
                float v = acc[0];
                if (MODE == kPlain && p.residual != nullptr) v += h2f(p.residual[row]);
                p.out[m][row] = f2h(v);
            }
        }
    }
}

constexpr int kMaxFastK = 64 * 8 * 32;   // LPR 64 x 8 chunks x 32 elements
constexpr int kMaxGenericK = 32768;      // Q8_1 staging: 1.53 B per element of LDS

// LPR: the widest segment that still gives each lane >= 3 chunks (enough
// independent 16-byte loads in flight per lane); NCH rounded up to an
// instantiated register budget.
struct Plan {
    int lpr;
    int nch;
};

Plan plan_for(int K) {
    const int KC = K / 32;
    int lpr = 8;
    for (int c : {64, 32, 16, 8}) {
        if ((KC + c - 1) / c >= 3) { lpr = c; break; }
    }
    int nch = (KC + lpr - 1) / lpr;
    static const int kNch[] = {1, 2, 3, 4, 5, 6, 8};
    for (int n : kNch) {
        if (n >= nch) { nch = n; break; }
    }
    return {lpr, nch};
}

template <int MODE, bool F16IN, int LPR>
hipError_t launch_lpr(int nch, const GemvParams& p, int grid, size_t lds, hipStream_t s) {
    switch (nch) {
#define QE_NCH(N) \
    case N: gemv_w4_kernel<LPR, N, MODE, F16IN><<<grid, 256, lds, s>>>(p); break;
        QE_NCH(1) QE_NCH(2) QE_NCH(3) QE_NCH(4) QE_NCH(5) QE_NCH(6) QE_NCH(8)
#undef QE_NCH
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

template <int MODE, bool F16IN>
int launch_gemv(const GemvParams& p, bool fast_ok, hipStream_t stream, const char* what) {
    const int K = p.K;
    if (p.n_out <= 0) return QE_OK;
    const int max_grid = cu_count() * 8;
    if (fast_ok && K <= kMaxFastK) {
        const Plan pl = plan_for(K);
        const int segs = 256 / pl.lpr;
        int grid = (p.n_out + segs - 1) / segs;
        if (grid > max_grid) grid = max_grid;
        const size_t lds = F16IN ? static_cast<size_t>(K) + K / 2 + K / 32 : 0;
        hipError_t e = hipSuccess;
        switch (pl.lpr) {
            case 8: e = launch_lpr<MODE, F16IN, 8>(pl.nch, p, grid, lds, stream); break;
            case 16: e = launch_lpr<MODE, F16IN, 16>(pl.nch, p, grid, lds, stream); break;
            case 32: e = launch_lpr<MODE, F16IN, 32>(pl.nch, p, grid, lds, stream); break;
            default: e = launch_lpr<MODE, F16IN, 64>(pl.nch, p, grid, lds, stream); break;
        }
        if (e != hipSuccess) return fail(QE_ERR_UNSUPPORTED, "%s: no kernel for K=%d", what, K);
    } else {
        if (K > kMaxGenericK) return fail(QE_ERR_UNSUPPORTED, "%s: in_features=%d exceeds %d", what, K, kMaxGenericK);
        int grid = (p.n_out + 3) / 4;
        if (grid > max_grid) grid = max_grid;
        const size_t lds = static_cast<size_t>(K) + K / 2 + K / 32;
        gemv_w4_generic_kernel<MODE, F16IN><<<grid, 256, lds, stream>>>(p);
    }
    return check_launch(what);
}

int check_common(const char* what, int K, const void* q8, const void* xs, const void* s8, const void* x16) {
    QE_REQUIRE(K > 0 && K % 128 == 0, "%s: in_features=%d must be a positive multiple of 128", what, K);
    if (x16 == nullptr) QE_REQUIRE(q8 && xs && s8, "%s: Q8_1 input pointers must not be NULL", what);
    return QE_OK;
}

bool act_fast_ok(const GemvParams& p) {
    if (p.x16) return aligned(p.x16, 16);
    return aligned(p.q8, 16) && aligned(p.s8, 16);
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_launch_gemv_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                                   const float* input_scale, const int32_t* input_sum8, const uint16_t* residual,
                                   uint16_t* output_y, int out_features, int in_features, hipStream_t stream) {
    const char* what = "gemv_w4a8";
    if (int rc = check_common(what, in_features, input_q8, input_scale, input_sum8, nullptr)) return rc;
    QE_REQUIRE(qweight && scales && output_y, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(out_features >= 0, "%s: out_features=%d", what, out_features);
    QE_REQUIRE(aligned(qweight, 4) && aligned(scales, 2), "%s: weights must be 4-byte aligned", what);
    GemvParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = output_y;
    p.residual = residual;
    p.q8 = input_q8;
    p.xs = input_scale;
    p.s8 = input_sum8;
    p.n_out = out_features;
    p.K = in_features;
    const bool fast = aligned(qweight, 16) && act_fast_ok(p);
    return launch_gemv<kPlain, false>(p, fast, stream, what);
}

extern "C" int qe_launch_gemv_qkv_w4a8(const qe_qkv_view* view, const int8_t* input_q8, const float* input_scale,
                                       const int32_t* input_sum8, hipStream_t stream, int in_features,
                                       int num_q_heads, int num_kv_heads, int head_dim) {
    const char* what = "gemv_qkv_w4a8";
    if (int rc = check_common(what, in_features, input_q8, input_scale, input_sum8, nullptr)) return rc;
    QE_REQUIRE(view != nullptr, "%s: view is NULL", what);
    QE_REQUIRE(num_q_heads >= 0 && num_kv_heads >= 0 && head_dim >= 0, "%s: negative head shape", what);
    const int q_dim = num_q_heads * head_dim;
    const int kv_dim = num_kv_heads * head_dim;
    const void* w[3] = {view->q_weight, view->k_weight, view->v_weight};
    const uint16_t* s[3] = {view->q_scale, view->k_scale, view->v_scale};
    uint16_t* o[3] = {view->d_q, view->d_k, view->d_v};
    const int rows[3] = {q_dim, kv_dim, kv_dim};
    bool fast = true;
    GemvParams p{};
    for (int i = 0; i < 3; ++i) {
        if (rows[i] == 0) continue;
        QE_REQUIRE(w[i] && s[i] && o[i], "%s: NULL pointer in view (matrix %d)", what, i);
        QE_REQUIRE(aligned(w[i], 4) && aligned(s[i], 2), "%s: weights must be 4-byte aligned", what);
        fast = fast && aligned(w[i], 16);
        p.qw[i] = static_cast<const uint32_t*>(w[i]);
        p.sc[i] = s[i];
        p.out[i] = o[i];
    }
    p.row_begin[0] = 0;
    p.row_begin[1] = q_dim;
    p.row_begin[2] = q_dim + kv_dim;
    p.q8 = input_q8;
    p.xs = input_scale;
    p.s8 = input_sum8;
    p.n_out = q_dim + 2 * kv_dim;
    p.K = in_features;
    fast = fast && act_fast_ok(p);
    return launch_gemv<kQKV, false>(p, fast, stream, what);
}

extern "C" int qe_launch_gemv_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                                       const int8_t* input_q8, const float* input_scale,
                                                       const int32_t* input_sum8, uint16_t* output_mlp,
                                                       int hidden_size, int intermediate_size, hipStream_t stream) {
    const char* what = "gemv_dual_gate_up_swiglu_w4a8";
    if (int rc = check_common(what, hidden_size, input_q8, input_scale, input_sum8, nullptr)) return rc;
    QE_REQUIRE(gate_up_qweight && gate_up_scales && output_mlp, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(gate_up_qweight, 4) && aligned(gate_up_scales, 2), "%s: weights must be 4-byte aligned", what);
    GemvParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.q8 = input_q8;
    p.xs = input_scale;
    p.s8 = input_sum8;
    p.n_out = intermediate_size;
    p.K = hidden_size;
    const bool fast = aligned(gate_up_qweight, 16) && act_fast_ok(p);
    return launch_gemv<kSwiglu, false>(p, fast, stream, what);
}

extern "C" int qe_launch_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                                    const uint16_t* residual, uint16_t* output_y, int out_features, int in_features,
                                    hipStream_t stream) {
    const char* what = "gemv_w4a16";
    if (int rc = check_common(what, in_features, nullptr, nullptr, nullptr, input_x)) return rc;
    QE_REQUIRE(input_x && qweight && scales && output_y, "%s: NULL pointer", what);
    QE_REQUIRE(out_features >= 0, "%s: out_features=%d", what, out_features);
    QE_REQUIRE(aligned(qweight, 4) && aligned(scales, 2) && aligned(input_x, 2), "%s: misaligned buffer", what);
    GemvParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = output_y;
    p.residual = residual;
    p.x16 = input_x;
    p.n_out = out_features;
    p.K = in_features;
    const bool fast = aligned(qweight, 16) && act_fast_ok(p);
    return launch_gemv<kPlain, true>(p, fast, stream, what);
}

extern "C" int qe_launch_gemv_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight,
                                                        const uint16_t* gate_up_scales, const uint16_t* input_x,
                                                        uint16_t* output_mlp, int hidden_size, int intermediate_size,
                                                        hipStream_t stream) {
    const char* what = "gemv_dual_gate_up_swiglu_w4a16";
    if (int rc = check_common(what, hidden_size, nullptr, nullptr, nullptr, input_x)) return rc;
    QE_REQUIRE(input_x && gate_up_qweight && gate_up_scales && output_mlp, "%s: NULL pointer", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(gate_up_qweight, 4) && aligned(gate_up_scales, 2) && aligned(input_x, 2),
               "%s: misaligned buffer", what);
    GemvParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.x16 = input_x;
    p.n_out = intermediate_size;
    p.K = hidden_size;
    const bool fast = aligned(gate_up_qweight, 16) && act_fast_ok(p);
    return launch_gemv<kSwiglu, true>(p, fast, stream, what);
}
