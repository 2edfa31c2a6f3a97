// Prefill W4A16 dequant-GEMM on CDNA4 matrix cores (gfx950).
//
// Math of src/kernels/gemm_prefill.cu: Y[M,N] = A[M,K] . Wdq[N,K]^T with
// Wdq = fp16((q-8)*s) (unpack_w4_to_half2_quad, quant_primitives.cuh:92-115),
// fp32 accumulation, fp16 output; residual added after rounding as an fp16
// add (the vector epilogue, gemm_prefill.cu:261-275); QKV split over three
// outputs (:392-489); gate/up SwiGLU over interleaved columns (:559-609).
//
// MI355X design:
//   * 256-thread blocks (4 wave64s in a 2x2 grid), block tile BM x BN with
//     BM, BN in {64, 128}; each wave owns (BM/2) x (BN/2) as 32x32 tiles of
//     v_mfma_f32_32x32x16_f16 (fp32 accumulators in VGPR/AGPR).
//   * K advances 32 at a time.  Per step, one 16-byte load brings the 32
//     packed int4 of one weight row (exactly one uint4), which a thread
//     dequantizes to 32 fp16 and stores to LDS; the A tile streams through
//     16-byte loads.  LDS is double-buffered (one barrier per K step) and
//     the next step's global loads are issued before the current MFMAs.
//   * LDS rows are padded to 40 halves (80 B) so the 16-byte fragment reads
//     of 32 consecutive rows spread over the banks.
//   * Tile shape is chosen per launch so the grid covers the 256 CUs.
#include "qe_common.hpp"

namespace qe {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPlain = 0;
constexpr int kQKV = 1;
constexpr int kSwiglu = 2;
constexpr int BK = 32;
constexpr int LDS_STRIDE = 40;  // halves per LDS row (32 + 8 pad)

struct GemmParams {
    const uint32_t* qw[3];
    const uint16_t* sc[3];
    uint16_t* out[3];
    int col_begin[3];  // first virtual column of each matrix (QKV)
    int out_stride[3]; // row stride of each output
    const uint16_t* A;
    const uint16_t* residual;
    int M, N, K;       // N = virtual columns (SwiGLU: 2*I)
};

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_w4a16_mfma_kernel(GemmParams p) {
    constexpr int WM = BM / 2;  // rows per wave
    constexpr int WN = BN / 2;  // cols per wave
    constexpr int MI = WM / 32;
    constexpr int NI = WN / 32;
    constexpr int A_U4 = BM * BK / 8 / 256;  // uint4 (8 halves) per thread for the A tile: 1 or 2
    static_assert(A_U4 >= 1, "tile too small");

    __shared__ __align__(16) _Float16 sA[2][BM * LDS_STRIDE];
    __shared__ __align__(16) _Float16 sB[2][BN * LDS_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = p.K;
    const int G = K >> 7;
    const int KT = K / BK;

    // ---- per-thread load assignments -----------------------------------
    // A: thread covers A_U4 consecutive uint4 of one row: row = tid / (4/A_U4)
    const int a_per_row = 4 / A_U4;            // threads per A row (BK/8 = 4 uint4 per row)
    const int a_row = tid / a_per_row;
    const int a_col = (tid % a_per_row) * A_U4 * 8;  // halves
    const int a_grow = m0 + a_row;
    const bool a_ok = a_row < BM && a_grow < p.M;
    const uint16_t* a_src = p.A + static_cast<size_t>(a_ok ? a_grow : 0) * K + a_col;
    // B: thread < BN owns weight row n0 + tid
    const bool b_thread = tid < BN;
    const int b_vcol = n0 + tid;
    bool b_ok = b_thread && b_vcol < p.N;
    const uint32_t* b_src = nullptr;
    const uint16_t* b_sc = nullptr;
    if (b_ok) {
        int m = 0, local = b_vcol;
        if constexpr (MODE == kQKV) {
            m = (b_vcol >= p.col_begin[1]) + (b_vcol >= p.col_begin[2]);
            local = b_vcol - p.col_begin[m];
        }
        b_src = p.qw[m] + static_cast<size_t>(local) * (K >> 3);
        b_sc = p.sc[m] + static_cast<size_t>(local) * G;
    }

    uint4 a_reg[A_U4];
    uint4 b_reg = make_uint4(0, 0, 0, 0);
    uint16_t b_s = 0;

    auto load_global = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < A_U4; ++i)
            a_reg[i] = a_ok ? *reinterpret_cast<const uint4*>(a_src + k0 + i * 8) : make_uint4(0, 0, 0, 0);
        if (b_ok) {
            b_reg = *reinterpret_cast<const uint4*>(b_src + (k0 >> 3));
            b_s = b_sc[k0 >> 7];
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_U4; ++i)
            *reinterpret_cast<uint4*>(&sA[buf][a_row * LDS_STRIDE + a_col + i * 8]) = a_reg[i];
        if (b_thread) {
            const _Float16 s = __builtin_bit_cast(_Float16, b_s);
            const uint32_t w[4] = {b_reg.x, b_reg.y, b_reg.z, b_reg.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qwen::qe_half8_t h = b_ok ? qwen::unpack_w4_to_half8(w[j], s) : qwen::qe_half8_t{};
                *reinterpret_cast<qwen::qe_half8_t*>(&sB[buf][tid * LDS_STRIDE + j * 8]) = h;
            }
        }
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int fr = lane & 31;        // fragment row (A) / column (B)
    const int fk = (lane >> 5) * 8;  // k offset of the lane's 8 halves
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) load_global(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            f16x8 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(&sA[buf][(wm * WM + i * 32 + fr) * LDS_STRIDE + kk + fk]);
#pragma unroll
            for (int j = 0; j < NI; ++j)
                bf[j] = *reinterpret_cast<const f16x8*>(&sB[buf][(wn * WN + j * 32 + fr) * LDS_STRIDE + kk + fk]);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) store_lds(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: D[i][j], j = lane%32, i = 8*(v/4) + 4*(lane/32) + v%4 ----
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int col = n0 + wn * WN + j * 32 + fr;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const float a = acc[i][j][v];
                if constexpr (MODE == kSwiglu) {
                    const float partner = __shfl_xor(a, 1);
                    if ((fr & 1) == 0 && row < p.M && col < p.N)
                        p.out[0][static_cast<size_t>(row) * p.out_stride[0] + (col >> 1)] = f2h(silu_mul(a, partner));
                } else {
                    if (row < p.M && col < p.N) {
                        int m = 0, local = col;
                        if constexpr (MODE == kQKV) {
                            m = (col >= p.col_begin[1]) + (col >= p.col_begin[2]);
                            local = col - p.col_begin[m];
                        }
                        const size_t off = static_cast<size_t>(row) * p.out_stride[m] + local;
                        _Float16 h = static_cast<_Float16>(a);
                        if (MODE == kPlain && p.residual != nullptr)
                            h = h + __builtin_bit_cast(_Float16, p.residual[off]);  // fp16 add, RNE
                        p.out[m][off] = __builtin_bit_cast(uint16_t, h);
                    }
                }
            }
        }
    }
}

template <int MODE>
int launch_gemm(const GemmParams& p, hipStream_t stream, const char* what) {
    if (p.M <= 0 || p.N <= 0) return QE_OK;
    const int cus = cu_count();
    auto blocks = [&](int bm, int bn) { return ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn); };
    // largest tile that still gives >= 1 block per CU; else the smallest tile
    int bm = 64, bn = 64;
    if (blocks(128, 128) >= cus) { bm = 128; bn = 128; }
    else if (blocks(64, 128) >= cus) { bm = 64; bn = 128; }
    else if (blocks(128, 64) >= cus) { bm = 128; bn = 64; }
    const dim3 grid((p.N + bn - 1) / bn, (p.M + bm - 1) / bm);
    if (grid.y > 65535) return fail(QE_ERR_UNSUPPORTED, "%s: M=%d too large", what, p.M);
    if (bm == 128 && bn == 128) gemm_w4a16_mfma_kernel<128, 128, MODE><<<grid, 256, 0, stream>>>(p);
    else if (bm == 64 && bn == 128) gemm_w4a16_mfma_kernel<64, 128, MODE><<<grid, 256, 0, stream>>>(p);
    else if (bm == 128 && bn == 64) gemm_w4a16_mfma_kernel<128, 64, MODE><<<grid, 256, 0, stream>>>(p);
    else gemm_w4a16_mfma_kernel<64, 64, MODE><<<grid, 256, 0, stream>>>(p);
    return check_launch(what);
}

int check_gemm_common(const char* what, const uint16_t* A, int M, int K) {
    QE_REQUIRE(A != nullptr, "%s: input_x is NULL", what);
    QE_REQUIRE(M >= 0, "%s: M=%d", what, M);
    QE_REQUIRE(K > 0 && K % 128 == 0, "%s: K=%d must be a positive multiple of 128", what, K);
    QE_REQUIRE(aligned(A, 16), "%s: input_x must be 16-byte aligned", what);
    return QE_OK;
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_launch_gemm_prefill_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                                            const uint16_t* residual, uint16_t* output_y, int M, int N, int K,
                                            hipStream_t stream, int sm_count) {
    (void)sm_count;
    const char* what = "gemm_prefill_w4a16";
    if (int rc = check_gemm_common(what, input_x, M, K)) return rc;
    QE_REQUIRE(qweight && scales && output_y, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(N >= 0, "%s: N=%d", what, N);
    QE_REQUIRE(aligned(qweight, 16) && aligned(scales, 2), "%s: qweight must be 16-byte aligned", what);
    GemmParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = output_y;
    p.out_stride[0] = N;
    p.A = input_x;
    p.residual = residual;
    p.M = M;
    p.N = N;
    p.K = K;
    return launch_gemm<kPlain>(p, stream, what);
}

extern "C" int qe_launch_gemm_prefill_qkv_w4a16(const qe_qkv_view* view, const uint16_t* input_x, int M,
                                                hipStream_t stream, int in_features, int num_q_heads,
                                                int num_kv_heads, int head_dim, int sm_count) {
    (void)sm_count;
    const char* what = "gemm_prefill_qkv_w4a16";
    if (int rc = check_gemm_common(what, input_x, M, in_features)) return rc;
    QE_REQUIRE(view != nullptr, "%s: view is NULL", what);
    QE_REQUIRE(num_q_heads >= 0 && num_kv_heads >= 0 && head_dim >= 0, "%s: negative head shape", what);
    const int q_dim = num_q_heads * head_dim;
    const int kv_dim = num_kv_heads * head_dim;
    const void* w[3] = {view->q_weight, view->k_weight, view->v_weight};
    const uint16_t* s[3] = {view->q_scale, view->k_scale, view->v_scale};
    uint16_t* o[3] = {view->d_q, view->d_k, view->d_v};
    const int cols[3] = {q_dim, kv_dim, kv_dim};
    GemmParams p{};
    for (int i = 0; i < 3; ++i) {
        p.out_stride[i] = cols[i];
        if (cols[i] == 0) continue;
        QE_REQUIRE(w[i] && s[i] && o[i], "%s: NULL pointer in view (matrix %d)", what, i);
        QE_REQUIRE(aligned(w[i], 16) && aligned(s[i], 2), "%s: weights must be 16-byte aligned", what);
        p.qw[i] = static_cast<const uint32_t*>(w[i]);
        p.sc[i] = s[i];
        p.out[i] = o[i];
    }
    p.col_begin[0] = 0;
    p.col_begin[1] = q_dim;
    p.col_begin[2] = q_dim + kv_dim;
    p.A = input_x;
    p.M = M;
    p.N = q_dim + 2 * kv_dim;
    p.K = in_features;
    return launch_gemm<kQKV>(p, stream, what);
}

extern "C" int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight,
                                                                const uint16_t* gate_up_scales,
                                                                const uint16_t* input_x, uint16_t* output_mlp, int M,
                                                                hipStream_t stream, int hidden_size,
                                                                int intermediate_size) {
    const char* what = "gemm_prefill_dual_gate_up_swiglu_w4a16";
    if (int rc = check_gemm_common(what, input_x, M, hidden_size)) return rc;
    QE_REQUIRE(gate_up_qweight && gate_up_scales && output_mlp, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(gate_up_qweight, 16) && aligned(gate_up_scales, 2), "%s: qweight must be 16-byte aligned",
               what);
    GemmParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.out_stride[0] = intermediate_size;
    p.A = input_x;
    p.M = M;
    p.N = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemm<kSwiglu>(p, stream, what);
}
