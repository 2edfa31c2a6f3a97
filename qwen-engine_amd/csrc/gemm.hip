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
//     v_mfma_f32_32x32x16_f16 (fp32 accumulators).
//   * The B operand of a lane (8 consecutive k of one weight column) is one
//     packed int4 word: each lane loads its 16-byte run of 32 k straight from
//     global memory and dequantizes it in registers ((q-8) via the 0x6400
//     bias, one fp16 RNE multiply by the group scale) - no LDS round trip and
//     no barrier for the weights.  A (fp16 activations) is staged through a
//     double-buffered LDS tile.  K advances 64 per step; A and B loads run in
//     a 4-stage register ring, so three steps of loads are in flight.
//   * Tile shape is chosen per launch so the grid covers the 256 CUs; when
//     64x64 tiles still leave CUs idle (small M, e.g. K = 8960 at M = 128)
//     K is split into slices whose fp32 partials a second kernel reduces in
//     slice order.
#include <algorithm>

#include "qe_common.hpp"

namespace qe {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPlain = 0;
constexpr int kQKV = 1;
constexpr int kSwiglu = 2;
constexpr int BK = 64;
constexpr int A_STRIDE = 72;  // halves per LDS row of the A tile (64 + 8 pad)

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

// Split-K scratch: fp32 partial tiles of the K slices, reduced by a second
// kernel on the same stream (deterministic order, no atomics or fences).  A
// file-scope device array, so launches stay allocation-free and
// graph-capture safe.  Split-K launches issued concurrently on different
// streams of one device would share it; the engine issues its GEMMs on one
// stream.
constexpr size_t kWsFloats = size_t(8) << 20;  // 32 MiB
__device__ float g_splitk_ws[kWsFloats];

template <int BM, int BN, int MODE>
__device__ __forceinline__ void epilogue(const GemmParams& p, const f32x16 (&acc)[BM / 64][BN / 64], int m0, int n0,
                                         int wm, int wn, int lane) {
    constexpr int WM = BM / 2, WN = BN / 2, MI = WM / 32, NI = WN / 32;
    const int fr = lane & 31;
    // D[i][j] of a 32x32 MFMA tile: j = lane%32, i = 8*(v/4) + 4*(lane/32) + v%4
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

// Block tile BM x BN, 4 waves in a 2x2 grid, wave tile (BM/2) x (BN/2) of
// 32x32 MFMA tiles.  K advances BK = 64 per step.  grid (N tiles, M tiles,
// K slices); with more than one slice the fp32 partials go to the scratch.
//
// Operand layout.  v_mfma_f32_32x32x16_f16 takes, per lane l, 8 consecutive
// k of A row (l % 32) and of B column (l % 32), the lane half h = l / 32
// holding the second 8.  The k order inside the instruction is free as long
// as A and B agree, so within a 64-wide step lane half h takes k in
// [32h, 32h + 32) and sub-step s the 8 values at 8s: for B that is word s of
// one 16-byte load of packed int4 - the lane's B operand comes straight from
// global memory and is dequantized in registers (no LDS for B).  A is staged
// through LDS (rows padded to 72 halves: conflict-free 16-byte reads).
template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_w4a16_mfma_kernel(GemmParams p) {
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_U4 = BM * BK / 8 / 256;  // 16-byte A chunks per thread per step (4 or 2)
    // A rows are loaded 8 threads per 128-byte row, 32 rows per pass
    constexpr int D = (BM == 128 && BN == 128) ? 3 : 4;  // stages of the register ring
    static_assert(A_U4 * 32 == BM, "A tile passes");

    __shared__ __align__(16) _Float16 sA[2][BM * A_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = p.K;
    const int G = K >> 7;
    const int KT_all = K / BK;
    const int slices = gridDim.z;
    const int kt_begin = static_cast<int>((static_cast<long long>(blockIdx.z) * KT_all) / slices);
    const int kt_end = static_cast<int>((static_cast<long long>(blockIdx.z + 1) * KT_all) / slices);
    const int KT = kt_end - kt_begin;
    const int fr = lane & 31;
    const int h = lane >> 5;

    // A: rows past M read row M-1 (valid) and are never stored
    const int a_row = tid >> 3;
    const int a_col = (tid & 7) * 8;  // halves
    const uint16_t* a_src[A_U4];
#pragma unroll
    for (int i = 0; i < A_U4; ++i)
        a_src[i] = p.A + static_cast<size_t>(min(m0 + a_row + 32 * i, p.M - 1)) * K + a_col;
    // B: lane's column for fragment j; columns past N read column N-1
    const u32x4* b_src[NI];
    const uint16_t* b_sc[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int col = min(n0 + wn * WN + j * 32 + fr, p.N - 1);
        int m = 0, local = col;
        if constexpr (MODE == kQKV) {
            m = (col >= p.col_begin[1]) + (col >= p.col_begin[2]);
            local = col - p.col_begin[m];
        }
        b_src[j] = reinterpret_cast<const u32x4*>(p.qw[m] + static_cast<size_t>(local) * (K >> 3)) + h;
        b_sc[j] = p.sc[m] + static_cast<size_t>(local) * G;
    }

    struct Stage {
        u32x4 a[A_U4];
        u32x4 b[NI];
        uint16_t s[NI];
    };
    Stage st[D];
    auto load_global = [&](int kt, Stage& S) __attribute__((always_inline)) {
        const int k0 = (kt_begin + kt) * BK;
#pragma unroll
        for (int i = 0; i < A_U4; ++i) S.a[i] = *reinterpret_cast<const u32x4*>(a_src[i] + k0);
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            S.b[j] = __builtin_nontemporal_load(b_src[j] + (k0 >> 5));  // 16 B = 32 k of lane half h
            S.s[j] = b_sc[j][k0 >> 7];
        }
    };
    auto store_a = [&](int buf, const Stage& S) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_U4; ++i)
            *reinterpret_cast<u32x4*>(&sA[buf][(a_row + 32 * i) * A_STRIDE + a_col]) = S.a[i];
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

#pragma unroll
    for (int d = 0; d < D; ++d) load_global(min(d, KT - 1), st[d]);
    store_a(0, st[0]);
    __syncthreads();

    auto step = [&](int kt, int d) __attribute__((always_inline)) {
        const int buf = kt & 1;
        const Stage& S = st[d];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            f16x8 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(&sA[buf][(wm * WM + i * 32 + fr) * A_STRIDE + h * 32 + s * 8]);
#pragma unroll
            for (int j = 0; j < NI; ++j)
                bf[j] = __builtin_bit_cast(f16x8, qwen::unpack_w4_to_half8(S.b[j][s], __builtin_bit_cast(_Float16, S.s[j])));
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        load_global(min(kt + D, KT - 1), st[d]);  // step kt is consumed: refill with step kt + D
        store_a(buf ^ 1, st[(d + 1) % D]);          // A of step kt + 1, loaded D - 1 steps ago
        __syncthreads();
    };
    int kt = 0;
    for (; kt + D <= KT; kt += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(kt + d, d);
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
        if (kt + d < KT) step(kt + d, d);  // tail: fewer than D steps

    if (slices == 1) {
        epilogue<BM, BN, MODE>(p, acc, m0, n0, wm, wn, lane);
        return;
    }
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    float* mine = g_splitk_ws + (static_cast<size_t>(blockIdx.z) * n_tiles + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[((i * NI + j) * 16 + v) * 256 + tid] = acc[i][j][v];
}

// Sums the K-slice partials of each tile in slice order and applies the
// epilogue.  grid (N tiles, M tiles), 256 threads (the MFMA lane layout).
template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmParams p, int slices) {
    constexpr int MI = BM / 64, NI = BN / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};
    for (int z = 0; z < slices; ++z) {
        const float* part = g_splitk_ws + (static_cast<size_t>(z) * n_tiles + tile) * (BM * BN);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] += part[((i * NI + j) * 16 + v) * 256 + tid];
    }
    epilogue<BM, BN, MODE>(p, acc, blockIdx.y * BM, blockIdx.x * BN, wave >> 1, wave & 1, lane);
}

template <int BM, int BN, int MODE>
void launch_tiles(const GemmParams& p, int slices, hipStream_t s) {
    const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, slices);
    gemm_w4a16_mfma_kernel<BM, BN, MODE><<<grid, 256, 0, s>>>(p);
    if (slices > 1) gemm_splitk_reduce_kernel<BM, BN, MODE><<<dim3(grid.x, grid.y), 256, 0, s>>>(p, slices);
}

template <int MODE>
int launch_gemm(const GemmParams& p, hipStream_t stream, const char* what) {
    if (p.M <= 0 || p.N <= 0) return QE_OK;
    const int cus = cu_count();
    auto tiles = [&](int bm, int bn) { return ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn); };
    // largest tile that still gives >= 1 block per CU; else 64x64 tiles and K slices
    int bm = 64, bn = 64;
    if (tiles(128, 128) >= cus) { bm = 128; bn = 128; }
    else if (tiles(64, 128) >= cus) { bm = 64; bn = 128; }
    else if (tiles(128, 64) >= cus) { bm = 128; bn = 64; }
    const int nt = tiles(bm, bn);
    const int KT = p.K / BK;
    int slices = 1;
    if (nt < cus && gemm_split_k_enabled()) {
        slices = (2 * cus + nt - 1) / nt;   // about two blocks per CU
        slices = std::min(slices, KT / 8);  // >= 8 steps of 64 per slice
        slices = std::min(slices, 32);
        slices = std::max(slices, 1);
        while (slices > 1 && static_cast<size_t>(slices) * nt * bm * bn > kWsFloats) --slices;
    }
    if ((p.M + bm - 1) / bm > 65535) return fail(QE_ERR_UNSUPPORTED, "%s: M=%d too large", what, p.M);
    if (bm == 128 && bn == 128) launch_tiles<128, 128, MODE>(p, slices, stream);
    else if (bm == 64 && bn == 128) launch_tiles<64, 128, MODE>(p, slices, stream);
    else if (bm == 128 && bn == 64) launch_tiles<128, 64, MODE>(p, slices, stream);
    else launch_tiles<64, 64, MODE>(p, slices, stream);
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
