// Prefill W4A16 dequant-GEMM on CDNA4 matrix cores (gfx950).
//
// Math of src/kernels/gemm_prefill.cu: Y[M,N] = A[M,K] . Wdq[N,K]^T with
// Wdq = fp16((q-8)*s) (unpack_w4_to_half2_quad, quant_primitives.cuh:92-115),
// fp32 accumulation, fp16 output; residual added after rounding as an fp16
// add (the vector epilogue, gemm_prefill.cu:261-275); QKV split over three
// outputs (:392-489); gate/up SwiGLU over interleaved columns (:559-609).
//
// MI355X design:
//   * 256-thread blocks (4 wave64s), block tiles 64x64 and 128x64 with the
//     waves in a 2x2 grid, 64x128 and 128x128 with the waves side by side
//     (1x4: each wave owns all BM rows and 32 columns, so no two waves
//     dequantize the same weights); 32x32 tiles of
//     v_mfma_f32_32x32x16_f16 with fp32 accumulators.
//   * The B operand of a lane (8 consecutive k of one weight column) is one
//     packed int4 word: each lane loads its 16-byte run of 32 k straight from
//     global memory and dequantizes it in registers ((q-8) via the 0x6400
//     bias, one fp16 RNE multiply by the group scale) - no LDS round trip and
//     no barrier for the weights.  A (fp16 activations) is staged through a
//     double-buffered LDS tile.  K advances 64 per step; A loads run in a
//     4-stage register ring, weights a whole 256-k quad ahead.
//   * Tile shape and K slices are chosen per launch from a fitted time model
//     (blocks per CU, steps per block, split-K overhead); split-K partials
//     are reduced by a second kernel in slice order.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "qe_common.hpp"


namespace qe {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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
    const int8_t* A8;         // W4A8 variant: Q8_1 rows of the activation
    const float* A8_scale;
    const int32_t* A8_sum8;
    float* ws;         // split-K partials (slices > 1 only)
    int M, N, K;       // N = virtual columns (SwiGLU: 2*I)
};

// silu(g) * u = g * u / (1 + e^-g) with the hardware exp2 and reciprocal
// (about 1 ulp each in fp32; the result is rounded to fp16)
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * u * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.44269504088896341f * g));
}

// Split-K partials: fp32 tiles of the K slices, reduced by a second kernel
// on the same stream (deterministic order, no atomics or fences).  They live
// in a workspace of kWsFloats floats that belongs to the launching stream
// (gemm_workspace below), so GEMMs in flight on different streams never
// share partials.
constexpr size_t kWsFloats = size_t(8) << 20;  // 32 MiB

struct Workspace {
    float* ptr = nullptr;
    size_t floats = 0;
};

// One 32x32 accumulator fragment whose rows start at r0 and whose lane
// column is col.  D[i][j] of a 32x32 MFMA tile: j = lane%32,
// i = 8*(v/4) + 4*(lane/32) + v%4
// Value of the neighbouring lane (lane ^ 1), by DPP within the quad.
__device__ __forceinline__ float swap_adjacent(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
}

template <int MODE>
__device__ __forceinline__ void epilogue_frag(const GemmParams& p, const f32x16& acc, int r0, int col, int lane) {
    const int fr = lane & 31;
    // rows of element v: r0 + 8 * (v / 4) + 4 * (lane / 32) + v % 4 (static
    // offsets from the lane's first row; every index into acc is static)
    const int lrow = r0 + 4 * (lane >> 5);
    const bool cols_ok = col < p.N;
    const bool rows_ok = r0 + 32 <= p.M;  // the whole fragment: no per-row checks
    if constexpr (MODE == kSwiglu) {
        // lane pair (gate column, up column): the gate lane finishes rows
        // v < 8 and the up lane rows v >= 8 (16 further down), so every lane
        // evaluates 8 silu; the partner's values arrive by DPP swaps
        const bool gate = (fr & 1) == 0;
        const int row0 = lrow + (gate ? 0 : 16);
        const int stride = p.out_stride[0];
        uint16_t* out = p.out[0] + (col >> 1);
#pragma unroll
        for (int v = 0; v < 8; ++v) {
            const float lo = acc[v], hi = acc[v + 8];
            const float lo_x = swap_adjacent(lo), hi_x = swap_adjacent(hi);
            const float g = gate ? lo : hi_x;
            const float u = gate ? lo_x : hi;
            const int row = row0 + 8 * (v >> 2) + (v & 3);
            if (cols_ok && (rows_ok || row < p.M)) out[static_cast<size_t>(row) * stride] = f2h(silu_mul(g, u));
        }
        return;
    }
    int m = 0, local = col;
    if constexpr (MODE == kQKV) {
        m = (col >= p.col_begin[1]) + (col >= p.col_begin[2]);
        local = col - p.col_begin[m];
    }
    const int stride = MODE == kQKV ? (m == 0 ? p.out_stride[0] : m == 1 ? p.out_stride[1] : p.out_stride[2])
                                    : p.out_stride[0];
    uint16_t* out = (MODE == kQKV ? (m == 0 ? p.out[0] : m == 1 ? p.out[1] : p.out[2]) : p.out[0]) + local;
    const uint16_t* res = (MODE == kPlain && p.residual != nullptr) ? p.residual + local : nullptr;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int row = lrow + 8 * (v >> 2) + (v & 3);
        if (cols_ok && (rows_ok || row < p.M)) {
            const size_t off = static_cast<size_t>(row) * stride;
            _Float16 h = static_cast<_Float16>(acc[v]);
            if (MODE == kPlain && res != nullptr) h = h + __builtin_bit_cast(_Float16, res[off]);  // fp16 add, RNE
            out[off] = __builtin_bit_cast(uint16_t, h);
        }
    }
}

template <int BM, int BN, int WGM, int MODE>
__device__ __forceinline__ void epilogue(const GemmParams& p, const f32x16 (&acc)[BM / WGM / 32][BN / (4 / WGM) / 32],
                                         int m0, int n0, int wm, int wn, int lane) {
    constexpr int WM = BM / WGM, WN = BN / (4 / WGM), MI = WM / 32, NI = WN / 32;
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
            epilogue_frag<MODE>(p, acc[i][j], m0 + wm * WM + i * 32, n0 + wn * WN + j * 32 + (lane & 31), lane);
}

// Nibble order of a word of the tiled copy: k0 at bits 0-3, k1 at 16-19, k2 at
// 4-7, k3 at 20-23, k4 at 8-11, k5 at 24-27, k6 at 12-15, k7 at 28-31.  A
// nibble in bits 0-3 of a 16-bit half under the exponent of 1024.0 (0x6400)
// reads as 1024 + q; in bits 4-7 under the exponent of 64.0 (0x5400) as
// 64 + q.  So the 8 values in K order cost five bit operations (two masked
// ORs, a shift, two masked ORs), then the exact subtraction of 1032 or 72 and
// the one fp16 RNE multiply by the scale of unpack_w4_to_half8 - the same
// values as unpack_w4_to_half8 on the original word.
// The four masks live in VGPRs (TiledMasks, set up once per kernel): gfx9
// VOP3 instructions take no literal constants, so with literal masks the
// compiler emits separate AND and OR instructions instead of V_AND_OR_B32.
struct TiledMasks {
    uint32_t lo, hi, bias_lo, bias_hi;
};
__device__ __forceinline__ TiledMasks tiled_masks() {
    TiledMasks m{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
    asm volatile("" : "+v"(m.lo), "+v"(m.hi), "+v"(m.bias_lo), "+v"(m.bias_hi));
    return m;
}
__device__ __forceinline__ qwen::qe_half8_t unpack_w4t_to_half8(uint32_t w, _Float16 scale, const TiledMasks& m) {
    const uint32_t w8 = w >> 8;
    const uint32_t u01 = (w & m.lo) | m.bias_lo;
    const uint32_t u23 = (w & m.hi) | m.bias_hi;
    const uint32_t u45 = (w8 & m.lo) | m.bias_lo;
    const uint32_t u67 = (w8 & m.hi) | m.bias_hi;
    const qwen::qe_half2_t b1 = {(_Float16)1032.0f, (_Float16)1032.0f};
    const qwen::qe_half2_t b2 = {(_Float16)72.0f, (_Float16)72.0f};
    const qwen::qe_half2_t sc = {scale, scale};
    const qwen::qe_half2_t h01 = (__builtin_bit_cast(qwen::qe_half2_t, u01) - b1) * sc;
    const qwen::qe_half2_t h23 = (__builtin_bit_cast(qwen::qe_half2_t, u23) - b2) * sc;
    const qwen::qe_half2_t h45 = (__builtin_bit_cast(qwen::qe_half2_t, u45) - b1) * sc;
    const qwen::qe_half2_t h67 = (__builtin_bit_cast(qwen::qe_half2_t, u67) - b2) * sc;
    return qwen::qe_half8_t{h01[0], h01[1], h23[0], h23[1], h45[0], h45[1], h67[0], h67[1]};
}

// The same 8 values of an original word, in the tiled word's nibble order.
__device__ __forceinline__ uint32_t w4_word_to_tiled(uint32_t w) {
    uint32_t q[8];
    q[0] = w & 15u;          q[4] = (w >> 4) & 15u;
    q[1] = (w >> 8) & 15u;   q[5] = (w >> 12) & 15u;
    q[2] = (w >> 16) & 15u;  q[6] = (w >> 20) & 15u;
    q[3] = (w >> 24) & 15u;  q[7] = (w >> 28) & 15u;
    return q[0] | (q[2] << 4) | (q[4] << 8) | (q[6] << 12) | (q[1] << 16) | (q[3] << 20) | (q[5] << 24) |
           (q[7] << 28);
}

// Block tile BM x BN, 4 waves in a WGM x (4/WGM) grid, wave tile WM x WN of
// 32x32 MFMA tiles.  K advances 64 per step.  grid (N tiles, M tiles, K
// slices); with more than one slice the fp32 partials go to the scratch.
//
// Operand layout.  v_mfma_f32_32x32x16_f16 takes, per lane l, 8 consecutive
// k of A row (l % 32) and of B column (l % 32), the lane half h = l / 32
// holding the second 8.  The k order inside the instruction is free as long
// as A and B agree, and that freedom is used to feed B straight from global
// memory: one packed int4 word is exactly the 8 k of one lane's operand, so
// each lane dequantizes its own words in registers and the weights never go
// through LDS.  A (fp16 activations) is staged through a double-buffered
// LDS tile (rows padded to 72 halves: conflict-free 16-byte reads).
//
// QUAD (K % 256 == 0): weights are read 256 k at a time, one 128-byte line
// per column - lane half h loads the 64 bytes of k in [128h, 128h + 128) as
// four 16-byte loads, with its single group scale - and the four 64-k steps
// of the quad take k = 128h + 32t + 8s in step t, sub-step s.  A step then
// spans two 32-k pieces of A, 128 k apart.  Without QUAD each step loads
// 16 bytes per lane (k = 32h + 8s) and one scale.
template <int BM, int BN, int WGM, int MODE, bool QUAD, bool TILED = false>
__global__ __launch_bounds__(256, 2) void gemm_w4a16_mfma_kernel(GemmParams p) {
    static_assert(QUAD || !TILED, "the tiled weight layout is read quad by quad");
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_U4 = BM / 32;  // 16-byte A chunks per thread per step: 8 threads per row, 32 rows per pass
    constexpr int D = (QUAD || BM == 64) ? 4 : 3;  // stages of the A register ring
    static_assert(MI >= 1 && NI >= 1, "wave tile");

    __shared__ __align__(16) _Float16 sA[2][BM * A_STRIDE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = p.K;
    const int G = K >> 7;
    const int slices = gridDim.z;
    constexpr int UNIT = QUAD ? 4 : 1;  // steps per slicing unit
    const int U_all = K / (BK * UNIT);
    const int kt_begin = UNIT * static_cast<int>((static_cast<long long>(blockIdx.z) * U_all) / slices);
    const int kt_end = UNIT * static_cast<int>((static_cast<long long>(blockIdx.z + 1) * U_all) / slices);
    const int KT = kt_end - kt_begin;
    const int fr = lane & 31;
    const int h = lane >> 5;
    const TiledMasks tmask = tiled_masks();

    // A: rows past M read row M-1 (valid) and are never stored
    const int a_row = tid >> 3;
    const int c = tid & 7;
    const int a_col = c * 8;  // halves within the LDS row
    const int a_k = QUAD ? 128 * (c >> 2) + 8 * (c & 3) : 8 * c;
    const uint16_t* a_src[A_U4];
#pragma unroll
    for (int i = 0; i < A_U4; ++i)
        a_src[i] = p.A + static_cast<size_t>(min(m0 + a_row + 32 * i, p.M - 1)) * K + a_k;
    auto a_koff = [&](int kt) __attribute__((always_inline)) {
        const int g = kt_begin + kt;
        return QUAD ? 256 * (g >> 2) + 32 * (g & 3) : 64 * g;
    };
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
        if constexpr (TILED) {
            const size_t tq = static_cast<size_t>(local >> 5) * (K >> 8);  // first quad of the column tile
            b_src[j] = reinterpret_cast<const u32x4*>(p.qw[m]) + tq * 256 + 32 * h + (local & 31);
            b_sc[j] = p.sc[m] + tq * 64 + 32 * h + (local & 31);
        } else {
            b_src[j] = reinterpret_cast<const u32x4*>(p.qw[m] + static_cast<size_t>(local) * (K >> 3)) + (QUAD ? 4 : 1) * h;
            b_sc[j] = p.sc[m] + static_cast<size_t>(local) * G + (QUAD ? h : 0);
        }
    }

    u32x4 ra[D][A_U4];
    u32x4 rb[QUAD ? 2 : D][NI][QUAD ? 4 : 1];
    uint16_t rs[QUAD ? 2 : D][NI];
    auto load_a = [&](int kt, int d) __attribute__((always_inline)) {
        const int k0 = a_koff(kt);
#pragma unroll
        for (int i = 0; i < A_U4; ++i) ra[d][i] = *reinterpret_cast<const u32x4*>(a_src[i] + k0);
    };
    // QUAD: quad qd (relative to the slice) into buffer e; else step qd into ring slot e
    auto load_b = [&](int qd, int e) __attribute__((always_inline)) {
        const int g = (kt_begin / UNIT) + qd;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
#pragma unroll
            for (int i = 0; i < (QUAD ? 4 : 1); ++i)  // cached: every M tile of the column reads it
                rb[e][j][i] = TILED ? b_src[j][256 * g + 64 * i] : b_src[j][QUAD ? 8 * g + i : 2 * g];
            rs[e][j] = TILED ? b_sc[j][64 * g] : b_sc[j][QUAD ? 2 * g : (g >> 1)];
        }
    };
    auto store_a = [&](int buf, int d) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_U4; ++i)
            *reinterpret_cast<u32x4*>(&sA[buf][(a_row + 32 * i) * A_STRIDE + a_col]) = ra[d][i];
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

    // prologue loads in the order of the steady state (QUAD: the quad's
    // weights, then the A ring; else A and weights step by step): the wait at
    // the loop head is sized for both the entry and the back edge, so an
    // entry that issued the weights last would make every iteration drain
    // its loads there
    if constexpr (QUAD) {
        load_b(0, 0);
#pragma unroll
        for (int d = 0; d < D; ++d) load_a(min(d, KT - 1), d);
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load_a(min(d, KT - 1), d);
            load_b(min(d, KT - 1), d);
        }
    }
    store_a(0, 0);
    __syncthreads();

    // step kt: A ring slot d = kt % D; QUAD: weight buffer e = (kt / 4) % 2,
    // t = kt % 4; else weight ring slot e = d
    auto step = [&](int kt, int d, int e, int t) __attribute__((always_inline)) {
        const int buf = kt & 1;
        if (QUAD && t == 0) load_b(min(kt / 4 + 1, KT / 4 - 1), e ^ 1);  // next quad
        auto read_a = [&](int s, f16x8 (&af)[MI]) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(&sA[buf][(wm * WM + i * 32 + fr) * A_STRIDE + h * 32 + s * 8]);
        };
        auto dequant = [&](int s, f16x8 (&bf)[NI]) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const uint32_t w = QUAD ? rb[e][j][t][s] : rb[e][j][0][s];
                const _Float16 sc = __builtin_bit_cast(_Float16, rs[e][j]);
                bf[j] = __builtin_bit_cast(f16x8, TILED ? unpack_w4t_to_half8(w, sc, tmask) : qwen::unpack_w4_to_half8(w, sc));
            }
        };
        // software pipeline over the four sub-steps: the A fragments and the
        // dequantized weights of sub-step s + 1 go to a second register set
        // while the MFMAs of sub-step s run, so a wave does not stall on its
        // own LDS latency or dequantization
        f16x8 af[2][MI], bf[2][NI];
        read_a(0, af[0]);
        dequant(0, bf[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int c = s & 1;
            if (s < 3) {
                read_a(s + 1, af[c ^ 1]);
                dequant(s + 1, bf[c ^ 1]);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[c][i], bf[c][j], acc[i][j], 0, 0, 0);
        }
        load_a(min(kt + D, KT - 1), d);      // step kt is consumed: refill with step kt + D
        if (!QUAD) load_b(min(kt + D, KT - 1), d);
        store_a(buf ^ 1, (d + 1) % D);        // A of step kt + 1, loaded D - 1 steps ago
        // scheduling hint: each MFMA followed by one LDS read and five VALU
        // ops (the next sub-step's operands), so the matrix core is fed while
        // they issue
#pragma unroll
        for (int i = 0; i < MI * NI * 4; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        __syncthreads();
    };
    int kt = 0;
    if constexpr (QUAD) {
        // KT is a multiple of 4; 8 steps per iteration keep every index static
        for (; kt + 8 <= KT; kt += 8) {
#pragma unroll
            for (int u = 0; u < 8; ++u) step(kt + u, u % D, u / 4, u % 4);
        }
        if (kt < KT) {
#pragma unroll
            for (int u = 0; u < 4; ++u) step(kt + u, u % D, 0, u);
        }
    } else {
        for (; kt + D <= KT; kt += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) step(kt + d, d, d, 0);
        }
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (kt + d < KT) step(kt + d, d, d, 0);  // tail: fewer than D steps
    }

    if (slices == 1) {
        epilogue<BM, BN, WGM, MODE>(p, acc, m0, n0, wm, wn, lane);
        return;
    }
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    float* mine = p.ws + (static_cast<size_t>(blockIdx.z) * n_tiles + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) mine[((i * NI + j) * 16 + v) * 256 + tid] = acc[i][j][v];
}

// K % 256 == 0, 512 threads: two groups of four waves split the k steps of
// the tile between them (group g takes the steps 2 i + g, i.e. steps g and
// g + 2 of every 256-k quad), each with its own A staging, and add their
// accumulators through LDS at the end.  For grids of at most one block per
// CU (M = 128 prefill) this gives every SIMD two waves without split-K
// partials in memory.  Per group the step is the register-staged kernel's:
// A through a 4-stage register ring and a double-buffered LDS tile, weights
// a quad ahead (the group's two 16-byte pieces of each column and quad),
// the four sub-steps software-pipelined.
template <int BM, int BN, int WGM, int MODE, bool TILED = false>
__global__ __launch_bounds__(512, 1) void gemm_w4a16_ks2_kernel(GemmParams p) {
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_U4 = BM / 32;
    constexpr int D = 4;
    constexpr int TILE_H = BM * A_STRIDE;
    static_assert(MI >= 1 && NI >= 1, "wave tile");
    __shared__ __align__(16) _Float16 sA[2][2][TILE_H];  // [group][buffer]
    static_assert(sizeof(sA) >= sizeof(float) * MI * NI * 16 * 256, "the group exchange reuses the A tiles");

    const int tid = threadIdx.x;
    const int kg = tid >> 8;      // k group
    const int gtid = tid & 255;   // thread within the group
    const int lane = tid & 63;
    const int wave = gtid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = p.K;
    const int G = K >> 7;
    const int slices = gridDim.z;
    const int U_all = K / (BK * 4);
    const int kt_begin = 4 * static_cast<int>((static_cast<long long>(blockIdx.z) * U_all) / slices);
    const int kt_end = 4 * static_cast<int>((static_cast<long long>(blockIdx.z + 1) * U_all) / slices);
    const int KTL = (kt_end - kt_begin) / 2;  // steps per group
    const int fr = lane & 31;
    const int h = lane >> 5;
    const TiledMasks tmask = tiled_masks();

    const int a_row = gtid >> 3;
    const int c = gtid & 7;
    const int a_col = c * 8;
    const int a_k = 128 * (c >> 2) + 8 * (c & 3);
    const uint16_t* a_src[A_U4];
#pragma unroll
    for (int i = 0; i < A_U4; ++i)
        a_src[i] = p.A + static_cast<size_t>(min(m0 + a_row + 32 * i, p.M - 1)) * K + a_k;
    // local step i of group kg is global step 2 i + kg of the slice
    auto a_koff = [&](int i) __attribute__((always_inline)) {
        const int g = kt_begin + 2 * i + kg;
        return 256 * (g >> 2) + 32 * (g & 3);
    };
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
        if constexpr (TILED) {
            const size_t tq = static_cast<size_t>(local >> 5) * (K >> 8);
            b_src[j] = reinterpret_cast<const u32x4*>(p.qw[m]) + tq * 256 + 64 * kg + 32 * h + (local & 31);
            b_sc[j] = p.sc[m] + tq * 64 + 32 * h + (local & 31);
        } else {
            b_src[j] = reinterpret_cast<const u32x4*>(p.qw[m] + static_cast<size_t>(local) * (K >> 3)) + 4 * h + kg;
            b_sc[j] = p.sc[m] + static_cast<size_t>(local) * G + h;
        }
    }

    u32x4 ra[D][A_U4];
    u32x4 rb[2][NI][2];  // [quad buffer][column][the group's two steps of the quad]
    uint16_t rs[2][NI];
    auto load_a = [&](int i, int d) __attribute__((always_inline)) {
        const int k0 = a_koff(i);
#pragma unroll
        for (int u = 0; u < A_U4; ++u) ra[d][u] = *reinterpret_cast<const u32x4*>(a_src[u] + k0);
    };
    auto load_b = [&](int qd, int e) __attribute__((always_inline)) {
        const int g = (kt_begin >> 2) + qd;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            rb[e][j][0] = TILED ? b_src[j][256 * g] : b_src[j][8 * g];
            rb[e][j][1] = TILED ? b_src[j][256 * g + 128] : b_src[j][8 * g + 2];
            rs[e][j] = TILED ? b_sc[j][64 * g] : b_sc[j][2 * g];
        }
    };
    auto store_a = [&](int buf, int d) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < A_U4; ++u)
            *reinterpret_cast<u32x4*>(&sA[kg][buf][(a_row + 32 * u) * A_STRIDE + a_col]) = ra[d][u];
    };
    auto read_a = [&](int buf, int s, f16x8 (&af)[MI]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
            af[i] = *reinterpret_cast<const f16x8*>(&sA[kg][buf][(wm * WM + i * 32 + fr) * A_STRIDE + h * 32 + s * 8]);
    };
    auto dequant = [&](int e, int tt, int s, f16x8 (&bf)[NI]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NI; ++j)
            bf[j] = __builtin_bit_cast(f16x8, TILED ? unpack_w4t_to_half8(rb[e][j][tt][s],
                                                                          __builtin_bit_cast(_Float16, rs[e][j]), tmask)
                                                    : qwen::unpack_w4_to_half8(rb[e][j][tt][s],
                                                                               __builtin_bit_cast(_Float16, rs[e][j])));
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f32x16{};

    load_b(0, 0);
#pragma unroll
    for (int d = 0; d < D; ++d) load_a(min(d, KTL - 1), d);
    store_a(0, 0);
    __syncthreads();

    // local step i: ring slot d = i % D, LDS buffer i % 2, quad i / 2 in
    // buffer e = (i / 2) % 2, the group's piece tt = i % 2 of it
    auto step = [&](int i, int d, int e, int tt) __attribute__((always_inline)) {
        const int buf = i & 1;
        if (tt == 0) load_b(min(i / 2 + 1, KTL / 2 - 1), e ^ 1);  // next quad
        f16x8 af[2][MI], bf[2][NI];
        read_a(buf, 0, af[0]);
        dequant(e, tt, 0, bf[0]);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int cs = s & 1;
            if (s < 3) {
                read_a(buf, s + 1, af[cs ^ 1]);
                dequant(e, tt, s + 1, bf[cs ^ 1]);
            }
#pragma unroll
            for (int a = 0; a < MI; ++a)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[a][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cs][a], bf[cs][j], acc[a][j], 0, 0, 0);
        }
        load_a(min(i + D, KTL - 1), d);
        store_a(buf ^ 1, (d + 1) % D);
#pragma unroll
        for (int x = 0; x < MI * NI * 4; ++x) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
        __syncthreads();
    };
    int i = 0;
    for (; i + 4 <= KTL; i += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) step(i + u, u % D, (u / 2) & 1, u & 1);
    }
    if (i < KTL) {  // KTL is even: two steps (one quad) left
#pragma unroll
        for (int u = 0; u < 2; ++u) step(i + u, u % D, 0, u);
    }

    // the groups add their accumulators: group 0 keeps fragments a < MI / 2
    // (all when MI == 1: then group 1 hands over everything), group 1 the rest;
    // each writes the fragments the other keeps into the (now idle) A tiles
    constexpr int KEEP0 = MI == 1 ? 1 : MI / 2;
    float* xch = reinterpret_cast<float*>(&sA[0][0][0]);
    auto slot = [&](int a, int j, int v) __attribute__((always_inline)) {
        return ((a * NI + j) * 16 + v) * 256 + gtid;
    };
#pragma unroll
    for (int a = 0; a < MI; ++a) {
        const bool mine = kg == 0 ? a < KEEP0 : a >= KEEP0;
        if (!mine)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) xch[slot(a, j, v)] = acc[a][j][v];
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < MI; ++a) {
        const bool mine = kg == 0 ? a < KEEP0 : a >= KEEP0;
        if (mine)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[a][j][v] += xch[slot(a, j, v)];
    }
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    float* part = p.ws + (static_cast<size_t>(blockIdx.z) * n_tiles + tile) * (BM * BN);
#pragma unroll
    for (int a = 0; a < MI; ++a) {
        const bool mine = kg == 0 ? a < KEEP0 : a >= KEEP0;
        if (!mine) continue;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            if (slices == 1) {
                epilogue_frag<MODE>(p, acc[a][j], m0 + wm * WM + a * 32, n0 + wn * WN + j * 32 + fr, lane);
            } else {
#pragma unroll
                for (int v = 0; v < 16; ++v) part[((a * NI + j) * 16 + v) * 256 + gtid] = acc[a][j][v];
            }
        }
    }
}

// Sums the K-slice partials in slice order and applies the epilogue.  grid
// (N tiles, M tiles, fragments): block z takes the 32x32 fragment z of its
// tile, 256 threads in the MFMA lane layout of the 4 waves.  S > 0: all S
// slices are requested before the first add (one memory latency, not S);
// S = 0: a loop over the slices.
template <int BM, int BN, int WGM, int MODE, int S>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(GemmParams p, int slices) {
    constexpr int WGN = 4 / WGM;
    constexpr int WM = BM / WGM, WN = BN / WGN, NI = WN / 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    const int f = blockIdx.z, i = f / NI, j = f % NI;
    const size_t slice_stride = static_cast<size_t>(n_tiles) * (BM * BN);
    const float* part = p.ws + static_cast<size_t>(tile) * (BM * BN) + f * 16 * 256 + tid;
    f32x16 acc = f32x16{};
    if constexpr (S > 0) {
        float x[S][16];
#pragma unroll
        for (int z = 0; z < S; ++z)
#pragma unroll
            for (int v = 0; v < 16; ++v) x[z][v] = part[z * slice_stride + v * 256];
#pragma unroll
        for (int z = 0; z < S; ++z)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] += x[z][v];
    } else {
        for (int z = 0; z < slices; ++z)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[v] += part[z * slice_stride + v * 256];
    }
    const int wm = wave / WGN, wn = wave % WGN;
    epilogue_frag<MODE>(p, acc, blockIdx.y * BM + wm * WM + i * 32, blockIdx.x * BN + wn * WN + j * 32 + (lane & 31),
                        lane);
}

template <int BM, int BN, int WGM, int MODE>
void launch_reduce(const GemmParams& p, dim3 tiles, int slices, hipStream_t s) {
    constexpr int FR = (BM / WGM / 32) * (BN / (4 / WGM) / 32);  // fragments per wave
    const dim3 grid(tiles.x, tiles.y, FR);
    switch (slices) {
        case 2: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 2><<<grid, 256, 0, s>>>(p, slices); break;
        case 3: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 3><<<grid, 256, 0, s>>>(p, slices); break;
        case 4: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 4><<<grid, 256, 0, s>>>(p, slices); break;
        case 6: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 6><<<grid, 256, 0, s>>>(p, slices); break;
        case 8: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 8><<<grid, 256, 0, s>>>(p, slices); break;
        default: gemm_splitk_reduce_kernel<BM, BN, WGM, MODE, 0><<<grid, 256, 0, s>>>(p, slices); break;
    }
}

template <int BM, int BN, int WGM, int MODE, bool TILED = false>
void launch_tiles(const GemmParams& p, int slices, hipStream_t s) {
    const dim3 grid((p.N + BN - 1) / BN, (p.M + BM - 1) / BM, slices);
    // two k groups per block when the grid leaves every CU with at most one
    // block (its SIMDs would otherwise run one wave each)
    const int ks2 = gemm_ks2_mode();
    const bool two = p.K % 256 == 0 && ks2 != 1 &&
                     (ks2 == 2 || static_cast<long long>(grid.x) * grid.y * grid.z <= cu_count());
    if (two) {
        gemm_w4a16_ks2_kernel<BM, BN, WGM, MODE, TILED><<<grid, 512, 0, s>>>(p);
        if (slices > 1) launch_reduce<BM, BN, WGM, MODE>(p, grid, slices, s);
        return;
    }
    if (TILED || p.K % 256 == 0)
        gemm_w4a16_mfma_kernel<BM, BN, WGM, MODE, true, TILED><<<grid, 256, 0, s>>>(p);
    else if constexpr (!TILED)
        gemm_w4a16_mfma_kernel<BM, BN, WGM, MODE, false><<<grid, 256, 0, s>>>(p);
    if (slices > 1) launch_reduce<BM, BN, WGM, MODE>(p, grid, slices, s);
}

// Launch-time model of one configuration (tile, K slices), in microseconds,
// fitted to MI355X measurements of this kernel over M in {128..2048} and the
// Qwen2.5-1.5B projection shapes.  Blocks run at most two per CU; a CU with
// two co-resident blocks advances each more slowly than a CU with one.
struct TileCost {
    int bm, bn, wgm;
    float step1, step2;    // us per 64-k step: one block on the CU / two
    float split, split_mb; // split-K: fixed cost, cost per MB of fp32 partials
    float fixed;
};
constexpr TileCost kTiles[4] = {
    {64, 64, 2, 0.277f, 0.543f, 3.85f, 0.014f, 4.80f},
    {64, 128, 1, 0.321f, 0.683f, 5.37f, 0.012f, 5.24f},
    {128, 64, 2, 0.410f, 0.845f, 5.41f, 0.018f, 5.24f},
    {128, 128, 1, 0.535f, 1.152f, 29.8f, 0.0f, 6.50f},
};

// The same model fitted to the kernels on the tiled weight copy (sweep of the
// 4 tiles x slices {1, 2, 3, 4, 6} over M in {128..2048} at the Qwen2.5-1.5B
// shapes; the choice lands within 1.4 % of the best measured plan in total).
constexpr TileCost kTilesTiled[4] = {
    {64, 64, 2, 0.198f, 0.438f, 3.77f, 0.0f, 5.61f},
    {64, 128, 1, 0.241f, 0.617f, 5.72f, 0.0016f, 4.71f},
    {128, 64, 2, 0.331f, 0.760f, 5.44f, 0.0055f, 4.67f},
    {128, 128, 1, 0.392f, 1.113f, 4.04f, 0.0038f, 7.91f},
};

float predict_us(const TileCost& t, int M, int N, int K, int slices, int cus) {
    const long long blocks = static_cast<long long>((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * slices;
    const float steps = static_cast<float>(K / BK) / slices;
    const long long slots = 2LL * cus;
    const long long rounds = (blocks + slots - 1) / slots;
    const long long last = blocks - (rounds - 1) * slots;
    float us = t.fixed + static_cast<float>(rounds - 1) * steps * t.step2 + steps * (last <= cus ? t.step1 : t.step2);
    if (slices > 1) us += t.split + t.split_mb * (static_cast<float>(slices) * M * N * 8.0f / 1e6f);
    return us;
}

// Tile and K-slice plan of a prefill GEMM: the configuration the time model
// predicts fastest among those whose split-K partials fit ws_floats, then the
// gemm_tile / gemm_slices overrides.
void plan_gemm(int M, int N, int K, size_t ws_floats, bool tiled, int& ti, int& slices) {
    const int cus = cu_count();
    const int KT = K / BK;
    const int max_slices = (K % 256 == 0) ? KT / 4 : KT;  // QUAD slices whole 256-k quads
    auto fits = [&](const TileCost& t, int s) {
        const size_t tiles = static_cast<size_t>((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
        return s == 1 || (s <= max_slices && KT / s >= 4 && static_cast<size_t>(s) * tiles * t.bm * t.bn <= ws_floats);
    };
    ti = 0;
    slices = 1;
    float best = 1e30f;
    for (int i = 0; i < 4; ++i) {
        for (int s : {1, 2, 3, 4, 6}) {
            if (s > 1 && !gemm_split_k_enabled()) break;
            if (!fits(kTiles[i], s)) continue;
            const float us = predict_us(tiled ? kTilesTiled[i] : kTiles[i], M, N, K, s, cus);
            if (us < best) { best = us; ti = i; slices = s; }
        }
    }
    if (const int f = gemm_forced_tile()) ti = f - 1;
    if (const int f = gemm_forced_slices()) slices = f;
    while (slices > 1 && !fits(kTiles[ti], slices)) --slices;
}

template <int MODE>
int launch_gemm(GemmParams p, hipStream_t stream, const char* what, Workspace ws, bool tiled = false) {
    if (p.M <= 0 || p.N <= 0) return QE_OK;
    p.ws = ws.ptr;
    const size_t ws_floats = ws.ptr == nullptr ? 0 : ws.floats;
    int ti = 0, slices = 1;
    plan_gemm(p.M, p.N, p.K, ws_floats, tiled, ti, slices);
    const TileCost& t = kTiles[ti];
    if ((p.M + t.bm - 1) / t.bm > 65535) return fail(QE_ERR_UNSUPPORTED, "%s: M=%d too large", what, p.M);
    if (tiled) {
        switch (ti) {
            case 0: launch_tiles<64, 64, 2, MODE, true>(p, slices, stream); break;
            case 1: launch_tiles<64, 128, 1, MODE, true>(p, slices, stream); break;
            case 2: launch_tiles<128, 64, 2, MODE, true>(p, slices, stream); break;
            default: launch_tiles<128, 128, 1, MODE, true>(p, slices, stream); break;
        }
    } else {
        switch (ti) {
            case 0: launch_tiles<64, 64, 2, MODE>(p, slices, stream); break;
            case 1: launch_tiles<64, 128, 1, MODE>(p, slices, stream); break;
            case 2: launch_tiles<128, 64, 2, MODE>(p, slices, stream); break;
            default: launch_tiles<128, 128, 1, MODE>(p, slices, stream); break;
        }
    }
    return check_launch(what);
}

// ---- W4A8 variant: int8 activations on the int8 matrix cores ----------------------
// v_mfma_i32_32x32x32_i8 takes 16 int8 k per lane; within one 128-group a
// lane half h covers k in [64h, 64h + 64), 16 per MFMA j (k = 64h + 16j), for
// both operands.  The weights enter as their unsigned nibbles q (two ops per
// 4 bytes: & 0x0F0F0F0F and >> 4); sum (q - 8) a = sum q a + the Q8_1 sum8
// terms (-8 * sum a per 8 elements), so the correction per row and group is
// the sum of its 16 sum8 words.  Per group: 4 MFMAs into an int32 tile from
// zero, then fp32 += float(int dot + correction) * (w_scale * x_scale) - the
// GEMV's per-chunk arithmetic with the four chunk dots summed first (integer
// addition; evaluated as w_s * (float(dot) * x_s + float(corr) * x_s), two
// fused multiply-adds per element and group).  A (Q8_1 int8 rows) and the
// per-row group scale/correction go through LDS; weights straight from
// global as in the fp16 kernel; K split into slices when the tile grid leaves
// CUs idle (partials reduced by the fp16 kernel's reduce pass).
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
constexpr int A8_STRIDE = 144;  // bytes per LDS row of the int8 A tile (128 + 16 pad)

template <int BM, int MODE>
__global__ __launch_bounds__(256, 2) void gemm_w4a8_mfma_kernel(GemmParams p) {
    constexpr int BN = 128, WGM = 1, MI = BM / 32;
    constexpr int A_U = BM / 32;  // 16-byte A chunks per thread per step: 8 threads per 128-byte row, 32 rows per pass
    constexpr int D = 2;          // stages of the register ring
    __shared__ __align__(16) int8_t sA[2][BM * A8_STRIDE];
    __shared__ __align__(16) float s_xs[2][BM];
    __shared__ __align__(16) float s_cr[2][BM];  // float(correction) * x_scale

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wn = tid >> 6;
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int K = p.K;
    const int G = K >> 7;
    const int slices = gridDim.z;
    const int g_begin = static_cast<int>((static_cast<long long>(blockIdx.z) * G) / slices);
    const int g_end = static_cast<int>((static_cast<long long>(blockIdx.z + 1) * G) / slices);
    const int KT = g_end - g_begin;  // one 128-group per step
    const int fr = lane & 31;
    const int h = lane >> 5;

    const int a_row = tid >> 3, a_c = tid & 7;
    const int8_t* a_src[A_U];
#pragma unroll
    for (int i = 0; i < A_U; ++i)
        a_src[i] = p.A8 + static_cast<size_t>(min(m0 + a_row + 32 * i, p.M - 1)) * K + 16 * a_c;
    const int srow = tid % BM;  // row whose group scale / correction this thread fetches
    const size_t srow_g = static_cast<size_t>(min(m0 + srow, p.M - 1));
    // B: the lane's column; columns past N read column N-1
    const int col = min(n0 + wn * 32 + fr, p.N - 1);
    int m = 0, local = col;
    if constexpr (MODE == kQKV) {
        m = (col >= p.col_begin[1]) + (col >= p.col_begin[2]);
        local = col - p.col_begin[m];
    }
    const u32x4* b_src = reinterpret_cast<const u32x4*>(p.qw[m] + static_cast<size_t>(local) * (K >> 3)) + 2 * h;
    const uint16_t* b_sc = p.sc[m] + static_cast<size_t>(local) * G;

    struct Stage {
        i32x4 a[A_U];
        float xs;
        i32x4 s8[4];
        u32x4 b[2];
        uint32_t bs;
    };
    Stage st[D];
    auto load = [&](int kt, Stage& S) __attribute__((always_inline)) {
        const int g = g_begin + kt;
#pragma unroll
        for (int i = 0; i < A_U; ++i) S.a[i] = *reinterpret_cast<const i32x4*>(a_src[i] + g * 128);
        S.xs = p.A8_scale[srow_g * G + g];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            S.s8[j] = *reinterpret_cast<const i32x4*>(p.A8_sum8 + srow_g * (K >> 3) + 16 * g + 4 * j);
        S.b[0] = b_src[4 * g];  // cached: every M tile of the column reads it
        S.b[1] = b_src[4 * g + 1];
        S.bs = b_sc[g];
    };
    auto store = [&](int buf, const Stage& S) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_U; ++i)
            *reinterpret_cast<i32x4*>(&sA[buf][(a_row + 32 * i) * A8_STRIDE + 16 * a_c]) = S.a[i];
        int cr = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) cr += S.s8[j].x + S.s8[j].y + S.s8[j].z + S.s8[j].w;
        s_xs[buf][srow] = S.xs;  // threads srow and srow + BM write the same values
        s_cr[buf][srow] = static_cast<float>(cr) * S.xs;
    };

    f32x16 f[MI][1];
#pragma unroll
    for (int i = 0; i < MI; ++i) f[i][0] = f32x16{};

#pragma unroll
    for (int d = 0; d < D; ++d) load(min(d, KT - 1), st[d]);
    store(0, st[0]);
    __syncthreads();

    auto step = [&](int kt, int d) __attribute__((always_inline)) {
        const int buf = kt & 1;
        const Stage& S = st[d];
        i32x16 acc[MI];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w0 = S.b[j >> 1][(2 * j) & 3], w1 = S.b[j >> 1][(2 * j + 1) & 3];
            const i32x4 bop = {static_cast<int>(w0 & 0x0F0F0F0Fu), static_cast<int>((w0 >> 4) & 0x0F0F0F0Fu),
                               static_cast<int>(w1 & 0x0F0F0F0Fu), static_cast<int>((w1 >> 4) & 0x0F0F0F0Fu)};
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const i32x4 aop =
                    *reinterpret_cast<const i32x4*>(&sA[buf][(i * 32 + fr) * A8_STRIDE + 64 * h + 16 * j]);
                acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aop, bop, j == 0 ? i32x16{} : acc[i], 0, 0, 0);
            }
        }
        const float ws = h2f(static_cast<uint16_t>(S.bs));
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4) {
                const int r0 = i * 32 + 8 * v4 + 4 * h;  // rows r0..r0+3 hold elements 4*v4 .. 4*v4+3
                const f32x4 xs4 = *reinterpret_cast<const f32x4*>(&s_xs[buf][r0]);
                const f32x4 cr4 = *reinterpret_cast<const f32x4*>(&s_cr[buf][r0]);
#pragma unroll
                for (int q = 0; q < 4; ++q) {  // f += w_s * (float(dot) * x_s + float(corr) * x_s)
                    const int v = 4 * v4 + q;
                    f[i][0][v] = fmaf(ws, fmaf(static_cast<float>(acc[i][v]), xs4[q], cr4[q]), f[i][0][v]);
                }
            }
        }
        load(min(kt + D, KT - 1), st[d]);  // step kt is consumed: refill with step kt + D
        store(buf ^ 1, st[(d + 1) % D]);   // step kt + 1, loaded D - 1 steps ago
        __syncthreads();
    };
    int kt = 0;
    for (; kt + D <= KT; kt += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) step(kt + d, d);
    }
    if (kt < KT) step(kt, 0);  // tail (D = 2)
    if (slices == 1) {
        epilogue<BM, BN, WGM, MODE>(p, f, m0, n0, 0, wn, lane);
        return;
    }
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    const int n_tiles = gridDim.x * gridDim.y;
    float* mine = p.ws + (static_cast<size_t>(blockIdx.z) * n_tiles + tile) * (BM * BN);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) mine[(i * 16 + v) * 256 + tid] = f[i][0][v];
}

template <int MODE>
int launch_gemm_w4a8(GemmParams p, hipStream_t stream, const char* what, Workspace ws) {
    if (p.M <= 0 || p.N <= 0) return QE_OK;
    p.ws = ws.ptr;
    const size_t ws_floats = ws.ptr == nullptr ? 0 : ws.floats;
    // 128-row tiles when they already give one block per CU, else 64-row tiles
    const int cus = cu_count();
    const int nt128 = ((p.M + 127) / 128) * ((p.N + 127) / 128);
    const bool big = nt128 >= cus;
    const int bm = big ? 128 : 64;
    if ((p.M + bm - 1) / bm > 65535) return fail(QE_ERR_UNSUPPORTED, "%s: M=%d too large", what, p.M);
    const dim3 grid((p.N + 127) / 128, (p.M + bm - 1) / bm);
    const int tiles = static_cast<int>(grid.x * grid.y);
    const int G = p.K / 128;
    int slices = 1;  // about two blocks per CU, >= 4 groups per slice
    if (tiles < cus && gemm_split_k_enabled()) slices = std::max(1, std::min((2 * cus + tiles - 1) / tiles, G / 4));
    if (const int f = gemm_forced_slices()) slices = std::max(1, std::min(f, G));
    while (slices > 1 && static_cast<size_t>(slices) * tiles * bm * 128 > ws_floats) --slices;
    const dim3 g3(grid.x, grid.y, slices);
    if (big) gemm_w4a8_mfma_kernel<128, MODE><<<g3, 256, 0, stream>>>(p);
    else gemm_w4a8_mfma_kernel<64, MODE><<<g3, 256, 0, stream>>>(p);
    if (slices > 1) {
        if (big) launch_reduce<128, 128, 1, MODE>(p, grid, slices, stream);
        else launch_reduce<64, 128, 1, MODE>(p, grid, slices, stream);
    }
    return check_launch(what);
}

// Tiled weight layout of the prefill GEMM (K % 256 == 0): the weights of 32
// columns and one 256-k quad are 4 KB in the order the kernel's lanes load
// them - load i of lane (h, c) reads 16-byte chunk 8 g + 4 h + i of column c -
// so each load instruction of a wave reads 1 KB of contiguous memory instead
// of 64 pieces of different columns, and each word holds its 8 nibbles in the
// order unpack_w4t_to_half8 reads fastest.  Columns padded to a multiple of
// 32 (weights q = 8, scales 0: the padding is zero).  Scales: for each 32 columns and quad, the 64 fp16
// scales the lanes need (group 2 g + h of column c at 32 h + c).
__global__ __launch_bounds__(256) void repack_w4_tiled_kernel(const u32x4* __restrict__ w, const uint16_t* __restrict__ sc,
                                                           int N, int K, u32x4* __restrict__ wt,
                                                           uint16_t* __restrict__ st) {
    const int Q = K >> 8;
    const int n_pad = (N + 31) & ~31;
    const size_t chunks = static_cast<size_t>(n_pad) * (K >> 5);
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    for (size_t t = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; t < chunks; t += stride) {
        // destination-ordered: t = ((ct * Q + g) * 4 + i) * 64 + 32 h + c
        const int c = static_cast<int>(t & 31), h = static_cast<int>((t >> 5) & 1), i = static_cast<int>((t >> 6) & 3);
        const size_t ctg = t >> 8;
        const int g = static_cast<int>(ctg % Q);
        const int col = static_cast<int>(ctg / Q) * 32 + c;
        u32x4 v = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};  // padding: q = 8, i.e. 0
        if (col < N) {
            v = w[static_cast<size_t>(col) * (K >> 5) + 8 * g + 4 * h + i];
            v = u32x4{w4_word_to_tiled(v.x), w4_word_to_tiled(v.y), w4_word_to_tiled(v.z), w4_word_to_tiled(v.w)};
        }
        wt[t] = v;
        if (i == 0) {
            const size_t so = (ctg << 6) + 32 * h + c;
            st[so] = col < N ? sc[static_cast<size_t>(col) * (K >> 7) + 2 * g + h] : uint16_t(0);
        }
    }
}

// Split-K workspaces, one per (device, stream).  A launch only looks its
// stream's workspace up and never allocates: a stream without one runs its
// GEMMs without K slices, eagerly and under capture alike, so the plan and
// the bits of a launch depend only on the shape, the tuning switches and
// whether the stream holds a workspace.  qe_gemm_reserve_workspace
// allocates one (the library owns it), qe_gemm_attach_workspace registers
// caller memory (the engine's arena), qe_gemm_release_workspace drops the
// entry.  hipStreamPerThread names a different stream in each thread, so it
// never holds a workspace (its GEMMs run unsplit); the null stream is the one
// legacy stream of the device (this library is built without per-thread
// default streams), shared correctly ordered by every thread.
constexpr int kMaxWsStreams = 64;
struct WsSlot {
    hipStream_t stream;
    float* ptr;
    size_t floats;
    bool owned;  // allocated by qe_gemm_reserve_workspace
};
std::mutex g_ws_mutex;
WsSlot g_ws[64][kMaxWsStreams];
int g_ws_count[64];
std::atomic<long> g_ws_allocations{0};  // hipMalloc calls made for workspaces

bool per_thread_handle(hipStream_t stream) { return stream == hipStreamPerThread; }

Workspace gemm_workspace(hipStream_t stream) {
    if (!gemm_split_k_enabled() || per_thread_handle(stream)) return {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return {};
    }
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    for (int i = 0; i < g_ws_count[dev]; ++i)
        if (g_ws[dev][i].stream == stream) return {g_ws[dev][i].ptr, g_ws[dev][i].floats};
    return {};
}

// registers (ptr, floats) for `stream` on the current device; the caller
// holds g_ws_mutex.  Returns the slot or nullptr when the table is full.
WsSlot* ws_find_or_add(int dev, hipStream_t stream, bool* found) {
    for (int i = 0; i < g_ws_count[dev]; ++i)
        if (g_ws[dev][i].stream == stream) {
            *found = true;
            return &g_ws[dev][i];
        }
    *found = false;
    if (g_ws_count[dev] == kMaxWsStreams) return nullptr;
    WsSlot* s = &g_ws[dev][g_ws_count[dev]++];
    *s = WsSlot{stream, nullptr, 0, false};
    return s;
}

int current_device(const char* what, int* dev) {
    if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= 64) {
        (void)hipGetLastError();
        return fail(QE_ERR_HIP, "%s: no current device", what);
    }
    return QE_OK;
}

}  // namespace
}  // namespace qe

extern "C" int qe_gemm_reserve_workspace(hipStream_t stream) {
    const char* what = "gemm_reserve_workspace";
    QE_REQUIRE(!qe::per_thread_handle(stream), "%s: hipStreamPerThread cannot hold a workspace (its GEMMs run "
               "without K slices)", what);
    int dev = 0;
    QE_TRY(qe::current_device(what, &dev));
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return qe::fail(QE_ERR_HIP, "%s: invalid stream", what);
    }
    QE_REQUIRE(st == hipStreamCaptureStatusNone, "%s: stream is capturing", what);
    std::lock_guard<std::mutex> lock(qe::g_ws_mutex);
    bool found = false;
    qe::WsSlot* s = qe::ws_find_or_add(dev, stream, &found);
    if (s == nullptr)
        return qe::fail(QE_ERR_UNSUPPORTED, "%s: %d streams already hold a workspace on this device", what,
                        qe::kMaxWsStreams);
    if (found && s->floats >= qe::kWsFloats) {
        qe::clear_error();
        return QE_OK;
    }
    void* ptr = nullptr;
    ++qe::g_ws_allocations;
    if (hipMalloc(&ptr, qe::kWsFloats * sizeof(float)) != hipSuccess) {
        (void)hipGetLastError();
        if (!found) --qe::g_ws_count[dev];
        return qe::fail(QE_ERR_HIP, "%s: hipMalloc of %zu bytes failed", what, qe::kWsFloats * sizeof(float));
    }
    if (found && s->owned) (void)hipFree(s->ptr);
    *s = qe::WsSlot{stream, static_cast<float*>(ptr), qe::kWsFloats, true};
    qe::clear_error();
    return QE_OK;
}

extern "C" int qe_gemm_attach_workspace(hipStream_t stream, void* workspace, size_t bytes) {
    const char* what = "gemm_attach_workspace";
    QE_REQUIRE(!qe::per_thread_handle(stream), "%s: hipStreamPerThread cannot hold a workspace", what);
    QE_REQUIRE(workspace != nullptr && qe::aligned(workspace, 256), "%s: workspace must be non-NULL and "
               "256-byte aligned", what);
    QE_REQUIRE(bytes >= (size_t(1) << 20), "%s: %zu bytes is below the 1 MiB minimum", what, bytes);
    int dev = 0;
    QE_TRY(qe::current_device(what, &dev));
    std::lock_guard<std::mutex> lock(qe::g_ws_mutex);
    bool found = false;
    qe::WsSlot* s = qe::ws_find_or_add(dev, stream, &found);
    if (s == nullptr)
        return qe::fail(QE_ERR_UNSUPPORTED, "%s: %d streams already hold a workspace on this device", what,
                        qe::kMaxWsStreams);
    if (found && s->owned) (void)hipFree(s->ptr);
    *s = qe::WsSlot{stream, static_cast<float*>(workspace), std::min(bytes / sizeof(float), qe::kWsFloats), false};
    qe::clear_error();
    return QE_OK;
}

extern "C" int qe_gemm_release_workspace(hipStream_t stream) {
    int dev = 0;
    QE_TRY(qe::current_device("gemm_release_workspace", &dev));
    std::lock_guard<std::mutex> lock(qe::g_ws_mutex);
    for (int i = 0; i < qe::g_ws_count[dev]; ++i)
        if (qe::g_ws[dev][i].stream == stream) {
            if (qe::g_ws[dev][i].owned) (void)hipFree(qe::g_ws[dev][i].ptr);
            qe::g_ws[dev][i] = qe::g_ws[dev][--qe::g_ws_count[dev]];
            break;
        }
    qe::clear_error();
    return QE_OK;
}

extern "C" long qe_gemm_workspace_allocations(void) { return qe::g_ws_allocations.load(); }

namespace qe {
namespace {

// Scratch of the allocation-free entry point: a file-scope device array of
// the same capacity as a stream's workspace, so that entry point makes the
// same tile and K-slice plan as qe_launch_gemm_prefill_w4a16.  Its device
// address comes from hipGetSymbolAddress, once per device; host code uses
// only that address (the array's name is not a device address on the host).
__device__ __align__(256) float scratch[kWsFloats];
std::mutex g_scratch_mutex;
float* g_scratch_ptr[64];

float* scratch_address(int dev) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            (void)hipGetLastError();
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<float*>(ptr);
    }
    return g_scratch_ptr[dev];
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
    return launch_gemm<kPlain>(p, stream, what, gemm_workspace(stream));
}

extern "C" int qe_launch_gemm_prefill_w4a16_noalloc(const uint32_t* qweight, const uint16_t* scales,
                                                    const uint16_t* input_x, const uint16_t* residual,
                                                    uint16_t* output_y, int M, int N, int K, hipStream_t stream,
                                                    int sm_count) {
    (void)sm_count;
    const char* what = "gemm_prefill_w4a16_noalloc";
    if (int rc = check_gemm_common(what, input_x, M, K)) return rc;
    QE_REQUIRE(qweight && scales && output_y, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(N >= 0, "%s: N=%d", what, N);
    QE_REQUIRE(aligned(qweight, 16) && aligned(scales, 2), "%s: qweight must be 16-byte aligned", what);
    // the largest shape whose K-slice plan this entry point accepts: one
    // fp32 partial tile set of M x N per slice must fit the scratch at least
    // once (larger shapes are rejected rather than silently left unsplit)
    QE_REQUIRE(static_cast<size_t>(M) * static_cast<size_t>(N) <= kWsFloats,
               "%s: M*N=%zu exceeds the scratch of %zu floats", what,
               static_cast<size_t>(M) * static_cast<size_t>(N), kWsFloats);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return fail(QE_ERR_HIP, "%s: no current device", what);
    float* ws = gemm_split_k_enabled() ? scratch_address(dev) : nullptr;
    if (gemm_split_k_enabled() && ws == nullptr)
        return fail(QE_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed", what);
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
    return launch_gemm<kPlain>(p, stream, what, Workspace{ws, kWsFloats});
}

extern "C" int qe_gemm_prefill_plan(int M, int N, int K, int tiled, int* tile, int* slices) {
    QE_REQUIRE(M > 0 && N > 0 && K > 0 && K % 128 == 0 && tile && slices, "gemm_prefill_plan: bad arguments");
    int ti = 0, s = 1;
    plan_gemm(M, N, K, kWsFloats, tiled != 0, ti, s);
    *tile = ti + 1;
    *slices = s;
    return QE_OK;
}

extern "C" int qe_w4_tiled_bytes(int N, int K, size_t* weight_bytes, size_t* scale_bytes) {
    QE_REQUIRE(N > 0 && K > 0 && K % 256 == 0, "w4_tiled_bytes: N=%d K=%d (K must be a multiple of 256)", N, K);
    QE_REQUIRE(weight_bytes && scale_bytes, "w4_tiled_bytes: NULL output");
    const size_t n_pad = (static_cast<size_t>(N) + 31) & ~size_t(31);
    *weight_bytes = n_pad * K / 2;
    *scale_bytes = n_pad * (K / 128) * 2;
    return QE_OK;
}

extern "C" int qe_repack_w4_tiled(const uint32_t* qweight, const uint16_t* scales, int N, int K,
                                  uint32_t* tiled_weight, uint16_t* tiled_scales, hipStream_t stream) {
    const char* what = "repack_w4_tiled";
    QE_REQUIRE(qweight && scales && tiled_weight && tiled_scales, "%s: NULL pointer", what);
    QE_REQUIRE(N > 0 && K > 0 && K % 256 == 0, "%s: N=%d K=%d (K must be a multiple of 256)", what, N, K);
    QE_REQUIRE(aligned(qweight, 16) && aligned(tiled_weight, 16) && aligned(scales, 2) && aligned(tiled_scales, 2),
               "%s: weights must be 16-byte aligned", what);
    const size_t chunks = ((static_cast<size_t>(N) + 31) & ~size_t(31)) * (K >> 5);
    const unsigned grid = static_cast<unsigned>(std::min<size_t>((chunks + 255) / 256, size_t(cu_count()) * 16));
    repack_w4_tiled_kernel<<<grid, 256, 0, stream>>>(reinterpret_cast<const u32x4*>(qweight), scales, N, K,
                                                     reinterpret_cast<u32x4*>(tiled_weight), tiled_scales);
    return check_launch(what);
}

extern "C" int qe_launch_gemm_prefill_w4a16_tiled(const uint32_t* tiled_weight, const uint16_t* tiled_scales,
                                                  const uint16_t* input_x, const uint16_t* residual,
                                                  uint16_t* output_y, int M, int N, int K, hipStream_t stream) {
    const char* what = "gemm_prefill_w4a16_tiled";
    if (int rc = check_gemm_common(what, input_x, M, K)) return rc;
    QE_REQUIRE(K % 256 == 0, "%s: K=%d must be a multiple of 256", what, K);
    QE_REQUIRE(tiled_weight && tiled_scales && output_y, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(N >= 0, "%s: N=%d", what, N);
    QE_REQUIRE(aligned(tiled_weight, 16) && aligned(tiled_scales, 2), "%s: weights must be 16-byte aligned", what);
    GemmParams p{};
    p.qw[0] = tiled_weight;
    p.sc[0] = tiled_scales;
    p.out[0] = output_y;
    p.out_stride[0] = N;
    p.A = input_x;
    p.residual = residual;
    p.M = M;
    p.N = N;
    p.K = K;
    return launch_gemm<kPlain>(p, stream, what, gemm_workspace(stream), true);
}

extern "C" int qe_launch_gemm_prefill_qkv_w4a16_tiled(const qe_qkv_view* view, const uint16_t* input_x, int M,
                                                      hipStream_t stream, int in_features, int num_q_heads,
                                                      int num_kv_heads, int head_dim) {
    const char* what = "gemm_prefill_qkv_w4a16_tiled";
    if (int rc = check_gemm_common(what, input_x, M, in_features)) return rc;
    QE_REQUIRE(in_features % 256 == 0, "%s: in_features=%d must be a multiple of 256", what, in_features);
    QE_REQUIRE(view != nullptr, "%s: view is NULL", what);
    QE_REQUIRE(num_q_heads >= 0 && num_kv_heads >= 0 && head_dim >= 0, "%s: negative head shape", what);
    const int q_dim = num_q_heads * head_dim;
    const int kv_dim = num_kv_heads * head_dim;
    // a 32-column tile must not straddle two matrices
    QE_REQUIRE(q_dim % 32 == 0 && kv_dim % 32 == 0, "%s: q and kv widths must be multiples of 32", what);
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
    return launch_gemm<kQKV>(p, stream, what, gemm_workspace(stream), true);
}

extern "C" int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(const uint32_t* tiled_weight,
                                                                      const uint16_t* tiled_scales,
                                                                      const uint16_t* input_x, uint16_t* output_mlp,
                                                                      int M, hipStream_t stream, int hidden_size,
                                                                      int intermediate_size) {
    const char* what = "gemm_prefill_dual_gate_up_swiglu_w4a16_tiled";
    if (int rc = check_gemm_common(what, input_x, M, hidden_size)) return rc;
    QE_REQUIRE(hidden_size % 256 == 0, "%s: hidden_size=%d must be a multiple of 256", what, hidden_size);
    QE_REQUIRE(tiled_weight && tiled_scales && output_mlp, "%s: NULL weight/scale/output", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(tiled_weight, 16) && aligned(tiled_scales, 2), "%s: weights must be 16-byte aligned", what);
    GemmParams p{};
    p.qw[0] = tiled_weight;
    p.sc[0] = tiled_scales;
    p.out[0] = output_mlp;
    p.out_stride[0] = intermediate_size;
    p.A = input_x;
    p.M = M;
    p.N = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemm<kSwiglu>(p, stream, what, gemm_workspace(stream), true);
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
    return launch_gemm<kQKV>(p, stream, what, gemm_workspace(stream));
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
    return launch_gemm<kSwiglu>(p, stream, what, gemm_workspace(stream));
}

// ---- W4A8 prefill GEMM entry points --------------------------------------------------
namespace {
int check_gemm_a8(const char* what, const int8_t* q8, const float* xs, const int32_t* s8, int M, int K) {
    QE_REQUIRE(q8 && xs && s8, "%s: Q8_1 input pointers must not be NULL", what);
    QE_REQUIRE(M >= 0, "%s: M=%d", what, M);
    QE_REQUIRE(K > 0 && K % 128 == 0, "%s: K=%d must be a positive multiple of 128", what, K);
    QE_REQUIRE(aligned(q8, 16) && aligned(s8, 16) && aligned(xs, 4), "%s: Q8_1 rows must be 16-byte aligned", what);
    return QE_OK;
}
}  // namespace

extern "C" int qe_launch_gemm_prefill_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                                           const float* input_scale, const int32_t* input_sum8,
                                           const uint16_t* residual, uint16_t* output_y, int M, int N, int K,
                                           hipStream_t stream) {
    const char* what = "gemm_prefill_w4a8";
    if (int rc = check_gemm_a8(what, input_q8, input_scale, input_sum8, M, K)) return rc;
    QE_REQUIRE(qweight && scales && output_y && N >= 0, "%s: NULL weight/scale/output or N < 0", what);
    QE_REQUIRE(aligned(qweight, 16) && aligned(scales, 2), "%s: qweight must be 16-byte aligned", what);
    GemmParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = output_y;
    p.out_stride[0] = N;
    p.A8 = input_q8;
    p.A8_scale = input_scale;
    p.A8_sum8 = input_sum8;
    p.residual = residual;
    p.M = M;
    p.N = N;
    p.K = K;
    return launch_gemm_w4a8<kPlain>(p, stream, what, gemm_workspace(stream));
}

extern "C" int qe_launch_gemm_prefill_qkv_w4a8(const qe_qkv_view* view, const int8_t* input_q8,
                                               const float* input_scale, const int32_t* input_sum8, int M,
                                               hipStream_t stream, int in_features, int num_q_heads,
                                               int num_kv_heads, int head_dim) {
    const char* what = "gemm_prefill_qkv_w4a8";
    if (int rc = check_gemm_a8(what, input_q8, input_scale, input_sum8, M, in_features)) return rc;
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
    p.A8 = input_q8;
    p.A8_scale = input_scale;
    p.A8_sum8 = input_sum8;
    p.M = M;
    p.N = q_dim + 2 * kv_dim;
    p.K = in_features;
    return launch_gemm_w4a8<kQKV>(p, stream, what, gemm_workspace(stream));
}

extern "C" int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight,
                                                               const uint16_t* gate_up_scales,
                                                               const int8_t* input_q8, const float* input_scale,
                                                               const int32_t* input_sum8, uint16_t* output_mlp, int M,
                                                               hipStream_t stream, int hidden_size,
                                                               int intermediate_size) {
    const char* what = "gemm_prefill_dual_gate_up_swiglu_w4a8";
    if (int rc = check_gemm_a8(what, input_q8, input_scale, input_sum8, M, hidden_size)) return rc;
    QE_REQUIRE(gate_up_qweight && gate_up_scales && output_mlp && intermediate_size >= 0, "%s: bad arguments", what);
    QE_REQUIRE(aligned(gate_up_qweight, 16) && aligned(gate_up_scales, 2), "%s: qweight must be 16-byte aligned",
               what);
    GemmParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.out_stride[0] = intermediate_size;
    p.A8 = input_q8;
    p.A8_scale = input_scale;
    p.A8_sum8 = input_sum8;
    p.M = M;
    p.N = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemm_w4a8<kSwiglu>(p, stream, what, gemm_workspace(stream));
}
