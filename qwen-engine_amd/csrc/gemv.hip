// W4A8 / W4A16 group-128 decode GEMV family for gfx950.
//
// Math (bit-for-bit on the integer stage) of src/kernels/gemv_w4a16.cu:
//   per 32-element chunk: dot = sum of 4 dp4a_w4_q8_oct seeded with sum8,
//   acc += float(dot) * (float(w_scale) * x_scale),  y = fp16(acc [+ res]).
// The four sum8 seeds of a chunk are added before the dot (integer
// addition, so the dot is unchanged).
//
// Work layout (MI355X-first; these launches are latency-bound, so the
// critical path is kept to one round of loads):
//   * A "segment" of LPR lanes (16 or 64, inside one wave64) owns RPS
//     consecutive weight rows per iteration; lane l owns the 32-element
//     chunks c = l + i*LPR (i < NCH) of every row, so the only per-row
//     traffic is one 16-byte global_load_dwordx4 (nt) per chunk plus the
//     fp16 scale.  Segment loads are contiguous (16*LPR bytes).
//   * Q8_1 activations (W4A8): each lane loads just its own chunks straight
//     into VGPRs - no LDS, no barrier.  fp16 activations (W4A16, and the
//     fused RMSNorm entry points): the 256-thread block quantizes the vector
//     once, 8 elements per thread (a 128-group is one 16-lane DPP row), into
//     LDS, and each lane then reads its chunks.
//   * The first row set's weights are requested at kernel entry, before
//     the activation, and each iteration prefetches the next row set.
//   * Partial sums are reduced in the segment with DPP row operations
//     (quad_perm, row_half_mirror, row_mirror), ds_swizzle for 32 lanes.
//   * 64-thread blocks unless the matrix is large enough for 256-thread
//     persistent blocks (grid capped per CU).
// Shapes outside the fast kernel (weights not 16-byte aligned, K > 16384)
// use a generic wave-per-row kernel that stages Q8_1 in LDS.
#include <algorithm>

#include "attn_common.hpp"
#include "rms_common.hpp"
#include "rope_common.hpp"
#include "sample_common.hpp"

namespace qe {
namespace {

constexpr int kPlain = 0;
constexpr int kQKV = 1;
constexpr int kSwiglu = 2;
constexpr int kSample = 3;  // LM head: plain rows, logits optional, (value, index) partial per block

constexpr int kXQ8 = 0;   // Q8_1 activation
constexpr int kXF16 = 1;  // fp16 activation, quantized in the block
constexpr int kXRMS = 2;  // fp16 activation, RMSNorm then quantized in the block
// flash-decode split partials, combined and quantized in the block; the
// first 4, 8 or all 16 splits are read
constexpr int kXATTN4 = 3;
constexpr int kXATTN8 = 4;
constexpr int kXATTN16 = 5;

constexpr float kRmsEps = 1e-6f;  // RMS_NORM_EPS, include/config.cuh:20

struct GemvParams {
    const uint32_t* qw[3];
    const uint16_t* sc[3];
    uint16_t* out[3];
    int row_begin[3];  // first physical row of each matrix (QKV mode)
    const uint16_t* residual;
    const int8_t* q8;
    const float* xs;
    const int32_t* s8;
    const uint16_t* x16;    // fp16 activation (kXF16 / kXRMS)
    const uint16_t* gamma;  // RMSNorm weight (kXRMS)
    uint16_t* norm_out;     // optional fp16 copy of the staged activation (kXRMS: normalized,
                            // attention: combined attention output; block 0 writes)
    const float* part_o;    // attention: split partials [head][16][128]
    const float* part_lse;  // attention: (max, denominator) [head][16][2]
    float* s_val;           // kSample: per-block best value / index
    int32_t* s_idx;
    const qe_device_control_block* ctl;  // kSample: temperature, rng_seed, seq_pos; QKV rope: seq_pos
    // QKV with rope != 0: bias, NeoX RoPE (head_dim 128) and the KV-cache append in the epilogue
    int rope;
    const uint16_t* bias[3];
    uint16_t* kcache;
    uint16_t* vcache;
    int max_seq;
    float rope_theta;
    int n_rows;             // physical weight rows
    int K;
};

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

__device__ __forceinline__ void unpack8(const uint4 raw, float vals[8]) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        vals[2 * j] = h2f(static_cast<uint16_t>(w[j] & 0xFFFFu));
        vals[2 * j + 1] = h2f(static_cast<uint16_t>(w[j] >> 16));
    }
}

__device__ __forceinline__ uint4 load8_f16(const uint16_t* p, bool vec) {
    if (vec) return *reinterpret_cast<const uint4*>(p);
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = static_cast<uint32_t>(p[2 * j]) | (static_cast<uint32_t>(p[2 * j + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// fp16(fp16(x*h)*g) for 8 packed values: the two fp16 multiplies of the
// reference RMSNorm (src/kernels/rmsnorm_rope.cu:214-227).
__device__ __forceinline__ uint4 rms_apply8(uint4 xv, uint4 gv, _Float16 h) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const qwen::qe_half2_t hh = {h, h};
        qwen::qe_half2_t n = __builtin_bit_cast(qwen::qe_half2_t, xw[j]) * hh;
        n = n * __builtin_bit_cast(qwen::qe_half2_t, gw[j]);
        o[j] = __builtin_bit_cast(uint32_t, n);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Stage the activation of the whole block in LDS: s_q8[K] and, per
// 32-element chunk, s_rec[c] = {sum8[4c..4c+3] summed, bits of x_scale}.
// VEC: 16-byte vector loads are legal for the activation buffers.
// kXRMS: s_units holds K / 8 floats for the sum of squares.
template <int XM, int BT, bool VEC>
__device__ __forceinline__ void stage_activation(const GemvParams& p, int8_t* s_q8, int2* s_rec,
                                                 float* s_units) {
    const int K = p.K;
    const int G = K >> 7;
    if constexpr (XM == kXQ8) {
        if (VEC) {
            for (int i = threadIdx.x; i < (K >> 4); i += BT)
                reinterpret_cast<uint4*>(s_q8)[i] = reinterpret_cast<const uint4*>(p.q8)[i];
        } else {
            for (int i = threadIdx.x; i < K; i += BT) s_q8[i] = p.q8[i];
        }
        for (int c = threadIdx.x; c < (K >> 5); c += BT) {
            const int32_t* s = p.s8 + 4 * c;
            s_rec[c] = make_int2(s[0] + s[1] + s[2] + s[3], __builtin_bit_cast(int, p.xs[c >> 2]));
        }
    } else {
        _Float16 h = static_cast<_Float16>(0.0f);
        if constexpr (XM == kXRMS) {
            for (int i = threadIdx.x; i < (K >> 3); i += BT) s_units[i] = rms_unit_sq(load8_f16(p.x16 + 8 * i, VEC));
            h = rms_inv_f16_each_wave(s_units, K >> 3, K, kRmsEps);
        }
        const int sub = threadIdx.x & 15;
        for (int g = threadIdx.x >> 4; g < G; g += BT / 16) {
            uint4 raw = load8_f16(p.x16 + g * 128 + sub * 8, VEC);
            if constexpr (XM == kXRMS) {
                raw = rms_apply8(raw, load8_f16(p.gamma + g * 128 + sub * 8, VEC), h);
                if (p.norm_out != nullptr && blockIdx.x == 0) {
                    uint16_t* o = p.norm_out + g * 128 + sub * 8;
                    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        o[2 * j] = static_cast<uint16_t>(w[j] & 0xFFFFu);
                        o[2 * j + 1] = static_cast<uint16_t>(w[j] >> 16);
                    }
                }
            }
            float vals[8];
            unpack8(raw, vals);
            const qwen::Q8Group q = qwen::quantize_group128_q8_1(vals);
            *reinterpret_cast<int2*>(s_q8 + g * 128 + sub * 8) = make_int2(q.x_lo, q.x_hi);
            // chunk j of the group = lanes 4j..4j+3 of the 16-lane row
            int csum = q.sum8;
            csum += qwen::dpp_i32<0xB1>(csum);
            csum += qwen::dpp_i32<0x4E>(csum);
            if ((sub & 3) == 0) s_rec[g * 4 + (sub >> 2)] = make_int2(csum, __builtin_bit_cast(int, q.d));
        }
    }
}

__device__ __forceinline__ int32_t chunk_dot(const u32x4 w, const int4 xa, const int4 xb, int32_t seed) {
    int32_t d = qwen::dp4a_w4_q8_oct(w.x, xa.x, xa.y, seed);
    d = qwen::dp4a_w4_q8_oct(w.y, xa.z, xa.w, d);
    d = qwen::dp4a_w4_q8_oct(w.z, xb.x, xb.y, d);
    return qwen::dp4a_w4_q8_oct(w.w, xb.z, xb.w, d);
}

// Pointers of physical row `row`.  QKV: `urow` is a row of the same matrix
// that is uniform across the wave (the launch guarantees that the matrix
// boundaries fall on whole blocks), so the matrix choice is scalar and
// selects between kernel arguments instead of indexing them in memory.
template <int MODE>
__device__ __forceinline__ void row_ptrs(const GemvParams& p, int row, int urow, const u32x4*& w, const uint16_t*& s,
                                         int& m, int& local) {
    m = 0;
    local = row;
    const uint32_t* qw = p.qw[0];
    const uint16_t* sc = p.sc[0];
    if constexpr (MODE == kQKV) {
        const int u = __builtin_amdgcn_readfirstlane(urow);
        m = (u >= p.row_begin[1]) + (u >= p.row_begin[2]);
        local = row - (m == 0 ? 0 : (m == 1 ? p.row_begin[1] : p.row_begin[2]));
        qw = m == 0 ? p.qw[0] : (m == 1 ? p.qw[1] : p.qw[2]);
        sc = m == 0 ? p.sc[0] : (m == 1 ? p.sc[1] : p.sc[2]);
    } else {
        (void)urow;
    }
    w = reinterpret_cast<const u32x4*>(qw + static_cast<size_t>(local) * (p.K >> 3));
    s = sc + static_cast<size_t>(local) * (p.K >> 7);
}

// QKV: the per-matrix kernel arguments, loaded together at entry and held in
// scalar registers (the asm makes their values opaque, so the compiler does
// not re-derive a selected pointer as a dependent load from the argument
// block later).
// Global (address space 1) pointer types: after the asm the compiler cannot
// see where a pointer came from, and a generic one would be read with flat
// loads (which also count against the scalar-load counter).
typedef const uint32_t __attribute__((address_space(1)))* g_u32p;
typedef const uint16_t __attribute__((address_space(1)))* g_u16p;
typedef uint16_t __attribute__((address_space(1)))* g_u16p_mut;

struct QkvArgs {
    g_u32p qw[3];
    g_u16p sc[3];
    g_u16p bias[3];
    g_u16p_mut out[3];
    int rb1, rb2;
};

__device__ __forceinline__ QkvArgs load_qkv_args(const GemvParams& p) {
    QkvArgs a{{(g_u32p)p.qw[0], (g_u32p)p.qw[1], (g_u32p)p.qw[2]},
              {(g_u16p)p.sc[0], (g_u16p)p.sc[1], (g_u16p)p.sc[2]},
              {(g_u16p)p.bias[0], (g_u16p)p.bias[1], (g_u16p)p.bias[2]},
              {(g_u16p_mut)p.out[0], (g_u16p_mut)p.out[1], (g_u16p_mut)p.out[2]},
              p.row_begin[1],
              p.row_begin[2]};
    asm volatile("" : "+s"(a.qw[0]), "+s"(a.qw[1]), "+s"(a.qw[2]), "+s"(a.sc[0]), "+s"(a.sc[1]), "+s"(a.sc[2]),
                 "+s"(a.bias[0]), "+s"(a.bias[1]), "+s"(a.bias[2]), "+s"(a.out[0]), "+s"(a.out[1]), "+s"(a.out[2]),
                 "+s"(a.rb1), "+s"(a.rb2));
    return a;
}

template <typename T>
__device__ __forceinline__ T pick3(const T (&v)[3], int m) {
    return m == 0 ? v[0] : (m == 1 ? v[1] : v[2]);
}

__device__ __forceinline__ void row_ptrs_qkv(const QkvArgs& a, int K, int row, int urow, const u32x4*& w,
                                             const uint16_t*& s, int& m, int& local) {
    const int u = __builtin_amdgcn_readfirstlane(urow);
    m = (u >= a.rb1) + (u >= a.rb2);
    local = row - (m == 0 ? 0 : (m == 1 ? a.rb1 : a.rb2));
    w = reinterpret_cast<const u32x4*>((const uint32_t*)(pick3(a.qw, m) + static_cast<size_t>(local) * (K >> 3)));
    s = (const uint16_t*)(pick3(a.sc, m) + static_cast<size_t>(local) * (K >> 7));
}

// Q8_1 activation staged by the whole block: thread t copies chunk
// c = t + BT*j (32 q8 bytes, its four sum8 words summed, its group scale)
// into LDS.  stage_issue_q8 requests the loads (clamped, so every thread
// issues the same count); stage_finish_q8 stores them.
template <int BT, int MQ>
__device__ __forceinline__ void stage_issue_q8(const GemvParams& p, u32x4 (&qa)[MQ], u32x4 (&qb)[MQ],
                                               int4 (&s4)[MQ], float (&xd)[MQ]) {
    const int KC = p.K >> 5;
#pragma unroll
    for (int j = 0; j < MQ; ++j) {
        const int c = min(static_cast<int>(threadIdx.x) + BT * j, KC - 1);
        qa[j] = *reinterpret_cast<const u32x4*>(p.q8 + c * 32);
        qb[j] = *reinterpret_cast<const u32x4*>(p.q8 + c * 32 + 16);
        s4[j] = *reinterpret_cast<const int4*>(p.s8 + c * 4);
        xd[j] = p.xs[c >> 2];
    }
}

// Threads past the last chunk store to a dummy LDS slot (s_rec[KC]) rather
// than branching: a branch would let the compiler sink the activation loads
// below the weight loads and wait for both.
template <int BT, int MQ>
__device__ __forceinline__ void stage_finish_q8(const GemvParams& p, const u32x4 (&qa)[MQ], const u32x4 (&qb)[MQ],
                                                const int4 (&s4)[MQ], const float (&xd)[MQ], int8_t* s_q8,
                                                int2* s_rec) {
    const int KC = p.K >> 5;
#pragma unroll
    for (int j = 0; j < MQ; ++j) {
        const int c = static_cast<int>(threadIdx.x) + BT * j;
        const bool ok = c < KC;
        int8_t* dq = ok ? s_q8 + c * 32 : reinterpret_cast<int8_t*>(s_rec + KC);
        *reinterpret_cast<u32x4*>(dq) = qa[j];
        *reinterpret_cast<u32x4*>(dq + 16) = qb[j];
        s_rec[ok ? c : KC] = make_int2(s4[j].x + s4[j].y + s4[j].z + s4[j].w, __builtin_bit_cast(int, xd[j]));
    }
}

// fp16 activation staged by the whole block: thread t quantizes the 8
// elements 8u..8u+7 for u = t + BT*j (a 128-group is one 16-lane DPP row,
// the quantizer is quantize_group128_q8_1), RMS-normalizing first for kXRMS.
// stage_issue_f16 requests the loads (before the weights, so the
// activation is not queued behind them); stage_finish_f16 computes.  Output
// in LDS: q8[K] and per 32-element chunk {summed sum8 of its 4 words, scale}.
template <int XM, int BT, int MAXP>
__device__ __forceinline__ void stage_issue_f16(const GemvParams& p, uint4 (&raw)[MAXP], uint4 (&graw)[MAXP]) {
    const int U = p.K >> 3;  // 8-element units
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < MAXP; ++j) {
        const int u = min(t + BT * j, U - 1);
        raw[j] = *reinterpret_cast<const uint4*>(p.x16 + 8 * u);
        if constexpr (XM == kXRMS) graw[j] = *reinterpret_cast<const uint4*>(p.gamma + 8 * u);
    }
}

template <int XM, int BT, int MAXP>
__device__ __forceinline__ void stage_finish_f16(const GemvParams& p, uint4 (&raw)[MAXP], const uint4 (&graw)[MAXP],
                                                 int8_t* s_q8, int2* s_rec, float* s_units) {
    const int K = p.K;
    const int U = K >> 3;  // 8-element units
    const int t = threadIdx.x;
    if constexpr (XM == kXRMS) {
#pragma unroll
        for (int j = 0; j < MAXP; ++j)
            if (t + BT * j < U) s_units[t + BT * j] = rms_unit_sq(raw[j]);
        const _Float16 h = rms_inv_f16_each_wave(s_units, U, K, kRmsEps);
        const bool write_norm = p.norm_out != nullptr && blockIdx.x == 0;
#pragma unroll
        for (int j = 0; j < MAXP; ++j) {
            raw[j] = rms_apply8(raw[j], graw[j], h);
            if (write_norm && t + BT * j < U) *reinterpret_cast<uint4*>(p.norm_out + 8 * (t + BT * j)) = raw[j];
        }
    }
    // every thread quantizes (units past the end repeat the last unit; a
    // 16-lane row is a whole group, so such rows never mix with real ones)
    // and stores to a dummy LDS slot (s_rec[KC]) when out of range
    const int KC = K >> 5;
    const int wave_first = __builtin_amdgcn_readfirstlane(t) & ~63;
#pragma unroll
    for (int j = 0; j < MAXP; ++j) {
        // a wave whose units all lie past the end skips the pass (wave-uniform;
        // U is a multiple of 16, so a 16-lane group is all real or all past)
        if (BT * j < U && (j == 0 || wave_first + BT * j < U)) {
            const int u = t + BT * j;
            const bool ok = u < U;
            float vals[8];
            unpack8(raw[j], vals);
            const qwen::Q8Group q = qwen::quantize_group128_q8_1(vals);
            int8_t* dq = ok ? s_q8 + 8 * u : reinterpret_cast<int8_t*>(s_rec + KC);
            *reinterpret_cast<int2*>(dq) = make_int2(q.x_lo, q.x_hi);
            int csum = q.sum8;  // chunk = the 4 words of a DPP quad
            csum += qwen::dpp_i32<0xB1>(csum);
            csum += qwen::dpp_i32<0x4E>(csum);
            s_rec[(ok && (u & 3) == 0) ? (u >> 2) : KC] = make_int2(csum, __builtin_bit_cast(int, q.d));
        }
    }
}

// Flash-decode combine staged by the whole block (K = heads * 128): thread
// t < K/8 owns elements 8t..8t+7 of head t/16, so a head is one 16-lane DPP
// row.  The kernel body is instantiated for LS = 4, 8 or 16 loaded splits
// and picks the smallest that covers the splits holding positions (from the
// control block), so every load is unconditional.  stage_issue_attn requests
// the head's (max, denominator) pairs and the thread's 8 partial values of
// splits s < LS; stage_finish_attn merges them (flash_split_weights /
// flash_combine: the stand-alone combine kernel's arithmetic; splits without
// positions have denominator 0 and contribute nothing) and quantizes with the
// attention epilogue's Q8_1 (rint, one group per head).
constexpr int attn_splits(int XM) { return XM == kXATTN4 ? 4 : (XM == kXATTN8 ? 8 : 16); }
constexpr bool is_attn(int XM) { return XM >= kXATTN4; }

template <int LS>
__device__ __forceinline__ void stage_issue_attn(const GemvParams& p, float4 (&po)[LS][2], float4 (&pl)[LS / 2]) {
    const int u = min(static_cast<int>(threadIdx.x), (p.K >> 3) - 1);
    const int h = u >> 4, d0 = 8 * (u & 15);
    const float* lse = p.part_lse + static_cast<size_t>(h) * kFlashSplits * 2;
#pragma unroll
    for (int i = 0; i < LS / 2; ++i) pl[i] = *reinterpret_cast<const float4*>(lse + 4 * i);
    const float* o = p.part_o + static_cast<size_t>(h) * kFlashSplits * 128 + d0;
#pragma unroll
    for (int s = 0; s < LS; ++s) {
        po[s][0] = *reinterpret_cast<const float4*>(o + s * 128);
        po[s][1] = *reinterpret_cast<const float4*>(o + s * 128 + 4);
    }
}

template <int LS>
__device__ __forceinline__ void stage_finish_attn(const GemvParams& p, const float4 (&po)[LS][2],
                                                  const float4 (&pl)[LS / 2], int8_t* s_q8, int2* s_rec) {
    const int U = p.K >> 3, KC = p.K >> 5;
    const int u = threadIdx.x;
    const bool ok = u < U;
    float ms[kFlashSplits], ds[kFlashSplits], wt[kFlashSplits];
#pragma unroll
    for (int s = 0; s < kFlashSplits; ++s) {
        ms[s] = -INFINITY;
        ds[s] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < LS / 2; ++i) {
        ms[2 * i] = pl[i].x;
        ds[2 * i] = pl[i].y;
        ms[2 * i + 1] = pl[i].z;
        ds[2 * i + 1] = pl[i].w;
    }
    flash_split_weights(ms, ds, wt);
    float acc[8];
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float os[kFlashSplits];
#pragma unroll
        for (int s = 0; s < kFlashSplits; ++s) {
            if (s < LS) {
                const float4 v = po[s][e >> 2];
                os[s] = (e & 3) == 0 ? v.x : ((e & 3) == 1 ? v.y : ((e & 3) == 2 ? v.z : v.w));
            } else {
                os[s] = 0.0f;
            }
        }
        acc[e] = flash_combine(ds, wt, os);
        mx = fmaxf(mx, fabsf(acc[e]));
    }
    if (p.norm_out != nullptr && blockIdx.x == 0 && ok) {
        uint32_t hw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
            hw[j] = static_cast<uint32_t>(f2h(acc[2 * j])) | (static_cast<uint32_t>(f2h(acc[2 * j + 1])) << 16);
        *reinterpret_cast<uint4*>(p.norm_out + 8 * u) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    }
    const float d = flash_q8_scale(qwen::seg_max_nonneg<16>(mx));  // mx: fmaxf from +0, never NaN
    uint32_t b[8];
    int qsum = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int v = flash_q8_value(acc[e], d);
        qsum += v;
        b[e] = static_cast<uint32_t>(v) & 0xFFu;
    }
    int8_t* dq = ok ? s_q8 + 8 * u : reinterpret_cast<int8_t*>(s_rec + KC);
    *reinterpret_cast<int2*>(dq) = make_int2(static_cast<int>(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24)),
                                             static_cast<int>(b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)));
    int csum = -8 * qsum;  // chunk = the 4 units of a DPP quad
    csum += qwen::dpp_i32<0xB1>(csum);
    csum += qwen::dpp_i32<0x4E>(csum);
    s_rec[(ok && (u & 3) == 0) ? (u >> 2) : KC] = make_int2(csum, __builtin_bit_cast(int, d));
}

// QKV with RoPE: set s of block group g = s / 16 covers head g / 8; its
// segments 2t and 2t + 1 (t < 8) take rows j*8 + t and 64 + j*8 + t
// (j = g % 8) of that head — a rotation pair sits in neighbouring 16-lane
// segments of one wave and meets through a 32-lane swizzle
__device__ __forceinline__ int rope_row(int set) {
    const int g = set >> 4, s = set & 15;
    const int i = (g & 7) * 8 + (s >> 1);
    return (g >> 3) * 128 + ((s & 1) ? 64 + i : i);
}

template <int BT, int LPR, int NCH, int RPS, int MODE, int XM, bool LOOP>
__device__ __forceinline__ void gemv_w4_body(const GemvParams& p) {
    // SwiGLU: a segment owns a (gate, up) row pair (RPS 2), or, with 16-lane
    // segments and RPS 1, segments 2s and 2s+1 own the gate and up row and
    // meet through a 32-lane swizzle
    constexpr bool PAIR = MODE == kSwiglu && RPS == 1;
    static_assert(MODE != kSwiglu || RPS == 2 || LPR == 16, "SwiGLU row pairing");
    constexpr int SEGS = BT / LPR;
    const int K = p.K;
    const int KC = K >> 5;
    const int seg = threadIdx.x / LPR;
    const int l = threadIdx.x % LPR;
    const int n_sets = (p.n_rows + RPS - 1) / RPS;
    const int set_stride = SEGS * gridDim.x;

    // ---- activation loads first (a few KB, needed first), then the first
    //      row set's weights; the activation math overlaps the weight stream.
    //      Every load is unconditional (indices clamped), so the wait for the
    //      activation does not also wait for the weights.
    constexpr int MAXP = (LPR * NCH * 4 + BT - 1) / BT;  // K <= 32*LPR*NCH: 8-element units per thread
    constexpr int MQ = (LPR * NCH + BT - 1) / BT;        // 32-element chunks per thread (Q8_1 staging)
    int4 xa[NCH], xb[NCH];
    int32_t xsum[NCH];
    float xd[NCH];
    constexpr bool XF16 = XM == kXF16 || XM == kXRMS;
    uint4 raw[XF16 ? MAXP : 1], graw[XF16 ? MAXP : 1];
    u32x4 qa[XM == kXQ8 ? MQ : 1], qb[XM == kXQ8 ? MQ : 1];
    int4 qs4[XM == kXQ8 ? MQ : 1];
    float qxd[XM == kXQ8 ? MQ : 1];
    constexpr int LS = attn_splits(XM);
    float4 apo[is_attn(XM) ? LS : 1][2], apl[is_attn(XM) ? LS / 2 : 1];
    if constexpr (XM == kXQ8) stage_issue_q8<BT, MQ>(p, qa, qb, qs4, qxd);
    else if constexpr (is_attn(XM)) stage_issue_attn<LS>(p, apo, apl);
    else stage_issue_f16<XM, BT, MAXP>(p, raw, graw);
    constexpr bool ROPE_EPI = MODE == kQKV && LPR == 16 && RPS == 1 && BT == 256 && !LOOP;
    QkvArgs qka{};
    if constexpr (MODE == kQKV) qka = load_qkv_args(p);
    uint16_t rope_bias = 0;  // fp16 bits of this lane's row bias (QKV with RoPE)
    int rope_pos = 0;        // the position (clamped later)
    if constexpr (ROPE_EPI) {
        // requested here, ahead of the weights (first used after the GEMV)
        if (p.rope) {
            const int row = rope_row(min(blockIdx.x * SEGS + seg, n_sets - 1));
            const int u = __builtin_amdgcn_readfirstlane(row & ~127);
            const int m = (u >= qka.rb1) + (u >= qka.rb2);
            const int local = row - (m == 0 ? 0 : (m == 1 ? qka.rb1 : qka.rb2));
            const g_u16p b = pick3(qka.bias, m);
            rope_bias = b != nullptr ? b[local] : 0;
            typedef const int __attribute__((address_space(1)))* g_i32p;
            rope_pos = p.ctl != nullptr ? *(g_i32p)&p.ctl->seq_pos : 0;
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads

    int set = blockIdx.x * SEGS + seg;
    u32x4 w[RPS][NCH];
    uint32_t hs[RPS][NCH];  // fp16 scale bits, one per VGPR (no packing, so no early wait)
    auto load_set = [&](int st, u32x4 (&wr)[RPS][NCH], uint32_t (&hr)[RPS][NCH]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RPS; ++r) {
            int row = min(st * RPS + r, p.n_rows - 1);  // clamped: tail rows are loaded, not stored
            int urow = min((st - seg) * RPS, p.n_rows - 1);
            if (MODE == kQKV && p.rope) {  // segments s and s + 8 hold the rotation pair (i, i + 64) of a head
                row = rope_row(min(st, n_sets - 1));
                urow = row & ~127;
            }
            const u32x4* wp;
            const uint16_t* sp;
            int m, local;
            if constexpr (MODE == kQKV) row_ptrs_qkv(qka, p.K, row, urow, wp, sp, m, local);
            else row_ptrs<MODE>(p, row, urow, wp, sp, m, local);
#pragma unroll
            for (int i = 0; i < NCH; ++i) {
                const int c = min(l + i * LPR, KC - 1);
                wr[r][i] = __builtin_nontemporal_load(wp + c);
                hr[r][i] = sp[c >> 2];
            }
        }
    };
    load_set(min(set, n_sets - 1), w, hs);
    __builtin_amdgcn_sched_barrier(0);
    // QKV with RoPE: position and angle of this lane's row, while the loads
    // are in flight (the bias was requested with the activation, ahead of the
    // weights, so using it does not wait for them)
    float rope_sn = 0.0f, rope_cs = 1.0f;
    if constexpr (ROPE_EPI) {
        if (p.rope) {
            rope_pos = rope_pos < p.max_seq ? rope_pos : p.max_seq - 1;
            rope_sincos(rope_pos, rope_row(min(set, n_sets - 1)) & 63, 128, p.rope_theta, rope_sn, rope_cs);
        }
    }

    // ---- activation slice in VGPRs, through LDS ----------------------------------
    {
        extern __shared__ __align__(16) uint8_t s_mem[];
        int8_t* s_q8 = reinterpret_cast<int8_t*>(s_mem);
        int2* s_rec = reinterpret_cast<int2*>(s_mem + K);
        if constexpr (XM == kXQ8) stage_finish_q8<BT, MQ>(p, qa, qb, qs4, qxd, s_q8, s_rec);
        else if constexpr (is_attn(XM)) stage_finish_attn<LS>(p, apo, apl, s_q8, s_rec);
        else stage_finish_f16<XM, BT, MAXP>(p, raw, graw, s_q8, s_rec,
                                            reinterpret_cast<float*>(s_mem + K + (K >> 5) * 8 + 32));
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = l + i * LPR;
            const int cc = min(c, KC - 1);
            xa[i] = *reinterpret_cast<const int4*>(s_q8 + cc * 32);
            xb[i] = *reinterpret_cast<const int4*>(s_q8 + cc * 32 + 16);
            const int2 rec = s_rec[cc];
            xsum[i] = rec.x;
            xd[i] = __builtin_bit_cast(float, rec.y);
            if (c >= KC) {
                xa[i] = xb[i] = make_int4(0, 0, 0, 0);
                xsum[i] = 0;
                xd[i] = 0.0f;
            }
        }
    }

    // ---- row sets: one pass, or a grid-stride loop with the next set prefetched
    float temp = 0.0f;
    uint64_t seed = 0;
    uint32_t seq_pos = 0;
    if constexpr (MODE == kSample) {
        if (p.ctl != nullptr) {
            temp = p.ctl->temperature;
            seed = p.ctl->rng_seed;
            seq_pos = static_cast<uint32_t>(p.ctl->seq_pos);
        }
    }
    Best best{-1e30f, 0};
    auto finish_set = [&](int st) __attribute__((always_inline)) {
        float acc[RPS];
#pragma unroll
        for (int r = 0; r < RPS; ++r) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < NCH; ++i)
                a += static_cast<float>(chunk_dot(w[r][i], xa[i], xb[i], xsum[i])) *
                     (h2f(static_cast<uint16_t>(hs[r][i])) * xd[i]);
            acc[r] = qwen::seg_sum<LPR>(a);
        }
        if constexpr (PAIR) acc[0] = silu_mul(acc[0], qwen::swz_xor16_f32(acc[0]));  // gate (even set) x up
        if constexpr (ROPE_EPI) {
            if (p.rope) {  // block-uniform: one pass over 16-row groups of one head
                const int row = rope_row(st);
                const int u = __builtin_amdgcn_readfirstlane(row & ~127);
                const int m = (u >= qka.rb1) + (u >= qka.rb2);
                const int local = row - (m == 0 ? 0 : (m == 1 ? qka.rb1 : qka.rb2));
                // GEMV output rounded to fp16, then the bias (loaded at entry) added in fp16,
                // as the separate kernels do
                const bool has_bias = pick3(qka.bias, m) != nullptr;
                _Float16 v = static_cast<_Float16>(acc[0]);
                if (has_bias) v = v + __builtin_bit_cast(_Float16, rope_bias);
                const float y = qwen::swz_xor16_f32(static_cast<float>(v));  // the partner row (segment s ^ 1)
                if (l == 0) {
                    const int pos = rope_pos;
                    const int e = local & 127, head = local >> 7;
                    uint16_t outv = __builtin_bit_cast(uint16_t, v);
                    if (m < 2)  // q and k rows rotate with their partner
                        outv = f2h(rope_rotate(static_cast<float>(v), y, e < 64, rope_sn, rope_cs));
                    pick3(qka.out, m)[local] = outv;
                    if (m > 0) {
                        uint16_t* cache = m == 1 ? p.kcache : p.vcache;
                        cache[(static_cast<size_t>(head) * p.max_seq + pos) * 128 + e] = outv;
                    }
                }
                return;
            }
        }
        if (l == 0 && st < n_sets) {
            if constexpr (MODE == kSample) {
                const uint16_t logit = f2h(acc[0]);
                if (p.out[0] != nullptr) p.out[0][st] = logit;
                const float v = sample_value(h2f(logit), temp, seed, static_cast<uint32_t>(st), seq_pos);
                best = better(best, Best{v, st});
            } else if constexpr (PAIR) {
                if ((st & 1) == 0) p.out[0][st >> 1] = f2h(acc[0]);
            } else if constexpr (MODE == kSwiglu) {
                p.out[0][st] = f2h(silu_mul(acc[0], acc[1]));
            } else {
#pragma unroll
                for (int r = 0; r < RPS; ++r) {
                    const int row = st * RPS + r;
                    if (row < p.n_rows) {
                        const u32x4* wp;
                        const uint16_t* sp;
                        int m, local;
                        if constexpr (MODE == kQKV) row_ptrs_qkv(qka, p.K, row, (st - seg) * RPS, wp, sp, m, local);
                        else row_ptrs<MODE>(p, row, (st - seg) * RPS, wp, sp, m, local);
                        float v = acc[r];
                        if (MODE == kPlain && p.residual != nullptr) v += h2f(p.residual[local]);
                        uint16_t* o = p.out[0];
                        if constexpr (MODE == kQKV) o = (uint16_t*)pick3(qka.out, m);
                        o[local] = f2h(v);
                    }
                }
            }
        }
    };
    if constexpr (!LOOP) {
        finish_set(set);  // the grid covers every set once
    } else {
        for (; set < n_sets; set += set_stride) {
            u32x4 wn[RPS][NCH];
            uint32_t hn[RPS][NCH];
            load_set(min(set + set_stride, n_sets - 1), wn, hn);
            finish_set(set);
#pragma unroll
            for (int r = 0; r < RPS; ++r)
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    w[r][i] = wn[r][i];
                    hs[r][i] = hn[r][i];
                }
        }
    }
    if constexpr (MODE == kSample) {  // segment leaders -> one partial per block
        __shared__ float s_bv[SEGS];
        __shared__ int32_t s_bi[SEGS];
        if (l == 0) {
            s_bv[seg] = best.v;
            s_bi[seg] = best.i;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            Best b{s_bv[0], s_bi[0]};
            for (int g = 1; g < SEGS; ++g) b = better(b, Best{s_bv[g], s_bi[g]});
            p.s_val[blockIdx.x] = b.v;
            p.s_idx[blockIdx.x] = b.i;
        }
    }
}

// The kernels read the parameter block in place (the kernel-argument
// segment, scalar loads): binding the by-value parameter to a reference would
// make the compiler copy it to private memory.
__device__ __forceinline__ const GemvParams& kernel_params() {
    return *(const GemvParams*)__builtin_amdgcn_kernarg_segment_ptr();  // C cast: drops the address space
}

template <int BT, int LPR, int NCH, int RPS, int MODE, int XM, bool LOOP>
__global__ __launch_bounds__(BT) void gemv_w4_kernel(GemvParams) {
    gemv_w4_body<BT, LPR, NCH, RPS, MODE, XM, LOOP>(kernel_params());
}

// O projection with the flash-decode combine in its staging: the number of
// splits to read follows from the control block's position (block-uniform),
// one straight-line body per count.  256 threads, 16 rows per block.
template <int NCH>
__global__ __launch_bounds__(256) void gemv_attn_o_kernel(GemvParams) {
    const GemvParams& p = kernel_params();
    const int live = p.ctl != nullptr ? flash_live_splits(min(p.ctl->seq_pos + 1, p.max_seq)) : kFlashSplits;
    if (live <= 4) gemv_w4_body<256, 16, NCH, 1, kPlain, kXATTN4, false>(p);
    else if (live <= 8) gemv_w4_body<256, 16, NCH, 1, kPlain, kXATTN8, false>(p);
    else gemv_w4_body<256, 16, NCH, 1, kPlain, kXATTN16, false>(p);
}

// Generic kernel: one wave per output (row or SwiGLU pair), dword weight
// loads, scalar staging.  Covers any K % 128 == 0 up to the LDS limit and any
// 4-byte weight alignment (the reference's uint32 fallback,
// src/kernels/gemv_w4a16.cu:264-630).
template <int MODE, int XM>
__global__ __launch_bounds__(256) void gemv_w4_generic_kernel(GemvParams p) {
    extern __shared__ __align__(16) uint8_t s_mem[];
    const int K = p.K;
    const int KW = K >> 3;
    int8_t* s_q8 = reinterpret_cast<int8_t*>(s_mem);
    int2* s_rec = reinterpret_cast<int2*>(s_mem + K);
    stage_activation<XM, 256, false>(p, s_q8, s_rec, reinterpret_cast<float*>(s_mem + K + (K >> 5) * 8));
    __syncthreads();
    const int wave = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int32_t* xq = reinterpret_cast<const int32_t*>(s_q8);
    const int n_out = (MODE == kSwiglu) ? p.n_rows / 2 : p.n_rows;
    for (int o = blockIdx.x * 4 + wave; o < n_out; o += 4 * gridDim.x) {
        constexpr int NR = (MODE == kSwiglu) ? 2 : 1;
        float acc[NR];
        int m = 0, local = o;
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int row = (MODE == kSwiglu) ? 2 * o + k : o;
            const u32x4* wv;
            const uint16_t* sp;
            row_ptrs<MODE>(p, row, row, wv, sp, m, local);
            const uint32_t* wr = reinterpret_cast<const uint32_t*>(wv);
            float a = 0.0f;
            // word wd covers elements 8wd..8wd+7: chunk wd/4, group wd/16.  The
            // chunk's pre-summed sum8 seeds the first word of the chunk only.
            for (int wd = l; wd < KW; wd += 64) {
                const int2 rec = s_rec[wd >> 2];
                const int32_t seed = (wd & 3) == 0 ? rec.x : 0;
                const int32_t d = qwen::dp4a_w4_q8_oct(wr[wd], xq[2 * wd], xq[2 * wd + 1], seed);
                a += static_cast<float>(d) * (h2f(sp[wd >> 4]) * __builtin_bit_cast(float, rec.y));
            }
            acc[k] = qwen::seg_sum<64>(a);
        }
        if (l == 0) {
            if constexpr (MODE == kSwiglu) {
                p.out[0][o] = f2h(silu_mul(acc[0], acc[NR - 1]));
            } else {
                float v = acc[0];
                if (MODE == kPlain && p.residual != nullptr) v += h2f(p.residual[local]);
                p.out[m][local] = f2h(v);
            }
        }
    }
}

constexpr int kMaxFastK = 64 * 8 * 32;   // LPR 64 x 8 chunks x 32 elements
constexpr int kMaxGenericK = 32768;      // LDS: K + K/4 bytes

struct Plan {
    int bt, lpr, nch, rps;
};

Plan plan_for(int K, int n_rows, int mode, bool f16_input) {
    const int KC = K / 32;
    Plan pl{};
    if (KC <= 16 * 6) {
        pl.lpr = 16;
        const int n = (KC + 15) / 16;
        pl.nch = n <= 2 ? 2 : (n <= 3 ? 3 : 6);
    } else {
        pl.lpr = 64;
        const int n = (KC + 63) / 64;
        pl.nch = n <= 3 ? 3 : (n <= 5 ? 5 : 8);
    }
    // one row per segment (SwiGLU with 16-lane segments pairs neighbouring
    // segments); 64-lane SwiGLU segments own a row pair
    pl.rps = (mode == kSwiglu && pl.lpr == 64) ? 2 : 1;
    (void)n_rows;
    // fp16 input over long rows (K = 8960): 512-thread blocks halve the
    // per-thread share of the in-block quantization, which is on the
    // critical path; 256 everywhere else (measured on MI355X)
    pl.bt = (f16_input && pl.lpr == 64) ? 512 : 256;
    if (const int f = gemv_forced_bt()) pl.bt = f;
    return pl;
}

template <int MODE, int XM, int BT, int LPR, int NCH, int RPS>
int launch_fast(const GemvParams& p, hipStream_t s) {
    constexpr int SEGS = BT / LPR;
    const int sets = (p.n_rows + RPS - 1) / RPS;
    int grid = (sets + SEGS - 1) / SEGS;
    int cap = cu_count() * 8 * 256 / BT;
    // fp16 input: every block quantizes (and RMS-normalizes) the whole
    // activation, so fewer, looping blocks win once the grid exceeds three per
    // CU (measured: RMSNorm+gate/up 1536 -> 2x8960 5.6 -> 4.9 us)
    if constexpr (XM == kXF16 || XM == kXRMS) cap = std::min(cap, 3 * cu_count());
    if (const int f = gemv_forced_cap()) cap = f;
    if (MODE == kSample && cap > QE_LM_HEAD_SAMPLE_PARTS) cap = QE_LM_HEAD_SAMPLE_PARTS;
    // q8, chunk records + dummy slot, and (RMSNorm) the unit sums of squares
    const size_t lds = static_cast<size_t>(p.K) + (p.K >> 5) * 8 + 32 + (XM == kXRMS ? (p.K >> 3) * 4 : 0);
    if (grid > cap) {
        gemv_w4_kernel<BT, LPR, NCH, RPS, MODE, XM, true><<<cap, BT, lds, s>>>(p);
        return cap;
    }
    gemv_w4_kernel<BT, LPR, NCH, RPS, MODE, XM, false><<<grid, BT, lds, s>>>(p);
    return grid;
}

template <int MODE, int XM, int BT, int RPS>
int dispatch_chunks(const Plan& pl, const GemvParams& p, hipStream_t s) {
    if (pl.lpr == 16) {
        switch (pl.nch) {
            case 2: return launch_fast<MODE, XM, BT, 16, 2, RPS>(p, s);
            case 3: return launch_fast<MODE, XM, BT, 16, 3, RPS>(p, s);
            case 6: return launch_fast<MODE, XM, BT, 16, 6, RPS>(p, s);
        }
    } else if constexpr (!(MODE == kSwiglu && RPS == 1)) {
        switch (pl.nch) {
            case 3: return launch_fast<MODE, XM, BT, 64, 3, RPS>(p, s);
            case 5: return launch_fast<MODE, XM, BT, 64, 5, RPS>(p, s);
            case 8: return launch_fast<MODE, XM, BT, 64, 8, RPS>(p, s);
        }
    }
    return 0;
}

template <int MODE, int XM, int BT>
int dispatch_rps(const Plan& pl, const GemvParams& p, hipStream_t s) {
    if (pl.rps == 2) {
        if constexpr (MODE == kSwiglu) return dispatch_chunks<MODE, XM, BT, 2>(pl, p, s);
        return 0;
    }
    return dispatch_chunks<MODE, XM, BT, 1>(pl, p, s);
}

template <int MODE, int XM>
int dispatch_fast(const Plan& pl, const GemvParams& p, hipStream_t s) {  // grid size, 0 if none
    switch (pl.bt) {
        case 512: return dispatch_rps<MODE, XM, 512>(pl, p, s);
        case 1024: return dispatch_rps<MODE, XM, 1024>(pl, p, s);
        default: return dispatch_rps<MODE, XM, 256>(pl, p, s);
    }
}

template <int MODE, int XM>
int launch_gemv(GemvParams& p, bool fast_ok, hipStream_t stream, const char* what) {
    const int K = p.K;
    if (p.n_rows <= 0) return QE_OK;
    if (fast_ok && K <= kMaxFastK) {
        const Plan pl = plan_for(K, p.n_rows, MODE, XM != kXQ8);
        bool qkv_ok = true;
        if (MODE == kQKV) {  // matrix boundaries on whole blocks (row_ptrs)
            const int rows_per_block = pl.bt / pl.lpr * pl.rps;
            qkv_ok = (p.row_begin[1] % rows_per_block == 0) && (p.row_begin[2] % rows_per_block == 0);
        }
        if (qkv_ok) {
            if (!dispatch_fast<MODE, XM>(pl, p, stream))
                return fail(QE_ERR_UNSUPPORTED, "%s: no kernel for K=%d", what, K);
            return check_launch(what);
        }
    }
    if (K > kMaxGenericK) return fail(QE_ERR_UNSUPPORTED, "%s: in_features=%d exceeds %d", what, K, kMaxGenericK);
    const int n_out = (MODE == kSwiglu) ? p.n_rows / 2 : p.n_rows;
    int grid = (n_out + 3) / 4;
    if (grid > cu_count() * 8) grid = cu_count() * 8;
    const size_t lds = static_cast<size_t>(K) + (K >> 5) * 8 + (XM == kXRMS ? (K >> 3) * 4 : 0);
    gemv_w4_generic_kernel<MODE, XM><<<grid, 256, lds, stream>>>(p);
    return check_launch(what);
}

int check_k(const char* what, int K) {
    QE_REQUIRE(K > 0 && K % 128 == 0, "%s: in_features=%d must be a positive multiple of 128", what, K);
    return QE_OK;
}

bool act_fast_ok(const GemvParams& p) {
    if (p.x16)
        return aligned(p.x16, 16) && (p.gamma == nullptr || aligned(p.gamma, 16)) &&
               (p.norm_out == nullptr || aligned(p.norm_out, 16));
    return aligned(p.q8, 16) && aligned(p.s8, 16);
}

int fill_qkv(GemvParams& p, const qe_qkv_view* view, int num_q_heads, int num_kv_heads, int head_dim, bool& fast,
             const char* what) {
    QE_REQUIRE(view != nullptr, "%s: view is NULL", what);
    QE_REQUIRE(num_q_heads >= 0 && num_kv_heads >= 0 && head_dim >= 0, "%s: negative head shape", what);
    const int q_dim = num_q_heads * head_dim;
    const int kv_dim = num_kv_heads * head_dim;
    const void* w[3] = {view->q_weight, view->k_weight, view->v_weight};
    const uint16_t* s[3] = {view->q_scale, view->k_scale, view->v_scale};
    uint16_t* o[3] = {view->d_q, view->d_k, view->d_v};
    const int rows[3] = {q_dim, kv_dim, kv_dim};
    fast = true;
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
    p.n_rows = q_dim + 2 * kv_dim;
    return QE_OK;
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_launch_gemv_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                                   const float* input_scale, const int32_t* input_sum8, const uint16_t* residual,
                                   uint16_t* output_y, int out_features, int in_features, hipStream_t stream) {
    const char* what = "gemv_w4a8";
    if (int rc = check_k(what, in_features)) return rc;
    QE_REQUIRE(input_q8 && input_scale && input_sum8, "%s: Q8_1 input pointers must not be NULL", what);
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
    p.n_rows = out_features;
    p.K = in_features;
    return launch_gemv<kPlain, kXQ8>(p, aligned(qweight, 16) && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_gemv_qkv_w4a8(const qe_qkv_view* view, const int8_t* input_q8, const float* input_scale,
                                       const int32_t* input_sum8, hipStream_t stream, int in_features,
                                       int num_q_heads, int num_kv_heads, int head_dim) {
    const char* what = "gemv_qkv_w4a8";
    if (int rc = check_k(what, in_features)) return rc;
    QE_REQUIRE(input_q8 && input_scale && input_sum8, "%s: Q8_1 input pointers must not be NULL", what);
    GemvParams p{};
    bool fast = true;
    if (int rc = fill_qkv(p, view, num_q_heads, num_kv_heads, head_dim, fast, what)) return rc;
    p.q8 = input_q8;
    p.xs = input_scale;
    p.s8 = input_sum8;
    p.K = in_features;
    return launch_gemv<kQKV, kXQ8>(p, fast && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_gemv_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                                       const int8_t* input_q8, const float* input_scale,
                                                       const int32_t* input_sum8, uint16_t* output_mlp,
                                                       int hidden_size, int intermediate_size, hipStream_t stream) {
    const char* what = "gemv_dual_gate_up_swiglu_w4a8";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input_q8 && input_scale && input_sum8, "%s: Q8_1 input pointers must not be NULL", what);
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
    p.n_rows = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemv<kSwiglu, kXQ8>(p, aligned(gate_up_qweight, 16) && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                                    const uint16_t* residual, uint16_t* output_y, int out_features, int in_features,
                                    hipStream_t stream) {
    const char* what = "gemv_w4a16";
    if (int rc = check_k(what, in_features)) return rc;
    QE_REQUIRE(input_x && qweight && scales && output_y, "%s: NULL pointer", what);
    QE_REQUIRE(out_features >= 0, "%s: out_features=%d", what, out_features);
    QE_REQUIRE(aligned(qweight, 4) && aligned(scales, 2) && aligned(input_x, 2), "%s: misaligned buffer", what);
    GemvParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = output_y;
    p.residual = residual;
    p.x16 = input_x;
    p.n_rows = out_features;
    p.K = in_features;
    return launch_gemv<kPlain, kXF16>(p, aligned(qweight, 16) && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_gemv_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight,
                                                        const uint16_t* gate_up_scales, const uint16_t* input_x,
                                                        uint16_t* output_mlp, int hidden_size, int intermediate_size,
                                                        hipStream_t stream) {
    const char* what = "gemv_dual_gate_up_swiglu_w4a16";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input_x && gate_up_qweight && gate_up_scales && output_mlp, "%s: NULL pointer", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(gate_up_qweight, 4) && aligned(gate_up_scales, 2) && aligned(input_x, 2),
               "%s: misaligned buffer", what);
    GemvParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.x16 = input_x;
    p.n_rows = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemv<kSwiglu, kXF16>(p, aligned(gate_up_qweight, 16) && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_rmsnorm_gemv_qkv_w4a16(const uint16_t* input, const uint16_t* gamma,
                                                uint16_t* output_fp16_opt, const qe_qkv_view* view,
                                                hipStream_t stream, int hidden_size, int num_q_heads,
                                                int num_kv_heads, int head_dim) {
    const char* what = "rmsnorm_gemv_qkv_w4a16";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input && gamma, "%s: input/gamma is NULL", what);
    QE_REQUIRE(aligned(input, 2) && aligned(gamma, 2) && aligned(output_fp16_opt, 2), "%s: misaligned buffer", what);
    GemvParams p{};
    bool fast = true;
    if (int rc = fill_qkv(p, view, num_q_heads, num_kv_heads, head_dim, fast, what)) return rc;
    p.x16 = input;
    p.gamma = gamma;
    p.norm_out = output_fp16_opt;
    p.K = hidden_size;
    return launch_gemv<kQKV, kXRMS>(p, fast && act_fast_ok(p), stream, what);
}

extern "C" int qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(const uint16_t* input, const uint16_t* gamma,
                                                                uint16_t* output_fp16_opt,
                                                                const uint32_t* gate_up_qweight,
                                                                const uint16_t* gate_up_scales, uint16_t* output_mlp,
                                                                int hidden_size, int intermediate_size,
                                                                hipStream_t stream) {
    const char* what = "rmsnorm_gemv_dual_gate_up_swiglu_w4a16";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input && gamma && gate_up_qweight && gate_up_scales && output_mlp, "%s: NULL pointer", what);
    QE_REQUIRE(intermediate_size >= 0, "%s: intermediate_size=%d", what, intermediate_size);
    QE_REQUIRE(aligned(gate_up_qweight, 4) && aligned(gate_up_scales, 2) && aligned(input, 2) && aligned(gamma, 2) &&
                   aligned(output_fp16_opt, 2),
               "%s: misaligned buffer", what);
    GemvParams p{};
    p.qw[0] = gate_up_qweight;
    p.sc[0] = gate_up_scales;
    p.out[0] = output_mlp;
    p.x16 = input;
    p.gamma = gamma;
    p.norm_out = output_fp16_opt;
    p.n_rows = 2 * intermediate_size;
    p.K = hidden_size;
    return launch_gemv<kSwiglu, kXRMS>(p, aligned(gate_up_qweight, 16) && act_fast_ok(p), stream, what);
}

// ---- flash-decode combine folded into the O projection ------------------------------
namespace qe {
namespace {
constexpr int kMaxAttnK = 2048;  // one 8-element unit per thread of a 256-thread block

int launch_attn_o(const GemvParams& p, hipStream_t s) {
    const int KC = p.K / 32;
    const int grid = (p.n_rows + 15) / 16;
    const size_t lds = static_cast<size_t>(p.K) + KC * 8 + 32;
    if (KC <= 32) gemv_attn_o_kernel<2><<<grid, 256, lds, s>>>(p);
    else if (KC <= 48) gemv_attn_o_kernel<3><<<grid, 256, lds, s>>>(p);
    else gemv_attn_o_kernel<6><<<grid, 256, lds, s>>>(p);
    return grid;
}
}  // namespace
}  // namespace qe

extern "C" int qe_launch_attention_combine_gemv_o_w4a8(const float* splitk_partial_out,
                                                       const float* splitk_partial_lse, const uint32_t* o_qweight,
                                                       const uint16_t* o_scales, const uint16_t* residual,
                                                       uint16_t* output_y, uint16_t* attn_out_opt,
                                                       const qe_device_control_block* d_control, int out_features,
                                                       int num_q_heads, int head_dim, int max_seq_len,
                                                       hipStream_t stream) {
    const char* what = "attention_combine_gemv_o_w4a8";
    QE_REQUIRE(splitk_partial_out && splitk_partial_lse && o_qweight && o_scales && output_y, "%s: NULL pointer",
               what);
    QE_REQUIRE(head_dim == 128, "%s: head_dim=%d (only 128 is built)", what, head_dim);
    const int K = num_q_heads * head_dim;
    QE_REQUIRE(num_q_heads > 0 && K <= kMaxAttnK, "%s: %d q heads (at most %d)", what, num_q_heads,
               kMaxAttnK / 128);
    QE_REQUIRE(out_features > 0, "%s: out_features=%d", what, out_features);
    QE_REQUIRE(max_seq_len > 0, "%s: max_seq_len=%d", what, max_seq_len);
    QE_REQUIRE(aligned(splitk_partial_out, 16) && aligned(splitk_partial_lse, 16) && aligned(o_qweight, 16) &&
                   aligned(o_scales, 2) && aligned(residual, 2) && aligned(output_y, 2) && aligned(attn_out_opt, 16),
               "%s: misaligned buffer (partials, weights and attn_out 16-byte aligned)", what);
    GemvParams p{};
    p.qw[0] = o_qweight;
    p.sc[0] = o_scales;
    p.out[0] = output_y;
    p.residual = residual;
    p.part_o = splitk_partial_out;
    p.part_lse = splitk_partial_lse;
    p.norm_out = attn_out_opt;
    p.ctl = d_control;
    p.max_seq = max_seq_len;
    p.n_rows = out_features;
    p.K = K;
    if (!launch_attn_o(p, stream)) return fail(QE_ERR_UNSUPPORTED, "%s: no kernel for K=%d", what, K);
    return check_launch(what);
}


// ---- fused LM head + sampling ------------------------------------------------------
namespace qe {
int launch_sample_stage2(const float* val, const int32_t* idx, int nparts, qe_device_control_block* d_control,
                         int32_t* d_pinned, hipStream_t stream);
namespace {
template <int XM>
int launch_lm_head_sample(GemvParams& p, float* scratch_val, int32_t* scratch_idx, qe_device_control_block* d_control,
                          int32_t* d_pinned, hipStream_t stream, const char* what) {
    QE_REQUIRE(scratch_val && scratch_idx, "%s: sample scratch is NULL", what);
    QE_REQUIRE(p.K <= kMaxFastK, "%s: in_features=%d exceeds %d", what, p.K, kMaxFastK);
    QE_REQUIRE(aligned(p.qw[0], 16) && act_fast_ok(p), "%s: weights and activations must be 16-byte aligned", what);
    if (p.n_rows <= 0) return fail(QE_ERR_INVALID_ARGUMENT, "%s: vocab_size=%d", what, p.n_rows);
    p.s_val = scratch_val;
    p.s_idx = scratch_idx;
    p.ctl = d_control;
    const Plan pl = plan_for(p.K, p.n_rows, kPlain, XM != kXQ8);
    const int parts = dispatch_fast<kSample, XM>(pl, p, stream);
    if (parts <= 0) return fail(QE_ERR_UNSUPPORTED, "%s: no kernel for K=%d", what, p.K);
    if (parts > QE_LM_HEAD_SAMPLE_PARTS) return fail(QE_ERR_UNSUPPORTED, "%s: %d partials", what, parts);
    launch_sample_stage2(scratch_val, scratch_idx, parts, d_control, d_pinned, stream);
    return check_launch(what);
}
}  // namespace
}  // namespace qe

extern "C" int qe_launch_gemv_lm_head_sample_w4a8(const uint32_t* qweight, const uint16_t* scales,
                                                  const int8_t* input_q8, const float* input_scale,
                                                  const int32_t* input_sum8, uint16_t* logits_opt,
                                                  float* sample_scratch_val, int32_t* sample_scratch_idx,
                                                  qe_device_control_block* d_control, int32_t* d_mapped_pinned_token,
                                                  int vocab_size, int in_features, hipStream_t stream) {
    const char* what = "gemv_lm_head_sample_w4a8";
    if (int rc = check_k(what, in_features)) return rc;
    QE_REQUIRE(input_q8 && input_scale && input_sum8 && qweight && scales, "%s: NULL pointer", what);
    GemvParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = logits_opt;
    p.q8 = input_q8;
    p.xs = input_scale;
    p.s8 = input_sum8;
    p.n_rows = vocab_size;
    p.K = in_features;
    return launch_lm_head_sample<kXQ8>(p, sample_scratch_val, sample_scratch_idx, d_control, d_mapped_pinned_token,
                                       stream, what);
}

extern "C" int qe_launch_rmsnorm_gemv_lm_head_sample_w4a16(const uint16_t* input, const uint16_t* gamma,
                                                           uint16_t* output_fp16_opt, const uint32_t* qweight,
                                                           const uint16_t* scales, uint16_t* logits_opt,
                                                           float* sample_scratch_val, int32_t* sample_scratch_idx,
                                                           qe_device_control_block* d_control,
                                                           int32_t* d_mapped_pinned_token, int vocab_size,
                                                           int hidden_size, hipStream_t stream) {
    const char* what = "rmsnorm_gemv_lm_head_sample_w4a16";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input && gamma && qweight && scales, "%s: NULL pointer", what);
    GemvParams p{};
    p.qw[0] = qweight;
    p.sc[0] = scales;
    p.out[0] = logits_opt;
    p.x16 = input;
    p.gamma = gamma;
    p.norm_out = output_fp16_opt;
    p.n_rows = vocab_size;
    p.K = hidden_size;
    return launch_lm_head_sample<kXRMS>(p, sample_scratch_val, sample_scratch_idx, d_control, d_mapped_pinned_token,
                                        stream, what);
}

extern "C" int qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(
    const uint16_t* input, const uint16_t* gamma, uint16_t* output_fp16_opt, const qe_qkv_view* view,
    const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias, uint16_t* layer_k_cache,
    uint16_t* layer_v_cache, const qe_device_control_block* d_control, hipStream_t stream, int hidden_size,
    int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len, int rotary_dim, float rope_theta) {
    const char* what = "rmsnorm_gemv_qkv_rope_kv_append_w4a16";
    if (int rc = check_k(what, hidden_size)) return rc;
    QE_REQUIRE(input && gamma && layer_k_cache && layer_v_cache, "%s: NULL pointer", what);
    QE_REQUIRE(head_dim == 128 && (rotary_dim == 0 || rotary_dim == 128) && max_seq_len > 0,
               "%s: head_dim %d / rotary_dim %d (built for 128 / full rotation)", what, head_dim, rotary_dim);
    QE_REQUIRE(hidden_size <= 3072, "%s: hidden_size %d above 3072", what, hidden_size);
    GemvParams p{};
    bool fast = true;
    if (int rc = fill_qkv(p, view, num_q_heads, num_kv_heads, head_dim, fast, what)) return rc;
    p.x16 = input;
    p.gamma = gamma;
    p.norm_out = output_fp16_opt;
    p.K = hidden_size;
    QE_REQUIRE(fast && act_fast_ok(p) && aligned(output_fp16_opt, 16), "%s: buffers must be 16-byte aligned", what);
    p.rope = 1;
    p.bias[0] = q_bias;
    p.bias[1] = k_bias;
    p.bias[2] = v_bias;
    p.kcache = layer_k_cache;
    p.vcache = layer_v_cache;
    p.ctl = d_control;
    p.max_seq = max_seq_len;
    p.rope_theta = rope_theta;
    const Plan pl = plan_for(p.K, p.n_rows, kQKV, true);
    QE_REQUIRE(pl.lpr == 16 && pl.bt == 256 && pl.rps == 1 && (p.n_rows + 15) / 16 <= cu_count() * 8,
               "%s: shape outside the single-pass kernel", what);
    if (dispatch_fast<kQKV, kXRMS>(pl, p, stream) <= 0) return fail(QE_ERR_UNSUPPORTED, "%s: no kernel", what);
    return check_launch(what);
}
