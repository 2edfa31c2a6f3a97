// Decode-loop kernels around the matrix path (gfx950): W4 embedding lookup,
// QKV bias + NeoX RoPE + KV-cache append, split-K flash-decode attention with
// the fused Q8_1 epilogue that feeds the O projection, and causal prefill
// attention.
//
// Reference behaviour: src/kernels/rmsnorm_rope.cu:15-51 (embedding),
// :320-423 (bias/RoPE/KV), src/kernels/attention_gqa.cu:20-311 (flash decode,
// stage-2 Q8_1 epilogue :263-310), :322-462 (prefill).  Layouts: KV cache
// [kv_head][max_seq][head_dim] fp16 per layer; q [T][q_dim], k/v [T][kv_dim].
// Head dim 128: one wave64 covers a head with 2 elements per lane, dot
// products reduce with DPP/swizzle (seg_sum<64>).
#include "attn_common.hpp"
#include "rope_common.hpp"

namespace qe {
namespace {

constexpr int kSplits = kFlashSplits;
constexpr int kHeadDim = 128;
constexpr int kVocab = 151936;  // VOCAB_SIZE: out-of-range token ids map to 0


// ---- embedding ---------------------------------------------------------------
__global__ __launch_bounds__(256) void embed_lookup_w4a16_kernel(const uint32_t* __restrict__ qw,
                                                                 const uint16_t* __restrict__ sc,
                                                                 const int32_t* __restrict__ ids,
                                                                 uint16_t* __restrict__ out,
                                                                 const qe_device_control_block* ctl, int H) {
    const int t = blockIdx.x;
    int32_t tok = 0;
    if (ids != nullptr) tok = ids[t];
    else if (ctl != nullptr) tok = ctl->token_id;
    if (tok < 0 || tok >= kVocab) tok = 0;
    const uint32_t* row = qw + static_cast<size_t>(tok) * (H / 8);
    const uint16_t* srow = sc + static_cast<size_t>(tok) * (H / 128);
    for (int i = threadIdx.x; i < H / 8; i += blockDim.x) {
        const qwen::qe_half8_t h = qwen::unpack_w4_to_half8(row[i], __builtin_bit_cast(_Float16, srow[i >> 4]));
        *reinterpret_cast<qwen::qe_half8_t*>(out + static_cast<size_t>(t) * H + i * 8) = h;
    }
}

// ---- QKV bias + NeoX RoPE + KV append ------------------------------------------
// grid (tokens, ceil((nq + nkv) / 2)), 256 threads: thread (hl, e) owns
// element e of head 2*blockIdx.y + hl of the combined [q heads, k heads]
// list; threads of a k head also own element e of the matching v head.
// Every operand is loaded once up front, one barrier separates the reads
// of the rotation partner from the in-place writes.
__global__ __launch_bounds__(256) void qkv_bias_rope_kv_append_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, uint16_t* __restrict__ v, const uint16_t* __restrict__ qb,
    const uint16_t* __restrict__ kb, const uint16_t* __restrict__ vb, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const qe_device_control_block* ctl, int nq, int nkv, int hd, int max_seq,
    int rotary_dim, float rope_theta) {
    const int m = blockIdx.x;
    int pos = ctl != nullptr ? ctl->seq_pos + m : 0;
    if (pos >= max_seq) pos = max_seq - 1;
    const int per_block = blockDim.x / hd;  // heads per block (hd <= 256)
    const int hl = threadIdx.x / hd, e = threadIdx.x % hd;
    const int head = blockIdx.y * per_block + hl;
    const bool live = hl < per_block && head < nq + nkv;
    const bool is_k = head >= nq;
    const int q_dim = nq * hd, kv_dim = nkv * hd;
    const int rot = (rotary_dim > 0 && rotary_dim <= hd) ? rotary_dim : hd;
    const int half_rot = rot / 2;
    const int pe = e < rot ? (e < half_rot ? e + half_rot : e - half_rot) : e;  // rotation partner
    _Float16* hp = nullptr;
    const uint16_t* bp = nullptr;
    if (live) {
        hp = is_k ? reinterpret_cast<_Float16*>(k + static_cast<size_t>(m) * kv_dim + (head - nq) * hd)
                  : reinterpret_cast<_Float16*>(q + static_cast<size_t>(m) * q_dim + head * hd);
        bp = is_k ? (kb ? kb + (head - nq) * hd : nullptr) : (qb ? qb + head * hd : nullptr);
    }
    _Float16 xe = 0, xp = 0, ve = 0;
    if (live) {
        xe = hp[e];
        xp = hp[pe];
        if (bp) {  // bias added in fp16 (rounded) before the rotation
            xe = xe + __builtin_bit_cast(_Float16, bp[e]);
            xp = xp + __builtin_bit_cast(_Float16, bp[pe]);
        }
        if (is_k) {
            const size_t vo = static_cast<size_t>(m) * kv_dim + (head - nq) * hd + e;
            ve = __builtin_bit_cast(_Float16, v[vo]);
            if (vb) ve = ve + __builtin_bit_cast(_Float16, vb[(head - nq) * hd + e]);
        }
    }
    float outv = static_cast<float>(xe);
    if (e < rot) {
        float sn, cs;
        rope_sincos(pos, e < half_rot ? e : e - half_rot, rot, rope_theta, sn, cs);
        outv = rope_rotate(static_cast<float>(xe), static_cast<float>(xp), e < half_rot, sn, cs);
    }
    __syncthreads();  // partners read before anyone writes
    if (!live) return;
    const _Float16 o = static_cast<_Float16>(outv);
    hp[e] = o;
    if (is_k) {
        const size_t co = (static_cast<size_t>(head - nq) * max_seq + pos) * hd + e;
        kc[co] = __builtin_bit_cast(uint16_t, o);
        v[static_cast<size_t>(m) * kv_dim + (head - nq) * hd + e] = __builtin_bit_cast(uint16_t, ve);
        vc[co] = __builtin_bit_cast(uint16_t, ve);
    }
}

// ---- flash decode, stage 1 -----------------------------------------------------
// grid (num_q_heads, kSplits), NT = 512 threads, one q head per block (GH = 1:
// the group's blocks each re-read the kv head's K and V rows, from L2 after
// the first, and every block merges one head's lane-group states; measured
// against half a GQA group per block: 2.85 vs 3.83 us at 128 positions, 4.27
// vs 6.52 us at 3000, the same bits per head).  A split is a contiguous run of
// flash_split_len(seq_len) positions (the reference's ceil(seq_len / 16), at
// least kFlashMinSplit).  The NT/16 lane groups of the block (16 lanes each)
// each take one position per step; lane j of a group holds dims 8j..8j+7 (one
// 16-byte K and V load per position), so a score is a v_dot2 chain plus a
// 16-lane DPP sum.  A round is 64 positions whose K and V rows are requested
// together; with more than one round the next round's rows are requested
// before the current one is used.  Softmax state per lane group in the exp2
// domain, rescaled once per round.  The lane-group states are merged through
// LDS (max, weights, weighted sum).
// Output per (q head, split): unnormalized o relative to the split max m, and
// (m, denominator) with m in natural-log units, as attention_gqa.cu's stage 1
// writes them.

constexpr int kFlashThreads = 512;  // stage-1 block: one q head, 32 lane groups

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int GH>
struct FlashState {
    float m[GH], l[GH], o[GH][8];
};

// One round: step st < kSteps at positions r0 + NG*st + gid (NG lane groups).
template <int GH, int NG>
__device__ __forceinline__ void flash_round(FlashState<GH>& S, const u32x4 (&qraw)[GH], const u32x4 (&kr)[64 / NG],
                                            const u32x4 (&vr)[64 / NG], int r0, int t1, int gid) {
    constexpr int kSteps = 64 / NG;
    constexpr float kScale = 1.4426950408889634f * 0.08838834764831845f;  // log2(e) / sqrt(128)
    const int steps = min(kSteps, (t1 - r0 + NG - 1) / NG);
    float sc[GH][kSteps];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const bool valid = st < steps && r0 + st * NG + gid < t1;
#pragma unroll
        for (int h = 0; h < GH; ++h) {
            float d = 0.0f;
            if (st < steps) {  // block-uniform
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // copy the vector element first: a bit_cast straight from an
                    // element of an ext_vector always read element 0 (clang 22)
                    const uint32_t qw = qraw[h][i], kw = kr[st][i];
                    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, qw), __builtin_bit_cast(f16x2, kw), d, false);
                }
                d = qwen::seg_sum<16>(d) * kScale;
            }
            sc[h][st] = valid ? d : -INFINITY;
        }
    }
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        float mn = S.m[h];
#pragma unroll
        for (int st = 0; st < kSteps; ++st) mn = fmaxf(mn, sc[h][st]);
        // no valid position yet: keep everything at zero
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(S.m[h] - mn);
        float l = S.l[h] * alpha;
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = S.o[h][i] * alpha;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            if (st < steps) {
                const float p = sc[h][st] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[h][st] - mn);
                l += p;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // rows past the context may hold anything: never multiplied in
                    const uint32_t vw = sc[h][st] == -INFINITY ? 0u : static_cast<uint32_t>(vr[st][i]);
                    const f16x2 v2 = __builtin_bit_cast(f16x2, vw);
                    o[2 * i] += p * static_cast<float>(v2.x);
                    o[2 * i + 1] += p * static_cast<float>(v2.y);
                }
            }
        }
        S.m[h] = mn;
        S.l[h] = l;
#pragma unroll
        for (int i = 0; i < 8; ++i) S.o[h][i] = o[i];
    }
}

// One block: GH q heads (qh0..qh0+GH-1) of kv head kvh over positions [t0, t1)
// with NT threads (NT/16 lane groups).
template <int GH, int NT>
__device__ __forceinline__ void flash_decode_split(const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                                   float* __restrict__ part_o, float* __restrict__ part_lse,
                                                   const u32x4 (&qraw)[GH], u32x4 (&ka)[64 / (NT / 16)],
                                                   u32x4 (&va)[64 / (NT / 16)], int kvh, int qh0, int split, int t0,
                                                   int t1, int max_seq) {
    constexpr int NG = NT / 16, kSteps = 64 / NG;
    const int gid = threadIdx.x >> 4, j = threadIdx.x & 15;  // lane group of the block, lane in the group
    const size_t base = static_cast<size_t>(kvh) * max_seq * kHeadDim + 8 * j;
    // every load is unconditional (positions clamped to the split)
    auto load_round = [&](int r0, u32x4 (&kr)[kSteps], u32x4 (&vr)[kSteps]) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const int t = min(r0 + st * NG + gid, t1 - 1);
            kr[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kc + base + static_cast<size_t>(t) * kHeadDim));
            vr[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vc + base + static_cast<size_t>(t) * kHeadDim));
        }
    };
    FlashState<GH> S;
#pragma unroll
    for (int h = 0; h < GH; ++h) {
        S.m[h] = -INFINITY;
        S.l[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) S.o[h][i] = 0.0f;
    }
    if (t1 - t0 <= 64) {  // one round (every split of a context up to 16 * 64 positions)
        flash_round<GH, NG>(S, qraw, ka, va, t0, t1, gid);
    } else {  // ping-pong: the next round's rows are in flight while this one is used
        u32x4 kb[kSteps], vb[kSteps];
        for (int r0 = t0;;) {
            load_round(min(r0 + 64, t1 - 1), kb, vb);
            __builtin_amdgcn_sched_barrier(0);
            flash_round<GH, NG>(S, qraw, ka, va, r0, t1, gid);
            r0 += 64;
            if (r0 >= t1) break;
            load_round(min(r0 + 64, t1 - 1), ka, va);
            __builtin_amdgcn_sched_barrier(0);
            flash_round<GH, NG>(S, qraw, kb, vb, r0, t1, gid);
            r0 += 64;
            if (r0 >= t1) break;
        }
    }
    // merge the NG lane-group states through LDS, HP heads per pass (48 KB):
    // M = max_g m_g, w_g = exp2(m_g - M), L = sum_g l_g w_g, o = sum_g w_g o_g
    constexpr int HP = (GH * NG <= 96) ? GH : 96 / NG;
    __shared__ __align__(16) float s_o[NG][HP][kHeadDim];
    __shared__ float s_m[NG][HP], s_l[NG][HP], s_w[HP][NG];
    constexpr float kLn2 = 0.6931471805599453f;
#pragma unroll
    for (int h0 = 0; h0 < GH; h0 += HP) {
        if (h0 > 0) __syncthreads();  // the previous pass has read s_o
#pragma unroll
        for (int hh = 0; hh < HP; ++hh) {
            if (h0 + hh < GH) {
                float4* dst = reinterpret_cast<float4*>(&s_o[gid][hh][8 * j]);
                dst[0] = make_float4(S.o[h0 + hh][0], S.o[h0 + hh][1], S.o[h0 + hh][2], S.o[h0 + hh][3]);
                dst[1] = make_float4(S.o[h0 + hh][4], S.o[h0 + hh][5], S.o[h0 + hh][6], S.o[h0 + hh][7]);
                if (j == 0) {
                    s_m[gid][hh] = S.m[h0 + hh];
                    s_l[gid][hh] = S.l[h0 + hh];
                }
            }
        }
        __syncthreads();
        const int t = threadIdx.x;
        const int nh = min(HP, GH - h0);
        if (t < nh * NG) {  // thread (head t/NG, lane group t%NG): NG consecutive lanes per head
            const int hh = t / NG, g = t % NG;
            const float m = s_m[g][hh];
            const float mx = qwen::seg_max<NG>(m);
            const float w = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mx);
            const float lt = qwen::seg_sum<NG>(s_l[g][hh] * w);
            s_w[hh][g] = w;
            if (g == 0) {
                const size_t row = static_cast<size_t>(qh0 + h0 + hh) * kSplits + split;
                part_lse[row * 2] = mx * kLn2;  // natural-log units (-inf with no positions; lt is 0 then)
                part_lse[row * 2 + 1] = lt;
            }
        }
        __syncthreads();
        // thread (head t/(32Q), dims 4*((t/Q)%32)..+3, quarter t%Q of the lane groups); the Q
        // partial sums of an output meet through a DPP quad reduction
        constexpr int Q = NT >= 128 * HP ? 4 : 1;
        if (t < nh * 32 * Q) {
            const int hh = t / (32 * Q), d = 4 * ((t / Q) & 31), qg = t % Q;
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int gi = 0; gi < NG / Q; ++gi) {
                const int g = qg * (NG / Q) + gi;
                const float w = s_w[hh][g];
                const float4 v = *reinterpret_cast<const float4*>(&s_o[g][hh][d]);
                o.x += w * v.x;
                o.y += w * v.y;
                o.z += w * v.z;
                o.w += w * v.w;
            }
            if constexpr (Q == 4) {
                o.x = qwen::seg_sum<4>(o.x);
                o.y = qwen::seg_sum<4>(o.y);
                o.z = qwen::seg_sum<4>(o.z);
                o.w = qwen::seg_sum<4>(o.w);
            }
            if (qg == 0) {
                const size_t row = static_cast<size_t>(qh0 + h0 + hh) * kSplits + split;
                *reinterpret_cast<float4*>(part_o + row * kHeadDim + d) = o;
            }
        }
    }
}

// grid (num_kv_heads * group / GH, kSplits): block x covers q heads
// GH*x .. GH*x + GH - 1 (kv head GH*x / group).
template <int GH, int NT>
__global__ __launch_bounds__(NT) void flash_decode_stage1_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ kc,
                                                                 const uint16_t* __restrict__ vc,
                                                                 float* __restrict__ part_o,
                                                                 float* __restrict__ part_lse,
                                                                 const qe_device_control_block* ctl, int group,
                                                                 int max_seq) {
    constexpr int NG = NT / 16, kSteps = 64 / NG;
    const int qh0 = blockIdx.x * GH, split = blockIdx.y;
    const int kvh = qh0 / group;
    const int gid = threadIdx.x >> 4, j = threadIdx.x & 15;
    // q and the split's first 64 rows are requested before the position is
    // known: with splits of 64 positions (contexts up to 16 * 64) the rows are
    // those of split * 64 onwards; rows past the context are masked later
    u32x4 qraw[GH];
#pragma unroll
    for (int h = 0; h < GH; ++h) qraw[h] = *reinterpret_cast<const u32x4*>(q + (qh0 + h) * kHeadDim + 8 * j);
    u32x4 ka[kSteps], va[kSteps];
    {
        const size_t base = static_cast<size_t>(kvh) * max_seq * kHeadDim + 8 * j;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const int t = min(split * kFlashMinSplit + st * NG + gid, max_seq - 1);
            ka[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kc + base + static_cast<size_t>(t) * kHeadDim));
            va[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vc + base + static_cast<size_t>(t) * kHeadDim));
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    const int seq_pos = ctl != nullptr ? ctl->seq_pos : 0;
    const int seq_len = min(seq_pos + 1, max_seq);
    const int per = flash_split_len(seq_len);
    const int t0 = split * per;
    const int t1 = min(t0 + per, seq_len);
    if (t0 >= t1) {
        if (threadIdx.x < GH) {
            const size_t li = (static_cast<size_t>(qh0 + threadIdx.x) * kSplits + split) * 2;
            part_lse[li] = -INFINITY;
            part_lse[li + 1] = 0.0f;
        }
        return;
    }
    if (per != kFlashMinSplit) {  // longer splits: the first round starts elsewhere
        const size_t base = static_cast<size_t>(kvh) * max_seq * kHeadDim + 8 * j;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            const int t = min(t0 + st * NG + gid, t1 - 1);
            ka[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kc + base + static_cast<size_t>(t) * kHeadDim));
            va[st] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vc + base + static_cast<size_t>(t) * kHeadDim));
        }
    }
    flash_decode_split<GH, NT>(kc, vc, part_o, part_lse, qraw, ka, va, kvh, qh0, split, t0, t1, max_seq);
}

// ---- flash decode, stage 2 + Q8_1 epilogue ---------------------------------------
// grid num_q_heads, 128 threads (one per element of the head).  Every
// thread loads the 16 (m, d) pairs and its 16 partials up front.
// acc = sum_s exp(m_s - m) / d * o_s; attn_out = fp16(acc).  Epilogue
// (attention_gqa.cu:263-310): d = max(max|acc|/127, 1e-8) per head (= one
// 128-group), q = clamp(rint(acc / d)), sum8 over 8 adjacent elements.
__global__ __launch_bounds__(128) void flash_decode_stage2_kernel(const float* __restrict__ part_o,
                                                                  const float* __restrict__ part_lse,
                                                                  uint16_t* __restrict__ attn_out,
                                                                  int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                                  int32_t* __restrict__ q_sum8) {
    const int qh = blockIdx.x, tid = threadIdx.x;
    float ms[kSplits], ds[kSplits], os[kSplits];
#pragma unroll
    for (int s = 0; s < kSplits; ++s) {
        const size_t row = static_cast<size_t>(qh) * kSplits + s;
        const float2 ml = *reinterpret_cast<const float2*>(part_lse + row * 2);
        ms[s] = ml.x;
        ds[s] = ml.y;
        os[s] = part_o[row * kHeadDim + tid];
    }
    float wt[kSplits];
    flash_split_weights(ms, ds, wt);
    const float acc = flash_combine(ds, wt, os);
    attn_out[static_cast<size_t>(qh) * kHeadDim + tid] = f2h(acc);
    if (q8 == nullptr) return;  // uniform across the block
    __shared__ float s_wmax[2];
    float mx = qwen::seg_max<64>(fabsf(acc));
    if ((tid & 63) == 0) s_wmax[tid >> 6] = mx;
    __syncthreads();
    const float d = flash_q8_scale(fmaxf(s_wmax[0], s_wmax[1]));
    if (tid == 0 && q_scale != nullptr) q_scale[qh] = d;
    const int v = flash_q8_value(acc, d);
    q8[static_cast<size_t>(qh) * kHeadDim + tid] = static_cast<int8_t>(v);
    int s8 = -8 * v;
    s8 += qwen::dpp_i32<0xB1>(s8);
    s8 += qwen::dpp_i32<0x4E>(s8);
    s8 += qwen::dpp_i32<0x141>(s8);  // row_half_mirror: sum over 8 lanes
    if ((tid & 7) == 0 && q_sum8 != nullptr) q_sum8[qh * (kHeadDim / 8) + (tid >> 3)] = s8;
}

// ---- causal prefill attention (matrix cores) ---------------------------------------
// grid (num_q_heads / WPB, ceil(T/32)), WPB waves: wave w is q head
// blockIdx.x*WPB + w (the WPB heads of a block share one kv head), the block's
// 32 queries are m0..m0+31 (position base + m; keys [0, base + m]).
// v_mfma_f32_32x32x16_f16 with queries as the columns:
//   S^T (32 keys x 32 queries) = K (keys x 128 dims) . Q^T — lane l holds key
//   row l%32 / query column l%32, dims 8*(l/32) + 16*kk: one 16-byte load each
//   from the K cache and from q, no LDS;
//   the result has lane l = query l%32 holding 16 keys (8*(v/4) + 4*(l/32) +
//   v%4), so a query's max and sum are 16 in-lane values plus one lane^32 swap;
//   O^T (128 dims x 32 queries) += V^T . P^T — P^T is the lane's own 16
//   probabilities (fp16, k order = the keys it holds; the k order inside an
//   MFMA is free when both operands agree) and V^T comes from an LDS tile the
//   block stores transposed as key pairs (one 32-bit word = two keys of one
//   dim; rows of 18 words: conflict-free stores and 8-byte reads).
// Online softmax in the exp2 domain (the 1/sqrt(d) scale folded into the
// exponent's fused multiply-add), fp32 accumulation; the output is O / L.
// Tiles wholly below the diagonal and inside the context skip the mask; the
// accumulator rescale is skipped when no lane's running max moved.
constexpr int kPqTile = 32;      // queries per block
constexpr int kPkTile = 32;      // keys per step
constexpr int kVtWords = 18;     // 32-bit words per LDS row of V^T (16 key pairs + 2 pad)
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int WPB>
__global__ __launch_bounds__(64 * WPB) void prefill_attention_mfma_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    uint16_t* __restrict__ out, const qe_device_control_block* ctl, int T, int nq, int group, int max_seq,
    int out_stride) {
    constexpr int NT = 64 * WPB;
    __shared__ __align__(16) uint32_t sVt[2][kHeadDim * kVtWords];
    const int qh0 = blockIdx.x * WPB, kvh = qh0 / group, m0 = blockIdx.y * kPqTile;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int qh = qh0 + wave;
    const int fr = lane & 31, h = lane >> 5;
    const int base = ctl != nullptr ? ctl->seq_pos : 0;
    const int m = m0 + fr;                       // this lane's query
    const int qpos = base + m;                    // its position
    const int last = min(m0 + kPqTile - 1, T - 1);
    const int kv_len = min(base + last + 1, max_seq);
    const int first_diag = base + m0;             // keys below this are visible to every query of the block
    const size_t hb = static_cast<size_t>(kvh) * max_seq * kHeadDim;
    constexpr float kScale = 1.4426950408889634f * 0.08838834764831845f;  // log2(e) / sqrt(128)

    // Q^T operand: 8 k-steps of 16 dims, 8 halves per lane
    u32x4 qf[8];
    {
        const uint16_t* qr = q + static_cast<size_t>(min(m, T - 1)) * (static_cast<size_t>(nq) * kHeadDim) +
                             qh * kHeadDim + 8 * h;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qf[kk] = *reinterpret_cast<const u32x4*>(qr + 16 * kk);
    }
    f32x16 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x16{};
    float mrow = -INFINITY, lrow = 0.0f;

    // K and V of a tile are requested two tiles ahead: the loop runs over
    // pairs of tiles with two register slots (an odd tile count ends with a
    // fully masked tile), so the loads of tile i + 2 are in flight while tile
    // i computes and every load is unconditional (positions clamped).
    constexpr int VC = (kPkTile / 2 * 16 + NT - 1) / NT;  // (key pair, 8 dims) chunks per thread
    auto load_k = [&](int t0, u32x4 (&kf)[8]) __attribute__((always_inline)) {
        const int kpos = min(t0 + fr, max_seq - 1);
        const uint16_t* kr = kc + hb + static_cast<size_t>(kpos) * kHeadDim + 8 * h;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) kf[kk] = *reinterpret_cast<const u32x4*>(kr + 16 * kk);
    };
    // chunk c: key pair c%16 (keys 2(c%16), +1), dims 8*(c/16)..+7
    auto load_v = [&](int t0, u32x4 (&vr)[VC][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < VC; ++i) {
            const int c = min(static_cast<int>(threadIdx.x) + NT * i, kPkTile / 2 * 16 - 1);
            const int kp = c & 15, d0 = 8 * (c >> 4);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int pos = min(t0 + 2 * kp + r, max_seq - 1);
                vr[i][r] = *reinterpret_cast<const u32x4*>(vc + hb + static_cast<size_t>(pos) * kHeadDim + d0);
            }
        }
    };
    // -> LDS as V^T key pairs: word (dim d, pair kp) = V[2kp][d] | V[2kp+1][d] << 16
    auto store_v = [&](const u32x4 (&vr)[VC][2], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < VC; ++i) {
            const int c = static_cast<int>(threadIdx.x) + NT * i;
            if (c < kPkTile / 2 * 16) {
                const int kp = c & 15, d0 = 8 * (c >> 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t a = vr[i][0][e], b = vr[i][1][e];  // dims d0+2e (low half), d0+2e+1
                    sVt[buf][(d0 + 2 * e) * kVtWords + kp] = __builtin_amdgcn_perm(b, a, 0x05040100u);
                    sVt[buf][(d0 + 2 * e + 1) * kVtWords + kp] = __builtin_amdgcn_perm(b, a, 0x07060302u);
                }
            }
        }
    };
    // one tile: S^T = K . Q^T, online softmax, O^T += V^T . P^T (V^T in sVt[buf])
    auto tile = [&](int t0, const u32x4 (&kf)[8], int buf) __attribute__((always_inline)) {
        f32x16 sacc = f32x16{};
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
            sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, kf[kk]),
                                                          __builtin_bit_cast(f16x8, qf[kk]), sacc, 0, 0, 0);
        // raw scores of this lane's 16 keys; masked ones -inf
        float sv[16];
        if (t0 + kPkTile > first_diag || t0 + kPkTile > kv_len) {  // block-uniform
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int key = t0 + 8 * (v >> 2) + 4 * h + (v & 3);
                sv[v] = (key < kv_len && key <= qpos && m < T) ? sacc[v] : -INFINITY;
            }
        } else {
#pragma unroll
            for (int v = 0; v < 16; ++v) sv[v] = sacc[v];
        }
        float mx = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sv[v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(mrow, mx * kScale);  // scaling is monotonic: max of the scaled scores
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mrow - mn);
        mrow = mn;
        const float neg = mn == -INFINITY ? 0.0f : -mn;  // masked scores give exp2(-inf) = 0
        float ps = 0.0f;
        uint32_t pw[8];
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
            const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[v], kScale, neg));
            const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[v + 1], kScale, neg));
            ps += p0 + p1;
            pw[v >> 1] = static_cast<uint32_t>(f2h(p0)) | (static_cast<uint32_t>(f2h(p1)) << 16);
        }
        lrow = lrow * alpha + ps;
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[dt][v] *= alpha;
        }
        // two 16-key halves of the tile
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const u32x4 pf = {pw[4 * ks], pw[4 * ks + 1], pw[4 * ks + 2], pw[4 * ks + 3]};
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
                const uint32_t* row = &sVt[buf][(32 * dt + fr) * kVtWords + 8 * ks + 2 * h];
                const uint2 lo = *reinterpret_cast<const uint2*>(row);      // keys 16ks + 4h .. +3
                const uint2 hi = *reinterpret_cast<const uint2*>(row + 4);  // keys 16ks + 8 + 4h .. +3
                const u32x4 vf = {lo.x, lo.y, hi.x, hi.y};
                acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, vf),
                                                                 __builtin_bit_cast(f16x8, pf), acc[dt], 0, 0, 0);
            }
        }
    };
    u32x4 k0[8], k1[8], v0[VC][2], v1[VC][2];
    load_k(0, k0);
    load_v(0, v0);
    load_k(kPkTile, k1);
    load_v(kPkTile, v1);
    store_v(v0, 0);
    __syncthreads();
    for (int t0 = 0; t0 < kv_len; t0 += 2 * kPkTile) {
        load_v(t0 + 2 * kPkTile, v0);  // sVt[0] holds tile t0; v0 is free
        tile(t0, k0, 0);
        load_k(t0 + 2 * kPkTile, k0);
        store_v(v1, 1);  // tile t0 + 32, requested one tile ago
        __syncthreads();
        load_v(t0 + 3 * kPkTile, v1);
        tile(t0 + kPkTile, k1, 1);
        load_k(t0 + 3 * kPkTile, k1);
        store_v(v0, 0);  // tile t0 + 64
        __syncthreads();
    }
    lrow += __shfl_xor(lrow, 32);
    if (m < T) {
        const float inv = lrow > 0.0f ? 1.0f / lrow : 0.0f;
        uint16_t* o = out + static_cast<size_t>(m) * out_stride + qh * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {  // dims 32dt + 8g + 4h .. +3
                const uint32_t w0 = static_cast<uint32_t>(f2h(acc[dt][4 * g] * inv)) |
                                    (static_cast<uint32_t>(f2h(acc[dt][4 * g + 1] * inv)) << 16);
                const uint32_t w1 = static_cast<uint32_t>(f2h(acc[dt][4 * g + 2] * inv)) |
                                    (static_cast<uint32_t>(f2h(acc[dt][4 * g + 3] * inv)) << 16);
                *reinterpret_cast<uint2*>(o + 32 * dt + 8 * g + 4 * h) = make_uint2(w0, w1);
            }
    }
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_launch_embed_lookup_w4a16(const uint32_t* embed_qweight, const uint16_t* embed_scales,
                                            const int32_t* d_token_ids, uint16_t* out_hidden,
                                            const qe_device_control_block* d_control, int num_tokens,
                                            hipStream_t stream, int hidden_size) {
    QE_REQUIRE(embed_qweight && embed_scales && out_hidden, "embed_lookup_w4a16: NULL pointer");
    QE_REQUIRE(hidden_size > 0 && hidden_size % 128 == 0, "embed_lookup_w4a16: hidden_size=%d", hidden_size);
    QE_REQUIRE(aligned(out_hidden, 16), "embed_lookup_w4a16: out_hidden must be 16-byte aligned");
    if (num_tokens <= 0) return QE_OK;
    embed_lookup_w4a16_kernel<<<num_tokens, 256, 0, stream>>>(embed_qweight, embed_scales, d_token_ids, out_hidden,
                                                              d_control, hidden_size);
    return check_launch("embed_lookup_w4a16");
}

extern "C" int qe_launch_qkv_bias_rope_kv_append(uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* q_bias,
                                                 const uint16_t* k_bias, const uint16_t* v_bias,
                                                 uint16_t* layer_k_cache, uint16_t* layer_v_cache,
                                                 const qe_device_control_block* d_control, int num_tokens,
                                                 hipStream_t stream, int num_q_heads, int num_kv_heads, int head_dim,
                                                 int max_seq_len, int rotary_dim, float rope_theta) {
    QE_REQUIRE(q && k && v && layer_k_cache && layer_v_cache, "qkv_bias_rope_kv_append: NULL pointer");
    QE_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && max_seq_len > 0,
               "qkv_bias_rope_kv_append: bad head shape");
    if (num_tokens <= 0) return QE_OK;
    QE_REQUIRE(head_dim <= 256, "qkv_bias_rope_kv_append: head_dim=%d > 256", head_dim);
    const int heads_per_block = 256 / head_dim;
    const dim3 grid(num_tokens, (num_q_heads + num_kv_heads + heads_per_block - 1) / heads_per_block);
    qkv_bias_rope_kv_append_kernel<<<grid, 256, 0, stream>>>(q, k, v, q_bias, k_bias, v_bias, layer_k_cache,
                                                                   layer_v_cache, d_control, num_q_heads,
                                                                   num_kv_heads, head_dim, max_seq_len,
                                                                   rotary_dim, rope_theta);
    return check_launch("qkv_bias_rope_kv_append");
}

namespace qe {
namespace {
int launch_flash_stage1(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, float* part_o, float* part_lse,
                        const qe_device_control_block* ctl, hipStream_t stream, int num_q_heads, int num_kv_heads,
                        int head_dim, int max_seq_len, const char* what) {
    QE_REQUIRE(q && kc && vc && part_o && part_lse, "%s: NULL pointer", what);
    QE_REQUIRE(head_dim == kHeadDim, "%s: head_dim=%d (only 128 is built)", what, head_dim);
    QE_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, "%s: %d q heads over %d kv heads", what,
               num_q_heads, num_kv_heads);
    const int group = num_q_heads / num_kv_heads;
    QE_REQUIRE(max_seq_len > 0, "%s: max_seq_len=%d", what, max_seq_len);
    const dim3 grid(num_q_heads, kSplits);
    flash_decode_stage1_kernel<1, kFlashThreads><<<grid, kFlashThreads, 0, stream>>>(q, kc, vc, part_o, part_lse, ctl,
                                                                                    group, max_seq_len);
    return QE_OK;
}
}  // namespace
}  // namespace qe

extern "C" int qe_launch_attention_gqa_flash_decode(const uint16_t* q, const uint16_t* layer_k_cache,
                                                    const uint16_t* layer_v_cache, float* splitk_partial_out,
                                                    float* splitk_partial_lse, uint16_t* attn_out,
                                                    const qe_device_control_block* d_control, hipStream_t stream,
                                                    int num_q_heads, int num_kv_heads, int head_dim,
                                                    int max_seq_len, int8_t* out_q8, float* out_scale,
                                                    int32_t* out_sum8) {
    QE_REQUIRE(attn_out, "attention_gqa_flash_decode: NULL pointer");
    QE_TRY(launch_flash_stage1(q, layer_k_cache, layer_v_cache, splitk_partial_out, splitk_partial_lse, d_control,
                               stream, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                               "attention_gqa_flash_decode"));
    flash_decode_stage2_kernel<<<num_q_heads, 128, 0, stream>>>(splitk_partial_out, splitk_partial_lse, attn_out,
                                                                 out_q8, out_scale, out_sum8);
    return check_launch("attention_gqa_flash_decode");
}


extern "C" int qe_launch_attention_gqa_flash_decode_partials(const uint16_t* q, const uint16_t* layer_k_cache,
                                                             const uint16_t* layer_v_cache, float* splitk_partial_out,
                                                             float* splitk_partial_lse,
                                                             const qe_device_control_block* d_control,
                                                             hipStream_t stream, int num_q_heads, int num_kv_heads,
                                                             int head_dim, int max_seq_len) {
    QE_TRY(launch_flash_stage1(q, layer_k_cache, layer_v_cache, splitk_partial_out, splitk_partial_lse, d_control,
                               stream, num_q_heads, num_kv_heads, head_dim, max_seq_len,
                               "attention_gqa_flash_decode_partials"));
    return check_launch("attention_gqa_flash_decode_partials");
}

extern "C" int qe_launch_attention_gqa_flash_decode_combine(const float* splitk_partial_out,
                                                            const float* splitk_partial_lse, uint16_t* attn_out,
                                                            hipStream_t stream, int num_q_heads, int8_t* out_q8,
                                                            float* out_scale, int32_t* out_sum8) {
    QE_REQUIRE(splitk_partial_out && splitk_partial_lse && attn_out, "flash_decode_combine: NULL pointer");
    QE_REQUIRE(num_q_heads > 0, "flash_decode_combine: num_q_heads=%d", num_q_heads);
    flash_decode_stage2_kernel<<<num_q_heads, 128, 0, stream>>>(splitk_partial_out, splitk_partial_lse, attn_out,
                                                                 out_q8, out_scale, out_sum8);
    return check_launch("flash_decode_combine");
}

extern "C" int qe_launch_attention_gqa_prefill(const uint16_t* q, const uint16_t* layer_k_cache,
                                               const uint16_t* layer_v_cache, uint16_t* attn_out,
                                               const qe_device_control_block* d_control, int num_tokens,
                                               hipStream_t stream, int num_q_heads, int num_kv_heads, int head_dim,
                                               int max_seq_len, int hidden_size) {
    QE_REQUIRE(q && layer_k_cache && layer_v_cache && attn_out, "attention_gqa_prefill: NULL pointer");
    QE_REQUIRE(head_dim == kHeadDim, "attention_gqa_prefill: head_dim=%d (only 128 is built)", head_dim);
    QE_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, "attention_gqa_prefill: bad head counts");
    QE_REQUIRE(hidden_size >= num_q_heads * head_dim, "attention_gqa_prefill: hidden_size=%d", hidden_size);
    if (num_tokens <= 0) return QE_OK;
    QE_REQUIRE(aligned(q, 16) && aligned(attn_out, 8) && hidden_size % 4 == 0,
               "attention_gqa_prefill: q must be 16-byte and attn_out 8-byte aligned");
    const int group = num_q_heads / num_kv_heads;
    // two q heads per block when the group splits evenly (one wave per SIMD,
    // group/2 blocks per kv head and query tile), else one
    const int wpb = group % 2 == 0 ? 2 : 1;
    const dim3 grid(num_q_heads / wpb, (num_tokens + kPqTile - 1) / kPqTile);
    if (wpb == 2)
        prefill_attention_mfma_kernel<2><<<grid, 128, 0, stream>>>(q, layer_k_cache, layer_v_cache, attn_out, d_control,
                                                                   num_tokens, num_q_heads, group, max_seq_len,
                                                                   hidden_size);
    else
        prefill_attention_mfma_kernel<1><<<grid, 64, 0, stream>>>(q, layer_k_cache, layer_v_cache, attn_out, d_control,
                                                                  num_tokens, num_q_heads, group, max_seq_len,
                                                                  hidden_size);
    return check_launch("attention_gqa_prefill");
}
