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

__device__ __forceinline__ float2 h2f2(uint32_t w) {
    return make_float2(h2f(static_cast<uint16_t>(w & 0xFFFFu)), h2f(static_cast<uint16_t>(w >> 16)));
}

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
// grid (num_kv_heads, kSplits), 256 threads.  A split is a contiguous run
// of at most 256 positions.  Each wave takes 4 positions per step, one per
// 16-lane group; lane j of a group holds dims 8j..8j+7 (one 16-byte K and V
// load per position), so a score is a 16-lane DPP sum.  K and V rows of
// four steps (64 positions per block) are requested before any of them is
// used.  Online softmax per lane group in the exp2 domain; the 4 groups and
// 4 waves are merged at the end.  Output per (q head, split): unnormalized
// o relative to the split max m, and (m, denominator) with m in natural-log
// units, as attention_gqa.cu's stage 1 writes them.
constexpr int kRound = 4;  // wave steps per round of loads

__device__ __forceinline__ void unpack8_f32(const u32x4 w, float (&f)[8]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = h2f(static_cast<uint16_t>(w[i] & 0xFFFFu));
        f[2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
    }
}

template <int GROUP>
__device__ __forceinline__ void flash_decode_split(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                                   const uint16_t* __restrict__ vc, float* __restrict__ part_o,
                                                   float* __restrict__ part_lse, int kvh, int split, int t0, int t1,
                                                   int max_seq) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane >> 4, j = lane & 15;
    const int qh0 = kvh * GROUP;
    constexpr float kLog2e = 1.4426950408889634f;
    const float sc2 = kLog2e / sqrtf(static_cast<float>(kHeadDim));  // scores scaled into the exp2 domain
    float qf[GROUP][8];
#pragma unroll
    for (int h = 0; h < GROUP; ++h) {
        float f[8];
        unpack8_f32(*reinterpret_cast<const u32x4*>(q + (qh0 + h) * kHeadDim + 8 * j), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[h][i] = f[i] * sc2;
    }
    float mh[GROUP], lh[GROUP], oh[GROUP][8];
#pragma unroll
    for (int h = 0; h < GROUP; ++h) {
        mh[h] = -INFINITY;
        lh[h] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) oh[h][i] = 0.0f;
    }
    const size_t base = static_cast<size_t>(kvh) * max_seq * kHeadDim + 8 * j;
    for (int r0 = t0; r0 < t1; r0 += 64) {
        u32x4 kr[kRound], vr[kRound];
#pragma unroll
        for (int st = 0; st < kRound; ++st) {
            const int t = min(r0 + st * 16 + wave * 4 + g, t1 - 1);
            kr[st] = *reinterpret_cast<const u32x4*>(kc + base + static_cast<size_t>(t) * kHeadDim);
            vr[st] = *reinterpret_cast<const u32x4*>(vc + base + static_cast<size_t>(t) * kHeadDim);
        }
        const int steps = min(kRound, (t1 - r0 + 15) / 16);  // block-uniform: skip empty steps
#pragma unroll
        for (int st = 0; st < kRound; ++st) {
            if (st >= steps) break;
            const bool valid = r0 + st * 16 + wave * 4 + g < t1;
            float kf[8], vf[8];
            unpack8_f32(kr[st], kf);
            unpack8_f32(vr[st], vf);
#pragma unroll
            for (int h = 0; h < GROUP; ++h) {
                float d = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) d += qf[h][i] * kf[i];
                const float sc = qwen::seg_sum<16>(d);
                const float mn = valid ? fmaxf(mh[h], sc) : mh[h];
                const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mh[h] - mn);
                const float p = valid ? __builtin_amdgcn_exp2f(sc - mn) : 0.0f;
                lh[h] = lh[h] * alpha + p;
#pragma unroll
                for (int i = 0; i < 8; ++i) oh[h][i] = oh[h][i] * alpha + p * vf[i];
                mh[h] = mn;
            }
        }
    }
    // merge the 4 lane groups of the wave (lanes j, j+16, j+32, j+48)
#pragma unroll
    for (int h = 0; h < GROUP; ++h) {
#pragma unroll
        for (int sh = 0; sh < 2; ++sh) {
            const float mo = sh == 0 ? qwen::swz_xor16_f32(mh[h]) : __shfl_xor(mh[h], 32);
            const float lo = sh == 0 ? qwen::swz_xor16_f32(lh[h]) : __shfl_xor(lh[h], 32);
            const float mn = fmaxf(mh[h], mo);
            const float a = mh[h] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mh[h] - mn);
            const float b = mo == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mn);
            lh[h] = lh[h] * a + lo * b;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float oo = sh == 0 ? qwen::swz_xor16_f32(oh[h][i]) : __shfl_xor(oh[h][i], 32);
                oh[h][i] = oh[h][i] * a + oo * b;
            }
            mh[h] = mn;
        }
    }
    // merge the 4 waves through LDS; wave 0 writes
    __shared__ float s_ml[4][GROUP][2];
    __shared__ float s_o[4][GROUP][kHeadDim];
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < GROUP; ++h) {
            if (lane == 0) {
                s_ml[wave][h][0] = mh[h];
                s_ml[wave][h][1] = lh[h];
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) s_o[wave][h][8 * j + i] = oh[h][i];
        }
    }
    __syncthreads();
    // thread (h, d) for h < GROUP, d < 128: 2 elements per thread over 256 threads
    constexpr float kLn2 = 0.6931471805599453f;
    for (int idx = threadIdx.x; idx < GROUP * kHeadDim; idx += 256) {
        const int h = idx / kHeadDim, d = idx % kHeadDim;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mx = fmaxf(mx, s_ml[w][h][0]);
        float lt = 0.0f, o = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float f = s_ml[w][h][0] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s_ml[w][h][0] - mx);
            lt += s_ml[w][h][1] * f;
            o += s_o[w][h][d] * f;
        }
        const size_t row = static_cast<size_t>(qh0 + h) * kSplits + split;
        part_o[row * kHeadDim + d] = o;
        if (d == 0) {
            part_lse[row * 2] = mx * kLn2;  // natural-log units
            part_lse[row * 2 + 1] = lt;
        }
    }
}

__global__ __launch_bounds__(256) void flash_decode_stage1_kernel(const uint16_t* __restrict__ q,
                                                                  const uint16_t* __restrict__ kc,
                                                                  const uint16_t* __restrict__ vc,
                                                                  float* __restrict__ part_o,
                                                                  float* __restrict__ part_lse,
                                                                  const qe_device_control_block* ctl, int nq,
                                                                  int nkv, int max_seq) {
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int group = nq / nkv;
    const int seq_pos = ctl != nullptr ? ctl->seq_pos : 0;
    const int seq_len = min(seq_pos + 1, max_seq);
    const int per = (seq_len + kSplits - 1) / kSplits;
    const int t0 = split * per;
    const int t1 = min(t0 + per, seq_len);
    if (t0 >= t1) {
        if (threadIdx.x < group) {
            const size_t li = (static_cast<size_t>(kvh * group + threadIdx.x) * kSplits + split) * 2;
            part_lse[li] = -INFINITY;
            part_lse[li + 1] = 0.0f;
        }
        return;
    }
    switch (group) {  // q heads per kv head: compile-time so every array stays in VGPRs
        case 1: flash_decode_split<1>(q, kc, vc, part_o, part_lse, kvh, split, t0, t1, max_seq); break;
        case 2: flash_decode_split<2>(q, kc, vc, part_o, part_lse, kvh, split, t0, t1, max_seq); break;
        case 4: flash_decode_split<4>(q, kc, vc, part_o, part_lse, kvh, split, t0, t1, max_seq); break;
        case 6: flash_decode_split<6>(q, kc, vc, part_o, part_lse, kvh, split, t0, t1, max_seq); break;
        case 8: flash_decode_split<8>(q, kc, vc, part_o, part_lse, kvh, split, t0, t1, max_seq); break;
        default: break;  // rejected on the host
    }
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

// ---- causal prefill attention ----------------------------------------------------
// grid (num_q_heads, ceil(T/16)), 256 threads: wave w owns query rows
// 4w..4w+3 of the 16-row tile; lane l holds dims 2l, 2l+1.  K/V tiles of 32
// positions are staged in LDS.  Query m sits at position base + m and sees
// keys [0, base + m].
__global__ __launch_bounds__(256) void prefill_attention_kernel(const uint16_t* __restrict__ q,
                                                                const uint16_t* __restrict__ kc,
                                                                const uint16_t* __restrict__ vc,
                                                                uint16_t* __restrict__ out,
                                                                const qe_device_control_block* ctl, int T, int nq,
                                                                int nkv, int max_seq, int out_stride) {
    constexpr int BR = 16, BC = 32;
    const int qh = blockIdx.x;
    const int m0 = blockIdx.y * BR;
    const int group = nq / nkv;
    const int kvh = qh / group;
    const int base = ctl != nullptr ? ctl->seq_pos : 0;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q_dim = nq * kHeadDim;
    int qpos[4];
    float2 qv[4], o[4];
    float mi[4], di[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + wave * 4 + r;
        qpos[r] = m < T ? min(base + m, max_seq - 1) : -1;
        qv[r] = m < T ? h2f2(reinterpret_cast<const uint32_t*>(q + static_cast<size_t>(m) * q_dim + qh * kHeadDim)[lane])
                      : make_float2(0, 0);
        o[r] = make_float2(0, 0);
        mi[r] = -INFINITY;
        di[r] = 0.0f;
    }
    const int last = min(m0 + BR - 1, T - 1);
    const int kv_len = min(base + last, max_seq - 1) + 1;
    __shared__ __align__(16) uint32_t sK[BC][kHeadDim / 2], sV[BC][kHeadDim / 2];
    const float scale = 1.0f / sqrtf(static_cast<float>(kHeadDim));
    const size_t hb = static_cast<size_t>(kvh) * max_seq * kHeadDim;
    for (int tb = 0; tb < kv_len; tb += BC) {
        const int len = min(BC, kv_len - tb);
        for (int i = threadIdx.x; i < len * 16; i += 256) {
            const int r = i >> 4, c = i & 15;
            const size_t src = hb + static_cast<size_t>(tb + r) * kHeadDim + c * 8;
            *reinterpret_cast<uint4*>(&sK[r][c * 4]) = *reinterpret_cast<const uint4*>(kc + src);
            *reinterpret_cast<uint4*>(&sV[r][c * 4]) = *reinterpret_cast<const uint4*>(vc + src);
        }
        __syncthreads();
        for (int j = 0; j < len; ++j) {
            const int kp = tb + j;
            const float2 kv = h2f2(sK[j][lane]);
            const float2 vv = h2f2(sV[j][lane]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (qpos[r] >= kp) {  // wave-uniform
                    const float s = qwen::seg_sum<64>(qv[r].x * kv.x + qv[r].y * kv.y) * scale;
                    const float mc = fmaxf(mi[r], s);
                    const float alpha = expf(mi[r] - mc);
                    const float beta = expf(s - mc);
                    di[r] = di[r] * alpha + beta;
                    o[r].x = o[r].x * alpha + beta * vv.x;
                    o[r].y = o[r].y * alpha + beta * vv.y;
                    mi[r] = mc;
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + wave * 4 + r;
        if (m < T) {
            const float inv = di[r] > 0.0f ? 1.0f / di[r] : 0.0f;
            const uint32_t w = static_cast<uint32_t>(f2h(o[r].x * inv)) | (static_cast<uint32_t>(f2h(o[r].y * inv)) << 16);
            reinterpret_cast<uint32_t*>(out + static_cast<size_t>(m) * out_stride + qh * kHeadDim)[lane] = w;
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
    QE_REQUIRE(group == 1 || group == 2 || group == 4 || group == 6 || group == 8,
               "%s: %d q heads per kv head (built: 1, 2, 4, 6, 8)", what, group);
    QE_REQUIRE(max_seq_len > 0, "%s: max_seq_len=%d", what, max_seq_len);
    flash_decode_stage1_kernel<<<dim3(num_kv_heads, kSplits), 256, 0, stream>>>(
        q, kc, vc, part_o, part_lse, ctl, num_q_heads, num_kv_heads, max_seq_len);
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
    prefill_attention_kernel<<<dim3(num_q_heads, (num_tokens + 15) / 16), 256, 0, stream>>>(
        q, layer_k_cache, layer_v_cache, attn_out, d_control, num_tokens, num_q_heads, num_kv_heads, max_seq_len,
        hidden_size);
    return check_launch("attention_gqa_prefill");
}
