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
#include "qe_common.hpp"

namespace qe {
namespace {

constexpr int kSplits = 16;   // FLASH_DECODE_SPLITS, include/config.cuh:29
constexpr int kHeadDim = 128;
constexpr int kMaxGroup = 8;  // q heads per kv head handled by stage 1
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
__global__ __launch_bounds__(256) void qkv_bias_rope_kv_append_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, uint16_t* __restrict__ v, const uint16_t* __restrict__ qb,
    const uint16_t* __restrict__ kb, const uint16_t* __restrict__ vb, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const qe_device_control_block* ctl, int nq, int nkv, int hd, int max_seq,
    int rotary_dim, float rope_theta) {
    const int m = blockIdx.x;
    int pos = ctl != nullptr ? ctl->seq_pos + m : 0;
    if (pos >= max_seq) pos = max_seq - 1;
    const int q_dim = nq * hd, kv_dim = nkv * hd;
    _Float16* qm = reinterpret_cast<_Float16*>(q + static_cast<size_t>(m) * q_dim);
    _Float16* km = reinterpret_cast<_Float16*>(k + static_cast<size_t>(m) * kv_dim);
    _Float16* vm = reinterpret_cast<_Float16*>(v + static_cast<size_t>(m) * kv_dim);
    // 1. bias (fp16 adds)
    for (int i = threadIdx.x; i < q_dim; i += blockDim.x)
        if (qb) qm[i] = qm[i] + __builtin_bit_cast(_Float16, qb[i]);
    for (int i = threadIdx.x; i < kv_dim; i += blockDim.x) {
        if (kb) km[i] = km[i] + __builtin_bit_cast(_Float16, kb[i]);
        if (vb) vm[i] = vm[i] + __builtin_bit_cast(_Float16, vb[i]);
    }
    __syncthreads();
    // 2. rotate pairs (i, i + rot/2) of the first rot elements of each q/k head
    const int rot = (rotary_dim > 0 && rotary_dim <= hd) ? rotary_dim : hd;
    const int half_rot = rot / 2;
    const float log2_theta = log2f(rope_theta);
    const int pairs = (nq + nkv) * half_rot;
    for (int pi = threadIdx.x; pi < pairs; pi += blockDim.x) {
        const int head = pi / half_rot;
        const int i = pi % half_rot;
        const float inv_freq = exp2f(-2.0f * static_cast<float>(i) / static_cast<float>(rot) * log2_theta);
        float sn, cs;
        sincosf(static_cast<float>(pos) * inv_freq, &sn, &cs);
        _Float16* hp = head < nq ? qm + head * hd : km + (head - nq) * hd;
        const float x0 = static_cast<float>(hp[i]);
        const float x1 = static_cast<float>(hp[i + half_rot]);
        hp[i] = static_cast<_Float16>(x0 * cs - x1 * sn);
        hp[i + half_rot] = static_cast<_Float16>(x0 * sn + x1 * cs);
    }
    __syncthreads();
    // 3. append rotated k and biased v at position pos
    for (int i = threadIdx.x; i < kv_dim; i += blockDim.x) {
        const int head = i / hd, d = i % hd;
        const size_t off = (static_cast<size_t>(head) * max_seq + pos) * hd + d;
        kc[off] = __builtin_bit_cast(uint16_t, km[i]);
        vc[off] = __builtin_bit_cast(uint16_t, vm[i]);
    }
}

// ---- flash decode, stage 1 -----------------------------------------------------
// grid (num_kv_heads, kSplits), 256 threads (4 waves).  Wave w walks tokens
// split_start + w, +4, ...; lane l holds dims 2l, 2l+1 of every q head of
// the group.  Writes unnormalized partial outputs and (max, denominator).
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
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int qh0 = kvh * group;
    if (t0 >= t1) {
        if (threadIdx.x < group) {
            const size_t li = (static_cast<size_t>(qh0 + threadIdx.x) * kSplits + split) * 2;
            part_lse[li] = -INFINITY;
            part_lse[li + 1] = 0.0f;
        }
        return;
    }
    float2 qv[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h)
        qv[h] = h < group ? h2f2(reinterpret_cast<const uint32_t*>(q + (qh0 + h) * kHeadDim)[lane]) : make_float2(0, 0);
    float mi[kMaxGroup], di[kMaxGroup];
    float2 oi[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) {
        mi[h] = -INFINITY;
        di[h] = 0.0f;
        oi[h] = make_float2(0.0f, 0.0f);
    }
    const float scale = 1.0f / sqrtf(static_cast<float>(kHeadDim));
    const size_t base = static_cast<size_t>(kvh) * max_seq * kHeadDim;
    for (int t = t0 + wave; t < t1; t += 4) {
        const float2 kv = h2f2(reinterpret_cast<const uint32_t*>(kc + base + static_cast<size_t>(t) * kHeadDim)[lane]);
        const float2 vv = h2f2(reinterpret_cast<const uint32_t*>(vc + base + static_cast<size_t>(t) * kHeadDim)[lane]);
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h) {
            if (h < group) {
                const float s = qwen::seg_sum<64>(qv[h].x * kv.x + qv[h].y * kv.y) * scale;
                const float mc = fmaxf(mi[h], s);
                const float alpha = expf(mi[h] - mc);
                const float beta = expf(s - mc);
                di[h] = di[h] * alpha + beta;
                oi[h].x = oi[h].x * alpha + beta * vv.x;
                oi[h].y = oi[h].y * alpha + beta * vv.y;
                mi[h] = mc;
            }
        }
    }
    __shared__ float s_m[kMaxGroup][4], s_d[kMaxGroup][4];
    __shared__ float2 s_o[4][kMaxGroup][64];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) {
        if (h < group) {
            if (lane == 0) {
                s_m[h][wave] = mi[h];
                s_d[h][wave] = di[h];
            }
            s_o[wave][h][lane] = oi[h];
        }
    }
    __syncthreads();
    // merge the 4 waves: thread (h, lane) for h = wave, wave + 4
    for (int h = wave; h < group; h += 4) {
        float mmax = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            if (s_d[h][w] > 0.0f) mmax = fmaxf(mmax, s_m[h][w]);
        float dt = 0.0f;
        float2 o = make_float2(0.0f, 0.0f);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (s_d[h][w] > 0.0f) {
                const float f = expf(s_m[h][w] - mmax);
                dt += s_d[h][w] * f;
                o.x += f * s_o[w][h][lane].x;
                o.y += f * s_o[w][h][lane].y;
            }
        }
        const size_t oi_ = (static_cast<size_t>(qh0 + h) * kSplits + split) * kHeadDim + 2 * lane;
        part_o[oi_] = dt > 0.0f ? o.x : 0.0f;
        part_o[oi_ + 1] = dt > 0.0f ? o.y : 0.0f;
        if (lane == 0) {
            const size_t li = (static_cast<size_t>(qh0 + h) * kSplits + split) * 2;
            part_lse[li] = mmax;
            part_lse[li + 1] = dt;
        }
    }
}

// ---- flash decode, stage 2 + Q8_1 epilogue ---------------------------------------
// grid num_q_heads, 128 threads (one per element of the head).
// acc = sum_s exp(m_s - m) / d * o_s; attn_out = fp16(acc).  Epilogue
// (attention_gqa.cu:263-310): d = max(max|acc|/127, 1e-8) per head (= one
// 128-group), q = clamp(rint(acc / d)), sum8 over 8 adjacent elements.
__global__ __launch_bounds__(128) void flash_decode_stage2_kernel(const float* __restrict__ part_o,
                                                                  const float* __restrict__ part_lse,
                                                                  uint16_t* __restrict__ attn_out,
                                                                  int8_t* __restrict__ q8, float* __restrict__ q_scale,
                                                                  int32_t* __restrict__ q_sum8) {
    const int qh = blockIdx.x, tid = threadIdx.x;
    __shared__ float s_m[kSplits], s_d[kSplits];
    __shared__ float s_mg, s_dg;
    __shared__ float s_wmax[2];
    if (tid < kSplits) {
        const size_t li = (static_cast<size_t>(qh) * kSplits + tid) * 2;
        s_m[tid] = part_lse[li];
        s_d[tid] = part_lse[li + 1];
    }
    __syncthreads();
    if (tid == 0) {
        float mg = -INFINITY;
        for (int s = 0; s < kSplits; ++s)
            if (s_d[s] > 0.0f) mg = fmaxf(mg, s_m[s]);
        float dg = 0.0f;
        for (int s = 0; s < kSplits; ++s)
            if (s_d[s] > 0.0f) dg += s_d[s] * expf(s_m[s] - mg);
        s_mg = mg;
        s_dg = dg;
    }
    __syncthreads();
    const float mg = s_mg, dg = s_dg;
    float acc = 0.0f;
    if (dg > 0.0f) {
        const float inv = 1.0f / dg;
        for (int s = 0; s < kSplits; ++s) {
            if (s_d[s] > 0.0f) {
                const float wgt = expf(s_m[s] - mg) * inv;
                acc += wgt * part_o[(static_cast<size_t>(qh) * kSplits + s) * kHeadDim + tid];
            }
        }
    }
    attn_out[static_cast<size_t>(qh) * kHeadDim + tid] = f2h(acc);
    if (q8 == nullptr) return;  // uniform across the block
    float mx = qwen::seg_max<64>(fabsf(acc));
    if ((tid & 63) == 0) s_wmax[tid >> 6] = mx;
    __syncthreads();
    const float d = fmaxf(fmaxf(s_wmax[0], s_wmax[1]) / 127.0f, 1e-8f);
    if (tid == 0 && q_scale != nullptr) q_scale[qh] = d;
    int v = static_cast<int>(rintf(acc / d));
    v = max(-127, min(127, v));
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
    qkv_bias_rope_kv_append_kernel<<<num_tokens, 256, 0, stream>>>(q, k, v, q_bias, k_bias, v_bias, layer_k_cache,
                                                                   layer_v_cache, d_control, num_q_heads,
                                                                   num_kv_heads, head_dim, max_seq_len,
                                                                   rotary_dim, rope_theta);
    return check_launch("qkv_bias_rope_kv_append");
}

extern "C" int qe_launch_attention_gqa_flash_decode(const uint16_t* q, const uint16_t* layer_k_cache,
                                                    const uint16_t* layer_v_cache, float* splitk_partial_out,
                                                    float* splitk_partial_lse, uint16_t* attn_out,
                                                    const qe_device_control_block* d_control, hipStream_t stream,
                                                    int num_q_heads, int num_kv_heads, int head_dim,
                                                    int max_seq_len, int8_t* out_q8, float* out_scale,
                                                    int32_t* out_sum8) {
    QE_REQUIRE(q && layer_k_cache && layer_v_cache && splitk_partial_out && splitk_partial_lse && attn_out,
               "attention_gqa_flash_decode: NULL pointer");
    QE_REQUIRE(head_dim == kHeadDim, "attention_gqa_flash_decode: head_dim=%d (only 128 is built)", head_dim);
    QE_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= kMaxGroup,
               "attention_gqa_flash_decode: %d q heads over %d kv heads", num_q_heads, num_kv_heads);
    QE_REQUIRE(max_seq_len > 0, "attention_gqa_flash_decode: max_seq_len=%d", max_seq_len);
    flash_decode_stage1_kernel<<<dim3(num_kv_heads, kSplits), 256, 0, stream>>>(
        q, layer_k_cache, layer_v_cache, splitk_partial_out, splitk_partial_lse, d_control, num_q_heads, num_kv_heads,
        max_seq_len);
    flash_decode_stage2_kernel<<<num_q_heads, 128, 0, stream>>>(splitk_partial_out, splitk_partial_lse, attn_out,
                                                                 out_q8, out_scale, out_sum8);
    return check_launch("attention_gqa_flash_decode");
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
