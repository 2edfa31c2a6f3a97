// Minimal decode engine over the W4A16 G128 path (gfx950): random-init
// Qwen2.5-style weights in the packed layout or a .qwenbin v2 file (loaded as
// the reference's setup_arena does: one device copy of the payload, tensors
// addressed by offset), chunked prefill on the MFMA
// dequant-GEMMs, and a decode step captured once into a HIP graph that is
// replayed per token, driven by a device control block (token id, position)
// so the graph needs no parameter updates.
//
// Reference behaviour: QwenEngine in src/engine.cu (arena layout :210-348,
// decode layer :361-403, decode pass :405-451, graph capture :453-470,
// prefill :472-590, decode_step :592-610).  The decode layer here uses this
// build's fused launches (RMSNorm+Q8_1 inside the QKV and gate/up GEMVs, the
// down GEMV quantizing its fp16 input in-launch); the reference's 7-launch
// sequence is available with fused_decode = 0.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "qe_common.hpp"
#include "qe_engine.h"
#include "qwenbin_internal.hpp"

namespace qe {
namespace {

// counter-based generator for the random weights (splitmix64 finalizer)
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i) {
    const uint64_t a = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 1));
    const uint64_t b = mix64(seed + 0x9E3779B97F4A7C15ull * (2 * i + 2));
    const float u1 = (static_cast<float>(a >> 40) + 1.0f) * (1.0f / 16777216.0f);
    const float u2 = static_cast<float>(b >> 40) * (1.0f / 16777216.0f);
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}

// words: uniform 32-bit (nibbles uniform in [0,15]); scales fp16 |N(0,1)|*scale_mul
__global__ void init_w4_kernel(uint32_t* __restrict__ w, size_t n_words, uint16_t* __restrict__ s, size_t n_scales,
                               uint64_t seed, float scale_mul) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_words; i += stride)
        w[i] = static_cast<uint32_t>(mix64(seed ^ (0xD1B54A32D192ED03ull * (i + 1))));
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_scales; i += stride)
        s[i] = f2h(fabsf(normal_at(seed ^ 0x5DEECE66Dull, i)) * scale_mul);
}

__global__ void init_f16_kernel(uint16_t* __restrict__ x, size_t n, uint64_t seed, float mean, float stdv) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        x[i] = f2h(mean + (stdv != 0.0f ? stdv * normal_at(seed, i) : 0.0f));
}

__global__ void set_position_kernel(qe_device_control_block* ctl, int seq_pos) { ctl->seq_pos = seq_pos; }

struct Mat {
    uint32_t* w = nullptr;
    uint16_t* s = nullptr;
    int rows = 0, K = 0;
};

struct Layer {
    uint16_t *ln1, *ln2, *q_bias, *k_bias, *v_bias;
    Mat q, k, v, o, gate_up, down;
    Mat tq, tk, tv, to, tgate_up, tdown;  // tiled copies for the prefill GEMMs (qe_repack_w4_tiled)
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

}  // namespace
}  // namespace qe

struct qe_engine {
    qe_engine_config cfg{};
    hipStream_t stream = nullptr;
    char* arena = nullptr;
    size_t arena_size = 0, arena_used = 0;
    std::vector<qe::Layer> layers;
    qe::Mat embed;
    qe::Mat lm;           // LM head: the embedding when tied
    void* payload = nullptr;  // weights loaded from a .qwenbin (one device copy of the file's payload)
    uint16_t* final_norm = nullptr;
    // workspace
    uint16_t *act0 = nullptr, *act1 = nullptr, *dq = nullptr, *dk = nullptr, *dv = nullptr, *attn = nullptr,
             *mlp = nullptr, *logits = nullptr;
    int8_t* q8 = nullptr;
    float* q8_scale = nullptr;
    int32_t* q8_sum8 = nullptr;
    float *part_o = nullptr, *part_lse = nullptr, *sample_val = nullptr;
    int32_t *sample_idx = nullptr, *tokens = nullptr;
    uint16_t *kcache = nullptr, *vcache = nullptr;
    qe_device_control_block* ctl = nullptr;
    int32_t* h_token = nullptr;  // mapped pinned
    int32_t* d_token = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    int seq_pos = 0;
    bool tiled = false;        // prefill GEMMs read the tiled copies
    bool want_tiled = false;   // engine_tiled_prefill, read once at create
    float* gemm_ws = nullptr;  // split-K workspace of the engine's stream (in the arena)

    std::vector<std::pair<size_t, size_t>> spans;  // (offset, bytes) of every buffer taken
    template <class T>
    T* take(size_t bytes) {
        size_t off = qe::align256(arena_used);
        arena_used = off + bytes;
        spans.emplace_back(off, bytes);
        return reinterpret_cast<T*>(arena + off);
    }
    size_t kv_stride() const { return static_cast<size_t>(cfg.num_kv_heads) * cfg.max_seq_len * cfg.head_dim; }
};

namespace qe {
namespace {

#define QE_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t e_ = (call);                                                        \
        if (e_ != hipSuccess) return fail(QE_ERR_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

size_t mat_bytes(int rows, int K) { return align256(static_cast<size_t>(rows) * K / 2) + align256(static_cast<size_t>(rows) * (K / 128) * 2); }

Mat alloc_mat(qe_engine* e, int rows, int K) {
    Mat m;
    m.rows = rows;
    m.K = K;
    m.w = e->take<uint32_t>(static_cast<size_t>(rows) * K / 2);
    m.s = e->take<uint16_t>(static_cast<size_t>(rows) * (K / 128) * 2);
    return m;
}

// Group scales |N(0,1)| * c with c = 1/sqrt(21.5 K): E[(q-8)^2] = 21.5 for
// uniform nibbles, so a projection keeps the variance of its input and the
// 28-layer residual stream stays inside fp16 (with c = 0.02 it overflows
// after a few layers).  The embedding uses c = 0.02.
int init_mat(qe_engine* e, const Mat& m, uint64_t seed, bool variance_preserving = true) {
    const float c = variance_preserving ? 1.0f / sqrtf(21.5f * static_cast<float>(m.K)) : 0.02f;
    init_w4_kernel<<<2048, 256, 0, e->stream>>>(m.w, static_cast<size_t>(m.rows) * m.K / 8, m.s,
                                                static_cast<size_t>(m.rows) * (m.K / 128), seed, c);
    QE_HIP(hipGetLastError());
    return QE_OK;
}

int init_vec(qe_engine* e, uint16_t* x, size_t n, uint64_t seed, float mean, float stdv) {
    init_f16_kernel<<<256, 256, 0, e->stream>>>(x, n, seed, mean, stdv);
    QE_HIP(hipGetLastError());
    return QE_OK;
}

qe_qkv_view view_of(const qe_engine* e, const Layer& L, uint16_t* q, uint16_t* k, uint16_t* v) {
    return qe_qkv_view{L.q.w, L.q.s, q, L.k.w, L.k.s, k, L.v.w, L.v.s, v};
}

// One decode token, all launches on e->stream.  times (optional): per-launch
// category accumulation with events, for the profile entry point.
struct Timer {
    hipEvent_t ev[2] = {nullptr, nullptr};
    float acc[3] = {0, 0, 0};  // gemv, attention, other
    bool on = false;
    int cur = 0;
};

int mark(qe_engine* e, Timer* t, int cat) {
    if (t == nullptr || !t->on) return QE_OK;
    QE_HIP(hipEventRecord(t->ev[1], e->stream));
    QE_HIP(hipEventSynchronize(t->ev[1]));
    float ms = 0.0f;
    QE_HIP(hipEventElapsedTime(&ms, t->ev[0], t->ev[1]));
    t->acc[cat] += ms;
    QE_HIP(hipEventRecord(t->ev[0], e->stream));
    return QE_OK;
}

int decode_pass(qe_engine* e, Timer* t) {
    const qe_engine_config& c = e->cfg;
    const int H = c.hidden_size, I = c.intermediate_size;
    hipStream_t s = e->stream;
    if (t && t->on) QE_HIP(hipEventRecord(t->ev[0], s));
    QE_TRY(qe_launch_embed_lookup_w4a16(e->embed.w, e->embed.s, nullptr, e->act0, e->ctl, 1, s, H));
    QE_TRY(mark(e, t, 2));
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = e->layers[l];
        uint16_t* kc = e->kcache + l * e->kv_stride();
        uint16_t* vc = e->vcache + l * e->kv_stride();
        const qe_qkv_view view = view_of(e, L, e->dq, e->dk, e->dv);
        if (c.fused_decode && H <= 3072) {  // RMSNorm + QKV + bias + RoPE + KV append in one launch
            QE_TRY(qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(e->act0, L.ln1, nullptr, &view, L.q_bias, L.k_bias,
                                                                   L.v_bias, kc, vc, e->ctl, s, H, c.num_q_heads,
                                                                   c.num_kv_heads, c.head_dim, c.max_seq_len,
                                                                   c.head_dim, c.rope_theta));
            QE_TRY(mark(e, t, 0));
        } else {
            if (c.fused_decode) {
                QE_TRY(qe_launch_rmsnorm_gemv_qkv_w4a16(e->act0, L.ln1, nullptr, &view, s, H, c.num_q_heads,
                                                        c.num_kv_heads, c.head_dim));
            } else {
                QE_TRY(qe_launch_rmsnorm_q8_1(e->act0, L.ln1, nullptr, e->q8, e->q8_scale, e->q8_sum8, s, H));
                QE_TRY(qe_launch_gemv_qkv_w4a8(&view, e->q8, e->q8_scale, e->q8_sum8, s, H, c.num_q_heads,
                                               c.num_kv_heads, c.head_dim));
            }
            QE_TRY(mark(e, t, 0));
            QE_TRY(qe_launch_qkv_bias_rope_kv_append(e->dq, e->dk, e->dv, L.q_bias, L.k_bias, L.v_bias, kc, vc, e->ctl,
                                                     1, s, c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_seq_len,
                                                     c.head_dim, c.rope_theta));
            QE_TRY(mark(e, t, 2));
        }
        if (c.fused_decode && c.num_q_heads * c.head_dim <= 2048) {  // split partials, then combine + O
            QE_TRY(qe_launch_attention_gqa_flash_decode_partials(e->dq, kc, vc, e->part_o, e->part_lse, e->ctl, s,
                                                                 c.num_q_heads, c.num_kv_heads, c.head_dim,
                                                                 c.max_seq_len));
            QE_TRY(mark(e, t, 1));
            QE_TRY(qe_launch_attention_combine_gemv_o_w4a8(e->part_o, e->part_lse, L.o.w, L.o.s, e->act0, e->act0,
                                                           nullptr, e->ctl, H, c.num_q_heads, c.head_dim,
                                                           c.max_seq_len, s));
        } else {
            QE_TRY(qe_launch_attention_gqa_flash_decode(e->dq, kc, vc, e->part_o, e->part_lse, e->attn, e->ctl, s,
                                                        c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_seq_len,
                                                        e->q8, e->q8_scale, e->q8_sum8));
            QE_TRY(mark(e, t, 1));
            QE_TRY(qe_launch_gemv_w4a8(L.o.w, L.o.s, e->q8, e->q8_scale, e->q8_sum8, e->act0, e->act0, H,
                                       c.num_q_heads * c.head_dim, s));
        }
        if (c.fused_decode) {
            QE_TRY(qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(e->act0, L.ln2, nullptr, L.gate_up.w, L.gate_up.s,
                                                                    e->mlp, H, I, s));
            QE_TRY(qe_launch_gemv_w4a16(L.down.w, L.down.s, e->mlp, e->act0, e->act0, H, I, s));
        } else {
            QE_TRY(qe_launch_rmsnorm_q8_1(e->act0, L.ln2, nullptr, e->q8, e->q8_scale, e->q8_sum8, s, H));
            QE_TRY(qe_launch_gemv_dual_gate_up_swiglu_w4a8(L.gate_up.w, L.gate_up.s, e->q8, e->q8_scale, e->q8_sum8,
                                                           e->mlp, H, I, s));
            QE_TRY(qe_launch_quantize_fp16_to_q8_1(e->mlp, e->q8, e->q8_scale, e->q8_sum8, I, s));
            QE_TRY(qe_launch_gemv_w4a8(L.down.w, L.down.s, e->q8, e->q8_scale, e->q8_sum8, e->act0, e->act0, H, I,
                                       s));
        }
        QE_TRY(mark(e, t, 0));
    }
    if (c.fused_decode) {  // final RMSNorm + tied LM head + sampling stage 1, then stage 2 + advance
        QE_TRY(qe_launch_rmsnorm_gemv_lm_head_sample_w4a16(e->act0, e->final_norm, nullptr, e->lm.w, e->lm.s,
                                                           e->logits, e->sample_val, e->sample_idx, e->ctl,
                                                           e->d_token, c.vocab_size, H, s));
        QE_TRY(mark(e, t, 0));
        return QE_OK;
    }
    QE_TRY(qe_launch_rmsnorm_q8_1(e->act0, e->final_norm, nullptr, e->q8, e->q8_scale, e->q8_sum8, s, H));
    QE_TRY(mark(e, t, 2));
    QE_TRY(qe_launch_gemv_w4a8(e->lm.w, e->lm.s, e->q8, e->q8_scale, e->q8_sum8, nullptr, e->logits,
                               c.vocab_size, H, s));
    QE_TRY(mark(e, t, 0));
    QE_TRY(qe_launch_sample_and_advance(e->logits, e->sample_val, e->sample_idx, e->ctl, e->d_token, s,
                                        c.vocab_size));
    QE_TRY(mark(e, t, 2));
    return QE_OK;
}

int prefill_chunk(qe_engine* e, int start, int len) {
    const qe_engine_config& c = e->cfg;
    const int H = c.hidden_size, I = c.intermediate_size;
    hipStream_t s = e->stream;
    set_position_kernel<<<1, 1, 0, s>>>(e->ctl, start);
    QE_HIP(hipGetLastError());
    QE_TRY(qe_launch_embed_lookup_w4a16(e->embed.w, e->embed.s, e->tokens + start, e->act0, nullptr, len, s, H));
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = e->layers[l];
        uint16_t* kc = e->kcache + l * e->kv_stride();
        uint16_t* vc = e->vcache + l * e->kv_stride();
        QE_TRY(qe_launch_rmsnorm_fp16(e->act0, L.ln1, e->act1, len, s, H));
        if (e->tiled) {
            const qe_qkv_view tv{L.tq.w, L.tq.s, e->dq, L.tk.w, L.tk.s, e->dk, L.tv.w, L.tv.s, e->dv};
            QE_TRY(qe_launch_gemm_prefill_qkv_w4a16_tiled(&tv, e->act1, len, s, H, c.num_q_heads, c.num_kv_heads,
                                                          c.head_dim));
        } else {
            const qe_qkv_view view = view_of(e, L, e->dq, e->dk, e->dv);
            QE_TRY(qe_launch_gemm_prefill_qkv_w4a16(&view, e->act1, len, s, H, c.num_q_heads, c.num_kv_heads,
                                                    c.head_dim, 0));
        }
        QE_TRY(qe_launch_qkv_bias_rope_kv_append(e->dq, e->dk, e->dv, L.q_bias, L.k_bias, L.v_bias, kc, vc, e->ctl,
                                                 len, s, c.num_q_heads, c.num_kv_heads, c.head_dim, c.max_seq_len,
                                                 c.head_dim, c.rope_theta));
        QE_TRY(qe_launch_attention_gqa_prefill(e->dq, kc, vc, e->attn, e->ctl, len, s, c.num_q_heads,
                                               c.num_kv_heads, c.head_dim, c.max_seq_len,
                                               c.num_q_heads * c.head_dim));
        const int qd = c.num_q_heads * c.head_dim;
        if (e->tiled) {
            QE_TRY(qe_launch_gemm_prefill_w4a16_tiled(L.to.w, L.to.s, e->attn, e->act0, e->act0, len, H, qd, s));
            QE_TRY(qe_launch_rmsnorm_fp16(e->act0, L.ln2, e->act1, len, s, H));
            QE_TRY(qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(L.tgate_up.w, L.tgate_up.s, e->act1, e->mlp,
                                                                          len, s, H, I));
            QE_TRY(qe_launch_gemm_prefill_w4a16_tiled(L.tdown.w, L.tdown.s, e->mlp, e->act0, e->act0, len, H, I, s));
        } else {
            QE_TRY(qe_launch_gemm_prefill_w4a16(L.o.w, L.o.s, e->attn, e->act0, e->act0, len, H, qd, s, 0));
            QE_TRY(qe_launch_rmsnorm_fp16(e->act0, L.ln2, e->act1, len, s, H));
            QE_TRY(qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16(L.gate_up.w, L.gate_up.s, e->act1, e->mlp, len,
                                                                    s, H, I));
            QE_TRY(qe_launch_gemm_prefill_w4a16(L.down.w, L.down.s, e->mlp, e->act0, e->act0, len, H, I, s, 0));
        }
    }
    return QE_OK;
}

int capture_graph(qe_engine* e) {
    QE_HIP(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal));
    const int rc = decode_pass(e, nullptr);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(e->stream, &g);
    if (rc != QE_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    QE_HIP(end);
    e->graph = g;
    QE_HIP(hipGraphInstantiate(&e->graph_exec, g, nullptr, nullptr, 0));
    return QE_OK;
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" void qe_engine_default_config(qe_engine_config* c) {
    c->num_layers = 28;
    c->hidden_size = 1536;
    c->intermediate_size = 8960;
    c->num_q_heads = 12;
    c->num_kv_heads = 2;
    c->head_dim = 128;
    c->vocab_size = 151936;
    c->max_seq_len = 4096;
    c->rope_theta = 1000000.0f;
    c->prefill_chunk = 1024;
    c->fused_decode = 1;
}

extern "C" void qe_engine_destroy(qe_engine* e) {
    if (e == nullptr) return;
    if (e->graph_exec) (void)hipGraphExecDestroy(e->graph_exec);
    if (e->graph) (void)hipGraphDestroy(e->graph);
    // the stream's workspace registration goes before the arena that holds it
    if (e->stream && e->gemm_ws) (void)qe_gemm_release_workspace(e->stream);
    if (e->h_token) (void)hipHostFree(e->h_token);
    if (e->arena) (void)hipFree(e->arena);
    if (e->payload) (void)hipFree(e->payload);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

namespace qe {
namespace {

bool config_ok(const qe_engine_config& c) {
    return c.num_layers > 0 && c.hidden_size > 0 && c.hidden_size % 128 == 0 && c.intermediate_size > 0 &&
           c.intermediate_size % 128 == 0 && c.head_dim == 128 && c.num_kv_heads > 0 &&
           c.num_q_heads % c.num_kv_heads == 0 && c.vocab_size > 0 && c.max_seq_len > 0 && c.prefill_chunk > 0 &&
           c.num_q_heads * c.head_dim == c.hidden_size;
}

size_t weight_bytes(const qe_engine_config& c) {
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim;
    const size_t per_layer = mat_bytes(qd, H) + 2 * mat_bytes(kvd, H) + mat_bytes(H, qd) + mat_bytes(2 * I, H) +
                             mat_bytes(H, I) + align256(H * 2) * 2 + align256(qd * 2) + align256(kvd * 2) * 2;
    return per_layer * c.num_layers + mat_bytes(c.vocab_size, H) + align256(H * 2);
}

// Tiled copies of the layer matrices for the prefill GEMMs: every K a
// multiple of 256 and the QKV widths multiples of 32 (0 bytes otherwise, or
// when switched off with qe_set_tuning("engine_tiled_prefill", 0)).
size_t tiled_mat_bytes(int rows, int K) {
    size_t w = 0, sb = 0;
    if (qe_w4_tiled_bytes(rows, K, &w, &sb) != QE_OK) return 0;
    return align256(w) + align256(sb);
}

bool tiled_ok(const qe_engine_config& c, bool want_tiled) {
    const int qd = c.num_q_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
    return want_tiled && c.hidden_size % 256 == 0 && c.intermediate_size % 256 == 0 && qd % 256 == 0 &&
           qd % 32 == 0 && kvd % 32 == 0;
}

size_t tiled_bytes(const qe_engine_config& c, bool want_tiled) {
    if (!tiled_ok(c, want_tiled)) return 0;
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim;
    return static_cast<size_t>(c.num_layers) *
           (tiled_mat_bytes(qd, H) + 2 * tiled_mat_bytes(kvd, H) + tiled_mat_bytes(H, qd) +
            tiled_mat_bytes(2 * I, H) + tiled_mat_bytes(H, I));
}

// Carves the tiled copies out of the arena and writes them (on the engine's
// stream, after the weights are in place).
int setup_tiled(qe_engine* e) {
    if (!tiled_ok(e->cfg, e->want_tiled)) return QE_OK;
    auto tile = [&](const Mat& m, Mat& t) -> int {
        size_t wb = 0, sb = 0;
        QE_TRY(qe_w4_tiled_bytes(m.rows, m.K, &wb, &sb));
        t.rows = m.rows;
        t.K = m.K;
        t.w = e->take<uint32_t>(wb);
        t.s = e->take<uint16_t>(sb);
        return qe_repack_w4_tiled(m.w, m.s, m.rows, m.K, t.w, t.s, e->stream);
    };
    for (Layer& L : e->layers) {
        QE_TRY(tile(L.q, L.tq));
        QE_TRY(tile(L.k, L.tk));
        QE_TRY(tile(L.v, L.tv));
        QE_TRY(tile(L.o, L.to));
        QE_TRY(tile(L.gate_up, L.tgate_up));
        QE_TRY(tile(L.down, L.tdown));
    }
    e->tiled = true;
    return QE_OK;
}

// Q8_1 scratch holds the longest quantized activation: the down input (I),
// the normalized hidden state (H) or the attention output (q_dim)
int q8_len(const qe_engine_config& c) {
    return std::max(c.intermediate_size, std::max(c.hidden_size, c.num_q_heads * c.head_dim));
}

// The engine's split-K workspace for its prefill GEMMs (registered for the
// engine's stream with qe_gemm_attach_workspace, released at destroy).
constexpr size_t kEngineGemmWsBytes = size_t(32) << 20;

size_t workspace_bytes(const qe_engine_config& c, bool want_tiled) {
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim, T = c.prefill_chunk, QN = q8_len(c);
    size_t bytes = 2 * align256(static_cast<size_t>(c.num_layers) * c.num_kv_heads * c.max_seq_len * c.head_dim * 2);
    bytes += 2 * align256(static_cast<size_t>(T) * H * 2) + align256(static_cast<size_t>(T) * qd * 2) +
             2 * align256(static_cast<size_t>(T) * kvd * 2) + align256(static_cast<size_t>(T) * qd * 2) +
             align256(static_cast<size_t>(T) * I * 2) + align256(static_cast<size_t>(c.vocab_size) * 2);
    bytes += align256(QN) + align256(QN / 128 * 4) + align256(QN / 8 * 4);
    bytes += 2 * align256(static_cast<size_t>(c.num_q_heads) * 16 * 128 * 4) +
             2 * align256(QE_LM_HEAD_SAMPLE_PARTS * 4) + align256(static_cast<size_t>(c.max_seq_len) * 4) + 256 +
             256 + 4096 + kEngineGemmWsBytes;
    return bytes + tiled_bytes(c, want_tiled);
}

int begin_engine(qe_engine* e, const qe_engine_config& c, bool want_tiled, size_t arena_bytes) {
    e->cfg = c;
    e->want_tiled = want_tiled;
    QE_HIP(hipStreamCreate(&e->stream));
    QE_HIP(hipMalloc(&e->arena, arena_bytes));
    e->arena_size = arena_bytes;
    QE_HIP(hipHostMalloc(reinterpret_cast<void**>(&e->h_token), sizeof(int32_t), hipHostMallocMapped));
    QE_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&e->d_token), e->h_token, 0));
    return QE_OK;
}

void layout_workspace(qe_engine* e) {
    const qe_engine_config& c = e->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim, T = c.prefill_chunk, QN = q8_len(c);
    const size_t kvb = static_cast<size_t>(c.num_layers) * e->kv_stride() * 2;
    e->kcache = e->take<uint16_t>(kvb);
    e->vcache = e->take<uint16_t>(kvb);
    e->act0 = e->take<uint16_t>(static_cast<size_t>(T) * H * 2);
    e->act1 = e->take<uint16_t>(static_cast<size_t>(T) * H * 2);
    e->dq = e->take<uint16_t>(static_cast<size_t>(T) * qd * 2);
    e->dk = e->take<uint16_t>(static_cast<size_t>(T) * kvd * 2);
    e->dv = e->take<uint16_t>(static_cast<size_t>(T) * kvd * 2);
    e->attn = e->take<uint16_t>(static_cast<size_t>(T) * qd * 2);
    e->mlp = e->take<uint16_t>(static_cast<size_t>(T) * I * 2);
    e->logits = e->take<uint16_t>(static_cast<size_t>(c.vocab_size) * 2);
    e->q8 = e->take<int8_t>(QN);
    e->q8_scale = e->take<float>(QN / 128 * 4);
    e->q8_sum8 = e->take<int32_t>(QN / 8 * 4);
    e->part_o = e->take<float>(static_cast<size_t>(c.num_q_heads) * 16 * 128 * 4);
    e->part_lse = e->take<float>(static_cast<size_t>(c.num_q_heads) * 16 * 2 * 4);
    e->sample_val = e->take<float>(QE_LM_HEAD_SAMPLE_PARTS * 4);
    e->sample_idx = e->take<int32_t>(QE_LM_HEAD_SAMPLE_PARTS * 4);
    e->tokens = e->take<int32_t>(static_cast<size_t>(c.max_seq_len) * 4);
    e->ctl = e->take<qe_device_control_block>(sizeof(qe_device_control_block));
    e->gemm_ws = e->take<float>(kEngineGemmWsBytes);
}

// KV cache cleared, control block at position 0, decode graph captured
int finish_engine(qe_engine* e) {
    QE_TRY(setup_tiled(e));
    QE_REQUIRE(e->arena_used <= e->arena_size, "engine_create: arena overflow (%zu > %zu)", e->arena_used,
               e->arena_size);
    QE_TRY(qe_gemm_attach_workspace(e->stream, e->gemm_ws, kEngineGemmWsBytes));
    (void)cu_count();  // cache the device fact before graph capture
    const size_t kvb = static_cast<size_t>(e->cfg.num_layers) * e->kv_stride() * 2;
    QE_HIP(hipMemsetAsync(e->kcache, 0, kvb, e->stream));
    QE_HIP(hipMemsetAsync(e->vcache, 0, kvb, e->stream));
    const qe_device_control_block init = {0, 0, 0.0f, 0, 1337ull};
    QE_HIP(hipMemcpyAsync(e->ctl, &init, sizeof(init), hipMemcpyHostToDevice, e->stream));
    QE_HIP(hipStreamSynchronize(e->stream));
    return capture_graph(e);
}

}  // namespace
}  // namespace qe

extern "C" int qe_engine_create(const qe_engine_config* cfg, uint64_t seed, qe_engine** out) {
    QE_REQUIRE(cfg && out, "engine_create: NULL argument");
    *out = nullptr;
    const qe_engine_config& c = *cfg;
    QE_REQUIRE(config_ok(c), "engine_create: unsupported configuration");
    std::unique_ptr<qe_engine, void (*)(qe_engine*)> e(new qe_engine(), qe_engine_destroy);
    const bool want_tiled = engine_tiled_prefill() != 0;
    QE_TRY(begin_engine(e.get(), c, want_tiled, weight_bytes(c) + workspace_bytes(c, want_tiled)));
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim;
    // layout first, then check, then initialize
    e->layers.resize(c.num_layers);
    for (int l = 0; l < c.num_layers; ++l) {
        Layer& L = e->layers[l];
        L.q = alloc_mat(e.get(), qd, H);
        L.k = alloc_mat(e.get(), kvd, H);
        L.v = alloc_mat(e.get(), kvd, H);
        L.o = alloc_mat(e.get(), H, qd);
        L.gate_up = alloc_mat(e.get(), 2 * I, H);
        L.down = alloc_mat(e.get(), H, I);
        L.ln1 = e->take<uint16_t>(H * 2);
        L.ln2 = e->take<uint16_t>(H * 2);
        L.q_bias = e->take<uint16_t>(qd * 2);
        L.k_bias = e->take<uint16_t>(kvd * 2);
        L.v_bias = e->take<uint16_t>(kvd * 2);
    }
    e->embed = alloc_mat(e.get(), c.vocab_size, H);
    e->lm = e->embed;
    e->final_norm = e->take<uint16_t>(H * 2);
    layout_workspace(e.get());
    QE_REQUIRE(e->arena_used <= e->arena_size, "engine_create: arena overflow (%zu > %zu)", e->arena_used,
               e->arena_size);
    uint64_t sd = seed * 0x100000001B3ull + 17;
    for (int l = 0; l < c.num_layers; ++l) {
        Layer& L = e->layers[l];
        for (Mat* m : {&L.q, &L.k, &L.v, &L.o, &L.gate_up, &L.down}) QE_TRY(init_mat(e.get(), *m, sd++));
        QE_TRY(init_vec(e.get(), L.ln1, H, sd++, 1.0f, 0.0f));
        QE_TRY(init_vec(e.get(), L.ln2, H, sd++, 1.0f, 0.0f));
        QE_TRY(init_vec(e.get(), L.q_bias, qd, sd++, 0.0f, 0.02f));
        QE_TRY(init_vec(e.get(), L.k_bias, kvd, sd++, 0.0f, 0.02f));
        QE_TRY(init_vec(e.get(), L.v_bias, kvd, sd++, 0.0f, 0.02f));
    }
    QE_TRY(init_mat(e.get(), e->embed, sd++, false));
    QE_TRY(init_vec(e.get(), e->final_norm, H, sd++, 1.0f, 0.0f));
    QE_TRY(finish_engine(e.get()));
    *out = e.release();
    clear_error();
    return QE_OK;
}

extern "C" int qe_engine_create_from_qwenbin(const char* path, int max_seq_len, int prefill_chunk, int fused_decode,
                                             qe_engine** out) {
    QE_REQUIRE(path && out, "engine_create_from_qwenbin: NULL argument");
    *out = nullptr;
    MappedFile file;
    QE_TRY(file.open(path));
    QwenbinModel m;
    QE_TRY(qwenbin_parse(file, m));
    const qe_qwenbin_info& in = m.info;
    qe_engine_config c{};
    c.num_layers = in.num_layers;
    c.hidden_size = in.hidden_size;
    c.intermediate_size = in.intermediate_size;
    c.num_q_heads = in.num_q_heads;
    c.num_kv_heads = in.num_kv_heads;
    c.head_dim = in.head_dim;
    c.vocab_size = in.vocab_size;
    c.rope_theta = in.rope_theta;
    // context window: the caller's, capped by the file's; the file's when 0
    // (src/engine.cu:128-132 caps the same way); 4096 when neither is usable
    const int file_seq = (in.max_seq_len > 0 && in.max_seq_len <= 32768) ? in.max_seq_len : 4096;
    c.max_seq_len = max_seq_len > 0 ? std::min(max_seq_len, file_seq) : file_seq;
    c.prefill_chunk = prefill_chunk > 0 ? prefill_chunk : 1024;
    c.fused_decode = fused_decode;
    QE_REQUIRE(config_ok(c), "engine_create_from_qwenbin: unsupported configuration");
    std::unique_ptr<qe_engine, void (*)(qe_engine*)> e(new qe_engine(), qe_engine_destroy);
    const bool want_tiled = engine_tiled_prefill() != 0;
    QE_TRY(begin_engine(e.get(), c, want_tiled, workspace_bytes(c, want_tiled)));
    // one device copy of the payload [weights_offset, end of file) (src/engine.cu:271-272)
    QE_HIP(hipMalloc(&e->payload, std::max<uint64_t>(in.weights_bytes, 256)));
    QE_HIP(hipMemcpy(e->payload, file.data() + in.weights_offset, in.weights_bytes, hipMemcpyHostToDevice));
    char* base = static_cast<char*>(e->payload);
    auto at = [&](uint64_t off) -> char* { return off == 0 ? nullptr : base + (off - in.weights_offset); };
    auto mat = [&](uint64_t w, uint64_t sc, int rows, int K) {
        Mat x;
        x.w = reinterpret_cast<uint32_t*>(at(w));
        x.s = reinterpret_cast<uint16_t*>(at(sc));
        x.rows = rows;
        x.K = K;
        return x;
    };
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim;
    const qe_qwenbin_header& h = m.header;
    e->embed = mat(h.embed_tokens_offset, h.reserved[0], c.vocab_size, H);
    e->lm = m.untied_lm_head ? mat(h.lm_head_offset, h.reserved[1], c.vocab_size, H) : e->embed;
    e->final_norm = reinterpret_cast<uint16_t*>(at(h.final_norm_offset));
    e->layers.resize(c.num_layers);
    for (int l = 0; l < c.num_layers; ++l) {
        const qe_qwenbin_layer& d = m.layers[l];
        Layer& L = e->layers[l];
        L.ln1 = reinterpret_cast<uint16_t*>(at(d.norm1_weight_offset));
        L.ln2 = reinterpret_cast<uint16_t*>(at(d.norm2_weight_offset));
        L.q_bias = reinterpret_cast<uint16_t*>(at(d.q_bias_offset));
        L.k_bias = reinterpret_cast<uint16_t*>(at(d.k_bias_offset));
        L.v_bias = reinterpret_cast<uint16_t*>(at(d.v_bias_offset));
        L.q = mat(d.qkv_weight_offset, d.q_scale_offset, qd, H);
        L.k = mat(d.k_weight_offset, d.k_scale_offset, kvd, H);
        L.v = mat(d.v_weight_offset, d.v_scale_offset, kvd, H);
        L.o = mat(d.attn_out_weight_offset, d.attn_out_scale_offset, H, qd);
        L.gate_up = mat(d.mlp_gate_offset, d.mlp_gate_scale_offset, 2 * I, H);
        L.down = mat(d.mlp_down_offset, d.mlp_down_scale_offset, H, I);
    }
    layout_workspace(e.get());
    QE_TRY(finish_engine(e.get()));
    *out = e.release();
    clear_error();
    return QE_OK;
}

extern "C" int qe_engine_save_qwenbin(qe_engine* e, const char* path) {
    QE_REQUIRE(e && path, "engine_save_qwenbin: NULL argument");
    QE_HIP(hipStreamSynchronize(e->stream));
    const qe_engine_config& c = e->cfg;
    const int H = c.hidden_size, I = c.intermediate_size, qd = c.num_q_heads * c.head_dim,
              kvd = c.num_kv_heads * c.head_dim;
    QwenbinWriter wr(c.num_layers);
    std::vector<uint8_t> host;
    int rc = QE_OK;
    // copy a device tensor into the container; 0 for an absent (NULL) tensor
    auto put = [&](const void* dptr, size_t bytes) -> uint64_t {
        if (dptr == nullptr || rc != QE_OK) return 0;
        host.resize(bytes);
        const hipError_t err = hipMemcpy(host.data(), dptr, bytes, hipMemcpyDeviceToHost);
        if (err != hipSuccess) {
            rc = fail(QE_ERR_HIP, "engine_save_qwenbin: %s", hipGetErrorString(err));
            return 0;
        }
        return wr.add(host.data(), bytes);
    };
    auto wbytes = [](const Mat& x) { return static_cast<size_t>(x.rows) * x.K / 2; };
    auto sbytes = [](const Mat& x) { return static_cast<size_t>(x.rows) * (x.K / 128) * 2; };
    qe_qwenbin_header& h = wr.header();
    // the exporter's order (tools/export_qwen25.py:238-362)
    h.embed_tokens_offset = put(e->embed.w, wbytes(e->embed));
    h.reserved[0] = put(e->embed.s, sbytes(e->embed));
    const bool tied = e->lm.w == e->embed.w;
    if (tied) {
        h.lm_head_offset = h.embed_tokens_offset;
    } else {
        h.lm_head_offset = put(e->lm.w, wbytes(e->lm));
        h.reserved[1] = put(e->lm.s, sbytes(e->lm));
    }
    h.final_norm_offset = put(e->final_norm, static_cast<size_t>(H) * 2);
    for (int l = 0; l < c.num_layers; ++l) {
        const Layer& L = e->layers[l];
        qe_qwenbin_layer& d = wr.layer(l);
        d.type = QE_QWENBIN_LAYER_GQA;
        d.norm1_weight_offset = put(L.ln1, static_cast<size_t>(H) * 2);
        d.qkv_weight_offset = put(L.q.w, wbytes(L.q));
        d.q_scale_offset = put(L.q.s, sbytes(L.q));
        d.k_weight_offset = put(L.k.w, wbytes(L.k));
        d.k_scale_offset = put(L.k.s, sbytes(L.k));
        d.v_weight_offset = put(L.v.w, wbytes(L.v));
        d.v_scale_offset = put(L.v.s, sbytes(L.v));
        d.q_bias_offset = put(L.q_bias, static_cast<size_t>(qd) * 2);
        d.k_bias_offset = put(L.k_bias, static_cast<size_t>(kvd) * 2);
        d.v_bias_offset = put(L.v_bias, static_cast<size_t>(kvd) * 2);
        d.attn_out_weight_offset = put(L.o.w, wbytes(L.o));
        d.attn_out_scale_offset = put(L.o.s, sbytes(L.o));
        d.norm2_weight_offset = put(L.ln2, static_cast<size_t>(H) * 2);
        d.mlp_gate_offset = d.mlp_up_offset = put(L.gate_up.w, wbytes(L.gate_up));
        d.mlp_gate_scale_offset = d.mlp_up_scale_offset = put(L.gate_up.s, sbytes(L.gate_up));
        d.mlp_down_offset = put(L.down.w, wbytes(L.down));
        d.mlp_down_scale_offset = put(L.down.s, sbytes(L.down));
        d.quant_scales_offset = d.q_scale_offset;
    }
    if (rc != QE_OK) return rc;
    h.hidden_size = static_cast<uint32_t>(H);
    h.intermediate_size = static_cast<uint32_t>(I);
    h.num_attention_heads = static_cast<uint32_t>(c.num_q_heads);
    h.num_kv_heads = static_cast<uint32_t>(c.num_kv_heads);
    h.head_dim = static_cast<uint32_t>(c.head_dim);
    h.vocab_size = static_cast<uint32_t>(c.vocab_size);
    h.max_seq_len = static_cast<uint32_t>(c.max_seq_len);
    h.tie_word_embeddings = tied ? 1u : 0u;
    h.rms_norm_eps = 1e-6f;
    h.rope_theta = c.rope_theta;
    return wr.write(path);
}

extern "C" int qe_engine_reset(qe_engine* e) {
    QE_REQUIRE(e, "engine_reset: NULL engine");
    const qe_device_control_block init = {0, 0, 0.0f, 0, 1337ull};
    QE_HIP(hipMemcpyAsync(e->ctl, &init, sizeof(init), hipMemcpyHostToDevice, e->stream));
    QE_HIP(hipStreamSynchronize(e->stream));
    e->seq_pos = 0;
    return QE_OK;
}

extern "C" int qe_engine_prefill(qe_engine* e, const int32_t* tokens, int n, int32_t* first_token) {
    QE_REQUIRE(e && tokens && n > 0, "engine_prefill: bad arguments");
    QE_REQUIRE(n < e->cfg.max_seq_len, "engine_prefill: prompt length %d exceeds the context window %d", n,
               e->cfg.max_seq_len);
    const qe_engine_config& c = e->cfg;
    for (int i = 0; i < n; ++i)
        QE_REQUIRE(tokens[i] >= 0 && tokens[i] < c.vocab_size, "engine_prefill: token %d at %d outside [0, %d)",
                   tokens[i], i, c.vocab_size);
    QE_HIP(hipMemcpyAsync(e->tokens, tokens, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, e->stream));
    for (int start = 0; start < n; start += c.prefill_chunk) {
        const int len = std::min(c.prefill_chunk, n - start);
        QE_TRY(prefill_chunk(e, start, len));
    }
    // last row -> logits -> first generated token; position = n - 1, advanced to n
    set_position_kernel<<<1, 1, 0, e->stream>>>(e->ctl, n - 1);
    QE_HIP(hipGetLastError());
    const int last = (n - 1) % c.prefill_chunk;
    QE_TRY(qe_launch_rmsnorm_q8_1(e->act0 + static_cast<size_t>(last) * c.hidden_size, e->final_norm, nullptr, e->q8,
                                  e->q8_scale, e->q8_sum8, e->stream, c.hidden_size));
    QE_TRY(qe_launch_gemv_w4a8(e->lm.w, e->lm.s, e->q8, e->q8_scale, e->q8_sum8, nullptr, e->logits,
                               c.vocab_size, c.hidden_size, e->stream));
    QE_TRY(qe_launch_sample_and_advance(e->logits, e->sample_val, e->sample_idx, e->ctl, e->d_token, e->stream,
                                        c.vocab_size));
    QE_HIP(hipStreamSynchronize(e->stream));
    e->seq_pos = n;
    if (first_token) *first_token = *e->h_token;
    return QE_OK;
}

extern "C" int qe_engine_decode(qe_engine* e, int n_steps, int use_graph, int32_t* tokens, float* step_ms) {
    QE_REQUIRE(e && n_steps >= 0, "engine_decode: bad arguments");
    QE_REQUIRE(e->seq_pos + n_steps <= e->cfg.max_seq_len, "engine_decode: context window %d exceeded",
               e->cfg.max_seq_len);
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    if (step_ms) {
        QE_HIP(hipEventCreate(&ev0));
        QE_HIP(hipEventCreate(&ev1));
    }
    int rc = QE_OK;
    for (int i = 0; i < n_steps && rc == QE_OK; ++i) {
        if (step_ms) (void)hipEventRecord(ev0, e->stream);
        if (use_graph) {
            const hipError_t ge = hipGraphLaunch(e->graph_exec, e->stream);
            if (ge != hipSuccess) rc = fail(QE_ERR_HIP, "hipGraphLaunch: %s", hipGetErrorString(ge));
        } else {
            rc = decode_pass(e, nullptr);
        }
        if (rc != QE_OK) break;
        if (step_ms) (void)hipEventRecord(ev1, e->stream);
        const hipError_t se = hipStreamSynchronize(e->stream);
        if (se != hipSuccess) {
            rc = fail(QE_ERR_HIP, "decode step: %s", hipGetErrorString(se));
            break;
        }
        if (step_ms) (void)hipEventElapsedTime(&step_ms[i], ev0, ev1);
        if (tokens) tokens[i] = *e->h_token;
        ++e->seq_pos;
    }
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    return rc;
}

extern "C" int qe_engine_profile_decode(qe_engine* e, float* stage_ms) {
    QE_REQUIRE(e && stage_ms, "engine_profile_decode: bad arguments");
    QE_REQUIRE(e->seq_pos + 1 <= e->cfg.max_seq_len, "engine_profile_decode: context window exceeded");
    Timer t;
    t.on = true;
    QE_HIP(hipEventCreate(&t.ev[0]));
    QE_HIP(hipEventCreate(&t.ev[1]));
    int rc = decode_pass(e, &t);
    if (rc == QE_OK) {
        const hipError_t se = hipStreamSynchronize(e->stream);
        if (se != hipSuccess) rc = fail(QE_ERR_HIP, "profile step: %s", hipGetErrorString(se));
    }
    (void)hipEventDestroy(t.ev[0]);
    (void)hipEventDestroy(t.ev[1]);
    if (rc != QE_OK) return rc;
    ++e->seq_pos;
    stage_ms[0] = t.acc[0];
    stage_ms[1] = t.acc[1];
    stage_ms[2] = t.acc[2];
    stage_ms[3] = t.acc[0] + t.acc[1] + t.acc[2];
    return QE_OK;
}

extern "C" int qe_engine_seq_pos(const qe_engine* e) { return e ? e->seq_pos : -1; }

extern "C" const uint16_t* qe_engine_logits(const qe_engine* e) { return e ? e->logits : nullptr; }

extern "C" const uint16_t* qe_engine_hidden(const qe_engine* e) { return e ? e->act0 : nullptr; }

extern "C" int qe_engine_read_logits(qe_engine* e, uint16_t* host, int n) {
    QE_REQUIRE(e && host && n >= 0 && n <= e->cfg.vocab_size, "engine_read_logits: bad arguments");
    QE_HIP(hipStreamSynchronize(e->stream));
    QE_HIP(hipMemcpy(host, e->logits, static_cast<size_t>(n) * 2, hipMemcpyDeviceToHost));
    return QE_OK;
}

extern "C" int qe_engine_read_hidden(qe_engine* e, uint16_t* host, int n) {
    QE_REQUIRE(e && host && n >= 0 && n <= e->cfg.hidden_size * e->cfg.prefill_chunk, "engine_read_hidden: bad arguments");
    QE_HIP(hipStreamSynchronize(e->stream));
    QE_HIP(hipMemcpy(host, e->act0, static_cast<size_t>(n) * 2, hipMemcpyDeviceToHost));
    return QE_OK;
}

extern "C" int qe_engine_arena_spans(const qe_engine* e, size_t* offsets, size_t* sizes, int capacity, int* count,
                                     size_t* arena_bytes) {
    QE_REQUIRE(e && count && capacity >= 0 && (capacity == 0 || (offsets && sizes)),
               "engine_arena_spans: bad arguments");
    const int n = static_cast<int>(e->spans.size());
    for (int i = 0; i < n && i < capacity; ++i) {
        offsets[i] = e->spans[i].first;
        sizes[i] = e->spans[i].second;
    }
    *count = n;
    if (arena_bytes) *arena_bytes = e->arena_size;
    return QE_OK;
}

extern "C" int qe_engine_read_buffer(qe_engine* e, const char* name, void* host, size_t bytes) {
    QE_REQUIRE(e && name && host, "engine_read_buffer: bad arguments");
    const qe_engine_config& c = e->cfg;
    const int qn = std::max(c.intermediate_size, std::max(c.hidden_size, c.num_q_heads * c.head_dim));
    struct Item { const char* n; const void* p; size_t size; };
    const Item items[] = {
        {"logits", e->logits, static_cast<size_t>(c.vocab_size) * 2},
        {"hidden", e->act0, static_cast<size_t>(c.prefill_chunk) * c.hidden_size * 2},
        {"q8", e->q8, static_cast<size_t>(qn)},
        {"q8_scale", e->q8_scale, static_cast<size_t>(qn / 128) * 4},
        {"q8_sum8", e->q8_sum8, static_cast<size_t>(qn / 8) * 4},
        {"embed_w", e->embed.w, static_cast<size_t>(c.vocab_size) * c.hidden_size / 2},
        {"embed_s", e->embed.s, static_cast<size_t>(c.vocab_size) * (c.hidden_size / 128) * 2},
        {"lm_head_w", e->lm.w, static_cast<size_t>(c.vocab_size) * c.hidden_size / 2},
        {"lm_head_s", e->lm.s, static_cast<size_t>(c.vocab_size) * (c.hidden_size / 128) * 2},
        {"final_norm", e->final_norm, static_cast<size_t>(c.hidden_size) * 2},
        {"control", e->ctl, sizeof(qe_device_control_block)},
    };
    // "layer<l>.<tensor>" and the LM head
    int l = -1;
    char t[32] = {0};
    if (std::sscanf(name, "layer%d.%31s", &l, t) == 2) {
        QE_REQUIRE(l >= 0 && l < c.num_layers, "engine_read_buffer: layer %d outside [0, %d)", l, c.num_layers);
        const Layer& L = e->layers[l];
        const int H = c.hidden_size, qd = c.num_q_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
        auto wb = [](const Mat& x) { return static_cast<size_t>(x.rows) * x.K / 2; };
        auto sb = [](const Mat& x) { return static_cast<size_t>(x.rows) * (x.K / 128) * 2; };
        const Item li[] = {
            {"ln1", L.ln1, static_cast<size_t>(H) * 2}, {"ln2", L.ln2, static_cast<size_t>(H) * 2},
            {"q_w", L.q.w, wb(L.q)}, {"q_s", L.q.s, sb(L.q)}, {"k_w", L.k.w, wb(L.k)}, {"k_s", L.k.s, sb(L.k)},
            {"v_w", L.v.w, wb(L.v)}, {"v_s", L.v.s, sb(L.v)}, {"o_w", L.o.w, wb(L.o)}, {"o_s", L.o.s, sb(L.o)},
            {"gate_up_w", L.gate_up.w, wb(L.gate_up)}, {"gate_up_s", L.gate_up.s, sb(L.gate_up)},
            {"down_w", L.down.w, wb(L.down)}, {"down_s", L.down.s, sb(L.down)},
            {"q_bias", L.q_bias, static_cast<size_t>(qd) * 2}, {"k_bias", L.k_bias, static_cast<size_t>(kvd) * 2},
            {"v_bias", L.v_bias, static_cast<size_t>(kvd) * 2},
        };
        for (const Item& it : li) {
            if (std::strcmp(it.n, t) == 0) {
                QE_REQUIRE(it.p != nullptr, "engine_read_buffer: '%s' is absent", name);
                QE_REQUIRE(bytes <= it.size, "engine_read_buffer: %zu bytes requested, '%s' holds %zu", bytes, name,
                           it.size);
                QE_HIP(hipStreamSynchronize(e->stream));
                QE_HIP(hipMemcpy(host, it.p, bytes, hipMemcpyDeviceToHost));
                return QE_OK;
            }
        }
        return fail(QE_ERR_INVALID_ARGUMENT, "engine_read_buffer: unknown layer tensor '%s'", t);
    }
    for (const Item& it : items) {
        if (std::strcmp(it.n, name) == 0) {
            QE_REQUIRE(bytes <= it.size, "engine_read_buffer: %zu bytes requested, '%s' holds %zu", bytes, name, it.size);
            QE_HIP(hipStreamSynchronize(e->stream));
            QE_HIP(hipMemcpy(host, it.p, bytes, hipMemcpyDeviceToHost));
            return QE_OK;
        }
    }
    return fail(QE_ERR_INVALID_ARGUMENT, "engine_read_buffer: unknown buffer '%s'", name);
}
