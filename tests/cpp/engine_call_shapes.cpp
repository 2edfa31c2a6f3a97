// Compile-only check (hipcc -fsyntax-only): every launcher call that the
// reference's decode and prefill loops make (src/engine.cu:361-450 decode,
// :472-580 prefill and the prefill LM head) compiles against kernels.hpp with
// the same argument lists, relying on the same default arguments.
#include "kernels.hpp"

using namespace qwen;

struct Layer {
    const void *q_weight, *k_weight, *v_weight, *o_weight, *gate_up_weight, *down_weight;
    const half *q_scale, *k_scale, *v_scale, *o_scale, *gate_up_scale, *down_scale;
    const half *q_bias, *k_bias, *v_bias, *input_layernorm, *post_attention_layernorm;
};

struct Workspace {
    half *d_act_0, *d_act_1, *d_q, *d_k, *d_v, *d_attn_out, *d_mlp_act, *d_logits;
    int8_t* d_act_q8;
    float *d_act_scale, *d_splitk_out, *d_splitk_lse, *d_sample_val;
    int32_t *d_act_sum8, *d_sample_idx, *d_prompt_tokens;
};

void decode_layer(const Layer& L, Workspace& ws, half* layer_k, half* layer_v, DeviceControlBlock* ctl,
                  hipStream_t stream, int max_seq, float rope_theta) {
    launch_rmsnorm_q8_1(ws.d_act_0, L.input_layernorm, nullptr, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8, stream,
                        HIDDEN_SIZE);
    QKVProjectionView view = {L.q_weight, L.q_scale, ws.d_q, L.k_weight, L.k_scale, ws.d_k,
                              L.v_weight, L.v_scale, ws.d_v};
    launch_gemv_qkv_w4a8(view, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8, stream, HIDDEN_SIZE, NUM_Q_HEADS,
                         NUM_KV_HEADS, HEAD_DIM);
    launch_qkv_bias_rope_kv_append(ws.d_q, ws.d_k, ws.d_v, L.q_bias, L.k_bias, L.v_bias, layer_k, layer_v, ctl, 1,
                                   stream, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM, max_seq, HEAD_DIM, rope_theta);
    launch_attention_gqa_flash_decode(ws.d_q, layer_k, layer_v, ws.d_splitk_out, ws.d_splitk_lse, ws.d_attn_out,
                                      ctl, stream, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM, max_seq, ws.d_act_q8,
                                      ws.d_act_scale, ws.d_act_sum8);
    launch_gemv_w4a8(reinterpret_cast<const uint32_t*>(L.o_weight), L.o_scale, ws.d_act_q8, ws.d_act_scale,
                     ws.d_act_sum8, ws.d_act_0, ws.d_act_0, HIDDEN_SIZE, Q_DIM, stream);
}

void decode_pass(const Layer* layers, Workspace& ws, const uint32_t* embed_w, const half* embed_s,
                 const half* final_norm, const uint32_t* lm_w, const half* lm_s, half* k_cache, half* v_cache,
                 DeviceControlBlock* ctl, int32_t* pinned_token, hipStream_t stream, int max_seq, float theta) {
    launch_embed_lookup_w4a16(embed_w, embed_s, nullptr, ws.d_act_0, ctl, 1, stream, HIDDEN_SIZE);
    const size_t kv_stride = static_cast<size_t>(NUM_KV_HEADS) * max_seq * HEAD_DIM;
    for (int l = 0; l < NUM_LAYERS; ++l) {
        decode_layer(layers[l], ws, k_cache + l * kv_stride, v_cache + l * kv_stride, ctl, stream, max_seq, theta);
        launch_rmsnorm_q8_1(ws.d_act_0, layers[l].post_attention_layernorm, nullptr, ws.d_act_q8, ws.d_act_scale,
                            ws.d_act_sum8, stream, HIDDEN_SIZE);
        launch_gemv_dual_gate_up_swiglu_w4a8(reinterpret_cast<const uint32_t*>(layers[l].gate_up_weight),
                                             layers[l].gate_up_scale, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8,
                                             ws.d_mlp_act, HIDDEN_SIZE, INTERMEDIATE_SIZE, stream);
        launch_quantize_fp16_to_q8_1(ws.d_mlp_act, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8, INTERMEDIATE_SIZE,
                                     stream);
        launch_gemv_w4a8(reinterpret_cast<const uint32_t*>(layers[l].down_weight), layers[l].down_scale, ws.d_act_q8,
                         ws.d_act_scale, ws.d_act_sum8, ws.d_act_0, ws.d_act_0, HIDDEN_SIZE, INTERMEDIATE_SIZE,
                         stream);
    }
    launch_rmsnorm_q8_1(ws.d_act_0, final_norm, nullptr, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8, stream,
                        HIDDEN_SIZE);
    launch_gemv_w4a8(lm_w, lm_s, ws.d_act_q8, ws.d_act_scale, ws.d_act_sum8, nullptr, ws.d_logits, VOCAB_SIZE,
                     HIDDEN_SIZE, stream);
    launch_sample_and_advance(ws.d_logits, ws.d_sample_val, ws.d_sample_idx, ctl, pinned_token, stream, VOCAB_SIZE);
}

void prefill_chunk(const Layer* layers, Workspace& ws, const uint32_t* embed_w, const half* embed_s,
                   half* k_cache, half* v_cache, DeviceControlBlock* ctl, hipStream_t stream, int chunk_start,
                   int chunk_len, int max_seq, float theta, int sm_count) {
    launch_embed_lookup_w4a16(embed_w, embed_s, ws.d_prompt_tokens + chunk_start, ws.d_act_0, nullptr, chunk_len,
                              stream, HIDDEN_SIZE);
    const size_t kv_stride = static_cast<size_t>(NUM_KV_HEADS) * max_seq * HEAD_DIM;
    for (int l = 0; l < NUM_LAYERS; ++l) {
        const Layer& L = layers[l];
        half* layer_k = k_cache + l * kv_stride;
        half* layer_v = v_cache + l * kv_stride;
        launch_rmsnorm_fp16(ws.d_act_0, L.input_layernorm, ws.d_act_1, chunk_len, stream, HIDDEN_SIZE);
        QKVProjectionView view = {L.q_weight, L.q_scale, ws.d_q, L.k_weight, L.k_scale, ws.d_k,
                                  L.v_weight, L.v_scale, ws.d_v};
        launch_gemm_prefill_qkv_w4a16(view, ws.d_act_1, chunk_len, stream, HIDDEN_SIZE, NUM_Q_HEADS, NUM_KV_HEADS,
                                      HEAD_DIM, sm_count);
        launch_qkv_bias_rope_kv_append(ws.d_q, ws.d_k, ws.d_v, L.q_bias, L.k_bias, L.v_bias, layer_k, layer_v, ctl,
                                       chunk_len, stream, NUM_Q_HEADS, NUM_KV_HEADS, HEAD_DIM, max_seq, HEAD_DIM,
                                       theta);
        launch_attention_gqa_prefill(ws.d_q, layer_k, layer_v, ws.d_attn_out, ctl, chunk_len, stream, NUM_Q_HEADS,
                                     NUM_KV_HEADS, HEAD_DIM, max_seq, Q_DIM);
        launch_gemm_prefill_w4a16(reinterpret_cast<const uint32_t*>(L.o_weight), L.o_scale, ws.d_attn_out,
                                  ws.d_act_0, ws.d_act_0, chunk_len, HIDDEN_SIZE, Q_DIM, stream, sm_count);
        launch_rmsnorm_fp16(ws.d_act_0, L.post_attention_layernorm, ws.d_act_1, chunk_len, stream, HIDDEN_SIZE);
        launch_gemm_prefill_dual_gate_up_swiglu_w4a16(reinterpret_cast<const uint32_t*>(L.gate_up_weight),
                                                      L.gate_up_scale, ws.d_act_1, ws.d_mlp_act, chunk_len, stream,
                                                      HIDDEN_SIZE, INTERMEDIATE_SIZE);
        launch_gemm_prefill_w4a16(reinterpret_cast<const uint32_t*>(L.down_weight), L.down_scale, ws.d_mlp_act,
                                  ws.d_act_0, ws.d_act_0, chunk_len, HIDDEN_SIZE, INTERMEDIATE_SIZE, stream,
                                  sm_count);
    }
}

// The defaults the reference's header gives: rotary_dim = 0 (full head), no
// Q8_1 epilogue, Qwen2.5-1.5B dimensions, sm_count = 0.
void defaults(half* q, half* k, half* v, const half* b, half* kc, half* vc, const DeviceControlBlock* ctl,
              float* po, float* pl, half* out, const QKVProjectionView& view, const uint32_t* w, const half* s,
              hipStream_t st) {
    launch_qkv_bias_rope_kv_append(q, k, v, b, b, b, kc, vc, ctl, 1, st);
    launch_attention_gqa_flash_decode(q, kc, vc, po, pl, out, ctl, st);
    launch_attention_gqa_prefill(q, kc, vc, out, ctl, 16, st);
    launch_embed_lookup_w4a16(w, s, nullptr, out, ctl, 1, st);
    launch_gemm_prefill_qkv_w4a16(view, out, 128, st);
    launch_gemm_prefill_w4a16(w, s, out, nullptr, out, 128, HIDDEN_SIZE, Q_DIM, st);
    launch_gemm_prefill_dual_gate_up_swiglu_w4a16(w, s, out, out, 128, st);
    launch_gemv_qkv_w4a8(view, nullptr, nullptr, nullptr, st);
    launch_rmsnorm_q8_1(out, s, nullptr, nullptr, nullptr, nullptr, st);
    launch_rmsnorm_fp16(out, s, out, 4, st);
}
