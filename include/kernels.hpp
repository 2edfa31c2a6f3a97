// kernels.hpp — C++20 host API of the W4A16 G128 matrix path, drop-in for
// the reference's include/kernels.cuh launchers (namespace qwen, same names,
// same argument order and defaults).  `cudaStream_t` becomes `hipStream_t`;
// `half` is HIP's __half.  Every launcher forwards to the C-ABI in
// qe_kernels.h and throws std::runtime_error on failure, as the reference's
// CUDA_KERNEL_CHECK does (include/tensor.cuh:11-23).
//
// Every launcher of kernels.cuh that src/engine.cu calls is declared here:
// the matrix path, and the embedding, RoPE/KV-append, attention and sampling
// launchers of the decode and prefill loops.  The prefill GEMMs that split K
// keep their partial sums in a workspace per stream (see qe_kernels.h).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "qe_kernels.h"

namespace qwen {

// Qwen2.5-1.5B dimensions, include/config.cuh:10-22.
constexpr int32_t NUM_LAYERS = 28;
constexpr int32_t HIDDEN_SIZE = 1536;
constexpr int32_t INTERMEDIATE_SIZE = 8960;
constexpr int32_t NUM_Q_HEADS = 12;
constexpr int32_t NUM_KV_HEADS = 2;
constexpr int32_t HEAD_DIM = 128;
constexpr int32_t Q_DIM = 1536;
constexpr int32_t KV_DIM = 256;
constexpr int32_t VOCAB_SIZE = 151936;
constexpr float RMS_NORM_EPS = 1e-6f;
constexpr int32_t MAX_SEQ_LEN = 4096;
constexpr float ROPE_THETA = 1000000.0f;
constexpr int32_t QUANT_GROUP_SIZE = 128;

// include/tensor.cuh:28-34
using DeviceControlBlock = qe_device_control_block;
static_assert(sizeof(DeviceControlBlock) == 256, "DeviceControlBlock layout");

// include/kernels.cuh:23-27
struct QKVProjectionView {
    const void* q_weight; const half* q_scale; half* d_q;
    const void* k_weight; const half* k_scale; half* d_k;
    const void* v_weight; const half* v_scale; half* d_v;
};
static_assert(sizeof(QKVProjectionView) == sizeof(qe_qkv_view), "QKVProjectionView layout");

namespace detail {
inline void check(int rc, const char* what) {
    if (rc != QE_OK) throw std::runtime_error(std::string(what) + ": " + qe_last_error());
}
inline const uint16_t* h(const half* p) { return reinterpret_cast<const uint16_t*>(p); }
inline uint16_t* h(half* p) { return reinterpret_cast<uint16_t*>(p); }
inline const qe_qkv_view* v(const QKVProjectionView& view) { return reinterpret_cast<const qe_qkv_view*>(&view); }
}  // namespace detail

// include/kernels.cuh:39-48
inline void launch_rmsnorm_q8_1(const half* input, const half* gamma, half* output_fp16_opt, int8_t* out_q8,
                                float* out_scale, int32_t* out_sum8, hipStream_t stream,
                                int hidden_size = HIDDEN_SIZE) {
    detail::check(qe_launch_rmsnorm_q8_1(detail::h(input), detail::h(gamma), detail::h(output_fp16_opt), out_q8,
                                         out_scale, out_sum8, stream, hidden_size),
                  "launch_rmsnorm_q8_1");
}

// include/kernels.cuh:11-20
inline void launch_embed_lookup_w4a16(const uint32_t* embed_qweight, const half* embed_scales,
                                      const int32_t* d_token_ids, half* out_hidden,
                                      const DeviceControlBlock* d_control, int num_tokens, hipStream_t stream,
                                      int hidden_size = HIDDEN_SIZE) {
    detail::check(qe_launch_embed_lookup_w4a16(embed_qweight, detail::h(embed_scales), d_token_ids,
                                               detail::h(out_hidden), d_control, num_tokens, stream, hidden_size),
                  "launch_embed_lookup_w4a16");
}

// include/kernels.cuh:30-37
inline void launch_rmsnorm_fp16(const half* input, const half* gamma, half* output, int num_tokens,
                                hipStream_t stream, int hidden_size = HIDDEN_SIZE) {
    detail::check(qe_launch_rmsnorm_fp16(detail::h(input), detail::h(gamma), detail::h(output), num_tokens, stream,
                                         hidden_size),
                  "launch_rmsnorm_fp16");
}

// include/kernels.cuh:50-57
inline void launch_quantize_fp16_to_q8_1(const half* input_x, int8_t* out_q8, float* out_scale, int32_t* out_sum8,
                                         int num_elements, hipStream_t stream) {
    detail::check(qe_launch_quantize_fp16_to_q8_1(detail::h(input_x), out_q8, out_scale, out_sum8, num_elements,
                                                  stream),
                  "launch_quantize_fp16_to_q8_1");
}

// include/kernels.cuh:60-69
inline void launch_gemv_w4a16(const uint32_t* qweight, const half* scales, const half* input_x, const half* residual,
                              half* output_y, int out_features, int in_features, hipStream_t stream) {
    detail::check(qe_launch_gemv_w4a16(qweight, detail::h(scales), detail::h(input_x), detail::h(residual),
                                       detail::h(output_y), out_features, in_features, stream),
                  "launch_gemv_w4a16");
}

// include/kernels.cuh:71-82
inline void launch_gemv_w4a8(const uint32_t* qweight, const half* scales, const int8_t* input_q8,
                             const float* input_scale, const int32_t* input_sum8, const half* residual,
                             half* output_y, int out_features, int in_features, hipStream_t stream) {
    detail::check(qe_launch_gemv_w4a8(qweight, detail::h(scales), input_q8, input_scale, input_sum8,
                                      detail::h(residual), detail::h(output_y), out_features, in_features, stream),
                  "launch_gemv_w4a8");
}

// include/kernels.cuh:84-94
inline void launch_gemv_qkv_w4a8(const QKVProjectionView& view, const int8_t* input_q8, const float* input_scale,
                                 const int32_t* input_sum8, hipStream_t stream, int in_features = HIDDEN_SIZE,
                                 int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS,
                                 int head_dim = HEAD_DIM) {
    detail::check(qe_launch_gemv_qkv_w4a8(detail::v(view), input_q8, input_scale, input_sum8, stream, in_features,
                                          num_q_heads, num_kv_heads, head_dim),
                  "launch_gemv_qkv_w4a8");
}

// include/kernels.cuh:96-104
inline void launch_gemv_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight, const half* gate_up_scales,
                                                  const half* input_x, half* output_mlp, int hidden_size,
                                                  int intermediate_size, hipStream_t stream) {
    detail::check(qe_launch_gemv_dual_gate_up_swiglu_w4a16(gate_up_qweight, detail::h(gate_up_scales),
                                                           detail::h(input_x), detail::h(output_mlp), hidden_size,
                                                           intermediate_size, stream),
                  "launch_gemv_dual_gate_up_swiglu_w4a16");
}

// include/kernels.cuh:106-116
inline void launch_gemv_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const half* gate_up_scales,
                                                 const int8_t* input_q8, const float* input_scale,
                                                 const int32_t* input_sum8, half* output_mlp, int hidden_size,
                                                 int intermediate_size, hipStream_t stream) {
    detail::check(qe_launch_gemv_dual_gate_up_swiglu_w4a8(gate_up_qweight, detail::h(gate_up_scales), input_q8,
                                                          input_scale, input_sum8, detail::h(output_mlp),
                                                          hidden_size, intermediate_size, stream),
                  "launch_gemv_dual_gate_up_swiglu_w4a8");
}

// include/kernels.cuh:119-130
inline void launch_gemm_prefill_w4a16(const uint32_t* qweight, const half* scales, const half* input_x,
                                      const half* residual, half* output_y, int M, int N, int K, hipStream_t stream,
                                      int sm_count = 0) {
    detail::check(qe_launch_gemm_prefill_w4a16(qweight, detail::h(scales), detail::h(input_x), detail::h(residual),
                                               detail::h(output_y), M, N, K, stream, sm_count),
                  "launch_gemm_prefill_w4a16");
}

// include/kernels.cuh:132-142
inline void launch_gemm_prefill_qkv_w4a16(const QKVProjectionView& view, const half* input_x, int M,
                                          hipStream_t stream, int in_features = HIDDEN_SIZE,
                                          int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS,
                                          int head_dim = HEAD_DIM, int sm_count = 0) {
    detail::check(qe_launch_gemm_prefill_qkv_w4a16(detail::v(view), detail::h(input_x), M, stream, in_features,
                                                   num_q_heads, num_kv_heads, head_dim, sm_count),
                  "launch_gemm_prefill_qkv_w4a16");
}

// include/kernels.cuh:144-153
inline void launch_gemm_prefill_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight,
                                                          const half* gate_up_scales, const half* input_x,
                                                          half* output_mlp, int M, hipStream_t stream,
                                                          int hidden_size = HIDDEN_SIZE,
                                                          int intermediate_size = INTERMEDIATE_SIZE) {
    detail::check(qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16(gate_up_qweight, detail::h(gate_up_scales),
                                                                   detail::h(input_x), detail::h(output_mlp), M,
                                                                   stream, hidden_size, intermediate_size),
                  "launch_gemm_prefill_dual_gate_up_swiglu_w4a16");
}

// include/kernels.cuh:156-174
inline void launch_qkv_bias_rope_kv_append(half* q, half* k, half* v, const half* q_bias, const half* k_bias,
                                           const half* v_bias, half* layer_k_cache, half* layer_v_cache,
                                           const DeviceControlBlock* d_control, int num_tokens, hipStream_t stream,
                                           int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS,
                                           int head_dim = HEAD_DIM, int max_seq_len = MAX_SEQ_LEN,
                                           int rotary_dim = 0, float rope_theta = ROPE_THETA) {
    detail::check(qe_launch_qkv_bias_rope_kv_append(detail::h(q), detail::h(k), detail::h(v), detail::h(q_bias),
                                                    detail::h(k_bias), detail::h(v_bias), detail::h(layer_k_cache),
                                                    detail::h(layer_v_cache), d_control, num_tokens, stream,
                                                    num_q_heads, num_kv_heads, head_dim, max_seq_len, rotary_dim,
                                                    rope_theta),
                  "launch_qkv_bias_rope_kv_append");
}

// include/kernels.cuh:177-193
inline void launch_attention_gqa_flash_decode(const half* q, const half* layer_k_cache, const half* layer_v_cache,
                                              float* splitk_partial_out, float* splitk_partial_lse, half* attn_out,
                                              const DeviceControlBlock* d_control, hipStream_t stream,
                                              int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS,
                                              int head_dim = HEAD_DIM, int max_seq_len = MAX_SEQ_LEN,
                                              int8_t* out_q8 = nullptr, float* out_scale = nullptr,
                                              int32_t* out_sum8 = nullptr) {
    detail::check(qe_launch_attention_gqa_flash_decode(detail::h(q), detail::h(layer_k_cache),
                                                       detail::h(layer_v_cache), splitk_partial_out,
                                                       splitk_partial_lse, detail::h(attn_out), d_control, stream,
                                                       num_q_heads, num_kv_heads, head_dim, max_seq_len, out_q8,
                                                       out_scale, out_sum8),
                  "launch_attention_gqa_flash_decode");
}

// include/kernels.cuh:195-207
inline void launch_attention_gqa_prefill(const half* q, const half* layer_k_cache, const half* layer_v_cache,
                                         half* attn_out, const DeviceControlBlock* d_control, int num_tokens,
                                         hipStream_t stream, int num_q_heads = NUM_Q_HEADS,
                                         int num_kv_heads = NUM_KV_HEADS, int head_dim = HEAD_DIM,
                                         int max_seq_len = MAX_SEQ_LEN, int hidden_size = HIDDEN_SIZE) {
    detail::check(qe_launch_attention_gqa_prefill(detail::h(q), detail::h(layer_k_cache), detail::h(layer_v_cache),
                                                  detail::h(attn_out), d_control, num_tokens, stream, num_q_heads,
                                                  num_kv_heads, head_dim, max_seq_len, hidden_size),
                  "launch_attention_gqa_prefill");
}

// include/kernels.cuh:209-217 (greedy decoding)
inline void launch_sample_and_advance(const half* logits, float* sample_scratch_val, int32_t* sample_scratch_idx,
                                      DeviceControlBlock* d_control, int32_t* d_mapped_pinned_token,
                                      hipStream_t stream, int vocab_size = VOCAB_SIZE) {
    detail::check(qe_launch_sample_and_advance(detail::h(logits), sample_scratch_val, sample_scratch_idx, d_control,
                                               d_mapped_pinned_token, stream, vocab_size),
                  "launch_sample_and_advance");
}

// ---- W4A8 prefill GEMM of this build (int8 MFMA; no counterpart in kernels.cuh) ----
inline void launch_gemm_prefill_w4a8(const uint32_t* qweight, const half* scales, const int8_t* input_q8,
                                     const float* input_scale, const int32_t* input_sum8, const half* residual,
                                     half* output_y, int M, int N, int K, hipStream_t stream) {
    detail::check(qe_launch_gemm_prefill_w4a8(qweight, detail::h(scales), input_q8, input_scale, input_sum8,
                                              detail::h(residual), detail::h(output_y), M, N, K, stream),
                  "launch_gemm_prefill_w4a8");
}

inline void launch_gemm_prefill_qkv_w4a8(const QKVProjectionView& view, const int8_t* input_q8,
                                         const float* input_scale, const int32_t* input_sum8, int M,
                                         hipStream_t stream, int in_features = HIDDEN_SIZE,
                                         int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS,
                                         int head_dim = HEAD_DIM) {
    detail::check(qe_launch_gemm_prefill_qkv_w4a8(detail::v(view), input_q8, input_scale, input_sum8, M, stream,
                                                  in_features, num_q_heads, num_kv_heads, head_dim),
                  "launch_gemm_prefill_qkv_w4a8");
}

inline void launch_gemm_prefill_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const half* gate_up_scales,
                                                         const int8_t* input_q8, const float* input_scale,
                                                         const int32_t* input_sum8, half* output_mlp, int M,
                                                         hipStream_t stream, int hidden_size = HIDDEN_SIZE,
                                                         int intermediate_size = INTERMEDIATE_SIZE) {
    detail::check(qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a8(gate_up_qweight, detail::h(gate_up_scales),
                                                                  input_q8, input_scale, input_sum8,
                                                                  detail::h(output_mlp), M, stream, hidden_size,
                                                                  intermediate_size),
                  "launch_gemm_prefill_dual_gate_up_swiglu_w4a8");
}

// ---- fused decode launchers of this build (no counterpart in kernels.cuh) ----
inline void launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(
    const half* input, const half* gamma, half* output_fp16_opt, const QKVProjectionView& view, const half* q_bias,
    const half* k_bias, const half* v_bias, half* layer_k_cache, half* layer_v_cache,
    const DeviceControlBlock* d_control, hipStream_t stream, int hidden_size = HIDDEN_SIZE,
    int num_q_heads = NUM_Q_HEADS, int num_kv_heads = NUM_KV_HEADS, int head_dim = HEAD_DIM,
    int max_seq_len = MAX_SEQ_LEN, int rotary_dim = HEAD_DIM, float rope_theta = ROPE_THETA) {
    detail::check(qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(
                      detail::h(input), detail::h(gamma), detail::h(output_fp16_opt), detail::v(view),
                      detail::h(q_bias), detail::h(k_bias), detail::h(v_bias), detail::h(layer_k_cache),
                      detail::h(layer_v_cache), d_control, stream, hidden_size, num_q_heads, num_kv_heads,
                      head_dim, max_seq_len, rotary_dim, rope_theta),
                  "launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16");
}

inline void launch_gemv_lm_head_sample_w4a8(const uint32_t* qweight, const half* scales, const int8_t* input_q8,
                                            const float* input_scale, const int32_t* input_sum8, half* logits_opt,
                                            float* sample_scratch_val, int32_t* sample_scratch_idx,
                                            DeviceControlBlock* d_control, int32_t* d_mapped_pinned_token,
                                            hipStream_t stream, int vocab_size = VOCAB_SIZE,
                                            int in_features = HIDDEN_SIZE) {
    detail::check(qe_launch_gemv_lm_head_sample_w4a8(qweight, detail::h(scales), input_q8, input_scale, input_sum8,
                                                     detail::h(logits_opt), sample_scratch_val, sample_scratch_idx,
                                                     d_control, d_mapped_pinned_token, vocab_size, in_features,
                                                     stream),
                  "launch_gemv_lm_head_sample_w4a8");
}

inline void launch_rmsnorm_gemv_lm_head_sample_w4a16(const half* input, const half* gamma, half* output_fp16_opt,
                                                     const uint32_t* qweight, const half* scales, half* logits_opt,
                                                     float* sample_scratch_val, int32_t* sample_scratch_idx,
                                                     DeviceControlBlock* d_control, int32_t* d_mapped_pinned_token,
                                                     hipStream_t stream, int vocab_size = VOCAB_SIZE,
                                                     int hidden_size = HIDDEN_SIZE) {
    detail::check(qe_launch_rmsnorm_gemv_lm_head_sample_w4a16(
                      detail::h(input), detail::h(gamma), detail::h(output_fp16_opt), qweight, detail::h(scales),
                      detail::h(logits_opt), sample_scratch_val, sample_scratch_idx, d_control,
                      d_mapped_pinned_token, vocab_size, hidden_size, stream),
                  "launch_rmsnorm_gemv_lm_head_sample_w4a16");
}

inline void launch_rmsnorm_gemv_qkv_w4a16(const half* input, const half* gamma, half* output_fp16_opt,
                                          const QKVProjectionView& view, hipStream_t stream,
                                          int hidden_size = HIDDEN_SIZE, int num_q_heads = NUM_Q_HEADS,
                                          int num_kv_heads = NUM_KV_HEADS, int head_dim = HEAD_DIM) {
    detail::check(qe_launch_rmsnorm_gemv_qkv_w4a16(detail::h(input), detail::h(gamma), detail::h(output_fp16_opt),
                                                   detail::v(view), stream, hidden_size, num_q_heads, num_kv_heads,
                                                   head_dim),
                  "launch_rmsnorm_gemv_qkv_w4a16");
}

inline void launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(const half* input, const half* gamma,
                                                          half* output_fp16_opt, const uint32_t* gate_up_qweight,
                                                          const half* gate_up_scales, half* output_mlp,
                                                          int hidden_size, int intermediate_size,
                                                          hipStream_t stream) {
    detail::check(qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(
                      detail::h(input), detail::h(gamma), detail::h(output_fp16_opt), gate_up_qweight,
                      detail::h(gate_up_scales), detail::h(output_mlp), hidden_size, intermediate_size, stream),
                  "launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16");
}

}  // namespace qwen
