/*
 * qe_kernels.h — C-ABI of the MI355X (gfx950) W4A16 group-128 matrix path.
 *
 * One extern "C" entry point per launcher of the reference's kernel API
 * (Areen-09/qwen-engine include/kernels.cuh).  Plain pointers and sizes only:
 *   - fp16 buffers are `uint16_t*` (IEEE binary16 bit patterns),
 *   - packed int4 weights are `uint32_t[N][K/8]`, nibble order
 *     q0|q4<<4|q1<<8|q5<<12|q2<<16|q6<<20|q3<<24|q7<<28 (element 8w+j = q_j),
 *   - group scales are fp16 `[N][K/128]`, zero point 8,
 *   - Q8_1 activations are int8 q8[K], fp32 scale[K/128], int32 sum8[K/8]
 *     with sum8 = -8 * (sum of the 8 q8 values it covers),
 *   - `stream` is a hipStream_t (NULL = the null stream).
 * Every call is asynchronous on `stream`, never synchronizes, and is safe
 * under HIP graph capture.  `residual` may alias the output.  A NULL
 * optional pointer means "skip", as in the reference.  No launcher
 * allocates (the reference's launchers keep no state and allocate nothing,
 * src/kernels/gemm_prefill.cu:616-684).  The prefill GEMMs may split K over
 * several blocks and then keep fp32 partial sums in a workspace registered
 * for the launching stream, ahead of time, by qe_gemm_reserve_workspace (the
 * library allocates 32 MiB) or qe_gemm_attach_workspace (caller memory).  A
 * stream without a workspace runs its GEMMs without K slices, eagerly and
 * under graph capture alike: the plan, and so the bits, of a launch depend
 * only on the shape, the qe_set_tuning switches and whether the stream holds
 * a workspace.  GEMMs on different streams never share partials.
 * hipStreamPerThread never holds a workspace (it names a different stream
 * in every thread); the null stream is the device's legacy stream.
 *
 * Return value: QE_OK, or a QE_ERR_* code; qe_last_error() then describes
 * the failure (thread-local).  The C++ mirror in kernels.hpp turns a
 * non-zero status into std::runtime_error, as the reference's
 * CUDA_KERNEL_CHECK does (include/tensor.cuh:11-23).
 */
#ifndef QE_KERNELS_H
#define QE_KERNELS_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QE_OK 0
#define QE_ERR_INVALID_ARGUMENT 1 /* shape / alignment precondition violated */
#define QE_ERR_UNSUPPORTED 2      /* shape outside what this build implements */
#define QE_ERR_HIP 3              /* HIP runtime error at launch */

/* Description of the last failure on the calling thread ("" if none). */
const char* qe_last_error(void);
/* Library version string. */
const char* qe_version(void);

/* Device control block, same layout as the reference's DeviceControlBlock
 * (include/tensor.cuh:28-34). */
typedef struct __attribute__((aligned(256))) qe_device_control_block {
    int32_t token_id;
    int32_t seq_pos;
    float temperature;
    uint32_t reserved;
    uint64_t rng_seed;
} qe_device_control_block;

/* Fused-QKV descriptor, same layout as QKVProjectionView
 * (include/kernels.cuh:23-27). */
typedef struct qe_qkv_view {
    const void* q_weight; const uint16_t* q_scale; uint16_t* d_q;
    const void* k_weight; const uint16_t* k_scale; uint16_t* d_k;
    const void* v_weight; const uint16_t* v_scale; uint16_t* d_v;
} qe_qkv_view;

/* ---- Q8_1 quantizers ---------------------------------------------------- */

/* Replaces launch_quantize_fp16_to_q8_1, include/kernels.cuh:50-57.
 * fp16[num_elements] -> Q8_1.  num_elements % 128 == 0, input 16-byte aligned. */
int qe_launch_quantize_fp16_to_q8_1(const uint16_t* input_x, int8_t* out_q8, float* out_scale,
                                    int32_t* out_sum8, int num_elements, hipStream_t stream);

/* Replaces launch_rmsnorm_q8_1, include/kernels.cuh:39-48.  One token:
 * fp16 RMSNorm (optionally written to output_fp16_opt) then Q8_1 of the
 * fp16-rounded normalized vector.  hidden_size % 128 == 0. */
int qe_launch_rmsnorm_q8_1(const uint16_t* input, const uint16_t* gamma, uint16_t* output_fp16_opt,
                           int8_t* out_q8, float* out_scale, int32_t* out_sum8,
                           hipStream_t stream, int hidden_size);

/* Replaces launch_rmsnorm_fp16, include/kernels.cuh:30-37 (prefill rows). */
int qe_launch_rmsnorm_fp16(const uint16_t* input, const uint16_t* gamma, uint16_t* output,
                           int num_tokens, hipStream_t stream, int hidden_size);

/* ---- decode GEMV (W4A8: Q8_1 activations) -------------------------------- */

/* Replaces launch_gemv_w4a8, include/kernels.cuh:71-82.
 * y[n] = fp16( sum_g dot_g(n) * (s[n,g]*x_scale[g]) [+ residual[n]] ). */
int qe_launch_gemv_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                        const float* input_scale, const int32_t* input_sum8, const uint16_t* residual,
                        uint16_t* output_y, int out_features, int in_features, hipStream_t stream);

/* Replaces launch_gemv_qkv_w4a8, include/kernels.cuh:84-94.  Rows
 * [0,q_dim) -> d_q, [q_dim,q_dim+kv_dim) -> d_k, rest -> d_v. */
int qe_launch_gemv_qkv_w4a8(const qe_qkv_view* view, const int8_t* input_q8, const float* input_scale,
                            const int32_t* input_sum8, hipStream_t stream, int in_features,
                            int num_q_heads, int num_kv_heads, int head_dim);

/* Replaces launch_gemv_dual_gate_up_swiglu_w4a8, include/kernels.cuh:106-116.
 * Weight rows are interleaved (2i = gate_i, 2i+1 = up_i);
 * out[i] = fp16(silu(gate_i) * up_i). */
int qe_launch_gemv_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                            const int8_t* input_q8, const float* input_scale,
                                            const int32_t* input_sum8, uint16_t* output_mlp,
                                            int hidden_size, int intermediate_size, hipStream_t stream);

/* ---- decode GEMV (W4A16: fp16 activations, quantized inside the launch) -- */

/* Replaces launch_gemv_w4a16, include/kernels.cuh:60-69. */
int qe_launch_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                         const uint16_t* residual, uint16_t* output_y, int out_features, int in_features,
                         hipStream_t stream);

/* Replaces launch_gemv_dual_gate_up_swiglu_w4a16, include/kernels.cuh:96-104. */
int qe_launch_gemv_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                             const uint16_t* input_x, uint16_t* output_mlp,
                                             int hidden_size, int intermediate_size, hipStream_t stream);

/* ---- fused decode entry points (no counterpart in the reference API) ---- */

/* RMSNorm + Q8_1 + fused-QKV GEMV in one launch: the same results as
 * qe_launch_rmsnorm_q8_1 followed by qe_launch_gemv_qkv_w4a8 (the reference's
 * src/engine.cu:367-379 pair), without the Q8_1 round trip through memory.
 * output_fp16_opt (optional) receives the fp16 normalized activation. */
int qe_launch_rmsnorm_gemv_qkv_w4a16(const uint16_t* input, const uint16_t* gamma, uint16_t* output_fp16_opt,
                                     const qe_qkv_view* view, hipStream_t stream, int hidden_size,
                                     int num_q_heads, int num_kv_heads, int head_dim);

/* RMSNorm + Q8_1 + gate/up SwiGLU GEMV in one launch: the same results as
 * qe_launch_rmsnorm_q8_1 followed by qe_launch_gemv_dual_gate_up_swiglu_w4a8
 * (src/engine.cu:414-424). */
int qe_launch_rmsnorm_gemv_dual_gate_up_swiglu_w4a16(const uint16_t* input, const uint16_t* gamma,
                                                     uint16_t* output_fp16_opt, const uint32_t* gate_up_qweight,
                                                     const uint16_t* gate_up_scales, uint16_t* output_mlp,
                                                     int hidden_size, int intermediate_size, hipStream_t stream);

/* ---- prefill dequant-GEMM (MFMA) ----------------------------------------- */

/* Allocates a 32 MiB split-K workspace for `stream` on the current device
 * (hipMalloc; the only allocation of the kernel API) and registers it, so
 * prefill GEMMs on that stream may split K.  Call it before the first GEMM
 * on the stream, outside graph capture (QE_ERR_INVALID_ARGUMENT while the
 * stream is capturing, or for hipStreamPerThread).  At most 64 streams per
 * device hold a workspace (QE_ERR_UNSUPPORTED beyond).  No counterpart in the
 * reference (its GEMMs never split K). */
int qe_gemm_reserve_workspace(hipStream_t stream);

/* Registers caller memory (>= 1 MiB, 256-byte aligned; at most 32 MiB is
 * used) as the split-K workspace of `stream` on the current device, in place
 * of one allocated by qe_gemm_reserve_workspace (which is then freed).  The
 * memory must stay valid until qe_gemm_release_workspace(stream).  No
 * counterpart in the reference. */
int qe_gemm_attach_workspace(hipStream_t stream, void* workspace, size_t bytes);

/* Drops the workspace of `stream` on the current device (freed if the
 * library allocated it; call it before destroying the stream).  Later GEMMs
 * on the stream run without K slices.  QE_OK also when there was none. */
int qe_gemm_release_workspace(hipStream_t stream);

/* Number of hipMalloc calls the library has made for GEMM workspaces in this
 * process (only qe_gemm_reserve_workspace makes them).  Test hook. */
long qe_gemm_workspace_allocations(void);

/* The tile (1 64x64, 2 64x128, 3 128x64, 4 128x128) and K-slice count a
 * prefill GEMM of this shape would use on the current device with a stream
 * workspace (tiled != 0: the tiled-layout launchers), after the qe_set_tuning
 * overrides.  Host only; no counterpart in the reference. */
int qe_gemm_prefill_plan(int M, int N, int K, int tiled, int* tile, int* slices);

/* Replaces launch_gemm_prefill_w4a16, include/kernels.cuh:119-130.
 * Y[M,N] = fp16(A[M,K] . dequant(W)[N,K]^T), fp32 accumulation;
 * residual added as fp16(fp16(acc) + residual).  `sm_count` is accepted for
 * signature parity; tile selection uses the device's CU count.  K-slice
 * partials are summed in slice order, so a given plan is deterministic; a
 * stream without a workspace (see above) runs unsplit, which may round
 * differently in fp32 from a split plan. */
int qe_launch_gemm_prefill_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                                 const uint16_t* residual, uint16_t* output_y, int M, int N, int K,
                                 hipStream_t stream, int sm_count);

/* qe_launch_gemm_prefill_w4a16 without any allocation, for callers that
 * cannot allocate or register a workspace (code under graph capture,
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same arguments, same tile and K-slice plan and same results as
 * qe_launch_gemm_prefill_w4a16; the split-K partials go to a 32 MiB device
 * array of the library (one per GPU, held until the process ends) instead of
 * the stream's workspace.  Rejects M * N > 8388608 (QE_ERR_INVALID_ARGUMENT).
 * Every call on one GPU shares that array: calls that overlap in time on one
 * GPU (different streams, no ordering between them) race and give wrong
 * results.  Calls ordered on one stream are safe; nothing needs clearing
 * between calls (each slice writes its partials before they are read). */
int qe_launch_gemm_prefill_w4a16_noalloc(const uint32_t* qweight, const uint16_t* scales, const uint16_t* input_x,
                                         const uint16_t* residual, uint16_t* output_y, int M, int N, int K,
                                         hipStream_t stream, int sm_count);

/* Replaces launch_gemm_prefill_qkv_w4a16, include/kernels.cuh:132-142. */
int qe_launch_gemm_prefill_qkv_w4a16(const qe_qkv_view* view, const uint16_t* input_x, int M,
                                     hipStream_t stream, int in_features, int num_q_heads,
                                     int num_kv_heads, int head_dim, int sm_count);

/* Replaces launch_gemm_prefill_dual_gate_up_swiglu_w4a16, include/kernels.cuh:144-153. */
int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16(const uint32_t* gate_up_qweight,
                                                     const uint16_t* gate_up_scales, const uint16_t* input_x,
                                                     uint16_t* output_mlp, int M, hipStream_t stream,
                                                     int hidden_size, int intermediate_size);

/* ---- prefill GEMM on a load-time copy of the weights in the tiled layout ----
 * No counterpart in the reference (its GEMM reads the .qwenbin layout).  The
 * tiled layout holds the same int4 weights and fp16 scales, reordered once so
 * that each 16-byte load of a wave reads 1 KB of contiguous memory: for every
 * 32 columns and 256-k quad g, 4 KB of weights as [i 0..3][h 0..1][c 0..31]
 * 16-byte chunks (chunk 8g + 4h + i of column c), and 64 fp16 scales as
 * [h][c] (group 2g + h of column c).  Columns are padded to a multiple of 32
 * (zeros), and each word holds its nibbles in the order the dequantization
 * reads fastest.  Requires K % 256 == 0.  For a given tile and K-slice plan
 * the results equal the .qwenbin-layout launchers' bit for bit; the plan
 * comes from a time model fitted to these kernels.  10-20 % faster on
 * MI355X at the Qwen2.5-1.5B shapes. */

/* Bytes of the tiled copy of an N x K matrix (weights, scales). */
int qe_w4_tiled_bytes(int N, int K, size_t* weight_bytes, size_t* scale_bytes);

/* Writes the tiled copy of qweight [N][K/8] / scales [N][K/128] (asynchronous
 * on `stream`; destinations of qe_w4_tiled_bytes' sizes, 16-byte aligned). */
int qe_repack_w4_tiled(const uint32_t* qweight, const uint16_t* scales, int N, int K, uint32_t* tiled_weight,
                       uint16_t* tiled_scales, hipStream_t stream);

/* qe_launch_gemm_prefill_w4a16 on tiled weights. */
int qe_launch_gemm_prefill_w4a16_tiled(const uint32_t* tiled_weight, const uint16_t* tiled_scales,
                                       const uint16_t* input_x, const uint16_t* residual, uint16_t* output_y, int M,
                                       int N, int K, hipStream_t stream);

/* qe_launch_gemm_prefill_qkv_w4a16 with the view's weights/scales tiled
 * (each of Q, K, V repacked on its own; q and kv widths multiples of 32). */
int qe_launch_gemm_prefill_qkv_w4a16_tiled(const qe_qkv_view* view, const uint16_t* input_x, int M,
                                           hipStream_t stream, int in_features, int num_q_heads, int num_kv_heads,
                                           int head_dim);

/* qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16 on the tiled copy of the
 * interleaved gate/up matrix (2 * intermediate_size columns). */
int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16_tiled(const uint32_t* tiled_weight, const uint16_t* tiled_scales,
                                                           const uint16_t* input_x, uint16_t* output_mlp, int M,
                                                           hipStream_t stream, int hidden_size,
                                                           int intermediate_size);

/* ---- greedy sampling ------------------------------------------------------ */

/* Replaces launch_sample_and_advance, include/kernels.cuh:209-217
 * (src/kernels/sampling.cu:60-232): argmax over the fp16 logits, or, when
 * the control block's temperature T > 1e-5, over logit / T plus Gumbel
 * noise -log(-log(u)) with u from Philox-4x32-10 keyed by rng_seed at
 * counter (index, seq_pos); lowest index on ties, NaN never wins; then
 * token_id = winner, seq_pos += 1, rng_seed += 0x9E3779B97F4A7C15.
 * sample_scratch_val/idx hold >= 256 entries. */
int qe_launch_sample_and_advance(const uint16_t* logits, float* sample_scratch_val,
                                 int32_t* sample_scratch_idx, qe_device_control_block* d_control,
                                 int32_t* d_mapped_pinned_token, hipStream_t stream, int vocab_size);

/* W4A8 prefill GEMM on the int8 matrix cores (v_mfma_i32_32x32x32_i8): the
 * activation rows enter as Q8_1 (input_q8 [M][K], input_scale [M][K/128],
 * input_sum8 [M][K/8], e.g. qe_launch_quantize_fp16_to_q8_1 over M*K
 * elements), so every output row is the W4A8 GEMV of that row
 * (gemv_w4a16.cu:74-121 math, integer group dots exact, fp32 scale and
 * accumulation, fp16 out; residual added as fp16(fp16(acc) + res) like the
 * fp16 GEMM).  The int8 prefill alternative named in design_draft.md:117-120
 * of the reference; no counterpart in its API.  K % 128 == 0, 16-byte
 * aligned Q8_1 rows and weights. */
int qe_launch_gemm_prefill_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                                const float* input_scale, const int32_t* input_sum8, const uint16_t* residual,
                                uint16_t* output_y, int M, int N, int K, hipStream_t stream);
int qe_launch_gemm_prefill_qkv_w4a8(const qe_qkv_view* view, const int8_t* input_q8, const float* input_scale,
                                    const int32_t* input_sum8, int M, hipStream_t stream, int in_features,
                                    int num_q_heads, int num_kv_heads, int head_dim);
int qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a8(const uint32_t* gate_up_qweight, const uint16_t* gate_up_scales,
                                                    const int8_t* input_q8, const float* input_scale,
                                                    const int32_t* input_sum8, uint16_t* output_mlp, int M,
                                                    hipStream_t stream, int hidden_size, int intermediate_size);

/* RMSNorm + QKV GEMV with the bias add, NeoX RoPE and KV-cache append in the
 * epilogue: the same results, bit for bit, as qe_launch_rmsnorm_gemv_qkv_w4a16
 * followed by qe_launch_qkv_bias_rope_kv_append for one token (GEMV output
 * rounded to fp16, bias added in fp16, rotation in fp32 at position
 * d_control->seq_pos), in one launch (src/engine.cu:367-385).  head_dim 128,
 * full rotation (rotary_dim 0 or 128), hidden_size <= 3072, 16-byte aligned
 * buffers; no counterpart in the reference (QE_ERR_UNSUPPORTED outside). */
int qe_launch_rmsnorm_gemv_qkv_rope_kv_append_w4a16(
    const uint16_t* input, const uint16_t* gamma, uint16_t* output_fp16_opt, const qe_qkv_view* view,
    const uint16_t* q_bias, const uint16_t* k_bias, const uint16_t* v_bias, uint16_t* layer_k_cache,
    uint16_t* layer_v_cache, const qe_device_control_block* d_control, hipStream_t stream, int hidden_size,
    int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len, int rotary_dim, float rope_theta);

/* Partials written by the fused LM-head + sampling launches: the sample
 * scratch of those two entry points holds at least this many entries (the
 * reference's launch_sample_and_advance needs 256). */
#define QE_LM_HEAD_SAMPLE_PARTS 2048

/* LM-head GEMV fused with the first sampling stage, then the second stage:
 * the same result as launch_gemv_w4a8 (logits, written when logits_opt is
 * not NULL) followed by launch_sample_and_advance
 * (src/engine.cu:437-447 -> src/kernels/sampling.cu:60-232), in two launches
 * instead of three and without reading the logits back.  The compared value
 * of index i is the fp16 logit, or logit / T + Gumbel(Philox(rng_seed, i,
 * seq_pos)) when the control block's temperature T > 1e-5; ties keep the
 * lowest index, NaN never wins; then token_id = winner, seq_pos += 1,
 * rng_seed += 0x9E3779B97F4A7C15.  Needs 16-byte aligned weights and
 * activations and in_features <= 16384 (QE_ERR_UNSUPPORTED otherwise). */
int qe_launch_gemv_lm_head_sample_w4a8(const uint32_t* qweight, const uint16_t* scales, const int8_t* input_q8,
                                       const float* input_scale, const int32_t* input_sum8, uint16_t* logits_opt,
                                       float* sample_scratch_val, int32_t* sample_scratch_idx,
                                       qe_device_control_block* d_control, int32_t* d_mapped_pinned_token,
                                       int vocab_size, int in_features, hipStream_t stream);

/* The same with the final RMSNorm (fp16 hidden state + gamma) quantized to
 * Q8_1 inside the launch, replacing launch_rmsnorm_q8_1 + the above
 * (src/engine.cu:433-447). */
int qe_launch_rmsnorm_gemv_lm_head_sample_w4a16(const uint16_t* input, const uint16_t* gamma,
                                                uint16_t* output_fp16_opt, const uint32_t* qweight,
                                                const uint16_t* scales, uint16_t* logits_opt,
                                                float* sample_scratch_val, int32_t* sample_scratch_idx,
                                                qe_device_control_block* d_control, int32_t* d_mapped_pinned_token,
                                                int vocab_size, int hidden_size, hipStream_t stream);

/* ---- decode-loop kernels around the matrix path ---------------------------- */

/* Replaces launch_embed_lookup_w4a16, include/kernels.cuh:11-20.  Token ids
 * from d_token_ids, else d_control->token_id; ids outside [0, 151936) read
 * row 0.  Rows are dequantized exactly as unpack_w4_to_half2_quad. */
int qe_launch_embed_lookup_w4a16(const uint32_t* embed_qweight, const uint16_t* embed_scales,
                                 const int32_t* d_token_ids, uint16_t* out_hidden,
                                 const qe_device_control_block* d_control, int num_tokens, hipStream_t stream,
                                 int hidden_size);

/* Replaces launch_qkv_bias_rope_kv_append, include/kernels.cuh:156-174. */
int qe_launch_qkv_bias_rope_kv_append(uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* q_bias,
                                      const uint16_t* k_bias, const uint16_t* v_bias, uint16_t* layer_k_cache,
                                      uint16_t* layer_v_cache, const qe_device_control_block* d_control,
                                      int num_tokens, hipStream_t stream, int num_q_heads, int num_kv_heads,
                                      int head_dim, int max_seq_len, int rotary_dim, float rope_theta);

/* Replaces launch_attention_gqa_flash_decode, include/kernels.cuh:177-193
 * (16 splits; head_dim 128).  With out_q8 != NULL the combine stage also
 * writes the Q8_1 of the attention output (one group per head): d =
 * max(max|acc|/127, 1e-8), q = clamp(rint(acc / d)), as
 * src/kernels/attention_gqa.cu:263-310. */
int qe_launch_attention_gqa_flash_decode(const uint16_t* q, const uint16_t* layer_k_cache,
                                         const uint16_t* layer_v_cache, float* splitk_partial_out,
                                         float* splitk_partial_lse, uint16_t* attn_out,
                                         const qe_device_control_block* d_control, hipStream_t stream,
                                         int num_q_heads, int num_kv_heads, int head_dim, int max_seq_len,
                                         int8_t* out_q8, float* out_scale, int32_t* out_sum8);

/* The combine stage alone (stage 2 of the flash decode plus the Q8_1
 * epilogue), over caller-provided split partials [head][16][128] and
 * (max, denominator) pairs [head][16][2].  No counterpart in the reference
 * API (the reference launches it only inside flash_decode). */
int qe_launch_attention_gqa_flash_decode_combine(const float* splitk_partial_out, const float* splitk_partial_lse,
                                                 uint16_t* attn_out, hipStream_t stream, int num_q_heads,
                                                 int8_t* out_q8, float* out_scale, int32_t* out_sum8);

/* Stage 1 of the flash decode alone: the 16 split partials of every q head
 * ([head][16][128] unnormalized outputs, [head][16][2] (max, denominator)),
 * src/kernels/attention_gqa.cu:20-228.  No separate entry point in the
 * reference API (its flash_decode launches stage 1 and stage 2 together);
 * it feeds qe_launch_attention_combine_gemv_o_w4a8. */
int qe_launch_attention_gqa_flash_decode_partials(const uint16_t* q, const uint16_t* layer_k_cache,
                                                  const uint16_t* layer_v_cache, float* splitk_partial_out,
                                                  float* splitk_partial_lse, const qe_device_control_block* d_control,
                                                  hipStream_t stream, int num_q_heads, int num_kv_heads, int head_dim,
                                                  int max_seq_len);

/* Flash-decode stage 2 + Q8_1 epilogue (src/kernels/attention_gqa.cu:230-310)
 * folded into the O projection's W4A8 GEMV (launch_gemv_w4a8 with residual,
 * include/kernels.cuh:88-97): y = fp16(W_o . Q8_1(combine(partials)) +
 * residual) in one launch, bit-identical to qe_launch_attention_gqa_flash_decode
 * followed by qe_launch_gemv_w4a8.  attn_out_opt (16-byte aligned) receives
 * the fp16 attention output when not NULL.  d_control (seq_pos) and
 * max_seq_len tell which splits hold positions: only the first 4, 8 or 16
 * splits' partials are read, the fewest that cover them (all 16 when
 * d_control is NULL).  head_dim 128, at most 16 q heads,
 * out_features rows.  No counterpart in the reference (a fusion of two of
 * its launches). */
int qe_launch_attention_combine_gemv_o_w4a8(const float* splitk_partial_out, const float* splitk_partial_lse,
                                            const uint32_t* o_qweight, const uint16_t* o_scales,
                                            const uint16_t* residual, uint16_t* output_y, uint16_t* attn_out_opt,
                                            const qe_device_control_block* d_control, int out_features,
                                            int num_q_heads, int head_dim, int max_seq_len, hipStream_t stream);

/* Replaces launch_attention_gqa_prefill, include/kernels.cuh:195-207. */
int qe_launch_attention_gqa_prefill(const uint16_t* q, const uint16_t* layer_k_cache, const uint16_t* layer_v_cache,
                                    uint16_t* attn_out, const qe_device_control_block* d_control, int num_tokens,
                                    hipStream_t stream, int num_q_heads, int num_kv_heads, int head_dim,
                                    int max_seq_len, int hidden_size);

/* ---- measurement ---------------------------------------------------------------- */

/* Reads `bytes` from `data` with the GEMV weight-stream access pattern
 * (16-byte nontemporal loads); `sink` receives nothing in practice (>= 16384
 * uint32).  Used by bench.py for the streaming ceiling and to scale
 * rocprofv3 FETCH_SIZE.  No counterpart in the reference. */
int qe_stream_read(const void* data, size_t bytes, uint32_t* sink, hipStream_t stream);

/* Process-wide tuning switches (no counterpart in the reference):
 *   "gemm_split_k" 0/1 (default 1) - split K across blocks for prefill GEMMs
 *   whose tile grid leaves CUs idle;
 *   "gemm_tile" 0..4 (default 0 = chosen per shape) - force the prefill GEMM
 *   block tile: 1 64x64, 2 64x128, 3 128x64, 4 128x128 (rows x columns);
 *   "gemm_slices" 0..64 (default 0 = chosen per shape) - force the number of
 *   K slices;
 *   "gemm_ks2" 0..2 (default 0) - prefill GEMMs with K % 256 == 0 split the k
 *   steps of a block over two groups of four waves: 0 when the grid has at
 *   most one block per CU, 1 never, 2 always;
 *   "gemv_block" 0, 256, 512, 1024 (default 0 = chosen per shape) - force the
 *   decode GEMV block size;
 *   "gemv_grid_cap" 0..65536 (default 0 = 8 blocks of 256 threads per CU) -
 *   largest decode GEMV grid; larger row counts loop over row sets;
 *   "engine_tiled_prefill" 0/1 (default 1) - engines created afterwards keep
 *   a tiled copy of every layer matrix (qe_repack_w4_tiled) for their prefill
 *   GEMMs (about 0.75 GB more for Qwen2.5-1.5B; same results).
 *   Returns QE_ERR_INVALID_ARGUMENT for an unknown key or value. */
int qe_set_tuning(const char* key, int value);

#ifdef __cplusplus
}
#endif

#endif
