/*
 * qwenbin.h — the .qwenbin v2 weight container read (and written) by this
 * build, byte-compatible with the reference's format: QwenBinHeaderV2 and
 * LayerDescriptor (include/config.cuh:107-172), as written by
 * tools/export_qwen25.py:218-419 (struct formats "<12I2f2I11Q" for the header
 * in a 4096-byte page and "<2I26Q" per 216-byte layer descriptor, every
 * tensor 256-byte aligned).  Offsets are absolute file offsets; tensors of
 * W4A16_G128 models are packed int4 uint32[N][K/8] plus fp16 scales
 * [N][K/128]; gate and up rows are interleaved in one matrix (2i gate,
 * 2i+1 up).
 */
#ifndef QE_QWENBIN_H
#define QE_QWENBIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QE_QWENBIN_MAGIC 0x5157454Eu /* "QWEN" */
#define QE_QWENBIN_QUANT_W4A16_G128 1u
#define QE_QWENBIN_LAYER_GQA 0u

/* QwenBinHeaderV2 (include/config.cuh:107-133). */
typedef struct qe_qwenbin_header {
    uint32_t magic;
    uint32_t version;
    uint32_t hidden_size;
    uint32_t intermediate_size;
    uint32_t num_layers;
    uint32_t num_attention_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t vocab_size;
    uint32_t max_seq_len;
    uint32_t quant_type;
    uint32_t tie_word_embeddings;
    float rms_norm_eps;
    float rope_theta;
    uint32_t reserved_flags;
    uint32_t padding0;
    uint64_t layer_table_offset;
    uint64_t embed_tokens_offset;
    uint64_t final_norm_offset;
    uint64_t lm_head_offset;
    uint64_t weights_offset;
    uint64_t reserved[6]; /* [0] embed scales, [1] untied lm_head scales */
} qe_qwenbin_header;

/* LayerDescriptor (include/config.cuh:135-172), 216 bytes. */
typedef struct qe_qwenbin_layer {
    uint32_t type;
    uint32_t reserved;
    uint64_t norm1_weight_offset;
    uint64_t norm2_weight_offset;
    uint64_t qkv_weight_offset; /* Q weight */
    uint64_t q_bias_offset;
    uint64_t k_bias_offset;
    uint64_t v_bias_offset;
    uint64_t attn_out_weight_offset;
    uint64_t reserved_deltanet[5];
    uint64_t mlp_gate_offset; /* interleaved gate/up weight */
    uint64_t mlp_up_offset;   /* == mlp_gate_offset */
    uint64_t mlp_down_offset;
    uint64_t quant_scales_offset;
    uint64_t quant_zeros_offset;
    uint64_t k_weight_offset;
    uint64_t v_weight_offset;
    uint64_t q_scale_offset;
    uint64_t k_scale_offset;
    uint64_t v_scale_offset;
    uint64_t attn_out_scale_offset;
    uint64_t mlp_gate_scale_offset;
    uint64_t mlp_up_scale_offset;
    uint64_t mlp_down_scale_offset;
} qe_qwenbin_layer;

/* What qe_qwenbin_inspect found in a valid container. */
typedef struct qe_qwenbin_info {
    uint32_t version;
    uint32_t quant_type;
    uint32_t tie_word_embeddings;
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t num_layers;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t vocab_size;
    int32_t max_seq_len;
    float rms_norm_eps;
    float rope_theta;
    uint64_t file_size;
    uint64_t weights_offset;
    uint64_t weights_bytes; /* file_size - weights_offset: the payload copied to the device */
} qe_qwenbin_info;

/* Map the file read-only and validate it for this build without touching a
 * GPU: magic, version 2, W4A16_G128, GQA layers, dimensions the kernels
 * support (hidden and intermediate multiples of 128, head_dim 128,
 * q_heads * head_dim == hidden), every tensor inside the file and 16-byte
 * aligned relative to weights_offset, gate and up interleaved in one matrix.
 * Returns QE_OK, QE_ERR_INVALID_ARGUMENT (malformed or truncated) or
 * QE_ERR_UNSUPPORTED (valid but outside this build, e.g. version 1 or FP16
 * weights); qe_last_error() names the failing field.  Replaces
 * QwenEngine::load_model_file (src/engine.cu:85-208) for version 2. */
int qe_qwenbin_inspect(const char* path, qe_qwenbin_info* info);

#ifdef __cplusplus
}  /* extern "C" */
static_assert(sizeof(qe_qwenbin_layer) == 216, "LayerDescriptor is 216 bytes");
static_assert(offsetof(qe_qwenbin_header, layer_table_offset) == 64, "header field offsets");
static_assert(offsetof(qe_qwenbin_header, reserved) == 104, "header field offsets");
static_assert(offsetof(qe_qwenbin_layer, mlp_gate_offset) == 104, "descriptor field offsets");
static_assert(offsetof(qe_qwenbin_layer, mlp_down_scale_offset) == 208, "descriptor field offsets");
#endif

#endif /* QE_QWENBIN_H */
