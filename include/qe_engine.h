/*
 * qe_engine.h — C-ABI of the minimal Qwen2.5-style decode engine built on the
 * W4A16 G128 path.  Weights are either random-initialized on the device in
 * the packed .qwenbin layout (uint32 [N][K/8] nibbles, fp16 [N][K/128]
 * scales, LM head tied to the embedding) or loaded from a .qwenbin v2 file
 * (include/qwenbin.h).  One engine = one HIP stream, one device arena
 * (allocated at create), one captured decode graph.  Besides the weights
 * (or the .qwenbin payload, one device copy), the KV cache and the
 * activations, the arena holds a 32 MiB split-K workspace for the prefill
 * GEMMs (registered for the engine's stream) and, unless
 * qe_set_tuning("engine_tiled_prefill", 0) was set before create, a tiled
 * copy of every layer matrix for the prefill GEMMs (+0.75 GB at
 * Qwen2.5-1.5B: about 0.8x the layer weights).  The switch is read once at
 * create.  qe_engine_arena_spans reports the arena's size.
 *
 * Counterpart of the reference's QwenEngine (include/engine.cuh:104-226):
 * construction from a .qwenbin (load_model_file + setup_arena), prefill
 * (:prefill), decode_step (:decode_step) and profile_stages.  Session
 * leasing, rollback and prefix reuse are not part of this build.
 */
#ifndef QE_ENGINE_H
#define QE_ENGINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qe_engine qe_engine;

typedef struct qe_engine_config {
    int num_layers;         /* 28 */
    int hidden_size;        /* 1536 */
    int intermediate_size;  /* 8960 */
    int num_q_heads;        /* 12 */
    int num_kv_heads;       /* 2 */
    int head_dim;           /* 128 (the only value built) */
    int vocab_size;         /* 151936 */
    int max_seq_len;        /* 4096 */
    float rope_theta;       /* 1e6 */
    int prefill_chunk;      /* tokens per prefill chunk */
    int fused_decode;       /* 1: fused RMSNorm/quantize launches, 0: reference launch sequence */
} qe_engine_config;

/* Qwen2.5-1.5B dimensions. */
void qe_engine_default_config(qe_engine_config* cfg);

/* Allocate, random-initialize (seeded) and capture the decode graph. */
int qe_engine_create(const qe_engine_config* cfg, uint64_t seed, qe_engine** out);
void qe_engine_destroy(qe_engine* e);

/* Build an engine from a .qwenbin v2 file (QwenEngine::QwenEngine ->
 * load_model_file + setup_arena, src/engine.cu:85-348): the file is validated
 * as qe_qwenbin_inspect does, its payload [weights_offset, end) is copied to
 * the device once and every tensor is addressed by its offset; an untied
 * lm_head is used when present.  max_seq_len: 0 takes the file's (4096 when
 * the file's is 0 or above 32768), otherwise capped by the file's.
 * prefill_chunk 0 means 1024.  The reference also requires the exact
 * Qwen2.5-1.5B dimensions; this build accepts any the kernels support. */
int qe_engine_create_from_qwenbin(const char* path, int max_seq_len, int prefill_chunk, int fused_decode,
                                  qe_engine** out);

/* Write the engine's weights as a .qwenbin v2 file in the layout of the
 * reference's exporter (tools/export_qwen25.py:218-419): 4096-byte header,
 * layer table at 4096, 256-byte aligned tensors. */
int qe_engine_save_qwenbin(qe_engine* e, const char* path);

/* Position 0, token 0 (the KV cache is overwritten as positions advance). */
int qe_engine_reset(qe_engine* e);

/* Prefill n host tokens from position 0; *first_token receives the greedy
 * next token.  Fails if n >= max_seq_len. */
int qe_engine_prefill(qe_engine* e, const int32_t* tokens, int n, int32_t* first_token);

/* n greedy decode steps (graph replay when use_graph != 0, else eager
 * launches).  tokens[i] and step_ms[i] (hipEvent time of step i) are
 * optional host arrays. */
int qe_engine_decode(qe_engine* e, int n_steps, int use_graph, int32_t* tokens, float* step_ms);

/* One eager decode step with events between launches: stage_ms[0] GEMV
 * (projections + LM head), [1] attention, [2] other, [3] total. */
int qe_engine_profile_decode(qe_engine* e, float* stage_ms);

/* Next position to be written (tokens processed so far). */
int qe_engine_seq_pos(const qe_engine* e);

/* Device pointers of the last logits (fp16 [vocab]) and of the residual
 * stream (fp16 [prefill_chunk][hidden]; row 0 after a decode step). */
const uint16_t* qe_engine_logits(const qe_engine* e);
const uint16_t* qe_engine_hidden(const qe_engine* e);

/* Synchronize the engine's stream and copy the first n fp16 values of the
 * logits / residual stream to host memory. */
int qe_engine_read_logits(qe_engine* e, uint16_t* host, int n);
int qe_engine_read_hidden(qe_engine* e, uint16_t* host, int n);

/* Synchronize and copy the first `bytes` of a named engine buffer to host
 * memory: "logits", "hidden", "q8", "q8_scale", "q8_sum8", "embed_w",
 * "embed_s", "lm_head_w", "lm_head_s", "final_norm", "control", or a layer
 * tensor "layer<l>.<t>" with t one of ln1 ln2 q_w q_s k_w k_s v_w v_s o_w o_s
 * gate_up_w gate_up_s down_w down_s q_bias k_bias v_bias. */
int qe_engine_read_buffer(qe_engine* e, const char* name, void* host, size_t bytes);

/* The arena layout: every buffer the engine carved out of its one device
 * allocation, in allocation order, as (offset, bytes) pairs; *count receives
 * the number of buffers (at most `capacity` are written), *arena_bytes the
 * allocation's size.  For layout checks like the reference's scratch
 * non-overlap test (tests/test_kernels.cu:687-705); host only. */
int qe_engine_arena_spans(const qe_engine* e, size_t* offsets, size_t* sizes, int capacity, int* count,
                          size_t* arena_bytes);

#ifdef __cplusplus
}
#endif

#endif
