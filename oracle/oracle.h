/*
 * CPU oracle for the W4A16 group-128 matrix path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only the tests,
 * the smoke entry (__graft_entry__.smoke) and the cpu_baseline leg of
 * bench.py may load it.  The product path (libqe_amd.so) never links or
 * calls it, and there is no CPU fallback built on it.
 *
 * fp16 values cross this interface as uint16_t bit patterns.
 * Every function restates a piece of the reference (Areen-09/qwen-engine);
 * the citation is on the definition in oracle.cpp.
 */
#ifndef QE_ORACLE_H
#define QE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 <-> fp32, IEEE round-to-nearest-even (host __float2half semantics). */
float    oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void     oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n);
void     oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);

/* Q8_1 group-128 quantizer of the reference CPU golden. */
void oracle_quantize_q8_1(const uint16_t* x, int K, int8_t* q8, float* scale, int32_t* sum8);
/* Same quantizer on fp32 input (used for the fp16-rounded RMSNorm output). */
void oracle_quantize_q8_1_f32(const float* x, int K, int8_t* q8, float* scale, int32_t* sum8);
/* Flash-decode epilogue quantizer: one group per head, q = rint(acc / d). */
void oracle_quantize_q8_1_attn(const float* acc, int num_heads, int head_dim,
                               uint16_t* attn_out, int8_t* q8, float* scale, int32_t* sum8);

/* Packed W4 word helpers (nibble layout of the .qwenbin weights). */
void     oracle_unpack_w4(uint32_t packed, int32_t q[8]);
uint32_t oracle_pack_w4(const int32_t q[8]);
/* dequantized fp16 weights: out[n*K+k] = fp16((q-8) * s) */
void oracle_dequant_w4_f16(const uint32_t* qw, const uint16_t* scales, int N, int K, uint16_t* out);

/* Integer part of the W4A8 dot: per group g, sum over the group of the
 * 8-element dp4a chains seeded with sum8.  out[n*G+g]. */
void oracle_group_dots(const uint32_t* qw, const int8_t* q8, const int32_t* sum8,
                       int N, int K, int32_t* out);

/* W4A8 GEMV: y[n] = fp16( sum_g dot[n,g] * (float)(s[n,g]*xs[g]) [+ res[n]] ),
 * double accumulation.  y_exact (optional) receives the double value before
 * rounding, abs_bound (optional) sum_g |dot*factor| (for tolerance). */
void oracle_gemv_w4a8(const uint32_t* qw, const uint16_t* scales,
                      const int8_t* q8, const float* xs, const int32_t* sum8,
                      const uint16_t* residual, uint16_t* y, int N, int K,
                      double* y_exact, double* abs_bound);
/* Fused gate/up (rows 2i, 2i+1) + SwiGLU: out[i] = fp16(silu(g)*u). */
void oracle_gemv_swiglu_w4a8(const uint32_t* qw, const uint16_t* scales,
                             const int8_t* q8, const float* xs, const int32_t* sum8,
                             uint16_t* out, int K, int I, double* out_exact, double* abs_bound);
/* W4A16 entry points: quantize x, then the W4A8 math. */
void oracle_gemv_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* x,
                       const uint16_t* residual, uint16_t* y, int N, int K,
                       double* y_exact, double* abs_bound);
void oracle_gemv_swiglu_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* x,
                              uint16_t* out, int K, int I, double* out_exact, double* abs_bound);

/* Prefill dequant-GEMM: acc[m,n] = sum_k A[m,k]*Wdq[n,k] (double);
 * y = fp16(acc), residual added as fp16(fp16(acc)+res) (vector epilogue). */
void oracle_gemm_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* A,
                       const uint16_t* residual, uint16_t* y, int M, int N, int K,
                       double* y_exact, double* abs_bound);
void oracle_gemm_swiglu_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* A,
                              uint16_t* out, int M, int K, int I,
                              double* out_exact, double* abs_bound);

/* oracle_gemv_swiglu_w4a8's fp16 outputs computed by `threads` host threads. */
void oracle_gemv_swiglu_w4a8_mt(const uint32_t* qw, const uint16_t* scales, const int8_t* q8, const float* xs,
                                const int32_t* sum8, uint16_t* out, int K, int I, int threads);

/* RMSNorm of the reference kernels: fp16(fp16(x * fp16(inv_rms)) * gamma). */
void oracle_rmsnorm_fp16(const uint16_t* x, const uint16_t* gamma, uint16_t* out,
                         int num_tokens, int H, float eps);

/* Greedy argmax over fp16 logits: strict '>', lowest index on ties,
 * NaN never wins, floor -1e30 with default index 0. */
int32_t oracle_argmax_f16(const uint16_t* logits, int n);

/* Philox-4x32-10 block (10 rounds, key bumped after each round). */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* Uniform of sampling.cu: counter (subsequence, offset, 0, 0), key = seed. */
float oracle_philox_uniform(uint64_t seed, uint32_t subsequence, uint32_t offset);
/* sample_stage1/2 of sampling.cu: Gumbel-max over logit/temperature when
 * temperature > 1e-5, else greedy; out_values (optional) gets the compared
 * value of every index. */
int32_t oracle_sample_f16(const uint16_t* logits, int n, float temperature, uint64_t seed, uint32_t seq_pos,
                          float* out_values);

/* Inputs of the reference's synthetic SwiGLU suite (std::mt19937(42+H)):
 * x[H] fp16, qw[2I*H/8], scales[2I*H/128] fp16. */
void oracle_suite3_inputs(int H, int I, uint16_t* x, uint32_t* qw, uint16_t* scales);

/* Seeded synthetic W4 G128 weights of the benchmark configs:
 * nibbles uniform in [0,15], scales fp16(|N(0,1)|*0.02). */
void oracle_synth_w4(uint64_t seed, int N, int K, uint32_t* qw, uint16_t* scales);
/* fp16 ~N(0,1) vector. */
void oracle_synth_f16_normal(uint64_t seed, int64_t n, uint16_t* x);

#ifdef __cplusplus
}
#endif

#endif
