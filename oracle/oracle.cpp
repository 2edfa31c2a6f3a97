// CPU oracle for the W4A16 group-128 matrix path.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP library, loaded by the
// tests, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg.
// Nothing in the product path links or calls it.
//
// Citations are path:line in the reference tree (Areen-09/qwen-engine).
// Host arithmetic is plain IEEE binary32/binary64 (x86-64 SSE, no x87 excess
// precision); build flags exclude -ffast-math and FMA contraction
// (-ffp-contract=off) so that every float expression rounds as written.
#include "oracle.h"

#include <cmath>
#include <cstring>
#include <random>
#include <thread>
#include <vector>
#include <algorithm>

namespace {

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

inline double silu_times(double g, double u) { return g / (1.0 + std::exp(-g)) * u; }

inline uint16_t f64_to_f16(double v) { return oracle_f32_to_f16(static_cast<float>(v)); }

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// fp16 <-> fp32.  The reference converts with __half2float / __float2half
// (round-to-nearest-even), e.g. tests/test_kernels.cu:272,305,362.
// ---------------------------------------------------------------------------
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        // subnormal: man * 2^-24, exact in fp32
        float v = static_cast<float>(man) * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return static_cast<uint16_t>(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520 -> inf
    uint32_t e = ax >> 23;
    if (ax < 0x38800000u) {  // below 2^-14: fp16 subnormal or zero
        int shift = 126 - static_cast<int>(e);
        if (shift > 24) return static_cast<uint16_t>(sign);
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t res = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (res & 1u))) ++res;
        return static_cast<uint16_t>(sign | res);
    }
    uint32_t res = ((e - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (res & 1u))) ++res;
    return static_cast<uint16_t>(sign | res);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

// ---------------------------------------------------------------------------
// Q8_1 group-128 quantizer.
// Follows the CPU golden tests/test_kernels.cu:311-326: d = max(max|x|/127, 1e-8)
// with IEEE division, inv_d = 1/d, q = clamp(std::round(x*inv_d), -127, 127)
// (round half away from zero).  sum8 = -8 * sum of 8 consecutive q
// (include/quant_primitives.cuh:10-17, 81-84), scale stored as fp32 per group.
// ---------------------------------------------------------------------------
void oracle_quantize_q8_1_f32(const float* x, int K, int8_t* q8, float* scale, int32_t* sum8) {
    int G = K / 128;
    for (int g = 0; g < G; ++g) {
        float max_abs = 0.0f;
        for (int j = 0; j < 128; ++j) {
            float v = std::fabs(x[g * 128 + j]);
            if (v > max_abs) max_abs = v;
        }
        float d = std::max(max_abs / 127.0f, 1e-8f);
        float inv_d = 1.0f / d;
        if (scale) scale[g] = d;
        for (int j = 0; j < 128; ++j) {
            float val = x[g * 128 + j] * inv_d;
            int v = static_cast<int>(std::round(val));
            v = std::max(-127, std::min(127, v));
            q8[g * 128 + j] = static_cast<int8_t>(v);
        }
        if (sum8) {
            for (int w = 0; w < 16; ++w) {
                int32_t s = 0;
                for (int j = 0; j < 8; ++j) s += q8[g * 128 + w * 8 + j];
                sum8[g * 16 + w] = -8 * s;
            }
        }
    }
}

void oracle_quantize_q8_1(const uint16_t* x, int K, int8_t* q8, float* scale, int32_t* sum8) {
    std::vector<float> xf(K);
    oracle_f16_to_f32_array(x, xf.data(), K);
    oracle_quantize_q8_1_f32(xf.data(), K, q8, scale, sum8);
}

// Flash-decode stage-2 epilogue, src/kernels/attention_gqa.cu:260-310:
// attn_out = fp16(acc); per head d = max(max|acc|/127, 1e-8);
// q = clamp(rn(acc / d)) (division, round-half-even as __float2int_rn);
// sum8 over 8 adjacent elements; scale index = head.
void oracle_quantize_q8_1_attn(const float* acc, int num_heads, int head_dim,
                               uint16_t* attn_out, int8_t* q8, float* scale, int32_t* sum8) {
    for (int h = 0; h < num_heads; ++h) {
        const float* a = acc + static_cast<size_t>(h) * head_dim;
        float b_max = 0.0f;
        for (int i = 0; i < head_dim; ++i) b_max = std::max(b_max, std::fabs(a[i]));
        float d = std::max(b_max / 127.0f, 1e-8f);
        if (scale) scale[h] = d;
        for (int i = 0; i < head_dim; ++i) {
            if (attn_out) attn_out[h * head_dim + i] = oracle_f32_to_f16(a[i]);
            float r = std::nearbyint(a[i] / d);  // default FE_TONEAREST: ties to even
            int v = static_cast<int>(r);
            v = std::max(-127, std::min(127, v));
            q8[h * head_dim + i] = static_cast<int8_t>(v);
        }
        if (sum8) {
            for (int w = 0; w < head_dim / 8; ++w) {
                int32_t s = 0;
                for (int j = 0; j < 8; ++j) s += q8[h * head_dim + w * 8 + j];
                sum8[h * (head_dim / 8) + w] = -8 * s;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Nibble layout, include/quant_primitives.cuh:20-24 and tools/export_qwen25.py:72:
// word = q0 | q4<<4 | q1<<8 | q5<<12 | q2<<16 | q6<<20 | q3<<24 | q7<<28,
// element 8w+j of a row is q_j of word w.
// ---------------------------------------------------------------------------
void oracle_unpack_w4(uint32_t p, int32_t q[8]) {
    for (int j = 0; j < 4; ++j) {
        q[j] = static_cast<int32_t>((p >> (8 * j)) & 0xfu);
        q[j + 4] = static_cast<int32_t>((p >> (8 * j + 4)) & 0xfu);
    }
}

uint32_t oracle_pack_w4(const int32_t q[8]) {
    uint32_t p = 0;
    for (int j = 0; j < 4; ++j) {
        p |= (static_cast<uint32_t>(q[j]) & 0xfu) << (8 * j);
        p |= (static_cast<uint32_t>(q[j + 4]) & 0xfu) << (8 * j + 4);
    }
    return p;
}

// unpack_w4_to_half2_quad, include/quant_primitives.cuh:92-115: (q-8) is exact
// in fp16, then one fp16 multiply by the group scale (RNE).
void oracle_dequant_w4_f16(const uint32_t* qw, const uint16_t* scales, int N, int K, uint16_t* out) {
    int G = K / 128;
    for (int n = 0; n < N; ++n) {
        for (int w = 0; w < K / 8; ++w) {
            int32_t q[8];
            oracle_unpack_w4(qw[static_cast<size_t>(n) * (K / 8) + w], q);
            float s = oracle_f16_to_f32(scales[static_cast<size_t>(n) * G + (w * 8) / 128]);
            for (int j = 0; j < 8; ++j) {
                // product of an integer in [-8,7] and an fp16 value is exact in fp32
                out[static_cast<size_t>(n) * K + w * 8 + j] =
                    oracle_f32_to_f16(static_cast<float>(q[j] - 8) * s);
            }
        }
    }
}

// dp4a_w4_q8_oct, include/quant_primitives.cuh:28-32, chained over the 16
// words of a group: sum_w (sum8[w] + sum_j q_j * x_j).
static inline int32_t group_dot(const uint32_t* row_qw, const int8_t* q8, const int32_t* sum8, int g) {
    int32_t dot = 0;
    for (int w = 0; w < 16; ++w) {
        int32_t q[8];
        oracle_unpack_w4(row_qw[g * 16 + w], q);
        int32_t acc = sum8[g * 16 + w];
        for (int j = 0; j < 8; ++j) acc += q[j] * static_cast<int32_t>(q8[g * 128 + w * 8 + j]);
        dot += acc;
    }
    return dot;
}

void oracle_group_dots(const uint32_t* qw, const int8_t* q8, const int32_t* sum8,
                       int N, int K, int32_t* out) {
    int G = K / 128;
    for (int n = 0; n < N; ++n)
        for (int g = 0; g < G; ++g)
            out[static_cast<size_t>(n) * G + g] = group_dot(qw + static_cast<size_t>(n) * (K / 8), q8, sum8, g);
}

// Row evaluation of the CPU golden, tests/test_kernels.cu:330-357:
// acc(double) += group_dot * (double)(float)(w_scale * x_scale).
static double eval_row(const uint32_t* qw, const uint16_t* scales, const int8_t* q8,
                       const float* xs, const int32_t* sum8, int row, int K, double* bound) {
    int G = K / 128;
    const uint32_t* row_qw = qw + static_cast<size_t>(row) * (K / 8);
    const uint16_t* row_sc = scales + static_cast<size_t>(row) * G;
    double acc = 0.0, b = 0.0;
    for (int g = 0; g < G; ++g) {
        float w_sc = oracle_f16_to_f32(row_sc[g]);
        float group_factor = w_sc * xs[g];
        int32_t dot = group_dot(row_qw, q8, sum8, g);
        double t = static_cast<double>(dot) * static_cast<double>(group_factor);
        acc += t;
        b += std::fabs(t);
    }
    if (bound) *bound = b;
    return acc;
}

void oracle_gemv_w4a8(const uint32_t* qw, const uint16_t* scales,
                      const int8_t* q8, const float* xs, const int32_t* sum8,
                      const uint16_t* residual, uint16_t* y, int N, int K,
                      double* y_exact, double* abs_bound) {
    // src/kernels/gemv_w4a16.cu:116-120: optional fp16 residual added before rounding.
    for (int n = 0; n < N; ++n) {
        double b = 0.0;
        double acc = eval_row(qw, scales, q8, xs, sum8, n, K, &b);
        if (residual) {
            double r = oracle_f16_to_f32(residual[n]);
            acc += r;
            b += std::fabs(r);
        }
        y[n] = f64_to_f16(acc);
        if (y_exact) y_exact[n] = acc;
        if (abs_bound) abs_bound[n] = b;
    }
}

void oracle_gemv_swiglu_w4a8(const uint32_t* qw, const uint16_t* scales,
                             const int8_t* q8, const float* xs, const int32_t* sum8,
                             uint16_t* out, int K, int I, double* out_exact, double* abs_bound) {
    // tests/test_kernels.cu:359-362: gate row 2r, up row 2r+1, silu in double.
    for (int r = 0; r < I; ++r) {
        double bg = 0.0, bu = 0.0;
        double g = eval_row(qw, scales, q8, xs, sum8, 2 * r, K, &bg);
        double u = eval_row(qw, scales, q8, xs, sum8, 2 * r + 1, K, &bu);
        double v = silu_times(g, u);
        out[r] = f64_to_f16(v);
        if (out_exact) out_exact[r] = v;
        // |d(silu(g)u)| <= |u|*|dg|*1.1 + |silu(g)|*|du|
        if (abs_bound) abs_bound[r] = 1.1 * std::fabs(u) * bg + std::fabs(g) * bu;
    }
}

// The same rows split over `threads` host threads (contiguous row ranges):
// the multi-core form of the CPU golden, for the bench's CPU baseline.
void oracle_gemv_swiglu_w4a8_mt(const uint32_t* qw, const uint16_t* scales, const int8_t* q8, const float* xs,
                                const int32_t* sum8, uint16_t* out, int K, int I, int threads) {
    if (threads < 1) threads = 1;
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        const int r0 = static_cast<int>(static_cast<long long>(I) * t / threads);
        const int r1 = static_cast<int>(static_cast<long long>(I) * (t + 1) / threads);
        pool.emplace_back([=] {
            for (int r = r0; r < r1; ++r) {
                double bg = 0.0, bu = 0.0;
                const double g = eval_row(qw, scales, q8, xs, sum8, 2 * r, K, &bg);
                const double u = eval_row(qw, scales, q8, xs, sum8, 2 * r + 1, K, &bu);
                out[r] = f64_to_f16(silu_times(g, u));
            }
        });
    }
    for (auto& th : pool) th.join();
}

void oracle_gemv_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* x,
                       const uint16_t* residual, uint16_t* y, int N, int K,
                       double* y_exact, double* abs_bound) {
    std::vector<int8_t> q8(K);
    std::vector<float> xs(K / 128);
    std::vector<int32_t> s8(K / 8);
    oracle_quantize_q8_1(x, K, q8.data(), xs.data(), s8.data());
    oracle_gemv_w4a8(qw, scales, q8.data(), xs.data(), s8.data(), residual, y, N, K, y_exact, abs_bound);
}

void oracle_gemv_swiglu_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* x,
                              uint16_t* out, int K, int I, double* out_exact, double* abs_bound) {
    std::vector<int8_t> q8(K);
    std::vector<float> xs(K / 128);
    std::vector<int32_t> s8(K / 8);
    oracle_quantize_q8_1(x, K, q8.data(), xs.data(), s8.data());
    oracle_gemv_swiglu_w4a8(qw, scales, q8.data(), xs.data(), s8.data(), out, K, I, out_exact, abs_bound);
}

// ---------------------------------------------------------------------------
// Prefill dequant-GEMM, src/kernels/gemm_prefill.cu:319-386 (math) and the
// epilogue :261-275: out = fp16(acc), residual added as an fp16 add.
// ---------------------------------------------------------------------------
static void gemm_acc(const uint32_t* qw, const uint16_t* scales, const uint16_t* A,
                     int M, int N, int K, std::vector<double>& acc, std::vector<double>& bnd) {
    std::vector<uint16_t> wdq(static_cast<size_t>(N) * K);
    oracle_dequant_w4_f16(qw, scales, N, K, wdq.data());
    std::vector<float> wf(static_cast<size_t>(N) * K), af(static_cast<size_t>(M) * K);
    oracle_f16_to_f32_array(wdq.data(), wf.data(), static_cast<int64_t>(N) * K);
    oracle_f16_to_f32_array(A, af.data(), static_cast<int64_t>(M) * K);
    acc.assign(static_cast<size_t>(M) * N, 0.0);
    bnd.assign(static_cast<size_t>(M) * N, 0.0);
    for (int m = 0; m < M; ++m) {
        const float* a = af.data() + static_cast<size_t>(m) * K;
        for (int n = 0; n < N; ++n) {
            const float* w = wf.data() + static_cast<size_t>(n) * K;
            double s = 0.0, b = 0.0;
            for (int k = 0; k < K; ++k) {
                double t = static_cast<double>(a[k]) * static_cast<double>(w[k]);
                s += t;
                b += std::fabs(t);
            }
            acc[static_cast<size_t>(m) * N + n] = s;
            bnd[static_cast<size_t>(m) * N + n] = b;
        }
    }
}

void oracle_gemm_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* A,
                       const uint16_t* residual, uint16_t* y, int M, int N, int K,
                       double* y_exact, double* abs_bound) {
    std::vector<double> acc, bnd;
    gemm_acc(qw, scales, A, M, N, K, acc, bnd);
    for (size_t i = 0; i < acc.size(); ++i) {
        uint16_t h = f64_to_f16(acc[i]);
        if (residual) {
            float s = oracle_f16_to_f32(h) + oracle_f16_to_f32(residual[i]);  // exact in fp32
            h = oracle_f32_to_f16(s);
        }
        y[i] = h;
        if (y_exact) y_exact[i] = acc[i] + (residual ? oracle_f16_to_f32(residual[i]) : 0.0);
        if (abs_bound) abs_bound[i] = bnd[i];
    }
}

// src/kernels/gemm_prefill.cu:559-609: columns (2p, 2p+1) = (gate, up).
void oracle_gemm_swiglu_w4a16(const uint32_t* qw, const uint16_t* scales, const uint16_t* A,
                              uint16_t* out, int M, int K, int I,
                              double* out_exact, double* abs_bound) {
    std::vector<double> acc, bnd;
    gemm_acc(qw, scales, A, M, 2 * I, K, acc, bnd);
    for (int m = 0; m < M; ++m) {
        for (int i = 0; i < I; ++i) {
            size_t c = static_cast<size_t>(m) * 2 * I + 2 * i;
            double g = acc[c], u = acc[c + 1];
            double v = silu_times(g, u);
            out[static_cast<size_t>(m) * I + i] = f64_to_f16(v);
            if (out_exact) out_exact[static_cast<size_t>(m) * I + i] = v;
            if (abs_bound) abs_bound[static_cast<size_t>(m) * I + i] = 1.1 * std::fabs(u) * bnd[c] + std::fabs(g) * bnd[c + 1];
        }
    }
}

// ---------------------------------------------------------------------------
// RMSNorm, src/kernels/rmsnorm_rope.cu:75-138 and :214-232:
// inv_rms = 1/sqrt(mean(x^2) + eps), h = fp16(inv_rms),
// out = fp16(fp16(x*h) * gamma)  (two __hmul2).
// ---------------------------------------------------------------------------
void oracle_rmsnorm_fp16(const uint16_t* x, const uint16_t* gamma, uint16_t* out,
                         int num_tokens, int H, float eps) {
    for (int t = 0; t < num_tokens; ++t) {
        const uint16_t* xr = x + static_cast<size_t>(t) * H;
        double ss = 0.0;
        for (int i = 0; i < H; ++i) {
            double v = oracle_f16_to_f32(xr[i]);
            ss += v * v;
        }
        float mean = static_cast<float>(ss) / static_cast<float>(H);
        float inv_rms = 1.0f / std::sqrt(mean + eps);
        float h = oracle_f16_to_f32(oracle_f32_to_f16(inv_rms));
        for (int i = 0; i < H; ++i) {
            float n1 = oracle_f16_to_f32(oracle_f32_to_f16(oracle_f16_to_f32(xr[i]) * h));
            out[static_cast<size_t>(t) * H + i] = oracle_f32_to_f16(n1 * oracle_f16_to_f32(gamma[i]));
        }
    }
}

// ---------------------------------------------------------------------------
// Greedy argmax, src/kernels/sampling.cu:77-105 and :159-205 (temperature 0).
// ---------------------------------------------------------------------------
int32_t oracle_argmax_f16(const uint16_t* logits, int n) {
    float best = -1e30f;
    int32_t idx = 0;
    for (int i = 0; i < n; ++i) {
        float v = oracle_f16_to_f32(logits[i]);
        if (v > best) { best = v; idx = i; }
    }
    return idx;
}

// ---------------------------------------------------------------------------
// Temperature sampling, src/kernels/sampling.cu:13-53 and :60-105: Philox-4x32-10
// (Salmon et al., SC'11; multipliers 0xD2511F53 / 0xCD9E8D57, key bumps
// 0x9E3779B9 / 0xBB67AE85) with counter (subsequence, offset, 0, 0) and key
// (seed lo, seed hi); u = clamp((float(ctr0) + 1) / 4294967298.0f, 1e-7,
// 1 - 1e-7); value = logit / temperature - log(-log(u)); argmax as greedy.
// ---------------------------------------------------------------------------
void oracle_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = 0xD2511F53ull * c0;
        const uint64_t p1 = 0xCD9E8D57ull * c2;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = static_cast<uint32_t>(p1);
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = static_cast<uint32_t>(p0);
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float oracle_philox_uniform(uint64_t seed, uint32_t subsequence, uint32_t offset) {
    const uint32_t ctr[4] = {subsequence, offset, 0u, 0u};
    const uint32_t key[2] = {static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)};
    uint32_t o[4];
    oracle_philox4x32_10(ctr, key, o);
    const float u = (static_cast<float>(o[0]) + 1.0f) / 4294967298.0f;
    return std::fmin(std::fmax(u, 1e-7f), 1.0f - 1e-7f);
}

int32_t oracle_sample_f16(const uint16_t* logits, int n, float temperature, uint64_t seed, uint32_t seq_pos,
                          float* out_values) {
    float best = -1e30f;
    int32_t idx = 0;
    for (int i = 0; i < n; ++i) {
        float v = oracle_f16_to_f32(logits[i]);
        if (temperature > 1e-5f) {
            const float u = oracle_philox_uniform(seed, static_cast<uint32_t>(i), seq_pos);
            v = v / temperature + -std::log(-std::log(u));
        }
        if (out_values) out_values[i] = v;
        if (v > best) { best = v; idx = i; }
    }
    return idx;
}

// ---------------------------------------------------------------------------
// Synthetic inputs.
// ---------------------------------------------------------------------------
// Generator of tests/test_kernels.cu:265-306 (libstdc++ distributions).
void oracle_suite3_inputs(int H, int I, uint16_t* x, uint32_t* qw, uint16_t* scales) {
    std::mt19937 gen(42 + H);
    float scale_factor = 1.0f / std::sqrt(static_cast<float>(H));
    std::uniform_real_distribution<float> dis_x(-scale_factor, scale_factor);
    for (int i = 0; i < H; ++i) x[i] = oracle_f32_to_f16(dis_x(gen));
    size_t num_qwords = static_cast<size_t>(2 * I) * (H / 8);
    size_t num_scales = static_cast<size_t>(2 * I) * (H / 128);
    std::uniform_int_distribution<int> dis_nibble(2, 14);
    for (size_t i = 0; i < num_qwords; ++i) {
        int32_t q[8];
        q[0] = dis_nibble(gen); q[1] = dis_nibble(gen); q[2] = dis_nibble(gen); q[3] = dis_nibble(gen);
        q[4] = dis_nibble(gen); q[5] = dis_nibble(gen); q[6] = dis_nibble(gen); q[7] = dis_nibble(gen);
        qw[i] = oracle_pack_w4(q);
    }
    uint16_t sc = oracle_f32_to_f16(0.05f * scale_factor);
    for (size_t i = 0; i < num_scales; ++i) scales[i] = sc;
}

static inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline double normal_from(uint64_t& s) {
    // Box-Muller on two 53-bit uniforms in (0,1]
    double u1 = (static_cast<double>(splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    double u2 = static_cast<double>(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

void oracle_synth_w4(uint64_t seed, int N, int K, uint32_t* qw, uint16_t* scales) {
    uint64_t s = seed;
    size_t nw = static_cast<size_t>(N) * (K / 8);
    for (size_t i = 0; i < nw; i += 2) {
        uint64_t r = splitmix64(s);
        qw[i] = static_cast<uint32_t>(r);
        if (i + 1 < nw) qw[i + 1] = static_cast<uint32_t>(r >> 32);
    }
    size_t ns = static_cast<size_t>(N) * (K / 128);
    for (size_t i = 0; i < ns; ++i)
        scales[i] = oracle_f32_to_f16(static_cast<float>(std::fabs(normal_from(s)) * 0.02));
}

void oracle_synth_f16_normal(uint64_t seed, int64_t n, uint16_t* x) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; ++i) x[i] = oracle_f32_to_f16(static_cast<float>(normal_from(s)));
}

}  // extern "C"
