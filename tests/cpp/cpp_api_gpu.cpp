// GPU check of the C++ drop-in API (kernels.hpp): a host program in the style
// of the reference's engine (hipMalloc'd buffers, one stream, the qwen::
// launchers with their default arguments) runs the matrix path on inputs read
// from a file and writes the outputs back; tests/test_gpu_cpp_api.py compares
// them with the CPU oracle.
//
// usage: cpp_api_gpu <in.bin> <out.bin>
//        cpp_api_gpu --wrappers   (every other qwen:: launcher against its C-ABI
//                                  function on the same inputs, bit for bit)
//   in.bin : K=1536, N=2048, M=64 inputs - x fp16[K], gamma fp16[K], weights
//            uint32[N][K/8], scales fp16[N][K/128], A fp16[M][K]
//   out.bin: q8 int8[K], scale f32[K/128], sum8 i32[K/8] (rmsnorm_q8_1 of x),
//            y_w4a8 fp16[N] (on that Q8_1), y_w4a16 fp16[N] (on x),
//            qkv fp16[1536 + 256 + 256] (QKV view over the same matrix),
//            gemm fp16[M][N]
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "kernels.hpp"

#define CHECK(x)                                                                         \
    do {                                                                                 \
        hipError_t e_ = (x);                                                             \
        if (e_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                 \
            std::exit(2);                                                                \
        }                                                                                \
    } while (0)

template <class T>
T* upload(const std::vector<char>& blob, size_t& off, size_t count) {
    T* d = nullptr;
    CHECK(hipMalloc(&d, count * sizeof(T)));
    CHECK(hipMemcpy(d, blob.data() + off, count * sizeof(T), hipMemcpyHostToDevice));
    off += count * sizeof(T);
    return d;
}

template <class T>
void download(std::FILE* f, const T* d, size_t count) {
    std::vector<T> h(count);
    CHECK(hipMemcpy(h.data(), d, count * sizeof(T), hipMemcpyDeviceToHost));
    std::fwrite(h.data(), sizeof(T), count, f);
}

// ---- wrapper parity: each qwen:: launcher and the qe_ function it wraps, on
// the same inputs into separate outputs, must write the same bytes (an
// argument the wrapper passes in the wrong place changes them)
namespace wrappers {

uint32_t g_state = 12345u;
uint32_t next() {
    g_state = g_state * 1664525u + 1013904223u;
    return g_state;
}
// fp16 bits of a value in [-2, 2) (multiples of 2^-8: exact in fp16)
uint16_t rand_half_bits() {
    const float v = static_cast<float>(static_cast<int>(next() >> 22) - 512) / 256.0f;
    const _Float16 h = static_cast<_Float16>(v);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

template <class T>
T* dev_zero(size_t count) {
    T* d = nullptr;
    CHECK(hipMalloc(&d, count * sizeof(T)));
    CHECK(hipMemset(d, 0, count * sizeof(T)));
    return d;
}
half* dev_half(size_t count, float scale_pow2 = 1.0f) {
    std::vector<uint16_t> h(count);
    for (auto& x : h) {
        x = rand_half_bits();
        if (scale_pow2 != 1.0f) {
            _Float16 v;
            std::memcpy(&v, &x, 2);
            v = static_cast<_Float16>(static_cast<float>(v) * scale_pow2);
            std::memcpy(&x, &v, 2);
        }
    }
    half* d = dev_zero<half>(count);
    CHECK(hipMemcpy(d, h.data(), count * 2, hipMemcpyHostToDevice));
    return d;
}
half* dev_scales(size_t count) {  // positive group scales 2^-6 .. 2^-4
    std::vector<uint16_t> h(count);
    for (auto& x : h) {
        const _Float16 v = static_cast<_Float16>(1.0f / static_cast<float>(16 << (next() % 3)));
        std::memcpy(&x, &v, 2);
    }
    half* d = dev_zero<half>(count);
    CHECK(hipMemcpy(d, h.data(), count * 2, hipMemcpyHostToDevice));
    return d;
}
uint32_t* dev_words(size_t count) {
    std::vector<uint32_t> h(count);
    for (auto& x : h) x = next();
    uint32_t* d = dev_zero<uint32_t>(count);
    CHECK(hipMemcpy(d, h.data(), count * 4, hipMemcpyHostToDevice));
    return d;
}
template <class T>
T* dev_copy(const T* src, size_t count) {
    T* d = dev_zero<T>(count);
    CHECK(hipMemcpy(d, src, count * sizeof(T), hipMemcpyDeviceToDevice));
    return d;
}
qwen::DeviceControlBlock* make_ctl(int seq_pos) {
    qwen::DeviceControlBlock h{};
    h.token_id = 7;
    h.seq_pos = seq_pos;
    h.temperature = 0.0f;
    h.rng_seed = 99;
    qwen::DeviceControlBlock* d = nullptr;
    CHECK(hipMalloc(&d, sizeof(h)));
    CHECK(hipMemcpy(d, &h, sizeof(h), hipMemcpyHostToDevice));
    return d;
}
int failures = 0;
template <class T>
void same(const char* what, const T* a, const T* b, size_t count) {
    std::vector<T> ha(count), hb(count);
    CHECK(hipMemcpy(ha.data(), a, count * sizeof(T), hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(hb.data(), b, count * sizeof(T), hipMemcpyDeviceToHost));
    if (std::memcmp(ha.data(), hb.data(), count * sizeof(T)) != 0) {
        std::fprintf(stderr, "mismatch: %s\n", what);
        ++failures;
    }
}
uint16_t* u(half* p) { return reinterpret_cast<uint16_t*>(p); }
const uint16_t* u(const half* p) { return reinterpret_cast<const uint16_t*>(p); }

int run(hipStream_t st) {
    constexpr int H = qwen::HIDDEN_SIZE, I = qwen::INTERMEDIATE_SIZE, QD = qwen::Q_DIM, KVD = qwen::KV_DIM;
    constexpr int NQ = qwen::NUM_Q_HEADS, NKV = qwen::NUM_KV_HEADS, HD = qwen::HEAD_DIM, MS = qwen::MAX_SEQ_LEN;
    // embedding lookup
    {
        const int V = 1000, T = 4;
        uint32_t* w = dev_words(static_cast<size_t>(V) * H / 8);
        half* s = dev_scales(static_cast<size_t>(V) * H / 128);
        const int32_t ids_h[T] = {5, 999, 0, 123};
        int32_t* ids = dev_zero<int32_t>(T);
        CHECK(hipMemcpy(ids, ids_h, sizeof(ids_h), hipMemcpyHostToDevice));
        half *a = dev_zero<half>(T * H), *b = dev_zero<half>(T * H);
        qwen::launch_embed_lookup_w4a16(w, s, ids, a, nullptr, T, st);
        if (qe_launch_embed_lookup_w4a16(w, u(s), ids, u(b), nullptr, T, st, H)) return 3;
        CHECK(hipStreamSynchronize(st));
        same("launch_embed_lookup_w4a16", a, b, T * H);
    }
    // RMSNorm (fp16 output), fp16 -> Q8_1
    {
        const int T = 4;
        half *x = dev_half(T * H), *g = dev_half(H), *a = dev_zero<half>(T * H), *b = dev_zero<half>(T * H);
        qwen::launch_rmsnorm_fp16(x, g, a, T, st);
        if (qe_launch_rmsnorm_fp16(u(x), u(g), u(b), T, st, H)) return 3;
        int8_t *qa = dev_zero<int8_t>(I), *qb = dev_zero<int8_t>(I);
        float *sa = dev_zero<float>(I / 128), *sb = dev_zero<float>(I / 128);
        int32_t *ma = dev_zero<int32_t>(I / 8), *mb = dev_zero<int32_t>(I / 8);
        half* xi = dev_half(I);
        qwen::launch_quantize_fp16_to_q8_1(xi, qa, sa, ma, I, st);
        if (qe_launch_quantize_fp16_to_q8_1(u(xi), qb, sb, mb, I, st)) return 3;
        CHECK(hipStreamSynchronize(st));
        same("launch_rmsnorm_fp16", a, b, T * H);
        same("launch_quantize_fp16_to_q8_1 q8", qa, qb, I);
        same("launch_quantize_fp16_to_q8_1 scale", sa, sb, I / 128);
        same("launch_quantize_fp16_to_q8_1 sum8", ma, mb, I / 8);
    }
    // gate/up SwiGLU GEMVs (W4A16 and W4A8) and the prefill GEMMs (QKV, SwiGLU)
    {
        uint32_t* w = dev_words(static_cast<size_t>(2 * I) * H / 8);
        half* s = dev_scales(static_cast<size_t>(2 * I) * H / 128);
        half* x = dev_half(H);
        int8_t* q8 = dev_zero<int8_t>(H);
        float* xs = dev_zero<float>(H / 128);
        int32_t* s8 = dev_zero<int32_t>(H / 8);
        if (qe_launch_quantize_fp16_to_q8_1(u(x), q8, xs, s8, H, st)) return 3;
        half *a = dev_zero<half>(I), *b = dev_zero<half>(I), *c = dev_zero<half>(I), *d = dev_zero<half>(I);
        qwen::launch_gemv_dual_gate_up_swiglu_w4a16(w, s, x, a, H, I, st);
        if (qe_launch_gemv_dual_gate_up_swiglu_w4a16(w, u(s), u(x), u(b), H, I, st)) return 3;
        qwen::launch_gemv_dual_gate_up_swiglu_w4a8(w, s, q8, xs, s8, c, H, I, st);
        if (qe_launch_gemv_dual_gate_up_swiglu_w4a8(w, u(s), q8, xs, s8, u(d), H, I, st)) return 3;
        const int M = 32;
        half* A = dev_half(static_cast<size_t>(M) * H);
        half *ga = dev_zero<half>(static_cast<size_t>(M) * I), *gb = dev_zero<half>(static_cast<size_t>(M) * I);
        qwen::launch_gemm_prefill_dual_gate_up_swiglu_w4a16(w, s, A, ga, M, st);
        if (qe_launch_gemm_prefill_dual_gate_up_swiglu_w4a16(w, u(s), u(A), u(gb), M, st, H, I)) return 3;
        // QKV over the first QD + 2 KVD rows of the same matrix
        const size_t rw = H / 8, rs = H / 128;
        half *qa = dev_zero<half>(static_cast<size_t>(M) * (QD + 2 * KVD)),
             *qb = dev_zero<half>(static_cast<size_t>(M) * (QD + 2 * KVD));
        qwen::QKVProjectionView va{w, s, qa, w + QD * rw, s + QD * rs, qa + static_cast<size_t>(M) * QD,
                                   w + (QD + KVD) * rw, s + (QD + KVD) * rs,
                                   qa + static_cast<size_t>(M) * (QD + KVD)};
        qe_qkv_view vb{w, u(s), u(qb), w + QD * rw, u(s) + QD * rs, u(qb) + static_cast<size_t>(M) * QD,
                       w + (QD + KVD) * rw, u(s) + (QD + KVD) * rs, u(qb) + static_cast<size_t>(M) * (QD + KVD)};
        qwen::launch_gemm_prefill_qkv_w4a16(va, A, M, st);
        if (qe_launch_gemm_prefill_qkv_w4a16(&vb, u(A), M, st, H, NQ, NKV, HD, 0)) return 3;
        CHECK(hipStreamSynchronize(st));
        same("launch_gemv_dual_gate_up_swiglu_w4a16", a, b, I);
        same("launch_gemv_dual_gate_up_swiglu_w4a8", c, d, I);
        same("launch_gemm_prefill_dual_gate_up_swiglu_w4a16", ga, gb, static_cast<size_t>(M) * I);
        same("launch_gemm_prefill_qkv_w4a16", qa, qb, static_cast<size_t>(M) * (QD + 2 * KVD));
    }
    // bias + RoPE + KV append, flash decode (Q8_1 epilogue), prefill attention
    {
        const int T = 40, base = 200;
        half *q0 = dev_half(T * QD), *k0 = dev_half(T * KVD), *v0 = dev_half(T * KVD);
        half *qb_ = dev_half(QD, 1.0f / 8), *kb_ = dev_half(KVD, 1.0f / 8), *vb_ = dev_half(KVD, 1.0f / 8);
        const size_t cache = static_cast<size_t>(NKV) * MS * HD;
        half *kc0 = dev_half(cache), *vc0 = dev_half(cache);
        half *qa = dev_copy(q0, T * QD), *ka = dev_copy(k0, T * KVD), *va = dev_copy(v0, T * KVD);
        half *qb = dev_copy(q0, T * QD), *kb = dev_copy(k0, T * KVD), *vb = dev_copy(v0, T * KVD);
        half *kca = dev_copy(kc0, cache), *vca = dev_copy(vc0, cache), *kcb = dev_copy(kc0, cache),
             *vcb = dev_copy(vc0, cache);
        qwen::DeviceControlBlock* ctl = make_ctl(base);
        qwen::launch_qkv_bias_rope_kv_append(qa, ka, va, qb_, kb_, vb_, kca, vca, ctl, T, st);
        if (qe_launch_qkv_bias_rope_kv_append(u(qb), u(kb), u(vb), u(qb_), u(kb_), u(vb_), u(kcb), u(vcb), ctl, T, st,
                                              NQ, NKV, HD, MS, 0, qwen::ROPE_THETA))
            return 3;
        half *pa = dev_zero<half>(T * QD), *pb = dev_zero<half>(T * QD);
        qwen::launch_attention_gqa_prefill(qa, kca, vca, pa, ctl, T, st);
        if (qe_launch_attention_gqa_prefill(u(qb), u(kcb), u(vcb), u(pb), ctl, T, st, NQ, NKV, HD, MS, H)) return 3;
        qwen::DeviceControlBlock* ctl2 = make_ctl(base + T - 1);
        float *poa = dev_zero<float>(NQ * 16 * HD), *pob = dev_zero<float>(NQ * 16 * HD);
        float *pla = dev_zero<float>(NQ * 32), *plb = dev_zero<float>(NQ * 32);
        half *oa = dev_zero<half>(QD), *ob = dev_zero<half>(QD);
        int8_t *q8a = dev_zero<int8_t>(QD), *q8b = dev_zero<int8_t>(QD);
        float *sca = dev_zero<float>(NQ), *scb = dev_zero<float>(NQ);
        int32_t *s8a = dev_zero<int32_t>(QD / 8), *s8b = dev_zero<int32_t>(QD / 8);
        const half* qlast_a = qa + static_cast<size_t>(T - 1) * QD;
        const half* qlast_b = qb + static_cast<size_t>(T - 1) * QD;
        qwen::launch_attention_gqa_flash_decode(qlast_a, kca, vca, poa, pla, oa, ctl2, st, NQ, NKV, HD, MS, q8a, sca,
                                                s8a);
        if (qe_launch_attention_gqa_flash_decode(u(qlast_b), u(kcb), u(vcb), pob, plb, u(ob), ctl2, st, NQ, NKV, HD,
                                                 MS, q8b, scb, s8b))
            return 3;
        CHECK(hipStreamSynchronize(st));
        same("launch_qkv_bias_rope_kv_append q", qa, qb, T * QD);
        same("launch_qkv_bias_rope_kv_append k", ka, kb, T * KVD);
        same("launch_qkv_bias_rope_kv_append v", va, vb, T * KVD);
        same("launch_qkv_bias_rope_kv_append k cache", kca, kcb, cache);
        same("launch_qkv_bias_rope_kv_append v cache", vca, vcb, cache);
        same("launch_attention_gqa_prefill", pa, pb, T * QD);
        same("launch_attention_gqa_flash_decode out", oa, ob, QD);
        same("launch_attention_gqa_flash_decode q8", q8a, q8b, QD);
        same("launch_attention_gqa_flash_decode scale", sca, scb, NQ);
        same("launch_attention_gqa_flash_decode sum8", s8a, s8b, QD / 8);
    }
    // sampling (greedy and temperature) with the control-block advance
    for (float temp : {0.0f, 0.8f}) {
        const int V = qwen::VOCAB_SIZE;
        half* logits = dev_half(V);
        float *va = dev_zero<float>(256), *vb = dev_zero<float>(256);
        int32_t *ia = dev_zero<int32_t>(256), *ib = dev_zero<int32_t>(256);
        int32_t *ta = dev_zero<int32_t>(1), *tb = dev_zero<int32_t>(1);
        qwen::DeviceControlBlock *ca = make_ctl(50), *cb = make_ctl(50);
        CHECK(hipMemcpy(&ca->temperature, &temp, 4, hipMemcpyHostToDevice));
        CHECK(hipMemcpy(&cb->temperature, &temp, 4, hipMemcpyHostToDevice));
        qwen::launch_sample_and_advance(logits, va, ia, ca, ta, st);
        if (qe_launch_sample_and_advance(u(logits), vb, ib, cb, tb, st, V)) return 3;
        CHECK(hipStreamSynchronize(st));
        same("launch_sample_and_advance token", ta, tb, 1);
        same("launch_sample_and_advance control block", ca, cb, 1);
    }
    return failures == 0 ? 0 : 4;
}

}  // namespace wrappers

int main(int argc, char** argv) {
    if (argc == 2 && std::strcmp(argv[1], "--wrappers") == 0) {
        hipStream_t st;
        CHECK(hipStreamCreate(&st));
        int rc = 0;
        try {
            rc = wrappers::run(st);
        } catch (const std::runtime_error& e) {
            std::fprintf(stderr, "launch failed: %s\n", e.what());
            rc = 3;
        }
        if (rc == 0) std::printf("wrappers ok\n");
        return rc;
    }
    if (argc != 3) return 1;
    constexpr int K = qwen::HIDDEN_SIZE, N = 2048, M = 64;
    std::FILE* fi = std::fopen(argv[1], "rb");
    if (!fi) return 1;
    std::vector<char> blob;
    char buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), fi)) > 0) blob.insert(blob.end(), buf, buf + n);
    std::fclose(fi);
    size_t off = 0;
    half* x = upload<half>(blob, off, K);
    half* gamma = upload<half>(blob, off, K);
    uint32_t* w = upload<uint32_t>(blob, off, static_cast<size_t>(N) * K / 8);
    half* s = upload<half>(blob, off, static_cast<size_t>(N) * K / 128);
    half* A = upload<half>(blob, off, static_cast<size_t>(M) * K);
    if (off != blob.size()) return 1;

    int8_t* q8;
    float* xs;
    int32_t* s8;
    half *y8, *y16, *qkv, *gemm;
    CHECK(hipMalloc(&q8, K));
    CHECK(hipMalloc(&xs, K / 128 * 4));
    CHECK(hipMalloc(&s8, K / 8 * 4));
    CHECK(hipMalloc(&y8, N * 2));
    CHECK(hipMalloc(&y16, N * 2));
    CHECK(hipMalloc(&qkv, (qwen::Q_DIM + 2 * qwen::KV_DIM) * 2));
    CHECK(hipMalloc(&gemm, static_cast<size_t>(M) * N * 2));
    hipStream_t st;
    CHECK(hipStreamCreate(&st));
    try {
        qwen::launch_rmsnorm_q8_1(x, gamma, nullptr, q8, xs, s8, st);
        qwen::launch_gemv_w4a8(w, s, q8, xs, s8, nullptr, y8, N, K, st);
        qwen::launch_gemv_w4a16(w, s, x, nullptr, y16, N, K, st);
        // QKV view over rows [0, 1536), [1536, 1792), [1792, 2048) of the same matrix
        const size_t rw = K / 8, rs = K / 128;
        qwen::QKVProjectionView v{w, s, qkv,
                                  w + qwen::Q_DIM * rw, s + qwen::Q_DIM * rs, qkv + qwen::Q_DIM,
                                  w + (qwen::Q_DIM + qwen::KV_DIM) * rw, s + (qwen::Q_DIM + qwen::KV_DIM) * rs,
                                  qkv + qwen::Q_DIM + qwen::KV_DIM};
        qwen::launch_gemv_qkv_w4a8(v, q8, xs, s8, st);
        qwen::launch_gemm_prefill_w4a16(w, s, A, nullptr, gemm, M, N, K, st);
    } catch (const std::runtime_error& e) {
        std::fprintf(stderr, "launch failed: %s\n", e.what());
        return 3;
    }
    CHECK(hipStreamSynchronize(st));
    std::FILE* fo = std::fopen(argv[2], "wb");
    if (!fo) return 1;
    download(fo, q8, K);
    download(fo, xs, K / 128);
    download(fo, s8, K / 8);
    download(fo, y8, N);
    download(fo, y16, N);
    download(fo, qkv, qwen::Q_DIM + 2 * qwen::KV_DIM);
    download(fo, gemm, static_cast<size_t>(M) * N);
    std::fclose(fo);
    CHECK(hipStreamDestroy(st));
    std::printf("cpp_api_gpu ok\n");
    return 0;
}
