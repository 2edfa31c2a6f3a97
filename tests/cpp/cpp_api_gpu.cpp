// GPU check of the C++ drop-in API (kernels.hpp): a host program in the style
// of the reference's engine (hipMalloc'd buffers, one stream, the qwen::
// launchers with their default arguments) runs the matrix path on inputs read
// from a file and writes the outputs back; tests/test_gpu_cpp_api.py compares
// them with the CPU oracle.
//
// usage: cpp_api_gpu <in.bin> <out.bin>
//   in.bin : K=1536, N=2048, M=64 inputs - x fp16[K], gamma fp16[K], weights
//            uint32[N][K/8], scales fp16[N][K/128], A fp16[M][K]
//   out.bin: q8 int8[K], scale f32[K/128], sum8 i32[K/8] (rmsnorm_q8_1 of x),
//            y_w4a8 fp16[N] (on that Q8_1), y_w4a16 fp16[N] (on x),
//            qkv fp16[1536 + 256 + 256] (QKV view over the same matrix),
//            gemm fp16[M][N]
#include <cstdio>
#include <cstdlib>
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

int main(int argc, char** argv) {
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
