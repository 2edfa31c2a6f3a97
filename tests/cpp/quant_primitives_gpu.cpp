// Device code written against the reference's quant_primitives.cuh entry
// points (include/quant_primitives.cuh:13-115), compiled against this build's
// include/quant_primitives.hpp: the Q8_1 quantizer of a 16-lane group, the
// packed-word dot and the int4 -> half2 dequantization, called by the
// reference's names and parameter lists.  The kernels follow the shapes of the
// reference's own callers (the standalone quantizer, rmsnorm_rope.cu:273-299,
// and the embedding / GEMM B-tile dequantization, rmsnorm_rope.cu:15-51,
// gemm_prefill.cu:103-155).
//
//   quant_primitives_gpu IN OUT
// IN:  int32 K, int32 N, fp16 x[K], uint32 qw[N][K/8], fp16 scales[N][K/128]
// OUT: int8 q8[K], fp32 scale[K/128], int32 sum8[K/8], int32 sum8_again[K/8],
//      int32 group_dot[N][K/128], fp16 dequant[N][K]
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#include "quant_primitives.hpp"

using namespace qwen;

#define CHECK(x)                                                                    \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));     \
            std::exit(2);                                                           \
        }                                                                           \
    } while (0)

// one thread per 8 elements, 16 threads per 128-group (blockDim multiple of 16)
__global__ void quantize_kernel(const half* __restrict__ x, int K, int8_t* out_q8, float* out_scale,
                                int32_t* out_sum8) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int group_idx = t / 16, sub_lane = t % 16;
    if (group_idx * 128 >= K) return;  // whole groups only: all 16 lanes of a group stay active
    float vals[8];
    for (int j = 0; j < 8; ++j) vals[j] = __half2float(x[group_idx * 128 + sub_lane * 8 + j]);
    quantize_group128_fp16_to_q8_1(vals, group_idx, sub_lane, out_q8, out_scale, out_sum8);
}

// the zero-point seed recomputed from the stored q8 with compute_q8_sum8
__global__ void sum8_kernel(const int8_t* __restrict__ q8, int K, int32_t* out) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t * 8 >= K) return;
    const int2 v = reinterpret_cast<const int2*>(q8)[t];
    out[t] = compute_q8_sum8(v.x, v.y);
}

// group_dot[n][g] = sum over the 16 words of group g of dp4a_w4_q8_oct, each
// seeded with its 8 elements' sum8 (the reference GEMV's per-word seeding)
__global__ void group_dot_kernel(const uint32_t* __restrict__ qw, const int8_t* __restrict__ q8,
                                 const int32_t* __restrict__ sum8, int N, int K, int32_t* out) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int G = K / 128;
    if (t >= N * G) return;
    const int n = t / G, g = t % G;
    int32_t acc = 0;
    for (int w = 0; w < 16; ++w) {
        const int word = g * 16 + w;
        const int2 xv = reinterpret_cast<const int2*>(q8)[word];
        acc += dp4a_w4_q8_oct(qw[static_cast<size_t>(n) * (K / 8) + word], xv.x, xv.y, sum8[word]);
    }
    out[t] = acc;
}

// one thread per packed word: 8 fp16 out with one 16-byte store
__global__ void dequant_kernel(const uint32_t* __restrict__ qw, const half* __restrict__ scales, int N, int K,
                               half* out) {
    const size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t words = static_cast<size_t>(N) * (K / 8);
    if (t >= words) return;
    const size_t n = t / (K / 8), w = t % (K / 8);
    half2 h2[4];
    unpack_w4_to_half2_quad(qw[t], scales[n * (K / 128) + w / 16], h2);
    *reinterpret_cast<uint4*>(out + t * 8) = *reinterpret_cast<const uint4*>(h2);
}

template <class T>
static T* upload(const std::vector<T>& h) {
    T* d = nullptr;
    CHECK(hipMalloc(&d, h.size() * sizeof(T) + 16));
    CHECK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <class T>
static T* scratch(size_t n) {
    T* d = nullptr;
    CHECK(hipMalloc(&d, n * sizeof(T) + 16));
    return d;
}

template <class T>
static void download(FILE* f, const T* d, size_t n) {
    std::vector<T> h(n);
    CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    std::fwrite(h.data(), sizeof(T), n, f);
}

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s IN OUT\n", argv[0]);
        return 1;
    }
    FILE* fi = std::fopen(argv[1], "rb");
    if (!fi) return 1;
    int32_t K = 0, N = 0;
    if (std::fread(&K, 4, 1, fi) != 1 || std::fread(&N, 4, 1, fi) != 1 || K <= 0 || K % 128 || N <= 0) return 1;
    std::vector<uint16_t> x(K), sc(static_cast<size_t>(N) * (K / 128));
    std::vector<uint32_t> qw(static_cast<size_t>(N) * (K / 8));
    if (std::fread(x.data(), 2, x.size(), fi) != x.size() || std::fread(qw.data(), 4, qw.size(), fi) != qw.size() ||
        std::fread(sc.data(), 2, sc.size(), fi) != sc.size())
        return 1;
    std::fclose(fi);

    half* dx = reinterpret_cast<half*>(upload(x));
    uint32_t* dqw = upload(qw);
    half* dsc = reinterpret_cast<half*>(upload(sc));
    int8_t* q8 = scratch<int8_t>(K);
    float* xs = scratch<float>(K / 128);
    int32_t* s8 = scratch<int32_t>(K / 8);
    int32_t* s8b = scratch<int32_t>(K / 8);
    int32_t* dots = scratch<int32_t>(static_cast<size_t>(N) * (K / 128));
    half* deq = scratch<half>(static_cast<size_t>(N) * K);

    quantize_kernel<<<(K / 8 + 255) / 256, 256>>>(dx, K, q8, xs, s8);
    sum8_kernel<<<(K / 8 + 255) / 256, 256>>>(q8, K, s8b);
    group_dot_kernel<<<(N * (K / 128) + 255) / 256, 256>>>(dqw, q8, s8, N, K, dots);
    const size_t words = static_cast<size_t>(N) * (K / 8);
    dequant_kernel<<<static_cast<unsigned>((words + 255) / 256), 256>>>(dqw, dsc, N, K, deq);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());

    FILE* fo = std::fopen(argv[2], "wb");
    if (!fo) return 1;
    download(fo, q8, K);
    download(fo, xs, K / 128);
    download(fo, s8, K / 8);
    download(fo, s8b, K / 8);
    download(fo, dots, static_cast<size_t>(N) * (K / 128));
    download(fo, reinterpret_cast<uint16_t*>(deq), static_cast<size_t>(N) * K);
    std::fclose(fo);
    std::printf("quant_primitives ok\n");
    return 0;
}
