// Links against libqe_amd.so and calls the C++ API with a shape the path does
// not support: the wrapper must throw std::runtime_error carrying the C-ABI's
// message (the reference's CUDA_KERNEL_CHECK throws, include/tensor.cuh:11-23).
// Needs no GPU: the precondition is checked on the host before any HIP call.
#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "kernels.hpp"

int main() {
    int caught = 0;
    try {
        qwen::launch_gemv_w4a8(reinterpret_cast<const uint32_t*>(16), reinterpret_cast<const half*>(16),
                               reinterpret_cast<const int8_t*>(16), reinterpret_cast<const float*>(16),
                               reinterpret_cast<const int32_t*>(16), nullptr, reinterpret_cast<half*>(16), 4, 100,
                               nullptr);
    } catch (const std::runtime_error& e) {
        caught = std::strstr(e.what(), "launch_gemv_w4a8") && std::strstr(e.what(), "multiple of 128");
    }
    try {
        qwen::launch_attention_gqa_flash_decode(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                                nullptr);
    } catch (const std::runtime_error& e) {
        caught += std::strstr(e.what(), "launch_attention_gqa_flash_decode") != nullptr;
    }
    std::printf("%d\n", caught);
    return caught == 2 ? 0 : 1;
}
