// Shared host/device helpers of libqe_amd: status reporting, device facts,
// fp16 conversions.  gfx950 only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "qe_kernels.h"
#include "quant_primitives.hpp"

namespace qe {

// Native 128-bit vector (usable with __builtin_nontemporal_load).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Thread-local text of the last failure, returned by qe_last_error().
void set_error(const char* fmt, ...);
void clear_error();

// Number of compute units of the current device (cached per device).
int cu_count();

// Tuning switches (qe_set_tuning).
int gemm_split_k_enabled();
int gemm_forced_tile();    // 0 auto, 1 64x64, 2 64x128 (1x4 waves), 3 128x64, 4 128x128 (1x4 waves)
int gemm_forced_slices();  // 0 auto, else K slices
int gemm_ks2_mode();       // 0 auto, 1 never, 2 always (K % 256 == 0): the two-group k split
int gemv_forced_bt();      // 0 auto, else GEMV block size (256, 512, 1024)
int gemv_forced_cap();     // 0 auto, else the largest GEMV grid (larger grids loop over row sets)
int engine_tiled_prefill();  // engines created from now on keep tiled copies for the prefill GEMMs (default 1)

inline int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    set_error("%s", buf);
    return code;
}

// Checked at the end of every entry point, like CUDA_KERNEL_CHECK in the
// reference (include/tensor.cuh:23).
inline int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(QE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    clear_error();
    return QE_OK;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

__device__ __forceinline__ float h2f(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

}  // namespace qe

#define QE_TRY(call)                  \
    do {                              \
        const int rc_ = (call);       \
        if (rc_ != QE_OK) return rc_; \
    } while (0)

#define QE_REQUIRE(cond, ...)                                              \
    do {                                                                   \
        if (!(cond)) return ::qe::fail(QE_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
    } while (0)
