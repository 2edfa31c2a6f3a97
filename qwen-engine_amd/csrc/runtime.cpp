// Host-side runtime helpers of libqe_amd: thread-local error text, version,
// cached device facts.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <cstring>

#include "qe_common.hpp"

namespace qe {

namespace {
thread_local char g_last_error[1024] = "";
int g_cu_count[64] = {0};
int g_gemm_split_k = 1;
int g_gemm_tile = 0;
int g_gemm_slices = 0;
int g_gemm_ks2 = 0;
int g_gemv_bt = 0;
int g_gemv_cap = 0;
int g_engine_tiled = 1;
}  // namespace

int gemm_split_k_enabled() { return g_gemm_split_k; }
int gemm_forced_tile() { return g_gemm_tile; }
int gemm_forced_slices() { return g_gemm_slices; }
int gemm_ks2_mode() { return g_gemm_ks2; }
int gemv_forced_bt() { return g_gemv_bt; }
int gemv_forced_cap() { return g_gemv_cap; }
int engine_tiled_prefill() { return g_engine_tiled; }

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (g_cu_count[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        g_cu_count[dev] = n;
    }
    return g_cu_count[dev];
}

}  // namespace qe

extern "C" const char* qe_last_error(void) { return qe::g_last_error; }

extern "C" const char* qe_version(void) { return "qe_amd 0.1 (gfx950)"; }

extern "C" int qe_set_tuning(const char* key, int value) {
    if (key == nullptr) return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: key is NULL");
    if (std::strcmp(key, "gemm_split_k") == 0) {
        qe::g_gemm_split_k = value != 0;
        return QE_OK;
    }
    if (std::strcmp(key, "gemm_tile") == 0) {
        if (value < 0 || value > 4) return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: gemm_tile %d not in 0..4", value);
        qe::g_gemm_tile = value;
        return QE_OK;
    }
    if (std::strcmp(key, "gemv_block") == 0) {
        if (value != 0 && value != 256 && value != 512 && value != 1024)
            return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: gemv_block %d not in {0, 256, 512, 1024}", value);
        qe::g_gemv_bt = value;
        return QE_OK;
    }
    if (std::strcmp(key, "gemv_grid_cap") == 0) {
        if (value < 0 || value > 65536)
            return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: gemv_grid_cap %d not in 0..65536", value);
        qe::g_gemv_cap = value;
        return QE_OK;
    }
    if (std::strcmp(key, "gemm_ks2") == 0) {
        if (value < 0 || value > 2) return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: gemm_ks2 %d not in 0..2", value);
        qe::g_gemm_ks2 = value;
        return QE_OK;
    }
    if (std::strcmp(key, "engine_tiled_prefill") == 0) {
        qe::g_engine_tiled = value != 0;
        return QE_OK;
    }
    if (std::strcmp(key, "gemm_slices") == 0) {
        if (value < 0 || value > 64) return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: gemm_slices %d not in 0..64", value);
        qe::g_gemm_slices = value;
        return QE_OK;
    }
    return qe::fail(QE_ERR_INVALID_ARGUMENT, "set_tuning: unknown key '%s'", key);
}
