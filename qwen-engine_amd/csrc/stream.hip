// Streaming-read kernel with the access pattern of the GEMV weight stream
// (16-byte nontemporal loads, contiguous across lanes).  It computes nothing
// useful: bench.py times it for the achievable-bandwidth ceiling of a launch
// that reads N bytes, and uses it as the known-size reference when scaling
// rocprofv3 FETCH_SIZE counters.  Not part of the reference's API.
#include "qe_common.hpp"

namespace qe {
namespace {

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * 256;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v.x + v.y + v.z + v.w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;  // keeps the loads; practically never stores
}

}  // namespace
}  // namespace qe

using namespace qe;

extern "C" int qe_stream_read(const void* data, size_t bytes, uint32_t* sink, hipStream_t stream) {
    QE_REQUIRE(data && sink, "stream_read: NULL pointer");
    QE_REQUIRE(aligned(data, 16) && bytes % 16 == 0, "stream_read: data must be 16-byte aligned, bytes % 16 == 0");
    const size_t n16 = bytes / 16;
    if (n16 == 0) return QE_OK;
    size_t grid = (n16 + 255) / 256;
    if (grid > static_cast<size_t>(cu_count()) * 64) grid = static_cast<size_t>(cu_count()) * 64;
    stream_read_kernel<<<static_cast<unsigned>(grid), 256, 0, stream>>>(static_cast<const u32x4*>(data), n16, sink);
    return check_launch("stream_read");
}
