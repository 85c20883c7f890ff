// mvh_probe.hip -- device bandwidth probes (measurement, not part of the path).
//
// stream_read_kernel reads every byte of a buffer once with 16-byte loads
// (consecutive lanes on consecutive addresses, eight loads in flight per
// lane) and folds them into one word per lane; the word is stored only if it
// equals a value the data never produces, so the loads stay live without
// write traffic.  The kernel time of a buffer larger than the 256 MB
// Infinity Cache, read once, is the device's streaming-read bandwidth: the
// measured ceiling the GEMV roofline is stated against beside the 8 TB/s
// specification.
#include "mvh_kernels.hpp"

namespace mvh {
namespace {

constexpr int kReadT = 256, kReadV = 8;

__global__ __launch_bounds__(kReadT) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                             uint32_t* __restrict__ sink) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kReadT * kReadV;
    uint32_t acc = 0;
    for (size_t i0 = static_cast<size_t>(blockIdx.x) * kReadT * kReadV + threadIdx.x; i0 < n16; i0 += stride) {
        uint4 v[kReadV];
#pragma unroll
        for (int k = 0; k < kReadV; ++k) {
            const size_t i = i0 + static_cast<size_t>(k) * kReadT;
            v[k] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < kReadV; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x * kReadT + threadIdx.x] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, size_t sink_words, hipStream_t st) {
    const size_t n16 = bytes / 16;
    if (!n16) return hipSuccess;
    int dev = 0, cus = 256;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess && prop.multiProcessorCount > 0)
        cus = prop.multiProcessorCount;
    size_t grid = static_cast<size_t>(cus) * 8;  // eight workgroups of 4 waves per CU
    grid = std::min(grid, (n16 + kReadT * kReadV - 1) / (kReadT * kReadV));
    grid = std::min(grid, sink_words / kReadT);
    if (!grid) return hipErrorInvalidValue;
    stream_read_kernel<<<static_cast<unsigned>(grid), kReadT, 0, st>>>(static_cast<const uint4*>(buf), n16, sink);
    return hipGetLastError();
}

}  // namespace mvh
