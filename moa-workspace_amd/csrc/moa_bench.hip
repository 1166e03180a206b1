// moa_bench.hip -- measurement support (include/moa_bench.h). No counterpart in the reference:
// the attainable HBM read rate on this device and the floor of a one-token operator (an empty
// launch, a pure read of its weight bytes) at the launch shapes the operators use, so that a
// kernel's time can be split into launch, stream and the rest.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/moa_bench.h"
#include "../../include/moa_ops.h"
#include "moa_device.h"
#include "moa_internal.h"

namespace moa {
namespace {

// Workgroup b reads bytes [b * chunk, (b + 1) * chunk) of src (the last one up to n16), each wave
// 1 KB per load instruction (16 contiguous bytes per lane), eight loads in flight per lane,
// non-temporal, as the weight streams of the decode kernels read their rows. A slice that ends
// inside a batch of eight still issues that batch at once (the loads past the end are masked off),
// so no shape degrades to one load in flight. The XOR of all words is stored only when it equals
// a value no input here produces, so the loads cannot be removed and nothing is written.
constexpr int kUnroll = 8;

__global__ void stream_read_kernel(const uint4* __restrict__ src, uint64_t n16, uint32_t* sink) {
    const uint64_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t begin = (uint64_t)blockIdx.x * chunk;
    const uint64_t end = begin + chunk < n16 ? begin + chunk : n16;
    uint32_t acc = 0;
    const uint64_t step = (uint64_t)blockDim.x * kUnroll;
    for (uint64_t i = begin + threadIdx.x; i < end; i += step) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const uint64_t j = i + (uint64_t)u * blockDim.x;
            v[u] = j < end ? ld_stream(src + j) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace
}  // namespace moa

extern "C" int moa_bench_stream_read(const void* src, uint64_t bytes, int workgroups, int threads, uint32_t* sink,
                                     void* stream) {
    if ((bytes && !src) || !sink) return moa::set_error(MOA_ERROR_INVALID_VALUE, "src or sink is NULL");
    if (reinterpret_cast<uintptr_t>(src) % 16 || bytes % 16)
        return moa::set_error(MOA_ERROR_MISALIGNED, "src and bytes must be multiples of 16");
    if (workgroups < 1 || workgroups > (1 << 20) || threads < 64 || threads > 1024 || threads % 64)
        return moa::set_error(MOA_ERROR_INVALID_VALUE, "need 1 <= workgroups <= 2^20 and threads a multiple of 64 in [64, 1024]");
    hipLaunchKernelGGL(moa::stream_read_kernel, dim3(workgroups), dim3(threads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), bytes / 16, sink);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return moa::set_error(MOA_ERROR_HIP, (std::string("stream_read launch: ") + hipGetErrorString(e)).c_str());
    return MOA_SUCCESS;
}
