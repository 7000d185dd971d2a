// vtq_probe.hip -- measurement helpers for bench.py (libvtq_probe.so).
//
// Not part of the quantized-linear boundary (include/vtq.h): these kernels
// exist only to measure what the hardware gives a plain access pattern on
// the same buffers the benchmark's GEMVs read, so that each GEMV's rate can
// be quoted against a measured read ceiling as well as the published peak.
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace {

// Read-only stream: every thread reads 16-byte words i = g, g + G, g + 2G, ...
// (g = global thread index, G = grid threads), one load in flight per thread,
// and folds them into one word.  The store happens only if that word equals
// a constant the data never produces in practice; it keeps the loads alive
// without adding write traffic.
__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" {

// Launches the read of `bytes` (a multiple of 16) starting at device pointer
// `p` on `stream` with `workgroups` workgroups of 256 threads; `sink` is a
// device buffer of at least `workgroups` words.  Returns a hipError_t value.
int vtqp_stream_read(const void* p, size_t bytes, int workgroups, void* sink, void* stream) {
    if (!p || !sink || workgroups <= 0 || bytes % 16 != 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)workgroups), dim3(256), 0, (hipStream_t)stream,
                       static_cast<const uint4*>(p), bytes / 16, static_cast<uint32_t*>(sink));
    return (int)hipGetLastError();
}

}  // extern "C"
