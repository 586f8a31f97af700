// Measurement probes for bench.py (libnnq_probe.so, separate from libnnq.so): the floors
// the decode kernels are compared against.
//   probe_stream_read   reads nbytes with 16-byte non-temporal loads, the way the decode
//                       GEMVs stream their weights, and does no other work (the loaded
//                       words are folded into one value, stored only when it equals a
//                       given key, so the loads cannot be dropped); contiguous 64 KiB
//                       chunks per workgroup in a grid-stride loop.
//   probe_empty         an empty kernel: the per-launch cost of a graph of launches.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr size_t kChunk = 65536;  // bytes per workgroup step: 256 threads x 16 B x 16

__global__ __launch_bounds__(kThreads) void probe_stream_read_kernel(const uint8_t *p, size_t nchunks,
                                                                      uint32_t key, uint32_t *sink) {
    uint32_t acc = 0;
    for (size_t c = blockIdx.x; c < nchunks; c += gridDim.x) {
        const u32x4 *q = reinterpret_cast<const u32x4 *>(p + c * kChunk) + threadIdx.x;
        u32x4 v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = __builtin_nontemporal_load(q + i * kThreads);
#pragma unroll
        for (int i = 0; i < 16; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == key) sink[0] = acc;
}

__global__ void probe_empty_kernel() {}

}  // namespace

extern "C" {

// nbytes must be a multiple of 64 KiB; p and sink are device pointers.
int probe_stream_read(const void *p, size_t nbytes, int workgroups, uint32_t *sink, void *stream) {
    if (!p || !sink || nbytes % kChunk || workgroups <= 0) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(probe_stream_read_kernel, dim3((unsigned)workgroups), dim3(kThreads), 0, (hipStream_t)stream,
                       (const uint8_t *)p, nbytes / kChunk, 0x9E3779B9u, sink);
    return (int)hipGetLastError();
}

int probe_empty(void *stream) {
    hipLaunchKernelGGL(probe_empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
    return (int)hipGetLastError();
}

}  // extern "C"
