// Bandwidth probe for measurements (not part of the decode library or its C ABI): a read-only
// pass over a device buffer, the practical HBM read ceiling a streaming kernel reaches on this
// GPU.  bench.py times it beside the decode so the decode's rate can be read against both the
// published 8 TB/s and what a plain stream achieves.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// Grid-stride 16-byte non-temporal loads, U in flight per thread.  The XOR of everything read goes
// to `sink` only when it equals a value the probe's data never produces, so the loads stay (the
// compiler cannot drop them) and no store races in practice.
template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const v4u* __restrict__ p, uint64_t n16, uint32_t* sink) {
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    v4u acc = {0u, 0u, 0u, 0u};
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        v4u v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) sink[0] = x;
}

// The same read with each workgroup streaming its own contiguous chunk (many concurrent streams,
// as a decode over many sequences reads), U 4 KiB steps in flight per workgroup.
template <int U>
__global__ __launch_bounds__(256) void k_stream_read_chunk(const v4u* __restrict__ p, uint64_t n16, uint32_t* sink) {
    const uint64_t chunk = (n16 + gridDim.x - 1) / gridDim.x;
    const uint64_t beg = (uint64_t)blockIdx.x * chunk;
    const uint64_t end = beg + chunk < n16 ? beg + chunk : n16;
    uint64_t i = beg + threadIdx.x;
    v4u acc = {0u, 0u, 0u, 0u};
    for (; i + (U - 1) * 256 < end; i += U * 256) {
        v4u v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * 256);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (; i < end; i += 256) acc ^= __builtin_nontemporal_load(p + i);
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) sink[0] = x;
}

}  // namespace

// Reads `bytes` (a multiple of 16, 16-byte aligned) once with `blocks` workgroups of 256 threads and
// `unroll` (4, 8 or 16) loads in flight per thread, grid-stride (chunked 0) or one contiguous chunk
// per workgroup (chunked 1); 0 on success, else the HIP error code.
extern "C" int ssq_probe_stream_read(const void* buf, uint64_t bytes, uint32_t* sink, int blocks, int unroll,
                                     int chunked, void* stream) {
    if (!buf || !sink || bytes % 16 || (uintptr_t)buf % 16 || blocks < 1) return (int)hipErrorInvalidValue;
    const v4u* p = static_cast<const v4u*>(buf);
    const uint64_t n16 = bytes / 16;
    hipStream_t st = (hipStream_t)stream;
    const dim3 g((unsigned)blocks), b(256);
    if (chunked) {
        if (unroll == 4) hipLaunchKernelGGL(k_stream_read_chunk<4>, g, b, 0, st, p, n16, sink);
        else if (unroll == 8) hipLaunchKernelGGL(k_stream_read_chunk<8>, g, b, 0, st, p, n16, sink);
        else if (unroll == 16) hipLaunchKernelGGL(k_stream_read_chunk<16>, g, b, 0, st, p, n16, sink);
        else return (int)hipErrorInvalidValue;
    } else {
        if (unroll == 4) hipLaunchKernelGGL(k_stream_read<4>, g, b, 0, st, p, n16, sink);
        else if (unroll == 8) hipLaunchKernelGGL(k_stream_read<8>, g, b, 0, st, p, n16, sink);
        else if (unroll == 16) hipLaunchKernelGGL(k_stream_read<16>, g, b, 0, st, p, n16, sink);
        else return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}
