// calib_stream.hip -- streaming-read calibration for bench.py (config
// "stream"), built as its own library (libmxfa_calib.so), not part of the
// engine.  One pass over a device buffer with 16-byte loads: each of
// `blocks` workgroups of 256 threads reads one contiguous chunk with eight
// loads in flight per thread (the best of the forms measured on the box:
// grid-stride loops with 4 or 8 loads per thread reached 5.0-5.9 TB/s,
// contiguous chunks 6.1-6.3 TB/s), and the XOR of everything read decides
// a store that never happens in practice, so the loads stay and nothing is
// written.  It anchors the decode kernels' HBM figures to what a plain read
// reaches on the same box.

#include <hip/hip_runtime.h>

#include <cstdint>

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kUnroll = 8;

__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4_t *__restrict__ p, uint64_t per,
                                                          uint32_t *out) {
    const u32x4_t *q = p + (uint64_t)blockIdx.x * per;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    uint64_t i = threadIdx.x;
    for (; i + (kUnroll - 1) * 256 < per; i += kUnroll * 256) {
        u32x4_t v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = q[i + u * 256];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) acc ^= v[u];
    }
    for (; i < per; i += 256) acc ^= q[i];
    const uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) out[blockIdx.x] = x;
}

// Reads `bytes` (a multiple of 16 * blocks) from the 16-byte aligned `p`;
// `out` holds `blocks` words (never written in practice).
extern "C" int mxfa_calib_stream_read(const void *p, uint64_t bytes, uint32_t *out, int blocks, void *stream) {
    if (!p || !out || blocks <= 0 || ((uintptr_t)p & 15) || bytes % (16ull * (uint64_t)blocks))
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3((uint32_t)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4_t *)p, bytes / 16 / (uint64_t)blocks, out);
    return (int)hipGetLastError();
}
