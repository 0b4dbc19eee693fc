// probe.hip - a measurement reference, not part of the attention path: a plain
// streaming read of a device buffer, to put the decode kernels' HBM rate next
// to what a read-only kernel reaches on the same GPU (the datasheet 8 TB/s is
// not reachable by reads).  2048 workgroups of 512 threads, each streaming one
// contiguous share with 16-byte non-temporal loads, eight in flight per lane;
// the values are summed so the loads cannot be dropped, and the sum is
// written only under a condition the data never meets.
#include "lk_common.h"

__global__ void __launch_bounds__(512)
lk_k_read_probe(const lk_f4 * __restrict__ p, size_t n4, size_t per_block, float * __restrict__ sink) {
    const size_t b0 = (size_t) blockIdx.x * per_block;
    const size_t b1 = (b0 + per_block < n4) ? b0 + per_block : n4;
    lk_f4 acc = { 0.f, 0.f, 0.f, 0.f };
    for (size_t i = b0 + threadIdx.x; i < b1; i += 512 * 8) {
        lk_f4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const size_t j = i + (size_t) u * 512;
            v[u] = (j < b1) ? __builtin_nontemporal_load(p + j) : (lk_f4){ 0.f, 0.f, 0.f, 0.f };
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
    }
    if (acc[0] == -1.0f && acc[1] == 3.0f) sink[0] = acc[2];
}

extern "C" int lk_read_probe(const void * src, size_t bytes, float * sink, void * stream) {
    if (!src || !sink || bytes == 0 || (bytes & 15) || ((uintptr_t) src & 15))
        return lk_fail(hipErrorInvalidValue, "lk_read_probe: bad arguments");
    const int blocks = 2048;
    const size_t n4 = bytes / 16, per = (n4 + blocks - 1) / blocks;
    hipLaunchKernelGGL(lk_k_read_probe, dim3(blocks), dim3(512), 0, lk_stream(stream),
                       (const lk_f4 *) src, n4, per, sink);
    return lk_launch_status("lk_read_probe");
}
