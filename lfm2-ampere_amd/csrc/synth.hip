// synth.hip - the seeded synthetic inputs of the benchmark configurations,
// generated on the device: not part of the attention path (the configs of
// the measurement fill 0.1-3 GB of Q/K/V, minutes of host time).
//
// The generator is splitmix64 (S. Vigna's mixing of a Weyl sequence with
// increment 0x9e3779b97f4a7c15), u = ((x >> 11) + 1) / 2^53 in (0, 1], and
// Box-Muller in float64 -- implementation-independent, unlike
// std::normal_distribution.  The stream of a seed is counter-based: draw k
// (k = 1, 2, ...) is mix(seed + k * 0x9e3779b97f4a7c15), so every element is
// formed by its own thread with the same integers as the sequential host
// restatement (oracle lko_sm_normal / lko_sm_uniform / lko_sm_student4):
//   normal   pair j = elements 2j, 2j+1 from draws 2j+1, 2j+2:
//            r = sqrt(-2 ln u1), element 2j = r cos(2 pi u2), 2j+1 = r sin(2 pi u2)
//   uniform  element i from draw i+1: lo + (hi - lo) * (float) u
//   student4 element i from draws 10i+1 .. 10i+10: five normals (cos form),
//            z / sqrt((g1^2 + g2^2 + g3^2 + g4^2) / 4)
// The float64 functions are the device library's; they and the host's are
// both within an ulp in float64, so the rounded fp32 values agree except in
// the rare case of a float64 result one ulp from an fp32 rounding boundary.
#include "lk_common.h"

#define LK_SM_GAMMA 0x9e3779b97f4a7c15ull

__device__ __forceinline__ uint64_t lk_sm_draw(uint64_t seed, uint64_t k) {
    uint64_t z = seed + k * LK_SM_GAMMA;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ double lk_sm_u01(uint64_t seed, uint64_t k) {
    return ((double) (lk_sm_draw(seed, k) >> 11) + 1.0) / 9007199254740992.0;
}
__device__ __forceinline__ double lk_sm_nrm_cos(uint64_t seed, uint64_t k) {   // draws k, k+1
#pragma clang fp contract(off)
    const double u1 = lk_sm_u01(seed, k), u2 = lk_sm_u01(seed, k + 1);
    return sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
}

__global__ void __launch_bounds__(256)
lk_k_synth(int kind, uint64_t seed, size_t n, float lo, float hi, float * __restrict__ out) {
#pragma clang fp contract(off)
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x;
    if (kind == 0) {                                      // normal: one thread per pair
        const size_t e = 2 * i;
        if (e >= n) return;
        const double u1 = lk_sm_u01(seed, e + 1), u2 = lk_sm_u01(seed, e + 2);
        const double r = sqrt(-2.0 * log(u1));
        out[e] = (float) (r * cos(2.0 * M_PI * u2));
        if (e + 1 < n) out[e + 1] = (float) (r * sin(2.0 * M_PI * u2));
    } else if (kind == 1) {                               // uniform
        if (i >= n) return;
        out[i] = lo + (hi - lo) * (float) lk_sm_u01(seed, i + 1);
    } else {                                              // Student-t, nu = 4
        if (i >= n) return;
        const uint64_t k = 10 * (uint64_t) i + 1;
        const double z = lk_sm_nrm_cos(seed, k);
        double c = 0.0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const double g = lk_sm_nrm_cos(seed, k + 2 + 2 * j);
            c += g * g;
        }
        out[i] = (float) (z / sqrt(c / 4.0));
    }
}

extern "C" int lk_synth_f32(int kind, uint64_t seed, size_t n, float lo, float hi, float * out, void * stream) {
    if (kind < 0 || kind > 2) return lk_fail(hipErrorInvalidValue, "lk_synth_f32: kind %d not in 0..2", kind);
    if (n == 0) return 0;
    if (!out) return lk_fail(hipErrorInvalidValue, "lk_synth_f32: null pointer argument");
    const size_t threads = kind == 0 ? (n + 1) / 2 : n;
    const size_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffull) return lk_fail(hipErrorInvalidValue, "lk_synth_f32: n %zu too large", n);
    hipLaunchKernelGGL(lk_k_synth, dim3((unsigned) blocks), dim3(256), 0, lk_stream(stream), kind, seed, n, lo, hi, out);
    return lk_launch_status("lk_synth_f32");
}
