// qknr.hip - the producers of the attention inputs for gfx950: per-head RMS
// norm of q and k, NEOX rotary embedding, and the fp16 KV-cache write, for one
// decode token (lk_qk_norm_rope) and for a prefill chunk (lk_pf_qknr, which
// can also emit the int8 K copy of the new positions in the same pass).
//
// Reference behaviour: k_qk_norm_rope (/root/reference/src/kernels.cu:871-915,
// launched at engine.cu:606-608) and k_pf_qknr (prefill.cu:975-1016, launched
// at engine.cu:1069-1070); constants LK_EPS 1e-5, LK_ROPE_THETA 1e7, scale 1/8
// (kernels.cuh:22-24).  Per 64-wide row v of head h at position p:
//     ss  = sum v_d^2                (tree: d with d+32, then +16, ..., +1)
//     inv = 1 / sqrt(ss / 64 + eps)
//     y_d = v_d * inv * w_d          (w = q_norm or k_norm)
//     f_i = theta^(-i/32), a_i = (float) p * f_i        (i < 32, fp32 product)
//     out_i = y_i cos a_i - y_{i+32} sin a_i, out_{i+32} = y_i sin a_i + y_{i+32} cos a_i
// Q leaves as fp16(out / 8) (prefill) or fp32 in place (decode); K goes to the
// fp16 cache (decode also keeps it in place), V is copied to the fp16 cache.
//
// Arithmetic: every fp32 step rounds as written (contraction off).  The
// reference's rsqrtf / powf / sincosf are CUDA approximations; here 1/sqrt,
// theta^(-i/32) and the cosine and sine of the fp32 angle are evaluated in
// fp64 and rounded once to fp32, i.e. correctly rounded values (so the CPU
// oracle reproduces them bit for bit).  Against the reference's CUDA build the
// difference is therefore the approximation error of those three functions,
// at most a few fp32 ulp.
//
// MI355X design: one workgroup per token, 40 groups of 8 lanes (32 q heads,
// 8 k heads; the k groups also move V), 8 consecutive values per lane (32-byte
// loads, 16-byte fp16 stores); the 32 (cos, sin) pairs of the token are formed
// once in LDS; the RoPE partner of value d (d + 32) sits 4 lanes away and is
// fetched with one lane exchange per value.  HBM-bound: a 4096-token chunk
// reads 48 MiB of fp32 q|k|v and writes 24 MiB of fp16 (+2 MiB int8 K).
#include "lk_common.h"
#include <math.h>

#define LK_QKNR_ROWS    (LK_N_HEADS + LK_N_KV_HEADS)   // 40 groups per token
#define LK_QKNR_THREADS (LK_QKNR_ROWS * 8)              // 320

// The rotary frequency of table entry threadIdx.x (threads 0..31; others get
// entry 0, unused), to be loaded before anything else the table waits for.
__device__ __forceinline__ float lk_rope_freq_lane() {
    return lk_rope_freq(threadIdx.x < LK_HEAD_DIM / 2 ? (int) threadIdx.x : 0);
}
// (cos, sin) of the 32 rotary angles of position pos, into LDS (threads 0..31).
__device__ __forceinline__ void lk_rope_table(int pos, float f, float * s_c, float * s_s) {
    const int i = threadIdx.x;
    if (i < LK_HEAD_DIM / 2) lk_rope_angle(pos, f, s_c[i], s_s[i]);
}

// Norm + rotation of one 64-wide row held by an 8-lane group (lane j: values
// 8j .. 8j+7).  v in, out (rotated, fp32) out.
__device__ __forceinline__ void lk_norm_rope8(const float (&v)[8], const float (&w)[8],
                                              const float * s_c, const float * s_s, int j,
                                              float (&out)[8]) {
#pragma clang fp contract(off)
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = v[i] * v[i];
    // the sum tree over d: strides 32, 16, 8 pair lanes (xor 4, 2, 1), strides
    // 4, 2, 1 pair values inside the lane; both partners add the same two
    // values, so every lane of the group ends with the same bits
#pragma unroll
    for (int o = 4; o > 0; o >>= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i) t[i] += __shfl_xor(t[i], o, 64);
    const float u0 = t[0] + t[4], u1 = t[1] + t[5], u2 = t[2] + t[6], u3 = t[3] + t[7];
    const float ss = (u0 + u2) + (u1 + u3);
    const float arg = ss * (1.0f / LK_HEAD_DIM) + LK_EPS_F;   // ss / 64 is exact
    const float inv = (float) (1.0 / sqrt((double) arg));
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = (v[i] * inv) * w[i];
    const bool lo = j < 4;                                     // values d < 32
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = __shfl_xor(y[i], 4, 64);               // value d +- 32
        const int fi = 8 * (j & 3) + i;
        const float c = s_c[fi], s = s_s[fi];
        const float x0 = lo ? y[i] : p, x1 = lo ? p : y[i];
        out[i] = lo ? (x0 * c - x1 * s) : (x0 * s + x1 * c);
    }
}

__device__ __forceinline__ void lk_store8h(_Float16 * __restrict__ dst, const float (&v)[8], float mul) {
#pragma clang fp contract(off)
    lk_h8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16) (v[i] * mul);
    *(lk_h8 *) dst = h;
}
__device__ __forceinline__ void lk_load8f(const float * __restrict__ src, float (&v)[8]) {
    const lk_f4 a = *(const lk_f4 *) src, b = *(const lk_f4 *) (src + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
}

// Decode: one token at position *d_pos.  q and k rows are read from qs / ks
// (fp32 [32][64] / [8][64]) and written, normalised and rotated, to qf / kf
// (the same buffers for the in-place API); K and V rows go to the fp16 caches.
__global__ void __launch_bounds__(LK_QKNR_THREADS)
lk_k_qk_norm_rope(const float * qs, const float * ks, float * qf, float * kf, const float * __restrict__ vf,
                  const float * __restrict__ qn, const float * __restrict__ kn,
                  const int * __restrict__ d_pos, _Float16 * __restrict__ kc, _Float16 * __restrict__ vc) {
    __shared__ float s_c[LK_HEAD_DIM / 2], s_s[LK_HEAD_DIM / 2];
    // every load goes out before the table's barrier (loads do not move across it)
    const float rf = lk_rope_freq_lane();
    const int g = threadIdx.x >> 3, j = threadIdx.x & 7;
    const bool isq = g < LK_N_HEADS;
    const int h = isq ? g : g - LK_N_HEADS;
    const float * src = isq ? qs + h * LK_HEAD_DIM : ks + h * LK_HEAD_DIM;
    float * row = isq ? qf + h * LK_HEAD_DIM : kf + h * LK_HEAD_DIM;
    float v[8], out[8], vv[8];
    float wn[8];                                                  // norm weights of values 8j..8j+7
    lk_load8f(src + 8 * j, v);
    lk_load8f(vf + (isq ? 0 : h * LK_HEAD_DIM) + 8 * j, vv);      // V row (k groups)
    lk_load8f((isq ? qn : kn) + 8 * j, wn);
    const int pos = *d_pos;
    lk_rope_table(pos, rf, s_c, s_s);
    __syncthreads();
    lk_norm_rope8(v, wn, s_c, s_s, j, out);
    *(lk_f4 *) (row + 8 * j)     = (lk_f4){ out[0], out[1], out[2], out[3] };
    *(lk_f4 *) (row + 8 * j + 4) = (lk_f4){ out[4], out[5], out[6], out[7] };
    if (!isq) {
        const size_t off = ((size_t) pos * LK_N_KV_HEADS + h) * LK_HEAD_DIM + 8 * j;
        lk_store8h(kc + off, out, 1.0f);
        lk_store8h(vc + off, vv, 1.0f);
    }
}

// Prefill: token t of the chunk is at position P + t; Y is the q|k|v
// projection [m][3072] fp32.  Q -> qh fp16 [m][2048] (x 1/8), K/V -> caches;
// with k8 != nullptr the new K rows are also quantised to int8 exactly as
// lk_k_pf_k8 does from the cache (from the fp16-rounded values, minus cm).
__global__ void __launch_bounds__(LK_QKNR_THREADS)
lk_k_pf_qknr(const float * __restrict__ Y, const float * __restrict__ qn, const float * __restrict__ kn,
             int P, _Float16 * __restrict__ qh, _Float16 * __restrict__ kc, _Float16 * __restrict__ vc,
             int8_t * __restrict__ k8, float * __restrict__ ksc, int kstride, const float * __restrict__ cm) {
#pragma clang fp contract(off)
    __shared__ float s_c[LK_HEAD_DIM / 2], s_s[LK_HEAD_DIM / 2];
    const int t = blockIdx.x, pos = P + t;
    // every load goes out before the table's barrier (loads do not move across it)
    const float rf = lk_rope_freq_lane();
    const int g = threadIdx.x >> 3, j = threadIdx.x & 7;
    const bool isq = g < LK_N_HEADS;
    const int h = isq ? g : g - LK_N_HEADS;
    const float * y = Y + (size_t) t * 3072;
    float v[8], out[8], vv[8];
    lk_load8f(y + (isq ? h * LK_HEAD_DIM : 2048 + h * LK_HEAD_DIM) + 8 * j, v);
    lk_load8f(y + 2560 + (isq ? 0 : h * LK_HEAD_DIM) + 8 * j, vv);   // V row (k groups)
    float wn[8];                                                     // norm weights of values 8j..8j+7
    lk_load8f((isq ? qn : kn) + 8 * j, wn);
    lk_rope_table(pos, rf, s_c, s_s);
    __syncthreads();
    lk_norm_rope8(v, wn, s_c, s_s, j, out);
    if (isq) {
        lk_store8h(qh + (size_t) t * LK_HIDDEN + h * LK_HEAD_DIM + 8 * j, out, 0.125f);
        return;
    }
    const size_t off = ((size_t) pos * LK_N_KV_HEADS + h) * LK_HEAD_DIM + 8 * j;
    lk_store8h(kc + off, out, 1.0f);
    lk_store8h(vc + off, vv, 1.0f);
    if (k8) {                                                  // wave-uniform
        float kq[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            kq[i] = (float) (_Float16) out[i];
            if (cm) kq[i] -= cm[h * LK_HEAD_DIM + 8 * j + i];
        }
        lk_q8_row8(kq, k8 + off, ksc + (size_t) h * kstride + pos, 1.0f, j == 0);
    }
}

// ---------------------------------------------------------------------------
// C ABI
// qs/ks -> qf/kf (may alias: in place)
static int lk_qknr_decode_launch(const float * qs, const float * ks, float * qf, float * kf, const float * vf,
                                 const float * qn, const float * kn, const int * d_pos, void * kc, void * vc,
                                 hipStream_t st) {
    hipLaunchKernelGGL(lk_k_qk_norm_rope, dim3(1), dim3(LK_QKNR_THREADS), 0, st,
                       qs, ks, qf, kf, vf, qn, kn, d_pos, (_Float16 *) kc, (_Float16 *) vc);
    return lk_launch_status("lk_qk_norm_rope");
}

extern "C" int lk_qk_norm_rope(float * qf, float * kf, const float * vf, const float * qn,
                               const float * kn, const int * d_pos, void * kc, void * vc,
                               void * stream) {
    if (!qf || !kf || !vf || !qn || !kn || !d_pos || !kc || !vc)
        return lk_fail(hipErrorInvalidValue, "lk_qk_norm_rope: null pointer argument");
    // the widths the kernel loads and stores at: 16 bytes (8 fp32 in, 8 fp16 out)
    if (((uintptr_t) qf | (uintptr_t) kf | (uintptr_t) vf | (uintptr_t) qn | (uintptr_t) kn |
         (uintptr_t) kc | (uintptr_t) vc) & 15)
        return lk_fail(hipErrorInvalidValue, "lk_qk_norm_rope: qf, kf, vf, qn, kn, kc and vc must be 16-byte aligned");
    return lk_qknr_decode_launch(qf, kf, qf, kf, vf, qn, kn, d_pos, kc, vc, lk_stream(stream));
}

extern "C" int lk_pf_qknr(const float * Y, const float * qn, const float * kn, int m, int P,
                          void * qh, void * kc, void * vc, int8_t * k8, float * ksc, int kstride,
                          const float * cm, void * stream) {
    if (m < 0 || P < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_qknr: m %d / P %d negative", m, P);
    if (m == 0) return 0;
    if (!Y || !qn || !kn || !qh || !kc || !vc)
        return lk_fail(hipErrorInvalidValue, "lk_pf_qknr: null pointer argument");
    // the widths the kernel loads and stores at: Y, qn, kn, qh, kc, vc 16 bytes,
    // k8 8 bytes, ksc and cm 4 bytes
    if ((((uintptr_t) Y | (uintptr_t) qn | (uintptr_t) kn | (uintptr_t) qh | (uintptr_t) kc | (uintptr_t) vc) & 15) ||
        ((uintptr_t) k8 & 7) || (((uintptr_t) ksc | (uintptr_t) cm) & 3))
        return lk_fail(hipErrorInvalidValue, "lk_pf_qknr: misaligned argument (Y, qn, kn, qh, kc, vc 16 B; k8 8 B; ksc, cm 4 B)");
    if (k8 && (!ksc || kstride % 4 != 0 || kstride < P + m))
        return lk_fail(hipErrorInvalidValue, "lk_pf_qknr: k8 needs ksc and kstride %d (multiple of 4, >= P+m %d)",
                       kstride, P + m);
    hipLaunchKernelGGL(lk_k_pf_qknr, dim3(m), dim3(LK_QKNR_THREADS), 0, lk_stream(stream),
                       Y, qn, kn, P, (_Float16 *) qh, (_Float16 *) kc, (_Float16 *) vc, k8, ksc, kstride, cm);
    return lk_launch_status("lk_pf_qknr");
}
