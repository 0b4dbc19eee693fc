// gemv.hip - the consumer of the decode attention output for gfx950: the Q4_0
// weight x Q8_1 activation GEMV that applies attn_output.weight (2048 x 2048,
// 64 blocks of 32 per row) to the combine's block_q8_1 output and adds the
// residual, and the same GEMV for any other Q4_0 matrix of that format.
//
// Reference behaviour: k_gemv_q4_0 (/root/reference/src/kernels.cu:300-306,
// body k_gemv_q4_0_t kernels.cu:190-260 with LK_GEMV_ROWS = 1), launched for
// the attention output at engine.cu:655-657; the block dot dot_q4_0_q8_1
// (quant.cuh:131-158); warp_sum (kernels.cuh:28-32); the optional norm scale
// lk_norm_inv (kernels.cuh:441-447).  Per output row r:
//     lane l of the row's 32 lanes: acc_l = sum over k = l, l+32, ... (in
//         order) of d4 * (d8 * (float) sumi - 8 * sum8), where sumi is the
//         exact int32 sum over the block of nibble * q8 (nibbles 0..15: byte j
//         holds element j in its low nibble and element 16+j in its high
//         nibble; the -8 offset is carried by the activation sum), d4 the
//         weight block's fp16 scale, (d8, sum8) the activation block's fp16 ds
//     a = xor-butterfly 16, 8, 4, 2, 1 of acc_l (every lane ends with it)
//     a *= ninv when ssq is given, ninv = 1/sqrt(s/2048 + eps), s = the same
//         butterfly over ssq[l] + ssq[l+32]
//     y[r] = add_residual ? y[r] + a : a
//
// Arithmetic: contraction off, so every fp32 step rounds as written and the
// CPU oracle reproduces the output bit for bit.  The reference is compiled
// with contraction on (its results can differ by fp32 rounding) and uses the
// CUDA approximation rsqrtf; ninv here is 1/sqrt evaluated in fp64 and rounded
// once.
//
// MI355X design: one row per 32-lane half of a wave (the reference's warp, so
// the lane -> block mapping and the butterfly are the reference's), 8 rows per
// 256-thread workgroup, 256 workgroups for 2048 rows.  Each lane issues all of
// its loads at once -- 16-byte weight blocks, their fp16 scales, the 36-byte
// activation blocks (as nine dwords; 2.3 KB in total, read by every row from
// L2) and the residual -- and forms sumi with v_dot4_i32_i8 (nibbles 0..15 are non-negative
// int8 values, so the signed dot is exact).  HBM-bound on the weights: 18
// bytes per 32 weights, 2.36 MB for the 2048 x 2048 attention output matrix.
#include "lk_common.h"

#define LK_GEMV_THREADS 256
#define LK_GEMV_ROWS_PER_WG (LK_GEMV_THREADS / 32)
#define LK_GEMV_MAX_BPR 256              // blocks per row handled by the register loop (K <= 8192)

// d4 * (d8 * (float) sumi - 8 * sum8) for one block, as written.
__device__ __forceinline__ float lk_dot_q4_0_q8_1(const uint4 q, float d4, const int * __restrict__ xb) {
#pragma clang fp contract(off)
    const float d8  = (float) __builtin_bit_cast(_Float16, (unsigned short) (xb[0] & 0xffff));
    const float s8  = (float) __builtin_bit_cast(_Float16, (unsigned short) ((unsigned) xb[0] >> 16));
    const unsigned qw[4] = { q.x, q.y, q.z, q.w };
    int sumi = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        sumi = __builtin_amdgcn_sdot4((int) (qw[w] & 0x0F0F0F0Fu), xb[1 + w], sumi, false);          // elements 4w..4w+3
        sumi = __builtin_amdgcn_sdot4((int) ((qw[w] >> 4) & 0x0F0F0F0Fu), xb[5 + w], sumi, false);   // elements 16+4w..
    }
    const float t = d8 * (float) sumi;
    const float u = 8.0f * s8;
    return d4 * (t - u);
}

template <int NK>   // blocks per lane held in registers (bpr <= 32 * NK)
__global__ void __launch_bounds__(LK_GEMV_THREADS)
lk_k_gemv_q4_0(const uint4 * __restrict__ qs, const _Float16 * __restrict__ d,
               const int * __restrict__ xq, int out_rows, int bpr, float * __restrict__ y,
               int add_residual, const float * __restrict__ ssq, float eps) {
#pragma clang fp contract(off)
    const int l = threadIdx.x & 31;
    const int row = blockIdx.x * LK_GEMV_ROWS_PER_WG + (threadIdx.x >> 5);
    const bool live = row < out_rows;
    const int rowc = live ? row : out_rows - 1;           // clamped: loads stay in bounds
    const uint4 * qr = qs + (size_t) rowc * bpr;
    const _Float16 * dr = d + (size_t) rowc * bpr;
    // all loads first: weights, scales, activation blocks (9 dwords each)
    uint4 q[NK];
    float d4[NK];
    int xb[NK][9];
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        const int k = l + 32 * i;
        const int kc = (k < bpr) ? k : 0;
        q[i] = qr[kc];
        d4[i] = (float) dr[kc];
#pragma unroll
        for (int j = 0; j < 9; ++j) xb[i][j] = xq[(size_t) kc * 9 + j];
    }
    float ss = 0.0f;
    if (ssq) ss = ssq[l] + ssq[l + 32];
    const float yr = add_residual ? y[rowc] : 0.0f;      // issued with the other loads
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NK; ++i)
        if (l + 32 * i < bpr) acc = acc + lk_dot_q4_0_q8_1(q[i], d4[i], xb[i]);
    // the reference's xor butterfly (offsets 16, 8, 4, 2, 1 within the row's
    // 32 lanes, each partner adding the same two values) on a lane swap and
    // DPP instead of LDS permutes: bit-identical, 2.84 -> 2.71 us per launch
    // in a hipGraph
    acc = lk_bfly32_sum(acc);
    if (ssq) {
        ss = lk_bfly32_sum(ss);
        const float ninv = (float) (1.0 / sqrt((double) (ss * (1.0f / (float) LK_HIDDEN) + eps)));
        acc = acc * ninv;
    }
    if (live && l == 0) y[row] = add_residual ? yr + acc : acc;
}

template <int NK>
static void lk_gemv_launch(const uint4 * qs, const _Float16 * d, const int * xq, int out_rows, int bpr,
                           float * y, int add_residual, const float * ssq, float eps, hipStream_t st) {
    hipLaunchKernelGGL(lk_k_gemv_q4_0<NK>, dim3((out_rows + LK_GEMV_ROWS_PER_WG - 1) / LK_GEMV_ROWS_PER_WG),
                       dim3(LK_GEMV_THREADS), 0, st, qs, d, xq, out_rows, bpr, y, add_residual, ssq, eps);
}

extern "C" int lk_gemv_q4_0(const void * qs, const void * d, const lk_block_q8_1 * xq, int out_rows,
                            int bpr, float * y, int add_residual, const float * ssq, float eps,
                            void * stream) {
    if (out_rows < 0 || bpr < 1 || bpr > LK_GEMV_MAX_BPR)
        return lk_fail(hipErrorInvalidValue, "lk_gemv_q4_0: out_rows %d / bpr %d (1..%d)", out_rows, bpr, LK_GEMV_MAX_BPR);
    if (out_rows == 0) return 0;
    if (!qs || !d || !xq || !y)
        return lk_fail(hipErrorInvalidValue, "lk_gemv_q4_0: null pointer argument");
    if (((uintptr_t) qs & 15) || ((uintptr_t) d & 1) || ((uintptr_t) xq & 3) || ((uintptr_t) y & 3) ||
        ((uintptr_t) ssq & 3))
        return lk_fail(hipErrorInvalidValue, "lk_gemv_q4_0: misaligned argument (qs 16 B, d 2 B, xq, y, ssq 4 B)");
    const uint4 * q = (const uint4 *) qs;
    const _Float16 * dd = (const _Float16 *) d;
    const int * x = (const int *) xq;
    const hipStream_t st = lk_stream(stream);
    if (bpr <= 32)       lk_gemv_launch<1>(q, dd, x, out_rows, bpr, y, add_residual, ssq, eps, st);
    else if (bpr <= 64)  lk_gemv_launch<2>(q, dd, x, out_rows, bpr, y, add_residual, ssq, eps, st);
    else if (bpr <= 128) lk_gemv_launch<4>(q, dd, x, out_rows, bpr, y, add_residual, ssq, eps, st);
    else                 lk_gemv_launch<8>(q, dd, x, out_rows, bpr, y, add_residual, ssq, eps, st);
    return lk_launch_status("lk_gemv_q4_0");
}
