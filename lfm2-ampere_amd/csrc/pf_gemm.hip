// pf_gemm.hip - the consumer of the prefill attention output for gfx950: the
// Q4_0 weight x planar Q8_1 activation GEMM that applies attn_output.weight to
// the chunk's attention rows (as lk_pf_attn8_q81 emits them) and adds the
// residual, and the same GEMM for any dense Q4_0 matrix of that format.
//
// Reference behaviour: k_pf_mmq with the plain epilogue (EPI 0) for one dense
// weight tensor (/root/reference/src/prefill.cu:173-490, driven by
// pf_gemm_dense, prefill.cu:818-826; PfGemm / PfAct, prefill.cuh:33-69),
// launched for the attention output at engine.cu:1128-1131.  With PF_EPI2 (its
// default, prefill.cu:131-141), per output (token t, row r):
//     acc = 0; for each 32-element block b in order:
//         F   = float bits of (0x4B400000 + sumi)  = 1.5*2^23 + sumi exactly
//               (sumi = the exact int32 sum of nibble * q8 over the block)
//         c   = fma(d8, 1.5*2^23, s8)              (s8 = 8 * fp16 sum, from the sc plane)
//         acc = fma(d4, fma(d8, F, -c), acc)
//     a = acc * scale[t] (scale NULL: 1);  out[t][r] = add ? out[t][r] + a : a
// Every step is an explicit fma or a separately rounded product or sum
// (contraction off), so this kernel and the CPU oracle produce the same bits;
// so does the reference's main loop.  Its nvcc build may contract the
// epilogue's acc * scale + out into one fma, a difference of one rounding.
//
// MI355X design: workgroup = 64 weight rows x 64 tokens, 4 waves of 32 x 32,
// each a 2 x 2 grid of 16 x 16 v_mfma_i32_16x16x32_i8 tiles -- one 32-element
// Q4_0 block per MFMA, because the scales change from block to block.  A
// operand: lane l supplies weight row l%16, elements 8(l/16)..+7, i.e. the low
// or high nibbles of bytes 0-7 or 8-15 of the 16-byte block (one shift, one
// mask); B operand: 8 int8 of the activation row.  The accumulator is seeded
// with 0x4B400000 so the integer sum arrives as the float F.  The fp16 weight
// scales and the (d8, 8 sum) token scales of 32 blocks at a time are staged in
// LDS ([block][row] and [block][token]), so a lane reads its 4 rows' d4 as one
// 8-byte read; operands come straight from L2 into registers, 4 blocks ahead.
// The output tile is written as float4 (4 consecutive rows of one token).
#include "lk_common.h"

#define PFG_BM 64                  // weight rows per workgroup
#define PFG_BN 64                  // tokens per workgroup
#define PFG_KC 32                  // blocks staged in LDS at a time
#define PFG_AHEAD 4                // blocks of operands in flight

typedef int lk_i4g __attribute__((ext_vector_type(4)));
typedef float lk_f4g __attribute__((ext_vector_type(4)));

template <bool ADD>
__global__ void __launch_bounds__(256, 2)
lk_k_pf_gemm_q4_0(const uint8_t * __restrict__ qs, const _Float16 * __restrict__ d, int N, int bpr,
                  const int8_t * __restrict__ aqs, const float2 * __restrict__ asc, int ntok,
                  const float * __restrict__ scale, float * __restrict__ out, int out_ld) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) _Float16 s_d[PFG_KC][PFG_BM];   // [block][row]
    __shared__ __attribute__((aligned(16))) float2 s_s[PFG_KC][PFG_BN];     // [block][token]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * PFG_BM, tok0 = blockIdx.y * PFG_BN;
    const int wr = (w & 1) * 32, wt = (w >> 1) * 32;   // the wave's 32 x 32 sub-tile
    const int l16 = lane & 15, kg = lane >> 4;
    constexpr float MAGIC = 12582912.0f;               // 1.5 * 2^23 = float bits 0x4B400000

    // per-lane operand sources (row / token clamped: loads stay in bounds)
    const uint8_t * ap[2];
    const int8_t * bp[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        ap[i] = qs + ((size_t) (row0 + wr + 16 * i + l16) * bpr) * 16 + 8 * (kg & 1);
        const int t = tok0 + wt + 16 * i + l16;
        bp[i] = aqs + (size_t) (t < ntok ? t : ntok - 1) * bpr * 32 + 8 * kg;
    }
    const int sh = 4 * (kg >> 1);                      // low or high nibbles

    const int mb = 0x4B400000;
    const lk_i4g seed = { mb, mb, mb, mb };
    lk_f4g acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (lk_f4g){ 0.f, 0.f, 0.f, 0.f };

    for (int kb0 = 0; kb0 < bpr; kb0 += PFG_KC) {
        const int nk = (bpr - kb0 < PFG_KC) ? bpr - kb0 : PFG_KC;
        __syncthreads();                                   // the previous chunk's scales are consumed
        for (int e = tid; e < nk * PFG_BM; e += 256) {     // d4: coalesced along the row's blocks
            const int r = e / nk, b = e % nk;
            s_d[b][r] = d[(size_t) (row0 + r) * bpr + kb0 + b];
        }
        for (int e = tid; e < nk * PFG_BN; e += 256) {
            const int t = e / nk, b = e % nk;
            const int tc = (tok0 + t < ntok) ? tok0 + t : ntok - 1;
            s_s[b][t] = asc[(size_t) tc * bpr + kb0 + b];
        }
        __syncthreads();
        for (int b0 = 0; b0 < nk; b0 += PFG_AHEAD) {
            // operands of up to PFG_AHEAD blocks, all loads first
            uint2 a8[PFG_AHEAD][2];
            long b8[PFG_AHEAD][2];
#pragma unroll
            for (int u = 0; u < PFG_AHEAD; ++u) {
                const int b = kb0 + ((b0 + u < nk) ? b0 + u : b0);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    a8[u][i] = *(const uint2 *) (ap[i] + (size_t) b * 16);
                    b8[u][i] = *(const long *) (bp[i] + (size_t) b * 32);
                }
            }
#pragma unroll
            for (int u = 0; u < PFG_AHEAD; ++u) {
                if (b0 + u >= nk) break;                   // wave-uniform
                const int b = b0 + u;
                long a[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t lo = (a8[u][i].x >> sh) & 0x0F0F0F0Fu, hi = (a8[u][i].y >> sh) & 0x0F0F0F0Fu;
                    a[i] = (long) (((uint64_t) hi << 32) | lo);
                }
                lk_f4g F[2][2];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        F[i][j] = __builtin_bit_cast(lk_f4g, __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], b8[u][j], seed, 0, 0, 0));
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float2 s = s_s[b][wt + 16 * j + l16];
                    const float c = __builtin_fmaf(s.x, MAGIC, s.y);
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        // d4 of rows 4kg .. 4kg+3 of row tile i: one 8-byte read
                        const uint2 dw = *(const uint2 *) &s_d[b][wr + 16 * i + 4 * kg];
                        const float d4[4] = { (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.x & 0xffff)),
                                              (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.x >> 16)),
                                              (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.y & 0xffff)),
                                              (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.y >> 16)) };
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[i][j][e] = __builtin_fmaf(d4[e], __builtin_fmaf(s.x, F[i][j][e], -c), acc[i][j][e]);
                    }
                }
            }
        }
    }
    // epilogue: lane holds rows 4kg .. 4kg+3 of each row tile for token l16 of each token tile
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = tok0 + wt + 16 * j + l16;
        if (t >= ntok) continue;
        const float sc = scale ? scale[t] : 1.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float4 * p = (float4 *) (out + (size_t) t * out_ld + row0 + wr + 16 * i + 4 * kg);
            float4 v = make_float4(acc[i][j][0] * sc, acc[i][j][1] * sc, acc[i][j][2] * sc, acc[i][j][3] * sc);
            if (ADD) {
                const float4 o = *p;
                v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
            *p = v;
        }
    }
}

extern "C" int lk_pf_gemm_q4_0(const void * qs, const void * d, int N, int bpr, const int8_t * aqs,
                               const float * asc, int ntok, const float * scale, float * out, int out_ld,
                               int add, void * stream) {
    if (N < 0 || ntok < 0 || bpr < 1)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: N %d / ntok %d / bpr %d", N, ntok, bpr);
    if (N == 0 || ntok == 0) return 0;
    if (N % PFG_BM != 0 || out_ld % 4 != 0 || out_ld < N)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: N %d must be a multiple of %d, out_ld %d a multiple of 4 and >= N",
                       N, PFG_BM, out_ld);
    if (!qs || !d || !aqs || !asc || !out)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: null pointer argument");
    if (((uintptr_t) qs & 15) || ((uintptr_t) d & 1) || ((uintptr_t) aqs & 7) || ((uintptr_t) asc & 7) ||
        ((uintptr_t) out & 15) || ((uintptr_t) scale & 3))
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: misaligned argument (qs 16 B, out 16 B, aqs / asc 8 B)");
    const dim3 grid(N / PFG_BM, (ntok + PFG_BN - 1) / PFG_BN);
    const hipStream_t st = lk_stream(stream);
    if (add)
        hipLaunchKernelGGL(lk_k_pf_gemm_q4_0<true>, grid, dim3(256), 0, st, (const uint8_t *) qs, (const _Float16 *) d,
                           N, bpr, aqs, (const float2 *) asc, ntok, scale, out, out_ld);
    else
        hipLaunchKernelGGL(lk_k_pf_gemm_q4_0<false>, grid, dim3(256), 0, st, (const uint8_t *) qs, (const _Float16 *) d,
                           N, bpr, aqs, (const float2 *) asc, ntok, scale, out, out_ld);
    return lk_launch_status("lk_pf_gemm_q4_0");
}
