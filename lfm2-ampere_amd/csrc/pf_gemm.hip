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
// MI355X design: workgroup = 128 weight rows x 128 tokens, 4 waves of 64
// rows x 64 tokens, each a 4 x 4 grid of 16 x 16 v_mfma_i32_16x16x32_i8 tiles
// -- one 32-element Q4_0 block per MFMA, because the scales change from block
// to block; per token tile the 4 MFMAs go back to back, then their scale
// epilogue.  A operand: lane l supplies weight row l%16, elements 8(l/16)..+7,
// i.e. the low or high nibbles of bytes 0-7 or 8-15 of the 16-byte block (one
// shift, one mask); B operand: 8 int8 of the activation row.  The accumulator
// is seeded with 0x4B400000 so the integer sum arrives as the float F.
// Staging: 4 blocks at a time of the weight quants, the activation quants, the
// fp16 weight scales and the (d8, 8 sum) token scales go through LDS in two
// stages (16-byte coalesced global loads; the next stage's loads are in flight
// while the current one is computed); rows are padded (conflict-free 8-byte
// operand reads), the scales kept as [block][row] and [block][token], so a
// lane reads its 4 rows' d4 as one 8-byte read.  64 KB of LDS, 213 VGPRs: 2
// workgroups per CU.  Measured on C4's 4096 x 2048 x 2048: operands straight
// from L2 (8 scattered bytes per lane) 240 us; LDS staging at a 32 x 32 wave
// tile 95 us, 32 x 64 about 84 us, this 64 x 64 tile about 77 us.  The output
// tile is written as float4 (4 consecutive rows of one token).  Needs
// N % 128 == 0 and bpr % 8 == 0, as the reference's pf_gemm_dense does
// (PF_BM = 128).
#include "lk_common.h"

#define PFG_BM 128                 // weight rows per workgroup
#define PFG_BN 128                 // tokens per workgroup
#define PFG_KC 4                   // blocks per LDS stage (the staging below moves exactly 4)
#define PFG_TI 4                   // 16-row tiles per wave
#define PFG_TJ 4                   // 16-token tiles per wave
#define PFG_AP (PFG_KC * 16 + 16)  // LDS pitch of a weight row (bytes, padded)
#define PFG_BP (PFG_KC * 32 + 8)   // LDS pitch of an activation row (bytes; the 8-byte pad spreads the rows over the banks)
#ifndef PFG_ABL
#define PFG_ABL 0                  // measurement builds only: 2 no MFMA, 4 no fma epilogue
#endif

typedef int lk_i4g __attribute__((ext_vector_type(4)));
typedef float lk_f4g __attribute__((ext_vector_type(4)));

struct alignas(16) PfgStage {
    uint8_t  a[PFG_BM * PFG_AP];     // weight quant blocks [row][block][16]
    int8_t   b[PFG_BN * PFG_BP];     // activation quants [token][block][32]
    _Float16 d[PFG_KC][PFG_BM];      // weight scales [block][row]
    float2   s[PFG_KC][PFG_BN];      // token scales (d8, 8 sum) [block][token]
};

template <bool ADD>
__global__ void __launch_bounds__(256, 2)
lk_k_pf_gemm_q4_0(const uint8_t * __restrict__ qs, const _Float16 * __restrict__ d, int N, int bpr,
                  const int8_t * __restrict__ aqs, const float2 * __restrict__ asc, int ntok,
                  const float * __restrict__ scale, float * __restrict__ out, int out_ld) {
#pragma clang fp contract(off)
    __shared__ PfgStage stg[2];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row0 = blockIdx.x * PFG_BM, tok0 = blockIdx.y * PFG_BN;
    const int wr = (w & 1) * 64, wt = (w >> 1) * 64;   // the wave's 64 x 64 sub-tile
    const int l16 = lane & 15, kg = lane >> 4;
    constexpr float MAGIC = 12582912.0f;               // 1.5 * 2^23 = float bits 0x4B400000

    // ---- staging (4 blocks per stage): thread t moves weight row t/4 (16 of
    // its 64 bytes), token t/2 (64 of its 128 quant bytes, 2 of its 4 scale
    // pairs) and, for t < 64, the 4 fp16 scales of weight row t
    static_assert(PFG_KC == 4 && PFG_BM == 128 && PFG_BN == 128, "the staging assignment below");
    const int ar = tid >> 1, aq = tid & 1, bt = tid >> 1, bq = tid & 1;
    const int stok = (tok0 + bt < ntok) ? tok0 + bt : ntok - 1;     // clamped: loads stay in bounds
    const uint8_t * ga = qs + (size_t) (row0 + ar) * bpr * 16 + 32 * aq;             // + 16 kb0
    const int8_t * gb = aqs + (size_t) stok * bpr * 32 + 64 * bq;                     // + 32 kb0
    const _Float16 * gd = d + (size_t) (row0 + (tid & 127)) * bpr;                    // + kb0 (tid < 128)
    const float2 * gs = asc + (size_t) stok * bpr + 2 * bq;                           // + kb0
    // named registers, not arrays: a captured array stays in private memory
    uint4 ra0, ra1, rb0, rb1, rb2, rb3, rs;
    uint2 rd = make_uint2(0, 0);
    auto fetch = [&](int kb0) {
        ra0 = *(const uint4 *) (ga + 16 * kb0);
        ra1 = *(const uint4 *) (ga + 16 * kb0 + 16);
        rb0 = *(const uint4 *) (gb + 32 * kb0);
        rb1 = *(const uint4 *) (gb + 32 * kb0 + 16);
        rb2 = *(const uint4 *) (gb + 32 * kb0 + 32);
        rb3 = *(const uint4 *) (gb + 32 * kb0 + 48);
        if (tid < 128) rd = *(const uint2 *) (gd + kb0);
        rs = *(const uint4 *) (gs + kb0);
    };
    auto stash = [&](PfgStage & S) {
        *(uint4 *) (S.a + ar * PFG_AP + 32 * aq) = ra0;
        *(uint4 *) (S.a + ar * PFG_AP + 32 * aq + 16) = ra1;
        {   // 8-byte aligned rows: 8-byte stores
            uint2 * pb = (uint2 *) (S.b + bt * PFG_BP + 64 * bq);
            pb[0] = make_uint2(rb0.x, rb0.y); pb[1] = make_uint2(rb0.z, rb0.w);
            pb[2] = make_uint2(rb1.x, rb1.y); pb[3] = make_uint2(rb1.z, rb1.w);
            pb[4] = make_uint2(rb2.x, rb2.y); pb[5] = make_uint2(rb2.z, rb2.w);
            pb[6] = make_uint2(rb3.x, rb3.y); pb[7] = make_uint2(rb3.z, rb3.w);
        }
        if (tid < 128) {
            S.d[0][tid] = __builtin_bit_cast(_Float16, (unsigned short) (rd.x & 0xffff));
            S.d[1][tid] = __builtin_bit_cast(_Float16, (unsigned short) (rd.x >> 16));
            S.d[2][tid] = __builtin_bit_cast(_Float16, (unsigned short) (rd.y & 0xffff));
            S.d[3][tid] = __builtin_bit_cast(_Float16, (unsigned short) (rd.y >> 16));
        }
        S.s[2 * bq][bt]     = make_float2(__uint_as_float(rs.x), __uint_as_float(rs.y));
        S.s[2 * bq + 1][bt] = make_float2(__uint_as_float(rs.z), __uint_as_float(rs.w));
    };

    const int mb = 0x4B400000;
    const lk_i4g seed = { mb, mb, mb, mb };
    const int sh = 4 * (kg >> 1);                      // low or high nibbles
    lk_f4g acc[PFG_TI][PFG_TJ];
#pragma unroll
    for (int i = 0; i < PFG_TI; ++i)
#pragma unroll
        for (int j = 0; j < PFG_TJ; ++j) acc[i][j] = (lk_f4g){ 0.f, 0.f, 0.f, 0.f };

    const int nck = bpr / PFG_KC;
    fetch(0);
    for (int ck = 0; ck < nck; ++ck) {
        PfgStage & S = stg[ck & 1];
        stash(S);                                      // stage ck&1 was last read two chunks ago
        __syncthreads();
        if (ck + 1 < nck) fetch((ck + 1) * PFG_KC);    // the next chunk streams in during this one
#pragma unroll
        for (int b = 0; b < PFG_KC; ++b) {
            long a[PFG_TI], bv[PFG_TJ];
#pragma unroll
            for (int i = 0; i < PFG_TI; ++i) {
                const uint2 q = *(const uint2 *) (S.a + (wr + 16 * i + l16) * PFG_AP + 16 * b + 8 * (kg & 1));
                const uint32_t lo = (q.x >> sh) & 0x0F0F0F0Fu, hi = (q.y >> sh) & 0x0F0F0F0Fu;
                a[i] = (long) (((uint64_t) hi << 32) | lo);
            }
#pragma unroll
            for (int j = 0; j < PFG_TJ; ++j)
                bv[j] = *(const long *) (S.b + (wt + 16 * j + l16) * PFG_BP + 32 * b + 8 * kg);
            // d4 of rows 4kg .. 4kg+3 of each row tile: one 8-byte read each
            float d4[PFG_TI][4];
#pragma unroll
            for (int i = 0; i < PFG_TI; ++i) {
                const uint2 dw = *(const uint2 *) &S.d[b][wr + 16 * i + 4 * kg];
                d4[i][0] = (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.x & 0xffff));
                d4[i][1] = (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.x >> 16));
                d4[i][2] = (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.y & 0xffff));
                d4[i][3] = (float) __builtin_bit_cast(_Float16, (unsigned short) (dw.y >> 16));
            }
#pragma unroll
            for (int j = 0; j < PFG_TJ; ++j) {
                // the 4 MFMAs of this token tile back to back, then their scale epilogue
                lk_f4g F[PFG_TI];
#pragma unroll
                for (int i = 0; i < PFG_TI; ++i)
                    F[i] = (PFG_ABL & 2) ? __builtin_bit_cast(lk_f4g, (lk_i4g){ (int) a[i], (int) bv[j], (int) (a[i] >> 32), mb })
                                         : __builtin_bit_cast(lk_f4g, __builtin_amdgcn_mfma_i32_16x16x32_i8(a[i], bv[j], seed, 0, 0, 0));
                const float2 sv = S.s[b][wt + 16 * j + l16];
                const float c = __builtin_fmaf(sv.x, MAGIC, sv.y);
#pragma unroll
                for (int i = 0; i < PFG_TI; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[i][j][e] = (PFG_ABL & 4) ? acc[i][j][e] + F[i][e]
                                                     : __builtin_fmaf(d4[i][e], __builtin_fmaf(sv.x, F[i][e], -c), acc[i][j][e]);
            }
        }
        __syncthreads();                               // stage ck&1 fully read before it is refilled
    }
    // epilogue: lane holds rows 4kg .. 4kg+3 of each row tile for token l16 of each token tile
#pragma unroll
    for (int j = 0; j < PFG_TJ; ++j) {
        const int t = tok0 + wt + 16 * j + l16;
        if (t >= ntok) continue;
        const float sc = scale ? scale[t] : 1.0f;
#pragma unroll
        for (int i = 0; i < PFG_TI; ++i) {
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
    if (N % PFG_BM != 0 || bpr % 8 != 0 || out_ld % 4 != 0 || out_ld < N)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: N %d must be a multiple of %d, bpr %d of %d, out_ld %d a multiple of 4 and >= N",
                       N, PFG_BM, bpr, 8, out_ld);
    if (!qs || !d || !aqs || !asc || !out)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: null pointer argument");
    // the widths the kernel loads and stores at: qs, aqs, asc and out 16 bytes, d 8 bytes, scale 4
    if (((uintptr_t) qs & 15) || ((uintptr_t) d & 7) || ((uintptr_t) aqs & 15) || ((uintptr_t) asc & 15) ||
        ((uintptr_t) out & 15) || ((uintptr_t) scale & 3))
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: misaligned argument (qs, aqs, asc, out 16 B; d 8 B; scale 4 B)");
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
