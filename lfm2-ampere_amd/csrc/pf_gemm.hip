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
// MI355X design: workgroup = 128 weight rows x 128 tokens, 8 waves of 32
// rows x 64 tokens, each a 1 x 2 pair of 32 x 32 v_mfma_i32_32x32x32_i8
// tiles -- one 32-element Q4_0 block per MFMA, because the scales change from
// block to block.  The 32-deep 32 x 32 form does four times the work of the
// 16 x 16 one in about 2.2 times its issue time (15.4 against 7.1 ns per SIMD
// on MI355X).  A operand: lane l supplies weight row l%32 of the tile,
// elements 16(l/32)..+15, i.e. the low (l < 32) or high (l >= 32) nibbles of
// the 16 bytes of the block (one shift, one mask per dword); B operand: the
// same 16 elements of the activation row of token l%32.  The accumulator is
// seeded with 0x4B400000 so the integer sum arrives as the float F.  Lane l's
// 16 results of a tile are rows 8a + 4(l/32) + e (a, e = 0..3) of token l%32.
// Staging, 4 blocks per stage in two LDS stages: weight and activation quants
// by LDS DMA (no staging registers), the fp16 weight scales (each 32-row tile
// permuted so that the 16 rows a lane needs are contiguous: two 16-byte
// reads) and the (d8, 8 sum) token scales through registers; the next stage's
// loads are issued right after the stage barrier and land during the compute.
// 60 KB of LDS and at most 128 VGPRs: 2 workgroups, 4 waves per SIMD.
// Workgroups are mapped to tiles XCD by XCD (each XCD's L2 holds a few token
// tiles' activations).  The output tile is written as float4 (4 consecutive
// rows of one token).  Needs N % 128 == 0 and bpr % 8 == 0, as the
// reference's pf_gemm_dense does (PF_BM = 128).
#include "lk_common.h"

#define PFG_BM 128                 // weight rows per workgroup
#define PFG_BN 128                 // tokens per workgroup
#define PFG_KC 4                   // blocks per LDS stage (the staging below moves exactly 4)
#ifndef PFG_ABL
#define PFG_ABL 0                  // measurement builds only: 1 no loads after stage 0, 2 no MFMA, 4 one add, 8 no store
#endif

typedef int lk_i4g __attribute__((ext_vector_type(4)));
typedef int lk_i16g __attribute__((ext_vector_type(16)));
typedef float lk_f16g __attribute__((ext_vector_type(16)));

// One stage = 4 blocks.  a and b are filled by LDS DMA, 16 bytes per lane in
// lane order, so their layouts are 16-byte slots: a[block][row] (the 16 quant
// bytes of a weight block), b[block][half][token] (activation elements
// 16*half .. +15 of a block).  The operand reads of 32 consecutive rows or
// tokens are then 32 consecutive slots (conflict-free).
struct alignas(16) PfgStage {
    uint8_t  a[PFG_KC * PFG_BM * 16];        // 8 KB
    int8_t   b[PFG_KC * 2 * PFG_BN * 16];    // 16 KB
    _Float16 d[PFG_KC][PFG_BM];              // weight scales [block][row, permuted within 32-row tiles]
    float2   s[PFG_BN][PFG_KC + 1];          // token scales (d8, 8 sum) [token][block]; the pad spreads 32 tokens over the banks
};

// Position of row r (within a 32-row tile) in the permuted scale layout:
// r = 8a + 4h + e  ->  16h + 4a + e, so lane half h finds its 16 rows
// (a, e = 0..3) at 16h .. 16h+15.
__device__ __forceinline__ int pfg_dperm(int r) {
    return (r & ~31) | ((r & 4) << 2) | ((r >> 3 & 3) << 2) | (r & 3);
}

template <bool ADD>
__global__ void __launch_bounds__(512, 4)
lk_k_pf_gemm_q4_0(const uint8_t * __restrict__ qs, const _Float16 * __restrict__ d, int N, int bpr,
                  const int8_t * __restrict__ aqs, const float2 * __restrict__ asc, int ntok,
                  const float * __restrict__ scale, float * __restrict__ out, int out_ld) {
#pragma clang fp contract(off)
    __shared__ PfgStage stg[2];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // XCD-aware tile order: workgroups are dispatched round-robin over the 8
    // XCDs (id % 8), so consecutive tile indices L are given to one XCD and L
    // runs over the row tiles first: an XCD holds a few token tiles with all
    // row tiles, and its L2 fetches each activation row once instead of every
    // XCD fetching all of them.
    const int nrt = N / PFG_BM, ntile = gridDim.x;
    const int id = blockIdx.x;
    const int L = (ntile % 8 == 0) ? (id % 8) * (ntile / 8) + id / 8 : id;
    const int row0 = (L % nrt) * PFG_BM, tok0 = (L / nrt) * PFG_BN;
    const int wr = (w & 3) * 32, wt = (w >> 2) * 64;   // the wave's 32 x 64 sub-tile
    const int l32 = lane & 31, h = lane >> 5;
    constexpr float MAGIC = 12582912.0f;               // 1.5 * 2^23 = float bits 0x4B400000

    // ---- staging (4 blocks per stage).  LDS DMA: wave w brings block w/2 of
    // weight rows 64(w%2) .. +63 (one instruction) and half w%2 of block w/2
    // of all 128 tokens (two); through registers: for t < 128 the 4 fp16
    // scales of weight row t, and block t%4 of token t/4's scale pair.
    static_assert(PFG_KC == 4 && PFG_BM == 128 && PFG_BN == 128, "the staging assignment below");
    const int sb = w >> 1, sh = w & 1;                 // this wave's DMA block and row half / token half
    const uint32_t a_off = (uint32_t) ((64 * sh + lane) * bpr * 16 + 16 * sb);
    uint32_t b_off[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int t = tok0 + 64 * k + lane;
        b_off[k] = (uint32_t) ((t < ntok ? t : ntok - 1) * bpr * 32 + 32 * sb + 16 * sh);   // clamped: in bounds
    }
    const uint8_t * a_base = qs + (size_t) row0 * bpr * 16;
    const int bt = tid >> 2, bq = tid & 3;
    const int stok = (tok0 + bt < ntok) ? tok0 + bt : ntok - 1;
    const _Float16 * gd = d + (size_t) (row0 + (tid & 127)) * bpr;                    // + kb0 (tid < 128)
    const float2 * gs = asc + (size_t) stok * bpr + bq;                               // + kb0
    const int dp = pfg_dperm(tid & 127);
    uint2 rs, rd = make_uint2(0, 0);
    auto fetch = [&](int kb0, PfgStage & S) {
        lk_dma16c_so(a_base + 16 * kb0, a_off, lk_lds_addr(S.a + (sb * PFG_BM + 64 * sh) * 16));
#pragma unroll
        for (int k = 0; k < 2; ++k)
            lk_dma16c_so(aqs + 32 * kb0, b_off[k], lk_lds_addr(S.b + ((2 * sb + sh) * PFG_BN + 64 * k) * 16));
        if (tid < 128) rd = *(const uint2 *) (gd + kb0);
        rs = *(const uint2 *) (gs + kb0);
    };
    auto stash = [&](PfgStage & S) {
        if (tid < 128) {
            S.d[0][dp] = __builtin_bit_cast(_Float16, (unsigned short) (rd.x & 0xffff));
            S.d[1][dp] = __builtin_bit_cast(_Float16, (unsigned short) (rd.x >> 16));
            S.d[2][dp] = __builtin_bit_cast(_Float16, (unsigned short) (rd.y & 0xffff));
            S.d[3][dp] = __builtin_bit_cast(_Float16, (unsigned short) (rd.y >> 16));
        }
        S.s[bt][bq] = make_float2(__uint_as_float(rs.x), __uint_as_float(rs.y));
    };

    const int mb = 0x4B400000;
    const lk_i16g seed = { mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb, mb };
    const int nsh = 4 * h;                             // low or high nibbles
    lk_f16g acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;

    // One barrier per stage: the DMA into stage (ck+1)&1 is issued after the
    // barrier of stage ck, which every wave reaches only when done reading
    // stage ck-1 (the same buffer); the register-staged scales of stage ck go
    // into a buffer last read at ck-2.
    const int nck = bpr / PFG_KC;
    fetch(0, stg[0]);
    for (int ck = 0; ck < nck; ++ck) {
        PfgStage & S = stg[ck & 1];
        lk_wait_vm<0>();                               // this wave's DMA and scale loads of stage ck
        stash(S);
        __syncthreads();
        if (ck + 1 < nck && !((PFG_ABL & 1) && ck > 0)) fetch((ck + 1) * PFG_KC, stg[(ck + 1) & 1]);
#pragma unroll
        for (int b = 0; b < PFG_KC; ++b) {
            const uint4 q = *(const uint4 *) (S.a + (b * PFG_BM + wr + l32) * 16);
            const lk_i4g a = { (int) ((q.x >> nsh) & 0x0F0F0F0Fu), (int) ((q.y >> nsh) & 0x0F0F0F0Fu),
                               (int) ((q.z >> nsh) & 0x0F0F0F0Fu), (int) ((q.w >> nsh) & 0x0F0F0F0Fu) };
            // d4 of this lane's 16 rows of the row tile (fp16, two 16-byte reads)
            const lk_h8 d4lo = *(const lk_h8 *) &S.d[b][wr + 16 * h];
            const lk_h8 d4hi = *(const lk_h8 *) &S.d[b][wr + 16 * h + 8];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const lk_i4g bv = *(const lk_i4g *) (S.b + ((2 * b + h) * PFG_BN + wt + 32 * j + l32) * 16);
                const lk_f16g F = (PFG_ABL & 2) ? __builtin_bit_cast(lk_f16g, (lk_i16g){ a[0], a[1], a[2], a[3], bv[0], bv[1], bv[2], bv[3], a[0], a[1], a[2], a[3], bv[0], bv[1], bv[2], bv[3] })
                                                : __builtin_bit_cast(lk_f16g, __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bv, seed, 0, 0, 0));
                const float2 sv = S.s[wt + 32 * j + l32][b];
                const float c = __builtin_fmaf(sv.x, MAGIC, sv.y);
#pragma unroll
                for (int e = 0; e < 16; ++e)           // result e = row 8(e/4) + 4h + e%4 = scale slot e
                    acc[j][e] = (PFG_ABL & 4) ? acc[j][e] + F[e] :
                                __builtin_fmaf((float) (e < 8 ? d4lo[e] : d4hi[e - 8]),
                                               __builtin_fmaf(sv.x, F[e], -c), acc[j][e]);
            }
        }
    }
    // epilogue: lane holds rows 8a + 4h .. +3 of the row tile for token l32 of each token tile
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int t = tok0 + wt + 32 * j + l32;
        if (t >= ntok) continue;
        const float sc = scale ? scale[t] : 1.0f;
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
            float4 * p = (float4 *) (out + (size_t) t * out_ld + row0 + wr + 8 * a4 + 4 * h);
            float4 v = make_float4(acc[j][4 * a4] * sc, acc[j][4 * a4 + 1] * sc,
                                   acc[j][4 * a4 + 2] * sc, acc[j][4 * a4 + 3] * sc);
            if (ADD) {
                const float4 o = *p;
                v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
            if (!(PFG_ABL & 8) || v.x == 1234.5f) *p = v;
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
    // the kernel addresses activation rows with 32-bit byte offsets
    if ((size_t) ntok * bpr * 32 > 0xFFFFFFFFull)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: ntok %d x bpr %d activations exceed 4 GiB", ntok, bpr);
    if (!qs || !d || !aqs || !asc || !out)
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: null pointer argument");
    // the widths the kernel loads and stores at: qs, aqs, asc and out 16 bytes, d 8 bytes, scale 4
    if (((uintptr_t) qs & 15) || ((uintptr_t) d & 7) || ((uintptr_t) aqs & 15) || ((uintptr_t) asc & 15) ||
        ((uintptr_t) out & 15) || ((uintptr_t) scale & 3))
        return lk_fail(hipErrorInvalidValue, "lk_pf_gemm_q4_0: misaligned argument (qs, aqs, asc, out 16 B; d 8 B; scale 4 B)");
    const dim3 grid((N / PFG_BM) * ((ntok + PFG_BN - 1) / PFG_BN));
    const hipStream_t st = lk_stream(stream);
    if (add)
        hipLaunchKernelGGL(lk_k_pf_gemm_q4_0<true>, grid, dim3(512), 0, st, (const uint8_t *) qs, (const _Float16 *) d,
                           N, bpr, aqs, (const float2 *) asc, ntok, scale, out, out_ld);
    else
        hipLaunchKernelGGL(lk_k_pf_gemm_q4_0<false>, grid, dim3(512), 0, st, (const uint8_t *) qs, (const _Float16 *) d,
                           N, bpr, aqs, (const float2 *) asc, ntok, scale, out, out_ld);
    return lk_launch_status("lk_pf_gemm_q4_0");
}
