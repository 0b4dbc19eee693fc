// prefill.hip - chunked causal prefill attention for gfx950: the int8
// quantisers, the K smoothing mean, and the int8/fp16 flash attention.
//
// Reference behaviour: k_pf_q8 / k_pf_k8 / k_pf_kmean / k_pf_attn8 / k_pf_attn
// (/root/reference/src/prefill.cu:1252-1318, 1337-1571, 1029-1226), launched
// from pf_chunk at engine.cu:1082-1089, 1122.
//
// Attention design (MI355X-first; the reference's mma.m16n8k32 warp tiling is
// not used):
//   * workgroup = 4 waves = the 4 query heads of one kv head, over 64 query
//     rows; every K/V tile staged in LDS therefore serves 256 query rows;
//   * scores are computed TRANSPOSED, S^T = K . Q^T, so that in the MFMA
//     result layout (lane l holds rows 4*(l/16)+r, column l%16) each lane owns
//     one query (column) and 4 keys per 16x16 block: the row max / row sum of
//     the softmax are lane-local plus two cross-lane steps, and the
//     probabilities are ALREADY in the B-operand layout of the next MFMA;
//   * O^T = V^T . P^T accumulates in fp32 on v_mfma_f32_16x16x32_f16, A = V^T
//     read from a transposed LDS copy of the V tile, B = P^T from registers
//     (the B operand's 8 key slots of lane group g are keys 4g..4g+3 of two
//     16-key blocks -- a permutation of the reduction index applied to both
//     operands alike);
//   * int8 tiles: one v_mfma_i32_16x16x64_i8 covers the whole head_dim per
//     16x16 block; int32 sums are exact, then s = (float)sum * ksc * qsc;
//   * exact tiles (within `near` of a 32-query tile, and tile 0 with `sink`,
//     reference prefill.cu:1380-1382): fp16 Q.K^T with fp32 accumulation,
//     s = sum * log2(e) - qcs;
//   * online softmax in the log2 domain with v_exp_f32; P rounded to fp16 for
//     P.V (as the reference does), accumulation in fp32 throughout.
#include "lk_common.h"
#include <math.h>

// ---------------------------------------------------------------------------
// int8 quantisers.  One wave per 64-wide (row, head), one value per lane.
// am = max|v| (exact: a maximum does not depend on order); d = am/127 and
// 127/am are IEEE-correct fp32 divisions; q = round-to-nearest-even(v * id)
// (reference prefill.cu:1255-1267).  Bit-exact by construction.
__device__ __forceinline__ void lk_q8_row(float v, int8_t * __restrict__ dst,
                                          float * __restrict__ scl, float mul) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    float am = fabsf(v);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, 64));
    const float d = am / 127.0f;
    const float id = (am > 0.0f) ? 127.0f / am : 0.0f;
    const float x = v * id;
    dst[lane] = (int8_t) (int) __builtin_rintf(x);
    if (lane == 0) *scl = d * mul;
}

// Q: qh fp16 [m][2048] -> q8 [m][2048], qsc [m][32] = d*log2(e), qcs [m][32] =
// (q.c)*log2(e) where q.c is the lane products v_d*c_d summed by an xor
// butterfly 32,16,8,4,2,1 (fixed order), or 0 without cm.
__global__ void __launch_bounds__(256)
lk_k_pf_q8(const _Float16 * __restrict__ qh, int m, const float * __restrict__ cm,
           int8_t * __restrict__ q8, float * __restrict__ qsc, float * __restrict__ qcs) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= m * LK_N_HEADS) return;                      // wave-uniform
    const float v = (float) qh[(size_t) r * LK_HEAD_DIM + lane];
    lk_q8_row(v, q8 + (size_t) r * LK_HEAD_DIM, qsc + r, LK_LOG2E_F);
    float qc = 0.0f;
    if (cm) {
        qc = v * cm[((r % LK_N_HEADS) / LK_G) * LK_HEAD_DIM + lane];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) qc += __shfl_xor(qc, o, 64);
    }
    if (lane == 0) qcs[r] = qc * LK_LOG2E_F;
}

// K: positions [p0, p1) of kc [pos][8][64] -> k8 (same layout), ksc[h][pos].
__global__ void __launch_bounds__(256)
lk_k_pf_k8(const _Float16 * __restrict__ kc, int p0, int p1, const float * __restrict__ cm,
           int kstride, int8_t * __restrict__ k8, float * __restrict__ ksc) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int pos = p0 + r / LK_N_KV_HEADS, h = r % LK_N_KV_HEADS;
    if (pos >= p1) return;                                // wave-uniform
    const size_t row = (size_t) pos * LK_N_KV_HEADS + h;
    float v = (float) kc[row * LK_HEAD_DIM + lane];
    if (cm) v -= cm[h * LK_HEAD_DIM + lane];
    lk_q8_row(v, k8 + row * LK_HEAD_DIM, ksc + (size_t) h * kstride + pos, 1.0f);
}

// cm[h][d] = mean of kc over positions [0, n).  The summation order is the
// reference's (prefill.cu:1304-1318): 16 strided fp32 running sums (p = g,
// g+16, ...), then those 16 added in index order, then / n -- kept identical
// so the smoothing vector matches the reference bit for bit.
__global__ void __launch_bounds__(1024)
lk_k_pf_kmean(const _Float16 * __restrict__ kc, int n, float * __restrict__ cm) {
#pragma clang fp contract(off)
    __shared__ float part[16][LK_HEAD_DIM];
    const int h = blockIdx.x, d = threadIdx.x & 63, g = threadIdx.x >> 6;
    float s = 0.0f;
    for (int p = g; p < n; p += 16) s += (float) kc[((size_t) p * LK_N_KV_HEADS + h) * LK_HEAD_DIM + d];
    part[g][d] = s;
    __syncthreads();
    if (g == 0) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) t += part[i][d];
        cm[h * LK_HEAD_DIM + d] = t / (float) n;
    }
}

// ---------------------------------------------------------------------------
// Flash attention.
#define PF_BQ      64                     // query rows per workgroup (16 per block)
#define PF_BK      32                     // keys per tile (two 16-key blocks)
#define PF_QB      (PF_BQ / 16)
#define PF_K8_LD   80                     // LDS row pitch (bytes) of the int8 K tile
#define PF_KH_LD   144                    // LDS row pitch (bytes) of the fp16 K tile
#define PF_V_LD    144                    // LDS row pitch (bytes) of the fp16 V tile
#define PF_Q_LD    144                    // LDS row pitch (bytes) of the fp16 Q block

struct alignas(16) PfStage {
    int8_t   k8[PF_BK * PF_K8_LD];        // [key][64 B + pad]
    int8_t   kh[PF_BK * PF_KH_LD];        // [key][64 fp16 + pad]
    int8_t   v[PF_BK * PF_V_LD];          // [key][64 fp16 + pad], row-major
    float    ks[PF_BK];                   // int8 K scales of the tile
};

// Exact-tile predicate of the reference (prefill.cu:1380-1382), stated on its
// 64-key tiles: tile kt64 is exact for the 32-query tile qt32 iff
// kt64*64 + 64 > P + qt32*32 - near, or sink and kt64 == 0.
__device__ __forceinline__ bool lk_pf_exact(int P, int qt32, int kt64, int near, int sink) {
    return (kt64 * 64 + 64 > P + qt32 * 32 - near) || (sink && kt64 == 0);
}

// The int32 S^T block of 16 keys x 16 queries over the full head_dim: A = 16
// key rows (lane l: key l%16, bytes 16g..16g+15), B = Q^T (lane l: query l%16,
// the same bytes).  Shared by the attention kernel and the test hook.
__device__ __forceinline__ lk_i4 lk_mfma_qk8(lk_i4 kfrag, lk_i4 qfrag) {
    const lk_i4 z = { 0, 0, 0, 0 };
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(kfrag, qfrag, z, 0, 0, 0);
}

template <bool INT8>
__global__ void __launch_bounds__(256, 2)
lk_k_pf_attn(const int8_t * __restrict__ q8, const float * __restrict__ qsc,
             const float * __restrict__ qcs, const _Float16 * __restrict__ qh, int m, int P,
             const int8_t * __restrict__ k8, const float * __restrict__ ksc, int kstride,
             const _Float16 * __restrict__ kc, const _Float16 * __restrict__ vc,
             int near, int sink, float * __restrict__ o) {
    __shared__ PfStage st[2];
    __shared__ __attribute__((aligned(16))) int8_t s_q[4][PF_BQ * PF_Q_LD];   // fp16 Q, per head
    // Causal work grows with the query block.  Workgroups are dispatched in
    // linear order and the second half of the grid lands beside the first half
    // on the CUs, so kv heads 0-3 take the query blocks longest-first and kv
    // heads 4-7 shortest-first: co-resident workgroups then pair a long block
    // with a short one.
    const int kvh  = blockIdx.y;
    const int qt   = (kvh < LK_N_KV_HEADS / 2) ? (int) (gridDim.x - 1 - blockIdx.x) : (int) blockIdx.x;
    const int tid  = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int col  = lane & 15, g = lane >> 4;
    const int head = kvh * LK_G + w;
    const int qbase = qt * PF_BQ;
    const int qlast = (qbase + PF_BQ < m) ? (qbase + PF_BQ) : m;
    const int kend = P + qlast;
    const int nkt = (kend + PF_BK - 1) / PF_BK;
    const int qt32_lo = qbase / 32, qt32_hi = qbase / 32 + 1;   // qb 0-1, qb 2-3

    // ---- this wave's fp16 Q block (64 rows x 128 B) into LDS, for exact tiles --
    {
        const lk_h8 z8 = { 0, 0, 0, 0, 0, 0, 0, 0 };
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = (lane >> 3) + 8 * i, c = lane & 7;
            const int qr = qbase + r;
            const lk_h8 v = (qr < m) ? *(const lk_h8 *) (qh + (size_t) qr * LK_HIDDEN + head * LK_HEAD_DIM + 8 * c) : z8;
            *(lk_h8 *) (s_q[w] + r * PF_Q_LD + 16 * c) = v;
        }
    }
    // ---- int8 Q operands and per-query scalars (lane column = query) ----------
    lk_i4 qf8[PF_QB];
    float sq[PF_QB], isq[PF_QB], qc[PF_QB];
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) {
        const int qr = qbase + 16 * qb + col;
        const bool ok = qr < m;
        const lk_i4 zi = { 0, 0, 0, 0 };
        if (INT8) {
            qf8[qb] = ok ? *(const lk_i4 *) (q8 + (size_t) qr * LK_HIDDEN + head * LK_HEAD_DIM + 16 * g) : zi;
            const float d = ok ? qsc[(size_t) qr * LK_N_HEADS + head] : 0.0f;
            // scores are kept in units of 1/sq until the exponent (sq > 0 scales
            // commute with the max); an all-zero query row has sq = 0 and zero
            // int8 scores, so unit scaling is exact for it
            sq[qb] = (d > 0.0f) ? d : 1.0f;
            isq[qb] = 1.0f / sq[qb];
            qc[qb] = (ok && qcs) ? qcs[(size_t) qr * LK_N_HEADS + head] : 0.0f;
        } else {
            qf8[qb] = zi; sq[qb] = 1.0f; isq[qb] = 1.0f; qc[qb] = 0.0f;
        }
    }

    // ---- tile staging: global -> registers -> LDS ------------------------------
    // K8: threads 0..127 -> key t/4, 16-byte chunk t%4; threads 128..135 the
    // 32 scales.  Kh and V: every thread one 16-byte chunk, key t/8, chunk t%8.
    lk_i4 rk8, rkh, rv;
    const float * ks_h = INT8 ? ksc + (size_t) kvh * kstride : nullptr;
    auto tile_exact = [&](int kt, int qt32) {
        return !INT8 || lk_pf_exact(P, qt32, (kt * PF_BK) / 64, near, sink);
    };
    auto load_regs = [&](int kt) {
        const int kb0 = kt * PF_BK;
        const lk_i4 zi = { 0, 0, 0, 0 };
        if (INT8 && !tile_exact(kt, qt32_hi)) {
            if (tid < 128) {
                const int kpos = kb0 + (tid >> 2);
                rk8 = (kpos < kend) ? *(const lk_i4 *) (k8 + ((size_t) kpos * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 16 * (tid & 3)) : zi;
            } else if (tid < 136) {
                const int sp = kb0 + 4 * (tid - 128);
                rk8 = (sp < kend) ? *(const lk_i4 *) (ks_h + sp) : zi;
            }
        }
        const int kpos = kb0 + (tid >> 3);
        const size_t goff = ((size_t) kpos * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 8 * (tid & 7);
        if (tile_exact(kt, qt32_lo))
            rkh = (kpos < kend) ? *(const lk_i4 *) (kc + goff) : zi;
        rv = (kpos < kend) ? *(const lk_i4 *) (vc + goff) : zi;
    };
    auto store_lds = [&](int kt, PfStage & S) {
        if (INT8 && !tile_exact(kt, qt32_hi)) {
            if (tid < 128) *(lk_i4 *) (S.k8 + (tid >> 2) * PF_K8_LD + 16 * (tid & 3)) = rk8;
            else if (tid < 136) *(lk_i4 *) (S.ks + 4 * (tid - 128)) = rk8;
        }
        if (tile_exact(kt, qt32_lo)) *(lk_i4 *) (S.kh + (tid >> 3) * PF_KH_LD + 16 * (tid & 7)) = rkh;
        *(lk_i4 *) (S.v + (tid >> 3) * PF_V_LD + 16 * (tid & 7)) = rv;
    };

    // O^T blocks [dim block][query block]; block 4 multiplies P^T by an
    // all-ones A operand, so every lane of query column q accumulates
    // l_q = sum of the same fp16 P the numerator uses.
    lk_f4 acc[5][PF_QB];
#pragma unroll
    for (int db = 0; db < 5; ++db)
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) acc[db][qb] = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
    float mrun[PF_QB];                      // running max, units of 1/sq
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) mrun[qb] = -INFINITY;
    const _Float16 one = (_Float16) 1.0f;
    const lk_h8 ones = { one, one, one, one, one, one, one, one };
    // The running max is only raised when a score exceeds it by more than
    // 2^PF_HEADROOM in p (so most tiles skip the rescale); p <= 2^8 stays far
    // inside fp16 range and loses no relative precision.
    constexpr float PF_HEADROOM = 8.0f;

    load_regs(0);
    store_lds(0, st[0]);
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        if (kt + 1 < nkt) load_regs(kt + 1);
        const PfStage & S = st[kt & 1];
        const int kb0 = kt * PF_BK;
        const bool ex_lo = tile_exact(kt, qt32_lo);
        const bool ex_hi = tile_exact(kt, qt32_hi);

        // ---- scores S^T[kb][qb] (keys kb0+16kb+4g+r, query 16qb+col), x-units ----
        float x[2][PF_QB][4];
        if (ex_lo) {
            lk_h8 ka[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    ka[kb][ks] = *(const lk_h8 *) (S.kh + (16 * kb + col) * PF_KH_LD + 64 * ks + 16 * g);
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const bool ex = (qb < 2) ? ex_lo : ex_hi;
                if (!ex) continue;
                const int8_t * qrow = s_q[w] + (16 * qb + col) * PF_Q_LD + 16 * g;
                const lk_h8 qf0 = *(const lk_h8 *) qrow;
                const lk_h8 qf1 = *(const lk_h8 *) (qrow + 64);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    lk_f4 c = { 0.f, 0.f, 0.f, 0.f };
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][0], qf0, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][1], qf1, c, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        x[kb][qb][r] = INT8 ? fmaf(c[r], LK_LOG2E_F, -qc[qb]) * isq[qb] : c[r] * LK_LOG2E_F;
                }
            }
        }
        if (INT8 && !ex_hi) {
            lk_i4 ka8[2];
            float4 skv[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                ka8[kb] = *(const lk_i4 *) (S.k8 + (16 * kb + col) * PF_K8_LD + 16 * g);
                skv[kb] = *(const float4 *) (S.ks + 16 * kb + 4 * g);
            }
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const bool ex = (qb < 2) ? ex_lo : ex_hi;
                if (ex) continue;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const lk_i4 c = lk_mfma_qk8(ka8[kb], qf8[qb]);
                    x[kb][qb][0] = (float) c[0] * skv[kb].x;
                    x[kb][qb][1] = (float) c[1] * skv[kb].y;
                    x[kb][qb][2] = (float) c[2] * skv[kb].z;
                    x[kb][qb][3] = (float) c[3] * skv[kb].w;
                }
            }
        }

        // ---- causal mask (only tiles that reach past the block's first query) ---
        if (kb0 + PF_BK - 1 > P + qbase) {
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const int qpos = P + qbase + 16 * qb + col;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kb0 + 16 * kb + 4 * g + r > qpos) x[kb][qb][r] = -INFINITY;
            }
        }

        // ---- online softmax, per query (lane column); exponent = sq * (x - m) ---
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) {
            float mx = fmaxf(fmaxf(fmaxf(x[0][qb][0], x[0][qb][1]), fmaxf(x[0][qb][2], x[0][qb][3])),
                             fmaxf(fmaxf(x[1][qb][0], x[1][qb][1]), fmaxf(x[1][qb][2], x[1][qb][3])));
            mx = lk_xrow_max(mx);
            // key 0 is visible to every query, so mrun is finite after tile 0
            const bool need = mx > mrun[qb] + PF_HEADROOM * isq[qb];
            if (__ballot(need)) {                              // wave-uniform branch
                const float alpha = need ? lk_exp2((mrun[qb] - mx) * sq[qb]) : 1.0f;
                mrun[qb] = need ? mx : mrun[qb];
#pragma unroll
                for (int db = 0; db < 5; ++db) acc[db][qb] *= alpha;
            }
            const float msq = mrun[qb] * sq[qb];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) x[kb][qb][r] = lk_exp2(fmaf(x[kb][qb][r], sq[qb], -msq));
        }

        // ---- O^T += V^T . P^T over the 32 keys -----------------------------------
        lk_h8 pb[PF_QB];
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pb[qb][r]     = (_Float16) x[0][qb][r];
                pb[qb][4 + r] = (_Float16) x[1][qb][r];
            }
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int8_t * vp = S.v + (col >> 2) * PF_V_LD + 2 * (16 * db + 4 * (col & 3));
            const lk_h4 lo = lk_ds_tr4(vp + (4 * g) * PF_V_LD);
            const lk_h4 hi = lk_ds_tr4(vp + (16 + 4 * g) * PF_V_LD);
            const lk_h8 va = { lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3] };
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb)
                acc[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[qb], acc[db][qb], 0, 0, 0);
        }
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb)
            acc[4][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[qb], acc[4][qb], 0, 0, 0);

        if (kt + 1 < nkt) store_lds(kt + 1, st[(kt + 1) & 1]);
        __syncthreads();
    }

    // ---- epilogue: l over the 4 lane groups, then o[q][head*64 + d] -------------
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) {
        const float il = 1.0f / acc[4][qb][0];
        const int qr = qbase + 16 * qb + col;
        if (qr < m) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const lk_f4 a = acc[db][qb] * il;
                *(float4 *) (o + (size_t) qr * LK_HIDDEN + head * LK_HEAD_DIM + 16 * db + 4 * g) =
                    make_float4(a[0], a[1], a[2], a[3]);
            }
        }
    }
}

// Test hook: s[h][i][j] = int32 q8[i][h] . k8[j][h/4], one wave per 16x16 block.
__global__ void __launch_bounds__(64)
lk_k_pf_qk_i32(const int8_t * __restrict__ q8, int m, const int8_t * __restrict__ k8, int n,
               int32_t * __restrict__ s) {
    const int j0 = blockIdx.x * 16, i0 = blockIdx.y * 16, h = blockIdx.z;
    const int lane = threadIdx.x, col = lane & 15, g = lane >> 4;
    const lk_i4 kf = *(const lk_i4 *) (k8 + ((size_t) (j0 + col) * LK_N_KV_HEADS + h / LK_G) * LK_HEAD_DIM + 16 * g);
    const lk_i4 qf = *(const lk_i4 *) (q8 + (size_t) (i0 + col) * LK_HIDDEN + h * LK_HEAD_DIM + 16 * g);
    const lk_i4 c = lk_mfma_qk8(kf, qf);         // c[r] = S^T[key j0+4g+r][query i0+col]
#pragma unroll
    for (int r = 0; r < 4; ++r)
        s[((size_t) h * m + i0 + col) * n + j0 + 4 * g + r] = c[r];
}

// ---------------------------------------------------------------------------
// C ABI
extern "C" int lk_pf_q8(const void * qh, int m, const float * cm, int8_t * q8,
                        float * qsc, float * qcs, void * stream) {
    if (m < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_q8: m < 0");
    if (m == 0) return 0;
    if (!qh || !q8 || !qsc || !qcs) return lk_fail(hipErrorInvalidValue, "lk_pf_q8: null pointer argument");
    const int rows = m * LK_N_HEADS;
    hipLaunchKernelGGL(lk_k_pf_q8, dim3((rows + 3) / 4), dim3(256), 0, lk_stream(stream),
                       (const _Float16 *) qh, m, cm, q8, qsc, qcs);
    return lk_launch_status("lk_pf_q8");
}

extern "C" int lk_pf_k8(const void * kc, int p0, int p1, const float * cm, int kstride,
                        int8_t * k8, float * ksc, void * stream) {
    if (p0 < 0 || p1 < p0) return lk_fail(hipErrorInvalidValue, "lk_pf_k8: bad range [%d, %d)", p0, p1);
    if (kstride % 4 != 0 || kstride < p1)
        return lk_fail(hipErrorInvalidValue, "lk_pf_k8: kstride %d must be a multiple of 4 and >= p1 %d", kstride, p1);
    if (p1 == p0) return 0;
    if (!kc || !k8 || !ksc) return lk_fail(hipErrorInvalidValue, "lk_pf_k8: null pointer argument");
    const long rows = (long) (p1 - p0) * LK_N_KV_HEADS;
    hipLaunchKernelGGL(lk_k_pf_k8, dim3((unsigned) ((rows + 3) / 4)), dim3(256), 0, lk_stream(stream),
                       (const _Float16 *) kc, p0, p1, cm, kstride, k8, ksc);
    return lk_launch_status("lk_pf_k8");
}

extern "C" int lk_pf_kmean(const void * kc, int n, float * cm, void * stream) {
    if (n <= 0) return lk_fail(hipErrorInvalidValue, "lk_pf_kmean: n must be > 0");
    if (!kc || !cm) return lk_fail(hipErrorInvalidValue, "lk_pf_kmean: null pointer argument");
    hipLaunchKernelGGL(lk_k_pf_kmean, dim3(LK_N_KV_HEADS), dim3(1024), 0, lk_stream(stream),
                       (const _Float16 *) kc, n, cm);
    return lk_launch_status("lk_pf_kmean");
}

extern "C" int lk_pf_attn8(const int8_t * q8, const float * qsc, const float * qcs,
                           const void * qh, int m, int P, const int8_t * k8,
                           const float * ksc, int kstride, const void * kc,
                           const void * vc, int near, int sink, float * o, void * stream) {
    if (m < 0 || P < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: m %d / P %d negative", m, P);
    if (m == 0) return 0;
    if (kstride % 4 != 0 || kstride < P + m)
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: kstride %d must be a multiple of 4 and >= P+m %d", kstride, P + m);
    if (!q8 || !qsc || !qh || !k8 || !ksc || !kc || !vc || !o)
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: null pointer argument");
    hipLaunchKernelGGL(lk_k_pf_attn<true>, dim3((m + PF_BQ - 1) / PF_BQ, LK_N_KV_HEADS), dim3(256), 0,
                       lk_stream(stream), q8, qsc, qcs, (const _Float16 *) qh, m, P, k8, ksc, kstride,
                       (const _Float16 *) kc, (const _Float16 *) vc, near, sink, o);
    return lk_launch_status("lk_pf_attn8");
}

extern "C" int lk_pf_attn(const void * qh, int m, int P, const void * kc, const void * vc,
                          float * o, void * stream) {
    if (m < 0 || P < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_attn: m %d / P %d negative", m, P);
    if (m == 0) return 0;
    if (!qh || !kc || !vc || !o) return lk_fail(hipErrorInvalidValue, "lk_pf_attn: null pointer argument");
    hipLaunchKernelGGL(lk_k_pf_attn<false>, dim3((m + PF_BQ - 1) / PF_BQ, LK_N_KV_HEADS), dim3(256), 0,
                       lk_stream(stream), (const int8_t *) nullptr, (const float *) nullptr,
                       (const float *) nullptr, (const _Float16 *) qh, m, P, (const int8_t *) nullptr,
                       (const float *) nullptr, 0, (const _Float16 *) kc, (const _Float16 *) vc, 0, 0, o);
    return lk_launch_status("lk_pf_attn");
}

extern "C" int lk_pf_qk_i32(const int8_t * q8, int m, const int8_t * k8, int n,
                            int32_t * s, void * stream) {
    if (m <= 0 || n <= 0 || m % 16 || n % 16)
        return lk_fail(hipErrorInvalidValue, "lk_pf_qk_i32: m %d, n %d must be positive multiples of 16", m, n);
    if (!q8 || !k8 || !s) return lk_fail(hipErrorInvalidValue, "lk_pf_qk_i32: null pointer argument");
    hipLaunchKernelGGL(lk_k_pf_qk_i32, dim3(n / 16, m / 16, LK_N_HEADS), dim3(64), 0, lk_stream(stream),
                       q8, m, k8, n, s);
    return lk_launch_status("lk_pf_qk_i32");
}
