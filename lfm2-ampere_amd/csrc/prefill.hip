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
#define PF_BQ      64                     // query rows per workgroup
#define PF_BK      64                     // keys per tile
#define PF_QB      (PF_BQ / 16)           // 16-query blocks per wave
#define PF_K8_LD   80                     // LDS row pitch (bytes) of the int8 K tile
#define PF_KH_LD   72                     // LDS row pitch (halves) of the fp16 K tile
#define PF_VT_LD   68                     // LDS row pitch (halves) of the V^T tile

struct alignas(16) PfStage {
    int8_t   k8[PF_BK * PF_K8_LD];        // [key][64 B + pad]
    _Float16 kh[PF_BK * PF_KH_LD];        // [key][64 + pad]
    _Float16 vt[LK_HEAD_DIM * PF_VT_LD];  // [dim][64 keys + pad]
    float    ks[PF_BK];                   // int8 K scales of the tile
};

__device__ __forceinline__ bool lk_pf_exact(int P, int qt32, int kt, int near, int sink) {
    return (kt * PF_BK + PF_BK > P + qt32 * 32 - near) || (sink && kt == 0);
}

// The int32 S^T block of 16 keys x 16 queries over the full head_dim: A = 16
// key rows (lane l: key l%16, bytes 16g..16g+15), B = Q^T (lane l: query l%16,
// the same bytes).  Shared by the attention kernel and the test hook.
__device__ __forceinline__ lk_i4 lk_mfma_qk8(lk_i4 kfrag, lk_i4 qfrag) {
    const lk_i4 z = { 0, 0, 0, 0 };
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(kfrag, qfrag, z, 0, 0, 0);
}

template <bool INT8>
__global__ void __launch_bounds__(256)
lk_k_pf_attn(const int8_t * __restrict__ q8, const float * __restrict__ qsc,
             const float * __restrict__ qcs, const _Float16 * __restrict__ qh, int m, int P,
             const int8_t * __restrict__ k8, const float * __restrict__ ksc, int kstride,
             const _Float16 * __restrict__ kc, const _Float16 * __restrict__ vc,
             int near, int sink, float * __restrict__ o) {
    __shared__ PfStage st[2];
    const int qt   = gridDim.x - 1 - blockIdx.x;        // longest rows first
    const int kvh  = blockIdx.y;
    const int tid  = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int col  = lane & 15, g = lane >> 4;
    const int head = kvh * LK_G + w;
    const int qbase = qt * PF_BQ;
    const int qlast = (qbase + PF_BQ < m) ? (qbase + PF_BQ) : m;
    const int kend = P + qlast;
    const int nkt = (kend + PF_BK - 1) / PF_BK;
    const int qt32_lo = qbase / 32, qt32_hi = qbase / 32 + 1;   // qb 0-1, qb 2-3

    // ---- this lane's query operands (B of S^T), one per 16-query block -------
    // The int8 fragments stay in registers; the fp16 ones are re-read (from L2)
    // on the few exact tiles only.
    lk_i4 qf8[PF_QB];
    float rq[PF_QB], qc[PF_QB];
    const _Float16 * qrow[PF_QB];
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) {
        const int qr = qbase + 16 * qb + col;
        const bool ok = qr < m;
        const size_t base = (size_t) (ok ? qr : 0) * LK_HIDDEN + head * LK_HEAD_DIM;
        qrow[qb] = ok ? qh + base : nullptr;
        if (INT8) {
            const lk_i4 zi = { 0, 0, 0, 0 };
            qf8[qb] = ok ? *(const lk_i4 *) (q8 + base + 16 * g) : zi;
            rq[qb] = ok ? qsc[(size_t) qr * LK_N_HEADS + head] : 0.0f;
            qc[qb] = (ok && qcs) ? qcs[(size_t) qr * LK_N_HEADS + head] : 0.0f;
        } else {
            rq[qb] = 0.0f; qc[qb] = 0.0f;
        }
    }

    // ---- tile staging: global -> registers -> LDS ------------------------------
    // K8: thread t -> key t/4, 16-byte chunk t%4.   Kh: two 16-byte chunks,
    // ids t and t+256 -> key id/8, chunk id%8.   V: key pair t/8 (keys 2p, 2p+1),
    // dims 8*(t%8)..+7, written transposed as 8 packed (key 2p, key 2p+1) words.
    lk_i4 rk8;
    lk_h8 rkh[2], rv[2];
    float4 rks;
    const int kp8 = tid >> 2, c8 = tid & 3;
    const int vkp = tid >> 3, vc8 = tid & 7;
    const float * ks_h = INT8 ? ksc + (size_t) kvh * kstride : nullptr;

    auto tile_needs_exact = [&](int kt) {
        return !INT8 || lk_pf_exact(P, qt32_lo, kt, near, sink);
    };
    auto tile_needs_int8 = [&](int kt) {
        return INT8 && !lk_pf_exact(P, qt32_hi, kt, near, sink);
    };
    auto load_regs = [&](int kt) {
        const int kb0 = kt * PF_BK;
        const lk_h8 z8 = { 0, 0, 0, 0, 0, 0, 0, 0 };
        if (tile_needs_int8(kt)) {
            const int kpos = kb0 + kp8;
            const lk_i4 zi = { 0, 0, 0, 0 };
            rk8 = (kpos < kend) ? *(const lk_i4 *) (k8 + ((size_t) kpos * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 16 * c8) : zi;
            if (tid < 16) {
                const int sp = kb0 + 4 * tid;
                rks = (sp < kend) ? *(const float4 *) (ks_h + sp) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        if (tile_needs_exact(kt)) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int id = tid + 256 * i;
                const int kpos = kb0 + (id >> 3);
                rkh[i] = (kpos < kend) ? *(const lk_h8 *) (kc + ((size_t) kpos * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 8 * (id & 7)) : z8;
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int kpos = kb0 + 2 * vkp + i;
            rv[i] = (kpos < kend) ? *(const lk_h8 *) (vc + ((size_t) kpos * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 8 * vc8) : z8;
        }
    };
    auto store_lds = [&](int kt, PfStage & S) {
        if (tile_needs_int8(kt)) {
            *(lk_i4 *) (S.k8 + kp8 * PF_K8_LD + 16 * c8) = rk8;
            if (tid < 16) *(float4 *) (S.ks + 4 * tid) = rks;
        }
        if (tile_needs_exact(kt)) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int id = tid + 256 * i;
                *(lk_h8 *) (S.kh + (id >> 3) * PF_KH_LD + 8 * (id & 7)) = rkh[i];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            h2 pr = { rv[0][e], rv[1][e] };
            *(h2 *) (S.vt + (8 * vc8 + e) * PF_VT_LD + 2 * vkp) = pr;
        }
    };

    lk_f4 acc[4][PF_QB];                    // O^T blocks [dim block][query block]
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) acc[db][qb] = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
    float mrun[PF_QB], lrun[PF_QB];
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) { mrun[qb] = -INFINITY; lrun[qb] = 0.0f; }

    load_regs(0);
    store_lds(0, st[0]);
    __syncthreads();

    for (int kt = 0; kt < nkt; ++kt) {
        if (kt + 1 < nkt) load_regs(kt + 1);
        const PfStage & S = st[kt & 1];
        const int kb0 = kt * PF_BK;
        const bool ex_lo = !INT8 || lk_pf_exact(P, qt32_lo, kt, near, sink);
        const bool ex_hi = !INT8 || lk_pf_exact(P, qt32_hi, kt, near, sink);

        // ---- scores S^T[kb][qb] (keys 16kb+4g+r, query 16qb+col) ----------------
        float s[4][PF_QB][4];
        if (ex_lo) {
            // fp16 K fragments of the tile (A operand), 2 k-steps of 32 dims
            lk_h8 ka[4][2];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int ks = 0; ks < 2; ++ks)
                    ka[kb][ks] = *(const lk_h8 *) (S.kh + (16 * kb + col) * PF_KH_LD + 32 * ks + 8 * g);
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const bool ex = (qb < 2) ? ex_lo : ex_hi;
                if (!ex) continue;
                const lk_h8 z8 = { 0, 0, 0, 0, 0, 0, 0, 0 };
                const lk_h8 qf0 = qrow[qb] ? *(const lk_h8 *) (qrow[qb] + 8 * g) : z8;
                const lk_h8 qf1 = qrow[qb] ? *(const lk_h8 *) (qrow[qb] + 32 + 8 * g) : z8;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    lk_f4 c = { 0.f, 0.f, 0.f, 0.f };
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][0], qf0, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[kb][1], qf1, c, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        s[kb][qb][r] = INT8 ? fmaf(c[r], LK_LOG2E_F, -qc[qb]) : c[r] * LK_LOG2E_F;
                }
            }
        }
        if (INT8 && !ex_hi) {
            lk_i4 ka8[4];
            float4 skv[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                ka8[kb] = *(const lk_i4 *) (S.k8 + (16 * kb + col) * PF_K8_LD + 16 * g);
                skv[kb] = *(const float4 *) (S.ks + 16 * kb + 4 * g);
            }
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const bool ex = (qb < 2) ? ex_lo : ex_hi;
                if (ex) continue;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const lk_i4 c = lk_mfma_qk8(ka8[kb], qf8[qb]);
                    s[kb][qb][0] = (float) c[0] * skv[kb].x * rq[qb];
                    s[kb][qb][1] = (float) c[1] * skv[kb].y * rq[qb];
                    s[kb][qb][2] = (float) c[2] * skv[kb].z * rq[qb];
                    s[kb][qb][3] = (float) c[3] * skv[kb].w * rq[qb];
                }
            }
        }

        // ---- causal mask (only tiles that reach past the block's first query) ---
        if (kb0 + PF_BK - 1 > P + qbase) {
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const int qpos = P + qbase + 16 * qb + col;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (kb0 + 16 * kb + 4 * g + r > qpos) s[kb][qb][r] = -INFINITY;
            }
        }

        // ---- online softmax (log2 domain), per query = per lane column ----------
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) {
            float mx = s[0][qb][0];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][qb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mnew = fmaxf(mrun[qb], mx);      // finite: key 0 is always visible
            const float alpha = lk_exp2(mrun[qb] - mnew);
            mrun[qb] = mnew;
            float ls = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = lk_exp2(s[kb][qb][r] - mnew);
                    s[kb][qb][r] = p;
                    ls += p;
                }
            lrun[qb] = lrun[qb] * alpha + ls;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db][qb] *= alpha;
        }

        // ---- O^T += V^T . P^T ---------------------------------------------------
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            lk_h8 pb[PF_QB];
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pb[qb][r]     = (_Float16) s[2 * ks][qb][r];
                    pb[qb][4 + r] = (_Float16) s[2 * ks + 1][qb][r];
                }
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const _Float16 * vrow = S.vt + (16 * db + col) * PF_VT_LD + 32 * ks + 4 * g;
                const lk_h4 lo = *(const lk_h4 *) vrow;
                const lk_h4 hi = *(const lk_h4 *) (vrow + 16);
                const lk_h8 va = { lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3] };
#pragma unroll
                for (int qb = 0; qb < PF_QB; ++qb)
                    acc[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[qb], acc[db][qb], 0, 0, 0);
            }
        }

        if (kt + 1 < nkt) store_lds(kt + 1, st[(kt + 1) & 1]);
        __syncthreads();
    }

    // ---- epilogue: l over the 4 lane groups, then o[q][head*64 + d] -------------
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) {
        float l = lrun[qb];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const float il = 1.0f / l;
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
