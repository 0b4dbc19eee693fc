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
#include <algorithm>
#include <type_traits>
#include <atomic>
#include <mutex>

// ---------------------------------------------------------------------------
// int8 quantisers.  Eight lanes per 64-wide (row, head), eight consecutive
// values per lane (one 16-byte load, one 8-byte store), eight rows per wave.
// am = max|v| (exact: a maximum does not depend on order); d = am/127 and
// 127/am are IEEE-correct fp32 divisions; q = round-to-nearest-even(v * id)
// (reference prefill.cu:1255-1267).  Bit-exact by construction.  The row
// helpers (lk_q8_row8, lk_max8, lk_load8h) live in lk_common.h.

// Q: qh fp16 [m][2048] -> q8 [m][2048], qsc [m][32] = d*log2(e), qcs [m][32] =
// (q.c)*log2(e), or 0 without cm.  q.c is summed in the reference's order
// (prefill.cu:1279-1284, a 32-lane warp with values 2l, 2l+1 in lane l): the
// pair sums s_k = v[2k]*c[2k] + v[2k+1]*c[2k+1], then the butterfly over k with
// offsets 16, 8, 4, 2, 1.  Here lane j of the 8-lane group holds pairs
// k = 4j..4j+3, so offsets 16, 8, 4 are lane exchanges xor 4, 2, 1 and offsets
// 2, 1 pair the lane's own sums: (s0 + s2) + (s1 + s3).
__global__ void __launch_bounds__(256)
lk_k_pf_q8(const _Float16 * __restrict__ qh, int m, const float * __restrict__ cm,
           int8_t * __restrict__ q8, float * __restrict__ qsc, float * __restrict__ qcs) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 32 + (threadIdx.x >> 3), j = threadIdx.x & 7;
    if (r >= m * LK_N_HEADS) return;                      // whole 8-lane groups
    float v[8];
    lk_load8h(qh + (size_t) r * LK_HEAD_DIM + 8 * j, v);
    lk_q8_row8(v, q8 + (size_t) r * LK_HEAD_DIM + 8 * j, qsc + r, LK_LOG2E_F, j == 0);
    float qc = 0.0f;
    if (cm) {
        const float * c = cm + ((r % LK_N_HEADS) / LK_G) * LK_HEAD_DIM + 8 * j;
        float t[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = v[2 * i] * c[2 * i], b = v[2 * i + 1] * c[2 * i + 1];
            t[i] = a + b;
        }
#pragma unroll
        for (int o = 4; o > 0; o >>= 1)
#pragma unroll
            for (int i = 0; i < 4; ++i) t[i] += __shfl_xor(t[i], o, 64);
        qc = (t[0] + t[2]) + (t[1] + t[3]);
    }
    if (j == 0) qcs[r] = qc * LK_LOG2E_F;
}

// K: positions [p0, p1) of kc [pos][8][64] -> k8 (same layout), ksc[h][pos].
__global__ void __launch_bounds__(256)
lk_k_pf_k8(const _Float16 * __restrict__ kc, int p0, int p1, const float * __restrict__ cm,
           int kstride, int8_t * __restrict__ k8, float * __restrict__ ksc) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 32 + (threadIdx.x >> 3), j = threadIdx.x & 7;
    const int pos = p0 + r / LK_N_KV_HEADS, h = r % LK_N_KV_HEADS;
    if (pos >= p1) return;                                // whole 8-lane groups
    const size_t row = (size_t) pos * LK_N_KV_HEADS + h;
    float v[8];
    lk_load8h(kc + row * LK_HEAD_DIM + 8 * j, v);
    if (cm) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] -= cm[h * LK_HEAD_DIM + 8 * j + i];
    }
    lk_q8_row8(v, k8 + row * LK_HEAD_DIM + 8 * j, ksc + (size_t) h * kstride + pos, 1.0f, j == 0);
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
#define PF_BQ      64                     // query rows per workgroup (4 blocks of 16)
#define PF_BK      64                     // keys per tile = the reference's 64-key tile
#define PF_QB      (PF_BQ / 16)
#define PF_Q_LD    144                    // LDS row pitch (bytes) of the fp16 Q block

// Tile modes: which query blocks score in int8.  Exactness is decided per
// (32-query tile, 64-key tile) and can only be lost as the query index grows,
// so a 64-query block is all-int8, mixed (queries 0-31 exact, 32-63 int8) or
// all-exact.
enum { PF_INT8 = 0, PF_MIXED = 1, PF_EXACT = 2 };

// One LDS stage of a 64-key tile.  The tiles are filled by LDS DMA (64 lanes
// x 16 contiguous bytes per instruction, no padding possible), so bank
// conflicts are avoided by XOR-swizzling the 16-byte chunk index with row
// bits chosen for each array's read pattern:
//   k8 (64 B rows, 16 rows x one chunk per read)     chunk c at c ^ ((r>>2)&3)
//   kh (128 B rows, 16 rows x one chunk per read)    chunk c at c ^ ((r>>1)&7)
//   v  (128 B rows, transposed reads: 4 rows x 32 B) chunk c at c ^ (((r>>1)&3)<<1)
struct alignas(16) PfStage {
    int8_t k8[PF_BK * 64];                // int8 K [key][64]
    float  ks[PF_BK];                     // int8 K scales
    int8_t kh[PF_BK * 128];               // fp16 K [key][64] (exact tiles)
    int8_t v[PF_BK * 128];                // fp16 V [key][64]
};
__device__ __forceinline__ int pf_sw_k8(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int pf_sw_kh(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int pf_sw_v(int r)  { return ((r >> 1) & 3) << 1; }

// Exact-tile predicate of the reference (prefill.cu:1380-1382), stated on its
// 64-key tiles: tile kt64 is exact for the 32-query tile qt32 iff
// kt64*64 + 64 > P + qt32*32 - near, or sink and kt64 == 0.
__host__ __device__ __forceinline__ bool lk_pf_exact(int P, int qt32, int kt64, int near, int sink) {
    return (kt64 * 64 + 64 > P + qt32 * 32 - near) || (sink && kt64 == 0);
}

// The int32 S^T block of 16 keys x 16 queries over the full head_dim (A = 16
// key rows, lane l: key l%16, bytes 16g..16g+15; B = Q^T, lane l: query l%16,
// the same bytes), with the accumulator seeded by the bit pattern of
// PF_MAGIC = 1.5 * 2^23: |sum| <= 64 * 128 * 128 < 2^22, so the integer result
// is the fp32 bit pattern of PF_MAGIC + sum, exactly (the float conversion done
// by the integer add inside the MFMA).  sum * ks is then one fma,
// fma(PF_MAGIC + sum, ks', -PF_MAGIC * ks'), exact in its product when ks' has
// at most 22 significant bits: ks' = ks with the two low mantissa bits cleared
// (a relative change below 2^-22, far inside the fp32 rounding of the score).
constexpr float PF_MAGIC = 12582912.0f;                  // 0x4B400000
__device__ __forceinline__ lk_f4 lk_mfma_qk8_magic(lk_i4 kfrag, lk_i4 qfrag) {
    const int mb = 0x4B400000;
    const lk_i4 z = { mb, mb, mb, mb };
    return __builtin_bit_cast(lk_f4, __builtin_amdgcn_mfma_i32_16x16x64_i8(kfrag, qfrag, z, 0, 0, 0));
}
__device__ __forceinline__ float lk_pf_ks22(float ks) {
    return __builtin_bit_cast(float, __builtin_bit_cast(unsigned, ks) & ~3u);
}

// ---- split-K work items (load balance of causal chunks) -----------------------
// Query block qt of a chunk sees key tiles [0, nkt(qt)); with P = 0 that grows
// from 1 to m/64 tiles.  Work items are key ranges [kt_lo, kt_hi) of a block;
// a block cut into several ("parts") has every part write an unnormalised
// partial (m, l, acc), which lk_k_pf_combine merges in part order.  A part
// never starts after the block's first diagonal tile, so every query sees at
// least one key in every part.  The grid enumerates items with the kv head
// fastest, and the dispatcher sends kv head x of every item to XCD x: each
// XCD runs the same item sequence, greedily, on its slots.
__host__ __device__ inline int pf_nkt(int qt, int m, int P) {
    const int qlast = (qt * PF_BQ + PF_BQ < m) ? qt * PF_BQ + PF_BQ : m;
    return (P + qlast + PF_BK - 1) / PF_BK;
}
// Equal-size parts of at most lsplit tiles (the test hook's plan; host only).
static inline void pf_parts(int qt, int m, int P, int lsplit, int & np, int & per) {
    const int nkt = pf_nkt(qt, m, P);
    np = (lsplit > 0) ? (nkt + lsplit - 1) / lsplit : 1;
    if (np < 1) np = 1;
    per = (nkt + np - 1) / np;
    const int kdiag = (P + qt * PF_BQ) / PF_BK;        // tile holding the block's first query
    while (np > 1 && (np - 1) * per > kdiag) { --np; per = (nkt + np - 1) / np; }
}
// The launch's work list, built on the host and passed by value (two 32-bit
// words per item, read with uniform scalar loads): items in dispatch order;
// slot0[q] is the first partial slot of split block q, nparts[q] its part
// count; split_qt lists the split blocks.
#define PF_MAX_ITEMS 384
#define PF_MAX_QB    128
struct PfWork {
    int n_items, n_split;                              // n_items 0: unsplit launch
    int spin;                                          // PAIR: poll bound of a group barrier
    uint32_t item[PF_MAX_ITEMS];                       // qt | (partial slot + 1) << 16 (0: not split)
    uint32_t krange[PF_MAX_ITEMS];                     // kt_lo | kt_hi << 16
    int16_t slot0[PF_MAX_QB];
    uint8_t split_qt[PF_MAX_QB];
    uint8_t nparts[PF_MAX_QB];
};
// Partials of a part, per (slot, kv head): acc as [head][16 dim chunks][64
// rows] of float4 (coalesced for the writing lanes and the merging lanes),
// then (m, l) as [head][64 rows] of float2; m is in the log2 domain of p.
#define PF_PART_ACC   (LK_G * 16 * PF_BQ * 4)           // floats
#define PF_PART_SLOT  (PF_PART_ACC + LK_G * PF_BQ * 2)  // floats per (part, kv head)
// Static scratch for the partials, 64 MiB per device: the fallback of launches
// that bring no workspace of their own.
#define PF_PART_CAP   (16u << 20)                        // floats
__device__ float g_pf_part[PF_PART_CAP];
// Measurement builds only (-DPF_TIMING; no launch of the product reads them):
// per-wave timestamps of the paired kernel (s_memrealtime, 100 MHz) written
// into the static partial scratch, which paired launches do not use:
// [workgroup][wave][4] = start, prologue done, tile loop done, end.
#ifdef PF_TIMING
#define PF_TSTAMP(k) do { if (PAIR && lane == 0) { \
        ((unsigned long long *) g_pf_part)[((size_t) blockIdx.x * 8 + w) * 4 + (k) + lane] = \
            __builtin_amdgcn_s_memrealtime(); } } while (0)
#else
#define PF_TSTAMP(k) do { } while (0)
#endif
// Group barriers of the paired kernel that gave up waiting (poll bound spent),
// counted per device; the workgroup's outputs are then NaN.
__device__ unsigned g_pf_gsync_fault;

// ---- planar Q8_1 of the attention output (the next GEMM's input) -------------
// Reference k_pf_quant_rows / pf_quant_warp (prefill.cu:1574-1580, 90-103): per
// 32-value block am = max|x| (exact), sum = xor-butterfly over the block's
// dims with strides 16, 8, 4, 2, 1, d = am/127 (IEEE), q = roundf(x/d) (0 when
// am = 0), scale plane (float(fp16(d)), 8 * float(fp16(sum))).  Layout:
// qs int8 [rows][2048] (block b of a row at 32b), sc float2 [rows][64].
__device__ __forceinline__ float2 lk_q81_scales(float d, float sum) {
    return make_float2((float) (_Float16) d, 8.0f * (float) (_Float16) sum);
}
__device__ __forceinline__ int8_t lk_q81_q(float x, float am, float d) {
    return (am == 0.0f) ? (int8_t) 0 : (int8_t) roundf(x / d);
}
// The same q for the many values of one block with one division per block:
// with r = RN(1/d'), q0 = RN(x*r) is within an ulp of x/d' and
// RN(q0 + RN(x - q0*d')*r) (two fmas, the remainder exact) is RN(x/d')
// (Markstein's correction theorem), so roundf sees the bits of x / d.  The
// theorem needs x/d' and 1/d' in the normal range: blocks with am < 2^-64
// scale x and d by 2^64 (exact, the quotient unchanged); quotients that are
// subnormal may differ, but roundf gives 0 for both.  am = 0 (all x = 0)
// divides by 1.  tests/test_q81_division.py runs this arithmetic on the host
// against x / d over am in [2^-140, 2^100], ties and quotients next to .5
// included.
struct LkQ81Div { float s, d, r; };
__device__ __forceinline__ LkQ81Div lk_q81_div(float am, float d) {
    LkQ81Div q;
    q.s = am < 0x1p-64f ? 0x1p64f : 1.0f;
    q.d = am == 0.0f ? 1.0f : d * q.s;
    q.r = 1.0f / q.d;
    return q;
}
__device__ __forceinline__ int8_t lk_q81_qd(const LkQ81Div & q, float x) {
#pragma clang fp contract(off)
    const float xs = x * q.s;
    const float q0 = xs * q.r;
    const float e = __builtin_fmaf(-q0, q.d, xs);
    return (int8_t) roundf(__builtin_fmaf(e, q.r, q0));
}
// From the attention epilogue's layout: lane (col, g) holds, for its query row,
// dims 16db + 4g + r of the head (db, r = 0..3): block hb (dims 32hb ..
// 32hb+31) is db = 2hb, 2hb+1 on the 4 lanes g of the row.  The sum follows
// the reference's tree exactly: stride 16 = db pair (in lane), 8 and 4 = lanes
// xor 32 and 16, 2 and 1 = r pairs (in lane).
__device__ __forceinline__ void lk_pf_q81_epilogue(const lk_f4 (&a)[4], bool store, int8_t * __restrict__ qs,
                                                   float2 * __restrict__ sc, int g) {
#pragma clang fp contract(off)
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
        const lk_f4 x0 = a[2 * hb], x1 = a[2 * hb + 1];
        float am = 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) am = fmaxf(am, fmaxf(fabsf(x0[r]), fabsf(x1[r])));
        am = fmaxf(am, __shfl_xor(am, 32, 64));
        am = fmaxf(am, __shfl_xor(am, 16, 64));
        float t[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] = x0[r] + x1[r];
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] += __shfl_xor(t[r], 32, 64);
#pragma unroll
        for (int r = 0; r < 4; ++r) t[r] += __shfl_xor(t[r], 16, 64);
        const float sum = (t[0] + t[2]) + (t[1] + t[3]);
        const float d = am / 127.0f;
        const LkQ81Div qd = lk_q81_div(am, d);
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            w0 |= (uint32_t) (uint8_t) lk_q81_qd(qd, x0[r]) << (8 * r);
            w1 |= (uint32_t) (uint8_t) lk_q81_qd(qd, x1[r]) << (8 * r);
        }
        if (store) {
            *(uint32_t *) (qs + 32 * hb + 4 * g)      = w0;
            *(uint32_t *) (qs + 32 * hb + 16 + 4 * g) = w1;
            if (g == 0) sc[hb] = lk_q81_scales(d, sum);
        }
    }
}

// PAIR: workgroups of 8 waves, each over query blocks bi = pair index and
// bj = nq-1-bi of one kv head.  Waves 0-3 (group A) take bi and then bj's
// key tiles [0, xs); waves 4-7 (group B) take bj's tiles [xs, nkj); xs is
// chosen so that both groups score about the same number of tiles, and at the
// end A's part of bj is merged into B's through LDS.  Every workgroup then
// does the same work (about half of bi + bj), with no split-K partials in
// memory and no merge kernel.  The groups stream their own tiles and meet at
// barriers of their own (a counter in LDS), not at the workgroup barrier, so
// the two waves of a SIMD (one per group) drift into different phases of
// their tiles, as two unpaired workgroups do.
template <bool INT8, bool PAIR, bool Q81>
__global__ void __launch_bounds__(PAIR ? 512 : 256, PAIR ? 1 : 2)
lk_k_pf_attn(const int8_t * __restrict__ q8, const float * __restrict__ qsc,
             const float * __restrict__ qcs, const _Float16 * __restrict__ qh, int m, int P,
             const int8_t * __restrict__ k8, const float * __restrict__ ksc, int kstride,
             const _Float16 * __restrict__ kc, const _Float16 * __restrict__ vc,
             int near, int sink, float * __restrict__ o, int8_t * __restrict__ aqs,
             float2 * __restrict__ asc, const PfWork work, float * __restrict__ pbuf) {
    constexpr int NW = PAIR ? 8 : 4;                     // waves
    __shared__ PfStage st[PAIR ? 4 : 2];                  // PAIR: [stage][slot]
    __shared__ __attribute__((aligned(16))) int8_t s_q[NW][PF_BQ * PF_Q_LD];  // fp16 Q, per wave
    __shared__ __attribute__((aligned(16))) float s_kp[NW][2 * PF_BK];         // per wave: ks', -PF_MAGIC*ks'
    // PAIR: each lane's DMA source offsets (int8 K, fp16 K and V rows of key
    // group 0; all below 2^16), formed once and re-read per issue (see
    // issue_to).  They depend on the wave's head, not on its group.
    __shared__ uint16_t s_off[PAIR ? 4 : 1][3][64];
    // Causal work grows with the query block.  Unsplit launches: workgroups
    // are dispatched in linear order and the second half of the grid lands
    // beside the first half on the CUs, so kv heads 0-3 take the query blocks
    // longest-first and kv heads 4-7 shortest-first: co-resident workgroups
    // then pair a long block with a short one.  Split launches: one work item
    // (block, key range) per workgroup, longest first.
    const int tid  = threadIdx.x;
    const int lane = tid & 63;
    const int w    = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col  = lane & 15, g = lane >> 4;
    PF_TSTAMP(0);
    const int hw   = w & 3, grp = w >> 2;                 // head within the kv head; PAIR group
    int kvh, qt, kt_lo, kt_hi, pslot = -1;
    int bi = 0, bj = 0, nki = 0, nkj = 0, xs = 0;         // PAIR: the two blocks, their tile counts, the cut of bj
    if constexpr (PAIR) {
        kvh = blockIdx.x % LK_N_KV_HEADS;
        const int nq = (m + PF_BQ - 1) / PF_BQ;
        bi = (int) (blockIdx.x / LK_N_KV_HEADS);
        bj = nq - 1 - bi;
        nki = (bi == bj) ? 0 : pf_nkt(bi, m, P);
        nkj = pf_nkt(bj, m, P);
        // nki + xs = nkj - xs balances the groups; B's first tile must not lie
        // past bj's first query, so that every row of bj sees a key in B's part
        // (A's part starts at key 0)
        // (with an odd tile count the fp16 kernel gives the odd tile to A, which
        // measured faster -- B merges A's part at the end; the int8 kernel
        // measured faster with it in B)
        xs = (nkj - nki + (INT8 ? 0 : 1)) / 2;
        const int kdj = (P + bj * PF_BQ) / PF_BK;
        if (xs > kdj) xs = kdj;
        if (xs < 0) xs = 0;
        qt = (grp == 0 && nki > 0) ? bi : bj;             // group A starts on bi when it has one
        kt_lo = 0; kt_hi = 0;
    } else if (work.n_items == 0) {
        kvh = blockIdx.y;
        qt  = (kvh < LK_N_KV_HEADS / 2) ? (int) (gridDim.x - 1 - blockIdx.x) : (int) blockIdx.x;
        kt_lo = 0; kt_hi = pf_nkt(qt, m, P);
    } else {
        kvh = blockIdx.x % LK_N_KV_HEADS;
        const int i = blockIdx.x / LK_N_KV_HEADS;
        const uint32_t it = work.item[i], kr = work.krange[i];
        qt = (int) (it & 255);
        pslot = (int) (it >> 16) - 1;
        kt_lo = (int) (kr & 0xffff);
        kt_hi = (int) (kr >> 16);
    }
    const int head = kvh * LK_G + hw;
    int qbase = qt * PF_BQ;                           // the wave's block (PAIR group A moves to bj)
    // keys [0, kend) are visible to some row of the workgroup's blocks (PAIR: of bj)
    const int kend = P + (PAIR ? (bj * PF_BQ + PF_BQ < m ? bj * PF_BQ + PF_BQ : m)
                               : (qbase + PF_BQ < m ? qbase + PF_BQ : m));

    // tile mode for the 64-query block starting at query qb0
    auto mode_at = [&](int kt, int qb0) -> int {
        if (!INT8) return PF_EXACT;
        if (lk_pf_exact(P, qb0 / 32 + 1, kt, near, sink)) return PF_EXACT;
        return lk_pf_exact(P, qb0 / 32, kt, near, sink) ? PF_MIXED : PF_INT8;
    };
    auto mode_of = [&](int kt) -> int { return mode_at(kt, qbase); };
    // a tile needs the causal mask iff its last key lies past the first query
    auto mask_of = [&](int kt) -> bool { return kt * PF_BK + PF_BK - 1 > P + qbase; };

    // ---- LDS DMA of tile kt: wave hw (of the issuing four) fetches keys 16hw .. 16hw+15
    const uint32_t lds_st = lk_lds_addr(&st[0]);
    const float * ks_h = INT8 ? ksc + (size_t) kvh * kstride : nullptr;
    const int ks_clamp = ((kend - 1) / 4) * 4;        // last 16-byte chunk holding a visible key
    // Per-lane byte offsets of the DMA sources relative to the tile's first key
    // (the kv head folded in); the tile base itself is wave-uniform.
    // PAIR: these offsets are re-read from LDS at each issue (issue_to), and
    // what is still formed from the lane id (the key-scale offset, the clamped
    // rows of a block's last tile, the Q addresses of load_q below) from an
    // opaque copy of it; the compiler would otherwise form them once and keep
    // them live across the tile loop, at a register budget that leaves no room
    // for them (spills, and every reload waits for the tile DMA in flight).
    auto dma_lane = [&]() -> int {
        if constexpr (PAIR) {
            int l;
            asm volatile("v_mov_b32 %0, %1" : "=v"(l) : "v"(lane));
            return l;
        } else {
            return lane;
        }
    };
    auto so_k8_of = [&](int ln) -> uint32_t {
        const int r = 16 * hw + (ln >> 2);
        return (uint32_t) ((r * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM + 16 * ((ln & 3) ^ pf_sw_k8(r)));
    };
    auto so_ks_of = [&](int ln) -> uint32_t { return (uint32_t) (4 * (16 * hw + 4 * ln)); };
    auto so_kv_of = [&](int ln, int j, bool isv) -> uint32_t {
        const int r = 16 * hw + 8 * j + (ln >> 3);
        const uint32_t row = (uint32_t) ((r * LK_N_KV_HEADS + kvh) * LK_HEAD_DIM * 2);
        return row + 16 * ((ln & 7) ^ (isv ? pf_sw_v(r) : pf_sw_kh(r)));
    };
    // into stage buffer si; md = the union of the readers' tile modes
    auto issue_to = [&](int kt, int si, int md) {
        const uint32_t sb = lds_st + (uint32_t) (si * sizeof(PfStage));
        const int kb0 = kt * PF_BK;
        const int ln = dma_lane();
        uint32_t so_k8, so_kh[2], so_v[2];
        const uint32_t so_ks = so_ks_of(ln);
        if constexpr (PAIR) {
            // three LDS reads instead of forming five offsets (about 40 VALU
            // instructions per issue; measured at C4 93.0 -> 89.5 us int8,
            // 88.3 -> 86.7 us fp16); asm so that the compiler neither keeps
            // them live across the tile loop nor counts them
            uint32_t o0, o1, o2;
            const uint32_t oa = lk_lds_addr(&s_off[hw][0][0]) + 2u * (uint32_t) ln;
            asm volatile("ds_read_u16 %0, %3\n\tds_read_u16 %1, %3 offset:128\n\tds_read_u16 %2, %3 offset:256\n\t"
                         "s_waitcnt lgkmcnt(0)" : "=&v"(o0), "=&v"(o1), "=&v"(o2) : "v"(oa) : "memory");
            so_k8 = o0;
            so_kh[0] = o1; so_kh[1] = (o1 + 8192u) ^ 64u;     // key group 1: 8 rows on, swizzle bit 2 flipped
            so_v[0] = o2;  so_v[1] = o2 + 8192u;              // (the V swizzle repeats every 8 rows)
        } else {
            so_k8 = so_k8_of(ln);
            so_kh[0] = so_kv_of(ln, 0, false); so_kh[1] = so_kv_of(ln, 1, false);
            so_v[0] = so_kv_of(ln, 0, true); so_v[1] = so_kv_of(ln, 1, true);
        }
        if (kb0 + PF_BK <= kend) {                        // whole tile visible: no clamping
            const int8_t * kb8 = k8 + (size_t) kb0 * LK_KV_ROW;
            const _Float16 * kbh = kc + (size_t) kb0 * LK_KV_ROW;
            const _Float16 * kbv = vc + (size_t) kb0 * LK_KV_ROW;
            if (md != PF_EXACT) {
                lk_dma16c_so(kb8, so_k8, sb + (uint32_t) (offsetof(PfStage, k8) + 1024 * hw));
                if (lane < 4) lk_dma16c_so(ks_h + kb0, so_ks, sb + (uint32_t) (offsetof(PfStage, ks) + 64 * hw));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if (md != PF_INT8)
                    lk_dma16c_so(kbh, so_kh[j], sb + (uint32_t) (offsetof(PfStage, kh) + 1024 * (2 * hw + j)));
                lk_dma16c_so(kbv, so_v[j], sb + (uint32_t) (offsetof(PfStage, v) + 1024 * (2 * hw + j)));
            }
            return;
        }
        // the block's last tile: keys past kend are clamped to kend-1 (valid
        // memory, finite values); they are masked, so their p is exactly 0.
        // Same tile bases as above, clamped rows in the per-lane offsets.
        const int lim = kend - 1 - kb0;                   // >= 0: the tile holds a visible key
        const int8_t * kb8 = k8 + (size_t) kb0 * LK_KV_ROW;
        const _Float16 * kbh = kc + (size_t) kb0 * LK_KV_ROW;
        const _Float16 * kbv = vc + (size_t) kb0 * LK_KV_ROW;
        if (md != PF_EXACT) {
            const int r_k8 = 16 * hw + (ln >> 2);
            const int rr = (r_k8 < lim) ? r_k8 : lim;
            lk_dma16c_so(kb8, so_k8 + (uint32_t) ((rr - r_k8) * LK_KV_ROW),
                         sb + (uint32_t) (offsetof(PfStage, k8) + 1024 * hw));
            if (lane < 4) {
                const int s0 = 16 * hw + 4 * ln, sl = ks_clamp - kb0;
                lk_dma16c_so(ks_h + kb0, (uint32_t) (4 * (s0 < sl ? s0 : sl)),
                             sb + (uint32_t) (offsetof(PfStage, ks) + 64 * hw));
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int r = 16 * hw + 8 * j + (ln >> 3);
            const uint32_t dr = (uint32_t) ((((r < lim) ? r : lim) - r) * LK_KV_ROW * 2);
            if (md != PF_INT8)
                lk_dma16c_so(kbh, so_kh[j] + dr, sb + (uint32_t) (offsetof(PfStage, kh) + 1024 * (2 * hw + j)));
            lk_dma16c_so(kbv, so_v[j] + dr, sb + (uint32_t) (offsetof(PfStage, v) + 1024 * (2 * hw + j)));
        }
    };

    auto issue = [&](int kt) { issue_to(kt, kt & 1, mode_of(kt)); };
    // PAIR: step it of the wave's group: A bi's tiles then bj's [0, xs), B
    // bj's [xs, nkj); each group double-buffers in its own two stages
    const int g_ns = (grp == 0) ? nki + xs : nkj - xs;   // steps of the wave's group
    auto g_tile = [&](int it) -> int { return (grp == 0) ? (it < nki ? it : it - nki) : xs + it; };
    auto g_base = [&](int it) -> int { return (grp == 0 && it < nki) ? bi * PF_BQ : bj * PF_BQ; };
    auto issue_step = [&](int it) {
        const int kt = g_tile(it);
        issue_to(kt, 2 * grp + (it & 1), mode_at(kt, g_base(it)));
    };
    // PAIR: the group barrier, a counter per group in LDS that only grows
    // (4 arrivals per step); the poll is bounded (work.spin polls) so that a
    // wave can never hang the kernel.  A wave that gives up marks its group
    // (s_gbad) and counts the event in g_pf_gsync_fault: the group may then
    // have read a tile stage before all of its rows were in, so every output
    // the group writes afterwards is NaN, and the host can read the count
    // (lk_pf_gsync_faults).  The kernel still runs to its end.
    __shared__ unsigned s_gbar[2];
    __shared__ unsigned s_gbad[2];
    unsigned g_gen = 0;
    auto gsync = [&]() {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) __hip_atomic_fetch_add(&s_gbar[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        g_gen += 4;
        bool met = false;
        for (int n = 0; n < work.spin; ++n) {
            const unsigned c = __builtin_amdgcn_readfirstlane(
                __hip_atomic_load(&s_gbar[grp], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            if ((int) (c - g_gen) >= 0) { met = true; break; }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!met) {                                   // wave-uniform
            if (lane == 0) {
                __hip_atomic_store(&s_gbad[grp], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                __hip_atomic_fetch_add(&g_pf_gsync_fault, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    };
    if constexpr (PAIR) {
        if (grp == 0) {                               // group B's wave of the same head reads them too
            s_off[hw][0][lane] = (uint16_t) so_k8_of(lane);
            s_off[hw][1][lane] = (uint16_t) so_kv_of(lane, 0, false);
            s_off[hw][2][lane] = (uint16_t) so_kv_of(lane, 0, true);
        }
        __syncthreads();                              // before any wave's first issue
        if (tid < 2) { s_gbar[tid] = 0u; s_gbad[tid] = 0u; }
        // (the workgroup barrier after the Q prologue below orders this
        // before every group barrier)
    }

    // The first tile's DMA goes out before the Q loads below, so that the two
    // memory latencies overlap.
    if constexpr (PAIR) { if (g_ns > 0) issue_step(0); }
    else issue(kt_lo);

    // ---- this wave's fp16 Q block (64 rows x 128 B), for exact tiles, and the
    // int8 Q operands and scales below.  Every load reads a row clamped to m-1
    // and rows past m are zeroed by a select afterwards (a guarded load costs a
    // branch and a full memory wait each), and all of them are issued before
    // the first use: one memory round trip for the whole prologue.
    lk_i4 qf8[PF_QB];
    float sq[PF_QB], exa[PF_QB], exb[PF_QB];   // exa, exb: see below
    // q8 == nullptr: the int8 Q rows are quantised here from the fp16 block in
    // LDS (lk_k_pf_q8's arithmetic, without smoothing: q.c = 0) instead of
    // being loaded; src is the wave's s_q block that holds them.
    const bool fuse_q = INT8 && q8 == nullptr;
    auto fill_sq = [&](const lk_h8 (&qv16)[8]) {
        const lk_h8 z8 = { 0, 0, 0, 0, 0, 0, 0, 0 };
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = (lane >> 3) + 8 * i;
            *(lk_h8 *) (s_q[w] + r * PF_Q_LD + 16 * (lane & 7)) = (qbase + r < m) ? qv16[i] : z8;
        }
    };
    auto load_q = [&](bool fill_s_q, int src) {
        lk_h8 qv16[8];
        if (fill_s_q) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int qr = qbase + (lane >> 3) + 8 * i;
                qv16[i] = *(const lk_h8 *) (qh + (size_t) (qr < m ? qr : m - 1) * LK_HIDDEN + head * LK_HEAD_DIM + 8 * (lane & 7));
            }
            if (fuse_q) {                                 // wave-uniform
                fill_sq(qv16);
                __builtin_amdgcn_wave_barrier();          // a wave's LDS accesses complete in order
            }
        }
        // ---- int8 Q operands and per-query scalars (lane column = query) ------
        // (PAIR: the lane id through dma_lane, so that the addresses of the
        // second call are not formed early and kept live across the tiles)
        const int lq = dma_lane();
        const int qcol = lq & 15, qg = lq >> 4;
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) {
            const int qr = qbase + 16 * qb + qcol;
            const bool ok = qr < m;
            const int qrc = ok ? qr : m - 1;              // clamped: unconditional loads
            const lk_i4 zi = { 0, 0, 0, 0 };
            if (INT8) {
                lk_i4 qv;
                float dv, cv;
                if (fuse_q) {
#pragma clang fp contract(off)
                    // values 16qg .. 16qg+15 of row 16qb + qcol (rows past m are zero
                    // in s_q: am = 0 gives zero quants and d = 0)
                    const int8_t * rp = s_q[src] + (16 * qb + qcol) * PF_Q_LD + 32 * qg;
                    const lk_h8 h0 = *(const lk_h8 *) rp, h1 = *(const lk_h8 *) (rp + 16);
                    float v[16];
#pragma unroll
                    for (int i = 0; i < 8; ++i) { v[i] = (float) h0[i]; v[8 + i] = (float) h1[i]; }
                    float am = fabsf(v[0]);
#pragma unroll
                    for (int i = 1; i < 16; ++i) am = fmaxf(am, fabsf(v[i]));
                    am = lk_xrow_max(am);                 // the row's 64 values: lanes ^16, ^32
                    const float d = am / 127.0f;
                    const float id = (am > 0.0f) ? 127.0f / am : 0.0f;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        uint32_t wq = 0;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            wq |= (uint32_t) (uint8_t) (int8_t) (int) __builtin_rintf(v[4 * k + i] * id) << (8 * i);
                        qv[k] = (int) wq;
                    }
                    dv = d * LK_LOG2E_F;
                    cv = 0.0f;
                } else {
                    qv = *(const lk_i4 *) (q8 + (size_t) qrc * LK_HIDDEN + head * LK_HEAD_DIM + 16 * qg);
                    dv = qsc[(size_t) qrc * LK_N_HEADS + head];
                    cv = qcs ? qcs[(size_t) qrc * LK_N_HEADS + head] : 0.0f;
                }
                qf8[qb] = ok ? qv : zi;
                const float d = ok ? dv : 0.0f;
                // scores are kept in units of 1/sq until the exponent (sq > 0
                // scales commute with the max); an all-zero query row has sq = 0
                // and zero int8 scores, so unit scaling is exact for it
                sq[qb] = (d > 0.0f) ? d : 1.0f;
                // exact tiles' score in units of 1/sq: (sum*log2e - qc) / sq as one fma
                const float isq = 1.0f / sq[qb];
                const float qc = ok ? cv : 0.0f;
                // PAIR forms the exponent argument in the score step: an exact
                // tile's is sum*log2e - qc - moff, one fma
                exa[qb] = PAIR ? LK_LOG2E_F : LK_LOG2E_F * isq;
                exb[qb] = PAIR ? -qc : -qc * isq;
            } else {
                // every tile exact: scores stay the raw fp32 sums (natural-log
                // units) and log2(e) is the exponent's scale, so the exponent
                // argument is one fma of the raw sum
                qf8[qb] = zi; sq[qb] = LK_LOG2E_F; exa[qb] = PAIR ? LK_LOG2E_F : 1.0f; exb[qb] = 0.0f;
            }
        }
        if (fill_s_q && !fuse_q) fill_sq(qv16);
    };
    load_q(true, w);
    // PAIR: every wave's s_q block (group A reads group B's for bj) and the
    // group counters are in place before any group goes on
    if constexpr (PAIR) __syncthreads();
    PF_TSTAMP(1);
    int qw = w;                                       // the s_q block exact tiles read

    // O^T blocks [dim block][query block]; block 4 multiplies P^T by an
    // all-ones A operand, so every lane of query column q accumulates
    // l_q = sum of the same fp16 P the numerator uses.
    lk_f4 acc[5][PF_QB];
#pragma unroll
    for (int db = 0; db < 5; ++db)
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) acc[db][qb] = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
    // Per query, p = 2^(x*sq - moff) with the exponent offset moff = m*sq +
    // PF_P_BIAS for a running max m (score units), -inf before the first
    // tile.  mst holds m (unpaired launches) or moff itself (PAIR, whose
    // first tile sets moff from the tile max before any p is formed).
    float mst[PF_QB];
#pragma unroll
    for (int qb = 0; qb < PF_QB; ++qb) mst[qb] = -INFINITY;
    const _Float16 one = (_Float16) 1.0f;
    const lk_h8 ones = { one, one, one, one, one, one, one, one };
    // p is formed as 2^(sq*(x - m) - PF_P_BIAS): the max m the offset was set
    // from has p = 2^-5, and p is a normal fp16 down to 2^-9 of that p; below
    // it keeps an absolute step of 2^-24 (2^-19 of it).  The offset is only
    // raised once some p reaches 2^PF_P_BIG = 2^15 (fp16 ends at 2^16), i.e.
    // a score 20 log2 units past the running max: a p above 2^-5 only gains
    // relative precision, and the P.V and row-sum MFMAs accumulate in fp32.
    // (Raising it at p >= 2, a headroom of 6, rescaled 8-46% of the query
    // halves of shallow chunks and cost C4 about 8%.)  The test is two-level:
    // bit 14 of the OR of all p words (some p >= 2, inf or NaN: the first fp16
    // value with bit 14 set is 2), then, only then, the max of the words.
    // A larger bias costs accuracy on long diffuse rows: at 2^-7, rows over
    // 8000 keys measured 8e-4 relative error against float64, at 2^-5 about
    // 1e-4 to 2.6e-4 (as the unbiased form).  The bias cancels in
    // o = acc / l; partial records carry it in their max.
#ifndef PF_PBIAS
#define PF_PBIAS 5
#endif
    constexpr float PF_P_BIAS = (float) PF_PBIAS;
    constexpr float PF_P_BIG = 15.0f;
    auto moff = [&](int qb) -> float { return PAIR ? mst[qb] : fmaf(mst[qb], sq[qb], PF_P_BIAS); };

    // ---- per-lane LDS read offsets: the swizzles above depend only on the lane
    // here, so every read below is one of these bases plus a constant.
    const int o_k8 = col * 64 + 16 * (g ^ (col >> 2));               // + 1024*kb
    const int o_kh0 = col * 128 + 16 * (g ^ (col >> 1));             // + 2048*kb
    const int o_kh1 = col * 128 + 16 * ((4 + g) ^ (col >> 1));       // + 2048*kb
    const int vsw = (2 * g + ((col >> 2) >> 1)) & 3;                 // pf_sw_v(row) / 2
    const int o_v = (4 * g + (col >> 2)) * 128 + 8 * (col & 1);      // + 4096*kk (+2048 hi)
    int o_vd[4];                                                    // chunk of dims 16db + 4(col&3)
#pragma unroll
    for (int db = 0; db < 4; ++db) o_vd[db] = o_v + 32 * (db ^ vsw) + 16 * ((col & 3) >> 1);
    const int o_q = col * PF_Q_LD + 16 * g;                          // + 16*PF_Q_LD*qb

    // ---- one 64-key tile.  Mode and mask are wave-uniform run-time branches:
    // bodies specialised per mode (one loop each, or one loop with a branch to
    // each) measured 40% slower, the register allocator then spilled.
    auto tile = [&](const PfStage & S, int kt) {
        const int md = mode_of(kt);
        const bool msk = mask_of(kt);
        const int kb0 = kt * PF_BK;
        lk_i4 ka[4];                        // int8 K fragments (key row 16kb+col)
        lk_f4 sk[4], skb[4];                // scales (keys 16kb+4g+i), 22-bit, and -PF_MAGIC times them
        if (md != PF_EXACT) {
            // the int8 K fragments first (LDS accesses of a wave complete in
            // order: the MFMAs then wait for one LDS round trip, not for the
            // scale staging behind it), then the scale pair of the tile's 64
            // keys, one key per lane, through this wave's own LDS rows
            const float ks_l = S.ks[lane];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) ka[kb] = *(const lk_i4 *) (S.k8 + o_k8 + 1024 * kb);
            const float s22 = lk_pf_ks22(ks_l);
            s_kp[w][lane] = s22;
            s_kp[w][PF_BK + lane] = s22 * -PF_MAGIC;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                sk[kb] = *(const lk_f4 *) (&s_kp[w][16 * kb + 4 * g]);
                skb[kb] = *(const lk_f4 *) (&s_kp[w][PF_BK + 16 * kb + 4 * g]);
            }
        }
        lk_h8 pb[PF_QB][2];
        // Two query blocks at a time (scores of 64 keys x 32 queries in flight);
        // in a mixed tile the first pair is exact, the second int8.
#pragma unroll
        for (int hq = 0; hq < 2; ++hq) {
            const bool ex = (md == PF_EXACT) || (md == PF_MIXED && hq == 0);
            // x: unpaired launches, the score in units of 1/sq; PAIR, the
            // exponent argument x*sq - moff itself (one fma per score on exact
            // tiles instead of two), taken against offset 0 on a part's first
            // tile (every query at -inf: wave-uniform), whose offset is then set
            // from the tile max
            float x[4][2][4];               // [key block][query block 2hq+j][i]: key kb0+16kb+4g+i
            const bool first = PAIR &&
                __builtin_amdgcn_readfirstlane(__float_as_int(mst[2 * hq])) == __float_as_int(-INFINITY);
            float mo2[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) mo2[j] = first ? 0.0f : mst[2 * hq + j];
            if (ex) {
                lk_h8 qa[2][2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int8_t * qrow = s_q[qw] + o_q + 16 * PF_Q_LD * (2 * hq + j);
                    qa[j][0] = *(const lk_h8 *) qrow;
                    qa[j][1] = *(const lk_h8 *) (qrow + 64);
                }
                // PAIR: all eight K fragments in flight before the first MFMA
                // (C4 1.5% faster; in the unpaired kernel, deep chunks 0.6%
                // slower, so there each key block's pair is read at its use)
                lk_h8 kf[4][2];
                if constexpr (PAIR) {
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb) {
                        kf[kb][0] = *(const lk_h8 *) (S.kh + o_kh0 + 2048 * kb);
                        kf[kb][1] = *(const lk_h8 *) (S.kh + o_kh1 + 2048 * kb);
                    }
                }
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const lk_h8 k0 = PAIR ? kf[kb][0] : *(const lk_h8 *) (S.kh + o_kh0 + 2048 * kb);
                    const lk_h8 k1 = PAIR ? kf[kb][1] : *(const lk_h8 *) (S.kh + o_kh1 + 2048 * kb);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int qb = 2 * hq + j;
                        lk_f4 c = { 0.f, 0.f, 0.f, 0.f };
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qa[j][0], c, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qa[j][1], c, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            x[kb][j][i] = PAIR ? fmaf(c[i], exa[qb], exb[qb] - mo2[j])
                                               : INT8 ? fmaf(c[i], exa[qb], exb[qb]) : c[i];
                    }
                }
            } else {
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_setprio(1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const lk_f4 c = lk_mfma_qk8_magic(ka[kb], qf8[2 * hq + j]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float xs = fmaf(c[i], sk[kb][i], skb[kb][i]);
                            x[kb][j][i] = PAIR ? fmaf(xs, sq[2 * hq + j], -mo2[j]) : xs;
                        }
                    }
            }
            if (msk) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    // key kb0+16kb+4g+i is masked iff 16kb+i > qpos - kb0 - 4g
                    const int dq = P + qbase + 16 * (2 * hq + j) + col - kb0 - 4 * g;
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (16 * kb + i > dq) x[kb][j][i] = -INFINITY;
                }
            }
            // ---- online softmax, per query (lane column); p = 2^(x*sq - moff)
            // p is formed against the running offset first.  The exact tile max
            // is only needed when some p reaches 2^PF_P_BIG (or the max is still
            // -inf: first tile), which is first screened by bit 14 of an fp16 p
            // (p >= 2, inf or NaN) in the OR of the p words, with no cross-lane
            // reduction.
            auto make_p = [&]() {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int qb = 2 * hq + j;
                    if constexpr (PAIR) {
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                pb[qb][kk][i]     = (_Float16) lk_exp2(x[2 * kk][j][i]);
                                pb[qb][kk][4 + i] = (_Float16) lk_exp2(x[2 * kk + 1][j][i]);
                            }
                    } else {
                        const float mo = moff(qb);
#pragma unroll
                        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                pb[qb][kk][i]     = (_Float16) lk_exp2(fmaf(x[2 * kk][j][i], sq[qb], -mo));
                                pb[qb][kk][4 + i] = (_Float16) lk_exp2(fmaf(x[2 * kk + 1][j][i], sq[qb], -mo));
                            }
                    }
                }
            };
            auto row_max = [&](int j) -> float {
                float v = x[0][j][0];
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) v = fmaxf(v, x[kb][j][i]);
                return lk_xrow_max(v);                         // the 4 lane groups of this query
            };
            if constexpr (PAIR) {
                // a part's first tile: the offset from the exact tile max before
                // any p is formed (every query sees a key in it, so the max is
                // finite), and the arguments taken against it
                if (first) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float mn = row_max(j) + PF_P_BIAS;
                        mst[2 * hq + j] = mn;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                            for (int i = 0; i < 4; ++i) x[kb][j][i] -= mn;
                    }
                }
            }
            // Wave priorities by phase: exponent pass 2, int8 Q.K^T and the
            // rest of the softmax 1, P.V 0.  The two waves of a SIMD (one per
            // co-resident workgroup) then tend to be in different phases, VALU
            // beside MFMA; at one priority for every phase they drift into the
            // same phase (C5 72.6 ms against 66.0 ms with these levels; two
            // adjacent phases at the same level lose the gain).
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(2);
            __builtin_amdgcn_sched_barrier(0);
            make_p();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            __builtin_amdgcn_sched_barrier(0);
            unsigned pw[16];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const lk_i4 uw = __builtin_bit_cast(lk_i4, pb[2 * hq + j][kk]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) pw[8 * j + 4 * kk + e] = (unsigned) uw[e];
                }
#pragma unroll
            for (int n = 16; n > 1; n = (n + 2) / 3)                // OR tree, three words per op
#pragma unroll
                for (int t = 0; t < (n + 2) / 3; ++t)
                    pw[t] = pw[3 * t] | (3 * t + 1 < n ? pw[3 * t + 1] : 0u) | (3 * t + 2 < n ? pw[3 * t + 2] : 0u);
            if (__ballot(pw[0] & 0x40004000u)) {               // some p >= 2 (or inf/NaN)
                // any p >= 2^PF_P_BIG (or inf/NaN)?  The fp16 bit patterns of
                // p >= 0 order as unsigned integers: a packed u16 max of the
                // p words against 0x7800.
                lk_u16x8 pm = __builtin_elementwise_max(__builtin_bit_cast(lk_u16x8, pb[2 * hq][0]),
                                                        __builtin_bit_cast(lk_u16x8, pb[2 * hq][1]));
                pm = __builtin_elementwise_max(pm, __builtin_bit_cast(lk_u16x8, pb[2 * hq + 1][0]));
                pm = __builtin_elementwise_max(pm, __builtin_bit_cast(lk_u16x8, pb[2 * hq + 1][1]));
                const lk_u16x4 p4 = __builtin_elementwise_max(pm.s0123, pm.s4567);
                const lk_u16x2 p2 = __builtin_elementwise_max(p4.s01, p4.s23);
                const unsigned short p1 = p2.x > p2.y ? p2.x : p2.y;
                if (__ballot(p1 >= 0x7800u)) {                 // wave-uniform, rare
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int qb = 2 * hq + j;
                        if constexpr (PAIR) {
                            // the offset of the queries past the limit moves up
                            // by dm, to their max + PF_P_BIAS (x is already
                            // relative to the offset); their p are formed again
                            const float am = row_max(j);
                            const bool need = am > PF_P_BIG - 1.0f;
                            if (__ballot(need)) {
                                const float dm = need ? am + PF_P_BIAS : 0.0f;
                                const float alpha = need ? lk_exp2(-dm) : 1.0f;
                                mst[qb] += dm;
#pragma unroll
                                for (int db = 0; db < 5; ++db) acc[db][qb] *= alpha;
#pragma unroll
                                for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                                    for (int i = 0; i < 4; ++i) {
                                        pb[qb][kk][i]     = (_Float16) lk_exp2(x[2 * kk][j][i] - dm);
                                        pb[qb][kk][4 + i] = (_Float16) lk_exp2(x[2 * kk + 1][j][i] - dm);
                                    }
                            }
                        } else {
                            // the running max itself; key 0 is visible to every
                            // query, so mst is finite after tile 0
                            const float mx = row_max(j);
                            const bool need = (mx - mst[qb]) * sq[qb] > PF_P_BIG + PF_P_BIAS - 1.0f;
                            const float alpha = need ? lk_exp2((mst[qb] - mx) * sq[qb]) : 1.0f;
                            mst[qb] = need ? mx : mst[qb];
#pragma unroll
                            for (int db = 0; db < 5; ++db) acc[db][qb] *= alpha;
                            const float mo = moff(qb);
#pragma unroll
                            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                                for (int i = 0; i < 4; ++i) {
                                    pb[qb][kk][i]     = (_Float16) lk_exp2(fmaf(x[2 * kk][j][i], sq[qb], -mo));
                                    pb[qb][kk][4 + i] = (_Float16) lk_exp2(fmaf(x[2 * kk + 1][j][i], sq[qb], -mo));
                                }
                        }
                    }
                }
            }
        }
        // ---- O^T += V^T . P^T over the 64 keys, 32 per MFMA -----------------------
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const lk_h4 lo = lk_ds_tr4(S.v + o_vd[db] + 4096 * kk);          // keys 32kk + 4g + col/4
                const lk_h4 hi = lk_ds_tr4(S.v + o_vd[db] + 4096 * kk + 2048);   // keys +16
                const lk_h8 va = { lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3] };
#pragma unroll
                for (int qb = 0; qb < PF_QB; ++qb)
                    acc[db][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb[qb][kk], acc[db][qb], 0, 0, 0);
            }
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb)
                acc[4][qb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[qb][kk], acc[4][qb], 0, 0, 0);
        }
    };

    // ---- epilogue: l over the 4 lane groups, then o[q][head*64 + d] -------------
    auto emit = [&]() {
        // PAIR: NaN outputs when a group barrier of this workgroup gave up
        bool poison = false;
        if constexpr (PAIR)
            poison = (__hip_atomic_load(&s_gbad[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) |
                      __hip_atomic_load(&s_gbad[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) != 0u;
#pragma unroll
        for (int qb = 0; qb < PF_QB; ++qb) {
            const float il = poison ? __builtin_nanf("") : 1.0f / acc[4][qb][0];
            const int qr = qbase + 16 * qb + col;
            lk_f4 a[4];
#pragma unroll
            for (int db = 0; db < 4; ++db) a[db] = acc[db][qb] * il;
            if (o && qr < m) {
#pragma unroll
                for (int db = 0; db < 4; ++db)
                    *(float4 *) (o + (size_t) qr * LK_HIDDEN + head * LK_HEAD_DIM + 16 * db + 4 * g) =
                        make_float4(a[db][0], a[db][1], a[db][2], a[db][3]);
            }
            if constexpr (Q81) lk_pf_q81_epilogue(a, qr < m, aqs + (size_t) qr * LK_HIDDEN + head * LK_HEAD_DIM,
                                        asc + (size_t) qr * (LK_HIDDEN / 32) + 2 * head, g);
        }
    };

    if constexpr (!PAIR) {
        // ---- tile loop: one barrier per tile; tile kt+1 streams in while kt computes
        for (int kt = kt_lo; kt < kt_hi; ++kt) {
            lk_wait_vm<0>();                              // this wave's part of tile kt landed
            __syncthreads();                              // ... everyone's; tile kt-1 fully consumed
            if (kt + 1 < kt_hi) issue(kt + 1);            // into the stage tile kt-1 used
            tile(st[kt & 1], kt);
        }

        if (pslot >= 0) {                                 // a part: unnormalised partial
            float * R = pbuf + (size_t) (pslot * LK_N_KV_HEADS + kvh) * PF_PART_SLOT;
            lk_f4 * A = (lk_f4 *) R + (size_t) w * 16 * PF_BQ;             // [16 chunks][64 rows]
            float2 * ML = (float2 *) (R + PF_PART_ACC) + w * PF_BQ;       // [64 rows]
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const int row = 16 * qb + col;
#pragma unroll
                for (int db = 0; db < 4; ++db) A[(4 * db + g) * PF_BQ + row] = acc[db][qb];
                if (g == 0) ML[row] = make_float2(moff(qb), acc[4][qb][0]);
            }
            return;
        }
        emit();
    } else {
        // ---- the group's step loop: one group barrier per step; step it+1's
        // tile streams in during step it
        for (int it = 0; it < g_ns; ++it) {
            lk_wait_vm<0>();
            gsync();
            if (it + 1 < g_ns) issue_step(it + 1);
            tile(st[2 * grp + (it & 1)], g_tile(it));
            if (grp == 0 && it == nki - 1) {
                // bi is complete: write it; group A goes on with bj, whose fp16
                // Q block group B's wave of the same head holds in LDS
                emit();
                qt = bj;
                qbase = bj * PF_BQ;
                qw = hw + 4;
                load_q(false, qw);
#pragma unroll
                for (int db = 0; db < 5; ++db)
#pragma unroll
                    for (int qb = 0; qb < PF_QB; ++qb) acc[db][qb] = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
#pragma unroll
                for (int qb = 0; qb < PF_QB; ++qb) mst[qb] = -INFINITY;
            }
        }
        // ---- group A's part of bj into group B's, through LDS (the tile stages
        // are free now), in the split-partial layout; lane l of wave hw+4 reads
        // exactly what lane l of wave hw wrote.  Fixed order: B's part, then A's.
        PF_TSTAMP(2);
        __syncthreads();
        float * R = (float *) &st[0];
        lk_f4 * A = (lk_f4 *) R + (size_t) hw * 16 * PF_BQ;
        float2 * ML = (float2 *) (R + PF_PART_ACC) + hw * PF_BQ;
        if (grp == 0) {
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const int row = 16 * qb + col;
#pragma unroll
                for (int db = 0; db < 4; ++db) A[(4 * db + g) * PF_BQ + row] = acc[db][qb];
                ML[row] = make_float2(moff(qb), acc[4][qb][0]);
            }
        }
        __syncthreads();
        if (grp == 1) {
#pragma clang fp contract(off)
#pragma unroll
            for (int qb = 0; qb < PF_QB; ++qb) {
                const int row = 16 * qb + col;
                const float2 ml = ML[row];
                const float mb = moff(qb);
                const float mx = fmaxf(mb, ml.x);
                const float fb = lk_exp2(mb - mx), fa = lk_exp2(ml.x - mx);
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const lk_f4 pa = A[(4 * db + g) * PF_BQ + row];
                    acc[db][qb] = acc[db][qb] * fb + pa * fa;
                }
                acc[4][qb][0] = acc[4][qb][0] * fb + ml.y * fa;
            }
            emit();
        }
        PF_TSTAMP(3);
    }
}

// Merge of the parts of split query blocks: workgroup (split block, kv head,
// half of the dims), thread = (head, row) over 32 dims -- one Q8_1 block; the
// parts are weighted 2^(m_p - M) with the exact max M and summed in part
// order.  All of a thread's loads are independent, so it waits for memory
// about twice.
__global__ void __launch_bounds__(256)
lk_k_pf_combine(const float * __restrict__ pbuf, int m, int P, const PfWork work, float * __restrict__ o,
                int8_t * __restrict__ aqs, float2 * __restrict__ asc) {
#pragma clang fp contract(off)
    constexpr int MAXP = 4;                               // parts merged per pass
    const int kvh = blockIdx.y, hb = blockIdx.z;          // dims 32hb .. 32hb+31
    const int qt = work.split_qt[blockIdx.x];
    const int np = work.nparts[qt];
    const int slot = work.slot0[qt];
    const int row = threadIdx.x & 63, h = threadIdx.x >> 6;
    const int qr = qt * PF_BQ + row;
    if (qr >= m) return;
    auto base = [&](int p) { return pbuf + (size_t) ((slot + p) * LK_N_KV_HEADS + kvh) * PF_PART_SLOT; };
    float M = -INFINITY, L = 0.0f;
    lk_f4 A[8] = {};
    // one pass over parts [p0, p0 + W): all loads first (one memory round
    // trip), then the merge in part order
    auto pass = [&](auto wc, int p0) {
        constexpr int W = decltype(wc)::value;
        float2 ml[W];
        lk_f4 a[W][8];
#pragma unroll
        for (int i = 0; i < W; ++i) {
            const int p = (p0 + i < np) ? p0 + i : p0;    // clamped: loads stay in bounds
            ml[i] = ((const float2 *) (base(p) + PF_PART_ACC))[h * PF_BQ + row];
            const lk_f4 * src = (const lk_f4 *) base(p) + (size_t) (h * 16 + 8 * hb) * PF_BQ + row;
#pragma unroll
            for (int c = 0; c < 8; ++c) a[i][c] = src[c * PF_BQ];
        }
        float Mn = M;
#pragma unroll
        for (int i = 0; i < W; ++i) if (p0 + i < np) Mn = fmaxf(Mn, ml[i].x);
        const float r = lk_exp2(M - Mn);                  // 0 on the first pass (M = -inf)
        L *= r;
#pragma unroll
        for (int c = 0; c < 8; ++c) A[c] *= r;
#pragma unroll
        for (int i = 0; i < W; ++i) {
            if (p0 + i >= np) break;
            const float wgt = lk_exp2(ml[i].x - Mn);
            L += ml[i].y * wgt;
#pragma unroll
            for (int c = 0; c < 8; ++c) A[c] += a[i][c] * wgt;
        }
        M = Mn;
    };
    // two parts per block is the common case: no redundant loads for it
    if (np == 2) pass(std::integral_constant<int, 2>{}, 0);
    else for (int p0 = 0; p0 < np; p0 += MAXP) pass(std::integral_constant<int, MAXP>{}, p0);
    const float il = 1.0f / L;
    float x[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const lk_f4 v = A[c] * il;
#pragma unroll
        for (int r = 0; r < 4; ++r) x[4 * c + r] = v[r];
    }
    const size_t col0 = (size_t) (kvh * LK_G + h) * LK_HEAD_DIM + 32 * hb;
    if (o) {
        float * dst = o + (size_t) qr * LK_HIDDEN + col0;
#pragma unroll
        for (int c = 0; c < 8; ++c) *(float4 *) (dst + 4 * c) = make_float4(x[4 * c], x[4 * c + 1], x[4 * c + 2], x[4 * c + 3]);
    }
    if (aqs) {                                            // the block's Q8_1, in-thread, same tree
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) am = fmaxf(am, fabsf(x[i]));
        float t[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) t[i] = x[i];
#pragma unroll
        for (int st = 16; st > 0; st >>= 1)
#pragma unroll
            for (int i = 0; i < st; ++i) t[i] = t[i] + t[i + st];
        const float d = am / 127.0f;
        const LkQ81Div qd = lk_q81_div(am, d);
        int8_t * q = aqs + (size_t) qr * LK_HIDDEN + col0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            uint32_t w = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r) w |= (uint32_t) (uint8_t) lk_q81_qd(qd, x[4 * c + r]) << (8 * r);
            *(uint32_t *) (q + 4 * c) = w;
        }
        asc[(size_t) qr * (LK_HIDDEN / 32) + col0 / 32] = lk_q81_scales(d, t[0]);
    }
}

// Standalone planar Q8_1 of fp32 rows (reference k_pf_quant_rows,
// prefill.cu:1574-1580): grid (rows, ceil(kb/8)) x 256, one 32-lane half-wave
// per (row, block), one value per lane; the sum tree is the lane butterfly
// 16, 8, 4, 2, 1.
__global__ void __launch_bounds__(256)
lk_k_pf_quant_rows(const float * __restrict__ X, int ld, int kb, int8_t * __restrict__ qs,
                   float2 * __restrict__ sc) {
#pragma clang fp contract(off)
    const int r = blockIdx.x;
    const int b = blockIdx.y * 8 + (threadIdx.x >> 5), lane = threadIdx.x & 31;
    const bool ok = b < kb;                               // half-wave uniform
    const float x = ok ? X[(size_t) r * ld + b * 32 + lane] : 0.0f;
    const float am = lk_bfly32_max(fabsf(x)), sum = lk_bfly32_sum(x);
    const float d = am / 127.0f;
    if (!ok) return;
    qs[(size_t) r * kb * 32 + b * 32 + lane] = lk_q81_q(x, am, d);
    if (lane == 0) sc[(size_t) r * kb + b] = lk_q81_scales(d, sum);
}

// Test hook: s[h][i][j] = int32 q8[i][h] . k8[j][h/4], one wave per 16x16 block,
// by the routine the attention kernel scores int8 tiles with: the MFMA seeded
// with the bit pattern of PF_MAGIC, its result read back as fp32 PF_MAGIC + sum,
// returned as (bits - 0x4B400000), which equals the integer sum exactly while
// |sum| < 2^22 (the int8 bound is 64 * 128 * 128 = 2^20).
__global__ void __launch_bounds__(64)
lk_k_pf_qk_i32(const int8_t * __restrict__ q8, int m, const int8_t * __restrict__ k8, int n,
               int32_t * __restrict__ s) {
    const int j0 = blockIdx.x * 16, i0 = blockIdx.y * 16, h = blockIdx.z;
    const int lane = threadIdx.x, col = lane & 15, g = lane >> 4;
    const lk_i4 kf = *(const lk_i4 *) (k8 + ((size_t) (j0 + col) * LK_N_KV_HEADS + h / LK_G) * LK_HEAD_DIM + 16 * g);
    const lk_i4 qf = *(const lk_i4 *) (q8 + (size_t) (i0 + col) * LK_HIDDEN + h * LK_HEAD_DIM + 16 * g);
    // c[r] = PF_MAGIC + S^T[key j0+4g+r][query i0+col].  The whole vector is
    // reinterpreted, not an element: this compiler lowers __builtin_bit_cast of
    // a vector element (c[r]) to a load of element 0 for every r.
    const lk_i4 c = __builtin_bit_cast(lk_i4, lk_mfma_qk8_magic(kf, qf));
#pragma unroll
    for (int r = 0; r < 4; ++r)
        s[((size_t) h * m + i0 + col) * n + j0 + 4 * g + r] = c[r] - 0x4B400000;
}

// ---------------------------------------------------------------------------
// C ABI
extern "C" int lk_pf_q8(const void * qh, int m, const float * cm, int8_t * q8,
                        float * qsc, float * qcs, void * stream) {
    if (m < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_q8: m < 0");
    if (m == 0) return 0;
    if (!qh || !q8 || !qsc || !qcs) return lk_fail(hipErrorInvalidValue, "lk_pf_q8: null pointer argument");
    const int rows = m * LK_N_HEADS;
    hipLaunchKernelGGL(lk_k_pf_q8, dim3((rows + 31) / 32), dim3(256), 0, lk_stream(stream),
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
    hipLaunchKernelGGL(lk_k_pf_k8, dim3((unsigned) ((rows + 31) / 32)), dim3(256), 0, lk_stream(stream),
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

// ---- host: split choice -------------------------------------------------------
// Process-wide tuning knobs, atomics so that calls from several host threads
// may read them while a test sets them; each launch reads each knob once.
// -1: never split, 0: automatic, > 0: parts of at most that many tiles (test hook)
static std::atomic<int> g_pf_split_override{0};
// Poll bound of the paired kernel's group barrier (test hook; the default
// leaves ample time: a group waits for its slowest wave of one tile step,
// microseconds, while 2^22 polls of s_sleep 1 take about a quarter second).
#define PF_GSYNC_SPIN_DEFAULT (1 << 22)
static std::atomic<int> g_pf_gsync_spin{PF_GSYNC_SPIN_DEFAULT};

extern "C" int lk_pf_split_override(int tiles) {
    if (tiles < -1) return lk_fail(hipErrorInvalidValue, "lk_pf_split_override: %d < -1", tiles);
    g_pf_split_override.store(tiles, std::memory_order_relaxed);
    return 0;
}

extern "C" int lk_pf_gsync_limit(int polls) {
    if (polls < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_gsync_limit: %d < 0", polls);
    g_pf_gsync_spin.store(polls == 0 ? PF_GSYNC_SPIN_DEFAULT : polls, std::memory_order_relaxed);
    return 0;
}

extern "C" int lk_pf_gsync_faults(unsigned * count, int reset) {
    if (!count) return lk_fail(hipErrorInvalidValue, "lk_pf_gsync_faults: count is null");
    hipError_t e = hipMemcpyFromSymbol(count, HIP_SYMBOL(g_pf_gsync_fault), sizeof(unsigned), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return lk_fail((int) e, "lk_pf_gsync_faults: %s", hipGetErrorString(e));
    if (reset) {
        const unsigned z = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_pf_gsync_fault), &z, sizeof z, 0, hipMemcpyHostToDevice);
        if (e != hipSuccess) return lk_fail((int) e, "lk_pf_gsync_faults: %s", hipGetErrorString(e));
    }
    return 0;
}

extern "C" size_t lk_pf_part_bytes(void) { return (size_t) PF_PART_CAP * sizeof(float); }

#ifdef PF_TIMING
// Measurement builds only: the paired kernel's per-wave timestamps.
extern "C" int lk_pf_timing_read(unsigned long long * out, size_t n) {
    const hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(g_pf_part), n * sizeof(unsigned long long), 0,
                                             hipMemcpyDeviceToHost);
    return e == hipSuccess ? 0 : lk_fail((int) e, "lk_pf_timing_read: %s", hipGetErrorString(e));
}
#endif

// Device address of the partial scratch, per device (looked up once), and the
// guard of its single-stream use: the stream of the last splitting launch on
// each device and an event recorded after its combine.  A splitting launch on
// another stream while that event is still pending would overwrite partials
// the earlier launch has not merged yet; it is refused (hipErrorNotReady)
// instead.  Launches on one stream are ordered and always accepted.  Under
// stream capture the guard is not applied (the graph's own order decides).
// A launch holds g_pf_mu from the check to the record (pf_attn_launch), so
// that two host threads cannot both pass the check before either has recorded.
struct PfScratchUse {
    float * ptr = nullptr;
    hipStream_t last = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
};
static std::mutex g_pf_mu;
static PfScratchUse g_pf_use[LK_MAX_DEVICES];

// Called with g_pf_mu held.
static float * pf_part_acquire(hipStream_t st, int & err, int & dev_out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= LK_MAX_DEVICES) {
        err = lk_fail(e != hipSuccess ? (int) e : (int) hipErrorInvalidDevice, "prefill: no usable current device");
        return nullptr;
    }
    PfScratchUse & u = g_pf_use[dev];
    if (!u.ptr) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_pf_part));
        if (e != hipSuccess) { err = lk_fail((int) e, "prefill: scratch lookup: %s", hipGetErrorString(e)); return nullptr; }
        e = hipEventCreateWithFlags(&u.done, hipEventDisableTiming);
        if (e != hipSuccess) { err = lk_fail((int) e, "prefill: scratch guard event: %s", hipGetErrorString(e)); return nullptr; }
        u.ptr = (float *) p;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void) hipStreamIsCapturing(st, &cs);
    if (cs == hipStreamCaptureStatusNone && u.pending && u.last != st) {
        e = hipEventQuery(u.done);
        (void) hipGetLastError();                     // the query's status is not a launch error
        if (e == hipErrorNotReady) {
            err = lk_fail(hipErrorNotReady,
                          "prefill: a split-K launch on another stream of device %d is still pending; "
                          "split launches share one partial buffer per device: order them on one stream "
                          "(or wait for the earlier one)", dev);
            return nullptr;
        }
    }
    err = 0;
    dev_out = dev;
    return u.ptr;
}

// After the combine is enqueued on st: mark the scratch busy until it completes.
// Called with g_pf_mu held.
static int pf_part_release(hipStream_t st, int dev) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void) hipStreamIsCapturing(st, &cs);
    if (cs != hipStreamCaptureStatusNone) return 0;
    PfScratchUse & u = g_pf_use[dev];
    const hipError_t e = hipEventRecord(u.done, st);
    if (e != hipSuccess) return lk_fail((int) e, "prefill: scratch guard record: %s", hipGetErrorString(e));
    u.last = st;
    u.pending = true;
    return 0;
}

static int pf_slots_per_device() {
    // looked up once per device; threads that race here store the same value
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 512;
    int c = cus[dev].load(std::memory_order_relaxed);
    if (!c) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev].store(c, std::memory_order_relaxed);
    }
    return 2 * c;                                         // two attention workgroups per CU
}

// The work list of this chunk: n_items = 0 for an unsplit launch.
//
// Automatic plan.  Cost model, in units of one int8 tile on a CU shared by
// two workgroups (from per-workgroup timestamps on MI355X): int8 tile 1,
// exact or mixed tile 1.4, start-up of a workgroup 2.1.  T = total cost / the
// slots one kv head gets (a slot: one of the two workgroups of a CU).  When
// the costliest block exceeds 1.25 T (a causal chunk with P small against
// m), every block costlier than T is cut into pieces of cost T, from its
// first tile on, and the rest; items are dispatched costliest first, so the
// remainders and the short blocks fill the slots that free up early.  (A
// dispatch simulation calibrated on the measured spans of the C4 chunk: 113 ->
// 100 us, the floor being ~89.)  T grows when the parts would not fit the
// partial buffer or the item list.
#ifndef PF_PLAN_T
#define PF_PLAN_T 1.0f      // piece cost, in units of the mean cost per slot
#endif
static void pf_plan(int m, int P, int near, int sink, bool int8, int split_override, size_t cap_floats,
                    PfWork & wk) {
    wk.n_items = 0; wk.n_split = 0;
    const int nq = (m + PF_BQ - 1) / PF_BQ;
    if (split_override < 0 || nq > PF_MAX_QB) return;
    auto tcost = [&](int qt, int kt) -> float {
        return (!int8 || lk_pf_exact(P, 2 * qt, kt, near, sink)) ? 1.4f : 1.0f;
    };
    constexpr float START = 2.1f;
    // cost of key tiles [a, b) of block qt in closed form: the exact tiles of a
    // block are tile 0 with the sink and the run from the first tile within
    // `near` of the block's first 32 queries to the end (lk_pf_exact)
    auto rcost = [&](int qt, int a, int b) -> float {
        if (!int8) return START + 1.4f * (float) (b - a);
        const int lim = P + 2 * qt * 32 - near;               // exact iff kt*64 + 64 > lim
        const int kex = (lim < 64) ? 0 : (lim - 64) / 64 + 1;  // first such tile
        int nex = b - ((a > kex) ? a : kex);
        nex = (nex > 0) ? nex : 0;
        if (sink && a == 0 && kex > 0 && b > 0) ++nex;           // tile 0, outside the run
        return START + (float) (b - a) + 0.4f * (float) nex;
    };
    constexpr int MAXP = 64;                           // pieces per block
    int cut[PF_MAX_QB][MAXP + 1];                      // piece boundaries per block
    int npc[PF_MAX_QB];
    auto fits = [&]() {
        int items = 0, parts = 0;
        for (int qt = 0; qt < nq; ++qt) { items += npc[qt]; if (npc[qt] > 1) parts += npc[qt]; }
        return items <= PF_MAX_ITEMS && (size_t) parts * LK_N_KV_HEADS * PF_PART_SLOT <= cap_floats;
    };
    if (split_override > 0) {                          // equal parts of at most L tiles
        for (int L = split_override;; L *= 2) {
            bool ok = true;
            for (int qt = 0; qt < nq; ++qt) {
                int np, per;
                pf_parts(qt, m, P, L, np, per);
                const int nkt = pf_nkt(qt, m, P);
                if (np > MAXP) { np = 1; per = nkt; ok = false; }
                npc[qt] = np;
                for (int p = 0; p <= np; ++p) cut[qt][p] = (p * per < nkt) ? p * per : nkt;
            }
            if (ok && fits()) break;
        }
    } else {
        float total = 0.0f, cmax = 0.0f;
        float bc[PF_MAX_QB];
        for (int qt = 0; qt < nq; ++qt) {
            bc[qt] = rcost(qt, 0, pf_nkt(qt, m, P));
            total += bc[qt];
            cmax = (bc[qt] > cmax) ? bc[qt] : cmax;
        }
        float T = PF_PLAN_T * total * LK_N_KV_HEADS / (float) pf_slots_per_device();
        if (T < 8.0f) T = 8.0f;
        if (cmax <= 1.25f * T) return;
        for (;; T *= 1.25f) {
            for (int qt = 0; qt < nq; ++qt) {
                const int nkt = pf_nkt(qt, m, P);
                const int kdiag = (P + qt * PF_BQ) / PF_BK;
                int np = 0;
                cut[qt][np] = 0;
                float c = START;
                for (int kt = 0; kt < nkt; ++kt) {
                    c += tcost(qt, kt);
                    // close the piece at cost T if the next one may start at kt + 1
                    if (c >= T && kt + 1 < nkt && kt + 1 <= kdiag && np + 1 < MAXP) {
                        cut[qt][++np] = kt + 1;
                        c = START;
                    }
                }
                cut[qt][++np] = nkt;
                npc[qt] = np;
            }
            if (fits()) break;
        }
    }
    // items: block order from the last block down, then stable-sorted by cost
    struct It { float cost; int qt, lo, hi, slot; };
    It list[PF_MAX_ITEMS];
    int n = 0, slot = 0;
    for (int qt = nq - 1; qt >= 0; --qt) {
        const int np = npc[qt];
        wk.slot0[qt] = (int16_t) (np > 1 ? slot : -1);
        wk.nparts[qt] = (uint8_t) np;
        if (np > 1) wk.split_qt[wk.n_split++] = (uint8_t) qt;
        for (int p = 0; p < np; ++p)
            list[n++] = It{ rcost(qt, cut[qt][p], cut[qt][p + 1]), qt, cut[qt][p], cut[qt][p + 1],
                            np > 1 ? slot + p : -1 };
        if (np > 1) slot += np;
    }
    if (wk.n_split == 0) { wk.n_items = 0; return; }
    std::stable_sort(list, list + n, [](const It & a, const It & b) { return a.cost > b.cost; });
    for (int i = 0; i < n; ++i) {
        wk.item[i] = (uint32_t) list[i].qt | ((uint32_t) (list[i].slot + 1) << 16);
        wk.krange[i] = (uint32_t) list[i].lo | ((uint32_t) list[i].hi << 16);
    }
    wk.n_items = n;
}

extern "C" int lk_pf_plan_items(int m, int P, int near, int sink, int int8, int32_t * items, int max_items) {
    if (m < 1 || P < 0 || max_items < 0 || (!items && max_items > 0)) return -1;
    PfWork wk;
    pf_plan(m, P, near, sink, int8 != 0, g_pf_split_override.load(std::memory_order_relaxed), PF_PART_CAP, wk);
    for (int i = 0; i < wk.n_items && i < max_items; ++i) {
        items[4 * i + 0] = (int32_t) (wk.item[i] & 255);
        items[4 * i + 1] = (int32_t) (wk.krange[i] & 0xffff);
        items[4 * i + 2] = (int32_t) (wk.krange[i] >> 16);
        items[4 * i + 3] = (int32_t) (wk.item[i] >> 16) - 1;
    }
    return wk.n_items;
}

// Paired launches (8-wave workgroups over blocks i and nq-1-i): -1 never,
// 0 automatic, 1 whenever the chunk has at least two query blocks (test hook).
static std::atomic<int> g_pf_pair_override{0};

extern "C" int lk_pf_pair_override(int mode) {
    if (mode < -1 || mode > 1) return lk_fail(hipErrorInvalidValue, "lk_pf_pair_override: %d not in -1..1", mode);
    g_pf_pair_override.store(mode, std::memory_order_relaxed);
    return 0;
}

// Automatic choice: chunks of at least 64 query blocks (4096 rows, one paired
// workgroup per CU) with P <= m, where the causal triangle dominates the work.
// Measured (repetitions alternating, 4096-row chunks): P = 0 int8 103.4 us
// against 110.8 unpaired (split plan + combine), fp16 95.2 against 112.4;
// P = 4096 int8 265.7 against 271.5, fp16 254.1 against 279.5.  Deep chunks
// keep the split plan (P = 126976: int8 4383 us paired against 3862, fp16
// 4397 against 4173).  Not under a forced split size.
static bool pf_use_pair(int m, int P, int pair_override, int split_override) {
    const int nq = (m + PF_BQ - 1) / PF_BQ;
    if (pair_override < 0 || nq < 2) return false;
    if (pair_override > 0) return true;
    return split_override <= 0 && P <= m && nq >= 64;
}

template <bool INT8, bool Q81>
static int pf_attn_launch(const int8_t * q8, const float * qsc, const float * qcs, const _Float16 * qh,
                          int m, int P, const int8_t * k8, const float * ksc, int kstride,
                          const _Float16 * kc, const _Float16 * vc, int near, int sink, float * o,
                          int8_t * aqs, float2 * asc, float * work, size_t work_bytes, hipStream_t st,
                          const char * what) {
    PfWork wk;
    wk.spin = g_pf_gsync_spin.load(std::memory_order_relaxed);
    const int split_override = g_pf_split_override.load(std::memory_order_relaxed);
    if (pf_use_pair(m, P, g_pf_pair_override.load(std::memory_order_relaxed), split_override)) {
        wk.n_items = 0; wk.n_split = 0;
        const int npairs = ((m + PF_BQ - 1) / PF_BQ + 1) / 2;
        hipLaunchKernelGGL((lk_k_pf_attn<INT8, true, Q81>), dim3(npairs * LK_N_KV_HEADS), dim3(512), 0, st,
                           q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc, wk,
                           (float *) nullptr);
        return lk_launch_status(what);
    }
    // a caller workspace bounds the partials the plan may write (a smaller one
    // gives coarser pieces, none at all an unsplit launch); without one the
    // library's static scratch is used
    pf_plan(m, P, near, sink, INT8, split_override, work ? work_bytes / sizeof(float) : (size_t) PF_PART_CAP, wk);
    if (wk.n_items == 0) {
        hipLaunchKernelGGL((lk_k_pf_attn<INT8, false, Q81>), dim3((m + PF_BQ - 1) / PF_BQ, LK_N_KV_HEADS), dim3(256), 0, st,
                           q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc, wk,
                           (float *) nullptr);
        return lk_launch_status(what);
    }
    // the static scratch: the guard's check, the launches and its record under
    // one lock (a caller's workspace needs none)
    std::unique_lock<std::mutex> lock(g_pf_mu, std::defer_lock);
    if (!work) lock.lock();
    int err = 0, dev = 0;
    float * pbuf = work ? work : pf_part_acquire(st, err, dev);
    if (!pbuf) return err;
    hipLaunchKernelGGL((lk_k_pf_attn<INT8, false, Q81>), dim3(wk.n_items * LK_N_KV_HEADS), dim3(256), 0, st,
                       q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc, wk, pbuf);
    int rc = lk_launch_status(what);
    if (rc) return rc;
    hipLaunchKernelGGL(lk_k_pf_combine, dim3(wk.n_split, LK_N_KV_HEADS, 2), dim3(256), 0, st,
                       (const float *) pbuf, m, P, wk, o, aqs, asc);
    rc = lk_launch_status(what);
    if (rc) return rc;
    return work ? 0 : pf_part_release(st, dev);      // a caller's workspace is ordered by the caller
}

extern "C" int lk_pf_attn8_ws(const int8_t * q8, const float * qsc, const float * qcs,
                              const void * qh, int m, int P, const int8_t * k8,
                              const float * ksc, int kstride, const void * kc,
                              const void * vc, int near, int sink, float * o,
                              int8_t * aqs, float * asc, void * work, size_t work_bytes, void * stream) {
    if (m < 0 || P < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: m %d / P %d negative", m, P);
    if (work && ((uintptr_t) work % 16 != 0))
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: the workspace must be 16-byte aligned");
    if (m == 0) return 0;
    if (kstride % 4 != 0 || kstride < P + m)
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: kstride %d must be a multiple of 4 and >= P+m %d", kstride, P + m);
    if (!qh || !k8 || !ksc || !kc || !vc || (!o && !aqs) || (!aqs != !asc))
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: null pointer argument");
    // q8 = qsc = qcs = NULL: the kernel quantises qh itself (no smoothing)
    if (!q8 != !qsc || (!q8 && qcs))
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: q8 and qsc go together; without them (Q quantised in the kernel) qcs must be NULL too");
    // the Q8_1 epilogue is a template instance of its own, so that the plain
    // fp32-output kernel is compiled without it
    auto go = [&](auto launch) {
        return launch(q8, qsc, qcs, (const _Float16 *) qh, m, P, k8, ksc, kstride,
                      (const _Float16 *) kc, (const _Float16 *) vc, near, sink, o,
                      aqs, (float2 *) asc, (float *) work, work_bytes, lk_stream(stream), "lk_pf_attn8");
    };
    return aqs ? go(pf_attn_launch<true, true>) : go(pf_attn_launch<true, false>);
}

extern "C" int lk_pf_attn8_q81(const int8_t * q8, const float * qsc, const float * qcs,
                               const void * qh, int m, int P, const int8_t * k8,
                               const float * ksc, int kstride, const void * kc,
                               const void * vc, int near, int sink, float * o,
                               int8_t * aqs, float * asc, void * stream) {
    return lk_pf_attn8_ws(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o, aqs, asc,
                          nullptr, 0, stream);
}

extern "C" int lk_pf_attn8(const int8_t * q8, const float * qsc, const float * qcs,
                           const void * qh, int m, int P, const int8_t * k8,
                           const float * ksc, int kstride, const void * kc,
                           const void * vc, int near, int sink, float * o, void * stream) {
    if (m > 0 && !o) return lk_fail(hipErrorInvalidValue, "lk_pf_attn8: null pointer argument");
    return lk_pf_attn8_q81(q8, qsc, qcs, qh, m, P, k8, ksc, kstride, kc, vc, near, sink, o,
                           nullptr, nullptr, stream);
}

extern "C" int lk_pf_attn_ws(const void * qh, int m, int P, const void * kc, const void * vc,
                             float * o, int8_t * aqs, float * asc, void * work, size_t work_bytes,
                             void * stream) {
    if (m < 0 || P < 0) return lk_fail(hipErrorInvalidValue, "lk_pf_attn: m %d / P %d negative", m, P);
    if (work && ((uintptr_t) work % 16 != 0))
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn: the workspace must be 16-byte aligned");
    if (m == 0) return 0;
    if (!qh || !kc || !vc || (!o && !aqs) || (!aqs != !asc))
        return lk_fail(hipErrorInvalidValue, "lk_pf_attn: null pointer argument");
    auto go = [&](auto launch) {
        return launch(nullptr, nullptr, nullptr, (const _Float16 *) qh, m, P, nullptr, nullptr, 0,
                      (const _Float16 *) kc, (const _Float16 *) vc, 0, 0, o,
                      aqs, (float2 *) asc, (float *) work, work_bytes, lk_stream(stream), "lk_pf_attn");
    };
    return aqs ? go(pf_attn_launch<false, true>) : go(pf_attn_launch<false, false>);
}

extern "C" int lk_pf_attn_q81(const void * qh, int m, int P, const void * kc, const void * vc,
                              float * o, int8_t * aqs, float * asc, void * stream) {
    return lk_pf_attn_ws(qh, m, P, kc, vc, o, aqs, asc, nullptr, 0, stream);
}

extern "C" int lk_pf_attn(const void * qh, int m, int P, const void * kc, const void * vc,
                          float * o, void * stream) {
    if (m > 0 && !o) return lk_fail(hipErrorInvalidValue, "lk_pf_attn: null pointer argument");
    return lk_pf_attn_q81(qh, m, P, kc, vc, o, nullptr, nullptr, stream);
}

extern "C" int lk_pf_quant_rows(const float * X, int rows, int ld, int kb, int8_t * qs, float * sc,
                                void * stream) {
    if (rows < 0 || kb < 0 || ld < kb * 32)
        return lk_fail(hipErrorInvalidValue, "lk_pf_quant_rows: rows %d, kb %d, ld %d", rows, kb, ld);
    if (rows == 0 || kb == 0) return 0;
    if (!X || !qs || !sc) return lk_fail(hipErrorInvalidValue, "lk_pf_quant_rows: null pointer argument");
    hipLaunchKernelGGL(lk_k_pf_quant_rows, dim3(rows, (kb + 7) / 8), dim3(256), 0, lk_stream(stream),
                       X, ld, kb, qs, (float2 *) sc);
    return lk_launch_status("lk_pf_quant_rows");
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
