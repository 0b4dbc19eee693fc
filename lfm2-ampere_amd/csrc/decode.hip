// decode.hip - split-K GQA decode attention for gfx950.
//
// Reference behaviour: k_attn_split / k_attn_combine / k_attention_decode
// (/root/reference/src/kernels.cu:1303-1599, 768-852), launched per attention
// layer at engine.cu:638-641.  The arithmetic contract is the float64 host
// reference of tests/test_attn.cu:46-74:
//     out[h] = softmax(q[h] . K[0..seq)^T / 8) . V[0..seq)
// for the 32 query heads, K/V of kv head h/4 in the fp16 cache [pos][8][64].
//
// MI355X design (not a translation of the reference's warp-level loops):
//   * grid of LK_ATTN_SPLIT 8-wave workgroups, one per slice covering ALL 8
//     kv heads; the reference's slice count, but a slice is the set of tiles
//     of LK_DEC_TILE positions congruent to it modulo the slice count, not a
//     contiguous range (all workgroups then stream one moving front of the
//     cache: measured about 6% faster than contiguous shares at 32k-131k);
//     whole 1 KB cache rows are streamed once into LDS by LDS DMA
//     (algorithmic traffic: seq x 2 KB per layer); wave w then serves kv
//     head w and its 4 query heads;
//   * S^T = K . q^T on the matrix cores (v_mfma_f32_16x16x32_f16, keys as the
//     A operand).  q is fp32 in the interface, so it is split q = hi + lo into
//     two fp16 halves (22 significant bits; fp16 x fp16 products are exact in
//     fp32) and both halves are multiplied;
//   * online softmax in the log2 domain (v_exp_f32) with a lazily raised max;
//   * O^T += V^T . P^T on the matrix cores (v_mfma_f32_16x16x16_f16, V^T from
//     transposed LDS reads, P as hi + lo fp16 halves), l from an all-ones
//     operand -> one partial (m, l, acc[64]) per (query head, slice);
//   * the combine merges the slice partials in a fixed order (deterministic,
//     run-to-run bit-identical) and optionally emits Q8_1 blocks.
#include "lk_common.h"
#include <math.h>
#include <mutex>

// fp32 -> (hi, lo) fp16 pair with hi + lo == x to 22 bits.  x - (float)hi is
// exact in fp32 (hi is x rounded to 11 significant bits).
__device__ __forceinline__ void lk_split_h(float x, _Float16 & hi, _Float16 & lo) {
    hi = (_Float16) x;
    lo = (_Float16) (x - (float) hi);
}

// ---- decode split kernel ------------------------------------------------------
// The workgroup of slice sp covers ALL 8 kv heads of the tiles sp, sp + ns,
// sp + 2 ns, ... (tile T = positions 16T .. 16T+15, below seq): cache
// rows (one position = 8 heads x 64 dims = 1 KB of K, same of V) are fetched
// whole, 64 lanes x 16 contiguous bytes per instruction, straight into LDS
// (global_load_lds_dwordx4, no staging registers), into a ring of LK_DEC_NBUF
// tiles of LK_DEC_TILE positions; LK_DEC_NBUF-1 tiles are in flight while one
// is consumed.  Whole-row streaming is what lets HBM run near its peak: a
// per-head walk touches 128 of every 1024 bytes and measured ~40% slower.
// Wave w then serves kv head w (its 4 query heads) from the LDS tile.
// LDS rows are padded by 16 bytes so 16 lanes reading 16 bytes from 16
// consecutive rows hit 16 different bank groups.
#define LK_DEC_ROWB    (LK_KV_ROW * 2 + 16)                   // bytes per LDS row
#define LK_DEC_TILEB   (2 * LK_DEC_TILE * LK_DEC_ROWB)         // K rows + V rows
#define LK_DEC_THREADS 512                                     // 8 waves = 8 kv heads
// Measurement-only ablation (any non-zero value gives WRONG output): 1 = skip
// the P.V accumulate, 2 = skip Q.K^T and the softmax, 3 = skip both (the
// kernel then only streams K and V through LDS).
#ifndef LK_DEC_ABLATE
#define LK_DEC_ABLATE 0
#endif

// The decode producer (reference k_qk_norm_rope, kernels.cu:871-915) folded
// into the split kernel for the step graph: the inputs of one head row in the
// split kernel's q layout -- lane (col, g) holds dims 8g+i ("lo") and
// 32+8g+i ("hi"), i < 8, of the row, replicated over the columns -- normalised
// and rotated with the arithmetic of lk_k_qk_norm_rope bit for bit: squares
// rounded, the sum tree over d with strides 32 (in lane), 16 and 8 (lanes
// ^32, ^16: lk_xrow_sum adds in that order, both partners the same two
// values), then 4, 2, 1 in lane; 1/sqrt in fp64 rounded once; the rotation of
// the pair (d, d+32) with the table entry d.
__device__ __forceinline__ void lk_norm_rope_pair8(float (&lo)[8], float (&hi)[8], const float (&wlo)[8],
                                                   const float (&whi)[8], int g, const float * s_c, const float * s_s) {
#pragma clang fp contract(off)
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = lo[i] * lo[i], b = hi[i] * hi[i];
        t[i] = lk_xrow_sum(a + b);
    }
    const float u0 = t[0] + t[4], u1 = t[1] + t[5], u2 = t[2] + t[6], u3 = t[3] + t[7];
    const float ss = (u0 + u2) + (u1 + u3);
    const float arg = ss * (1.0f / LK_HEAD_DIM) + LK_EPS_F;
    const float inv = (float) (1.0 / sqrt((double) arg));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int d = 8 * g + i;
        const float yl = (lo[i] * inv) * wlo[i], yh = (hi[i] * inv) * whi[i];
        const float c = s_c[d], sn = s_s[d];
        lo[i] = yl * c - yh * sn;
        hi[i] = yl * sn + yh * c;
    }
}
// Pointers of the folded producer: projection rows in, working q / k rows out
// (the in-place API's buffers), norm weights; the cache row at *d_pos is
// written by the workgroup whose slice holds it.
struct LkDecProducer {
    const float * q_src, * k_src, * v_src, * q_norm, * k_norm;
    float * q_out, * k_out;
};

template <bool FUSED>
__global__ void __launch_bounds__(LK_DEC_THREADS)
lk_k_attn_split(const float * __restrict__ q, const _Float16 * kc,
                const _Float16 * vc, const int * __restrict__ d_pos,
                float * __restrict__ part, const LkDecProducer pr) {
    constexpr int RPW = 2 * LK_DEC_TILE / 8;                   // rows fetched per wave per tile
    constexpr int NG  = LK_DEC_TILE / 16;                      // 16-token groups per tile
    constexpr int D   = LK_DEC_NBUF - 1;                       // tiles in flight
    static_assert(LK_DEC_TILE % 16 == 0 && LK_DEC_NBUF >= 2, "decode tile shape");
    __shared__ __attribute__((aligned(16))) unsigned char s_tile[LK_DEC_NBUF][LK_DEC_TILEB];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave = kv head
    const int col = lane & 15, g = lane >> 4;

    // The inputs other than the cache tiles are loaded before the tile DMA
    // below: vector-memory loads complete in issue order, so a load issued
    // after the DMAs would wait for them (about 3 us at start-up).  This
    // lane's q values (dims 8g+i and 32+8g+i of head 4w + (col & 3)); with the
    // producer folded in also the rotary frequency of table entry 4w + lane
    // (lanes 0-3, a scalar load), the q norm weights and, after the slice
    // plan, the new row's k and v and the k norm weights (used only by the
    // workgroup whose slice holds the position).
    // Loaded untracked (lk_ld16_untracked) and awaited after the DMA issue
    // with a count that leaves the tile DMAs in flight: a tracked load here
    // would make the compiler wait for every tile in flight before the
    // first tile is consumed.  Vector r of each set holds values 4r..4r+3 of
    // the lane's 16 (8 "lo" at dims 8g.., 8 "hi" at dims 32+8g..).
    const int qrow = (w * LK_G + (col & 3)) * LK_HEAD_DIM + 8 * g;
    lk_f4 qv[4], qwv[4], kv4[4], vv4[4], kwv[4];
    float rfreq = 0.0f;
    {
        const float * qp = (FUSED ? pr.q_src : q) + qrow;
        qv[0] = lk_ld16_untracked(qp);      qv[1] = lk_ld16_untracked(qp + 4);
        qv[2] = lk_ld16_untracked(qp + 32); qv[3] = lk_ld16_untracked(qp + 36);
        if constexpr (FUSED) {
            rfreq = lk_rope_freq_quad(w, lane);
            const float * np = pr.q_norm + 8 * g;
            qwv[0] = lk_ld16_untracked(np);      qwv[1] = lk_ld16_untracked(np + 4);
            qwv[2] = lk_ld16_untracked(np + 32); qwv[3] = lk_ld16_untracked(np + 36);
        }
    }
    const int seq = *d_pos + 1;
    int ns, chunk;
    lk_attn_slices(seq, ns, chunk);
    (void) chunk;
    const int sp = blockIdx.x;
    // Slice sp holds tiles T = sp + ns * it, it < ntile, of the nt tiles that
    // cover [0, seq): slices differ by at most one tile.
    const int nt = (seq + LK_DEC_TILE - 1) / LK_DEC_TILE;
    const int ntile = (sp < ns && sp < nt) ? (nt - sp + ns - 1) / ns : 0;
    // A slice with no tiles (ntile = 0: sp >= nt or sp >= ns) takes the same
    // path with an empty tile loop, so its record is the neutral one (m =
    // -inf, l = 0, acc = 0) and every slot the combine reads is valid without
    // it knowing seq.  There is no early return: the untracked loads above
    // are in flight until the wait below, and code on a separate path would
    // be free to reuse their registers (a store address formed in one of
    // them would be overwritten by the arriving data).
    const int pos = seq - 1;
    const bool own_pos = FUSED && (nt - 1) % ns == sp;     // this slice holds position pos (its last tile)
    if constexpr (FUSED) {          // loaded by every workgroup: see the wait below
        const float * kp = pr.k_src + w * LK_HEAD_DIM + 8 * g;
        const float * vp = pr.v_src + w * LK_HEAD_DIM + 8 * g;
        const float * np = pr.k_norm + 8 * g;
        const int off[4] = { 0, 4, 32, 36 };
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            kv4[r] = lk_ld16_untracked(kp + off[r]);
            vv4[r] = lk_ld16_untracked(vp + off[r]);
            kwv[r] = lk_ld16_untracked(np + off[r]);
        }
    }

    // ---- fetch: wave w brings rows w, w+8, ... of each tile (K rows first) ----
    const char * kg = (const char *) kc + 16 * lane;
    const char * vg = (const char *) vc + 16 * lane;
    const uint32_t lds0 = lk_lds_addr(&s_tile[0][0]);
    // first position of the slice's tile it
    auto tile_pos = [&](int it) -> int { return (sp + ns * it) * LK_DEC_TILE; };
    const int clamp_row = ntile > 0 ? sp * LK_DEC_TILE : 0;
    auto fetch = [&](int it) {
        const uint32_t base = lds0 + (uint32_t) ((it % LK_DEC_NBUF) * LK_DEC_TILEB);
        const int p0 = tile_pos(it);
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int row = w + 8 * i;                         // 0 .. 2*TILE-1
            const bool isv = row >= LK_DEC_TILE;
            const int tp = p0 + (isv ? row - LK_DEC_TILE : row);
            // clamp: rows past seq and whole tiles past the slice's last fetch
            // the slice's first row (in range, and a different row in every
            // workgroup: a row shared by all of them would put every clamped
            // fetch on one L2 channel), all tiles of an empty slice row 0;
            // they are masked or land in buffers no tile of the slice uses
            const size_t o = (size_t) (it < ntile && tp < seq ? tp : clamp_row) * (LK_KV_ROW * 2);
            lk_dma16((isv ? vg : kg) + o, base + (uint32_t) (row * LK_DEC_ROWB));
        }
    };
    // Wait until tile `it` is resident for the whole workgroup.  When tile it
    // is awaited, this wave has issued tiles up to min(it + D - 1, ntile - 1)
    // (tile it + D is fetched only after tile it is awaited); its own fetches
    // complete in order, so the rows of those later tiles may stay pending.
    // The barrier then covers the other waves' rows.
    auto wait_tile = [&](int it) {
        const int later = (ntile - 1 - it < D - 1) ? ntile - 1 - it : D - 1;
        if (later >= 4)      lk_wait_vm<4 * RPW>();
        else if (later == 3) lk_wait_vm<3 * RPW>();
        else if (later == 2) lk_wait_vm<2 * RPW>();
        else if (later == 1) lk_wait_vm<RPW>();
        else                 lk_wait_vm<0>();
        __builtin_amdgcn_s_barrier();
    };
    static_assert(D - 1 <= 4 && 4 * RPW <= 63, "wait_tile handles at most four later tiles in flight");

    // Issue the first D tiles before anything else, so HBM starts streaming at
    // once.  All D are issued even for a slice of fewer tiles (the rows past
    // the slice are clamped to its first row and land in buffers no tile of
    // the slice uses), so that exactly D*RPW DMAs follow the early loads in
    // every workgroup and one wait with that count covers those loads.  The
    // early loads and the wait are unconditional too: the compiler does not
    // know an untracked load's registers are pending, and around a branch it
    // may copy them before the wait; lk_wait_vm_tie's operands pin every use
    // after it only in straight-line code.
#pragma unroll
    for (int i = 0; i < D; ++i) fetch(i);
    lk_wait_vm_tie<D * RPW>(qv);
    if constexpr (FUSED) {
        lk_wait_vm_tie<D * RPW>(qwv);
        lk_wait_vm_tie<D * RPW>(kv4); lk_wait_vm_tie<D * RPW>(vv4); lk_wait_vm_tie<D * RPW>(kwv);
    }
    float qlo[8], qhi[8], qwlo[8], qwhi[8];
    float klo[8], khi[8], vlo[8], vhi[8], kwlo[8], kwhi[8];
    auto unpack = [](const lk_f4 (&x)[4], float (&lo)[8], float (&hi)[8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) { lo[i] = x[0][i]; lo[4 + i] = x[1][i]; hi[i] = x[2][i]; hi[4 + i] = x[3][i]; }
    };
    unpack(qv, qlo, qhi);
    if constexpr (FUSED) {
        unpack(qwv, qwlo, qwhi);
        unpack(kv4, klo, khi); unpack(vv4, vlo, vhi); unpack(kwv, kwlo, kwhi);
    }

    // Folded producer: the 32 (cos, sin) entries of position seq-1, 4 per wave.
    __shared__ float s_c[FUSED ? LK_HEAD_DIM / 2 : 1], s_s[FUSED ? LK_HEAD_DIM / 2 : 1];
    lk_h8 kv_h[4];                                         // its K lo, K hi, V lo, V hi (fp16)
    if constexpr (FUSED) {
        if (lane < 4) lk_rope_angle(pos, rfreq, s_c[4 * w + lane], s_s[4 * w + lane]);
        __syncthreads();
        if (own_pos) {
            float lo[8], hi[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) { lo[i] = klo[i]; hi[i] = khi[i]; }
            lk_norm_rope_pair8(lo, hi, kwlo, kwhi, g, s_c, s_s);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kv_h[0][i] = (_Float16) lo[i]; kv_h[1][i] = (_Float16) hi[i];
                kv_h[2][i] = (_Float16) vlo[i]; kv_h[3][i] = (_Float16) vhi[i];
            }
            if (col == 0) {
                const size_t off = ((size_t) pos * LK_N_KV_HEADS + w) * LK_HEAD_DIM + 8 * g;
                _Float16 * kw = (_Float16 *) kc, * vw = (_Float16 *) vc;
                *(lk_h8 *) (kw + off) = kv_h[0]; *(lk_h8 *) (kw + off + 32) = kv_h[1];
                *(lk_h8 *) (vw + off) = kv_h[2]; *(lk_h8 *) (vw + off + 32) = kv_h[3];
                float * ko = pr.k_out + w * LK_HEAD_DIM + 8 * g;
                *(lk_f4 *) ko        = (lk_f4){ lo[0], lo[1], lo[2], lo[3] };
                *(lk_f4 *) (ko + 4)  = (lk_f4){ lo[4], lo[5], lo[6], lo[7] };
                *(lk_f4 *) (ko + 32) = (lk_f4){ hi[0], hi[1], hi[2], hi[3] };
                *(lk_f4 *) (ko + 36) = (lk_f4){ hi[4], hi[5], hi[6], hi[7] };
            }
        }
    }

    // Scores are computed transposed, S^T = K . Q^T (v_mfma_f32_16x16x32_f16):
    // A = 16 cache rows of the tile (lane: position col, dims 32ks+8g..+7),
    // B = Q^T with the 4 heads of kv head w replicated over the 16 columns
    // (column c = head 4w + (c & 3)).  Lane l then holds positions 4g..4g+3 of
    // one head, which is exactly the B operand of the P.V MFMA.  q is fp32 in
    // the interface: split q = hi + lo (fp16 x fp16 products are exact in fp32)
    // and both halves are multiplied.
    lk_h8 qbh[2], qbl[2];
    int qsh = 0;                                            // q of this lane's head is scaled by 2^-qsh
    {
        float lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { lo[i] = qlo[i]; hi[i] = qhi[i]; }
        if constexpr (FUSED) {
            lk_norm_rope_pair8(lo, hi, qwlo, qwhi, g, s_c, s_s);
            if (sp == 0 && col < 4) {                       // the working q, once
                float * qo = pr.q_out + qrow;
                *(lk_f4 *) qo        = (lk_f4){ lo[0], lo[1], lo[2], lo[3] };
                *(lk_f4 *) (qo + 4)  = (lk_f4){ lo[4], lo[5], lo[6], lo[7] };
                *(lk_f4 *) (qo + 32) = (lk_f4){ hi[0], hi[1], hi[2], hi[3] };
                *(lk_f4 *) (qo + 36) = (lk_f4){ hi[4], hi[5], hi[6], hi[7] };
            }
        }
        // The fp16 hi half of q must be finite: a head whose largest |q| reaches
        // 2^15 is scaled by 2^-k first (exact) so that it stays below 2^15, and
        // its scores are scaled back by 2^k below.  k = 0 for every other head
        // (the usual case, RMS-normed q), which leaves the arithmetic untouched.
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fmaxf(fabsf(lo[i]), fabsf(hi[i])));
        am = lk_xrow_max(am);                               // the head's 64 dims (lanes ^16, ^32)
        int e2 = 0;
        if (am >= 32768.0f && am <= 3.4e38f) {              // finite and too large for the fp16 split
            (void) frexpf(am, &e2);                         // am < 2^e2
            e2 -= 15;
#pragma unroll
            for (int i = 0; i < 8; ++i) { lo[i] = ldexpf(lo[i], -e2); hi[i] = ldexpf(hi[i], -e2); }
        }
        qsh = e2;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 h, l;
            lk_split_h(lo[i], h, l); qbh[0][i] = h; qbl[0][i] = l;
            lk_split_h(hi[i], h, l); qbh[1][i] = h; qbl[1][i] = l;
        }
    }
    // scores in log2 units; the power-of-2 factor undoes the q scaling above
    const float SC = ldexpf(0.125f * LK_LOG2E_F, qsh);
    // Running max is raised only when a score exceeds it by 2^8 in p: P stays
    // far inside fp16 range and most tiles skip the rescale.
    constexpr float HEADROOM = 8.0f;

    float mrun = -INFINITY;
    lk_f4 acc[4], accl;                     // O^T blocks (dims 16db..) and sum of p
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
    accl = (lk_f4){ 0.f, 0.f, 0.f, 0.f };
    const _Float16 one = (_Float16) 1.0f;
    const lk_h4 ones = { one, one, one, one };

    // ---- consume one tile: wave w = kv head w, NG blocks of 16 positions -----
    auto consume = [&](const unsigned char * buf, int it) {
#if LK_DEC_ABLATE == 3
        if (buf[lane] == 0x7f && it < 0) accl[0] += 1.0f;
        return;
#endif
        float x[NG][4];
        float mloc = -INFINITY;
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            const unsigned char * kr = buf + (16 * gi + col) * LK_DEC_ROWB + w * 128 + 16 * g;
            lk_f4 c = { 0.0f, 0.0f, 0.0f, 0.0f };
#if LK_DEC_ABLATE == 2
            c[0] = c[1] = c[2] = c[3] = (float) col;
#else
            const lk_h8 k0 = *(const lk_h8 *) kr;
            const lk_h8 k1 = *(const lk_h8 *) (kr + 64);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qbh[0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qbl[0], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qbh[1], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qbl[1], c, 0, 0, 0);
#endif
            const int t0g = tile_pos(it) + 16 * gi + 4 * g;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[gi][r] = (t0g + r < seq) ? c[r] * SC : -INFINITY;
                mloc = fmaxf(mloc, x[gi][r]);
            }
        }
        // every lane of a column (and its 3 replicas) sees the same max
        const float mx = lk_xrow_max(mloc);
        const bool need = mx > mrun + HEADROOM;
        if (__ballot(need)) {                                   // wave-uniform
            const float alpha = need ? lk_exp2(mrun - mx) : 1.0f;
            mrun = need ? mx : mrun;
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db] *= alpha;
            accl *= alpha;
        }
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
            lk_h4 ph, pl;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = lk_exp2(x[gi][r] - mrun);
                ph[r] = (_Float16) p;
                pl[r] = (_Float16) (p - (float) ph[r]);
            }
#if LK_DEC_ABLATE == 1
            accl[0] += (float) ph[0];
            continue;
#endif
            // V^T operand by transpose read: lane 4a+b of row group g supplies
            // V[position 4g+a][dims 16db+4b..+3]; lane c receives the 4
            // positions 4g..4g+3 of dim 16db + c.
            const unsigned char * vr = buf + (LK_DEC_TILE + 16 * gi + 4 * g + (col >> 2)) * LK_DEC_ROWB
                                     + w * 128 + 8 * (col & 3);
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const lk_h4 va = lk_ds_tr4(vr + 32 * db);
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc[db], 0, 0, 0);
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc[db], 0, 0, 0);
            }
            accl = __builtin_amdgcn_mfma_f32_16x16x16f16(ones, ph, accl, 0, 0, 0);
            accl = __builtin_amdgcn_mfma_f32_16x16x16f16(ones, pl, accl, 0, 0, 0);
        }
    };

    for (int it = 0; it < ntile; ++it) {
        wait_tile(it);
        // buffer (it + D) % NBUF = (it - 1) % NBUF: every wave finished reading
        // it before the barrier in wait_tile, so the next DMA goes out before
        // this tile is consumed (one barrier per tile)
        if (it + D < ntile) fetch(it + D);
        if (own_pos && it == ntile - 1 && col == 0) {
            // the new row, as the cache now holds it (the tile's copy may predate
            // the store above); wave w alone reads kv head w's bytes of a row
            const int rt = pos - tile_pos(it);
            unsigned char * b = s_tile[it % LK_DEC_NBUF] + w * 128 + 16 * g;
            *(lk_h8 *) (b + rt * LK_DEC_ROWB) = kv_h[0];
            *(lk_h8 *) (b + rt * LK_DEC_ROWB + 64) = kv_h[1];
            *(lk_h8 *) (b + (LK_DEC_TILE + rt) * LK_DEC_ROWB) = kv_h[2];
            *(lk_h8 *) (b + (LK_DEC_TILE + rt) * LK_DEC_ROWB + 64) = kv_h[3];
        }
        consume(s_tile[it % LK_DEC_NBUF], it);
    }
    // every tile DMA has landed before the workgroup ends (an empty slice
    // issued its first D tiles and never waited for them; for the others the
    // last wait_tile already waited for all)
    lk_wait_vm<0>();

    // Partial record of query head 4w + c, written by the lanes of columns
    // c = 0..3: O^T rows 16db + 4g + r; the sum of p is in every row of accl.
    if (col < 4) {
        const int h = w * LK_G + col;
#pragma unroll
        for (int db = 0; db < 4; ++db)          // dims 16db + 4g .. +3 of chunk db
            *(lk_f4 *) (part + lk_part_acc(h, db, sp) + 4 * g) = acc[db];
        if (g == 0) *(float2 *) (part + lk_part_ml(h, sp)) = make_float2(mrun, accl[0]);
    }
}

// Q8_1 quantisation of the 64 outputs of one head held by one wave, one value
// per lane, two 32-lane blocks (reference quant.cuh:106-121): exact max, a
// fixed xor butterfly 16,8,4,2,1 for the raw sum (lk_bfly32_sum), d = amax/127 (IEEE
// division), q = roundf(x/d), (d, sum) stored as fp16 RNE.
__device__ __forceinline__ void lk_quant_q8_1_wave(float x, lk_block_q8_1 * __restrict__ yq8) {
    const int lane = threadIdx.x & 63;
    const float am = lk_bfly32_max(fabsf(x)), sum = lk_bfly32_sum(x);
    const float d = am / 127.0f;
    const int8_t qv = (am == 0.0f) ? (int8_t) 0 : (int8_t) roundf(x / d);
    lk_block_q8_1 * b = yq8 + (lane >> 5);
    b->qs[lane & 31] = qv;
    if ((lane & 31) == 0) {
        const _Float16 dh = (_Float16) d, sh = (_Float16) sum;
        b->d = __builtin_bit_cast(uint16_t, dh);
        b->s = __builtin_bit_cast(uint16_t, sh);
    }
}

// The same quantiser for one 32-value block held by lanes 0..31 of a wave
// (lanes 32..63 hold a copy and write nothing).
__device__ __forceinline__ void lk_quant_q8_1_half(float x, lk_block_q8_1 * __restrict__ b) {
    const int lane = threadIdx.x & 63;
    const float am = lk_bfly32_max(fabsf(x)), sum = lk_bfly32_sum(x);
    const float d = am / 127.0f;
    const int8_t qv = (am == 0.0f) ? (int8_t) 0 : (int8_t) roundf(x / d);
    if (lane < 32) b->qs[lane] = qv;
    if (lane == 0) {
        const _Float16 dh = (_Float16) d, sh = (_Float16) sum;
        b->d = __builtin_bit_cast(uint16_t, dh);
        b->s = __builtin_bit_cast(uint16_t, sh);
    }
}


// Combine: grid (32 query heads, 2 halves of the 64 dims), 256 threads;
// workgroup (head, half) produces 32 output dims, wave w owns dims
// 32*half + 8w .. +7 over all slots, lane l the slots l, l+64, l+128, l+192.
// Slices that hold no tile (the reference's empty slices, kernels.cu:1573-1584,
// hold no tokens either) wrote the neutral record (m = -inf, l = 0, acc = 0), whose
// weight 2^(-inf - M) is exactly 0, so every slot is merged and d_pos is not
// read: all of a lane's loads go out at once, one memory round trip.  The max
// M is exact, the slot weights are 2^(m_s - M).  Every sum runs in a fixed
// order (per lane in slot order, then a fixed lane tree), so the output is
// run-to-run bit-identical.  Each half is exactly one Q8_1 block of the next
// GEMV's input.
static_assert(LK_ATTN_SPLIT <= 256 && LK_ATTN_SPLIT % 64 == 0, "combine: 1-4 whole slots per lane");
static_assert(lk_part_ml(LK_N_HEADS - 1, LK_ATTN_SPLIT - 1) + 2 <= (size_t) LK_N_HEADS * LK_ATTN_SPLIT * LK_ATTN_PARTW &&
              lk_part_acc(LK_N_HEADS - 1, 3, LK_ATTN_SPLIT - 1) + 16 <= lk_part_ml(0, 0),
              "the partial layout fits lk_attn_part_bytes() and its planes do not overlap");
__global__ void __launch_bounds__(256)
lk_k_attn_combine(const float * __restrict__ part, const int * __restrict__ d_pos,
                  float * __restrict__ out, lk_block_q8_1 * __restrict__ yq8, int * __restrict__ advance) {
    (void) d_pos;
    // the decode step's position advance (reference kernels.cu:994), folded
    // into the step's last combine: nothing in this kernel reads the position
    if (advance && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *advance = *advance + 1;
    constexpr int J = LK_ATTN_SPLIT / 64;
    const int head = blockIdx.x, half = blockIdx.y;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int d0 = 32 * half + 8 * wv;

    // (m, l) as a float2 from its own plane (a 16-byte load with dead lanes let
    // the register allocator reuse them while the load was in flight)
    float2 ml[J];
    lk_f4 a0[J], a1[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int s = lane + 64 * j;
        const float * R = part + lk_part_acc(head, 2 * half + (wv >> 1), s) + 8 * (wv & 1);
        ml[j] = *(const float2 *) (part + lk_part_ml(head, s));
        a0[j] = *(const lk_f4 *) R;
        a1[j] = *(const lk_f4 *) (R + 4);
    }
    float M = ml[0].x;
#pragma unroll
    for (int j = 1; j < J; ++j) M = fmaxf(M, ml[j].x);
    M = lk_xrow_max(lk_row_max16(M));                // finite: slice 0 always holds tokens
    float L = 0.0f;
    lk_f4 A0 = { 0.f, 0.f, 0.f, 0.f }, A1 = A0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float e = lk_exp2(ml[j].x - M);        // neutral records: exactly 0
        L += ml[j].y * e;
        A0 += a0[j] * e;
        A1 += a1[j] * e;
    }
    L = lk_xrow_sum(lk_row_sum16(L));
    float o[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[k]     = lk_xrow_sum(lk_row_sum16(A0[k]));
        o[4 + k] = lk_xrow_sum(lk_row_sum16(A1[k]));
    }
    const float il = 1.0f / L;
    __shared__ float s_o[32];
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            o[k] *= il;
            s_o[8 * wv + k] = o[k];
        }
        if (out) {
            *(lk_f4 *) (out + head * LK_HEAD_DIM + d0)     = (lk_f4){ o[0], o[1], o[2], o[3] };
            *(lk_f4 *) (out + head * LK_HEAD_DIM + d0 + 4) = (lk_f4){ o[4], o[5], o[6], o[7] };
        }
    }
    if (!yq8) return;                                 // workgroup-uniform
    __syncthreads();
    if (wv == 0) lk_quant_q8_1_half(s_o[lane & 31], yq8 + 2 * head + half);
}

// Serial cross-check (reference kernels.cu:768-852): one workgroup per query
// head keeps the whole score row in LDS, so it serves seq <= 8192 only and
// writes nothing beyond that.
__global__ void __launch_bounds__(256)
lk_k_attention_decode(const float * __restrict__ q, const _Float16 * __restrict__ kc,
                      const _Float16 * __restrict__ vc, const int * __restrict__ d_pos,
                      float * __restrict__ out, lk_block_q8_1 * __restrict__ yq8) {
    const int seq = *d_pos + 1;
    if (seq > LK_ATTN_DECODE_MAX_SEQ) return;
    const int head = blockIdx.x, kvh = head / LK_G;
    __shared__ float s_q[LK_HEAD_DIM];
    __shared__ float s_s[LK_ATTN_DECODE_MAX_SEQ];
    __shared__ float s_red[256];
    if (threadIdx.x < LK_HEAD_DIM) s_q[threadIdx.x] = q[head * LK_HEAD_DIM + threadIdx.x];
    __syncthreads();
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < seq; t += 256) {
        const _Float16 * k = kc + (size_t) t * LK_KV_ROW + kvh * LK_HEAD_DIM;
        float a = 0.0f;
        for (int d = 0; d < LK_HEAD_DIM; ++d) a += s_q[d] * (float) k[d];
        a *= 0.125f * LK_LOG2E_F;
        s_s[t] = a;
        mx = fmaxf(mx, a);
    }
    s_red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int) threadIdx.x < o) s_red[threadIdx.x] = fmaxf(s_red[threadIdx.x], s_red[threadIdx.x + o]);
        __syncthreads();
    }
    const float M = s_red[0];
    __syncthreads();
    float l = 0.0f;
    for (int t = threadIdx.x; t < seq; t += 256) {
        const float p = lk_exp2(s_s[t] - M);
        s_s[t] = p;
        l += p;
    }
    s_red[threadIdx.x] = l;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int) threadIdx.x < o) s_red[threadIdx.x] += s_red[threadIdx.x + o];
        __syncthreads();
    }
    const float inv = 1.0f / s_red[0];
    if (threadIdx.x < LK_HEAD_DIM) {
        const int d = threadIdx.x;
        float a = 0.0f;
        for (int t = 0; t < seq; ++t)
            a += s_s[t] * (float) vc[(size_t) t * LK_KV_ROW + kvh * LK_HEAD_DIM + d];
        const float o = a * inv;
        if (out) out[head * LK_HEAD_DIM + d] = o;
        if (yq8) lk_quant_q8_1_wave(o, yq8 + 2 * head);
    }
}

// ---------------------------------------------------------------------------
// C ABI
static int lk_split_launch(const float * q, const void * kc, const void * vc,
                           const int * d_pos, float * part, hipStream_t st) {
    hipLaunchKernelGGL(lk_k_attn_split<false>, dim3(LK_ATTN_SPLIT), dim3(LK_DEC_THREADS), 0, st,
                       q, (const _Float16 *) kc, (const _Float16 *) vc, d_pos, part, LkDecProducer{});
    return lk_launch_status("lk_attn_split");
}
// The step graph's attention node: the split kernel with the producer folded in.
static int lk_split_fused_launch(const lk_decode_layer & L, const int * d_pos, float * part, hipStream_t st) {
    const LkDecProducer pr{ L.q_src, L.k_src, L.v_src, L.q_norm, L.k_norm, L.q, L.k };
    hipLaunchKernelGGL(lk_k_attn_split<true>, dim3(LK_ATTN_SPLIT), dim3(LK_DEC_THREADS), 0, st,
                       (const float *) nullptr, (const _Float16 *) L.kc, (const _Float16 *) L.vc, d_pos, part, pr);
    return lk_launch_status("lk_decode_step_graph (split with producer)");
}
static int lk_combine_launch(const float * part, const int * d_pos, float * out,
                             lk_block_q8_1 * yq8, hipStream_t st, int * advance = nullptr) {
    hipLaunchKernelGGL(lk_k_attn_combine, dim3(LK_N_HEADS, 2), dim3(256), 0, st, part, d_pos, out, yq8, advance);
    return lk_launch_status("lk_attn_combine");
}

// The split kernel reads q with 16-byte loads (lk_ld16_untracked).
static bool lk_q_misaligned(const float * q) { return ((uintptr_t) q & 15u) != 0; }

extern "C" int lk_attn_split(const float * q, const void * kc, const void * vc,
                             const int * d_pos, float * part, void * stream) {
    if (!q || !kc || !vc || !d_pos || !part)
        return lk_fail(hipErrorInvalidValue, "lk_attn_split: null pointer argument");
    if (lk_q_misaligned(q))
        return lk_fail(hipErrorInvalidValue, "lk_attn_split: q must be 16-byte aligned");
    return lk_split_launch(q, kc, vc, d_pos, part, lk_stream(stream));
}

extern "C" int lk_attn_combine(const float * part, const int * d_pos, float * out,
                               lk_block_q8_1 * yq8, void * stream) {
    if (!part || !d_pos)
        return lk_fail(hipErrorInvalidValue, "lk_attn_combine: null pointer argument");
    return lk_combine_launch(part, d_pos, out, yq8, lk_stream(stream));
}

extern "C" int lk_attn_decode(const float * q, const void * kc, const void * vc,
                              const int * d_pos, float * part, float * out,
                              lk_block_q8_1 * yq8, void * stream) {
    int e = lk_attn_split(q, kc, vc, d_pos, part, stream);
    if (e) return e;
    return lk_attn_combine(part, d_pos, out, yq8, stream);
}

// ---- allocation-free decode ------------------------------------------------
// lk_attn_decode_noalloc keeps the slice partials in this file-scope device
// array instead of a caller buffer.  Its size is fixed: one record per (query
// head, slot), LK_N_HEADS x LK_ATTN_SPLIT x LK_ATTN_PARTW floats (2.2 MB), the
// most any sequence length uses (the slice count is capped at LK_ATTN_SPLIT).
// Each device holds its own copy until the process ends.  In host code the
// name `scratch` is a host-side stand-in, never a device address: the device
// address is looked up once per device with hipGetSymbolAddress and only that
// pointer is passed to kernels.
#define LK_DEC_SCRATCH_FLOATS ((size_t) LK_N_HEADS * LK_ATTN_SPLIT * LK_ATTN_PARTW)
static __device__ __align__(256) float scratch[LK_DEC_SCRATCH_FLOATS];

// Per device: the array's device address, and the guard of its single-stream
// use -- the stream of the last call and an event recorded after its combine.
// A call from another stream while that event is pending would overwrite
// partials the earlier call has not merged yet; it is refused
// (hipErrorNotReady) instead.  Calls on one stream are ordered and always
// accepted.  Under stream capture nothing is checked or recorded (the graph's
// own order decides).  Address and event are set up on a device's first call.
// A call holds g_dec_mu from the check to the record, so that two host
// threads cannot both pass the check before either has recorded.
struct LkDecScratchUse {
    float * ptr = nullptr;
    hipStream_t last = nullptr;
    hipEvent_t done = nullptr;
    bool pending = false;
};
static std::mutex g_dec_mu;
static LkDecScratchUse g_dec_use[LK_MAX_DEVICES];

static bool lk_capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void) hipStreamIsCapturing(st, &cs);
    return cs != hipStreamCaptureStatusNone;
}

// Called with g_dec_mu held.
static float * lk_dec_scratch_acquire(hipStream_t st, int & err, int & dev_out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= LK_MAX_DEVICES) {
        err = lk_fail(e != hipSuccess ? (int) e : (int) hipErrorInvalidDevice,
                      "lk_attn_decode_noalloc: no usable current device");
        return nullptr;
    }
    LkDecScratchUse & u = g_dec_use[dev];
    if (!u.ptr) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            err = lk_fail(e != hipSuccess ? (int) e : (int) hipErrorInvalidSymbol,
                          "lk_attn_decode_noalloc: scratch lookup on device %d: %s", dev, hipGetErrorString(e));
            return nullptr;
        }
        e = hipEventCreateWithFlags(&u.done, hipEventDisableTiming);
        if (e != hipSuccess) {
            err = lk_fail((int) e, "lk_attn_decode_noalloc: guard event: %s", hipGetErrorString(e));
            return nullptr;
        }
        u.ptr = (float *) p;
    }
    if (!lk_capturing(st) && u.pending && u.last != st) {
        e = hipEventQuery(u.done);
        (void) hipGetLastError();                     // the query's status is not a launch error
        if (e == hipErrorNotReady) {
            err = lk_fail(hipErrorNotReady,
                          "lk_attn_decode_noalloc: a call on another stream of device %d is still pending; "
                          "calls share one partial array per device: order them on one stream "
                          "(or wait for the earlier one)", dev);
            return nullptr;
        }
    }
    err = 0;
    dev_out = dev;
    return u.ptr;
}

// After the combine is enqueued on st: mark the array busy until it completes.
// Called with g_dec_mu held.
static int lk_dec_scratch_release(hipStream_t st, int dev) {
    if (lk_capturing(st)) return 0;
    LkDecScratchUse & u = g_dec_use[dev];
    const hipError_t e = hipEventRecord(u.done, st);
    if (e != hipSuccess) return lk_fail((int) e, "lk_attn_decode_noalloc: guard record: %s", hipGetErrorString(e));
    u.last = st;
    u.pending = true;
    return 0;
}

extern "C" int lk_attn_decode_noalloc(const float * q, const void * kc, const void * vc,
                                      const int * d_pos, float * out, lk_block_q8_1 * yq8,
                                      void * stream) {
    static_assert(LK_DEC_SCRATCH_FLOATS * sizeof(float) >= (size_t) LK_N_HEADS * LK_ATTN_SPLIT * LK_ATTN_PARTW * sizeof(float),
                  "scratch holds one full partial set");
    if (!q || !kc || !vc || !d_pos)
        return lk_fail(hipErrorInvalidValue, "lk_attn_decode_noalloc: null pointer argument");
    if (lk_q_misaligned(q))
        return lk_fail(hipErrorInvalidValue, "lk_attn_decode_noalloc: q must be 16-byte aligned");
    hipStream_t st = lk_stream(stream);
    std::lock_guard<std::mutex> lock(g_dec_mu);
    int err = 0, dev = 0;
    float * part = lk_dec_scratch_acquire(st, err, dev);
    if (!part) return err;
    int rc = lk_split_launch(q, kc, vc, d_pos, part, st);
    if (rc) return rc;
    rc = lk_combine_launch(part, d_pos, out, yq8, st);
    if (rc) return rc;
    return lk_dec_scratch_release(st, dev);
}

extern "C" int lk_attention_decode(const float * q, const void * kc, const void * vc,
                                   const int * d_pos, float * out, lk_block_q8_1 * yq8,
                                   void * stream) {
    if (!q || !kc || !vc || !d_pos)
        return lk_fail(hipErrorInvalidValue, "lk_attention_decode: null pointer argument");
    hipLaunchKernelGGL(lk_k_attention_decode, dim3(LK_N_HEADS), dim3(256), 0, lk_stream(stream),
                       q, (const _Float16 *) kc, (const _Float16 *) vc, d_pos, out, yq8);
    return lk_launch_status("lk_attention_decode");
}

// ---------------------------------------------------------------------------
// Decode graph: n_layers x (split, combine) captured once on the caller's
// stream (reference engine.cu:1333-1343 captures the whole step the same way,
// thread-local capture mode).  Only kernel nodes are recorded.
struct lk_decode_graph {
    hipGraph_t     graph = nullptr;
    hipGraphExec_t exec = nullptr;
    size_t         nodes = 0;
};

extern "C" int lk_decode_graph_create(int n_layers, const float * const * q,
                                      const void * const * kc, const void * const * vc,
                                      const int * d_pos, float * part,
                                      float * const * out, lk_block_q8_1 * const * yq8,
                                      void * stream, lk_decode_graph ** graph) {
    if (!graph) return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: graph is null");
    *graph = nullptr;
    if (n_layers <= 0 || !q || !kc || !vc || !d_pos || !part)
        return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: bad arguments");
    if (!stream)
        return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: capture needs a non-default stream");
    for (int i = 0; i < n_layers; ++i) {
        if (!q[i] || !kc[i] || !vc[i])
            return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: null pointer for layer %d", i);
        if (lk_q_misaligned(q[i]))
            return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: q of layer %d must be 16-byte aligned", i);
    }
    hipStream_t st = lk_stream(stream);
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return lk_fail((int) e, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    int rc = 0;
    for (int i = 0; i < n_layers && !rc; ++i) {
        rc = lk_split_launch(q[i], kc[i], vc[i], d_pos, part, st);
        if (!rc) rc = lk_combine_launch(part, d_pos, out ? out[i] : nullptr, yq8 ? yq8[i] : nullptr, st);
    }
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(st, &g);
    if (rc) { if (g) (void) hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return lk_fail((int) e, "hipStreamEndCapture: %s", hipGetErrorString(e));
    lk_decode_graph * G = new lk_decode_graph;
    G->graph = g;
    e = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void) hipGraphDestroy(g);
        delete G;
        return lk_fail((int) e, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    (void) hipGraphGetNodes(g, nullptr, &G->nodes);
    *graph = G;
    return 0;
}

extern "C" int lk_decode_step_graph_create(int n_layers, const lk_decode_layer * layers, int * d_pos,
                                           float * part, void * stream, lk_decode_graph ** graph) {
    if (!graph) return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: graph is null");
    *graph = nullptr;
    if (n_layers <= 0 || !layers || !d_pos || !part)
        return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: bad arguments");
    if (!stream)
        return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: capture needs a non-default stream");
    for (int i = 0; i < n_layers; ++i) {
        const lk_decode_layer & L = layers[i];
        if (!L.q_src || !L.k_src || !L.v_src || !L.q || !L.k || !L.q_norm || !L.k_norm || !L.kc || !L.vc)
            return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: null pointer for layer %d", i);
        if (lk_q_misaligned(L.q_src) || lk_q_misaligned(L.k_src) || lk_q_misaligned(L.v_src)
            || lk_q_misaligned(L.q_norm) || lk_q_misaligned(L.k_norm))
            return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: layer %d: q_src, k_src, v_src, "
                           "q_norm and k_norm must be 16-byte aligned (16-byte loads)", i);
        if (L.wo_qs && (!L.wo_d || !L.x || !L.yq8))
            return lk_fail(hipErrorInvalidValue, "lk_decode_step_graph_create: layer %d: the output projection needs wo_d, x and yq8", i);
    }
    hipStream_t st = lk_stream(stream);
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return lk_fail((int) e, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    int rc = 0;
    for (int i = 0; i < n_layers && !rc; ++i) {
        const lk_decode_layer & L = layers[i];
        // the producer (norm + RoPE of q and k, the cache append, the working
        // q / k rows) runs inside the split kernel: two nodes per layer
        rc = lk_split_fused_launch(L, d_pos, part, st);
        // the last layer's combine also advances *d_pos
        if (!rc) rc = lk_combine_launch(part, d_pos, L.out, L.yq8, st, i == n_layers - 1 ? d_pos : nullptr);
        // optional: the attention output projection into the residual stream
        if (!rc && L.wo_qs)
            rc = lk_gemv_q4_0(L.wo_qs, L.wo_d, L.yq8, LK_HIDDEN, LK_HIDDEN / 32, L.x, 1, nullptr, 0.0f, st);
    }
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(st, &g);
    if (rc) { if (g) (void) hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return lk_fail((int) e, "hipStreamEndCapture: %s", hipGetErrorString(e));
    lk_decode_graph * G = new lk_decode_graph;
    G->graph = g;
    e = hipGraphInstantiate(&G->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void) hipGraphDestroy(g);
        delete G;
        return lk_fail((int) e, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    (void) hipGraphGetNodes(g, nullptr, &G->nodes);
    *graph = G;
    return 0;
}

extern "C" int lk_decode_graph_run(lk_decode_graph * graph, int n_steps, void * stream) {
    if (!graph || !graph->exec || n_steps < 0)
        return lk_fail(hipErrorInvalidValue, "lk_decode_graph_run: bad arguments");
    for (int i = 0; i < n_steps; ++i) {
        const hipError_t e = hipGraphLaunch(graph->exec, lk_stream(stream));
        if (e != hipSuccess) return lk_fail((int) e, "hipGraphLaunch (step %d): %s", i, hipGetErrorString(e));
    }
    return 0;
}

extern "C" int lk_decode_graph_launch(lk_decode_graph * graph, void * stream) {
    if (!graph || !graph->exec) return lk_fail(hipErrorInvalidValue, "lk_decode_graph_launch: no graph");
    const hipError_t e = hipGraphLaunch(graph->exec, lk_stream(stream));
    if (e != hipSuccess) return lk_fail((int) e, "hipGraphLaunch: %s", hipGetErrorString(e));
    return 0;
}

extern "C" int lk_decode_graph_nodes(const lk_decode_graph * graph, size_t * n_nodes) {
    if (!graph || !n_nodes) return lk_fail(hipErrorInvalidValue, "lk_decode_graph_nodes: bad arguments");
    *n_nodes = graph->nodes;
    return 0;
}

extern "C" int lk_decode_graph_destroy(lk_decode_graph * graph) {
    if (!graph) return 0;
    if (graph->exec) (void) hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void) hipGraphDestroy(graph->graph);
    delete graph;
    return 0;
}
