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
//   * grid (8 kv heads x LK_ATTN_SPLIT slices) of 4-wave workgroups; a
//     workgroup streams its kv head's K and V slice exactly once for the four
//     query heads sharing it (algorithmic traffic: seq x 2 KB per layer);
//   * each wave takes 16-token groups; lane l loads 32 contiguous bytes
//     (dims 16g..16g+15 of token l%16, g = l/16) of K and of V with two
//     128-bit loads, LK_ATTN_UNROLL groups in flight before any is consumed;
//   * Q.K^T runs on the matrix cores: v_mfma_f32_16x16x32_f16 with the four
//     heads' q replicated over the 16 A rows, so every lane receives the four
//     heads' scores of its own token.  q is fp32 in the interface, so it is
//     split q = hi + lo into two fp16 halves (22 significant bits) and both
//     halves are multiplied (fp16 x fp16 products are exact in fp32);
//   * online softmax in the log2 domain per wave (v_exp_f32), P.V on the VALU
//     in fp32 (fma with fp16 V operands), then a fixed butterfly over the 16
//     token lanes and a fixed wave order in LDS -> one partial (m, l, acc[64])
//     per (query head, slice);
//   * the combine merges the slice partials in a fixed order (deterministic,
//     run-to-run bit-identical) and optionally emits Q8_1 blocks.
#include "lk_common.h"
#include <math.h>

// fp32 -> (hi, lo) fp16 pair with hi + lo == x to 22 bits.  x - (float)hi is
// exact in fp32 (hi is x rounded to 11 significant bits).
__device__ __forceinline__ void lk_split_h(float x, _Float16 & hi, _Float16 & lo) {
    hi = (_Float16) x;
    lo = (_Float16) (x - (float) hi);
}

template <int U>
__global__ void __launch_bounds__(256)
lk_k_attn_split(const float * __restrict__ q, const _Float16 * __restrict__ kc,
                const _Float16 * __restrict__ vc, const int * __restrict__ d_pos,
                float * __restrict__ part) {
    const int seq = *d_pos + 1;
    int ns, chunk;
    lk_attn_slices(seq, ns, chunk);
    const int kvh = blockIdx.x, sp = blockIdx.y;
    const int t0 = sp * chunk;
    const int t1 = (t0 + chunk < seq) ? (t0 + chunk) : seq;
    // Block-uniform early out before any barrier: dead slices write nothing
    // (the combine derives the same boundary and never reads them).
    if (t0 >= t1) return;
    const int n = t1 - t0;

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = lane & 15, g = lane >> 4;

    // A operand: row i = col carries query head kvh*4 + (i & 3); k-slots 8g..8g+7
    // of MFMA 0 are dims 16g..16g+7, of MFMA 1 dims 16g+8..16g+15 -- the same
    // dims this lane loads of its token, so A and B agree slot by slot.
    lk_h8 qa0h, qa0l, qa1h, qa1l;
    {
        const float * qp = q + (kvh * LK_G + (col & 3)) * LK_HEAD_DIM + 16 * g;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            _Float16 h, l;
            lk_split_h(qp[i], h, l);     qa0h[i] = h; qa0l[i] = l;
            lk_split_h(qp[8 + i], h, l); qa1h[i] = h; qa1l[i] = l;
        }
    }
    const float SC = 0.125f * LK_LOG2E_F;      // scores in log2 units

    float mrun[4], lrun[4], acc[4][16];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        mrun[r] = -1e30f; lrun[r] = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[r][k] = 0.0f;
    }

    const size_t lane_off = (size_t) kvh * LK_HEAD_DIM + 16 * g;
    const _Float16 * kb = kc + (size_t) t0 * LK_KV_ROW + lane_off;
    const _Float16 * vb = vc + (size_t) t0 * LK_KV_ROW + lane_off;

    for (int j0 = 16 * w; j0 < n; j0 += 64 * U) {
        lk_h8 k0[U], k1[U], v0[U], v1[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + 64 * u + col;
            ok[u] = j < n;
            // dead lanes read token t0 (always in range) and are masked below
            const size_t o = (size_t) (ok[u] ? j : 0) * LK_KV_ROW;
            k0[u] = *(const lk_h8 *) (kb + o);
            k1[u] = *(const lk_h8 *) (kb + o + 8);
            v0[u] = *(const lk_h8 *) (vb + o);
            v1[u] = *(const lk_h8 *) (vb + o + 8);
        }
        float s[U][4];
        float mloc[4] = { -INFINITY, -INFINITY, -INFINITY, -INFINITY };
#pragma unroll
        for (int u = 0; u < U; ++u) {
            lk_f4 c = { 0.0f, 0.0f, 0.0f, 0.0f };
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa0h, k0[u], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa0l, k0[u], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa1h, k1[u], c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa1l, k1[u], c, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[u][r] = ok[u] ? c[r] * SC : -INFINITY;
                mloc[r] = fmaxf(mloc[r], s[u][r]);
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) mloc[r] = fmaxf(mloc[r], __shfl_xor(mloc[r], o, 64));
            const float mnew = fmaxf(mrun[r], mloc[r]);
            const float alpha = lk_exp2(mrun[r] - mnew);
            mrun[r] = mnew;
            lrun[r] *= alpha;
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[r][k] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = lk_exp2(s[u][r] - mrun[r]);
                lrun[r] += p;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    acc[r][k]     += p * (float) v0[u][k];
                    acc[r][8 + k] += p * (float) v1[u][k];
                }
            }
        }
    }

    // Sum the 16 token lanes of each row group (fixed butterfly): afterwards
    // every lane of row group g holds l and acc for dims 16g..16g+15.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            lrun[r] += __shfl_xor(lrun[r], o, 64);
#pragma unroll
            for (int k = 0; k < 16; ++k) acc[r][k] += __shfl_xor(acc[r][k], o, 64);
        }
    }

    __shared__ float s_m[4][4], s_l[4][4];
    __shared__ float s_acc[4][4][LK_HEAD_DIM];
    if (col == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < 16; ++k) s_acc[w][r][16 * g + k] = acc[r][k];
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) { s_m[w][r] = mrun[r]; s_l[w][r] = lrun[r]; }
    }
    __syncthreads();
    {
        // thread -> (head r, dim d); waves merged in the fixed order 0,1,2,3.
        // A wave that owned no tokens holds m = -1e30, l = 0: weight 0.
        const int r = threadIdx.x >> 6, d = threadIdx.x & 63;
        float M = s_m[0][r];
#pragma unroll
        for (int ww = 1; ww < 4; ++ww) M = fmaxf(M, s_m[ww][r]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const float e = lk_exp2(s_m[ww][r] - M);
            L += s_l[ww][r] * e;
            A += s_acc[ww][r][d] * e;
        }
        float * P = part + ((size_t) (kvh * LK_G + r) * LK_ATTN_SPLIT + sp) * LK_ATTN_PARTW;
        if (d == 0) { P[0] = M; P[1] = L; }
        P[2 + d] = A;
    }
}

// Q8_1 quantisation of the 64 outputs of one head held by one wave, one value
// per lane, two 32-lane blocks (reference quant.cuh:106-121): exact max, a
// fixed xor butterfly 16,8,4,2,1 for the raw sum, d = amax/127 (IEEE
// division), q = roundf(x/d), (d, sum) stored as fp16 RNE.
__device__ __forceinline__ void lk_quant_q8_1_wave(float x, lk_block_q8_1 * __restrict__ yq8) {
    const int lane = threadIdx.x & 63;
    float am = fabsf(x), sum = x;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        am = fmaxf(am, __shfl_xor(am, o, 32));
        sum += __shfl_xor(sum, o, 32);
    }
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

// One workgroup per query head, 256 threads.  Slices s with s*chunk >= seq hold
// no tokens and are skipped (reference kernels.cu:1573-1584).  Slice weights
// are 2^(m_s - M); thread group j (64 lanes, one per dim) folds the j-th
// contiguous quarter of the slices serially, and the four quarter sums are
// added in the order 0,1,2,3: a fixed order, so output is bit-reproducible.
__global__ void __launch_bounds__(256)
lk_k_attn_combine(const float * __restrict__ part, const int * __restrict__ d_pos,
                  float * __restrict__ out, lk_block_q8_1 * __restrict__ yq8) {
    const int head = blockIdx.x;
    const int seq = *d_pos + 1;
    int ns, chunk;
    lk_attn_slices(seq, ns, chunk);
    const int nv = (seq + chunk - 1) / chunk;        // non-empty slices, <= ns
    const float * P = part + (size_t) head * LK_ATTN_SPLIT * LK_ATTN_PARTW;

    __shared__ float s_red[256];
    float mx = -1e30f;
    for (int s = threadIdx.x; s < nv; s += 256) mx = fmaxf(mx, P[(size_t) s * LK_ATTN_PARTW]);
    s_red[threadIdx.x] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if ((int) threadIdx.x < o) s_red[threadIdx.x] = fmaxf(s_red[threadIdx.x], s_red[threadIdx.x + o]);
        __syncthreads();
    }
    const float M = s_red[0];

    const int d = threadIdx.x & 63, j = threadIdx.x >> 6;
    const int q4 = (nv + 3) >> 2;
    const int sb = j * q4, se = (sb + q4 < nv) ? sb + q4 : nv;
    float L = 0.0f, A = 0.0f;
    for (int s = sb; s < se; ++s) {
        const float * ps = P + (size_t) s * LK_ATTN_PARTW;
        const float e = lk_exp2(ps[0] - M);
        L += ps[1] * e;
        A += ps[2 + d] * e;
    }
    __shared__ float s_a[4][64], s_l[4];
    s_a[j][d] = A;
    if (d == 0) s_l[j] = L;
    __syncthreads();
    if (j == 0) {
        const float Af = ((s_a[0][d] + s_a[1][d]) + s_a[2][d]) + s_a[3][d];
        const float Lf = ((s_l[0] + s_l[1]) + s_l[2]) + s_l[3];
        const float o = Af * (1.0f / Lf);
        if (out) out[head * LK_HEAD_DIM + d] = o;
        if (yq8) lk_quant_q8_1_wave(o, yq8 + 2 * head);
    }
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
    hipLaunchKernelGGL(lk_k_attn_split<LK_ATTN_UNROLL>, dim3(LK_N_KV_HEADS, LK_ATTN_SPLIT),
                       dim3(256), 0, st, q, (const _Float16 *) kc, (const _Float16 *) vc,
                       d_pos, part);
    return lk_launch_status("lk_attn_split");
}
static int lk_combine_launch(const float * part, const int * d_pos, float * out,
                             lk_block_q8_1 * yq8, hipStream_t st) {
    hipLaunchKernelGGL(lk_k_attn_combine, dim3(LK_N_HEADS), dim3(256), 0, st, part, d_pos, out, yq8);
    return lk_launch_status("lk_attn_combine");
}

extern "C" int lk_attn_split(const float * q, const void * kc, const void * vc,
                             const int * d_pos, float * part, void * stream) {
    if (!q || !kc || !vc || !d_pos || !part)
        return lk_fail(hipErrorInvalidValue, "lk_attn_split: null pointer argument");
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
    for (int i = 0; i < n_layers; ++i)
        if (!q[i] || !kc[i] || !vc[i])
            return lk_fail(hipErrorInvalidValue, "lk_decode_graph_create: null pointer for layer %d", i);
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
