/*
 * lk_attn.h - C ABI of the MI355X (gfx950) attention hot path of the
 * lfm2-ampere engine: split-K GQA decode attention over the fp16 KV cache with
 * a deterministic two-stage combine, and chunked causal prefill attention with
 * int8 Q.K^T scoring, exact fp16 tiles at the diagonal window and the sink,
 * online softmax and fp16 P.V.
 *
 * Conventions (the reference engine's, /root/reference/src/engine.cu:21-22,
 * 397-409, 974-985):
 *   - every buffer is caller-owned DEVICE memory; no entry point allocates,
 *     frees or synchronises.  Each one only enqueues work on `stream`
 *     (a hipStream_t passed as void*; NULL = the default stream);
 *   - the decode sequence length is read ON THE DEVICE from d_pos
 *     (seq = *d_pos + 1) and the grids are fixed, so the decode launches are
 *     position-independent and may be captured into a hipGraph;
 *   - every entry point returns 0 (hipSuccess) or a hipError_t code; argument
 *     errors the host can see return hipErrorInvalidValue (1) and launch
 *     nothing.  lk_last_error() describes the last failure in words.
 *
 * Model constants (reference kernels.cuh:12-24): 32 query heads, 8 KV heads
 * (GQA 4:1), head_dim 64, softmax scale 1/8.  The KV cache of one layer is
 * fp16 [max_seq][8][64].
 */
#ifndef LK_ATTN_H
#define LK_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LK_N_HEADS      32
#define LK_N_KV_HEADS   8
#define LK_HEAD_DIM     64
/* fp32 words per (query head, slot) of the decode partial buffer: it only sizes
 * that buffer (lk_attn_part_bytes); the layout inside is private to the
 * library (an acc plane and an (m, l) plane, not one record per slot). */
#define LK_ATTN_PARTW   (4 + LK_HEAD_DIM)

/* Q8_1 activation block (reference quant.cuh:27-31): fp16 d = amax/127 and
 * fp16 raw sum of the 32 values, then the 32 int8 quants.  36 bytes. */
typedef struct lk_block_q8_1 {
    uint16_t d;      /* fp16 bits */
    uint16_t s;      /* fp16 bits */
    int8_t   qs[32];
} lk_block_q8_1;

/* ---- build-time configuration ------------------------------------------- */

/* The split-K operating point this library was built with: the slice count is
 * clamp(ceil(seq / target_n), split_min, split_cap)
 * (reference kernels.cuh:630-635, retuned for 256 CUs). */
int lk_attn_config(int * split_cap, int * target_n, int * split_min);

/* Bytes the caller must allocate for `part` (32 x split_cap x 68 fp32; the
 * layout inside is the library's own).
 * Replaces the engine's own sizing at reference engine.cu:408-409. */
size_t lk_attn_part_bytes(void);

/* Human-readable description of the last error returned on this thread. */
const char * lk_last_error(void);

/* ---- decode attention ----------------------------------------------------
 * q   : fp32 [32][64], post-RoPE
 * kc  : fp16 [max_seq][8][64] K cache of this layer
 * vc  : fp16 [max_seq][8][64] V cache of this layer
 * d_pos: int32, device; the kernels attend to positions [0, *d_pos]
 * part: fp32 scratch of lk_attn_part_bytes() bytes (slice partials)
 * out : fp32 [32][64] or NULL
 * yq8 : lk_block_q8_1 [64] (two blocks per head) or NULL
 */

/* Replaces k_attn_split (reference kernels.cuh:647-649, kernels.cu:1303-1556).
 * Grid (split_cap) of 8-wave workgroups, each over all 8 kv heads of one
 * slice: the slice count is the reference's rule (lk_attn_slices), and slice
 * s holds the 16-position tiles s, s + ns, s + 2ns, ... of [0, seq).
 * Workgroups whose slice holds no tile write the neutral record (m = -inf,
 * l = 0, acc = 0) of their slot, so every one of the split_cap slots of part
 * is valid afterwards. */
int lk_attn_split(const float * q, const void * kc, const void * vc,
                  const int * d_pos, float * part, void * stream);

/* Replaces k_attn_combine (reference kernels.cuh:650-652, kernels.cu:1558-1599).
 * All split_cap slots of part (as lk_attn_split leaves them) are merged in a
 * fixed order, so output is run-to-run bit-identical.  d_pos is not read (the
 * neutral records carry weight exactly 0); the argument keeps the reference's
 * signature. */
int lk_attn_combine(const float * part, const int * d_pos, float * out,
                    lk_block_q8_1 * yq8, void * stream);

/* lk_attn_split followed by lk_attn_combine: the two graph nodes the engine
 * launches per attention layer (reference engine.cu:638-641). */
int lk_attn_decode(const float * q, const void * kc, const void * vc,
                   const int * d_pos, float * part, float * out,
                   lk_block_q8_1 * yq8, void * stream);

/* Allocation-free lk_attn_decode.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory or take a workspace (code under
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * slice partials live in a static device array of the library, one per GPU,
 * of the fixed size lk_attn_part_bytes() (2.2 MB: one record per query head
 * and slot, the most any sequence length uses), held until the process ends;
 * nothing is allocated at call time.  Same kernels and bit-identical results
 * as lk_attn_decode.  Every call on a GPU shares that GPU's array, so calls
 * that overlap in time on one GPU (different streams or threads) race; calls
 * ordered on one stream do not. */
int lk_attn_decode_noalloc(const float * q, const void * kc, const void * vc,
                           const int * d_pos, float * out, lk_block_q8_1 * yq8,
                           void * stream);

/* Replaces k_attention_decode (reference kernels.cuh:653-658,
 * kernels.cu:768-852): one workgroup per query head, a cross-check only.
 * Like the reference it only serves seq <= 8192; for longer sequences it
 * writes nothing (the reference prints FATAL and returns). */
#define LK_ATTN_DECODE_MAX_SEQ 8192
int lk_attention_decode(const float * q, const void * kc, const void * vc,
                        const int * d_pos, float * out, lk_block_q8_1 * yq8,
                        void * stream);

/* ---- decode graph --------------------------------------------------------
 * The engine captures its whole decode step once and replays it
 * (reference engine.cu:1333-1343); these capture just the attention slice:
 * n_layers x (split, combine) on one stream, into one hipGraph.  The arrays
 * hold one pointer per layer; `part` is shared by all layers (the layers run
 * in stream order).  out[i] / yq8[i] may be NULL, and so may the arrays. */
typedef struct lk_decode_graph lk_decode_graph;
int lk_decode_graph_create(int n_layers, const float * const * q,
                           const void * const * kc, const void * const * vc,
                           const int * d_pos, float * part,
                           float * const * out, lk_block_q8_1 * const * yq8,
                           void * stream, lk_decode_graph ** graph);
int lk_decode_graph_launch(lk_decode_graph * graph, void * stream);
int lk_decode_graph_nodes(const lk_decode_graph * graph, size_t * n_nodes);
int lk_decode_graph_destroy(lk_decode_graph * graph);

/* ---- decode step graph -----------------------------------------------------
 * The engine captures its whole position-independent decode step once and
 * replays it, its last kernel advancing d_pos on the device (reference
 * engine.cu:1328-1342 capture, 1750-1760 replay loop, kernels.cu:994 advance).
 * This is that step's attention slice: per layer, the q/k norm + RoPE of the
 * q/k/v projection rows (q_src, k_src, v_src fp32, the projection GEMV's
 * output) into the working q / k buffers with K/V appended at row *d_pos of the
 * layer's cache (lk_qk_norm_rope's arithmetic, out of place), split and
 * combine; then *d_pos += 1.  The producer runs inside the split kernel (each
 * workgroup forms q itself; the one whose slice holds *d_pos appends K/V and
 * uses the new row directly), so a layer is two graph nodes (three with the
 * optional output projection below); the last layer's combine advances *d_pos.
 * Replaying it n times runs n decode steps with no host work in between.
 * All pointers are device pointers owned by the caller; `part` is shared by
 * the layers. */
typedef struct lk_decode_layer {
    const float * q_src;            /* fp32 [32][64] */
    const float * k_src;            /* fp32 [8][64] */
    const float * v_src;            /* fp32 [8][64] */
    float *       q;                /* fp32 [32][64] working q (normalised + rotated) */
    float *       k;                /* fp32 [8][64] working k */
    const float * q_norm;           /* fp32 [64] */
    const float * k_norm;           /* fp32 [64] */
    void *        kc;               /* fp16 [max_seq][8][64] */
    void *        vc;               /* fp16 [max_seq][8][64] */
    float *       out;              /* fp32 [32][64] or NULL */
    lk_block_q8_1 * yq8;            /* [64] or NULL */
    /* Optional third node, the attention output projection (reference
     * engine.cu:655-657): when wo_qs is not NULL, x += W_o . yq8 by
     * lk_gemv_q4_0 after the combine (yq8 and x required). */
    const void *  wo_qs;            /* Q4_0 [2048][64] 16-byte blocks, or NULL */
    const void *  wo_d;             /* fp16 [2048][64] block scales */
    float *       x;                /* fp32 [2048] residual stream */
} lk_decode_layer;
int lk_decode_step_graph_create(int n_layers, const lk_decode_layer * layers, int * d_pos,
                                float * part, void * stream, lk_decode_graph ** graph);
/* Replays a graph n_steps times on `stream` (no synchronisation). */
int lk_decode_graph_run(lk_decode_graph * graph, int n_steps, void * stream);

/* ---- prefill: int8 quantisers ---------------------------------------------
 * Per (row, head) 64-wide absmax quantisation (reference prefill.cu:1255-1267):
 * d = amax/127, q = rint(v * (127/amax)), scale = d * mul.  Bit-exact. */

/* Replaces k_pf_q8 (reference prefill.cuh:98-99, prefill.cu:1271-1287).
 * qh : fp16 [m][2048] (already x 1/8)  ->  q8 int8 [m][2048],
 * qsc fp32 [m][32] = d * log2(e), qcs fp32 [m][32] = (q.c) * log2(e) when
 * cm != NULL else 0.  cm: fp32 [8][64] smoothing vector or NULL. */
int lk_pf_q8(const void * qh, int m, const float * cm, int8_t * q8,
             float * qsc, float * qcs, void * stream);

/* Replaces k_pf_k8 (reference prefill.cuh:100-101, prefill.cu:1291-1301).
 * Positions [p0, p1) of kc fp16 [pos][8][64] -> k8 int8 (same layout) and
 * ksc fp32 [8][kstride] (head-major).  kstride must be a multiple of 4 and
 * >= p1.  cm as above. */
int lk_pf_k8(const void * kc, int p0, int p1, const float * cm, int kstride,
             int8_t * k8, float * ksc, void * stream);

/* Replaces k_pf_kmean (reference prefill.cuh:102, prefill.cu:1304-1318):
 * cm[h][d] = mean over positions [0, n) of kc.  Fixed summation order. */
int lk_pf_kmean(const void * kc, int n, float * cm, void * stream);

/* ---- prefill attention -----------------------------------------------------
 * One causal chunk of m query positions starting at position P, attending to
 * key positions [0, P + m).  o: fp32 [m][2048] (row = query, col = head*64+d).
 */

/* Replaces k_pf_attn8 (reference prefill.cuh:105-109, prefill.cu:1337-1571).
 * Key tiles of 64 within `near` positions of a 32-query tile's first query,
 * and key tile 0 when `sink` != 0, are scored exactly in fp16; all others use
 * int8 Q.K^T with int32 sums.  q8, qsc and qcs may all be NULL (an extension,
 * no counterpart in the reference): the kernel then quantises qh itself, with
 * lk_pf_q8's arithmetic and no smoothing, from the fp16 Q block it stages for
 * the exact tiles; the output is bit-identical to lk_pf_q8 + this call, and
 * the separate quantiser pass and its traffic go away. */
int lk_pf_attn8(const int8_t * q8, const float * qsc, const float * qcs,
                const void * qh, int m, int P, const int8_t * k8,
                const float * ksc, int kstride, const void * kc,
                const void * vc, int near, int sink, float * o, void * stream);

/* Replaces k_pf_attn (reference prefill.cuh:94-96, prefill.cu:1029-1226):
 * the same attention with every tile exact fp16. */
int lk_pf_attn(const void * qh, int m, int P, const void * kc, const void * vc,
               float * o, void * stream);

/* The same two attention kernels also emitting their output as planar Q8_1,
 * the next GEMM's activation format (reference PfAct, prefill.cuh:27-36,
 * produced there by a separate k_pf_quant_rows pass, engine.cu:1126): aqs int8
 * [m][2048] and asc fp32 [m][64][2] = (float(fp16(d)), 8 * float(fp16(sum)))
 * per 32-value block, byte-identical to lk_pf_quant_rows of o.  o may be NULL
 * when aqs is given.  No counterpart in the reference: the quantisation pass
 * fused into the attention epilogue. */
int lk_pf_attn8_q81(const int8_t * q8, const float * qsc, const float * qcs,
                    const void * qh, int m, int P, const int8_t * k8,
                    const float * ksc, int kstride, const void * kc,
                    const void * vc, int near, int sink, float * o,
                    int8_t * aqs, float * asc, void * stream);
int lk_pf_attn_q81(const void * qh, int m, int P, const void * kc, const void * vc,
                   float * o, int8_t * aqs, float * asc, void * stream);

/* Replaces k_pf_quant_rows (reference prefill.cuh:107, prefill.cu:1574-1580 with
 * pf_quant_warp, prefill.cu:90-103): planar Q8_1 of fp32 rows X [rows][ld],
 * kb 32-value blocks per row -> qs int8 [rows][kb*32], sc fp32 [rows][kb][2]. */
int lk_pf_quant_rows(const float * X, int rows, int ld, int kb, int8_t * qs, float * sc,
                     void * stream);

/* The same attention entry points with a caller-owned workspace for the
 * split-K partials, the reference's convention that every buffer is the
 * engine's (engine.cu:974-985): work (16-byte aligned device memory) of
 * work_bytes bytes; lk_pf_part_bytes() (64 MiB) is the most any chunk uses, a
 * smaller workspace makes the planner cut coarser pieces (work_bytes 0: no
 * split).  Launches that share one workspace must be ordered (one stream, or
 * the caller's events), as in the reference; with its own workspace every
 * launch may be captured into a hipGraph.  work = NULL falls back to the
 * library's static scratch (below).  No counterpart in the reference (its
 * kernels do not split). */
size_t lk_pf_part_bytes(void);
int lk_pf_attn8_ws(const int8_t * q8, const float * qsc, const float * qcs,
                   const void * qh, int m, int P, const int8_t * k8,
                   const float * ksc, int kstride, const void * kc,
                   const void * vc, int near, int sink, float * o,
                   int8_t * aqs, float * asc, void * work, size_t work_bytes, void * stream);
int lk_pf_attn_ws(const void * qh, int m, int P, const void * kc, const void * vc,
                  float * o, int8_t * aqs, float * asc, void * work, size_t work_bytes,
                  void * stream);

/* Both attention entry points balance causal chunks by splitting the key range
 * of long query blocks across workgroups (merged by a second kernel, in a fixed
 * order: output stays run-to-run bit-identical).  The entry points without a
 * workspace put the partials in a static 64 MiB device scratch of the library;
 * a split launch from another stream while an earlier one on that device is
 * pending is refused with hipErrorNotReady (not checked under stream capture).
 * Process-wide knob, for tests and tuning: -1 never split, 0 automatic
 * (default), n > 0 parts of at most n key tiles of 64.  No counterpart in the
 * reference (its kernels do not split). */
int lk_pf_split_override(int tiles);

/* Paired launches: one 8-wave workgroup per (kv head, block pair i, nq-1-i) of
 * a chunk; one 4-wave half scores block i and the first part of block
 * nq-1-i, the other half the rest of it, and the two parts are merged in LDS
 * (fixed order).  Every workgroup does the same work, so a 4096-row chunk at
 * P = 0 needs no split.  Process-wide knob, for tests and tuning: -1 never,
 * 0 automatic (default: chunks of at least 64 blocks with P <= m), 1
 * whenever the chunk has two or more blocks.  No counterpart in the
 * reference. */
int lk_pf_pair_override(int mode);

/* The paired kernel's two 4-wave groups meet at barriers of their own (a
 * counter in LDS), each polled at most `polls` times so that no wave can hang
 * the kernel (default 2^22 polls, about a quarter second per barrier; 0 sets
 * the default back).  A barrier that gives up is counted per device and makes
 * every output its workgroup writes afterwards NaN; the kernel still runs to
 * its end.  lk_pf_gsync_faults reads that count (synchronously: a diagnostic,
 * not for graph capture) and clears it when reset != 0.  Process-wide test
 * hooks; no counterpart in the reference. */
int lk_pf_gsync_limit(int polls);
int lk_pf_gsync_faults(unsigned * count, int reset);

/* ---- attention-input producers ---------------------------------------------
 * Per-head RMS norm (eps 1e-5) of q and k with weights qn / kn (fp32 [64]),
 * NEOX rotary embedding (theta 1e7) at the token's position, and the fp16
 * KV-cache write [pos][8][64].  1/sqrt, theta^(-i/32) and the cos/sin of the
 * fp32 angle are correctly rounded fp32 values (the reference uses CUDA's
 * rsqrtf / powf / sincosf). */

/* Replaces k_qk_norm_rope (reference kernels.cuh:666-670, kernels.cu:871-915;
 * launched at engine.cu:606-608):
 * qf fp32 [32][64] and kf fp32 [8][64] are normalised and rotated in place at
 * position *d_pos (device int32, graph-capturable); K and vf fp32 [8][64] go
 * to row *d_pos of kc / vc. */
int lk_qk_norm_rope(float * qf, float * kf, const float * vf, const float * qn,
                    const float * kn, const int * d_pos, void * kc, void * vc,
                    void * stream);

/* Replaces k_pf_qknr (reference prefill.cuh:85-87, prefill.cu:975-1016;
 * launched at engine.cu:1069-1070):
 * Y fp32 [m][3072] (q | k | v projection rows) for positions P .. P+m-1 ->
 * qh fp16 [m][2048] (rotated q x 1/8), K and V into rows P .. P+m-1 of kc / vc.
 * With k8 != NULL the same pass also writes the int8 copy of those K rows
 * (k8 [pos][8][64], ksc [8][kstride], kstride a multiple of 4 and >= P+m),
 * byte-identical to lk_pf_k8 over [P, P+m) with the same cm (NULL: none) --
 * the new rows of the reference's separate k_pf_k8 pass (engine.cu:1082-1083)
 * fused away.  Keys written by decode steps since the last prefill, and a
 * first chunk whose smoothing vector is derived from these very keys, still
 * need lk_pf_k8 / lk_pf_kmean. */
int lk_pf_qknr(const float * Y, const float * qn, const float * kn, int m, int P,
               void * qh, void * kc, void * vc, int8_t * k8, float * ksc, int kstride,
               const float * cm, void * stream);

/* ---- prefill chunk driver ---------------------------------------------------
 * The attention slice of the engine's prefill chunk (reference engine.cu:1064-
 * 1124 in pf_chunk, state engine.cu:236-256): per attention layer and chunk of
 * m tokens at [pos0, pos0+m): producers (+ the new rows' int8 K), the int8 K
 * copy caught up over [k8_valid, pos0) (keys decode steps appended since the
 * last prefill), the smoothing mean re-derived on a new context (pos0 == 0)
 * when ksmooth, the Q quantiser and the int8 (attn8 != 0) or fp16 attention
 * into o fp32 [m][2048] and/or (aqs, asc) planar Q8_1 (see lk_pf_attn8_q81; the
 * reference's k_pf_quant_rows that follows, engine.cu:1126, fused in; either
 * output may be NULL, not both).  lk_pf_chunk_done(pos0 + m) after the chunk's last
 * layer sets k8_valid (engine.cu:1251).  create allocates the chunk buffers
 * and, per layer, the int8 K copy [max_seq][8][64], its scales and the mean
 * (engine.cu:974-985); nothing is allocated per call.  The chunking of a
 * prompt is the caller's loop (engine.cu:1255-1260; chunk 8192 by default,
 * engine.cu:1315). */
typedef struct lk_pf_ctx lk_pf_ctx;
int lk_pf_ctx_create(int n_layers, int max_chunk, int max_seq, int attn8, int ksmooth,
                     int near, int sink, lk_pf_ctx ** ctx);
int lk_pf_ctx_destroy(lk_pf_ctx * ctx);
int lk_pf_chunk_attn(lk_pf_ctx * ctx, int layer, const float * Y, const float * qn,
                     const float * kn, int m, int pos0, void * kc, void * vc, float * o,
                     int8_t * aqs, float * asc, void * stream);
int lk_pf_chunk_done(lk_pf_ctx * ctx, int pos_end);
/* The context's device buffers for one layer (any output may be NULL). */
int lk_pf_ctx_buffers(const lk_pf_ctx * ctx, int layer, void ** qh, int8_t ** k8,
                      float ** ksc, float ** cm, int * kstride, int * k8_valid);

/* ---- test hook --------------------------------------------------------------
 * The raw int32 Q.K^T sums of the int8 scoring path, computed by the same
 * matrix-core routine lk_pf_attn8 uses:  s[head][i][j] = sum_d q8[i][head][d] *
 * k8[j][head/4][d] for i < m, j < n  (s: int32 [32][m][n]).  m and n must be
 * multiples of 16.  No counterpart in the reference; exists so the int32 sums
 * can be checked bit-exactly. */
int lk_pf_qk_i32(const int8_t * q8, int m, const int8_t * k8, int n,
                 int32_t * s, void * stream);

/* The split work list lk_pf_attn8 (int8 != 0) or lk_pf_attn would launch for
 * a chunk (m, P, near, sink), under the current lk_pf_split_override and for
 * the current device's slot count (512 when no device is visible): items in
 * dispatch order as int32 quadruples (query block, first key tile, end key
 * tile, partial slot or -1) into items[4 * max_items].  Returns the item count
 * (0: an unsplit launch), or -1 on bad arguments.  Host-side only, no device
 * work; no counterpart in the reference (its kernels do not split). */
int lk_pf_plan_items(int m, int P, int near, int sink, int int8, int32_t * items, int max_items);

/* Test hook: the 32 rotary frequencies theta^(-i/32) (theta = 1e7, reference
 * kernels.cuh:22-24) the producers use, as fp32, into out[32].  The kernels
 * keep them as constants rather than forming them with an fp64 pow; this lets
 * a CPU test check them against the host's pow.  No counterpart in the
 * reference (its kernels call powf). */
int lk_rope_freq_table(float * out);

/* Measurement reference, not on the attention path: a plain streaming read of
 * `bytes` (a multiple of 16, 16-byte aligned) at `src`, for the practical HBM
 * read rate next to the decode kernels' (the datasheet peak is not reachable
 * by reads).  `sink`: one fp32, written only under a condition the data never
 * meets.  No counterpart in the reference. */
int lk_read_probe(const void * src, size_t bytes, float * sink, void * stream);

/* Measurement utility, not on the attention path: the seeded synthetic inputs
 * of the benchmark configurations, generated on the device.  n fp32 values of
 * the splitmix64 stream of `seed` (draw k = mix(seed + k * 0x9e3779b97f4a7c15),
 * k = 1, 2, ...; u = ((x >> 11) + 1) / 2^53) into out:
 *   kind 0: N(0,1) by Box-Muller in float64 (pair j: draws 2j+1, 2j+2; cos,
 *           then sin), kind 1: uniform lo + (hi - lo) * u, kind 2: Student-t
 *           with nu = 4 (draws 10i+1 .. 10i+10: z / sqrt(chi2_4 / 4)).
 * The same values as a sequential host generator of the same definition.  No
 * counterpart in the reference (its CUDA harnesses use their own generators). */
int lk_synth_f32(int kind, uint64_t seed, size_t n, float lo, float hi, float * out, void * stream);

/* ---- the consumer of the decode attention output ------------------------ */

/* Q4_0 x Q8_1 GEMV: replaces k_gemv_q4_0 (reference kernels.cu:300-306, body
 * kernels.cu:190-260, block dot quant.cuh:131-158), launched for the attention
 * output at engine.cu:655-657 with xq = the combine's yq8.
 *   qs  : [out_rows][bpr] 16-byte Q4_0 quant blocks (byte j: element j in the
 *         low nibble, element 16+j in the high nibble), 16-byte aligned
 *   d   : [out_rows][bpr] fp16 block scales
 *   xq  : [bpr] Q8_1 activation blocks (K = 32 * bpr, 1 <= bpr <= 256)
 *   y   : [out_rows] fp32; y = (add_residual ? y : 0) + W.x (times the norm
 *         scale below)
 *   ssq : NULL, or the 64 sum-of-squares partials of an RMSNorm folded into the
 *         activation's producer: the row result is multiplied by
 *         1/sqrt((sum of ssq)/2048 + eps) (reference lk_norm_inv,
 *         kernels.cuh:441-447)
 * Per row the lane sums and the xor-butterfly follow the reference's warp
 * (lane l takes blocks l, l+32, ...); fp32 steps round as written. */
int lk_gemv_q4_0(const void * qs, const void * d, const lk_block_q8_1 * xq, int out_rows,
                 int bpr, float * y, int add_residual, const float * ssq, float eps,
                 void * stream);

/* Q4_0 x planar Q8_1 GEMM for a prefill chunk: replaces pf_gemm_dense with one
 * weight tensor and the plain epilogue (reference k_pf_mmq EPI 0,
 * prefill.cu:173-490 with PF_EPI2; pf_gemm_dense prefill.cu:818-826; PfGemm,
 * prefill.cuh:38-69), launched for the attention output at engine.cu:1128-1131
 * with (aqs, asc) = the planar Q8_1 lk_pf_attn8_q81 writes.
 *   qs  : [N][bpr] 16-byte Q4_0 blocks (16-byte aligned), d: [N][bpr] fp16
 *   aqs : int8 [ntok][bpr * 32]; asc: float2 [ntok][bpr] = (d8, 8 * sum)
 *   out : fp32 [ntok][out_ld] (16-byte aligned, out_ld a multiple of 4, >= N);
 *         out[t][r] = (add ? out[t][r] : 0) + scale[t] * sum over blocks
 *   scale: fp32 [ntok] or NULL (1)
 * N must be a multiple of 128 and bpr of 8 (as pf_gemm_dense requires), and
 * the activation quants below 4 GiB (ntok * bpr * 32 bytes).  Per
 * (t, r) the blocks are accumulated in order
 * with the reference's fma sequence; the epilogue rounds the product and the
 * sum separately, as the reference's source writes them. */
int lk_pf_gemm_q4_0(const void * qs, const void * d, int N, int bpr, const int8_t * aqs,
                    const float * asc, int ntok, const float * scale, float * out, int out_ld,
                    int add, void * stream);

#ifdef __cplusplus
}
#endif
#endif /* LK_ATTN_H */
