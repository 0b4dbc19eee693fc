// pf_driver.cpp - the attention slice of the engine's prefill chunk
// (reference engine.cu:1064-1124 inside pf_chunk, state at engine.cu:236-256,
// k8_valid bookkeeping at engine.cu:1080 and 1251): per attention layer and
// chunk of m tokens at positions [pos0, pos0+m):
//   1. lk_pf_qknr: q/k norm + RoPE, K/V appended to the fp16 cache, and (int8
//      scoring, no smoothing-vector refresh) the int8 K copy of the new rows;
//   2. the int8 K copy caught up over [k8_valid, pos0) -- rows written by
//      decode steps since the last prefill; a new context (pos0 == 0) with
//      smoothing re-derives the mean vector from this chunk's keys first;
//   3. lk_pf_q8, then lk_pf_attn8 (or lk_pf_attn with int8 scoring off), the
//      output as fp32 and/or planar Q8_1 (the reference's k_pf_quant_rows
//      that follows, engine.cu:1126, fused into the attention epilogue);
//      without smoothing the attention kernel quantises Q itself (same bits).
// lk_pf_chunk_done(pos0 + m) after the chunk's last layer moves k8_valid,
// exactly where the reference does.  Buffers are allocated once, at create,
// the split-K partial workspace of the attention launches included, so that a
// context owns every buffer its launches touch (engine.cu:974-985) and the
// launches of two contexts never share scratch.
#include "lk_common.h"
#include <vector>

struct lk_pf_ctx {
    int n_layers = 0, max_chunk = 0, max_seq = 0, kstride = 0;
    int attn8 = 1, ksmooth = 0, near = 1024, sink = 1;
    int k8_valid = 0;
    _Float16 * qh = nullptr;
    int8_t * q8 = nullptr;
    float * qsc = nullptr, * qcs = nullptr;
    void * work = nullptr;                               // split-K partials (lk_pf_part_bytes())
    size_t work_bytes = 0;
    std::vector<int8_t *> k8;
    std::vector<float *> ksc, cm;
};

static void pf_ctx_free(lk_pf_ctx * c) {
    if (!c) return;
    (void) hipFree(c->qh); (void) hipFree(c->q8); (void) hipFree(c->qsc); (void) hipFree(c->qcs);
    (void) hipFree(c->work);
    for (auto p : c->k8) (void) hipFree(p);
    for (auto p : c->ksc) (void) hipFree(p);
    for (auto p : c->cm) (void) hipFree(p);
    delete c;
}

template <typename T>
static bool pf_alloc(T ** p, size_t n) {
    return hipMalloc((void **) p, n * sizeof(T)) == hipSuccess;
}

extern "C" int lk_pf_ctx_create(int n_layers, int max_chunk, int max_seq, int attn8, int ksmooth,
                                int near, int sink, lk_pf_ctx ** ctx) {
    if (!ctx) return lk_fail(hipErrorInvalidValue, "lk_pf_ctx_create: ctx is null");
    *ctx = nullptr;
    if (n_layers <= 0 || max_chunk <= 0 || max_seq < max_chunk)
        return lk_fail(hipErrorInvalidValue, "lk_pf_ctx_create: n_layers %d, max_chunk %d, max_seq %d",
                       n_layers, max_chunk, max_seq);
    lk_pf_ctx * c = new lk_pf_ctx;
    c->n_layers = n_layers; c->max_chunk = max_chunk; c->max_seq = max_seq;
    c->kstride = (max_seq + 3) & ~3;                     // engine.cu:249 (ksc row stride)
    c->attn8 = attn8 != 0; c->ksmooth = ksmooth != 0; c->near = near; c->sink = sink;
    bool ok = pf_alloc(&c->qh, (size_t) max_chunk * LK_HIDDEN);
    c->work_bytes = lk_pf_part_bytes();
    ok = ok && pf_alloc((char **) &c->work, c->work_bytes);
    if (c->attn8) {
        ok = ok && pf_alloc(&c->q8, (size_t) max_chunk * LK_HIDDEN) && pf_alloc(&c->qsc, (size_t) max_chunk * LK_N_HEADS)
                && pf_alloc(&c->qcs, (size_t) max_chunk * LK_N_HEADS);
        c->k8.assign(n_layers, nullptr); c->ksc.assign(n_layers, nullptr); c->cm.assign(n_layers, nullptr);
        for (int l = 0; l < n_layers && ok; ++l)
            ok = pf_alloc(&c->k8[l], (size_t) max_seq * LK_KV_ROW)
              && pf_alloc(&c->ksc[l], (size_t) LK_N_KV_HEADS * c->kstride + 4)
              && pf_alloc(&c->cm[l], (size_t) LK_N_KV_HEADS * LK_HEAD_DIM);
    }
    if (!ok) { pf_ctx_free(c); return lk_fail(hipErrorOutOfMemory, "lk_pf_ctx_create: out of device memory"); }
    *ctx = c;
    return 0;
}

extern "C" int lk_pf_ctx_destroy(lk_pf_ctx * ctx) { pf_ctx_free(ctx); return 0; }

extern "C" int lk_pf_chunk_attn(lk_pf_ctx * c, int layer, const float * Y, const float * qn, const float * kn,
                                int m, int pos0, void * kc, void * vc, float * o, int8_t * aqs, float * asc,
                                void * stream) {
    if (!c || layer < 0 || layer >= c->n_layers || m <= 0 || m > c->max_chunk || pos0 < 0
        || pos0 + m > c->max_seq || !Y || !qn || !kn || !kc || !vc || (!o && !aqs) || (!aqs != !asc))
        return lk_fail(hipErrorInvalidValue, "lk_pf_chunk_attn: bad arguments (layer %d, m %d, pos0 %d)",
                       layer, m, pos0);
    int rc;
    if (!c->attn8) {
        rc = lk_pf_qknr(Y, qn, kn, m, pos0, c->qh, kc, vc, nullptr, nullptr, 0, nullptr, stream);
        return rc ? rc : lk_pf_attn_ws(c->qh, m, pos0, kc, vc, o, aqs, asc, c->work, c->work_bytes, stream);
    }
    int8_t * k8 = c->k8[layer];
    float * ksc = c->ksc[layer];
    float * cm = c->ksmooth ? c->cm[layer] : nullptr;
    const bool refresh_mean = c->ksmooth && pos0 == 0;   // engine.cu:1081
    // the new rows' int8 K in the producer pass, unless the mean they need is
    // derived from these very rows
    rc = lk_pf_qknr(Y, qn, kn, m, pos0, c->qh, kc, vc, refresh_mean ? nullptr : k8, ksc, c->kstride,
                    cm, stream);
    if (rc) return rc;
    if (refresh_mean) {
        rc = lk_pf_kmean(kc, m, cm, stream);
        if (!rc) rc = lk_pf_k8(kc, 0, m, cm, c->kstride, k8, ksc, stream);
    } else {
        const int lo = (pos0 == 0) ? 0 : (c->k8_valid < pos0 ? c->k8_valid : pos0);   // engine.cu:1080
        if (lo < pos0) rc = lk_pf_k8(kc, lo, pos0, cm, c->kstride, k8, ksc, stream);
    }
    if (rc) return rc;
    if (!cm)   // no smoothing: the attention kernel quantises Q itself (same bits, one pass less)
        return lk_pf_attn8_ws(nullptr, nullptr, nullptr, c->qh, m, pos0, k8, ksc, c->kstride, kc, vc,
                              c->near, c->sink, o, aqs, asc, c->work, c->work_bytes, stream);
    rc = lk_pf_q8(c->qh, m, cm, c->q8, c->qsc, c->qcs, stream);
    if (rc) return rc;
    return lk_pf_attn8_ws(c->q8, c->qsc, c->qcs, c->qh, m, pos0, k8, ksc, c->kstride, kc, vc,
                          c->near, c->sink, o, aqs, asc, c->work, c->work_bytes, stream);
}

extern "C" int lk_pf_chunk_done(lk_pf_ctx * c, int pos_end) {
    if (!c || pos_end < 0 || pos_end > c->max_seq)
        return lk_fail(hipErrorInvalidValue, "lk_pf_chunk_done: bad arguments");
    c->k8_valid = pos_end;                                // engine.cu:1251
    return 0;
}

extern "C" int lk_pf_ctx_buffers(const lk_pf_ctx * c, int layer, void ** qh, int8_t ** k8, float ** ksc,
                                 float ** cm, int * kstride, int * k8_valid) {
    if (!c || layer < 0 || layer >= c->n_layers)
        return lk_fail(hipErrorInvalidValue, "lk_pf_ctx_buffers: bad arguments");
    if (qh) *qh = c->qh;
    if (k8) *k8 = c->attn8 ? c->k8[layer] : nullptr;
    if (ksc) *ksc = c->attn8 ? c->ksc[layer] : nullptr;
    if (cm) *cm = c->attn8 ? c->cm[layer] : nullptr;
    if (kstride) *kstride = c->kstride;
    if (k8_valid) *k8_valid = c->k8_valid;
    return 0;
}
