// capi_host.cpp - a C++ caller of the attention library that uses nothing but
// its C ABI (include/lk_attn.h), the way the engine's host code would after
// the swap: device buffers from hipMalloc, one stream, decode attention also
// captured into a graph, prefill with the engine's own workspace, errors as
// return codes.  Built as a shared library by tests/csrc/Makefile and driven
// in-process by tests/test_capi_host_gpu.py through ctypes, which hands in
// host inputs and checks the outputs against the oracle.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "lk_attn.h"

namespace {

struct Run {
    char * msg;
    int msglen;
    std::vector<void *> bufs;
    hipStream_t st = nullptr;

    int fail(int line, const char * what) {
        std::snprintf(msg, (size_t) msglen, "line %d: %s (lk_last_error: %s)", line, what, lk_last_error());
        return line;
    }
    template <class T> T * alloc(size_t bytes) {
        void * p = nullptr;
        if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
        bufs.push_back(p);
        return (T *) p;
    }
    ~Run() {
        if (st) (void) hipStreamSynchronize(st);
        for (void * p : bufs) (void) hipFree(p);
        if (st) (void) hipStreamDestroy(st);
    }
};

}  // namespace

#define REQ(cond, what) do { if (!(cond)) return R.fail(__LINE__, what); } while (0)
#define CALL(expr) do { const int rc_ = (expr); if (rc_ != 0) return R.fail(__LINE__, #expr); } while (0)

// Decode: q fp32 [32][64], kc/vc fp16 bits [seq][8][64].  dec_out receives
// three fp32 [32][64] results: lk_attn_decode with a caller workspace,
// lk_attn_decode_noalloc, and a one-layer lk_decode_graph replay.
// Prefill: qh fp16 bits [m][2048], kc/vc fp16 bits [P+m][8][64].  pf_out
// receives two fp32 [m][2048] results of the int8 attention with Q quantised
// in the kernel: lk_pf_attn8 (the library's static split scratch) and
// lk_pf_attn8_ws with a workspace the caller allocated; k8 / ksc receive
// lk_pf_k8's int8 K ([P+m][8][64]) and scales ([8][kstride], kstride = P+m
// rounded up to 4).  Returns 0, or the failing line with a message in msg.
extern "C" int capi_host_run(const float * q_h, const uint16_t * kc_h, const uint16_t * vc_h, int seq,
                             float * dec_out, const uint16_t * pq_h, const uint16_t * pk_h,
                             const uint16_t * pv_h, int m, int P, int near, int sink, float * pf_out,
                             int8_t * k8_out, float * ksc_out, char * msg, int msglen) {
    Run R{ msg, msglen };
    if (msglen > 0) msg[0] = '\0';
    REQ(seq >= 1 && m >= 1 && P >= 0, "arguments");
    REQ(hipStreamCreate(&R.st) == hipSuccess, "hipStreamCreate");
    void * st = (void *) R.st;

    // ---- decode ---------------------------------------------------------------
    const size_t row = 8 * 64;                                   // fp16 values per cache row
    float * q = R.alloc<float>(32 * 64 * sizeof(float));
    uint16_t * kc = R.alloc<uint16_t>((size_t) seq * row * 2);
    uint16_t * vc = R.alloc<uint16_t>((size_t) seq * row * 2);
    int * d_pos = R.alloc<int>(sizeof(int));
    float * part = R.alloc<float>(lk_attn_part_bytes());
    float * out[3];
    for (int i = 0; i < 3; ++i) out[i] = R.alloc<float>(32 * 64 * sizeof(float));
    REQ(q && kc && vc && d_pos && part && out[0] && out[1] && out[2], "hipMalloc (decode)");
    const int pos = seq - 1;
    REQ(hipMemcpy(q, q_h, 32 * 64 * sizeof(float), hipMemcpyHostToDevice) == hipSuccess, "copy q");
    REQ(hipMemcpy(kc, kc_h, (size_t) seq * row * 2, hipMemcpyHostToDevice) == hipSuccess, "copy kc");
    REQ(hipMemcpy(vc, vc_h, (size_t) seq * row * 2, hipMemcpyHostToDevice) == hipSuccess, "copy vc");
    REQ(hipMemcpy(d_pos, &pos, sizeof(int), hipMemcpyHostToDevice) == hipSuccess, "copy d_pos");

    CALL(lk_attn_decode(q, kc, vc, d_pos, part, out[0], nullptr, st));
    CALL(lk_attn_decode_noalloc(q, kc, vc, d_pos, out[1], nullptr, st));
    {
        const float * qs[1] = { q };
        const void * kcs[1] = { kc };
        const void * vcs[1] = { vc };
        float * outs[1] = { out[2] };
        lk_decode_graph * g = nullptr;
        CALL(lk_decode_graph_create(1, qs, kcs, vcs, d_pos, part, outs, nullptr, st, &g));
        size_t nodes = 0;
        const int rn = lk_decode_graph_nodes(g, &nodes);
        const int rl = lk_decode_graph_launch(g, st);
        const int rd = lk_decode_graph_destroy(g);
        REQ(rn == 0 && nodes == 2, "lk_decode_graph_nodes: one layer is (split, combine)");
        REQ(rl == 0 && rd == 0, "lk_decode_graph_launch / destroy");
    }
    // the error path: a NULL operand is refused with a message, nothing launched
    REQ(lk_attn_decode(nullptr, kc, vc, d_pos, part, out[0], nullptr, st) != 0, "NULL q accepted");
    REQ(std::strlen(lk_last_error()) > 0, "no error message");

    // ---- prefill --------------------------------------------------------------
    const int S = P + m, kstride = (S + 3) & ~3;
    uint16_t * qh = R.alloc<uint16_t>((size_t) m * 2048 * 2);
    uint16_t * pkc = R.alloc<uint16_t>((size_t) S * row * 2);
    uint16_t * pvc = R.alloc<uint16_t>((size_t) S * row * 2);
    int8_t * k8 = R.alloc<int8_t>((size_t) S * row);
    float * ksc = R.alloc<float>((size_t) (8 * kstride + 4) * sizeof(float));
    float * o[2];
    for (int i = 0; i < 2; ++i) o[i] = R.alloc<float>((size_t) m * 2048 * sizeof(float));
    const size_t work_bytes = lk_pf_part_bytes();
    void * work = R.alloc<void>(work_bytes);
    REQ(qh && pkc && pvc && k8 && ksc && o[0] && o[1] && work, "hipMalloc (prefill)");
    REQ(hipMemcpy(qh, pq_h, (size_t) m * 2048 * 2, hipMemcpyHostToDevice) == hipSuccess, "copy qh");
    REQ(hipMemcpy(pkc, pk_h, (size_t) S * row * 2, hipMemcpyHostToDevice) == hipSuccess, "copy prefill kc");
    REQ(hipMemcpy(pvc, pv_h, (size_t) S * row * 2, hipMemcpyHostToDevice) == hipSuccess, "copy prefill vc");

    CALL(lk_pf_k8(pkc, 0, S, nullptr, kstride, k8, ksc, st));
    CALL(lk_pf_attn8(nullptr, nullptr, nullptr, qh, m, P, k8, ksc, kstride, pkc, pvc, near, sink, o[0], st));
    CALL(lk_pf_attn8_ws(nullptr, nullptr, nullptr, qh, m, P, k8, ksc, kstride, pkc, pvc, near, sink, o[1],
                        nullptr, nullptr, work, work_bytes, st));

    REQ(hipStreamSynchronize(R.st) == hipSuccess, "hipStreamSynchronize");
    for (int i = 0; i < 3; ++i)
        REQ(hipMemcpy(dec_out + (size_t) i * 32 * 64, out[i], 32 * 64 * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess,
            "copy decode out");
    for (int i = 0; i < 2; ++i)
        REQ(hipMemcpy(pf_out + (size_t) i * m * 2048, o[i], (size_t) m * 2048 * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess,
            "copy prefill out");
    REQ(hipMemcpy(k8_out, k8, (size_t) S * row, hipMemcpyDeviceToHost) == hipSuccess, "copy k8");
    REQ(hipMemcpy(ksc_out, ksc, (size_t) 8 * kstride * sizeof(float), hipMemcpyDeviceToHost) == hipSuccess, "copy ksc");
    return 0;
}
