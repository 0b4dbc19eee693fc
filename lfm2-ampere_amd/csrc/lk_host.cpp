// lk_host.cpp - library-wide host entry points: configuration query, scratch
// sizing and the last-error string.
#include "lk_common.h"
#include <cstdarg>
#include <cstdio>
#include <cstring>

static thread_local char g_lk_err[512] = "no error";

int lk_fail(int code, const char * fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_lk_err, sizeof g_lk_err, fmt, ap);
    va_end(ap);
    return code;
}

int lk_launch_status(const char * what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return lk_fail((int) e, "%s: %s", what, hipGetErrorString(e));
    return 0;
}

extern "C" const char * lk_last_error(void) { return g_lk_err; }

extern "C" int lk_attn_config(int * split_cap, int * target_n, int * split_min) {
    if (split_cap) *split_cap = LK_ATTN_SPLIT;
    if (target_n)  *target_n  = LK_ATTN_TARGET_N;
    if (split_min) *split_min = LK_ATTN_SPLIT_MIN;
    return 0;
}

extern "C" size_t lk_attn_part_bytes(void) {
    return (size_t) LK_N_HEADS * LK_ATTN_SPLIT * LK_ATTN_PARTW * sizeof(float);
}

extern "C" int lk_rope_freq_table(float * out) {
    static const float tab[LK_HEAD_DIM / 2] = { LK_ROPE_FREQ_INIT };
    if (!out) return lk_fail(hipErrorInvalidValue, "lk_rope_freq_table: null pointer");
    memcpy(out, tab, sizeof tab);
    return 0;
}
