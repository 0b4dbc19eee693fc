// lk_common.h - shared constants, vector types and host-side error plumbing of
// the gfx950 attention library.  Device code here is CDNA4-only (wave64,
// MFMA); nothing is written for any other target.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/lk_attn.h"

// ---- model constants (reference kernels.cuh:12-24) --------------------------
#define LK_G        (LK_N_HEADS / LK_N_KV_HEADS)   // query heads per kv head
#define LK_HIDDEN   (LK_N_HEADS * LK_HEAD_DIM)     // 2048
#define LK_KV_ROW   (LK_N_KV_HEADS * LK_HEAD_DIM)  // 512 fp16 per cache position

// ---- split-K operating point --------------------------------------------------
// The reference's rule (kernels.cuh:630-635) with its cap/target retuned for
// MI355X: 8 kv heads x LK_ATTN_SPLIT workgroups is the fixed, graph-capturable
// grid; slices = clamp(ceil(seq/TARGET_N), SPLIT_MIN, SPLIT).  Overridable at
// build time (-D), like the reference's Makefile knobs.
#ifndef LK_ATTN_SPLIT
#define LK_ATTN_SPLIT      256
#endif
#ifndef LK_ATTN_TARGET_N
#define LK_ATTN_TARGET_N   128
#endif
#ifndef LK_ATTN_SPLIT_MIN
#define LK_ATTN_SPLIT_MIN  8
#endif
// 16-token groups a decode wave loads before it consumes any of them.
#ifndef LK_ATTN_UNROLL
#define LK_ATTN_UNROLL     4
#endif

// ---- vector types ---------------------------------------------------------------
typedef _Float16 lk_h8  __attribute__((ext_vector_type(8)));
typedef _Float16 lk_h4  __attribute__((ext_vector_type(4)));
typedef float    lk_f4  __attribute__((ext_vector_type(4)));
typedef int      lk_i4  __attribute__((ext_vector_type(4)));

#define LK_LOG2E_F 1.4426950408889634f

// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float lk_exp2(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_exp2f(x);
#else
    return exp2f(x);     // host pass only parses device bodies
#endif
}

__host__ __device__ __forceinline__ void lk_attn_slices(int seq, int & ns, int & chunk) {
    int s = (seq + LK_ATTN_TARGET_N - 1) / LK_ATTN_TARGET_N;
    if (s < LK_ATTN_SPLIT_MIN) s = LK_ATTN_SPLIT_MIN;
    if (s > LK_ATTN_SPLIT)     s = LK_ATTN_SPLIT;
    ns = s;
    chunk = (seq + s - 1) / s;
}

// ---- host-side error plumbing (lk_host.cpp) -----------------------------------
int lk_fail(int code, const char * fmt, ...);
// hipGetLastError after a launch, mapped into lk_fail.
int lk_launch_status(const char * what);
static inline hipStream_t lk_stream(void * s) { return (hipStream_t) s; }
