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
// grid; slices = clamp(ceil(seq/TARGET_N), SPLIT_MIN, SPLIT).  TARGET_N = 16
// (one LDS tile per workgroup) gives every one of the 256 CUs a slice from a
// 4096-position context up; from 4096 positions on the cap decides.  Measured
// per layer in a 10-layer graph against TARGET_N = 128: 2k 12.05 -> 8.79 us,
// 8k 12.29 -> 10.40 us, 16k 12.99 -> 11.89 us, 32k unchanged (capped).
// Overridable at build time (-D), like the reference's Makefile knobs.
#ifndef LK_ATTN_SPLIT
#define LK_ATTN_SPLIT      256
#endif
#ifndef LK_ATTN_TARGET_N
#define LK_ATTN_TARGET_N   16
#endif
#ifndef LK_ATTN_SPLIT_MIN
#define LK_ATTN_SPLIT_MIN  8
#endif
// Decode LDS ring: LK_DEC_NBUF tiles of LK_DEC_TILE cache positions (multiple
// of 16); LK_DEC_NBUF - 1 of them are in flight while one is consumed.
#ifndef LK_DEC_TILE
#define LK_DEC_TILE        16
#endif
#ifndef LK_DEC_NBUF
#define LK_DEC_NBUF        4
#endif

// ---- vector types ---------------------------------------------------------------
typedef unsigned short lk_u16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short lk_u16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 lk_h8  __attribute__((ext_vector_type(8)));
typedef _Float16 lk_h4  __attribute__((ext_vector_type(4)));
typedef unsigned short lk_u16x4 __attribute__((ext_vector_type(4)));
typedef float    lk_f4  __attribute__((ext_vector_type(4)));
typedef int      lk_i4  __attribute__((ext_vector_type(4)));

#define LK_LOG2E_F 1.4426950408889634f

// ---- cross-lane reductions over one 16-lane row (DPP, no LDS traffic) ------
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: a
// fixed butterfly after which EVERY lane of the row holds the same total
// (lane i and its partner add the same two operands, so the bits agree).
#define LK_DPP_QP_XOR1   0xB1
#define LK_DPP_QP_XOR2   0x4E
#define LK_DPP_HMIRROR   0x141
#define LK_DPP_MIRROR    0x140
#ifdef __HIP_DEVICE_COMPILE__
template <int CTRL>
__device__ __forceinline__ float lk_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
#else
template <int CTRL>
__device__ __forceinline__ float lk_dpp(float v) { return v; }
#endif
__device__ __forceinline__ float lk_row_sum16(float v) {
    v += lk_dpp<LK_DPP_QP_XOR1>(v);
    v += lk_dpp<LK_DPP_QP_XOR2>(v);
    v += lk_dpp<LK_DPP_HMIRROR>(v);
    v += lk_dpp<LK_DPP_MIRROR>(v);
    return v;
}
__device__ __forceinline__ float lk_row_max16(float v) {
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR1>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR2>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_HMIRROR>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_MIRROR>(v));
    return v;
}

// Max over the four 16-lane rows holding the same column (lanes l, l^16,
// l^32, l^48), with the gfx950 lane swaps (VALU, no LDS round trip):
// v_permlane32_swap exchanges the upper 32 lanes of its first operand with the
// lower 32 of its second, v_permlane16_swap the odd 16-lane rows of the first
// with the even rows of the second.  Swapping a value with a copy of itself
// leaves each lane holding itself and its partner; their max is symmetric, so
// all four lanes end with identical bits.  Written as inline asm (with the
// wait states the VALU -> permlane hazard needs) because the compiler folds
// max(r0, r1) of the builtin's two results to r0, which is wrong.
#ifdef __HIP_DEVICE_COMPILE__
__device__ __forceinline__ float lk_xrow_max(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    float c = fmaxf(a, b), d = c;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(c), "+v"(d));
    return fmaxf(c, d);
}
#else
__device__ __forceinline__ float lk_xrow_max(float x) { return x; }
#endif

// Sum over the four 16-lane rows (lanes l, l^16, l^32, l^48) with the gfx950
// lane swaps; like lk_xrow_max, every lane ends with identical bits.
#ifdef __HIP_DEVICE_COMPILE__
__device__ __forceinline__ float lk_xrow_sum(float x) {
    float a = x, b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    float c = a + b, d = c;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(c), "+v"(d));
    return c + d;
}
#else
__device__ __forceinline__ float lk_xrow_sum(float x) { return x; }
#endif

// The xor butterfly over the 32 lanes of each half-wave with offsets 16, 8,
// 4, 2, 1 (the order of __shfl_xor loops of width 32), on lane swaps and DPP
// instead of LDS permutes: offset 16 is v_permlane16_swap, 8 is row_ror:8
// (lane i of a 16-lane row meets i+8 mod 16 = i^8), 4 is row_ror:4 (lane i
// meets i+4 mod 16, which after the offset-8 step holds the same value as
// i^4), 2 and 1 are quad permutes.  Every step adds (or maxes) the same two
// operands in both partner lanes, so all 32 lanes end with identical bits,
// equal to the __shfl_xor butterfly's.
#define LK_DPP_ROR8      0x128
#define LK_DPP_ROR4      0x124
#ifdef __HIP_DEVICE_COMPILE__
__device__ __forceinline__ void lk_swap16(float & a, float & b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
#else
__device__ __forceinline__ void lk_swap16(float &, float &) {}
#endif
__device__ __forceinline__ float lk_bfly32_sum(float x) {
    float a = x, b = x;
    lk_swap16(a, b);
    float v = a + b;
    v += lk_dpp<LK_DPP_ROR8>(v);
    v += lk_dpp<LK_DPP_ROR4>(v);
    v += lk_dpp<LK_DPP_QP_XOR2>(v);
    v += lk_dpp<LK_DPP_QP_XOR1>(v);
    return v;
}
__device__ __forceinline__ float lk_bfly32_max(float x) {
    float a = x, b = x;
    lk_swap16(a, b);
    float v = fmaxf(a, b);
    v = fmaxf(v, lk_dpp<LK_DPP_ROR8>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_ROR4>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR2>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR1>(v));
    return v;
}

// Four fp16 of one column from a row-major LDS tile via the gfx950 transpose
// read (ds_read_b64_tr_b16).  Within each 16-lane group, lane 4a+b supplies
// the address of T[row0 + a][col0 + 4b .. +3]; lane c then receives
// T[row0 .. row0+3][col0 + c].
#ifdef __HIP_DEVICE_COMPILE__
__device__ __forceinline__ lk_h4 lk_ds_tr4(const void * p) {
    typedef short lk_s4 __attribute__((ext_vector_type(4)));
    const lk_s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) lk_s4 *) (p));
    return __builtin_bit_cast(lk_h4, v);
}
#else
__device__ __forceinline__ lk_h4 lk_ds_tr4(const void *) { return lk_h4{}; }
#endif

// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float lk_exp2(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_exp2f(x);
#else
    return exp2f(x);     // host pass only parses device bodies
#endif
}

// Slice partials in `part` (fp32; lk_attn_part_bytes() holds 32 x split_cap x
// LK_ATTN_PARTW floats, of which this layout uses 66 per (head, slot)):
//   acc plane: [head][chunk c = dims 16c..16c+15][slot][16]  (32 x 4 x split_cap x 16)
//   (m, l) plane after it: [head][slot][2]
// The combine's lanes take consecutive slots, so the four waves of a
// (head, half) workgroup together read runs of consecutive 64-byte pieces
// (acc; one wave 32 bytes of each) and one 512-byte run (m, l) per load,
// instead of 64 records 272 B apart; the split's four lanes of a (head, chunk)
// write one whole 64-byte piece.
__host__ __device__ constexpr size_t lk_part_acc(int head, int c, int slot) {
    return (((size_t) head * 4 + c) * LK_ATTN_SPLIT + slot) * 16;
}
__host__ __device__ constexpr size_t lk_part_ml(int head, int slot) {
    return (size_t) LK_N_HEADS * LK_HEAD_DIM * LK_ATTN_SPLIT + ((size_t) head * LK_ATTN_SPLIT + slot) * 2;
}

__host__ __device__ __forceinline__ void lk_attn_slices(int seq, int & ns, int & chunk) {
    int s = (seq + LK_ATTN_TARGET_N - 1) / LK_ATTN_TARGET_N;
    if (s < LK_ATTN_SPLIT_MIN) s = LK_ATTN_SPLIT_MIN;
    if (s > LK_ATTN_SPLIT)     s = LK_ATTN_SPLIT;
    ns = s;
    chunk = (seq + s - 1) / s;
}

// ---- rotary embedding constants and table entry (qknr.hip, decode.hip) -----------
// Reference kernels.cuh:22-24: LK_EPS 1e-5, LK_ROPE_THETA 1e7.  Entry i < 32 of
// position pos: f = theta^(-i/32) and the cosine and sine of the fp32 angle
// (float) pos * f, each evaluated in fp64 and rounded once to fp32.  The 32
// frequencies are constants: (float) pow(1e7, -i / 32.0) in fp64, rounded once
// (a test checks them against the host's pow, the oracle's formula); forming
// them on the device with pow costs a chain of about 220 dependent fp64
// instructions.
#define LK_EPS_F        1e-5f
#define LK_ROPE_THETA_D 10000000.0
#define LK_ROPE_FREQ_INIT \
    0x1p+0f, 0x1.356656p-1f, 0x1.75f034p-2f, 0x1.c3f06cp-3f, \
    0x1.111aeep-3f, 0x1.4a12aep-4f, 0x1.8eec7ep-5f, 0x1.e222ecp-6f, \
    0x1.235a72p-6f, 0x1.6020a4p-7f, 0x1.a99428p-8f, 0x1.012cfap-8f, \
    0x1.36d21ap-9f, 0x1.77a7d8p-10f, 0x1.c603c4p-11f, 0x1.125c04p-11f, \
    0x1.4b96bep-12f, 0x1.90c182p-13f, 0x1.e459c6p-14f, 0x1.24b0fep-14f, \
    0x1.61bea2p-15f, 0x1.ab8884p-16f, 0x1.025b58p-16f, 0x1.383f88p-17f, \
    0x1.796182p-18f, 0x1.c8198cp-19f, 0x1.139e96p-19f, 0x1.4d1c98p-20f, \
    0x1.9298acp-21f, 0x1.e69338p-22f, 0x1.26091cp-22f, 0x1.635e88p-23f
// Entry i (0..31) by a select tree over the bits of i on immediate constants:
// no memory access (a load of a constant table went to L2 or HBM at the start
// of every producer workgroup and cost more than the fp64 pow it replaced).
__device__ __forceinline__ float lk_rope_freq(int i) {
    constexpr float T[LK_HEAD_DIM / 2] = { LK_ROPE_FREQ_INIT };
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = (i & 1) ? T[2 * k + 1] : T[2 * k];
#pragma unroll
    for (int b = 1, n = 8; n >= 1; ++b, n >>= 1)
#pragma unroll
        for (int k = 0; k < n; ++k) v[k] = ((i >> b) & 1) ? v[2 * k + 1] : v[2 * k];
    return v[0];
}
// The same constants in constant memory, for a kernel whose index is
// wave-uniform: the four entries 4j..4j+3 come in by one scalar load
// (counted by lgkmcnt, so it never waits behind vector-memory DMA in flight,
// as a vector load of the table would), and lane l takes entry 4j + (l & 3).
static __constant__ float lk_rope_tab[LK_HEAD_DIM / 2] = { LK_ROPE_FREQ_INIT };
__device__ __forceinline__ float lk_rope_freq_quad(int j_uniform, int lane) {
    const float4 f = *(const float4 *) (lk_rope_tab + 4 * j_uniform);
    const float lo = (lane & 1) ? f.y : f.x, hi = (lane & 1) ? f.w : f.z;
    return (lane & 2) ? hi : lo;
}
__device__ __forceinline__ void lk_rope_angle(int pos, float f, float & c, float & s) {
    const float a = (float) pos * f;                           // fp32 product, as the reference
    double sd, cd;
    sincos((double) a, &sd, &cd);
    c = (float) cd;
    s = (float) sd;
}

// ---- int8 row quantiser on 8-lane groups (shared by prefill.hip, qknr.hip) -----
// A 64-wide row is held by 8 consecutive lanes, 8 consecutive values each.
__device__ __forceinline__ float lk_max8(float v) {     // max over the 8-lane group
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR1>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_QP_XOR2>(v));
    v = fmaxf(v, lk_dpp<LK_DPP_HMIRROR>(v));
    return v;
}
__device__ __forceinline__ void lk_q8_row8(const float (&v)[8], int8_t * __restrict__ dst8,
                                           float * __restrict__ scl, float mul, bool lead) {
#pragma clang fp contract(off)
    float am = fabsf(v[0]);
#pragma unroll
    for (int i = 1; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = lk_max8(am);
    const float d = am / 127.0f;
    const float id = (am > 0.0f) ? 127.0f / am : 0.0f;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w0 |= (uint32_t) (uint8_t) (int8_t) (int) __builtin_rintf(v[i] * id) << (8 * i);
        w1 |= (uint32_t) (uint8_t) (int8_t) (int) __builtin_rintf(v[4 + i] * id) << (8 * i);
    }
    *(uint2 *) dst8 = make_uint2(w0, w1);
    if (lead) *scl = d * mul;
}
__device__ __forceinline__ void lk_load8h(const _Float16 * __restrict__ src, float (&v)[8]) {
    const lk_h8 h = *(const lk_h8 *) src;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float) h[i];
}

// ---- LDS DMA (global_load_lds_dwordx4) --------------------------------------
// Byte address of an LDS object (the value M0 takes for an LDS DMA).
__device__ __forceinline__ uint32_t lk_lds_addr(const void * p) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) void *) p;
}
// One LDS DMA: each active lane's 16 bytes at `src` land at LDS byte
// lds + 16*lane (lds must be wave-uniform).  Issued as inline asm so the
// compiler does not serialise later LDS reads on it; completion is tracked by
// hand with vmcnt (in-order) plus a barrier.  M0 is written here; no other
// code in this library uses M0, so clobbering it is safe.  lk_dma16 is
// non-temporal (streams read once), lk_dma16c keeps the normal cache policy
// (tiles that other workgroups read again).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lk_dma16(const void * src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void lk_dma16c(const void * src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(src), "s"(lds) : "memory", "m0");
}
// The same with a wave-uniform 64-bit base (SGPRs) plus a per-lane 32-bit
// byte offset: moving the source costs only scalar adds.
__device__ __forceinline__ void lk_dma16c_so(const void * sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :: "v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop
// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void lk_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}
// A 16-byte global load the compiler does not track (inline asm), for loads
// issued ahead of the tile DMA (also inline asm, so untracked too): the
// compiler would otherwise wait for them with vmcnt(0), i.e. for every DMA
// issued after them.  Their completion is awaited with lk_wait_vm_tie, which
// takes the loaded registers as operands, so no use can move above it.
__device__ __forceinline__ lk_f4 lk_ld16_untracked(const void * p) {
    lk_f4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
template <int N>
__device__ __forceinline__ void lk_wait_vm_tie(lk_f4 (&a)[4]) {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]) : "n"(N));
}

// ---- host-side error plumbing (lk_host.cpp) -----------------------------------
int lk_fail(int code, const char * fmt, ...);
// hipGetLastError after a launch, mapped into lk_fail.
int lk_launch_status(const char * what);
static inline hipStream_t lk_stream(void * s) { return (hipStream_t) s; }
// Devices whose per-device scratch addresses the host side caches.
#define LK_MAX_DEVICES 64
