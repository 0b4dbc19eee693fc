// lk_oracle.cpp - CPU restatement of the lfm2-ampere attention hot path.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
// calls this file: only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg use it, and only as the checker (or as the timed CPU
// baseline), never as the thing measured or shipped.
//
// Every function cites the reference file:line it restates (paths relative to
// the lfm2-ampere repository).  Built with -ffp-contract=off and without
// -ffast-math, so every fp32 expression rounds exactly as written.
//
// Pinning (what checks each function against something other than itself) is
// listed in tests/test_oracle.py; a function with no such check would be
// marked "parity unpinned" here.  None is.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <vector>
#include <random>
#include <algorithm>
#include <omp.h>

#define LKO_H   32
#define LKO_KV  8
#define LKO_D   64
#define LKO_G   (LKO_H / LKO_KV)

extern "C" {

// ---------------------------------------------------------------------------
// IEEE binary16 <-> binary32.  h2f is exact; f2h rounds to nearest even, the
// rounding of __float2half / __floats2half2_rn (reference quant.cuh:119).
float lko_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {                               // subnormal: m * 2^-24, exact in fp32
            float f = (float) m * 5.9604644775390625e-08f;
            std::memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f; std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t lko_f2h(float f) {
    uint32_t x; std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)                               // inf / nan
        return sign | 0x7c00 | (ax > 0x7f800000u ? 0x200 : 0);
    if (ax >= 0x477ff000u) return sign | 0x7c00;         // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {                              // below 2^-14: subnormal half
        // value / 2^-24, rounded to nearest even integer (exact arithmetic in double)
        double v; float af; std::memcpy(&af, &ax, 4); v = (double) af / 5.9604644775390625e-08;
        double r = std::nearbyint(v);                    // default mode is RNE
        return sign | (uint16_t) r;                      // r <= 1024 (1024 = smallest normal)
    }
    // normal: keep 10 mantissa bits, RNE on the 13 dropped bits
    uint32_t e = (ax >> 23) - 112;
    uint32_t m = ax & 0x7fffff;
    uint32_t h = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h += 1;   // may carry into exponent: correct
    return sign | (uint16_t) h;
}

void lko_h2f_n(const uint16_t * h, float * f, size_t n) { for (size_t i = 0; i < n; ++i) f[i] = lko_h2f(h[i]); }
void lko_f2h_n(const float * f, uint16_t * h, size_t n) { for (size_t i = 0; i < n; ++i) h[i] = lko_f2h(f[i]); }

// ---------------------------------------------------------------------------
// Split-K slice rule (reference kernels.cuh:630-635, and the chunk/t0/t1
// derivation at kernels.cu:1324-1333): slices = clamp(ceil(seq/target_n),
// split_min, split_cap); chunk = ceil(seq / slices).
void lko_attn_slices(int seq, int split_cap, int target_n, int split_min,
                     int * nslices, int * chunk) {
    int s = (seq + target_n - 1) / target_n;
    if (s < split_min) s = split_min;
    if (s > split_cap) s = split_cap;
    *nslices = s;
    *chunk = (seq + s - 1) / s;
}

// ---------------------------------------------------------------------------
// Float64 decode attention (reference tests/test_attn.cu:46-74): for each of
// the 32 query heads, softmax(q . K^T * 1/8) . V over positions [0, seq) of
// the fp16 cache kc/vc [.][8][64].  q: fp32 [32][64].  out: double [32][64].
void lko_decode_ref(const float * q, const uint16_t * kc, const uint16_t * vc,
                    int seq, double * out) {
    // heads are independent: one per OpenMP iteration, each with its own score
    // row (the result does not depend on the thread count)
#pragma omp parallel for schedule(static)
    for (int head = 0; head < LKO_H; ++head) {
        std::vector<double> s(seq > 0 ? seq : 1);
        const int kv = head / LKO_G;
        double m = -1e300;
        for (int t = 0; t < seq; ++t) {
            const uint16_t * k = kc + ((size_t) t * LKO_KV + kv) * LKO_D;
            double a = 0.0;
            for (int d = 0; d < LKO_D; ++d) a += (double) q[head * LKO_D + d] * (double) lko_h2f(k[d]);
            a *= 0.125;
            s[t] = a;
            if (a > m) m = a;
        }
        double l = 0.0;
        for (int t = 0; t < seq; ++t) { s[t] = std::exp(s[t] - m); l += s[t]; }
        for (int d = 0; d < LKO_D; ++d) {
            double a = 0.0;
            for (int t = 0; t < seq; ++t)
                a += s[t] * (double) lko_h2f(vc[((size_t) t * LKO_KV + kv) * LKO_D + d]);
            out[head * LKO_D + d] = a / l;
        }
    }
}

// ---------------------------------------------------------------------------
// Q8_1 quantisation of 32 fp32 values (reference quant.cuh:106-121, the
// decode combine epilogue at kernels.cu:1598): am = max|x| (exact); sum = the
// xor-butterfly 16,8,4,2,1 in fp32 as lane 0 sees it; d = am/127;
// q = am == 0 ? 0 : roundf(x/d) (half away from zero); ds = (fp16 RNE d,
// fp16 RNE sum).  y: 36 bytes, layout of lk_block_q8_1.
void lko_quantize_q8_1(const float * x, uint8_t * y) {
    float am = 0.0f;
    for (int i = 0; i < 32; ++i) am = std::max(am, std::fabs(x[i]));
    float s[32];
    for (int i = 0; i < 32; ++i) s[i] = x[i];
    for (int o = 16; o > 0; o >>= 1) {
        float t[32];
        for (int i = 0; i < 32; ++i) t[i] = s[i] + s[i ^ o];
        std::memcpy(s, t, sizeof s);
    }
    const float d = am / 127.0f;
    const uint16_t dh = lko_f2h(d), sh = lko_f2h(s[0]);
    std::memcpy(y, &dh, 2);
    std::memcpy(y + 2, &sh, 2);
    for (int i = 0; i < 32; ++i) {
        const int8_t qv = (am == 0.0f) ? (int8_t) 0 : (int8_t) std::roundf(x[i] / d);
        y[4 + i] = (uint8_t) qv;
    }
}

// ---------------------------------------------------------------------------
// One 64-wide absmax int8 row (reference prefill.cu:1255-1267):
// am = max|v| (exact); d = am/127.0f; id = am > 0 ? 127.0f/am : 0;
// q = round-to-nearest-even(v * id) (|v*id| <= 127 so it never saturates);
// scale = d * mul.
void lko_q8_row(const float * v, int8_t * dst, float * scale, float mul) {
    float am = 0.0f;
    for (int d = 0; d < LKO_D; ++d) am = std::max(am, std::fabs(v[d]));
    const float dd = am / 127.0f;
    const float id = (am > 0.0f) ? 127.0f / am : 0.0f;
    for (int d = 0; d < LKO_D; ++d) {
        const float p = v[d] * id;
        dst[d] = (int8_t) (int) std::nearbyintf(p);     // default rounding mode: RNE
    }
    *scale = dd * mul;
}

static const float LKO_L2E = 1.4426950408889634f;

// q.c in the reference's order (prefill.cu:1279-1284): the row is held by a
// 32-lane warp, two values per lane, so lane l first forms the pair sum
// v[2l]*c[2l] + v[2l+1]*c[2l+1] (each product rounded, then the add: the
// source text, read without contraction -- nvcc's default -fmad=true may fuse
// one of the products into an fma, a difference of at most one rounding of
// the pair), then the xor butterfly over lanes with offsets 16, 8, 4, 2, 1;
// lane 0's value is returned.
static float lko_qc_ref(const float * v, const float * c) {
    float s[32];
    for (int l = 0; l < 32; ++l) {
        const float a = v[2 * l] * c[2 * l];
        const float b = v[2 * l + 1] * c[2 * l + 1];
        s[l] = a + b;
    }
    for (int o = 16; o > 0; o >>= 1) {
        float t[32];
        for (int l = 0; l < 32; ++l) t[l] = s[l] + s[l ^ o];
        std::memcpy(s, t, sizeof s);
    }
    return s[0];
}

// Q quantiser (reference prefill.cu:1271-1287): every (token, head) row of qh
// fp16 [m][2048] -> q8 int8 [m][2048], qsc [m][32] = d * log2(e),
// qcs [m][32] = (q . c) * log2(e) with c = cm[head/4] (0 without cm), q.c
// summed by lko_qc_ref.
void lko_pf_q8(const uint16_t * qh, int m, const float * cm,
               int8_t * q8, float * qsc, float * qcs) {
    float v[LKO_D];
    for (int r = 0; r < m * LKO_H; ++r) {
        for (int d = 0; d < LKO_D; ++d) v[d] = lko_h2f(qh[(size_t) r * LKO_D + d]);
        lko_q8_row(v, q8 + (size_t) r * LKO_D, qsc + r, LKO_L2E);
        float qc = 0.0f;
        if (cm) qc = lko_qc_ref(v, cm + ((r % LKO_H) / LKO_G) * LKO_D);
        qcs[r] = qc * LKO_L2E;
    }
}

// K quantiser (reference prefill.cu:1291-1301): positions [p0, p1) of kc fp16
// [pos][8][64] -> k8 (same layout) and ksc[h * kstride + pos] = d; with cm,
// the head's mean is subtracted first (fp32).
void lko_pf_k8(const uint16_t * kc, int p0, int p1, const float * cm, int kstride,
               int8_t * k8, float * ksc) {
    float v[LKO_D];
    for (int pos = p0; pos < p1; ++pos)
        for (int h = 0; h < LKO_KV; ++h) {
            const size_t row = (size_t) pos * LKO_KV + h;
            for (int d = 0; d < LKO_D; ++d) {
                v[d] = lko_h2f(kc[row * LKO_D + d]);
                if (cm) v[d] -= cm[h * LKO_D + d];
            }
            lko_q8_row(v, k8 + row * LKO_D, ksc + (size_t) h * kstride + pos, 1.0f);
        }
}

// K smoothing mean (reference prefill.cu:1304-1318): cm[h][d] = (sum of 16
// strided partials, each an fp32 running sum over p = g, g+16, ...) / n.
void lko_pf_kmean(const uint16_t * kc, int n, float * cm) {
    for (int h = 0; h < LKO_KV; ++h)
        for (int d = 0; d < LKO_D; ++d) {
            float part[16];
            for (int g = 0; g < 16; ++g) {
                float s = 0.0f;
                for (int p = g; p < n; p += 16) s += lko_h2f(kc[((size_t) p * LKO_KV + h) * LKO_D + d]);
                part[g] = s;
            }
            float t = 0.0f;
            for (int i = 0; i < 16; ++i) t += part[i];
            cm[h * LKO_D + d] = t / (float) n;
        }
}

// Exact-tile predicate of the int8 attention (reference prefill.cu:1380-1382):
// key tile kt (64 keys) is scored in fp16 for query tile qt (32 queries) iff
// kt*64 + 64 > P + qt*32 - near, or sink and kt == 0.
int lko_pf_exact(int P, int qt, int kt, int near, int sink) {
    const int near_lo = P + qt * 32 - near;
    return (kt * 64 + 64 > near_lo) || (sink && kt == 0);
}

// Float64 causal prefill attention (reference tests/test_prefill.cu:263-282):
// qh fp16 [m][2048] already carries 1/8; query t sits at position P + t and
// sees keys [0, P + t].  rows: the query rows to compute (NULL = all m),
// nrows entries; o: double [m][2048] (rows not listed are left untouched).
void lko_pf_ref(const uint16_t * qh, int m, int P, const uint16_t * kc, const uint16_t * vc,
                const int * rows, int nrows, double * o) {
    const int S = P + m;
    const int nr = rows ? nrows : m;
    // (row, head) pairs are independent: one per OpenMP iteration
#pragma omp parallel for schedule(dynamic, 1)
    for (long it = 0; it < (long) nr * LKO_H; ++it) {
        std::vector<double> sc(S), qd(LKO_D);
        const int ri = (int) (it / LKO_H), h = (int) (it % LKO_H);
        const int t = rows ? rows[ri] : ri;
        {
            const int kvh = h / LKO_G, qp = P + t;
            for (int d = 0; d < LKO_D; ++d) qd[d] = lko_h2f(qh[(size_t) t * 2048 + h * 64 + d]);
            double mx = -1e300;
            for (int j = 0; j <= qp; ++j) {
                double s = 0.0;
                const uint16_t * k = kc + ((size_t) j * 8 + kvh) * 64;
                for (int d = 0; d < LKO_D; ++d) s += qd[d] * (double) lko_h2f(k[d]);
                sc[j] = s; mx = std::max(mx, s);
            }
            double l = 0.0;
            for (int j = 0; j <= qp; ++j) { sc[j] = std::exp(sc[j] - mx); l += sc[j]; }
            for (int d = 0; d < LKO_D; ++d) {
                double r = 0.0;
                for (int j = 0; j <= qp; ++j) r += sc[j] * (double) lko_h2f(vc[((size_t) j * 8 + kvh) * 64 + d]);
                o[(size_t) t * 2048 + h * 64 + d] = r / l;
            }
        }
    }
}

// Float64 restatement of the int8-score attention's ALGORITHM (reference
// prefill.cu:1337-1571): the same scores, the same tile classification, the
// same log2-domain softmax, evaluated exactly.  Per (query t, key j):
//   exact tile (lko_pf_exact with qt = t/32, kt = j/64):
//       s = (sum_d qh.kc) * log2e - qcs[t][h]            (prefill.cu:1435-1468)
//   int8 tile:
//       s = (double) sumi * ksc[kvh][j] * qsc[t][h]      (prefill.cu:1469-1492)
//       sumi = sum_d q8[t][h][d] * k8[j][kvh][d]         (exact integer)
//   out = sum_j 2^(s_j - max) v_j / sum_j 2^(s_j - max)  over j <= P + t.
// The only differences from the HIP kernel are the kernel's own roundings
// (fp32 accumulation, fp16 P, hardware exp2), which the tolerance covers.
void lko_pf_ref8(const int8_t * q8, const float * qsc, const float * qcs, const uint16_t * qh,
                 int m, int P, const int8_t * k8, const float * ksc, int kstride,
                 const uint16_t * kc, const uint16_t * vc, int near, int sink,
                 const int * rows, int nrows, double * o) {
    const int S = P + m;
    const int nr = rows ? nrows : m;
    // (row, head) pairs are independent: one per OpenMP iteration
#pragma omp parallel for schedule(dynamic, 1)
    for (long it = 0; it < (long) nr * LKO_H; ++it) {
        std::vector<double> sc(S), qd(LKO_D);
        const int ri = (int) (it / LKO_H), h = (int) (it % LKO_H);
        const int t = rows ? rows[ri] : ri;
        const int qt = t / 32;
        {
            const int kvh = h / LKO_G, qp = P + t;
            for (int d = 0; d < LKO_D; ++d) qd[d] = lko_h2f(qh[(size_t) t * 2048 + h * 64 + d]);
            const int8_t * qi = q8 + (size_t) t * 2048 + h * 64;
            const double sq = qsc[(size_t) t * 32 + h];
            const double qc = qcs ? qcs[(size_t) t * 32 + h] : 0.0;
            double mx = -1e300;
            for (int j = 0; j <= qp; ++j) {
                double s;
                if (lko_pf_exact(P, qt, j / 64, near, sink)) {
                    const uint16_t * k = kc + ((size_t) j * 8 + kvh) * 64;
                    double a = 0.0;
                    for (int d = 0; d < LKO_D; ++d) a += qd[d] * (double) lko_h2f(k[d]);
                    s = a * (double) LKO_L2E - qc;
                } else {
                    const int8_t * k = k8 + ((size_t) j * 8 + kvh) * 64;
                    long sumi = 0;
                    for (int d = 0; d < LKO_D; ++d) sumi += (long) qi[d] * (long) k[d];
                    s = (double) sumi * (double) ksc[(size_t) kvh * kstride + j] * sq;
                }
                sc[j] = s; mx = std::max(mx, s);
            }
            double l = 0.0;
            for (int j = 0; j <= qp; ++j) { sc[j] = std::exp2(sc[j] - mx); l += sc[j]; }
            for (int d = 0; d < LKO_D; ++d) {
                double r = 0.0;
                for (int j = 0; j <= qp; ++j) r += sc[j] * (double) lko_h2f(vc[((size_t) j * 8 + kvh) * 64 + d]);
                o[(size_t) t * 2048 + h * 64 + d] = r / l;
            }
        }
    }
}

// Threads of the float64 references (decode_ref, pf_ref, pf_ref8); n <= 0
// leaves OpenMP's default (OMP_NUM_THREADS).  Returns the count in effect.
int lko_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

// Raw int32 Q.K^T sums: s[h][i][j] = sum_d q8[i][h][d] * k8[j][h/4][d].
void lko_qk_i32(const int8_t * q8, int m, const int8_t * k8, int n, int32_t * s) {
    for (int h = 0; h < LKO_H; ++h)
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j) {
                int32_t a = 0;
                const int8_t * qi = q8 + (size_t) i * 2048 + h * 64;
                const int8_t * kj = k8 + ((size_t) j * 8 + h / 4) * 64;
                for (int d = 0; d < LKO_D; ++d) a += (int32_t) qi[d] * (int32_t) kj[d];
                s[((size_t) h * m + i) * n + j] = a;
            }
}

// ---------------------------------------------------------------------------
// Seeded generators.
//
// (1) tests/test_attn.cu:35-40,89-98: xorshift64 from 0x9e3779b97f4a7c15,
//     urand = top 53 bits / 2^53, nrand = 2*urand - 1 (uniform in [-1, 1),
//     despite the name).  One case fills q (32*64, x1.5) and then the WHOLE
//     131072-position K and V caches, interleaved k, v per element.  The
//     generator state carries from case to case, as in the reference main().
void lko_xs_fill_attn_case(uint64_t * state, size_t cache_elems,
                           float * q, uint16_t * kc, uint16_t * vc) {
    uint64_t s = *state;
    auto urand = [&]() {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        return (double)((s >> 11) & ((1ull << 53) - 1)) / (double)(1ull << 53);
    };
    for (int i = 0; i < LKO_H * LKO_D; ++i) q[i] = (float)(urand() * 2.0 - 1.0) * 1.5f;
    for (size_t i = 0; i < cache_elems; ++i) {
        kc[i] = lko_f2h((float)(urand() * 2.0 - 1.0));
        vc[i] = lko_f2h((float)(urand() * 2.0 - 1.0));
    }
    *state = s;
}

// (2) BASELINE configs: splitmix64 + Box-Muller (implementation-independent).
static inline uint64_t lko_sm64(uint64_t & x) {
    uint64_t z = (x += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static inline double lko_u01(uint64_t & x) {            // (0, 1]
    return ((double)(lko_sm64(x) >> 11) + 1.0) / 9007199254740992.0;
}
// The raw stream: out[k] = draw k + 1 (known answers: seed 1234567 gives
// 6457827717110365317, 3203168211198807973, 9817491932198370423, ...).
void lko_sm64_n(uint64_t seed, uint64_t * out, size_t n) {
    uint64_t x = seed;
    for (size_t i = 0; i < n; ++i) out[i] = lko_sm64(x);
}
// n values N(0,1) in fp32 (Box-Muller, both outputs used).
void lko_sm_normal(uint64_t seed, float * out, size_t n) {
    uint64_t x = seed;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = lko_u01(x), u2 = lko_u01(x);
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = (float)(r * std::cos(2.0 * M_PI * u2));
        if (i + 1 < n) out[i + 1] = (float)(r * std::sin(2.0 * M_PI * u2));
    }
}
void lko_sm_uniform(uint64_t seed, float * out, size_t n, float lo, float hi) {
    uint64_t x = seed;
    for (size_t i = 0; i < n; ++i) out[i] = lo + (hi - lo) * (float) lko_u01(x);
}
// Student-t with nu = 4: z / sqrt(chi2_4 / 4), chi2_4 = sum of 4 squared N(0,1).
void lko_sm_student4(uint64_t seed, float * out, size_t n) {
    uint64_t x = seed;
    auto nrm = [&]() {
        const double u1 = lko_u01(x), u2 = lko_u01(x);
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2);
    };
    for (size_t i = 0; i < n; ++i) {
        const double z = nrm();
        double c = 0.0;
        for (int k = 0; k < 4; ++k) { const double g = nrm(); c += g * g; }
        out[i] = (float)(z / std::sqrt(c / 4.0));
    }
}

// (3) tests/test_prefill.cu:36,250-256,296-309: std::mt19937 with
//     std::normal_distribution<float>(0,1) and uniform_int_distribution(-127,127)
//     (libstdc++), drawn in the reference's order for ONE case: the 512
//     per-channel key offsets N*koff (only when with_off: attn8_err draws
//     them, test_attn does not), then K = N*1.5 + off[i % 512], V = N,
//     Q = N*1.5*0.125 (all fp16), then, when koff < 0, the lossless int8 grid
//     that overwrites K and Q.
void lko_mt_prefill_case(uint32_t seed, int m, int P, float koff, int with_off,
                         uint16_t * K, uint16_t * V, uint16_t * Q) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    const int S = P + m;
    std::vector<float> off(512, 0.0f);
    if (with_off) for (auto & x : off) x = nd(rng) * koff;
    const size_t nk = (size_t) S * 512, nq = (size_t) m * 2048;
    for (size_t i = 0; i < nk; ++i) K[i] = lko_f2h(nd(rng) * 1.5f + off[i % 512]);
    for (size_t i = 0; i < nk; ++i) V[i] = lko_f2h(nd(rng));
    for (size_t i = 0; i < nq; ++i) Q[i] = lko_f2h(nd(rng) * 1.5f * 0.125f);
    if (koff < 0.0f) {
        std::uniform_int_distribution<int> ui(-127, 127);
        for (size_t r = 0; r < nk / 64; ++r)
            for (int d = 0; d < 64; ++d) K[r * 64 + d] = lko_f2h((d == 0 ? 127 : ui(rng)) / 32.0f);
        for (size_t r = 0; r < nq / 64; ++r)
            for (int d = 0; d < 64; ++d) Q[r * 64 + d] = lko_f2h((d == 0 ? 127 : ui(rng)) / 1024.0f);
    }
}

// Planar Q8_1 of fp32 rows (reference k_pf_quant_rows, prefill.cu:1574-1580,
// with pf_quant_warp, prefill.cu:90-103): per 32-value block the arithmetic of
// lko_quantize_q8_1 (exact max, xor-butterfly sum 16..1, d = am/127, q =
// roundf(x/d)); planes qs int8 [rows][kb*32], sc [rows][kb][2] =
// (float(fp16(d)), 8 * float(fp16(sum))).
void lko_pf_quant_rows(const float * X, int rows, int ld, int kb, int8_t * qs, float * sc) {
    uint8_t blk[36];
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < kb; ++b) {
            lko_quantize_q8_1(X + (size_t) r * ld + b * 32, blk);
            std::memcpy(qs + ((size_t) r * kb + b) * 32, blk + 4, 32);
            uint16_t dh, sh;
            std::memcpy(&dh, blk, 2);
            std::memcpy(&sh, blk + 2, 2);
            sc[((size_t) r * kb + b) * 2]     = lko_h2f(dh);
            sc[((size_t) r * kb + b) * 2 + 1] = 8.0f * lko_h2f(sh);
        }
}

// ---------------------------------------------------------------------------
// Attention-input producers: per-head RMS norm + NEOX rotary embedding of one
// 64-wide row (reference kernels.cu:886-910 and prefill.cu:989-1009, identical
// arithmetic in both): ss = sum v^2 by the kernels' tree (d with d+32, then
// +16, ..., +1), inv = 1/sqrt(ss/64 + 1e-5), y = (v*inv)*w, angle a_i =
// (float)pos * theta^(-i/32) in fp32, then y_i c - y_{i+32} s and
// y_i s + y_{i+32} c.  The reference evaluates rsqrtf / powf / sincosf with
// CUDA's approximations; this restatement uses the correctly rounded fp32
// values of 1/sqrt, theta^(-i/32), cos and sin (computed in double, rounded
// once), the arithmetic the MI355X kernel implements.
void lko_norm_rope_row(const float * v, const float * w, int pos, float * out) {
    float a[64];
    for (int d = 0; d < 64; ++d) a[d] = v[d] * v[d];
    for (int o = 32; o > 0; o >>= 1)
        for (int d = 0; d < o; ++d) a[d] = a[d] + a[d + o];
    const float arg = a[0] * (1.0f / 64.0f) + 1e-5f;
    const float inv = (float) (1.0 / std::sqrt((double) arg));
    float y[64];
    for (int d = 0; d < 64; ++d) y[d] = (v[d] * inv) * w[d];
    for (int i = 0; i < 32; ++i) {
        const float f = (float) std::pow(10000000.0, -(double) i / 32.0);
        const float ang = (float) pos * f;
        const float c = (float) std::cos((double) ang), s = (float) std::sin((double) ang);
        const float x0 = y[i], x1 = y[i + 32];
        out[i]      = x0 * c - x1 * s;
        out[i + 32] = x0 * s + x1 * c;
    }
}

// k_qk_norm_rope (kernels.cu:871-915): qf [32][64], kf [8][64] in place; K and
// V rows (fp16) into kc / vc row pos ([pos][8][64]).
void lko_qk_norm_rope(float * qf, float * kf, const float * vf, const float * qn, const float * kn,
                      int pos, uint16_t * kc, uint16_t * vc) {
    float out[64];
    for (int h = 0; h < LKO_H; ++h) {
        lko_norm_rope_row(qf + h * 64, qn, pos, out);
        std::memcpy(qf + h * 64, out, sizeof out);
    }
    for (int h = 0; h < LKO_KV; ++h) {
        lko_norm_rope_row(kf + h * 64, kn, pos, out);
        std::memcpy(kf + h * 64, out, sizeof out);
        const size_t off = ((size_t) pos * LKO_KV + h) * 64;
        for (int d = 0; d < 64; ++d) {
            kc[off + d] = lko_f2h(out[d]);
            vc[off + d] = lko_f2h(vf[h * 64 + d]);
        }
    }
}

// k_pf_qknr (prefill.cu:975-1016): Y [m][3072] -> qh [m][2048] = fp16(q_rot *
// 1/8), K/V rows P+t of kc / vc.
void lko_pf_qknr(const float * Y, const float * qn, const float * kn, int m, int P,
                 uint16_t * qh, uint16_t * kc, uint16_t * vc) {
    float out[64];
    for (int t = 0; t < m; ++t) {
        const float * y = Y + (size_t) t * 3072;
        for (int h = 0; h < LKO_H; ++h) {
            lko_norm_rope_row(y + h * 64, qn, P + t, out);
            for (int d = 0; d < 64; ++d) qh[(size_t) t * 2048 + h * 64 + d] = lko_f2h(out[d] * 0.125f);
        }
        for (int h = 0; h < LKO_KV; ++h) {
            lko_norm_rope_row(y + 2048 + h * 64, kn, P + t, out);
            const size_t off = ((size_t) (P + t) * LKO_KV + h) * 64;
            for (int d = 0; d < 64; ++d) {
                kc[off + d] = lko_f2h(out[d]);
                vc[off + d] = lko_f2h(y[2560 + h * 64 + d]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Q4_0 x Q8_1 block dot (reference quant.cuh:131-158): sumi = exact int sum of
// nibble * q8 over the 32 elements (byte j of the 16-byte weight block holds
// element j in its low nibble and element 16+j in its high nibble; nibbles are
// 0..15, the -8 offset is carried by the activation sum); d4 = fp16 weight
// scale; (d8, sum8) = the activation block's fp16 ds;
// result = d4 * (d8 * (float) sumi - 8 * sum8), in fp32 as written.
float lko_dot_q4_0_q8_1(const uint8_t * qs16, uint16_t d, const uint8_t * xq36) {
    uint16_t dh, sh;
    std::memcpy(&dh, xq36, 2);
    std::memcpy(&sh, xq36 + 2, 2);
    const int8_t * q8 = (const int8_t *) (xq36 + 4);
    int sumi = 0;
    for (int j = 0; j < 16; ++j) {
        sumi += (int) (qs16[j] & 0x0F) * (int) q8[j];
        sumi += (int) (qs16[j] >> 4) * (int) q8[16 + j];
    }
    const float d4 = lko_h2f(d), d8 = lko_h2f(dh), s8 = lko_h2f(sh);
    const float t = d8 * (float) sumi;
    const float u = 8.0f * s8;
    return d4 * (t - u);
}

// Q4_0 GEMV (reference k_gemv_q4_0, kernels.cu:300-306, body kernels.cu:190-260
// with LK_GEMV_ROWS = 1): row r is one 32-lane warp; lane l sums blocks
// k = l, l+32, ... in order (fp32); warp_sum's xor-butterfly 16, 8, 4, 2, 1
// (kernels.cuh:28-32) as lane 0 sees it; times ninv = 1/sqrt(s/2048 + eps)
// when ssq is given, s = the same butterfly over ssq[l] + ssq[l+32]
// (lk_norm_inv, kernels.cuh:441-447; evaluated in fp64 and rounded once, where
// the reference uses the CUDA approximation rsqrtf); y[r] = add ? y[r] + a : a.
static float lko_warp_sum32(const float * v) {
    float s[32];
    for (int i = 0; i < 32; ++i) s[i] = v[i];
    for (int o = 16; o > 0; o >>= 1) {
        float t[32];
        for (int i = 0; i < 32; ++i) t[i] = s[i] + s[i ^ o];
        std::memcpy(s, t, sizeof s);
    }
    return s[0];
}

void lko_gemv_q4_0(const uint8_t * qs, const uint16_t * d, const uint8_t * xq, int rows, int bpr,
                   const float * ssq, float eps, float * y, int add) {
    float ninv = 1.0f;
    if (ssq) {
        float v[32];
        for (int l = 0; l < 32; ++l) v[l] = ssq[l] + ssq[l + 32];
        const float s = lko_warp_sum32(v);
        ninv = (float) (1.0 / std::sqrt((double) (s * (1.0f / 2048.0f) + eps)));
    }
    for (int r = 0; r < rows; ++r) {
        float acc[32];
        for (int l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (int k = l; k < bpr; k += 32) {
                const size_t b = (size_t) r * bpr + k;
                a = a + lko_dot_q4_0_q8_1(qs + 16 * b, d[b], xq + 36 * (size_t) k);
            }
            acc[l] = a;
        }
        float a = lko_warp_sum32(acc);
        if (ssq) a = a * ninv;
        y[r] = add ? y[r] + a : a;
    }
}

// ---------------------------------------------------------------------------
// Q4_0 x planar Q8_1 GEMM, dense, plain epilogue (reference k_pf_mmq EPI 0 with
// PF_EPI2, prefill.cu:131-141, 330-390, 470-490; pf_gemm_dense prefill.cu:818-826):
// for token t and row r, over the blocks b in order: F = 1.5*2^23 + sumi
// (exact), c = fma(d8, 1.5*2^23, s8), acc = fma(d4, fma(d8, F, -c), acc), with
// (d8, s8) = asc[t][b] (s8 = 8 * fp16 sum) and d4 = d[r][b]; then
// a = acc * scale[t] (1 without scale) and out[t][r] = add ? out[t][r] + a : a.
// qs [N][bpr][16], d fp16 [N][bpr], aqs int8 [ntok][bpr * 32], asc [ntok][bpr][2].
void lko_pf_gemm_q4_0(const uint8_t * qs, const uint16_t * d, int N, int bpr, const int8_t * aqs,
                      const float * asc, int ntok, const float * scale, float * out, int out_ld, int add) {
    const float M = 12582912.0f;
    for (int t = 0; t < ntok; ++t)
        for (int r = 0; r < N; ++r) {
            float acc = 0.0f;
            for (int b = 0; b < bpr; ++b) {
                const uint8_t * q = qs + ((size_t) r * bpr + b) * 16;
                const int8_t * x = aqs + (size_t) t * bpr * 32 + (size_t) b * 32;
                int sumi = 0;
                for (int j = 0; j < 16; ++j) sumi += (int) (q[j] & 0x0F) * x[j] + (int) (q[j] >> 4) * x[16 + j];
                const float F = M + (float) sumi;                 // exact: |sumi| < 2^22
                const float d8 = asc[((size_t) t * bpr + b) * 2], s8 = asc[((size_t) t * bpr + b) * 2 + 1];
                const float c = std::fmaf(d8, M, s8);
                acc = std::fmaf(lko_h2f(d[(size_t) r * bpr + b]), std::fmaf(d8, F, -c), acc);
            }
            const float a = acc * (scale ? scale[t] : 1.0f);
            float & o = out[(size_t) t * out_ld + r];
            o = add ? o + a : a;
        }
}

// max |a - b| / max |b| over n values (b is the reference).
double lko_rel_err(const float * a, const double * b, size_t n) {
    double e = 0.0, r = 0.0;
    for (size_t i = 0; i < n; ++i) {
        e = std::max(e, std::fabs((double) a[i] - b[i]));
        r = std::max(r, std::fabs(b[i]));
    }
    return r > 0.0 ? e / r : e;
}

}  // extern "C"
