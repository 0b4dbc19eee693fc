/* Host check of the Q8_1 rounding shortcut used by the prefill attention's
 * Q8_1 epilogue (lk_q81_div / lk_q81_qd in prefill.hip): with d = am/127 and
 * |x| <= am, roundf applied to the two-fma corrected quotient must equal
 * roundf(x / d), and the corrected quotient must be x / d bit for bit
 * whenever x / d is a normal number.  Compiled with -ffp-contract=off so that
 * every product and fma is as written.  Usage: q81_div_check N SEED; prints
 * "n <pairs> quotient_mismatches <k> round_mismatches <k>". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t s;
static uint64_t xr(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
static float uf(void) { return (float) ((xr() >> 11) * (1.0 / 9007199254740992.0)); }
static float nudge(float x, int k) { uint32_t b; memcpy(&b, &x, 4); b += (uint32_t) k; memcpy(&x, &b, 4); return x; }

int main(int argc, char ** argv) {
    long N = argc > 1 ? atol(argv[1]) : 10000000L;
    s = argc > 2 ? strtoull(argv[2], 0, 10) : 88172645463325252ull;
    long n = 0, badq = 0, badr = 0;
    for (long it = 0; it < N; ++it) {
        const float am = ldexpf(1.0f + uf(), (int) (xr() % 240) - 140);
        const volatile float d = am / 127.0f;
        float x;
        const int mode = (int) (xr() % 4), k = (int) (xr() % 255) - 127;
        if (mode == 0) x = (uf() * 2 - 1) * am;                           /* anywhere in the block range */
        else if (mode == 1) x = nudge((k + 0.5f) * d, (int) (xr() % 5) - 2);  /* next to a rounding tie */
        else if (mode == 2) x = (xr() & 1) ? am : -am;                     /* the block maximum */
        else x = nudge(k * d, (int) (xr() % 3) - 1);                        /* next to an integer */
        if (isnan(x) || fabsf(x) > am) continue;
        const volatile float ref = x / d;
        /* the kernel's arithmetic */
        const float sc = am < 0x1p-64f ? 0x1p64f : 1.0f;
        const volatile float ds = (am == 0.0f) ? 1.0f : d * sc;
        const volatile float r = 1.0f / ds;
        const volatile float xs = x * sc;
        const volatile float q0 = xs * r;
        const volatile float e = fmaf(-q0, ds, xs);
        const volatile float q1 = fmaf(e, r, q0);
        ++n;
        if (fabsf(ref) >= 0x1p-126f && memcmp((const void *) &ref, (const void *) &q1, 4)) ++badq;
        if (roundf(ref) != roundf(q1)) ++badr;
    }
    printf("n %ld quotient_mismatches %ld round_mismatches %ld\n", n, badq, badr);
    return 0;
}
