/*
 * fused_cases.c -- inputs on which the candidate forms of torch's fused=True AdamW chain
 * round apart (test fixture generator, CPU only).
 *
 * torch._fused_adamw_ (ATen/native/hip/fused_adam_utils.cuh adam_math) forms the
 * moments in float64 from fp32 values and rounds them once to fp32:
 *     m = f32(beta1*m + (1-beta1)*g),  v = f32(beta2*v + ((1-beta2)*g)*g).
 * Whether the compiler that built it fused each sum's left product, its right product,
 * or neither into one fused multiply-add changes the fp32 result only when the float64
 * value lies within an ulp of a float64 of an fp32 rounding boundary: about one input in
 * 2^29.  This program draws seeded random (m, g) and (v, g) pairs (the value ranges of
 * mid-training state) at beta1 = 0.9, beta2 = 0.95 and prints, for each pair of
 * candidate forms, the first 24 inputs on which those two round apart, as
 *     m<a><b> <m hex> <g hex>      or      v<a><b> <v hex> <g hex>
 * with forms 0 (no fma), 1 (left product fused), 2 (right product fused).
 * make_fused_golden.py runs torch's kernel on them on a GPU; the results select the
 * form.
 *
 *   gcc -O2 -ffp-contract=off tests/golden/fused_cases.c -lm -o /tmp/fused_cases
 *   /tmp/fused_cases > tests/golden/fused_cases.txt
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>

static uint64_t s = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { s ^= s << 13; s ^= s >> 7; s ^= s << 17; return s; }
static double unif(void) { return (rnd() >> 11) * (1.0 / 9007199254740992.0); }
static float gauss(float sd)
{
    double u1 = unif() + 1e-300, u2 = unif();
    return (float)(sd * sqrt(-2 * log(u1)) * cos(6.283185307179586 * u2));
}

enum { WANT = 24 };

int main(void)
{
    const double b1 = 0.9, b2 = 0.95, omb1 = 1.0 - b1, omb2 = 1.0 - b2;
    int nm[3] = {0, 0, 0}, nv[3] = {0, 0, 0};
    static const char *pair[3] = {"01", "02", "12"};
    for (long it = 0; it < 4000000000L; ++it) {
        float p = gauss(0.02f), g = gauss(1e-3f), m = gauss(1e-3f), v = fabsf(gauss(1e-6f));
        (void)p;   /* drawn to keep the sequence of the search this file records */
        {
            const double pm = b1 * (double)m, pg = omb1 * (double)g;
            const float c[3] = {(float)(pm + pg), (float)fma(b1, (double)m, pg),
                                (float)fma(omb1, (double)g, pm)};
            const int d[3] = {c[0] != c[1], c[0] != c[2], c[1] != c[2]};
            for (int k = 0; k < 3; ++k)
                if (d[k] && nm[k] < WANT) { printf("m%s %a %a\n", pair[k], m, g); ++nm[k]; }
        }
        {
            const double pv = b2 * (double)v, q = (omb2 * (double)g) * (double)g;
            const float c[3] = {(float)(pv + q), (float)fma(b2, (double)v, q),
                                (float)fma(omb2 * (double)g, (double)g, pv)};
            const int d[3] = {c[0] != c[1], c[0] != c[2], c[1] != c[2]};
            for (int k = 0; k < 3; ++k)
                if (d[k] && nv[k] < WANT) { printf("v%s %a %a\n", pair[k], v, g); ++nv[k]; }
        }
        int done = 1;
        for (int k = 0; k < 3; ++k) done &= nm[k] >= WANT && nv[k] >= WANT;
        if (done) return 0;
    }
    return 1;
}
