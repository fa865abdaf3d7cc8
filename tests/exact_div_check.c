/*
 * Checks the division the HIP encoder uses for fp16 inputs against IEEE fp32
 * division:
 *
 *   d = x / den  (x an fp16 value, den > 0 an fp32 value, rc = RN(1/den))
 *   q0 = RN(x * rc + (-0))
 *   e  = RN(q0 * den - x)        (exact: the residual of a faithful quotient)
 *   d  = RN(q0 + e * (-rc))      (Markstein's correction step)
 *
 * All three steps are single fma operations.  The result depends only on the
 * significands of x and den while no intermediate leaves the normal range, so
 * the full check runs every fp16 significand (1024) against every fp32
 * significand of den (2^23), with the quotient in both binades below and
 * above 1/2 .. 2 (x exponent 0 and -1 relative to den in [1, 2)), for both
 * signs, plus the signed zeros.
 *
 *   usage: exact_div_check [stride [naive]]   (stride 1 = exhaustive; default 1)
 * Prints the number of pairs checked and mismatches; exit status 1 on a
 * mismatch.  "naive" checks q0 alone (no correction step): a planted mistake
 * that must show mismatches.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int naive;

static float markstein(float x, float den, float rc)
{
    const float q0 = fmaf(x, rc, -0.0f);
    if (naive) return q0;
    const float e = fmaf(q0, den, -x);
    return fmaf(e, -rc, q0);
}

int main(int argc, char **argv)
{
    const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
    naive = argc > 2 && strcmp(argv[2], "naive") == 0;
    uint64_t checked = 0, bad = 0;
    /* signed zeros keep their sign */
    for (int s = 0; s < 2; ++s) {
        const float z = s ? -0.0f : 0.0f;
        const float den = 1.2345f, rc = (float)(1.0 / (double)den);
        const float d = markstein(z, den, rc);
        checked++;
        if (f_bits(d) != f_bits(z / den)) bad++;
    }
#pragma omp parallel for reduction(+ : checked, bad) schedule(dynamic, 1)
    for (int k = 0; k < 1024; ++k) {
        for (uint32_t m = 0; m < (1u << 23); m += stride) {
            const float den = bits_f(0x3f800000u | m);          /* [1, 2) */
            const float rc = (float)(1.0 / (double)den);        /* RN(1/den) */
            for (int ex = 0; ex < 2; ++ex)
                for (int sg = 0; sg < 2; ++sg) {
                    /* fp16 significand 1 + k/1024 as an fp32 value, exponent 0 or -1 */
                    const uint32_t xb = ((uint32_t)sg << 31) | ((uint32_t)(127 - ex) << 23) | ((uint32_t)k << 13);
                    const float x = bits_f(xb);
                    const float want = x / den;
                    const float got = markstein(x, den, rc);
                    checked++;
                    if (f_bits(got) != f_bits(want)) {
                        if (bad < 8)
                            printf("mismatch x=%a den=%a got=%a want=%a\n", (double)x, (double)den, (double)got,
                                   (double)want);
                        bad++;
                    }
                }
        }
    }
    printf("checked %llu pairs, %llu mismatches\n", (unsigned long long)checked, (unsigned long long)bad);
    return bad != 0;
}
