/*
 * Checks the code rounding the HIP encoder uses against the reference's
 *
 *   code = round_half_even(RN32(t / s))      (t = d - m >= 0, s > 0 fp32)
 *
 * where the encoder computes the quotient in fp32 without a division:
 *
 *   yh = RN32(1 / s),  yl = RN32(RN64(1 / s) - yh)     (once per channel)
 *   q  = RN(t * yh + RN(t * yl))                         (one multiply, one fma)
 *   code = bits(q + 1.5 * 2^23) - bits(1.5 * 2^23)
 *
 * Why a windowed check is exhaustive.  Write A = t / s.  yh + yl = (1/s)(1 + b)
 * with |b| <= 2^-48 (yl carries the reciprocal's next 24 bits, RN64(1/s) is
 * within 2^-53), and RN(t * yl) is within 2^-24 |t yl| <= 2^-47 A of t yl
 * (t * yl stays normal for s >= 2^-64, the encoder's fast-path condition).
 * So q = RN(A + e) with |e| < 2^-46 A < 2^-22 ulp(A): q differs from RN32(A)
 * only if a rounding midpoint M of the fp32 grid lies within |e| of A, and then
 * q and RN32(A) are the two floats next to M.  Their half-even integer
 * roundings differ only if one of the two is a half-integer h = k + 1/2 (no
 * float lies between two adjacent floats), i.e. only if M = h - ulp/2 or
 * h + ulp/2.  Everything scales with s by powers of two while t, s, yh, yl and
 * t * yl stay normal, so it suffices to take s in [1, 2) -- all 2^23
 * significands -- and, for each half-integer h below 2^5 - 1 (all 3-, 4- and
 * 5-bit levels), every t within K ulps of RN(M * s) for both midpoints next to
 * h, and of RN(h * s).
 *
 * The expected code uses the correctly rounded fp64 quotient rounded to fp32:
 * a quotient of 24-bit significands is exact or at least 2^-49 (relative)
 * away from an fp32 midpoint, so RN32(RN64(t/s)) = RN32(t/s).
 *
 *   usage: exact_code_check [stride [naive]]   (stride over the 2^23 s
 *   significands; 1 = exhaustive, the default)
 * "naive" takes RN(t * yh) as the quotient (no low part): a planted mistake
 * that must show mismatches.  Exit status 1 on a code mismatch.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static int naive;
static const float kMagic = 12582912.0f;   /* 1.5 * 2^23 */

static float quotient(float t, float yh, float yl)
{
    if (naive) return t * yh;
    return fmaf(t, yh, t * yl);
}

static uint32_t code_of(float q) { return f_bits(q + kMagic) - f_bits(kMagic); }

#define K 3

int main(int argc, char **argv)
{
    const uint32_t stride = argc > 1 ? (uint32_t)atoi(argv[1]) : 1u;
    naive = argc > 2 && strcmp(argv[2], "naive") == 0;
    uint64_t checked = 0, bad = 0, q_differs = 0;
#pragma omp parallel for reduction(+ : checked, bad, q_differs) schedule(dynamic, 1024)
    for (uint32_t m = 0; m < (1u << 23); m += stride) {
        const float s = bits_f(0x3f800000u | m);   /* [1, 2) */
        const double rs = 1.0 / (double)s;
        const float yh = (float)rs;
        const float yl = (float)(rs - (double)yh);
        for (int k = 0; k < 31; ++k) {
            const double h = k + 0.5;
            const float hf = (float)h;
            const double ulp_up = (double)nextafterf(hf, 2.0f * hf) - h;
            const double ulp_dn = h - (double)nextafterf(hf, 0.0f);
            const double centre[3] = {h - ulp_dn / 2, h, h + ulp_up / 2};
            for (int c = 0; c < 3; ++c) {
                /* centre * s has at most 26 + 24 significant bits: exact in double */
                const float t0 = (float)(centre[c] * (double)s);
                float t = t0;
                for (int j = 0; j < K; ++j) t = nextafterf(t, 0.0f);
                for (int j = -K; j <= K; ++j, t = nextafterf(t, INFINITY)) {
                    const float want_q = (float)((double)t / (double)s);
                    const float got_q = quotient(t, yh, yl);
                    checked++;
                    if (f_bits(got_q) != f_bits(want_q)) q_differs++;
                    if (code_of(got_q) != code_of(want_q)) {
#pragma omp critical
                        if (bad < 8)
                            printf("mismatch t=%a s=%a got q=%a want q=%a\n", (double)t, (double)s, (double)got_q,
                                   (double)want_q);
                        bad++;
                    }
                }
            }
        }
    }
    printf("checked %llu (t, s) pairs, %llu quotients differ from RN32(t/s), %llu code mismatches\n",
           (unsigned long long)checked, (unsigned long long)q_differs, (unsigned long long)bad);
    return bad != 0;
}
