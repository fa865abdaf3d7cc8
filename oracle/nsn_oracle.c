/*
 * CPU oracle for the NSN packed-KV hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the arithmetic of the reference's CPU
 * functions so that tests can check the HIP kernels bit-for-bit.  Nothing in
 * the shipped library links it; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it (through oracle/oracle.py).
 *
 * Reference functions restated (paths relative to the reference root):
 *   nsn_encode      experiments/ac08/source/loop_kv_pilot.py:195-213
 *   nsn_decode      experiments/ac08/source/loop_kv_pilot.py:216-225
 *   nsn_int3_qdq    papers/nsn-integrated/code/nsn_int3_core.py:11-21
 *   pack_codes      experiments/ac08/source/loop_kv_pilot.py:171-181
 *   unpack_codes_reference  experiments/ac08/source/loop_kv_pilot.py:183-193
 *
 * The reference computes in torch on the CPU.  The parts of torch's arithmetic
 * that decide the output bits are restated here:
 *   - torch.linalg.vector_norm(a, dim=-1) over a contiguous fp32 row runs an
 *     8-lane accumulator: lane j accumulates fma(x, x, acc) over elements
 *     j, j+8, j+16, ... in order, then the 8 lanes are summed left to right
 *     and sqrt is taken in fp32.  (Pinned against torch itself and against the
 *     golden vectors written from the reference; see tests/test_oracle.py.)
 *   - tensor division is IEEE fp32 division; torch.round is round-half-even;
 *     .to(float16) / .to(bfloat16) are round-to-nearest-even.
 *   - m + s*q is an unfused multiply then add.
 *   - the per-channel min / max treat -0 as below +0 (IEEE 754-2019 minimum /
 *     maximum).  Only the sign of a zero m or mx depends on this.  torch's
 *     own reductions keep whichever zero their (vector-width and
 *     backend dependent) order meets last, so no single reference rule
 *     exists for a tie of signed zeros; this one does not depend on order.
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off -mfma; fmaf is called
 * explicitly where torch fuses).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define NSN_DIM 128
#define NSN_BLOCK 64
#define NSN_EPS 1e-12f

/* ---- fp16 / bf16 conversions (round to nearest even) ------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t oracle_f32_to_f16(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                 /* inf or nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (ax < 0x38800000u) {                  /* result is subnormal or zero */
        /* value = ax_float; subnormal unit = 2^-24 */
        float a = u2f(ax);
        /* a * 2^24 rounded to nearest even integer gives the mantissa */
        float scaled = a * 16777216.0f;      /* exact: power of two scaling */
        float r = nearbyintf(scaled);        /* default mode = nearest even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    /* normal: rebias exponent, round mantissa from 23 to 10 bits */
    uint32_t mant = ax & 0x7fffffu;
    uint32_t exp = (ax >> 23) - 127 + 15;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

uint16_t oracle_f32_to_bf16(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float oracle_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ---- torch-CPU vector_norm over a row of 128 fp32 values --------------- */

/* Non-contiguous rows (last-dim stride != 1) take torch's generic reduction
 * instead: one fma chain over the row in order. */
float oracle_row_norm_seq(const float *row, int dim)
{
    float s = 0.0f;
    for (int d = 0; d < dim; ++d) s = fmaf(row[d], row[d], s);
    return sqrtf(s);
}

float oracle_row_norm(const float *row, int dim)
{
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int d = 0;
    for (; d + 8 <= dim; d += 8)
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(row[d + j], row[d + j], acc[j]);
    float s = acc[0];
    for (int j = 1; j < 8; ++j) s = s + acc[j];
    for (; d < dim; ++d) s = fmaf(row[d], row[d], s);
    return sqrtf(s);
}

void oracle_vector_norm(const float *rows, int64_t nrows, int dim, int order, float *out)
{
    for (int64_t r = 0; r < nrows; ++r)
        out[r] = order ? oracle_row_norm_seq(rows + r * dim, dim) : oracle_row_norm(rows + r * dim, dim);
}

/* ---- encode ------------------------------------------------------------ */

/* Error bits, same meaning as the device status word of the HIP library. */
#define ORACLE_ERR_NONFINITE_INPUT 1
#define ORACLE_ERR_META_NONFINITE 2
#define ORACLE_ERR_META_UNDERFLOW 4

/*
 * x: nblocks * 64 * 128 fp32 values (the input already converted by .float()).
 * q: nblocks*64*128 u8 codes.  n16: nblocks*64, m16/s16: nblocks*128 (fp16 bits).
 * n32/m32/s32 (nullable): the unrounded fp32 metadata.
 * zero_flat_scale: 1 reproduces nsn_encode's `q = where(s==0, 0, q)`,
 *                  0 reproduces nsn_int3_qdq (which omits it).
 * norm_order: 0 = 8-lane order (contiguous rows), 1 = one sequential fma chain
 *             (what torch does when x.float() has last-dim stride != 1).
 * Returns the OR of the error bits nsn_encode would raise on (all blocks are
 * still computed so that tests can inspect outputs).
 */
int oracle_nsn_encode(const float *x, int64_t nblocks, int bits, int zero_flat_scale,
                      int norm_order, uint8_t *q, uint16_t *n16, uint16_t *m16, uint16_t *s16,
                      float *n32, float *m32, float *s32)
{
    const float levels = (float)((1 << bits) - 1);
    int err = 0;
    static float d[NSN_BLOCK * NSN_DIM];
    for (int64_t b = 0; b < nblocks; ++b) {
        const float *a = x + b * NSN_BLOCK * NSN_DIM;
        float nrm[NSN_BLOCK], mn[NSN_DIM], sc[NSN_DIM];
        for (int i = 0; i < NSN_BLOCK * NSN_DIM; ++i)
            if (!isfinite(a[i])) err |= ORACLE_ERR_NONFINITE_INPUT;
        for (int t = 0; t < NSN_BLOCK; ++t) {
            nrm[t] = norm_order ? oracle_row_norm_seq(a + t * NSN_DIM, NSN_DIM)
                                : oracle_row_norm(a + t * NSN_DIM, NSN_DIM);
            float den = nrm[t] > NSN_EPS ? nrm[t] : NSN_EPS;   /* clamp_min */
            if (isnan(nrm[t])) den = nrm[t];
            for (int c = 0; c < NSN_DIM; ++c) d[t * NSN_DIM + c] = a[t * NSN_DIM + c] / den;
        }
        for (int c = 0; c < NSN_DIM; ++c) {
            float lo = d[c], hi = d[c];
            for (int t = 1; t < NSN_BLOCK; ++t) {
                float v = d[t * NSN_DIM + c];
                if (isnan(v) || v < lo) lo = (isnan(lo) ? lo : v);
                else if (v == lo && signbit(v) && !signbit(lo)) lo = v;   /* -0 < +0 */
                if (isnan(v) || v > hi) hi = (isnan(hi) ? hi : v);
                else if (v == hi && !signbit(v) && signbit(hi)) hi = v;   /* +0 > -0 */
            }
            mn[c] = lo;
            sc[c] = (hi - lo) / levels;
        }
        for (int t = 0; t < NSN_BLOCK; ++t)
            for (int c = 0; c < NSN_DIM; ++c) {
                float den = sc[c] == 0.0f ? 1.0f : sc[c];
                float v = nearbyintf((d[t * NSN_DIM + c] - mn[c]) / den);
                v = v < 0.0f ? 0.0f : (v > levels ? levels : v);
                uint8_t code = (uint8_t)v;   /* NaN never reaches valid outputs */
                if (zero_flat_scale && sc[c] == 0.0f) code = 0;
                q[(b * NSN_BLOCK + t) * NSN_DIM + c] = code;
            }
        for (int t = 0; t < NSN_BLOCK; ++t) {
            uint16_t h = oracle_f32_to_f16(nrm[t]);
            n16[b * NSN_BLOCK + t] = h;
            if (n32) n32[b * NSN_BLOCK + t] = nrm[t];
            if ((h & 0x7c00u) == 0x7c00u) err |= ORACLE_ERR_META_NONFINITE;
            if (nrm[t] != 0.0f && (h & 0x7fffu) == 0) err |= ORACLE_ERR_META_UNDERFLOW;
        }
        for (int c = 0; c < NSN_DIM; ++c) {
            uint16_t hm = oracle_f32_to_f16(mn[c]), hs = oracle_f32_to_f16(sc[c]);
            m16[b * NSN_DIM + c] = hm;
            s16[b * NSN_DIM + c] = hs;
            if (m32) m32[b * NSN_DIM + c] = mn[c];
            if (s32) s32[b * NSN_DIM + c] = sc[c];
            if ((hm & 0x7c00u) == 0x7c00u || (hs & 0x7c00u) == 0x7c00u) err |= ORACLE_ERR_META_NONFINITE;
            if (sc[c] != 0.0f && (hs & 0x7fffu) == 0) err |= ORACLE_ERR_META_UNDERFLOW;
        }
    }
    return err;
}

/* ---- decode ------------------------------------------------------------ */

/*
 * y[b,t,c] (fp32, before the final dtype cast) =
 *   n==0 ? 0 : n * (d / max(norm(d), 1e-12)),  d = m + s*q  (unfused).
 */
void oracle_nsn_decode(const uint8_t *q, const uint16_t *n16, const uint16_t *m16,
                       const uint16_t *s16, int64_t nblocks, float *y)
{
    for (int64_t b = 0; b < nblocks; ++b) {
        float m[NSN_DIM], s[NSN_DIM], d[NSN_DIM];
        for (int c = 0; c < NSN_DIM; ++c) {
            m[c] = oracle_f16_to_f32(m16[b * NSN_DIM + c]);
            s[c] = oracle_f16_to_f32(s16[b * NSN_DIM + c]);
        }
        for (int t = 0; t < NSN_BLOCK; ++t) {
            const uint8_t *qr = q + (b * NSN_BLOCK + t) * NSN_DIM;
            float n = oracle_f16_to_f32(n16[b * NSN_BLOCK + t]);
            for (int c = 0; c < NSN_DIM; ++c) {
                float prod = s[c] * (float)qr[c];
                d[c] = m[c] + prod;
            }
            float den = oracle_row_norm(d, NSN_DIM);
            den = den > NSN_EPS ? den : (isnan(den) ? den : NSN_EPS);
            float *yr = y + (b * NSN_BLOCK + t) * NSN_DIM;
            for (int c = 0; c < NSN_DIM; ++c) {
                float v = n * (d[c] / den);
                yr[c] = (n == 0.0f) ? 0.0f : v;
            }
        }
    }
}

/* ---- LSB-first bitstream ------------------------------------------------ */

int64_t oracle_pack_codes(const uint8_t *codes, int64_t count, int bits, uint8_t *out)
{
    int64_t nbytes = (count * bits + 7) / 8;
    memset(out, 0, (size_t)nbytes);
    for (int64_t i = 0; i < count; ++i) {
        int64_t pos = i * bits;
        uint32_t v = (uint32_t)codes[i] << (pos % 8);
        out[pos / 8] |= (uint8_t)(v & 0xffu);
        if (pos % 8 + bits > 8) out[pos / 8 + 1] |= (uint8_t)(v >> 8);
    }
    return nbytes;
}

void oracle_unpack_codes(const uint8_t *payload, int64_t count, int bits, uint8_t *out)
{
    for (int64_t i = 0; i < count; ++i) {
        int64_t pos = i * bits;
        uint32_t v = (uint32_t)payload[pos / 8] >> (pos % 8);
        if (pos % 8 + bits > 8) v |= (uint32_t)payload[pos / 8 + 1] << (8 - pos % 8);
        out[i] = (uint8_t)(v & ((1u << bits) - 1u));
    }
}
