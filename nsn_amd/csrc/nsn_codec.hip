// NSN codec kernels for gfx950: block encoder, bitstream pack/unpack, exact
// block restore (+ tail append), and the grouped finite scan.
//
// Reference semantics (paths relative to the reference root):
//   nsn_encode   experiments/ac08/source/loop_kv_pilot.py:195-213
//   nsn_decode   experiments/ac08/source/loop_kv_pilot.py:216-225
//   pack3/unpack3/encode_group/restore_group
//                experiments/ac08/source/loop_kv_pk01_cache.py:7-42
//   VF01 bridge materialize   experiments/ac08/source/loop_kv_vf01_kernel.py:47-54
//   finite checks             experiments/ac08/source/loop_kv_vf01_checks.py:20-63
#include <type_traits>

#include "nsn_common.hpp"

namespace nsn {

// =====================================================================
// Encoder: one 256-thread workgroup per 64x128 block.
//
// Thread tid holds rows r0 + 16*j (r0 = tid / 16, j = 0..3) x channels
// 8*cg .. 8*cg+7 (cg = tid % 16): each global load is 16 contiguous bytes
// and a wave reads 1 KiB of consecutive input.  The raw block is also staged
// in LDS for the norm, whose summation order must be torch's.
//
// The kernel is bound by VALU issue, so the per-element work is kept to
// about 10 instructions, every result still bit-exact:
//   - d = x / n: three fma for fp16 input (Markstein's correction of
//     x * RN(1/n)); one fp64 multiply by RN64(1/n) for bf16 / fp32 input;
//   - per-channel min / max: min3 / max3 over the thread's 4 rows, then the
//     16 row-group partials through LDS;
//   - codes: t = d - m, RN32(t / s) as RN(t * yh + RN(t * yl)) with
//     yh + yl = 1/s to about 2^-48 (one multiply, one fma; the half-even code
//     is exact for every scale s >= 2^-64, tests/exact_code_check.c), the
//     half-even rounding to an integer by adding 1.5 * 2^23, and a shift-add
//     of that word straight into the row's bitstream; blocks with a smaller
//     nonzero scale take a clamped copy of the loop on an fp64 multiply;
//   - decode factors (optional): each lane sums (m + s*code)^2 over its 8
//     channels per row, a 16-lane DPP tree finishes the row, and one lane per
//     row divides the fp16 norm by the root; no second pass over the block;
//   - no per-element finite test: a nonfinite input shows in its row norm.
// =====================================================================

struct EncodeParams {
    const void *x;
    int64_t n_blocks;
    int64_t x_outer_stride;
    int64_t x_token_offset;
    uint8_t *codes;
    uint16_t *norms, *mins, *scales;
    uint8_t *headers;
    float *factors;
    int64_t out_outer_blocks, out_block_offset, header_start_token;
    uint8_t *codes_unpacked;
    int32_t *status;
    int zero_flat_scale;
    int64_t total;   // n_outer * n_blocks, one workgroup each
};

constexpr int kXPadT = kDim + 8;  // LDS row pitch of the encode input block (elements; 16-byte rows)

template <int DT>
__device__ __forceinline__ void load_row8(const typename Elem<DT>::T *src, float (&v)[8]) {
    if constexpr (DT == NSN_DTYPE_F32) {
        const float4 a = *reinterpret_cast<const float4 *>(src);
        const float4 b = *reinterpret_cast<const float4 *>(src + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4 *>(src);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = Elem<DT>::load(static_cast<uint16_t>(w[k] & 0xffffu));
            v[2 * k + 1] = Elem<DT>::load(static_cast<uint16_t>(w[k] >> 16));
        }
    }
}

template <int DT>
__device__ __forceinline__ void store_row8(typename Elem<DT>::T *dst, const float (&v)[8]) {
    if constexpr (DT == NSN_DTYPE_F32) {
        *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = static_cast<uint32_t>(Elem<DT>::store(v[2 * k])) |
                   (static_cast<uint32_t>(Elem<DT>::store(v[2 * k + 1])) << 16);
        *reinterpret_cast<uint4 *>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Pack 32 codes (each < 2^BITS) LSB-first into BITS dwords.
template <int BITS>
__device__ __forceinline__ void pack32(const uint32_t (&c)[32], uint32_t (&w)[BITS]) {
#pragma unroll
    for (int k = 0; k < BITS; ++k) w[k] = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int pos = i * BITS, d = pos >> 5, sh = pos & 31;
        w[d] |= c[i] << sh;
        if (sh + BITS > 32) w[d + 1] |= c[i] >> (32 - sh);
    }
}

template <int BITS>
__device__ __forceinline__ void unpack32(const uint32_t (&w)[BITS], uint32_t (&c)[32]) {
    constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int pos = i * BITS, d = pos >> 5, sh = pos & 31;
        uint32_t v = w[d] >> sh;
        if (sh + BITS > 32) v |= w[d + 1] << (32 - sh);
        c[i] = v & mask;
    }
}

// Decode factors f_t = n_t / max(|d_t|, 1e-12) with d_t = m + s*q (fp16 metadata
// as fp32, unfused multiply/add, torch's 8-lane norm order) for the 64 rows of
// a block whose u8 codes are in LDS.  f_t * d_t is the row nsn_decode returns
// (up to the final rounding), so the decode kernels can renormalise a packed
// token with one multiply.  Writes f_t for t = tid/4 from lanes tid%4 == 0.
__device__ __forceinline__ void block_factors_lds(const uint8_t *codes_s, const float *m16f, const float *s16f,
                                                  const float *n16f, float *factors) {
    const int tid = threadIdx.x;
    const int r = tid >> 2, jp = (tid & 3) * 2;
    const uint8_t *cr = codes_s + r * kDim;
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int c = 8 * k + jp;
        const float p0 = s16f[c] * static_cast<float>(cr[c]);
        const float p1 = s16f[c + 1] * static_cast<float>(cr[c + 1]);
        const float d0 = m16f[c] + p0, d1 = m16f[c + 1] + p1;
        a0 = __builtin_fmaf(d0, d0, a0);
        a1 = __builtin_fmaf(d1, d1, a1);
    }
    const float b0 = __shfl_down(a0, 1), b1 = __shfl_down(a1, 1);
    const float c0 = __shfl_down(a0, 2), c1 = __shfl_down(a1, 2);
    const float d0 = __shfl_down(a0, 3), d1 = __shfl_down(a1, 3);
    if ((tid & 3) == 0) {
        const float acc[8] = {a0, a1, b0, b1, c0, c1, d0, d1};
        const float den = clamp_eps(sqrt_rn(lane8_sum(acc)));
        const float n = n16f[r];
        factors[r] = (n == 0.f) ? 0.f : div_by_recip(n, recip_rn(den));
    }
}

constexpr float kRoundMagic = 12582912.f;   // 1.5 * 2^23: q + this rounds q half-even into the low mantissa bits

typedef _Float16 enc_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t enc_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float half_lo(uint32_t w) { return static_cast<float>(__builtin_bit_cast(enc_h2, w)[0]); }
__device__ __forceinline__ float half_hi(uint32_t w) { return static_cast<float>(__builtin_bit_cast(enc_h2, w)[1]); }

// x / den correctly rounded, for x an fp16 value, den > 0 and rc = RN(1/den):
// q0 = RN(x * rc) is a faithful quotient, e = q0 * den - x is exact, and
// RN(q0 + e * -rc) is the IEEE quotient (Markstein's correction).  Checked for
// every fp16 significand against every fp32 significand of den, signed zeros
// included (tests/exact_div_check.c).  `neg0` is -0 hidden from the compiler:
// it keeps the first step an fma that reads x as fp16 (v_fma_mix_f32), and
// x = -0 keeps its sign through all three steps.
__device__ __forceinline__ float div_f16_markstein(float x, float den, float rc, float neg0) {
    const float q0 = __builtin_fmaf(x, rc, neg0);
    const float e = __builtin_fmaf(q0, den, -x);
    return __builtin_fmaf(e, -rc, q0);   // (negating rc, not e: -fma(.) -> fma(-., -.) would lose a -0)
}

// The constant the shift-add packing carries along: the sum over the codes k
// that start in the row's low dword of (bits of 1.5 * 2^23) << (BITS * k),
// mod 2^32 (all 8 codes at 3 and 4 bits; codes 0..6 at 5 bits).
template <int BITS>
__device__ __forceinline__ constexpr uint32_t magic_sum_lo() {
    uint32_t c = 0;
    for (int k = 0; k < 8; ++k)
        if (BITS * k < 32) c += 0x4B400000u << (BITS * k);
    return c;
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(x)));
}
// acc + (a << SH) as one v_lshl_add_u32 (left to itself the compiler turns a
// chain of these into separate shifts and three-input adds).
template <int SH>
__device__ __forceinline__ uint32_t lshl_add(uint32_t a, uint32_t acc) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "n"(SH), "v"(acc));
    return r;
}
// v_perm_b32: byte i of the result = byte sel[i] of {hi:lo} (0..3 = lo, 4..7 = hi, 0x0c = 0).
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

template <int DT, int BITS, int ORDER>
__global__ __launch_bounds__(256) void encode_kernel(EncodeParams p) {
    using T = typename Elem<DT>::T;
    constexpr float kLevels = static_cast<float>((1 << BITS) - 1);
    // The input block (in its own type) is only read by the norm pass; the
    // 16 row-group min/max partials reuse its bytes.
    // Keeping the block at 2 bytes per element (fp16/bf16 inputs) holds the
    // LDS to ~22 KB per workgroup: 7 workgroups per CU.
    constexpr int kXBytes = kBlockTok * kXPadT * static_cast<int>(sizeof(T));
    static_assert(kXBytes >= 2 * 16 * kDim * 4, "LDS aliasing");
    __shared__ __align__(16) uint8_t xraw[kXBytes];
    T *const xs = reinterpret_cast<T *>(xraw);
    float (*const pmin)[kDim] = reinterpret_cast<float (*)[kDim]>(xraw);           // [16][128], after the norms
    float (*const pmax)[kDim] = reinterpret_cast<float (*)[kDim]>(xraw + 8192);    // [16][128]
    __shared__ float nrm_s[kBlockTok], den_s[kBlockTok], rcp_s[kBlockTok];
    __shared__ double rden_s[DT == NSN_DTYPE_F16 ? 1 : kBlockTok];   // fp16 input divides by den and rcp
    // Per-channel constants, channel c at [chx(c)] = 16 * (c % 8) + c / 8: the
    // code pass reads channel 8*cg + e in lanes cg = 0..15 at once, which this
    // order puts on 16 consecutive words (channel-order storage put them 8
    // words apart: 4 lanes on each bank).
    auto chx = [](int c) { return 16 * (c & 7) + (c >> 3); };
    __shared__ float m_s[kDim];
    __shared__ double rs_s[kDim];
    __shared__ float yh_s[kDim], yl_s[kDim];
    __shared__ float mh_s[kDim], sh_s[kDim], nh_s[kBlockTok];
    __shared__ int bad_s, clamp_s;

    const int tid = threadIdx.x;
    const int cg = tid & 15, r0 = tid >> 4;
    const uint32_t f = blockIdx.x;   // block f: outer row f / n_blocks, block f % n_blocks
    const uint32_t o = f / static_cast<uint32_t>(p.n_blocks), i = f - o * static_cast<uint32_t>(p.n_blocks);
    const int64_t ob = static_cast<int64_t>(o) * p.out_outer_blocks + p.out_block_offset + i;
    constexpr int NW = (DT == NSN_DTYPE_F32) ? 8 : 4;   // dwords per 8 values
    int status_acc = 0;
    if (tid == 0) {
        bad_s = 0;
        clamp_s = 0;
    }
    {
        // ---- load: the thread's 4 rows x 8 channels as raw dwords (16-byte
        // loads; a wave reads 1 KiB of consecutive input per row group).  The
        // input is read once, so the loads carry the non-temporal hint (C2
        // encode 385.3 -> 377.8 us, mean of 4 alternating rounds).
        const T *x = static_cast<const T *>(p.x) + static_cast<int64_t>(o) * p.x_outer_stride +
                     (p.x_token_offset + static_cast<int64_t>(i) * kBlockTok) * kDim;
        uint32_t xw[4][NW];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const enc_u4 *src = reinterpret_cast<const enc_u4 *>(x + (r0 + 16 * j) * kDim + 8 * cg);
#pragma unroll
            for (int h = 0; h < NW / 4; ++h) {
                const enc_u4 a4 = __builtin_nontemporal_load(src + h);
                const uint4 a = make_uint4(a4[0], a4[1], a4[2], a4[3]);
                xw[j][4 * h] = a.x; xw[j][4 * h + 1] = a.y; xw[j][4 * h + 2] = a.z; xw[j][4 * h + 3] = a.w;
            }
        }

        // ---- stage the block in LDS for the norm pass
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint4 *dst = reinterpret_cast<uint4 *>(xs + (r0 + 16 * j) * kXPadT + 8 * cg);
#pragma unroll
            for (int h = 0; h < NW / 4; ++h)
                dst[h] = make_uint4(xw[j][4 * h], xw[j][4 * h + 1], xw[j][4 * h + 2], xw[j][4 * h + 3]);
        }
        __syncthreads();

        // ---- token norms, in torch's order.  A nonfinite input makes its row's
        // norm nonfinite; for fp16 the converse holds too (128 squares of finite
        // fp16 values stay below 2^40), otherwise the row is scanned.
        auto set_row = [&](int r, float n) {
            nrm_s[r] = n;
            const float den = clamp_eps(n);
            const double rd = recip_rn(den);
            den_s[r] = den;
            if constexpr (DT != NSN_DTYPE_F16) rden_s[r] = rd;
            rcp_s[r] = static_cast<float>(rd);   // RN32(RN64(1/den)) = RN32(1/den): 1/den is never that close to a tie
            if (!finite(n)) {
                bool row_bad = DT == NSN_DTYPE_F16;
                if (!row_bad)
                    for (int c = 0; c < kDim; ++c) row_bad |= !finite(Elem<DT>::load(xs[r * kXPadT + c]));
                if (row_bad) bad_s = 1;
            }
        };
        if constexpr (ORDER == NSN_NORM_LANES8) {
            const int r = tid >> 2, jp = (tid & 3) * 2;
            float a0 = 0.f, a1 = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                float q0, q1;
                if constexpr (DT == NSN_DTYPE_F32) {
                    const float2 q = *reinterpret_cast<const float2 *>(xs + r * kXPadT + 8 * k + jp);
                    q0 = q.x;
                    q1 = q.y;
                } else {
                    const uint32_t q = *reinterpret_cast<const uint32_t *>(xs + r * kXPadT + 8 * k + jp);
                    q0 = Elem<DT>::load(static_cast<uint16_t>(q & 0xffffu));
                    q1 = Elem<DT>::load(static_cast<uint16_t>(q >> 16));
                }
                a0 = __builtin_fmaf(q0, q0, a0);
                a1 = __builtin_fmaf(q1, q1, a1);
            }
            // the row's 4 threads are one quad of lanes: lane 0 gathers lanes 1..3
            const float b0 = dpp_f32<0xF9>(a0), b1 = dpp_f32<0xF9>(a1);   // quad_perm [1,2,3,3]
            const float c0 = dpp_f32<0xFE>(a0), c1 = dpp_f32<0xFE>(a1);   // quad_perm [2,3,3,3]
            const float d0 = dpp_f32<0xFF>(a0), d1 = dpp_f32<0xFF>(a1);   // quad_perm [3,3,3,3]
            if ((tid & 3) == 0) {
                const float acc[8] = {a0, a1, b0, b1, c0, c1, d0, d1};
                set_row(r, sqrt_rn(lane8_sum(acc)));
            }
        } else {
            if (tid < kBlockTok) {
                float s = 0.f;
                for (int c = 0; c < kDim; ++c) {
                    const float q = Elem<DT>::load(xs[tid * kXPadT + c]);
                    s = __builtin_fmaf(q, q, s);
                }
                set_row(tid, sqrt_rn(s));
            }
        }
        __syncthreads();

        // ---- directions d = x / max(n, eps), and the thread's min / max per channel
        float d[4][8];
        const float neg0 = keep_f32(-0.f);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = r0 + 16 * j;
            if constexpr (DT == NSN_DTYPE_F16) {
                const float dn = den_s[r], rc = rcp_s[r];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint32_t w = xw[j][e >> 1];
                    d[j][e] = div_f16_markstein((e & 1) ? half_hi(w) : half_lo(w), dn, rc, neg0);
                }
            } else {
                const double rd = rden_s[r];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float v;
                    if constexpr (DT == NSN_DTYPE_F32) v = __uint_as_float(xw[j][e]);
                    else v = __uint_as_float((e & 1) ? (xw[j][e >> 1] & 0xffff0000u) : (xw[j][e >> 1] << 16));
                    d[j][e] = div_by_recip(v, rd);
                }
            }
        }
        {
            float mn[8], mx[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                mn[e] = fminf(fminf(fminf(d[0][e], d[1][e]), d[2][e]), d[3][e]);
                mx[e] = fmaxf(fmaxf(fmaxf(d[0][e], d[1][e]), d[2][e]), d[3][e]);
            }
            float4 *pn = reinterpret_cast<float4 *>(&pmin[r0][8 * cg]);
            float4 *px = reinterpret_cast<float4 *>(&pmax[r0][8 * cg]);
            pn[0] = make_float4(mn[0], mn[1], mn[2], mn[3]);
            pn[1] = make_float4(mn[4], mn[5], mn[6], mn[7]);
            px[0] = make_float4(mx[0], mx[1], mx[2], mx[3]);
            px[1] = make_float4(mx[4], mx[5], mx[6], mx[7]);
        }
        __syncthreads();

        // ---- per-channel min / scale over the 16 row-group partials; fp16 metadata
        if (tid < kDim) {
            float lo = pmin[0][tid], hi = pmax[0][tid];
#pragma unroll
            for (int w = 1; w < 16; ++w) {
                lo = fminf(lo, pmin[w][tid]);
                hi = fmaxf(hi, pmax[w][tid]);
            }
            const float s = div_by_recip(hi - lo, recip_rn(kLevels));
            m_s[chx(tid)] = lo;
            // 1/s; for s == 0 the reference divides by 1 (every d - m is 0 then),
            // or zeroes the codes when zero_flat_scale is set: a factor of 0
            const double rs = (s == 0.f) ? (p.zero_flat_scale ? 0.0 : 1.0) : recip_rn(s);
            rs_s[chx(tid)] = rs;
            // 1/s as yh + yl: yh = RN32(1/s) (= RN32(RN64(1/s)): 1/s is never
            // within 2^-48 of an fp32 midpoint), yl = RN32(RN64(1/s) - yh).  s == 0
            // multiplies by 1 (or by 0 under zero_flat_scale) with yl = 0: exact.
            const float yh = static_cast<float>(rs);
            yh_s[chx(tid)] = yh;
            yl_s[chx(tid)] = static_cast<float>(rs - static_cast<double>(yh));
            // A nonzero s below 2^-64 takes the fp64 loop: the low product could
            // leave the normal range, and with a subnormal s the quotient
            // (d - m) / s can pass the top level (s then also underflows fp16,
            // which the status word reports), so that loop clamps.
            if (s != 0.f && !(s >= 5.42101086e-20f)) clamp_s = 1;
            const uint16_t hm = f32_to_f16_bits(lo), hs = f32_to_f16_bits(s);
            p.mins[ob * kDim + tid] = hm;
            p.scales[ob * kDim + tid] = hs;
            mh_s[chx(tid)] = f16_bits_to_f32(hm);
            sh_s[chx(tid)] = f16_bits_to_f32(hs);
            if ((hm & 0x7c00u) == 0x7c00u || (hs & 0x7c00u) == 0x7c00u) status_acc |= NSN_ST_META_NONFINITE;
            if (s != 0.f && (hs & 0x7fffu) == 0) status_acc |= NSN_ST_META_UNDERFLOW;
        } else if (tid < kDim + kBlockTok) {
            const int t = tid - kDim;
            const float n = nrm_s[t];
            const uint16_t hn = f32_to_f16_bits(n);
            p.norms[ob * kBlockTok + t] = hn;
            nh_s[t] = f16_bits_to_f32(hn);
            if ((hn & 0x7c00u) == 0x7c00u) status_acc |= NSN_ST_META_NONFINITE;
            if (n != 0.f && (hn & 0x7fffu) == 0) status_acc |= NSN_ST_META_UNDERFLOW;
        }
        __syncthreads();

        // ---- codes clamp(round_half_even((d - m) / s), 0, 2^b - 1), packed in place.
        // q = RN32(t / s) lies in [0, 2^b - 1 + 2^-20] for a normal s, so q + 1.5*2^23
        // rounds it half-even to an integer held in the low mantissa bits; the
        // shift-add of those words into the bitstream carries the constant
        // exponent bits along, removed once per row.
        // the lane's first output word (row r0); row r0 + 16j is 16j rows further on
        const int k4 = cg & 3, a4 = cg >> 2;
        uint8_t *const cbase = p.codes + ob * packed_block_bytes(BITS) + r0 * (16 * BITS);
        uint32_t *const cdst = reinterpret_cast<uint32_t *>(
            cbase + (BITS == 4 ? 4 * cg : (BITS == 3 ? 12 * a4 : 20 * a4) + 4 * k4));
        constexpr int kRowStride = 16 * 16 * BITS / 4;   // dwords per 16 rows
        uint2 *const udst = p.codes_unpacked
            ? reinterpret_cast<uint2 *>(p.codes_unpacked + static_cast<int64_t>(f) * (kBlockTok * kDim) +
                                        r0 * kDim + 8 * cg)
            : nullptr;
        float fsum[4];
        auto code_rows = [&](auto clamp_c, auto fac_c) {
            constexpr bool CLAMP = decltype(clamp_c)::value;
            constexpr bool FAC = decltype(fac_c)::value;
            // Channel-outer order: each channel's constants are loaded once and
            // used for the thread's 4 rows; every row's bitstream word (and, at
            // 5 bits, its fifth byte) and factor sum accumulate as it goes.
            uint32_t lo[4], hi5[4], v6[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) fsum[j] = 0.f;
            auto channel = [&](auto e_c) {
                constexpr int e = decltype(e_c)::value;
                const int c = 8 * cg + e;
                float yh = 0.f, yl = 0.f, mh = 0.f, sh = 0.f;
                double rs = 0.0;
                if (CLAMP) {
                    rs = rs_s[chx(c)];
                } else {
                    yh = yh_s[chx(c)];
                    yl = yl_s[chx(c)];
                }
                if (FAC) {
                    mh = mh_s[chx(c)];
                    sh = sh_s[chx(c)];
                }
                const float m = m_s[chx(c)];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float t = d[j][e] - m;
                    float q;
                    if (CLAMP) q = fminf(static_cast<float>(static_cast<double>(t) * rs), kLevels);
                    else q = __builtin_fmaf(t, yh, t * yl);
                    const float qm = q + kRoundMagic;
                    const uint32_t v = __float_as_uint(qm);
                    if (FAC) {
                        // the reconstructed direction from the fp16 metadata: m + s * code
                        const float dd = __builtin_fmaf(sh, qm - kRoundMagic, mh);
                        fsum[j] = __builtin_fmaf(dd, dd, fsum[j]);
                    }
                    if constexpr (e == 0) lo[j] = v - magic_sum_lo<BITS>();
                    else if constexpr (BITS * e < 32) lo[j] = lshl_add<BITS * e>(v, lo[j]);
                    if constexpr (BITS == 5 && e == 6) v6[j] = v;
                    if constexpr (BITS == 5 && e == 7)
                        hi5[j] = lshl_add<3>(v, (v6[j] >> 2) - ((0x4B400000u >> 2) + (0x4B400000u << 3)));
                }
            };
            // (scheduling barriers keep each channel's LDS loads next to their
            // use: hoisted together they would hold 40 registers at once)
            channel(std::integral_constant<int, 0>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 1>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 2>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 3>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 4>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 5>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 6>{});
            __builtin_amdgcn_sched_barrier(0);
            channel(std::integral_constant<int, 7>{});
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t *const dst = cdst + kRowStride * j;
                if constexpr (BITS == 3) {
                    // a quad of lanes holds 96 consecutive bits: lane k writes dword k < 3
                    const uint32_t nxt = dpp_u32<0xF9>(lo[j]);   // quad_perm [1,2,3,3]: lane k+1
                    const uint32_t D = (lo[j] >> (8 * k4)) | (nxt << (24 - 8 * k4));
                    if (k4 < 3) *dst = D;
                } else if constexpr (BITS == 4) {
                    *dst = lo[j];
                } else {
                    // 40 bits per lane, 160 per quad: lane k writes dword k, lane 3 also dword 4
                    const uint32_t plo = dpp_u32<0x90>(lo[j]), phi = dpp_u32<0x90>(hi5[j]);   // quad_perm [0,0,1,2]: lane k-1
                    const uint64_t P = (static_cast<uint64_t>(phi) << 32) | plo;
                    *dst = static_cast<uint32_t>(P >> (40 - 8 * k4)) | (lo[j] << (8 * k4));
                    if (k4 == 3) dst[1] = (lo[j] >> 8) | (hi5[j] << 24);
                }
            }
        };
        const bool want_factors = p.factors != nullptr;
        const bool clamp = clamp_s != 0;
        if (udst) {
            // u8 codes (the reference API's output), by the same rule as the packed codes below
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t w[2] = {0u, 0u};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int c = 8 * cg + e;
                    const float t = d[j][e] - m_s[chx(c)];
                    const float q = clamp ? fminf(static_cast<float>(static_cast<double>(t) * rs_s[chx(c)]), kLevels)
                                          : __builtin_fmaf(t, yh_s[chx(c)], t * yl_s[chx(c)]);
                    w[e >> 2] |= (__float_as_uint(q + kRoundMagic) & 0xffu) << (8 * (e & 3));
                }
                udst[256 * j] = make_uint2(w[0], w[1]);
            }
        }

        if (clamp) {
            if (want_factors) code_rows(std::true_type{}, std::true_type{});
            else code_rows(std::true_type{}, std::false_type{});
        } else {
            if (want_factors) code_rows(std::false_type{}, std::true_type{});
            else code_rows(std::false_type{}, std::false_type{});
        }
        if (want_factors) {
            // Sum the 16 lanes of each row (a DPP row is one r0): after the quad
            // butterflies, the half-row and row mirrors every lane holds the row's
            // sum.  Lane cg = j < 4 finishes row r0 + 16j:
            // f = n / max(sqrt(sum), 1e-12), 0 where n == 0.
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float x = fsum[j];
                x += dpp_f32<0xB1>(x);    // quad_perm [1,0,3,2]
                x += dpp_f32<0x4E>(x);    // quad_perm [2,3,0,1]
                x += dpp_f32<0x141>(x);   // row_half_mirror
                x += dpp_f32<0x140>(x);   // row_mirror
                fsum[j] = x;
            }
            if (cg < 4) {
                const float sum = cg == 0 ? fsum[0] : cg == 1 ? fsum[1] : cg == 2 ? fsum[2] : fsum[3];
                const int r = r0 + 16 * cg;
                const float n = nh_s[r];
                const float den = fmaxf(__builtin_sqrtf(sum), kEps);
                p.factors[ob * kBlockTok + r] = (n == 0.f) ? 0.f : n * __builtin_amdgcn_rcpf(den);
            }
        }
        if (tid == 0) {
            if (p.headers) {
                const uint64_t tok = static_cast<uint64_t>(p.header_start_token + static_cast<int64_t>(i) * kBlockTok);
                uint32_t *h = reinterpret_cast<uint32_t *>(p.headers + ob * 12);
                h[0] = static_cast<uint32_t>(tok);
                h[1] = static_cast<uint32_t>(tok >> 32);
                h[2] = 64u | (static_cast<uint32_t>(BITS) << 16);
            }
            if (bad_s) status_acc |= NSN_ST_NONFINITE_INPUT;
        }
    }
    raise_status(p.status, status_acc);
}

// =====================================================================
// Bitstream pack / unpack: one thread per 32-code group (BITS dwords).
// =====================================================================

template <int BITS>
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t *codes, int64_t count, uint8_t *out,
                                                   int64_t nbytes, int32_t *status) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t base = g * 32;
    if (base >= count) return;
    uint32_t c[32];
    bool bad = false;
    const bool full = base + 32 <= count;
    if (full && (reinterpret_cast<uintptr_t>(codes) & 15u) == 0) {
        const uint4 a = reinterpret_cast<const uint4 *>(codes + base)[0];
        const uint4 b = reinterpret_cast<const uint4 *>(codes + base)[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int k = 0; k < 32; ++k) c[k] = (w[k >> 2] >> (8 * (k & 3))) & 0xffu;
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) c[k] = (base + k < count) ? codes[base + k] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        bad |= c[k] >= (1u << BITS);
        c[k] &= (1u << BITS) - 1u;
    }
    uint32_t w[BITS];
    pack32<BITS>(c, w);
    const int64_t off = g * 4 * BITS;
    if (off + 4 * BITS <= nbytes && (reinterpret_cast<uintptr_t>(out) & 3u) == 0) {
        uint32_t *dst = reinterpret_cast<uint32_t *>(out + off);
#pragma unroll
        for (int k = 0; k < BITS; ++k) dst[k] = w[k];
    } else {
#pragma unroll
        for (int k = 0; k < 4 * BITS; ++k)
            if (off + k < nbytes) out[off + k] = static_cast<uint8_t>(w[k >> 2] >> (8 * (k & 3)));
    }
    if (bad) raise_status(status, NSN_ST_CODE_RANGE);
}

template <int BITS>
__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t *payload, int64_t count, int64_t nbytes,
                                                     uint8_t *out) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t base = g * 32;
    if (base >= count) return;
    const int64_t off = g * 4 * BITS;
    uint32_t w[BITS];
    if (off + 4 * BITS <= nbytes && (reinterpret_cast<uintptr_t>(payload) & 3u) == 0) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(payload + off);
#pragma unroll
        for (int k = 0; k < BITS; ++k) w[k] = src[k];
    } else {
#pragma unroll
        for (int k = 0; k < BITS; ++k) w[k] = 0;
#pragma unroll
        for (int k = 0; k < 4 * BITS; ++k)
            if (off + k < nbytes) w[k >> 2] |= static_cast<uint32_t>(payload[off + k]) << (8 * (k & 3));
    }
    uint32_t c[32];
    unpack32<BITS>(w, c);
    if (base + 32 <= count && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
        uint32_t o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = c[4 * k] | (c[4 * k + 1] << 8) | (c[4 * k + 2] << 16) | (c[4 * k + 3] << 24);
        uint4 *dst = reinterpret_cast<uint4 *>(out + base);
        dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
        dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k)
            if (base + k < count) out[base + k] = static_cast<uint8_t>(c[k]);
    }
}

// =====================================================================
// Restore (nsn_decode arithmetic, bit-exact) with tail append.
// Grid: n_outer x (n_blocks + tail tiles); one 256-thread workgroup per
// 64-token tile.
// =====================================================================

struct RestoreParams {
    const uint8_t *codes;
    int codes_unpacked;
    const uint16_t *norms, *mins, *scales;
    int64_t n_blocks, in_outer_blocks;
    void *out;
    int64_t out_outer_tokens;
    const void *tail;
    int64_t tail_len, tail_outer_tokens;
    int64_t tiles_per_outer;
    int32_t *status;
};

template <int BITS, int OUT_DT, int TAIL_DT>
__global__ __launch_bounds__(256) void restore_kernel(RestoreParams p) {
    using TO = typename Elem<OUT_DT>::T;
    __shared__ float m_s[kDim], s_s[kDim], n_s[kBlockTok];
    __shared__ double rden_s[kBlockTok];
    __shared__ uint32_t codes_s[kBlockTok * kDim / 4];

    const int tid = threadIdx.x;
    const int64_t o = blockIdx.x / p.tiles_per_outer;
    const int64_t i = blockIdx.x - o * p.tiles_per_outer;
    TO *out = static_cast<TO *>(p.out) + o * p.out_outer_tokens * kDim;
    const int cg = tid & 15, r0 = tid >> 4;
    bool bad = false;

    if (i >= p.n_blocks) {
        // tail tile: convert tokens [64*(i-n_blocks), ...) of the tail
        using TT = typename Elem<TAIL_DT>::T;
        const TT *tail = static_cast<const TT *>(p.tail) + o * p.tail_outer_tokens * kDim;
        const int64_t t0 = (i - p.n_blocks) * kBlockTok;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t t = t0 + r0 + 16 * j;
            if (t < p.tail_len) {
                float v[8];
                load_row8<TAIL_DT>(tail + t * kDim + 8 * cg, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[e] = Elem<OUT_DT>::load(Elem<OUT_DT>::store(v[e]));
                    bad |= !finite(v[e]);
                }
                store_row8<OUT_DT>(out + (p.n_blocks * kBlockTok + t) * kDim + 8 * cg, v);
            }
        }
        if (bad) raise_status(p.status, NSN_ST_NONFINITE_RESTORE);
        return;
    }

    const int64_t ib = o * p.in_outer_blocks + i;
    if (tid < kDim) {
        m_s[tid] = f16_bits_to_f32(p.mins[ib * kDim + tid]);
        s_s[tid] = f16_bits_to_f32(p.scales[ib * kDim + tid]);
    } else if (tid < kDim + kBlockTok) {
        n_s[tid - kDim] = f16_bits_to_f32(p.norms[ib * kBlockTok + tid - kDim]);
    }
    {
        const int g = tid;
        uint32_t c4[8];
        if (p.codes_unpacked) {
            const uint4 *src = reinterpret_cast<const uint4 *>(p.codes + ib * (kBlockTok * kDim)) + 2 * g;
            const uint4 a = src[0], b = src[1];
            c4[0] = a.x; c4[1] = a.y; c4[2] = a.z; c4[3] = a.w;
            c4[4] = b.x; c4[5] = b.y; c4[6] = b.z; c4[7] = b.w;
        } else {
            const uint32_t *src = reinterpret_cast<const uint32_t *>(p.codes + ib * packed_block_bytes(BITS)) + g * BITS;
            uint32_t w[BITS];
#pragma unroll
            for (int k = 0; k < BITS; ++k) w[k] = src[k];
            uint32_t c[32];
            unpack32<BITS>(w, c);
#pragma unroll
            for (int k = 0; k < 8; ++k) c4[k] = c[4 * k] | (c[4 * k + 1] << 8) | (c[4 * k + 2] << 16) | (c[4 * k + 3] << 24);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) codes_s[g * 8 + k] = c4[k];
    }
    __syncthreads();

    // norm of d = m + s*q in torch's 8-lane order (rows are contiguous)
    {
        const int r = tid >> 2, jp = (tid & 3) * 2;
        const uint8_t *cr = reinterpret_cast<const uint8_t *>(codes_s) + r * kDim;
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int c = 8 * k + jp;
            const float p0 = s_s[c] * static_cast<float>(cr[c]);
            const float p1 = s_s[c + 1] * static_cast<float>(cr[c + 1]);
            const float d0 = m_s[c] + p0, d1 = m_s[c + 1] + p1;
            a0 = __builtin_fmaf(d0, d0, a0);
            a1 = __builtin_fmaf(d1, d1, a1);
        }
        const float b0 = __shfl_down(a0, 1), b1 = __shfl_down(a1, 1);
        const float c0 = __shfl_down(a0, 2), c1 = __shfl_down(a1, 2);
        const float d0 = __shfl_down(a0, 3), d1 = __shfl_down(a1, 3);
        if ((tid & 3) == 0) {
            const float acc[8] = {a0, a1, b0, b1, c0, c1, d0, d1};
            rden_s[r] = recip_rn(clamp_eps(sqrt_rn(lane8_sum(acc))));
        }
    }
    __syncthreads();

#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + 16 * j;
        const uint8_t *cr = reinterpret_cast<const uint8_t *>(codes_s) + r * kDim;
        const float n = n_s[r];
        const double rd = rden_s[r];
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = 8 * cg + e;
            const float prod = s_s[c] * static_cast<float>(cr[c]);
            const float d = m_s[c] + prod;
            const float val = n * div_by_recip(d, rd);
            y[e] = (n == 0.f) ? 0.f : val;
            y[e] = Elem<OUT_DT>::load(Elem<OUT_DT>::store(y[e]));
            bad |= !finite(y[e]);
        }
        store_row8<OUT_DT>(out + (i * kBlockTok + r) * kDim + 8 * cg, y);
    }
    if (bad) raise_status(p.status, NSN_ST_NONFINITE_RESTORE);
}

// =====================================================================
// Decode factors of existing packed blocks (one 256-thread group per block).
// =====================================================================

template <int BITS>
__global__ __launch_bounds__(256) void factor_kernel(const uint8_t *codes, const uint16_t *norms, const uint16_t *mins,
                                                     const uint16_t *scales, int64_t n_blocks, int64_t in_outer_blocks,
                                                     float *factors, int32_t *status) {
    __shared__ float m_s[kDim], s_s[kDim], n_s[kBlockTok];
    __shared__ uint32_t codes_s[kBlockTok * kDim / 4];
    const int tid = threadIdx.x;
    const int64_t o = blockIdx.x / n_blocks, i = blockIdx.x - o * n_blocks;
    const int64_t ib = o * in_outer_blocks + i;
    bool bad = false;   // nonfinite metadata: the block's raw inputs fail the finite check
    if (tid < kDim) {
        m_s[tid] = f16_bits_to_f32(mins[ib * kDim + tid]);
        s_s[tid] = f16_bits_to_f32(scales[ib * kDim + tid]);
        bad = !finite(m_s[tid]) || !finite(s_s[tid]);
    } else if (tid < kDim + kBlockTok) {
        n_s[tid - kDim] = f16_bits_to_f32(norms[ib * kBlockTok + tid - kDim]);
        bad = !finite(n_s[tid - kDim]);
    }
    if (bad && status) raise_status(status, NSN_ST_NONFINITE_ATTN_INPUT);
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(codes + ib * packed_block_bytes(BITS)) + tid * BITS;
        uint32_t w[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) w[k] = src[k];
        uint32_t c[32];
        unpack32<BITS>(w, c);
#pragma unroll
        for (int k = 0; k < 8; ++k) codes_s[tid * 8 + k] = c[4 * k] | (c[4 * k + 1] << 8) | (c[4 * k + 2] << 16) | (c[4 * k + 3] << 24);
    }
    __syncthreads();
    block_factors_lds(reinterpret_cast<const uint8_t *>(codes_s), m_s, s_s, n_s, factors + ib * kBlockTok);
}

// =====================================================================
// Finite scan over up to 16 arrays.
// =====================================================================

struct ScanParams {
    const void *ptr[16];
    int64_t count[16];
    int dtype[16];
    int n;
    int32_t *flags;
    int32_t *status;
};

__global__ __launch_bounds__(256) void finite_scan_kernel(ScanParams p) {
    const int a = blockIdx.y;
    const int64_t n = p.count[a];
    bool bad = false;
    for (int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; k < n;
         k += static_cast<int64_t>(gridDim.x) * 256) {
        float v;
        if (p.dtype[a] == NSN_DTYPE_F32) v = static_cast<const float *>(p.ptr[a])[k];
        else if (p.dtype[a] == NSN_DTYPE_F16) v = f16_bits_to_f32(static_cast<const uint16_t *>(p.ptr[a])[k]);
        else v = bf16_bits_to_f32(static_cast<const uint16_t *>(p.ptr[a])[k]);
        bad |= !finite(v);
    }
    if (__any(bad) && (threadIdx.x & 63) == 0) {
        atomicOr(p.flags, 1 << a);
        atomicOr(p.status, NSN_ST_NONFINITE_SCAN);
    }
}

}  // namespace nsn

// =====================================================================
// C ABI
// =====================================================================

using namespace nsn;

namespace {

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
bool bits_ok(int bits) { return bits == 3 || bits == 4 || bits == 5; }
bool dtype_ok(int dt) { return dt == NSN_DTYPE_F16 || dt == NSN_DTYPE_BF16 || dt == NSN_DTYPE_F32; }
int launch_status() { return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH; }

template <int DT, int BITS, int ORDER>
void encode_launch(hipStream_t s, const EncodeParams &p) {
    hipLaunchKernelGGL((encode_kernel<DT, BITS, ORDER>), dim3(static_cast<unsigned>(p.total)), dim3(256), 0, s, p);
}

template <int DT, int BITS>
void encode_dispatch_order(int order, hipStream_t s, const EncodeParams &p) {
    if (order == NSN_NORM_SEQUENTIAL) encode_launch<DT, BITS, NSN_NORM_SEQUENTIAL>(s, p);
    else encode_launch<DT, BITS, NSN_NORM_LANES8>(s, p);
}

template <int DT>
void encode_dispatch_bits(int bits, int order, hipStream_t s, const EncodeParams &p) {
    if (bits == 3) encode_dispatch_order<DT, 3>(order, s, p);
    else if (bits == 4) encode_dispatch_order<DT, 4>(order, s, p);
    else encode_dispatch_order<DT, 5>(order, s, p);
}

template <int BITS, int OUT_DT>
void restore_dispatch_tail(int tail_dt, dim3 grid, hipStream_t s, const RestoreParams &p) {
    if (tail_dt == NSN_DTYPE_F16) hipLaunchKernelGGL((restore_kernel<BITS, OUT_DT, NSN_DTYPE_F16>), grid, dim3(256), 0, s, p);
    else if (tail_dt == NSN_DTYPE_BF16) hipLaunchKernelGGL((restore_kernel<BITS, OUT_DT, NSN_DTYPE_BF16>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((restore_kernel<BITS, OUT_DT, NSN_DTYPE_F32>), grid, dim3(256), 0, s, p);
}

template <int BITS>
void restore_dispatch_out(int out_dt, int tail_dt, dim3 grid, hipStream_t s, const RestoreParams &p) {
    if (out_dt == NSN_DTYPE_F16) restore_dispatch_tail<BITS, NSN_DTYPE_F16>(tail_dt, grid, s, p);
    else if (out_dt == NSN_DTYPE_BF16) restore_dispatch_tail<BITS, NSN_DTYPE_BF16>(tail_dt, grid, s, p);
    else restore_dispatch_tail<BITS, NSN_DTYPE_F32>(tail_dt, grid, s, p);
}

}  // namespace

extern "C" {

const char *nsn_version(void) { return "nsn_hip 0.2 gfx950"; }

int64_t nsn_abi_sizeof(int which) {
    switch (which) {
        case 0: return static_cast<int64_t>(sizeof(nsn_kv_side));
        case 1: return static_cast<int64_t>(sizeof(nsn_attn_args));
        case 2: return static_cast<int64_t>(sizeof(nsn_prefill_args));
        case 3: return static_cast<int64_t>(sizeof(nsn_kscore_args));
        default: return -1;
    }
}

int nsn_encode_blocks(const void *x, int x_dtype, int64_t n_outer, int64_t n_blocks, int64_t x_outer_stride,
                      int64_t x_token_offset, int bits, int norm_order, int zero_flat_scale, uint8_t *codes,
                      uint16_t *norms, uint16_t *mins, uint16_t *scales, uint8_t *headers, float *factors,
                      int64_t out_outer_blocks, int64_t out_block_offset, int64_t header_start_token,
                      uint8_t *codes_unpacked, int32_t *status, nsn_stream_t stream) {
    if (n_outer < 0 || n_blocks < 0 || !bits_ok(bits) || !dtype_ok(x_dtype)) return NSN_EINVAL;
    if (norm_order != NSN_NORM_LANES8 && norm_order != NSN_NORM_SEQUENTIAL) return NSN_EINVAL;
    if (n_outer == 0 || n_blocks == 0) return NSN_OK;
    if (!x || !codes || !norms || !mins || !scales) return NSN_EINVAL;
    const int esize = x_dtype == NSN_DTYPE_F32 ? 4 : 2;
    if (!aligned(x, 16) || (x_outer_stride * esize) % 16 || (x_token_offset * kDim * esize) % 16) return NSN_EINVAL;
    if (!aligned(codes, 16) || !aligned(norms, 2) || !aligned(mins, 2) || !aligned(scales, 2)) return NSN_EINVAL;
    if (headers && !aligned(headers, 4)) return NSN_EINVAL;
    if (factors && !aligned(factors, 4)) return NSN_EINVAL;
    if (codes_unpacked && !aligned(codes_unpacked, 16)) return NSN_EINVAL;
    if (out_outer_blocks < out_block_offset + n_blocks) return NSN_EINVAL;
    const int64_t total = n_outer * n_blocks;
    if (total > 0x7fffffff) return NSN_EINVAL;
    EncodeParams p{x, n_blocks, x_outer_stride, x_token_offset, codes, norms, mins, scales, headers, factors,
                   out_outer_blocks, out_block_offset, header_start_token, codes_unpacked, status,
                   zero_flat_scale, total};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (x_dtype == NSN_DTYPE_F16) encode_dispatch_bits<NSN_DTYPE_F16>(bits, norm_order, s, p);
    else if (x_dtype == NSN_DTYPE_BF16) encode_dispatch_bits<NSN_DTYPE_BF16>(bits, norm_order, s, p);
    else encode_dispatch_bits<NSN_DTYPE_F32>(bits, norm_order, s, p);
    return launch_status();
}

int nsn_pack_codes(const uint8_t *codes, int64_t count, int bits, uint8_t *out, int32_t *status,
                   nsn_stream_t stream) {
    if (count < 0 || !bits_ok(bits)) return NSN_EINVAL;
    if (count == 0) return NSN_OK;
    if (!codes || !out) return NSN_EINVAL;
    const int64_t groups = (count + 31) / 32;
    const int64_t nbytes = (count * bits + 7) / 8;
    const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (bits == 3) hipLaunchKernelGGL(pack_kernel<3>, grid, dim3(256), 0, s, codes, count, out, nbytes, status);
    else if (bits == 4) hipLaunchKernelGGL(pack_kernel<4>, grid, dim3(256), 0, s, codes, count, out, nbytes, status);
    else hipLaunchKernelGGL(pack_kernel<5>, grid, dim3(256), 0, s, codes, count, out, nbytes, status);
    return launch_status();
}

int nsn_unpack_codes(const uint8_t *payload, int64_t count, int bits, uint8_t *out, nsn_stream_t stream) {
    if (count < 0 || !bits_ok(bits)) return NSN_EINVAL;
    if (count == 0) return NSN_OK;
    if (!payload || !out) return NSN_EINVAL;
    const int64_t groups = (count + 31) / 32;
    const int64_t nbytes = (count * bits + 7) / 8;
    const dim3 grid(static_cast<unsigned>((groups + 255) / 256));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (bits == 3) hipLaunchKernelGGL(unpack_kernel<3>, grid, dim3(256), 0, s, payload, count, nbytes, out);
    else if (bits == 4) hipLaunchKernelGGL(unpack_kernel<4>, grid, dim3(256), 0, s, payload, count, nbytes, out);
    else hipLaunchKernelGGL(unpack_kernel<5>, grid, dim3(256), 0, s, payload, count, nbytes, out);
    return launch_status();
}

int nsn_restore_blocks(const uint8_t *codes, int codes_are_unpacked, const uint16_t *norms, const uint16_t *mins,
                       const uint16_t *scales, int64_t n_outer, int64_t n_blocks, int64_t in_outer_blocks, int bits,
                       void *out, int out_dtype, int64_t out_outer_tokens, const void *tail, int tail_dtype,
                       int64_t tail_len, int64_t tail_outer_tokens, int32_t *status, nsn_stream_t stream) {
    if (n_outer < 0 || n_blocks < 0 || tail_len < 0 || !bits_ok(bits)) return NSN_EINVAL;
    if (!dtype_ok(out_dtype) || !dtype_ok(tail_dtype)) return NSN_EINVAL;
    const int64_t tail_tiles = (tail_len + kBlockTok - 1) / kBlockTok;
    const int64_t tiles = n_blocks + tail_tiles;
    if (n_outer == 0 || tiles == 0) return NSN_OK;
    if (!out || !aligned(out, 16)) return NSN_EINVAL;
    const int oes = out_dtype == NSN_DTYPE_F32 ? 4 : 2;
    if ((out_outer_tokens * kDim * oes) % 16 || out_outer_tokens < n_blocks * kBlockTok + tail_len) return NSN_EINVAL;
    if (n_blocks > 0) {
        if (!codes || !norms || !mins || !scales || !aligned(codes, 16)) return NSN_EINVAL;
        if (in_outer_blocks < n_blocks) return NSN_EINVAL;
    }
    if (tail_len > 0) {
        const int tes = tail_dtype == NSN_DTYPE_F32 ? 4 : 2;
        if (!tail || !aligned(tail, 16) || (tail_outer_tokens * kDim * tes) % 16 || tail_outer_tokens < tail_len)
            return NSN_EINVAL;
    }
    if (n_outer * tiles > 0x7fffffff) return NSN_EINVAL;
    RestoreParams p{codes, codes_are_unpacked, norms, mins, scales, n_blocks, in_outer_blocks, out,
                    out_outer_tokens, tail, tail_len, tail_outer_tokens, tiles, status};
    const dim3 grid(static_cast<unsigned>(n_outer * tiles));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (bits == 3) restore_dispatch_out<3>(out_dtype, tail_dtype, grid, s, p);
    else if (bits == 4) restore_dispatch_out<4>(out_dtype, tail_dtype, grid, s, p);
    else restore_dispatch_out<5>(out_dtype, tail_dtype, grid, s, p);
    return launch_status();
}

int nsn_block_factors(const uint8_t *codes, const uint16_t *norms, const uint16_t *mins, const uint16_t *scales,
                      int64_t n_outer, int64_t n_blocks, int64_t in_outer_blocks, int bits, float *factors,
                      int32_t *status, nsn_stream_t stream) {
    if (n_outer < 0 || n_blocks < 0 || !bits_ok(bits) || in_outer_blocks < n_blocks) return NSN_EINVAL;
    if (n_outer == 0 || n_blocks == 0) return NSN_OK;
    if (!codes || !norms || !mins || !scales || !factors || !aligned(codes, 16)) return NSN_EINVAL;
    if (n_outer * n_blocks > 0x7fffffff) return NSN_EINVAL;
    const dim3 grid(static_cast<unsigned>(n_outer * n_blocks));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (bits == 3)
        hipLaunchKernelGGL(factor_kernel<3>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks,
                           factors, status);
    else if (bits == 4)
        hipLaunchKernelGGL(factor_kernel<4>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks,
                           factors, status);
    else
        hipLaunchKernelGGL(factor_kernel<5>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks,
                           factors, status);
    return launch_status();
}

int nsn_finite_scan(int n_arrays, const void *const *ptrs, const int64_t *counts, const int *dtypes, int32_t *flags,
                    int32_t *status, nsn_stream_t stream) {
    if (n_arrays < 0 || n_arrays > 16 || !flags || !status) return NSN_EINVAL;
    if (n_arrays == 0) return NSN_OK;
    ScanParams p{};
    int64_t maxn = 0;
    for (int a = 0; a < n_arrays; ++a) {
        if (counts[a] < 0 || !dtype_ok(dtypes[a]) || (counts[a] > 0 && !ptrs[a])) return NSN_EINVAL;
        p.ptr[a] = ptrs[a];
        p.count[a] = counts[a];
        p.dtype[a] = dtypes[a];
        maxn = counts[a] > maxn ? counts[a] : maxn;
    }
    p.n = n_arrays;
    p.flags = flags;
    p.status = status;
    int64_t bx = (maxn + 255) / 256;
    bx = bx < 1 ? 1 : (bx > 1024 ? 1024 : bx);
    hipLaunchKernelGGL(finite_scan_kernel, dim3(static_cast<unsigned>(bx), n_arrays), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), p);
    return launch_status();
}

}  // extern "C"
