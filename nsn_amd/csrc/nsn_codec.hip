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
#include "nsn_common.hpp"

namespace nsn {

// =====================================================================
// Encoder: one 256-thread workgroup per 64x128 block.
//
// Thread tid holds rows r0 + 16*j (r0 = tid / 16, j = 0..3) x channels
// 8*cg .. 8*cg+7 (cg = tid % 16): each global load is 16 contiguous bytes
// and a wave reads 1 KiB of consecutive input.  The block is also staged in
// LDS (fp32) for the norm, whose summation order must be torch's.
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

template <int DT, int BITS, int ORDER>
__global__ __launch_bounds__(256) void encode_kernel(EncodeParams p) {
    using T = typename Elem<DT>::T;
    constexpr float kLevels = static_cast<float>((1 << BITS) - 1);
    // The input block (in its own type) is only read by the norm pass; the
    // min/max partials and then the unpacked codes reuse its bytes.  Keeping
    // the block at 2 bytes per element (fp16/bf16 inputs) holds the LDS to
    // ~22 KB, so that six blocks share a CU.
    constexpr int kXBytes = kBlockTok * kXPadT * static_cast<int>(sizeof(T));
    static_assert(kXBytes >= 8192 + 2 * 4 * kDim * 4, "LDS aliasing");
    __shared__ __align__(16) uint8_t xraw[kXBytes];
    T *const xs = reinterpret_cast<T *>(xraw);
    uint32_t *const codes_s = reinterpret_cast<uint32_t *>(xraw);                  // bytes [0, 8K): after the norms
    float (*const redmin)[kDim] = reinterpret_cast<float (*)[kDim]>(xraw + 8192);   // [8K, 10K)
    float (*const redmax)[kDim] = reinterpret_cast<float (*)[kDim]>(xraw + 10240);  // [10K, 12K)
    __shared__ float nrm_s[kBlockTok];
    __shared__ double rden_s[kBlockTok];
    __shared__ float m_s[kDim];
    __shared__ double rs_s[kDim];
    __shared__ float mh_s[kDim], sh_s[kDim], nh_s[kBlockTok];
    __shared__ int bad_s;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int64_t blk = blockIdx.x;
    const int64_t o = blk / p.n_blocks, i = blk - o * p.n_blocks;
    const int64_t ob = o * p.out_outer_blocks + p.out_block_offset + i;
    const T *x = static_cast<const T *>(p.x) + o * p.x_outer_stride + (p.x_token_offset + i * kBlockTok) * kDim;

    if (tid == 0) bad_s = 0;
    const int cg = tid & 15, r0 = tid >> 4;
    float v[4][8];
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + 16 * j;
        const T *src = x + r * kDim + 8 * cg;
        T *dst = xs + r * kXPadT + 8 * cg;
        if constexpr (DT == NSN_DTYPE_F32) {
            load_row8<DT>(src, v[j]);
            *reinterpret_cast<float4 *>(dst) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
            *reinterpret_cast<float4 *>(dst + 4) = make_float4(v[j][4], v[j][5], v[j][6], v[j][7]);
        } else {
            const uint4 a = *reinterpret_cast<const uint4 *>(src);
            *reinterpret_cast<uint4 *>(dst) = a;
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[j][2 * k] = Elem<DT>::load(static_cast<uint16_t>(w[k] & 0xffffu));
                v[j][2 * k + 1] = Elem<DT>::load(static_cast<uint16_t>(w[k] >> 16));
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) bad |= !finite(v[j][e]);
    }
    __syncthreads();
    if (bad) bad_s = 1;

    // ---- token norms, in torch's order ----
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
        const float b0 = __shfl_down(a0, 1), b1 = __shfl_down(a1, 1);
        const float c0 = __shfl_down(a0, 2), c1 = __shfl_down(a1, 2);
        const float d0 = __shfl_down(a0, 3), d1 = __shfl_down(a1, 3);
        if ((tid & 3) == 0) {
            const float acc[8] = {a0, a1, b0, b1, c0, c1, d0, d1};
            const float n = sqrt_rn(lane8_sum(acc));
            nrm_s[r] = n;
            rden_s[r] = recip_rn(clamp_eps(n));
        }
    } else {
        if (tid < kBlockTok) {
            float s = 0.f;
            for (int c = 0; c < kDim; ++c) {
                const float q = Elem<DT>::load(xs[tid * kXPadT + c]);
                s = __builtin_fmaf(q, q, s);
            }
            const float n = sqrt_rn(s);
            nrm_s[tid] = n;
            rden_s[tid] = recip_rn(clamp_eps(n));
        }
    }
    __syncthreads();

    // ---- directions d = x / max(n, eps) and per-channel min / max ----
    float mn[8], mx[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const double rd = rden_s[r0 + 16 * j];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = div_by_recip(v[j][e], rd);
            v[j][e] = d;
            if (j == 0) { mn[e] = d; mx[e] = d; }
            else { mn[e] = d < mn[e] ? d : mn[e]; mx[e] = d > mx[e] ? d : mx[e]; }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            const float a = __shfl_xor(mn[e], off), b = __shfl_xor(mx[e], off);
            mn[e] = a < mn[e] ? a : mn[e];
            mx[e] = b > mx[e] ? b : mx[e];
        }
    }
    if ((tid & 63) < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) { redmin[wave][8 * cg + e] = mn[e]; redmax[wave][8 * cg + e] = mx[e]; }
    }
    __syncthreads();

    int meta_flags = 0;
    if (tid < kDim) {
        float lo = redmin[0][tid], hi = redmax[0][tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            lo = redmin[w][tid] < lo ? redmin[w][tid] : lo;
            hi = redmax[w][tid] > hi ? redmax[w][tid] : hi;
        }
        const float s = div_by_recip(hi - lo, recip_rn(kLevels));
        m_s[tid] = lo;
        // 1/s; for s == 0 the reference divides by 1 (every d - m is 0 then),
        // or zeroes the codes when zero_flat_scale is set: a factor of 0
        rs_s[tid] = (s == 0.f) ? (p.zero_flat_scale ? 0.0 : 1.0) : recip_rn(s);
        const uint16_t hm = f32_to_f16_bits(lo), hs = f32_to_f16_bits(s);
        p.mins[ob * kDim + tid] = hm;
        p.scales[ob * kDim + tid] = hs;
        mh_s[tid] = f16_bits_to_f32(hm);
        sh_s[tid] = f16_bits_to_f32(hs);
        if ((hm & 0x7c00u) == 0x7c00u || (hs & 0x7c00u) == 0x7c00u) meta_flags |= NSN_ST_META_NONFINITE;
        if (s != 0.f && (hs & 0x7fffu) == 0) meta_flags |= NSN_ST_META_UNDERFLOW;
    } else if (tid < kDim + kBlockTok) {
        const int t = tid - kDim;
        const float n = nrm_s[t];
        const uint16_t hn = f32_to_f16_bits(n);
        p.norms[ob * kBlockTok + t] = hn;
        nh_s[t] = f16_bits_to_f32(hn);
        if ((hn & 0x7c00u) == 0x7c00u) meta_flags |= NSN_ST_META_NONFINITE;
        if (n != 0.f && (hn & 0x7fffu) == 0) meta_flags |= NSN_ST_META_UNDERFLOW;
    }
    __syncthreads();

    // ---- codes: clamp(round_half_even((d - m) / s), 0, 2^b - 1) ----
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = 8 * cg + e;
            const float t = v[j][e] - m_s[c];
            // clamp(round_half_even(t / s), 0, 2^b - 1); t is finite for valid input
            const float qf = __builtin_amdgcn_fmed3f(__builtin_rintf(div_by_recip(t, rs_s[c])), 0.f, kLevels);
            packed[e >> 2] |= static_cast<uint32_t>(qf) << (8 * (e & 3));
        }
        const int r = r0 + 16 * j;
        codes_s[r * 32 + 2 * cg] = packed[0];
        codes_s[r * 32 + 2 * cg + 1] = packed[1];
    }
    __syncthreads();

    // ---- pack: thread g packs codes 32g .. 32g+31 (row g/4) into BITS dwords ----
    {
        const int g = tid;
        uint32_t c[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t w4 = codes_s[g * 8 + k];
            c[4 * k] = w4 & 0xffu; c[4 * k + 1] = (w4 >> 8) & 0xffu;
            c[4 * k + 2] = (w4 >> 16) & 0xffu; c[4 * k + 3] = w4 >> 24;
        }
        uint32_t w[BITS];
        pack32<BITS>(c, w);
        uint32_t *dst = reinterpret_cast<uint32_t *>(p.codes + ob * packed_block_bytes(BITS)) + g * BITS;
#pragma unroll
        for (int k = 0; k < BITS; ++k) dst[k] = w[k];
        if (p.codes_unpacked) {
            uint4 *du = reinterpret_cast<uint4 *>(p.codes_unpacked + (o * p.n_blocks + i) * (kBlockTok * kDim)) + 2 * g;
            du[0] = make_uint4(codes_s[g * 8], codes_s[g * 8 + 1], codes_s[g * 8 + 2], codes_s[g * 8 + 3]);
            du[1] = make_uint4(codes_s[g * 8 + 4], codes_s[g * 8 + 5], codes_s[g * 8 + 6], codes_s[g * 8 + 7]);
        }
    }
    if (p.factors)
        block_factors_lds(reinterpret_cast<const uint8_t *>(codes_s), mh_s, sh_s, nh_s, p.factors + ob * kBlockTok);
    if (tid == 0 && p.headers) {
        const uint64_t tok = static_cast<uint64_t>(p.header_start_token + i * kBlockTok);
        uint32_t *h = reinterpret_cast<uint32_t *>(p.headers + ob * 12);
        h[0] = static_cast<uint32_t>(tok);
        h[1] = static_cast<uint32_t>(tok >> 32);
        h[2] = 64u | (static_cast<uint32_t>(BITS) << 16);
    }
    if (tid == 0 && bad_s) meta_flags |= NSN_ST_NONFINITE_INPUT;
    raise_status(p.status, meta_flags);
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
                                                     float *factors) {
    __shared__ float m_s[kDim], s_s[kDim], n_s[kBlockTok];
    __shared__ uint32_t codes_s[kBlockTok * kDim / 4];
    const int tid = threadIdx.x;
    const int64_t o = blockIdx.x / n_blocks, i = blockIdx.x - o * n_blocks;
    const int64_t ib = o * in_outer_blocks + i;
    if (tid < kDim) {
        m_s[tid] = f16_bits_to_f32(mins[ib * kDim + tid]);
        s_s[tid] = f16_bits_to_f32(scales[ib * kDim + tid]);
    } else if (tid < kDim + kBlockTok) {
        n_s[tid - kDim] = f16_bits_to_f32(norms[ib * kBlockTok + tid - kDim]);
    }
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

template <int DT, int BITS>
void encode_dispatch_order(int order, dim3 grid, hipStream_t s, const EncodeParams &p) {
    if (order == NSN_NORM_SEQUENTIAL)
        hipLaunchKernelGGL((encode_kernel<DT, BITS, NSN_NORM_SEQUENTIAL>), grid, dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((encode_kernel<DT, BITS, NSN_NORM_LANES8>), grid, dim3(256), 0, s, p);
}

template <int DT>
void encode_dispatch_bits(int bits, int order, dim3 grid, hipStream_t s, const EncodeParams &p) {
    if (bits == 3) encode_dispatch_order<DT, 3>(order, grid, s, p);
    else if (bits == 4) encode_dispatch_order<DT, 4>(order, grid, s, p);
    else encode_dispatch_order<DT, 5>(order, grid, s, p);
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

const char *nsn_version(void) { return "nsn_hip 0.1 gfx950"; }

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
                   zero_flat_scale};
    const dim3 grid(static_cast<unsigned>(total));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (x_dtype == NSN_DTYPE_F16) encode_dispatch_bits<NSN_DTYPE_F16>(bits, norm_order, grid, s, p);
    else if (x_dtype == NSN_DTYPE_BF16) encode_dispatch_bits<NSN_DTYPE_BF16>(bits, norm_order, grid, s, p);
    else encode_dispatch_bits<NSN_DTYPE_F32>(bits, norm_order, grid, s, p);
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
                      nsn_stream_t stream) {
    if (n_outer < 0 || n_blocks < 0 || !bits_ok(bits) || in_outer_blocks < n_blocks) return NSN_EINVAL;
    if (n_outer == 0 || n_blocks == 0) return NSN_OK;
    if (!codes || !norms || !mins || !scales || !factors || !aligned(codes, 16)) return NSN_EINVAL;
    if (n_outer * n_blocks > 0x7fffffff) return NSN_EINVAL;
    const dim3 grid(static_cast<unsigned>(n_outer * n_blocks));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (bits == 3) hipLaunchKernelGGL(factor_kernel<3>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks, factors);
    else if (bits == 4) hipLaunchKernelGGL(factor_kernel<4>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks, factors);
    else hipLaunchKernelGGL(factor_kernel<5>, grid, dim3(256), 0, s, codes, norms, mins, scales, n_blocks, in_outer_blocks, factors);
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
