// Chunked-prefill attention over a packed K/V context (gfx950).
//
// One chunk of n_q queries per (sequence, q-head) attends the sequence's
// context -- packed 64-token blocks, then an fp16/bf16 tail -- and the chunk's
// own dense K/V, causally (chunk query i sees chunk tokens 0..i).  The
// products run in the chunk's dtype: v_mfma_f32_16x16x32_f16 for fp16 data,
// v_mfma_f32_16x16x32_bf16 for bf16 data (no value is squeezed into the
// fp16 range); a tail of the other dtype is converted as it is staged.  The
// reference path materialises the whole K/V (restore of every packed block
// plus the tail, loop_kv_pk01_cache.py:87-106) and runs dense attention on it;
// here the packed blocks are dequantised tile by tile into LDS and never reach
// HBM in dense form.
//
// Workgroup = 8 waves = 256 consecutive chunk queries of one (b, q-head);
// each wave owns 32 queries (two 16-query MFMA column tiles).  Per 64-token
// block:
//   1. the raw block (K/V codes, K/V min and scale, K/V decode factors; for
//      a tail or chunk block its dense K/V rows) is staged into LDS by DMA
//      two blocks ahead;
//   2. the 512 threads dequantise it once for the workgroup (threads 0-255
//      K', 256-511 V'^T) into K' [64 tok][128 ch] and V'^T [128 ch][64 tok]
//      (the reconstructed values f_t * (m + s*z), rounded to the compute
//      dtype), double-buffered so that the fill of the next block overlaps
//      the products of this one;
//   3. each wave computes S^T = K' Q^T and O^T += V'^T P^T on MFMA -- the
//      transposed products keep P in registers: the C layout of S^T is
//      already the B layout of P^T for a token order in which lane group g
//      of a 32-token step holds tokens 4g..4g+3 of both 16-token tiles.
// Softmax runs in the log2 domain: fp16 queries are pre-scaled by
// scale*log2(e); bf16 queries enter the product exactly and the scores are
// scaled after it.
#include "nsn_common.hpp"

namespace nsn {
namespace prefill {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;                // waves per workgroup
constexpr int kQTile = 32 * kWaves;      // chunk queries per workgroup
// LDS banking on gfx950 (measured): a ds_read_b128 serves lanes 0-31 and
// 32-63 in separate passes and is conflict-free when the 32 lanes of a pass
// hit 32 different 16-byte slots modulo 512 bytes; a ds_write_b32 serves 32
// lanes per pass over 4-byte slots modulo 128 bytes.
constexpr int kKP = 144;      // K' row pitch (halves): 288 B rows, so that the S^T operand reads
                              // (16 rows x 2 lane groups per pass) take 32 different slots
constexpr int kVP = 64;       // V'^T row pitch (halves): 128 B rows, slots kept apart by vchunk
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.f;  // running-maximum slack (log2 units): weights < 2^8

// D = A B + C on the compute dtype CT (NSN_DTYPE_F16 or NSN_DTYPE_BF16).
template <int CT>
__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (CT == NSN_DTYPE_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                       0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0,
                                                      0);
}
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// fp32 pair -> packed pair of the compute dtype (round to nearest even)
template <int CT>
__device__ __forceinline__ uint32_t pk(float a, float b) {
    if constexpr (CT == NSN_DTYPE_BF16) {
        const bf16x2 h = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
        return __builtin_bit_cast(uint32_t, h);
    } else {
        const half2v h = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
        return __builtin_bit_cast(uint32_t, h);
    }
}
// Maxima of scores as single v_max3_f32 / v_max_f32 instructions.  fmaxf
// compiles to the same instructions plus a self-max per operand that the
// compiler cannot prove canonical (MFMA results, lane swaps): the quieting of
// signalling NaNs, which a score never is (a NaN score is a quiet NaN out of
// the MFMA, ignored by the maximum as fmaxf ignores it, and it still reaches
// the output through its weight).  Half the maximum's instructions were those.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float max2f(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// Maximum over the four 16-lane rows of the wave (lanes l, l^16, l^32, l^48),
// on every lane, without LDS: v_permlane16_swap gives rows (0,0,2,2) and
// (1,1,3,3), v_permlane32_swap the halves (lo,lo) and (hi,hi).
__device__ __forceinline__ float rows4_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = max2f(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return max2f(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// fp32 pair -> bf16 hi (round to nearest even) + bf16 lo = rn(x - hi): the
// pair to ~2^-17 relative.
__device__ __forceinline__ void split_bf16(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = pk<NSN_DTYPE_BF16>(a, b);
    lo = pk<NSN_DTYPE_BF16>(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}
__device__ __forceinline__ float h16(uint32_t w, int hi) {
    return static_cast<float>(__builtin_bit_cast(half2v, w)[hi]);
}

// Channel order inside each group of 8 (the K' columns and the Q
// fragments share it): element p holds channel chE[p], whose 3-bit code the
// unpack leaves at bit kE[p] of an fp16 half (a subnormal z * 2^(kE-24)).
template <int BITS> struct Order;
template <> struct Order<3> {
    static constexpr int chE[8] = {0, 3, 1, 4, 2, 5, 6, 7};
    static constexpr int kE[8] = {0, 1, 3, 4, 6, 7, 2, 5};
};
template <> struct Order<5> {
    static constexpr int chE[8] = {0, 1, 2, 3, 4, 5, 6, 7};
    static constexpr int kE[8] = {0, 0, 0, 0, 0, 0, 0, 0};
};

// The 8 codes of one token's 8-channel group, from the staged code bytes:
// 4 dwords, element p (dword p/2, half p%2) = code of channel chE[p] at bit kE[p].
template <int BITS>
__device__ __forceinline__ void codes8(const uint8_t *row, int cg, uint32_t (&B)[4]) {
    const int byte = BITS * cg;   // the group's first byte within the token row
    const uint32_t *w = reinterpret_cast<const uint32_t *>(row + (byte & ~3));
    const uint32_t sh = 8u * static_cast<uint32_t>(byte & 3);
    const uint32_t x = __builtin_amdgcn_alignbit(w[1], w[0], sh);
    if constexpr (BITS == 3) {
        const uint32_t P = perm(x, x, 0x02010100u), Q = perm(x, x, 0x0C020C02u);
        B[0] = P & 0x000E0007u;
        B[1] = P & 0x00700038u;
        B[2] = P & 0x038001C0u;
        B[3] = Q & 0x00E0001Cu;
    } else {
        const uint32_t y = __builtin_amdgcn_alignbit(w[2], w[1], sh);   // code bits 32..63
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t z[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int e = 2 * i + h;
                z[h] = (e < 6) ? __builtin_amdgcn_ubfe(x, 5 * e, 5)
                     : (e == 6) ? (__builtin_amdgcn_alignbit(y, x, 30) & 31u)
                                : ((y >> 3) & 31u);
            }
            B[i] = z[0] | (z[1] << 16);
        }
    }
}

struct Side {
    const uint8_t *codes;
    const uint16_t *mins, *scales;
    const float *factors;
    const int32_t *blocks;
    int64_t block_cap;
    const uint16_t *tail;   // TDT
    int64_t tail_cap;
};

struct PrefillParams {
    const uint16_t *q;     // [B, Hq, n_q, 128] DT
    int64_t batch, heads_q, heads_kv, n_q;
    int group;
    float qscale;          // scale * log2(e)
    const int32_t *ctx_len;
    Side k, v;
    const uint16_t *kc, *vc;   // chunk K/V [B, Hkv, n_q, 128] DT
    uint16_t *out;             // [B, Hq, n_q, 128] DT
    int32_t *status;
    uint16_t *ka, *va;         // append: the K / V tails written (TDT), else null
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 16 bytes per lane from global memory straight into LDS at M0 + 16*lane,
// with the non-temporal hint: a workgroup streams each block of its context
// once (C4 last chunk 1241-1242 -> 1222-1228 us).
__device__ __forceinline__ void dma16(const void *src, void *dst) {
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds) : "memory", "m0");
}
#pragma clang diagnostic pop

// Staged block layout (bytes): [K codes NB | V codes NB | K min 256 | K scale 256 |
// V min 256 | V scale 256 | K factor 256 | V factor 256].
template <int BITS> struct Stage {
    static constexpr int NB = packed_block_bytes(BITS);
    static constexpr int META = 2 * NB;
    static constexpr int BYTES = 2 * NB + 1536;
    static constexpr int NI = 2 * NB / 1024 + 2;   // 1 KiB DMA instructions per block
};

// DMA of packed block ib of (b, kvh) into one stage; instruction i of the
// block is issued by wave i % kWaves.
template <int BITS>
__device__ __forceinline__ void stage_block(const PrefillParams &p, int64_t rk, int64_t rv, int wave, int l,
                                            uint8_t *st) {
    using S = Stage<BITS>;
    const int q = l & 15;
    for (int i = wave; i < S::NI; i += kWaves) {
        if (i < S::NB / 1024) {
            dma16(p.k.codes + rk * S::NB + 1024 * i + 16 * l, st + 1024 * i);
        } else if (i < 2 * S::NB / 1024) {
            const int c = i - S::NB / 1024;
            dma16(p.v.codes + rv * S::NB + 1024 * c + 16 * l, st + S::NB + 1024 * c);
        } else if (i == 2 * S::NB / 1024) {
            const uint16_t *src = (l < 16) ? p.k.mins + rk * kDim : (l < 32) ? p.k.scales + rk * kDim
                                : (l < 48) ? p.v.mins + rv * kDim : p.v.scales + rv * kDim;
            dma16(src + 8 * q, st + S::META);
        } else if (l < 32) {
            const float *src = (l < 16) ? p.k.factors + rk * kBlockTok : p.v.factors + rv * kBlockTok;
            dma16(src + 4 * q, st + S::META + 1024);
        }
    }
}

// A dense block (tail or chunk tokens, 2-byte elements) is staged by DMA
// like a packed one: K rows then V rows, 256 B each.  The 16-byte chunk c of
// row t sits at chunk position c ^ ((t >> 2) & 15) of the row, so that the
// 16 lanes of either fill role's reads (one row, 16 chunks; or 16 rows 4
// apart, one chunk) fall on 16 different bank groups.
constexpr int kDenseStage = 2 * kBlockTok * kDim * 2;   // 32 KiB
__device__ __forceinline__ int dswz(int t, int c) { return c ^ ((t >> 2) & 15); }

// DMA of the first `valid` rows of a dense block (K rows from xk, V rows
// from xv, 128-element row pitch) into a stage: instruction i writes rows
// 4*(i%16) .. +3 of side i/16 and is issued by wave i % kWaves; lane l
// writes chunk position l%16 of row l/16 and so reads chunk dswz(row, l%16).
// Rows past `valid` are neither read nor written.
__device__ __forceinline__ void stage_dense(const uint16_t *xk, const uint16_t *xv, int valid, int wave, int l,
                                            uint8_t *st) {
    const int r = l >> 4, cp = l & 15;
    for (int i = wave; i < 32; i += kWaves) {
        if (4 * (i & 15) >= valid) continue;   // (wave-uniform)
        const int t = 4 * (i & 15) + r;
        if (t < valid) dma16(((i < 16) ? xk : xv) + t * kDim + 8 * dswz(t, cp), st + 1024 * i);
    }
}

// V'^T keeps each channel's 64 tokens in the k order of the PV product:
// token t = 32a + 16h + 4g + i sits at position 32a + 8g + 4h + i, so the 8
// tokens that lane group g of 32-token step a contracts (4g..4g+3 of both
// 16-token tiles) are one 16-byte read.  Groups of 4 tokens stay together.
__device__ __forceinline__ int vpos(int t) {
    return (t & 32) | ((t & 12) << 1) | ((t & 16) >> 2) | (t & 3);
}

// V'^T row `r` keeps its 16-byte chunk c at position c ^ x(r), x(r) = 4 * bit 2
// of r + 2 * bit 3 of r.  Rows are 128 B, so rows r, r+4, r+8, r+12 start on
// the same banks:
//  - a PV operand read pass (rows 16*ct + 0..15, chunks c and c+1) gives
//    those four rows four different XORs in {0, 2, 4, 6}: 32 different slots;
//  - a fill write pass (32 lanes: 16 token groups of rows r and r+8) writes,
//    in each 16-byte chunk, the two words whose parity is bit 1 of the
//    chunk's index (fill_packed's pair order); x(r+8) = x(r) ^ 2 flips that
//    bit, so row r+8 writes the other two words of every chunk position and
//    the pass takes 32 different banks.
__device__ __forceinline__ int vchunk(int r, int c) { return c ^ ((r & 4) | ((r >> 2) & 2)); }
__device__ __forceinline__ int vcol_at(int r, int t) { return 8 * vchunk(r, vpos(t) >> 3) + (vpos(t) & 7); }

// The block buffer compute reads: K' [64 tok][kKP], V'^T [128 ch][kVP].
struct KV {
    uint16_t *kt, *vt;
};

// Fill one side of a KV buffer from a staged dense block of dtype DT
// (`valid` rows; rows past it are zero), rounded to CT.  Thread: tokens
// 4*rg .. 4*rg+3, channels 8*cg .. 8*cg+7; side 0 writes K' rows, side 1
// V'^T columns.  `app` (nullable): the block's rows also go to app + t*128,
// rounded to ADT (the chunk's append to the tail).
template <int BITS, int DT, int CT, int side, int ADT>
__device__ __forceinline__ void fill_dense(const uint8_t *st, int valid, int rg, int cg, const KV &kv,
                                           uint16_t *app) {
    using O = Order<BITS>;
    uint32_t vcol[8][2];   // V'^T: per channel, tokens 4rg..4rg+3 as 2 fp16 pairs
    float vprev[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = 4 * rg + i;
        float f[8];
        if (t < valid) {
            const uint4 a = *reinterpret_cast<const uint4 *>(st + kDenseStage / 2 * side + 256 * t + 16 * dswz(t, cg));
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = Elem<DT>::load(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
            if (app) {
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = static_cast<uint32_t>(Elem<ADT>::store(f[2 * e])) |
                           (static_cast<uint32_t>(Elem<ADT>::store(f[2 * e + 1])) << 16);
                *reinterpret_cast<uint4 *>(app + t * kDim + 8 * cg) = uint4{o[0], o[1], o[2], o[3]};
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = 0.f;
        }
        if constexpr (side == 0) {
            *reinterpret_cast<uint4 *>(kv.kt + t * kKP + 8 * cg) =
                uint4{pk<CT>(f[O::chE[0]], f[O::chE[1]]), pk<CT>(f[O::chE[2]], f[O::chE[3]]),
                      pk<CT>(f[O::chE[4]], f[O::chE[5]]), pk<CT>(f[O::chE[6]], f[O::chE[7]])};
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                if (i & 1) vcol[e][i >> 1] = pk<CT>(vprev[e], f[e]);
                else vprev[e] = f[e];
            }
        }
    }
    if constexpr (side == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            *reinterpret_cast<u32x2 *>(kv.vt + (8 * cg + e) * kVP + vcol_at(8 * cg + e, 4 * rg)) =
                u32x2{vcol[e][0], vcol[e][1]};
    }
}

// Fill one side of a KV buffer from a staged packed block: direction m + s*z
// per element (one fma with the code as an exact fp16 subnormal, scaled back
// by 2^(24-k)) times the token's decode factor -- the reconstructed value
// itself (|x| <= its fp16 norm, so within fp16 range by construction),
// rounded to CT.
template <int BITS, int CT, int side>
__device__ __forceinline__ void fill_packed(const uint8_t *st, int rg, int cg, const KV &kv) {
    using S = Stage<BITS>;
    using O = Order<BITS>;
    constexpr int ROWB = BITS * 16;   // code bytes per token row
    const uint4 m4 = *reinterpret_cast<const uint4 *>(st + S::META + 512 * side + 16 * cg);
    const uint4 s4 = *reinterpret_cast<const uint4 *>(st + S::META + 512 * side + 256 + 16 * cg);
    const float4 f4 = *reinterpret_cast<const float4 *>(st + S::META + 1024 + 256 * side + 16 * rg);
    const float fac[4] = {f4.x, f4.y, f4.z, f4.w};
    const uint32_t M[4] = {m4.x, m4.y, m4.z, m4.w}, SC[4] = {s4.x, s4.y, s4.z, s4.w};
    float mE[8], sE[8];   // per element p (channel chE[p])
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const int c = O::chE[p];
        mE[p] = h16(M[c >> 1], c & 1);
        sE[p] = h16(SC[c >> 1], c & 1) * static_cast<float>(1u << (24 - O::kE[p]));
    }
    const uint8_t *codes = st + S::NB * side;
    // V side (lanes = token groups): rows 4*rg are 48 B = 16 banks apart, so
    // the lanes of a pass alternate the order of their two token pairs
    // (4-way instead of 8-way bank sharing on the code reads).  Register slot
    // s holds pair s ^ pfirst; only the addresses change.
    const int pfirst = (side == 1) ? ((rg >> 1) & 1) : 0;
    uint32_t vcol[8][2];
    float vprev[8];
#pragma unroll
    for (int slot = 0; slot < 2; ++slot) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = 4 * rg + 2 * (slot ^ pfirst) + h;
            const float ft = pfirst ? fac[2 * (slot ^ 1) + h] : fac[2 * slot + h];
            uint32_t b[4];
            codes8<BITS>(codes + t * ROWB, cg, b);
            float d[8];
#pragma unroll
            for (int p = 0; p < 8; ++p) d[p] = __builtin_fmaf(h16(b[p >> 1], p & 1), sE[p], mE[p]) * ft;
            if constexpr (side == 0) {
                *reinterpret_cast<uint4 *>(kv.kt + t * kKP + 8 * cg) =
                    uint4{pk<CT>(d[0], d[1]), pk<CT>(d[2], d[3]), pk<CT>(d[4], d[5]), pk<CT>(d[6], d[7])};
            } else {
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    if (h) vcol[p][slot] = pk<CT>(vprev[p], d[p]);
                    else vprev[p] = d[p];
                }
            }
        }
    }
    if constexpr (side == 1) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            uint16_t *dst = kv.vt + (8 * cg + O::chE[p]) * kVP + vcol_at(8 * cg + O::chE[p], 4 * rg);
            *reinterpret_cast<uint32_t *>(dst + 2 * pfirst) = vcol[p][0];
            *reinterpret_cast<uint32_t *>(dst + 2 * (pfirst ^ 1)) = vcol[p][1];
        }
    }
}

// DT: dtype of the queries, the chunk K/V, the output and the products; TDT:
// dtype of the context tail.  LO (bf16 only): the softmax weights enter the
// PV product and the row sums as bf16 hi + lo (~2^-17 relative) instead of
// one bf16 rounding (2^-9) -- for chunks with little or no context, whose
// first queries attend a handful of tokens, where one weight's bf16 rounding
// moves the output by up to 2^-9 of |v|.  It costs ~24 % more time per
// block (36 more MFMA and ~80 more VALU per wave), so the caller asks for it.
template <int BITS, int DT, int TDT, bool LO>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(PrefillParams p) {
    using S = Stage<BITS>;
    using O = Order<BITS>;
    constexpr bool QPRE = DT == NSN_DTYPE_F16;   // fp16 queries carry scale*log2(e); bf16 ones stay exact
    static_assert(!LO || DT == NSN_DTYPE_BF16, "hi + lo weights are a bf16 form");
    __shared__ __align__(16) uint16_t kt[2][kBlockTok * kKP];
    __shared__ __align__(16) uint16_t vt[2][kDim * kVP];
    __shared__ __align__(16) uint8_t stg[2][S::BYTES > kDenseStage ? S::BYTES : kDenseStage];

    const int tid = threadIdx.x, l = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: the DMA targets are scalar)
    const int row = l & 15, g = l >> 4;
    // fill role: threads 0..255 fill K' (lanes over channel groups: each pass
    // writes whole K' rows), 256..511 V'^T (lanes over token groups: each pass
    // writes one contiguous V'^T row)
    const int side = __builtin_amdgcn_readfirstlane(tid >> 8);   // (wave-uniform)
    const int rg = side ? (tid & 15) : ((tid >> 4) & 15);
    const int cg = side ? ((tid >> 4) & 15) : (tid & 15);
    // Grid (q-head, sequence, query tile), tiles last and in reverse: every
    // workgroup of the last (longest: it sees the most causal chunk blocks)
    // tile is dispatched before any of the shorter ones, so the short ones
    // fill the CUs' last rounds.
    const int hq = blockIdx.x, b = blockIdx.y;
    const int kvh = hq / p.group;
    const int64_t q0 = static_cast<int64_t>(gridDim.z - 1 - blockIdx.z) * kQTile;
    const int64_t qw = q0 + 32 * wave;                     // this wave's first query
    const int64_t seqrow = static_cast<int64_t>(b) * p.heads_kv + kvh;

    // ---- Q fragments (B operand of S^T = K' Q^T): query qw + 16*qt + row,
    // channels 32*ks + 8*g + chE[e] (fp16: times scale*log2(e)); loaded
    // before the context lengths are needed, so the two round trips overlap
    u32x4 qf[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int64_t qi = qw + 16 * qt + row;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float x[8];
            if (qi < p.n_q) {
                const uint4 a = *reinterpret_cast<const uint4 *>(
                    p.q + ((static_cast<int64_t>(b) * p.heads_q + hq) * p.n_q + qi) * kDim + 32 * ks + 8 * g);
                const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[e] = Elem<DT>::load(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1))));
                    if (QPRE) x[e] *= p.qscale;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.f;
            }
            qf[qt][ks] = u32x4{pk<DT>(x[O::chE[0]], x[O::chE[1]]), pk<DT>(x[O::chE[2]], x[O::chE[3]]),
                               pk<DT>(x[O::chE[4]], x[O::chE[5]]), pk<DT>(x[O::chE[6]], x[O::chE[7]])};
        }
    }

    const int64_t T = p.ctx_len[b];
    const int64_t nbk = p.k.blocks ? p.k.blocks[b] : 0;
    const int64_t nbv = p.v.blocks ? p.v.blocks[b] : 0;
    const int64_t nb = nbk;                                // (== nbv, checked below)
    const int64_t ntail = T - nb * kBlockTok;
    const int64_t qend = (q0 + kQTile < p.n_q) ? q0 + kQTile : p.n_q;   // chunk tokens this workgroup sees
    const int64_t nt_blk = (ntail + kBlockTok - 1) / kBlockTok;
    const int64_t nblk = nb + nt_blk + (qend + kBlockTok - 1) / kBlockTok;
    if (nbk != nbv || nb < 0 || (nb > 0 && (nb > p.k.block_cap || nb > p.v.block_cap)) || ntail < 0 ||
        ntail > p.k.tail_cap || ntail > p.v.tail_cap) {
        if (tid == 0) raise_status(p.status, NSN_ST_CAPACITY);   // inconsistent cache (host checks first)
        return;
    }
    // append: the workgroup of the last query tile (it stages every chunk
    // block) of each kv-head's first q-head writes the chunk's K/V to tail
    // rows ntail .. ntail + n_q - 1 as it fills them; no room: flag, no append
    const bool app_wg = p.ka && blockIdx.z == 0 && hq % p.group == 0;
    const bool app_ok = app_wg && ntail + p.n_q <= p.k.tail_cap && ntail + p.n_q <= p.v.tail_cap;
    if (app_wg && !app_ok && tid == 0) raise_status(p.status, NSN_ST_CAPACITY);

    f32x4 acc[8][2];   // O^T tiles [channel tile ct][query tile qt]
#pragma unroll
    for (int ct = 0; ct < 8; ++ct)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) acc[ct][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY};
    // Row sums of the weights on the matrix core: a constant A tile whose row
    // 0 is all ones, so row 0 of lsum[qt] = sum over tokens of the P operand
    // (the rounded weights the PV product uses); lanes 0-15 hold it.
    f32x4 lsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const uint32_t one2 = (row == 0) ? (DT == NSN_DTYPE_BF16 ? 0x3F803F80u : 0x3C003C00u) : 0u;
    const u32x4 ones_a = u32x4{one2, one2, one2, one2};
    bool bad = false;

    // Block j: packed (j < nb), tail (nb <= j < nb + nt_blk), or chunk; its rows
    // in use and (chunk blocks) the chunk position of its first token.
    auto block_rows = [&](int64_t j, int &valid, int64_t &cpos) {
        cpos = -1;
        if (j < nb) {
            valid = kBlockTok;
        } else if (j < nb + nt_blk) {
            const int64_t t0 = (j - nb) * kBlockTok;
            valid = static_cast<int>((ntail - t0 < kBlockTok) ? ntail - t0 : kBlockTok);
        } else {
            cpos = (j - nb - nt_blk) * kBlockTok;
            valid = static_cast<int>((qend - cpos < kBlockTok) ? qend - cpos : kBlockTok);
        }
    };
    // Fill block j into KV buffer j & 1 (its raw stage j & 1 when packed).
    auto fill = [&](int64_t j) {
        const KV kv{kt[j & 1], vt[j & 1]};
        if (j < nb) {
            if (side) fill_packed<BITS, DT, 1>(stg[j & 1], rg, cg, kv);
            else fill_packed<BITS, DT, 0>(stg[j & 1], rg, cg, kv);
        } else {
            int valid;
            int64_t cpos;
            block_rows(j, valid, cpos);
            if (cpos < 0) {
                if (side) fill_dense<BITS, TDT, DT, 1, TDT>(stg[j & 1], valid, rg, cg, kv, nullptr);
                else fill_dense<BITS, TDT, DT, 0, TDT>(stg[j & 1], valid, rg, cg, kv, nullptr);
            } else {
                uint16_t *app = nullptr;
                if (app_ok)
                    app = side ? p.va + (seqrow * p.v.tail_cap + ntail + cpos) * kDim
                               : p.ka + (seqrow * p.k.tail_cap + ntail + cpos) * kDim;
                if (side) fill_dense<BITS, DT, DT, 1, TDT>(stg[j & 1], valid, rg, cg, kv, app);
                else fill_dense<BITS, DT, DT, 0, TDT>(stg[j & 1], valid, rg, cg, kv, app);
            }
        }
    };
    // Stage the raw data of block j into stage j & 1: packed codes and
    // metadata, or the valid rows of its tail / chunk tokens.
    auto stage = [&](int64_t j) {
        if (j < nb) {
            stage_block<BITS>(p, seqrow * p.k.block_cap + j, seqrow * p.v.block_cap + j, wave, l, stg[j & 1]);
        } else {
            int valid;
            int64_t cpos;
            block_rows(j, valid, cpos);
            if (cpos < 0) {
                const int64_t t0 = (j - nb) * kBlockTok;
                stage_dense(p.k.tail + (seqrow * p.k.tail_cap + t0) * kDim,
                            p.v.tail + (seqrow * p.v.tail_cap + t0) * kDim, valid, wave, l, stg[j & 1]);
            } else {
                stage_dense(p.kc + (seqrow * p.n_q + cpos) * kDim, p.vc + (seqrow * p.n_q + cpos) * kDim, valid,
                            wave, l, stg[j & 1]);
            }
        }
    };

    // ---- prologue: raw blocks 0 and 1 staged together (one round trip), block 0 filled
    stage(0);
    if (nblk > 1) stage(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    fill(0);

    // ---- one barrier per block: compute block j from KV buffer j & 1 while
    // filling block j + 1 into the other and staging raw block j + 2
    for (int64_t j = 0; j < nblk; ++j) {
        // KV buffer j & 1 is filled, raw block j + 1 is in, buffer (j + 1) & 1
        // and raw stage j & 1 are free
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (j + 2 < nblk) stage(j + 2);
        if (j + 1 < nblk) fill(j + 1);
        if (qw >= p.n_q) continue;   // (a wave past the chunk end only helps fill)
        int valid;
        int64_t cpos;
        block_rows(j, valid, cpos);
        const uint16_t *ktj = kt[j & 1];
        const uint16_t *vtj = vt[j & 1];

        // ---- S^T[token][query] = K' Q^T
        f32x4 s[4][2];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[tt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const u32x4 a = *reinterpret_cast<const u32x4 *>(ktj + (16 * tt + row) * kKP + 32 * ks + 8 * g);
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) s[tt][qt] = mfma<DT>(a, qf[qt][ks], s[tt][qt]);
            }
        }
        // ---- online softmax per query (lane's query qw + 16*qt + row).  The
        // running maximum (and the state's rescale) only moves when some
        // lane's block maximum exceeds it.
        const bool masked = valid < kBlockTok || cpos >= 0;   // (uniform) partial or causal block
        u32x4 pb[2][2];   // P''^T B operands [ks2][qt] (LO: the bf16 hi parts)
        u32x4 pl[2][2];   // LO: the bf16 lo parts
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            if (masked) {
                // allowed tokens of this block: tok < valid and (chunk blocks) tok <= query - cpos
                const int64_t rel = (cpos >= 0) ? qw + 16 * qt + row - cpos : kBlockTok;
                const int lim = static_cast<int>((rel < valid - 1) ? rel : valid - 1);
#pragma unroll
                for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (16 * tt + 4 * g + i > lim) s[tt][qt][i] = -INFINITY;
            }
            const f32x4 *v = &s[0][qt];   // (stride 2: s[tt][qt] = v[2 * tt])
            const float a0 = max3f(v[0][0], v[0][1], v[0][2]), a1 = max3f(v[0][3], v[2][0], v[2][1]);
            const float a2 = max3f(v[2][2], v[2][3], v[4][0]), a3 = max3f(v[4][1], v[4][2], v[4][3]);
            const float a4 = max3f(v[6][0], v[6][1], v[6][2]);
            float mx = max2f(max3f(a0, a1, a2), max3f(a3, a4, v[6][3]));
            mx = rows4_max(mx);
            if (!QPRE) mx *= p.qscale;   // (bf16: the scores scale inside the exponent below)
            // The running maximum moves only when a score passes it by more
            // than kLazy (log2 units): weights then stay below 2^kLazy, which
            // every weight form holds exactly as well as weights below 1.
            if (__builtin_amdgcn_ballot_w64(mx > m_run[qt] + kLazy)) {
                const float mnew = fmaxf(m_run[qt], mx);
                const float alpha = (m_run[qt] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[qt] - mnew);
                lsum[qt] *= alpha;
#pragma unroll
                for (int ct = 0; ct < 8; ++ct) acc[ct][qt] *= alpha;
                m_run[qt] = mnew;
            }
            const float msafe = (m_run[qt] == -INFINITY) ? 0.f : m_run[qt];
            float pw[4][4];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    pw[tt][i] = __builtin_amdgcn_exp2f(QPRE ? s[tt][qt][i] - msafe
                                                            : __builtin_fmaf(s[tt][qt][i], p.qscale, -msafe));
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2) {
                if constexpr (LO) {
                    uint32_t h[4], lo[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        split_bf16(pw[2 * ks2 + (e >> 1)][2 * (e & 1)], pw[2 * ks2 + (e >> 1)][2 * (e & 1) + 1], h[e],
                                   lo[e]);
                    pb[ks2][qt] = u32x4{h[0], h[1], h[2], h[3]};
                    pl[ks2][qt] = u32x4{lo[0], lo[1], lo[2], lo[3]};
                } else {
                    pb[ks2][qt] = u32x4{pk<DT>(pw[2 * ks2][0], pw[2 * ks2][1]), pk<DT>(pw[2 * ks2][2], pw[2 * ks2][3]),
                                        pk<DT>(pw[2 * ks2 + 1][0], pw[2 * ks2 + 1][1]),
                                        pk<DT>(pw[2 * ks2 + 1][2], pw[2 * ks2 + 1][3])};
                }
            }
        }
        // ---- O^T[channel][query] += V'^T P''^T (k order: tokens 4g..4g+3 of both 16-token tiles)
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
#pragma unroll
            for (int ks2 = 0; ks2 < 2; ++ks2) {
                const u32x4 a = *reinterpret_cast<const u32x4 *>(vtj + (16 * ct + row) * kVP +
                                                                 8 * vchunk(16 * ct + row, 4 * ks2 + g));
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) {
                    acc[ct][qt] = mfma<DT>(a, pb[ks2][qt], acc[ct][qt]);
                    if constexpr (LO) acc[ct][qt] = mfma<DT>(a, pl[ks2][qt], acc[ct][qt]);
                }
            }
        }
#pragma unroll
        for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                lsum[qt] = mfma<DT>(ones_a, pb[ks2][qt], lsum[qt]);
                if constexpr (LO) lsum[qt] = mfma<DT>(ones_a, pl[ks2][qt], lsum[qt]);
            }
    }

    // ---- output: O[q][c] = O^T / l, channels 16*ct + 4*g + i of query qw + 16*qt + row
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const float lt = __shfl(lsum[qt][0], row);   // (query row's sum, from lane row)
        const int64_t qi = qw + 16 * qt + row;
        if (qi >= p.n_q) continue;
        const float r = 1.f / lt;
        uint16_t *dst = p.out + ((static_cast<int64_t>(b) * p.heads_q + hq) * p.n_q + qi) * kDim;
#pragma unroll
        for (int ct = 0; ct < 8; ++ct) {
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[i] = acc[ct][qt][i] * r;
                bad |= !finite(o[i]);
            }
            const uint32_t w0 = static_cast<uint32_t>(Elem<DT>::store(o[0])) | (static_cast<uint32_t>(Elem<DT>::store(o[1])) << 16);
            const uint32_t w1 = static_cast<uint32_t>(Elem<DT>::store(o[2])) | (static_cast<uint32_t>(Elem<DT>::store(o[3])) << 16);
            *reinterpret_cast<u32x2 *>(dst + 16 * ct + 4 * g) = u32x2{w0, w1};
        }
    }
    if (bad) raise_status(p.status, NSN_ST_NONFINITE_OUTPUT);
}

}  // namespace prefill
}  // namespace nsn

using namespace nsn;

extern "C" int nsn_prefill_attention(const nsn_prefill_args *a, nsn_stream_t stream) {
    using namespace nsn::prefill;
    if (!a || !a->q || !a->ctx_len || !a->k_chunk || !a->v_chunk || !a->out) return NSN_EINVAL;
    if (a->batch <= 0 || a->heads_kv <= 0 || a->heads_q % a->heads_kv || a->n_q < 0) return NSN_EINVAL;
    if (a->n_q == 0) return NSN_OK;
    if (a->bits != 3 && a->bits != 5) return NSN_EINVAL;
    if (a->dtype != NSN_DTYPE_F16 && a->dtype != NSN_DTYPE_BF16) return NSN_EINVAL;
    auto side_ok = [](const nsn_kv_side &s) {
        if (s.blocks && (!s.codes || !s.mins || !s.scales || !s.factors || s.block_cap <= 0)) return false;
        if (s.codes && (reinterpret_cast<uintptr_t>(s.codes) & 15u)) return false;
        if (s.mins && (reinterpret_cast<uintptr_t>(s.mins) & 15u)) return false;
        if (s.scales && (reinterpret_cast<uintptr_t>(s.scales) & 15u)) return false;
        if (s.factors && (reinterpret_cast<uintptr_t>(s.factors) & 15u)) return false;
        if (s.tail && (reinterpret_cast<uintptr_t>(s.tail) & 15u)) return false;
        if (s.tail_cap > 0 && !s.tail) return false;
        return true;
    };
    if (!side_ok(a->k) || !side_ok(a->v)) return NSN_EINVAL;
    if (!a->k.blocks != !a->v.blocks) return NSN_EINVAL;
    if (a->append && (!a->k.tail || !a->v.tail || a->k.tail_cap <= 0 || a->v.tail_cap <= 0)) return NSN_EINVAL;
    auto tail_ok = [](const nsn_kv_side &s) {
        return !s.tail || s.tail_dtype == NSN_DTYPE_F16 || s.tail_dtype == NSN_DTYPE_BF16;
    };
    if (!tail_ok(a->k) || !tail_ok(a->v)) return NSN_EINVAL;
    if (a->k.tail && a->v.tail && a->k.tail_dtype != a->v.tail_dtype) return NSN_EINVAL;
    const nsn_kv_side &ts = a->k.tail ? a->k : a->v;
    const bool tbf = ts.tail ? ts.tail_dtype == NSN_DTYPE_BF16 : a->dtype == NSN_DTYPE_BF16;
    for (const void *ptr : {static_cast<const void *>(a->q), a->k_chunk, a->v_chunk, static_cast<const void *>(a->out)})
        if (reinterpret_cast<uintptr_t>(ptr) & 15u) return NSN_EINVAL;
    const int64_t qt = (a->n_q + kQTile - 1) / kQTile;
    if (qt > 65535 || a->heads_q > 0x7fffffff || a->batch > 65535) return NSN_EINVAL;
    PrefillParams p{};
    p.q = static_cast<const uint16_t *>(a->q);
    p.batch = a->batch;
    p.heads_q = a->heads_q;
    p.heads_kv = a->heads_kv;
    p.n_q = a->n_q;
    p.group = static_cast<int>(a->heads_q / a->heads_kv);
    p.qscale = a->scale * kLog2e;
    p.ctx_len = a->ctx_len;
    auto side = [](const nsn_kv_side &s) {
        return Side{s.codes, s.mins, s.scales, s.factors, s.blocks, s.block_cap,
                    static_cast<const uint16_t *>(s.tail), s.tail_cap};
    };
    p.k = side(a->k);
    p.v = side(a->v);
    p.kc = static_cast<const uint16_t *>(a->k_chunk);
    p.vc = static_cast<const uint16_t *>(a->v_chunk);
    p.out = static_cast<uint16_t *>(a->out);
    p.status = a->status;
    if (a->append) {   // the caller grants write access to the tails' rows past the context
        p.ka = static_cast<uint16_t *>(const_cast<void *>(a->k.tail));
        p.va = static_cast<uint16_t *>(const_cast<void *>(a->v.tail));
    }
    const dim3 grid(static_cast<unsigned>(a->heads_q), static_cast<unsigned>(a->batch), static_cast<unsigned>(qt));
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const bool bf = a->dtype == NSN_DTYPE_BF16;
#define NSN_PREFILL_LAUNCH(B_, D_, L_)                                                                              \
    do {                                                                                                            \
        if (tbf) hipLaunchKernelGGL((prefill_kernel<B_, D_, NSN_DTYPE_BF16, L_>), grid, dim3(64 * kWaves), 0, st, p); \
        else hipLaunchKernelGGL((prefill_kernel<B_, D_, NSN_DTYPE_F16, L_>), grid, dim3(64 * kWaves), 0, st, p);      \
    } while (0)
    const bool lo = bf && a->precise_weights;
    if (a->bits == 3) {
        if (lo) NSN_PREFILL_LAUNCH(3, NSN_DTYPE_BF16, true);
        else if (bf) NSN_PREFILL_LAUNCH(3, NSN_DTYPE_BF16, false);
        else NSN_PREFILL_LAUNCH(3, NSN_DTYPE_F16, false);
    } else {
        if (lo) NSN_PREFILL_LAUNCH(5, NSN_DTYPE_BF16, true);
        else if (bf) NSN_PREFILL_LAUNCH(5, NSN_DTYPE_BF16, false);
        else NSN_PREFILL_LAUNCH(5, NSN_DTYPE_F16, false);
    }
#undef NSN_PREFILL_LAUNCH
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}
