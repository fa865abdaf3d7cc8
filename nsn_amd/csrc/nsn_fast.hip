// Fast single-query decode attention over NSN-packed K/V for gfx950 (MFMA).
//
// Same work decomposition and partial format as the exact-order kernel in
// nsn_attn.hip: work unit = sequence x kv-head x context split; all G query
// heads of the kv-head are served by one pass over its blocks; the splits are
// merged with a log-sum-exp merge.  One wave per work unit.  Per 64-token
// packed block:
//
//   scores   S[h,t] = scale * f_K[t] * (q_h.m_K + sum_c (q_h[c] s_K[c]) z_K[t,c])
//            The channel contraction runs on v_mfma_f32_16x16x32_f16.  B holds
//            the raw 3-bit codes, masked in place inside 16-bit halves: a code
//            at bit k of its half is the fp16 subnormal z * 2^(k-24), exact.
//            A holds the coefficient rows q_h (.) s_K * 2^-k, split into fp16
//            hi + lo (error-free product on packed fp16 FMA).
//   softmax  online (running max / sum per head), exp2 with log2(e) folded.
//            One 16-lane row of the wave per query head.
//   output   acc[h,c] += s_V[c] * F * sum_t p'[h,t] z_V[t,c] + m_V[c] * sum_t p[h,t] f_V[t]
//            with p' = p f_V / F as fp16 hi + lo rows (F = block max of f_V).  V codes are
//            loaded channel-major (a lane owns 8 channels of 16 tokens), so
//            the tokens already sit on the contraction axis of the B operand.
//
// f_K, f_V are the per-token decode factors n / |m + s*z| of each packed block
// (nsn_block_factors).  They are constant once a block is encoded, so they are
// read, not recomputed.  Reconstruction equals nsn_decode's up to rounding
// (loop_kv_pilot.py:216-225); results match the fp64 oracle within the stated
// tolerance, not bit for bit.  Tokens past the packed prefix (the tail, or a
// fully dense K/V for the fp16 baseline) take the same MFMA path with the
// stored values themselves as operands: fp16 tails on the fp16 product, bf16
// tails on v_mfma_f32_16x16x32_bf16 with the query and the softmax weights as
// bf16 hi + lo rows (~16 bits), so bf16 values outside the fp16 range compute.
//
// Reference routes replaced: experiments/ac08/source/loop_kv_vf01_kernel.py:56-139
// (fused readout), experiments/nb06/source/loop_kv_nb06_kernel.py:54-154 (GQA),
// experiments/ac08/source/loop_kv_af01_kernel.py:13-68 (score-input readout).
#include <type_traits>

#include "nsn_common.hpp"
#include "nsn_unpack.hpp"

namespace nsn {
namespace fast {

using unpack::Layout;
using unpack::kunpack;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPartStride = 132;
constexpr int kMaxGroup = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kPScale = 16384.f;   // softmax weights enter the PV product as p * 2^14

__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
// The same product on bf16 operands (dense bf16 tail tokens).
__device__ __forceinline__ f32x4 mfma_bf16(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
}
template <bool BF>
__device__ __forceinline__ f32x4 mfma_t(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    if constexpr (BF) return mfma_bf16(a, b, c);
    else return mfma(a, b, c);
}
// v_perm_b32: byte i of the result = byte sel[i] of {hi:lo} (0..3 = lo, 4..7 = hi, 0x0c = 0).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ half2v as_h2(uint32_t x) { return __builtin_bit_cast(half2v, x); }
__device__ __forceinline__ uint32_t as_u(half2v x) { return __builtin_bit_cast(uint32_t, x); }
// Two fp32 -> packed fp16 pair, round toward zero (v_cvt_pkrtz_f16_f32).
__device__ __forceinline__ uint32_t pkrtz(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ float lo_f32(uint32_t p) { return static_cast<float>(__builtin_bit_cast(fp16x2, p)[0]); }
__device__ __forceinline__ float hi_f32(uint32_t p) { return static_cast<float>(__builtin_bit_cast(fp16x2, p)[1]); }
__device__ __forceinline__ float f16lo(uint32_t p) { return static_cast<float>(__builtin_bit_cast(half2v, p)[0]); }
__device__ __forceinline__ float f16hi(uint32_t p) { return static_cast<float>(__builtin_bit_cast(half2v, p)[1]); }

// fp32 pair -> fp16 hi (toward zero) + fp16 lo = rn(x - hi): ~22 significant bits.
__device__ __forceinline__ void split2(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = pkrtz(a, b);
    lo = pkrtz(a - lo_f32(hi), b - hi_f32(hi));
}

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t bf16_rn(float x) {
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
// fp32 pair -> bf16 hi (toward zero) + bf16 lo = rn(x - hi): ~16 significant bits.
__device__ __forceinline__ void split2_bf16(float a, float b, uint32_t &hi, uint32_t &lo) {
    const uint32_t ua = __builtin_bit_cast(uint32_t, a) & 0xFFFF0000u, ub = __builtin_bit_cast(uint32_t, b) & 0xFFFF0000u;
    hi = (ua >> 16) | ub;
    lo = bf16_rn(a - __builtin_bit_cast(float, ua)) | (bf16_rn(b - __builtin_bit_cast(float, ub)) << 16);
}
// An fp16 hi + lo pair of element pairs -> the bf16 hi + lo pair of the same values.
__device__ __forceinline__ void f16_to_bf16_pair(uint32_t h, uint32_t l, uint32_t &bh, uint32_t &bl) {
    split2_bf16(f16lo(h) + f16lo(l), f16hi(h) + f16hi(l), bh, bl);
}

// The 16-bit half of dword `S[a/2]` holding element a, paired with element b
// (a -> low half, b -> high half), for compile-time a, b.
__device__ __forceinline__ uint32_t half_pair(const uint32_t (&S)[4], int a, int b) {
    if (a / 2 == b / 2 && (a & 1) == 0 && (b & 1) == 1) return S[a / 2];
    const uint32_t s0 = (a & 1) ? 0x0302u : 0x0100u;
    const uint32_t s1 = (b & 1) ? 0x0706u : 0x0504u;
    return perm(S[b / 2], S[a / 2], s0 | (s1 << 16));
}

// Code layouts and the K-side unpack (Layout<BITS>, kunpack) live in
// nsn_unpack.hpp, shared with the K-score kernel.

// V: 16 token words w[t] (the lane's BITS*8 code bits of token t, aligned to
// bit 0; w1 = bits 32..63) -> per tile m, per token pair k: code(2k) | code(2k+1) << 16.
__device__ __forceinline__ void vpair3(uint32_t wa, uint32_t wb, uint32_t (&D)[8]) {
    const uint32_t X = perm(wb, wa, 0x05040100u), Y = perm(wb, wa, 0x06050201u), Z = perm(wb, wa, 0x0C060C02u);
    D[0] = X & 0x00070007u;
    D[1] = X & 0x00380038u;
    D[2] = X & 0x01C001C0u;
    D[3] = Y & 0x000E000Eu;
    D[4] = Y & 0x00700070u;
    D[5] = Y & 0x03800380u;
    D[6] = Z & 0x001C001Cu;
    D[7] = Z & 0x00E000E0u;
}
// 5-bit V: token words (w0 = code bits 0..31, w1 = 32..39) of tokens a, b ->
// per channel m: code m of a (low half) | of b (high half), at bit kV[m]
// (the byte windows of the K side; codes 3 and 6 from the words shifted by 14).
__device__ __forceinline__ void vpair5(uint32_t w0a, uint32_t w1a, uint32_t w0b, uint32_t w1b, uint32_t (&D)[8]) {
    const uint32_t X0 = perm(w0b, w0a, 0x05040100u);   // a b0 b1 | b b0 b1
    const uint32_t X1 = perm(w0b, w0a, 0x06050201u);   // b1 b2
    const uint32_t X2 = perm(w0b, w0a, 0x07060302u);   // b2 b3
    const uint32_t ta = __builtin_amdgcn_alignbit(w1a, w0a, 24), tb = __builtin_amdgcn_alignbit(w1b, w0b, 24);
    const uint32_t X3 = perm(tb, ta, 0x05040100u);     // b3 b4
    const uint32_t X4 = perm(tb, ta, 0x05050101u);     // b4
    const uint32_t sa = __builtin_amdgcn_alignbit(w1a, w0a, 14), sb = __builtin_amdgcn_alignbit(w1b, w0b, 14);
    const uint32_t X5 = perm(sb, sa, 0x05040100u);     // bits 14..29
    const uint32_t X6 = perm(sb, sa, 0x07060302u);     // bits 30..45
    D[0] = X0 & 0x001F001Fu;
    D[1] = X0 & 0x03E003E0u;
    D[2] = X1 & 0x007C007Cu;
    D[3] = X5 & 0x003E003Eu;
    D[4] = X2 & 0x01F001F0u;
    D[5] = X3 & 0x003E003Eu;
    D[6] = X6 & 0x001F001Fu;
    D[7] = X4 & 0x00F800F8u;
}

struct FastSide {
    const uint8_t *codes;
    const uint16_t *mins, *scales;
    const float *factors;
    const int32_t *blocks;
    int64_t block_cap;
    const uint16_t *tail;   // fp16, or bf16 in the TBF kernel variants
    int64_t tail_cap;
};

struct FastParams {
    const void *q;
    int64_t batch, heads_q, heads_kv;
    int group;
    float scale;
    const int32_t *seq_len;
    int n_splits;              // partial slots per (sequence, q-head)
    int64_t min_blocks;        // lower bound of the blocks per wave (keeps every stream within n_splits slots)
    FastSide k, v;
    const float *scores;
    int64_t scores_cap;
    float *partials;
    int32_t *status;
    int weighted;              // slot weighting: 0 none, 1 two waves per SIMD (5:4), 2 six waves per CU (8:7)
};

// Reductions over the 16 lanes of a row with DPP (quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror): every lane of the row
// ends with the full result.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float red16_max(float x) {
    x = fmaxf(x, dpp<0xb1>(x));
    x = fmaxf(x, dpp<0x4e>(x));
    x = fmaxf(x, dpp<0x141>(x));
    x = fmaxf(x, dpp<0x140>(x));
    return x;
}
__device__ __forceinline__ float red16_sum(float x) {
    x = x + dpp<0xb1>(x);
    x = x + dpp<0x4e>(x);
    x = x + dpp<0x141>(x);
    x = x + dpp<0x140>(x);
    return x;
}

// Quotient and remainder of uniform a >= 0 by b > 0.  A 64-bit division
// expands to over a hundred scalar instructions, and every wave of a CU
// shares one scalar unit while it partitions the work, so operands that fit
// in 32 bits (all practical sizes) take the 32-bit expansion.
__device__ __forceinline__ int64_t udivq(int64_t a, int64_t b) {
    if (((static_cast<uint64_t>(a) | static_cast<uint64_t>(b)) >> 32) == 0)
        return static_cast<int64_t>(static_cast<uint32_t>(a) / static_cast<uint32_t>(b));
    return a / b;
}
__device__ __forceinline__ int64_t uremq(int64_t a, int64_t b) { return a - udivq(a, b) * b; }

// 32-bit wave reductions and scan on DPP row operations plus scalar reads of
// the four row results: a few cycles per step instead of an LDS permute each.
template <int CTRL>
__device__ __forceinline__ int32_t dpp_i(int32_t x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, true);   // (lanes without a source read 0)
}
__device__ __forceinline__ int32_t rows4_sum(int32_t x) {
    return __builtin_amdgcn_readlane(x, 0) + __builtin_amdgcn_readlane(x, 16) + __builtin_amdgcn_readlane(x, 32) +
           __builtin_amdgcn_readlane(x, 48);
}
__device__ __forceinline__ int32_t wave_sum(int32_t x) {   // (uniform result)
    x += dpp_i<0xb1>(x);
    x += dpp_i<0x4e>(x);
    x += dpp_i<0x141>(x);
    x += dpp_i<0x140>(x);
    return rows4_sum(x);
}
__device__ __forceinline__ int32_t wave_max(int32_t x) {   // (uniform result)
    x = max(x, dpp_i<0xb1>(x));
    x = max(x, dpp_i<0x4e>(x));
    x = max(x, dpp_i<0x141>(x));
    x = max(x, dpp_i<0x140>(x));
    return max(max(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               max(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}
__device__ __forceinline__ int32_t wave_incl_scan32(int32_t x) {
    x += dpp_i<0x111>(x);   // row_shr:1, 2, 4, 8: inclusive scan inside each 16-lane row
    x += dpp_i<0x112>(x);
    x += dpp_i<0x114>(x);
    x += dpp_i<0x118>(x);
    const int l = threadIdx.x;
    const int32_t r0 = __builtin_amdgcn_readlane(x, 15), r1 = __builtin_amdgcn_readlane(x, 31),
                  r2 = __builtin_amdgcn_readlane(x, 47);
    return x + (l >= 16 ? r0 : 0) + (l >= 32 ? r1 : 0) + (l >= 48 ? r2 : 0);
}
__device__ __forceinline__ int64_t lane_get(int64_t x, int lane) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x >> 32), lane));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Nonzero iff one of the 8 fp16 values in w has an all-ones exponent (Inf/NaN):
// the masked exponent plus one exponent step carries into the half's sign bit.
__device__ __forceinline__ uint32_t f16x8_nonfinite(const uint4 &w) {
    const uint32_t m = 0x7C007C00u, one = 0x04000400u, top = 0x80008000u;
    return (((w.x & m) + one) | ((w.y & m) + one) | ((w.z & m) + one) | ((w.w & m) + one)) & top;
}
__device__ __forceinline__ uint32_t bf16x8_nonfinite(const uint4 &w) {
    const uint32_t m = 0x7F807F80u, one = 0x00800080u, top = 0x80008000u;
    return (((w.x & m) + one) | ((w.y & m) + one) | ((w.z & m) + one) | ((w.w & m) + one)) & top;
}
template <bool BF>
__device__ __forceinline__ uint32_t x8_nonfinite(const uint4 &w) {
    if constexpr (BF) return bf16x8_nonfinite(w);
    else return f16x8_nonfinite(w);
}

// LDS hand-off inside the single wave of a workgroup: the wave's LDS accesses
// complete in order, so waiting for them (and stopping the compiler from
// moving memory accesses across) is enough -- no s_barrier, and prefetched
// global loads stay in flight.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4):
// lane l's bytes land at dst + 16*l (dst uniform).  Issued as inline asm so the
// compiler does not track it: otherwise it waits for every pending DMA before
// any LDS read (it cannot tell the stages apart), which serialises the
// prefetch.  The kernel waits for its DMAs itself (vmcnt(0) at the top of each
// block); an untracked VMEM operation can only make the compiler's own vmcnt
// waits stricter, never looser.  M0 carries the LDS address.  The loads carry
// the non-temporal hint (`nt`): a step reads each packed block once, and
// without the hint the streamed blocks are kept in the caches at the expense
// of the step's own traffic (C2 split kernel 73.9 -> 67.1-67.7 us).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void *src, uint32_t *dst) {
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds) : "memory", "m0");
}
// The same with a uniform 64-bit base (SGPRs) and a 32-bit lane offset: the
// per-block address update is scalar and the lane offset loop-invariant.
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t *dst) {
    const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Per-wave LDS.  Separate objects, so that the compiler can tell the DMA
// targets of the next block from everything the current block reads (a DMA
// into one stage then holds back no read of the other stage or of the operand
// buffers).
//   afrag  A operands of the K-side MFMA, one 16-byte entry per (row, chunk,
//          kstep); the entry index is XOR-swizzled by the row so that the rows
//          of one fragment read fall on different banks.
//   pbuf   A operands of the PV MFMA: P' rows, fp16 per token, rows padded to
//          36 dwords.
//   Both store only the rows in use: the MFMA row of head h, part p (hi = 0,
//   lo = 1) is 4*(h%4) + 2*(h/4) + p; at most 4 heads per kv-head leave rows
//   with (row & 2) != 0 empty, read as zeros from a zero entry.
//   k/v/m  block stages (double-buffered): K codes, V codes (+4 dwords: a
//          lane's last code window may read past the block's last row) and
//          metadata: [K scale | K min | K factor | V scale | V min | V factor],
//          64 dwords each.
template <int BITS, int GRP> struct LdsShape {
    static constexpr int ROWS = GRP > 4 ? 16 : 8;
    static constexpr int NBW = packed_block_bytes(BITS) / 4 + 4;
    static constexpr int MW = 384;
};
template <int BITS, int GRP> struct Lds {
    using S = LdsShape<BITS, GRP>;
    u32x4 (&afrag)[S::ROWS * 16 + 1];
    uint32_t (&pbuf)[S::ROWS * 36 + 4];
    uint32_t (&k0)[S::NBW];
    uint32_t (&k1)[S::NBW];
    uint32_t (&v0)[S::NBW];
    uint32_t (&v1)[S::NBW];
    uint32_t (&m0)[S::MW];
    uint32_t (&m1)[S::MW];
};

// Compact storage row of MFMA row r (or -1: an empty row, read as zero).
template <int GRP>
__device__ __forceinline__ int crow(int r) {
    if (GRP > 4) return r;
    return (r & 2) ? -1 : ((r >> 2) << 1) | (r & 1);
}

// Issue the DMA of one packed block into a stage: K codes (unless SCORES),
// V codes, and the metadata of both sides.
template <int BITS, bool SCORES>
__device__ __forceinline__ void dma_block(const FastParams &p, int64_t ibk, int64_t ibv, int l, bool kside, bool vside,
                                          uint32_t *kst, uint32_t *vst, uint32_t *mst) {
    constexpr int NB = packed_block_bytes(BITS);
    const uint32_t off = 16u * static_cast<uint32_t>(l);
    if (!SCORES && kside) {
        const uint8_t *kc = p.k.codes + ibk * NB;
#pragma unroll
        for (int c = 0; c < NB / 1024; ++c) dma16s(kc + 1024 * c, off, kst + 256 * c);
    }
    if (vside) {
        const uint8_t *vc = p.v.codes + ibv * NB;
#pragma unroll
        for (int c = 0; c < NB / 1024; ++c) dma16s(vc + 1024 * c, off, vst + 256 * c);
    }
    // metadata: lanes 0-15 K scale, 16-31 K min, 32-47 K factor, 48-63 V scale;
    // then lanes 0-15 V min, 16-31 V factor
    const int q = l & 15;
    const uint16_t *vsc = vside ? p.v.scales + ibv * kDim : nullptr;
    const void *src;
    if (!SCORES && kside) {
        src = (l < 16) ? static_cast<const void *>(p.k.scales + ibk * kDim + 8 * q)
            : (l < 32) ? static_cast<const void *>(p.k.mins + ibk * kDim + 8 * q)
            : (l < 48) ? static_cast<const void *>(p.k.factors + ibk * kBlockTok + 4 * q)
            : vside    ? static_cast<const void *>(vsc + 8 * q)
                       : static_cast<const void *>(p.k.scales + ibk * kDim + 8 * q);   // (slot not read)
    } else {
        src = static_cast<const void *>(vsc + 8 * q);   // (no K metadata: those slots are not read)
    }
    if (vside || (!SCORES && kside)) dma16(src, mst);
    if (vside && l < 32)
        dma16((l < 16) ? static_cast<const void *>(p.v.mins + ibv * kDim + 8 * q)
                       : static_cast<const void *>(p.v.factors + ibv * kBlockTok + 4 * q),
              mst + 256);
}

// One stream segment: tokens [t_begin, t_end) of (sequence b, kv-head kvh),
// written as partial slot `slot` of each of the kv-head's G query heads.
// nbk_b / nbv_b: the sequence's packed K / V block counts (0 without blocks).
template <int BITS, int QDT, bool SCORES, int GRP, bool TBF>
__device__ __forceinline__ void segment(const FastParams &p, const Lds<BITS, GRP> &sh, int b, int kvh,
                                        int64_t t_begin, int64_t t_end, int64_t nbk_b, int64_t nbv_b, int slot,
                                        int count) {
    using LY = Layout<BITS>;
    constexpr int NJ = GRP > 4 ? 2 : 1;   // query heads per 16-lane row (head grp + 4j)
    constexpr int NB = packed_block_bytes(BITS);
    const int G = p.group;                // query heads per kv-head (<= GRP)

    const int l = threadIdx.x;
    const int row = l & 15, grp = l >> 4;
    const int64_t seqrow = static_cast<int64_t>(b) * p.heads_kv + kvh;
    const int64_t hq0 = static_cast<int64_t>(kvh) * G;

    // ---- the first packed block's DMA goes out before anything else, so its
    // latency overlaps the query loads and preparation below.  Blocks
    // [t_begin, t_fast) are fully packed on every side that has blocks.
    const int64_t nbk = SCORES ? 0 : nbk_b;
    const int64_t nbv = nbv_b;
    const int64_t kend = SCORES ? t_end : nbk * kBlockTok;
    int64_t t_fast = (kend < nbv * kBlockTok) ? kend : nbv * kBlockTok;
    t_fast = (t_fast < t_end) ? t_fast : t_end;
    // The fast blocks are walked from a per-wave starting offset (wrapping
    // round): waves then do not sweep the same relative addresses in step,
    // which measurably helps the HBM (~2 % on the C2 workload).
    const int64_t nfb = (t_fast > t_begin) ? (t_fast - t_begin) / kBlockTok : 0;
    const int64_t rot =
        (nfb > 1) ? uremq(static_cast<int64_t>((static_cast<uint32_t>(blockIdx.x) * 2654435761u) >> 8), nfb) : 0;
    auto fast_blk = [&](int64_t j) {   // token start of the j-th fast block walked
        const int64_t x = j + rot;
        return t_begin + ((x < nfb) ? x : x - nfb) * kBlockTok;
    };
    if (nfb > 0)
        dma_block<BITS, SCORES>(p, seqrow * p.k.block_cap + fast_blk(0) / kBlockTok,
                                seqrow * p.v.block_cap + fast_blk(0) / kBlockTok, l, true, true, &sh.k0[0], &sh.v0[0],
                                &sh.m0[0]);

    // ---- operand buffer addressing (loop invariant)
    const int rdrow = crow<GRP>(row);                        // this lane's A row when reading
    const u32x4 *af_rd = (rdrow < 0) ? &sh.afrag[GRP > 4 ? 16 * 16 : 8 * 16] : &sh.afrag[16 * rdrow];
    const int af_x = (rdrow < 0) ? -1 : (rdrow & 15);        // swizzle (-1: the zero entry)
    const uint32_t *pb_rd = (rdrow < 0) ? &sh.pbuf[(GRP > 4 ? 16 : 8) * 36] : &sh.pbuf[36 * rdrow];
    const int pb_step = (rdrow < 0) ? 0 : 1;

    // ---- query preparation.  Prep role of lane l: head grp + 4j, channels
    // pch .. pch+7 with pch = 32*wgq + 8*wkk (chunk wgq, K-step wkk).
    const int wgq = (l >> 2) & 3, wkk = l & 3;
    const int pch = 32 * wgq + 8 * wkk;
    bool bad_in = false;   // raw inputs read here (q, tail tokens): the fused finite check
    float c1[NJ], c1s[NJ];             // score scale: scale * log2(e) * 2^-sigma_h (c1s: times 2^24)
    uint32_t quh[NJ][4], qul[NJ][4];   // q * 2^sigma in element order (hi, lo): q.m and dense keys
    uint32_t qkh[NJ][4], qkl[NJ][4];   // the same * 2^-kE: the coefficient rows
    // Every lane loads its 8 channels (16 bytes) of an in-bounds head (the
    // group's first where head grp + 4j is past the group) without a branch,
    // so that the loads are in flight together and one wait covers them.
    uint16_t qraw[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int h = grp + 4 * j;
        const uint16_t *qr = static_cast<const uint16_t *>(p.q) +
                             (static_cast<int64_t>(b) * p.heads_q + hq0 + (h < G ? h : 0)) * kDim + pch;
        uint4 w;
        __builtin_memcpy(&w, qr, 16);
        asm volatile("" : "+v"(w.x), "+v"(w.y), "+v"(w.z), "+v"(w.w));   // (kept unconditional)
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int c = 0; c < 8; ++c) qraw[j][c] = static_cast<uint16_t>(ww[c / 2] >> (16 * (c % 2)));
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int h = grp + 4 * j;
        const bool valid = h < G;
        float qv[8];
        float mx = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            qv[c] = valid ? Elem<QDT>::load(qraw[j][c]) : 0.f;
            mx = fmaxf(mx, fabsf(qv[c]));
            bad_in |= !finite(qv[c]);
        }
        mx = red16_max(mx);
        // sigma: max|q| * 2^sigma in [2^13, 2^14), so every coefficient |q s| < 2^14 * 2/7 stays fp16
        int e2 = 0;
        (void)frexpf(mx, &e2);
        int sigma = (mx > 0.f && finite(mx)) ? 14 - e2 : 0;
        sigma = sigma < -100 ? -100 : (sigma > 100 ? 100 : sigma);
        const float pw = ldexpf(1.f, sigma);
        c1[j] = p.scale * kLog2e * ldexpf(1.f, -sigma);
        c1s[j] = c1[j] * 16777216.f;
        float qs[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) qs[c] = qv[c] * pw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int ca = LY::chE[2 * i], cb = LY::chE[2 * i + 1];
            split2(qs[ca], qs[cb], quh[j][i], qul[j][i]);
            split2(ldexpf(qs[ca], -LY::kE[2 * i]), ldexpf(qs[cb], -LY::kE[2 * i + 1]), qkh[j][i], qkl[j][i]);
        }
    }
    // write the A fragments (hi, lo rows) of head grp + 4j at the prep slot
    auto put_frag = [&](int j, const u32x4 &hi, const u32x4 &lo) {
        const int h = grp + 4 * j;
        const int r0 = crow<GRP>(4 * (h & 3) + 2 * (h >> 2));
        sh.afrag[16 * r0 + ((4 * wgq + wkk) ^ (r0 & 15))] = hi;
        sh.afrag[16 * (r0 + 1) + ((4 * wgq + wkk) ^ ((r0 + 1) & 15))] = lo;
    };
    auto get_frag = [&](int kk) { return af_x < 0 ? af_rd[0] : af_rd[(4 * grp + kk) ^ af_x]; };

    // V lane constants: the lane's code bytes BITS*row .. of a token row start
    // in dword vdw at bit vsh (a funnel shift of that dword and the next).
    constexpr int VROW_DW = 4 * BITS;
    const int vbyte = BITS * row;
    const int vdw = vbyte >> 2;
    const uint32_t vsh = 8u * static_cast<uint32_t>(vbyte & 3);

    float m_run[NJ], l_run[NJ], acc[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        m_run[j] = -INFINITY;
        l_run[j] = 0.f;
#pragma unroll
        for (int m = 0; m < 8; ++m) acc[j][m] = 0.f;
    }
    bool bad = false;

    const f32x4 zf = {0.f, 0.f, 0.f, 0.f};

    // ---- software pipeline over the fully packed blocks [t_begin, t_fast),
    // walked in the rotated order above: all data of the next block (codes
    // and metadata of K and V) is moved into the other LDS stage by DMA while
    // the current one is computed, and waited for with one vmcnt(0) at the
    // top of the next block.  No prefetched data lives in
    // registers, so the compiler never has to wait for it mid-block, and no
    // DMA is left in flight when the pipelined loop ends.  Blocks past t_fast
    // (tail, dense K or V) fetch their own data first.

    auto block = [&](auto fast, auto stage_c, const int64_t t0, const int64_t t_next) {
        constexpr bool FAST = decltype(fast)::value;
        constexpr int ST = decltype(stage_c)::value;
        uint32_t *const kst = ST ? &sh.k1[0] : &sh.k0[0];
        uint32_t *const vst = ST ? &sh.v1[0] : &sh.v0[0];
        uint32_t *const mst = ST ? &sh.m1[0] : &sh.m0[0];
        const int valid = static_cast<int>(t_end - t0 < kBlockTok ? t_end - t0 : kBlockTok);
        const bool kpacked = FAST ? !SCORES : (!SCORES && (t0 < nbk * kBlockTok));
        const bool vpacked = FAST ? true : (t0 < nbv * kBlockTok);
        if (!FAST && (kpacked || vpacked))
            dma_block<BITS, SCORES>(p, seqrow * p.k.block_cap + t0 / kBlockTok, seqrow * p.v.block_cap + t0 / kBlockTok,
                                    l, kpacked, vpacked, kst, vst, mst);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // block i's stage is in
        if (FAST && t_next >= 0) {   // ---- the next fast block's data, before any compute on this one
            const int64_t t1 = t_next;
            dma_block<BITS, SCORES>(p, seqrow * p.k.block_cap + t1 / kBlockTok, seqrow * p.v.block_cap + t1 / kBlockTok,
                                    l, true, true, ST ? &sh.k0[0] : &sh.k1[0], ST ? &sh.v0[0] : &sh.v1[0],
                                    ST ? &sh.m0[0] : &sh.m1[0]);
        }
        float s[NJ][4];   // scores (log2 domain) of head grp + 4j at tokens 16*nt + row

        // ------------------------------------------------------------ scores
        if constexpr (SCORES) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int h = grp + 4 * j;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const int tt = 16 * nt + row;
                    s[j][nt] = (tt < valid && h < G)
                                   ? p.scores[(static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.scores_cap + t0 + tt] * kLog2e
                                   : -INFINITY;
                }
            }
        } else {
            u32x4 af[4];
            f32x4 C[4];
            if (kpacked) {
                // coefficient rows W = q (.) s_K * 2^-kE (fp16 hi + lo) and q.m_K for head grp + 4j
                const uint4 ks4 = *reinterpret_cast<const uint4 *>(mst + pch / 2);
                const uint4 km4 = *reinterpret_cast<const uint4 *>(mst + 64 + pch / 2);
                const uint32_t S[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
                const uint32_t M[4] = {km4.x, km4.y, km4.z, km4.w};
                uint32_t s2[4], m2[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s2[i] = half_pair(S, LY::chE[2 * i], LY::chE[2 * i + 1]);
                    m2[i] = half_pair(M, LY::chE[2 * i], LY::chE[2 * i + 1]);
                }
                float qm[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    u32x4 wh, wl;
                    float d = 0.f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const half2v sv = as_h2(s2[i]);
                        const half2v hi = as_h2(qkh[j][i]) * sv;
                        const half2v er = __builtin_elementwise_fma(as_h2(qkh[j][i]), sv, -hi);
                        const half2v lo = __builtin_elementwise_fma(as_h2(qkl[j][i]), sv, er);
                        wh[i] = as_u(hi);
                        wl[i] = as_u(lo);
                        d = __builtin_amdgcn_fdot2(as_h2(quh[j][i]), as_h2(m2[i]), d, false);
                        d = __builtin_amdgcn_fdot2(as_h2(qul[j][i]), as_h2(m2[i]), d, false);
                    }
                    qm[j] = red16_sum(d) * (1.f / 16777216.f);   // (in units of the code scale 2^-24)
                    put_frag(j, wh, wl);
                }
                float fk[4];
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) fk[nt] = __builtin_bit_cast(float, mst[128 + 16 * nt + row]);
                lds_sync();
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) af[kk] = get_frag(kk);
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    uint32_t u[BITS];
                    const uint32_t *src = kst + (16 * nt + row) * VROW_DW + BITS * grp;
#pragma unroll
                    for (int w = 0; w < BITS; ++w) u[w] = src[w];
                    u32x4 Bz[4];
                    kunpack(u, Bz);
                    C[nt] = zf;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) C[nt] = mfma(af[kk], Bz[kk], C[nt]);
                }
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        s[j][nt] = ((C[nt][2 * j] + C[nt][2 * j + 1]) + qm[j]) * (fk[nt] * c1s[j]);
            } else {
                // dense keys (tokens t0 - 64*nbk + tt of the tail buffer): the A rows are the
                // query itself (q * 2^sigma, hi + lo; bf16 hi + lo for bf16 keys), channels in
                // the same element order
                if constexpr (TBF) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) {
                        u32x4 hi, lo;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            uint32_t bh, bl;
                            f16_to_bf16_pair(quh[j][i], qul[j][i], bh, bl);
                            hi[i] = bh;
                            lo[i] = bl;
                        }
                        put_frag(j, hi, lo);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        put_frag(j, u32x4{quh[j][0], quh[j][1], quh[j][2], quh[j][3]},
                                 u32x4{qul[j][0], qul[j][1], qul[j][2], qul[j][3]});
                }
                lds_sync();
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) af[kk] = get_frag(kk);
                const int64_t base = t0 - nbk * kBlockTok;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    // tokens past `valid` read the last valid token (in bounds); their
                    // scores are set to -inf below, so the value never counts
                    const int tt = (16 * nt + row < valid) ? 16 * nt + row : valid - 1;
                    const uint16_t *src = p.k.tail + (seqrow * p.k.tail_cap + base + tt) * kDim + 32 * grp;
                    C[nt] = zf;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const uint4 v = ld16(src + 8 * kk);
                        bad_in |= x8_nonfinite<TBF>(v) != 0;
                        const uint32_t X[4] = {v.x, v.y, v.z, v.w};
                        u32x4 Bd;
#pragma unroll
                        for (int i = 0; i < 4; ++i) Bd[i] = half_pair(X, LY::chE[2 * i], LY::chE[2 * i + 1]);
                        C[nt] = mfma_t<TBF>(af[kk], Bd, C[nt]);
                    }
                }
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        s[j][nt] = (16 * nt + row < valid) ? (C[nt][2 * j] + C[nt][2 * j + 1]) * c1[j] : -INFINITY;
            }
        }

        // ------------------------------------------------------------ softmax
        float bm[NJ];
        bool grow = false;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            bm[j] = fmaxf(fmaxf(s[j][0], s[j][1]), fmaxf(s[j][2], s[j][3]));   // this lane's tokens
            grow |= bm[j] > m_run[j];
        }
        // the row maximum is only reduced (and the state rescaled) when some
        // lane's score exceeds the running maximum -- rare after the first blocks
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const float mnew = fmaxf(m_run[j], red16_max(bm[j]));
                const float alpha = (m_run[j] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[j] - mnew);
                l_run[j] *= alpha;
#pragma unroll
                for (int m = 0; m < 8; ++m) acc[j][m] *= alpha;
                m_run[j] = mnew;
            }
        }
        // p' = p f_V / F * 2^14 in [0, 2^14]: the scale keeps small weights out
        // of the fp16 subnormal range (and the fp16 hi/lo split precise)
        float fv[4];
        float F = 1.f, rF = kPScale;
        if (vpacked) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) fv[nt] = __builtin_bit_cast(float, mst[320 + 16 * nt + row]);
            F = red16_max(fmaxf(fmaxf(fv[0], fv[1]), fmaxf(fv[2], fv[3])));
            F = fmaxf(F, 1e-30f);
            rF = __builtin_amdgcn_rcpf(F) * kPScale;
        }
        float spf[NJ];   // sum_t p f_V (packed V) -- the min term's weight
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const float msafe = (m_run[j] == -INFINITY) ? 0.f : m_run[j];
            float ls = 0.f, ps = 0.f, pp[4];
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const float pw = __builtin_amdgcn_exp2f(s[j][nt] - msafe);
                ls += pw;
                const float pf = vpacked ? pw * fv[nt] : pw;
                ps += pf;
                pp[nt] = pf * rF;
            }
            l_run[j] += ls;   // per lane; the row sum is taken once per segment
            spf[j] = red16_sum(ps);
            const int h = grp + 4 * j;
            // fp16 hi (toward zero) + lo rows: the weights keep ~22 bits
            const int r0 = crow<GRP>(4 * (h & 3) + 2 * (h >> 2));
            uint16_t *phi = reinterpret_cast<uint16_t *>(&sh.pbuf[36 * r0]);
            uint16_t *plo = reinterpret_cast<uint16_t *>(&sh.pbuf[36 * (r0 + 1)]);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                uint32_t hi, lo;
                if (TBF && !vpacked) split2_bf16(pp[2 * k], pp[2 * k + 1], hi, lo);   // dense bf16 V
                else split2(pp[2 * k], pp[2 * k + 1], hi, lo);
                phi[32 * k + row] = static_cast<uint16_t>(hi);
                phi[32 * k + 16 + row] = static_cast<uint16_t>(hi >> 16);
                plo[32 * k + row] = static_cast<uint16_t>(lo);
                plo[32 * k + 16 + row] = static_cast<uint16_t>(lo >> 16);
            }
        }
        lds_sync();

        // ------------------------------------------------------------ P'.V
        f32x4 O[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) O[m] = zf;
        if (vpacked) {
            // the lane's 16 token words first (one LDS round trip), then unpack:
            // w0 = code bits 0..31 of token 16*grp + i (i = 8*kk2 + e), w1 = bits 32..63
            uint32_t w0[16], w1[16];
            const uint32_t *vs0 = vst + 16 * grp * VROW_DW + vdw;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t *vp = vs0 + i * VROW_DW;
                w0[i] = __builtin_amdgcn_alignbit(vp[1], vp[0], vsh);
                w1[i] = (BITS == 3) ? 0u : __builtin_amdgcn_alignbit(vp[2], vp[1], vsh);
            }
#pragma unroll
            for (int kk2 = 0; kk2 < 2; ++kk2) {
                const uint4 pv = *reinterpret_cast<const uint4 *>(pb_rd + pb_step * (8 * grp + 4 * kk2));
                const u32x4 pa = {pv.x, pv.y, pv.z, pv.w};
                uint32_t D[8][4];   // [tile m][token pair k]
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int ia = 8 * kk2 + 2 * k, ib = ia + 1;
                    if constexpr (BITS == 3) {
                        uint32_t d8[8];
                        vpair3(w0[ia], w0[ib], d8);
#pragma unroll
                        for (int m = 0; m < 8; ++m) D[m][k] = d8[m];
                    } else {
                        uint32_t d8[8];
                        vpair5(w0[ia], w1[ia], w0[ib], w1[ib], d8);
#pragma unroll
                        for (int m = 0; m < 8; ++m) D[m][k] = d8[m];
                    }
                }
#pragma unroll
                for (int m = 0; m < 8; ++m) O[m] = mfma(pa, u32x4{D[m][0], D[m][1], D[m][2], D[m][3]}, O[m]);
            }
        } else {
#pragma unroll
            for (int kk2 = 0; kk2 < 2; ++kk2) {
                const uint4 pv = *reinterpret_cast<const uint4 *>(pb_rd + pb_step * (8 * grp + 4 * kk2));
                const u32x4 pa = {pv.x, pv.y, pv.z, pv.w};
                uint32_t D[8][4];
                // dense V: tokens 16*grp + 8*kk2 + e, channels 8*row .. 8*row+7.
                // Tokens past `valid` read the last valid token (in bounds); their
                // weights are zero.
                const uint16_t *vrow = p.v.tail + (seqrow * p.v.tail_cap + t0 - nbv * kBlockTok) * kDim + 8 * row;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int ta = 16 * grp + 8 * kk2 + 2 * k, tb = ta + 1;
                    const uint4 xa4 = ld16(vrow + (ta < valid ? ta : valid - 1) * kDim);
                    const uint4 xb4 = ld16(vrow + (tb < valid ? tb : valid - 1) * kDim);
                    bad_in |= (x8_nonfinite<TBF>(xa4) | x8_nonfinite<TBF>(xb4)) != 0;
                    const uint32_t xa[4] = {xa4.x, xa4.y, xa4.z, xa4.w};
                    const uint32_t xb[4] = {xb4.x, xb4.y, xb4.z, xb4.w};
#pragma unroll
                    for (int m = 0; m < 8; ++m)
                        D[m][k] = perm(xb[m >> 1], xa[m >> 1], (m & 1) ? 0x07060302u : 0x05040100u);
                }
#pragma unroll
                for (int m = 0; m < 8; ++m) O[m] = mfma_t<TBF>(pa, u32x4{D[m][0], D[m][1], D[m][2], D[m][3]}, O[m]);
            }
        }
        // ------------------------------------------------------------ epilogue
        if (vpacked) {
            const uint4 vs4 = *reinterpret_cast<const uint4 *>(mst + 192 + 4 * row);
            const uint4 vm4 = *reinterpret_cast<const uint4 *>(mst + 256 + 4 * row);
            const uint32_t VS[4] = {vs4.x, vs4.y, vs4.z, vs4.w};
            const uint32_t VM[4] = {vm4.x, vm4.y, vm4.z, vm4.w};
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                const float g = F * (static_cast<float>(1u << (24 - LY::kV[m])) / kPScale);
                const float sc = (m & 1) ? f16hi(VS[m >> 1]) : f16lo(VS[m >> 1]);
                const float mc = (m & 1) ? f16hi(VM[m >> 1]) : f16lo(VM[m >> 1]);
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    float a = __builtin_fmaf(mc, spf[j], acc[j][m]);
                    acc[j][m] = __builtin_fmaf(sc, (O[m][2 * j] + O[m][2 * j + 1]) * g, a);
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < 8; ++m)
#pragma unroll
                for (int j = 0; j < NJ; ++j) acc[j][m] += (O[m][2 * j] + O[m][2 * j + 1]) * (1.f / kPScale);
        }
    };

    using F_ = std::false_type;
    using T_ = std::true_type;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if (nfb > 0) {   // (block fast_blk(0) is already in flight to stage 0)
        for (int64_t j = 0;;) {
            block(T_{}, S0{}, fast_blk(j), (j + 1 < nfb) ? fast_blk(j + 1) : -1);
            if (++j >= nfb) break;
            block(T_{}, S1{}, fast_blk(j), (j + 1 < nfb) ? fast_blk(j + 1) : -1);
            if (++j >= nfb) break;
        }
    }
    for (int64_t t0 = (t_fast > t_begin) ? t_fast : t_begin; t0 < t_end; t0 += kBlockTok)
        block(F_{}, S0{}, t0, -1);   // (no DMA in flight here)

    // ---------------------------------------------------------------- partials
#pragma unroll
    for (int j = 0; j < NJ; ++j) l_run[j] = red16_sum(l_run[j]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int h = grp + 4 * j;
        if (h >= G) continue;
        const int64_t bh = static_cast<int64_t>(b) * p.heads_q + hq0 + h;
        float *dst = p.partials + (bh * p.n_splits + slot) * kPartStride;
        if (row == 0) {
            dst[0] = (m_run[j] == -INFINITY) ? -INFINITY : m_run[j] * kLn2;
            dst[1] = l_run[j];
            dst[2] = 0.f;
            dst[3] = 0.f;
            bad |= !finite(l_run[j]);
            // partial count of this (sequence, q-head), read by the merge
            reinterpret_cast<int32_t *>(p.partials + p.batch * p.heads_q * p.n_splits * kPartStride)[bh] = count;
        }
        float4 *o = reinterpret_cast<float4 *>(dst + 4 + 8 * row);
        o[0] = float4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
        o[1] = float4{acc[j][4], acc[j][5], acc[j][6], acc[j][7]};
#pragma unroll
        for (int m = 0; m < 8; ++m) bad |= !finite(acc[j][m]);
    }
    if (bad) raise_status(p.status, NSN_ST_NONFINITE_ATTN);
    if (bad_in) raise_status(p.status, NSN_ST_NONFINITE_ATTN_INPUT);
}

// Work partition over a fixed grid of waves, balanced whatever the ragged
// lengths.  Normally each (sequence, kv-head) stream is cut into near-equal
// contiguous ranges on waves of its own, one segment per wave (partial slot =
// range index).  With more streams than waves (or more than 64 sequences) the
// 64-token blocks of all streams are laid end to end and cut into equal
// ranges ("stream-K"); a range that crosses a stream boundary yields one
// partial per stream, wave w's for stream s in slot w - first_wave(s).
template <int BITS, int QDT, bool SCORES, int GRP, bool TBF>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) void attn_fast_kernel(FastParams p) {
    using S = LdsShape<BITS, GRP>;
    __shared__ u32x4 s_afrag[S::ROWS * 16 + 1];
    __shared__ uint32_t s_pbuf[S::ROWS * 36 + 4];
    __shared__ uint32_t s_k0[S::NBW], s_k1[S::NBW], s_v0[S::NBW], s_v1[S::NBW];
    __shared__ uint32_t s_m0[S::MW], s_m1[S::MW];
    const Lds<BITS, GRP> sh{s_afrag, s_pbuf, s_k0, s_k1, s_v0, s_v1, s_m0, s_m1};
    const int l = threadIdx.x;
    // Lane l of a chunk holds sequence c0 + l: its length, packed K / V block
    // counts and 64-token block count -- one vector load per field for 64
    // sequences rather than one dependent scalar load per sequence.  The
    // first chunk's fields are loaded before the LDS set-up, which then
    // overlaps their latency.
    auto fields = [&](int64_t bb, int32_t &t, int32_t &nk, int32_t &nv) {
        t = nk = nv = 0;
        if (bb < p.batch) {
            t = p.seq_len[bb];
            nk = (!SCORES && p.k.blocks) ? p.k.blocks[bb] : 0;
            nv = p.v.blocks ? p.v.blocks[bb] : 0;
        }
    };
    int32_t t_0, nk_0, nv_0;
    fields(l, t_0, nk_0, nv_0);
    // empty A rows and the zero entries stay zero
    for (int i = l; i < S::ROWS * 16 + 1; i += 64) s_afrag[i] = u32x4{0u, 0u, 0u, 0u};
    for (int i = l; i < S::ROWS * 36 + 4; i += 64) s_pbuf[i] = 0u;
    lds_sync();

    const int64_t H = p.heads_kv;
    int64_t c0 = 0;
    int32_t t_l = 0, nk_l = 0, nv_l = 0, nb_l = 0;
    int64_t incl = 0;   // blocks of sequences c0 .. c0 + l, all kv-heads
    // A sequence's length t, or 0 when its blocks (nk, nv) or tail lie past
    // the cache's capacity (the launch-time host checks cover checked calls;
    // a graph replay with device lengths has only this one): nothing of such
    // a sequence is read, and the status word says why.  (Lanes past the
    // batch hold t = nk = nv = 0, which is usable and empty.)
    bool over = false;
    auto usable = [&](int32_t t, int32_t &nk, int32_t &nv) -> int32_t {
        auto fits = [&](const FastSide &sd, int32_t nb, bool present) {
            if (!present) return true;
            if (nb < 0 || nb > sd.block_cap) return false;
            const int64_t rest = static_cast<int64_t>(t) - static_cast<int64_t>(nb) * kBlockTok;
            return rest <= 0 || (sd.tail != nullptr && rest <= sd.tail_cap);
        };
        const bool ok = (SCORES ? t <= p.scores_cap : fits(p.k, nk, true)) && fits(p.v, nv, true);
        if (!ok) {
            over = true;
            nk = nv = 0;
            return 0;
        }
        return t > 0 ? t : 0;
    };
    auto take_chunk = [&](int32_t t, int32_t nk, int32_t nv) {
        t_l = usable(t, nk, nv);
        nk_l = nk;
        nv_l = nv;
        nb_l = static_cast<int32_t>((static_cast<int64_t>(t_l) + kBlockTok - 1) / kBlockTok);
        incl = H * static_cast<int64_t>(static_cast<uint32_t>(wave_incl_scan32(nb_l)));   // (< 2^32: nb_l <= 2^25)
    };
    auto load_chunk = [&]() {
        int32_t t, nk, nv;
        fields(c0 + l, t, nk, nv);
        take_chunk(t, nk, nv);
    };
    // A sequence with no usable token gets no segment: wave 0 writes partial
    // count 0 for its q-heads, so that the merge never reads a stale slot.
    auto mark_empty = [&](int64_t c, int32_t t) {
        if (blockIdx.x != 0 || c + l >= p.batch || t != 0) return;
        int32_t *cnt = reinterpret_cast<int32_t *>(p.partials + p.batch * p.heads_q * p.n_splits * kPartStride) +
                       (c + l) * p.heads_q;
        for (int64_t h = 0; h < p.heads_q; ++h) cnt[h] = 0;
    };
    take_chunk(t_0, nk_0, nv_0);
    mark_empty(0, t_l);
    int64_t N = lane_get(incl, 63);
    for (int64_t c = 64; c < p.batch; c += 64) {   // sequences past the first 64
        int32_t tr, nk, nv;
        fields(c + l, tr, nk, nv);
        const int32_t t = usable(tr, nk, nv);
        mark_empty(c, t);
        const int32_t nbt = static_cast<int32_t>((static_cast<int64_t>(t) + kBlockTok - 1) / kBlockTok);
        N += H * static_cast<int64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(wave_incl_scan32(nbt), 63)));
    }
    if (blockIdx.x == 0 && __ballot(over)) raise_status(p.status, l == 0 ? NSN_ST_CAPACITY : 0);
    if (N == 0) return;
    const int64_t W = gridDim.x;
    int lane = 0;   // (uniform) the lane holding the current sequence
    auto at = [&](int32_t x) { return static_cast<int64_t>(__builtin_amdgcn_readlane(x, lane)); };

    const int64_t nstr = H * wave_sum(nb_l > 0);   // streams with blocks (first 64 sequences)
    if (p.batch <= 64 && nstr <= W) {
        // Per-stream partition (every stream fits on its own waves): stream s
        // gets n_s = ceil(nb_s / P) waves with contiguous block ranges, P the
        // smallest block count per wave with sum_s n_s <= W.  Each wave runs
        // exactly one segment.  Since sum_s ceil(nb_s / P) <= N / P + nstr,
        // the search starts below ceil(N / (W - nstr)).
        int64_t lo = udivq(N + W - 1, W), hi = wave_max(nb_l);
        lo = (lo > p.min_blocks) ? lo : p.min_blocks;
        if (nstr < W) {   // (any P >= ub fits; the answer is the first fit >= lo)
            int64_t ub = udivq(N + (W - nstr) - 1, W - nstr);
            ub = (ub > lo) ? ub : lo;
            hi = (ub < hi) ? ub : hi;
        }
        lo = (lo < hi) ? lo : hi;
        while (lo < hi) {
            const int32_t mid = static_cast<int32_t>((lo + hi) / 2);
            const int32_t ns = (nb_l + mid - 1) / mid;
            if (H * wave_sum(ns < W + 1 ? ns : static_cast<int32_t>(W + 1)) <= W) hi = mid;
            else lo = mid + 1;
        }
        const int32_t P = static_cast<int32_t>(lo);
        const int32_t n_l = (nb_l + P - 1) / P;
        const int64_t wincl = H * static_cast<int64_t>(wave_incl_scan32(n_l));   // waves of sequences 0 .. l
        // Wave index w.  The workgroups dispatched first take the first wave
        // slot of every SIMD; a second-slot wave shares its SIMD and loses
        // most issue conflicts, so first-slot waves get longer ranges, and
        // each stream's consecutive waves mix the slots:
        //   8 waves per CU (weighted 1): blockIdx < W/2 are first-slot waves
        //   at even w, the others at odd w; ranges 5:4 (measured: ~20 % more
        //   blocks per unit time);
        //   6 waves per CU (weighted 2; 4 SIMDs hold 4 first-slot and 2
        //   second-slot waves): blockIdx < 2W/3 are first-slot waves at
        //   w % 3 in {0, 1}, the others at w % 3 == 2; ranges 8:7 (measured:
        //   2.71 against 3.09 us per block).
        const int64_t bx = blockIdx.x;
        const int wm = (p.weighted == 1 && W % 2 == 0) ? 1 : (p.weighted == 2 && W % 6 == 0) ? 2 : 0;
        int64_t w = bx;
        if (wm == 1) w = (bx < W / 2) ? 2 * bx : 2 * (bx - W / 2) + 1;
        else if (wm == 2) w = (bx < 2 * W / 3) ? 3 * (bx >> 1) + (bx & 1) : 3 * (bx - 2 * W / 3) + 2;
        const uint64_t hit = __ballot(l < p.batch && wincl > w);
        if (!hit) return;   // a spare wave
        lane = __ffsll(static_cast<unsigned long long>(hit)) - 1;
        const int64_t n = at(n_l), nb = at(nb_l);
        const int64_t r = w - (lane_get(wincl, lane) - H * n);
        const int kvh = static_cast<int>(udivq(r, n));
        const int64_t k = r - kvh * n;
        const int64_t w0 = w - k;   // the stream's first wave
        auto cw = [&](int64_t j) -> int64_t {   // summed weight of the stream's waves 0 .. j-1
            if (wm == 1) {
                const int64_t first = (w0 + j + 1) / 2 - (w0 + 1) / 2;   // even w in [w0, w0 + j)
                return 5 * first + 4 * (j - first);
            }
            if (wm == 2) {
                const int64_t second = (w0 + j) / 3 - w0 / 3;   // w % 3 == 2 in [w0, w0 + j)
                return 8 * (j - second) + 7 * second;
            }
            return j;
        };
        // Cost units: a packed block 1, a block of dense fp16 tokens 3 (its
        // 32 KB per side are read without the prefetch pipeline).
        const int64_t nkb = SCORES ? at(nv_l) : at(nk_l), nvb = at(nv_l);
        int64_t nbp = (nkb < nvb) ? nkb : nvb;
        nbp = (nbp < nb) ? nbp : nb;
        const int64_t U = nbp + 3 * (nb - nbp), ctot = cw(n);
        auto blk = [&](int64_t c) { return (c <= nbp) ? c : nbp + (c - nbp + 1) / 3; };
        const int64_t i0 = blk(udivq(cw(k) * U, ctot)), i1 = blk(udivq(cw(k + 1) * U, ctot));
        const int64_t T = at(t_l);
        if (n <= p.n_splits) {
            segment<BITS, QDT, SCORES, GRP, TBF>(p, sh, lane, kvh, i0 * kBlockTok, (i1 * kBlockTok < T) ? i1 * kBlockTok : T,
                                            at(nk_l), at(nv_l), static_cast<int>(k), static_cast<int>(n));
        } else {
            raise_status(p.status, NSN_ST_WORKSPACE);   // workspace too small for this layout
        }
        return;
    }

    // Stream-K partition (more streams than waves, or more than 64
    // sequences): the blocks of all streams laid end to end, P per wave.
    int64_t P = udivq(N + W - 1, W);
    if (P < p.min_blocks) P = p.min_blocks;
    int64_t g = static_cast<int64_t>(blockIdx.x) * P;
    const int64_t g1 = (g + P < N) ? g + P : N;
    if (g >= g1) return;

    // the stream holding block g: first sequence whose blocks end past g
    int64_t base = 0;   // first block of chunk c0
    for (;;) {
        const uint64_t hit = __ballot(c0 + l < p.batch && base + incl > g);
        if (hit) {
            lane = __ffsll(static_cast<unsigned long long>(hit)) - 1;
            break;
        }
        base += lane_get(incl, 63);
        c0 += 64;
        if (c0 >= p.batch) return;   // (not reached: g < N)
        load_chunk();
    }
    int64_t nb = at(nb_l);
    int64_t start_b = base + lane_get(incl, lane) - H * nb;   // first block of sequence c0 + lane
    int kvh = static_cast<int>(udivq(g - start_b, nb));
    int64_t i0 = g - start_b - kvh * nb;
    while (g < g1) {
        const int64_t start_s = start_b + kvh * nb;
        const int64_t i1 = (i0 + (g1 - g) < nb) ? i0 + (g1 - g) : nb;
        const int64_t T = at(t_l);
        const int64_t s0 = udivq(start_s, P);
        const int slot = static_cast<int>(blockIdx.x - s0);
        const int count = static_cast<int>(udivq(start_s + nb - 1, P) - s0 + 1);
        if (slot < p.n_splits && count <= p.n_splits) {
            segment<BITS, QDT, SCORES, GRP, TBF>(p, sh, static_cast<int>(c0 + lane), kvh, i0 * kBlockTok,
                                            (i1 * kBlockTok < T) ? i1 * kBlockTok : T, at(nk_l), at(nv_l), slot,
                                            count);
        } else {
            raise_status(p.status, NSN_ST_WORKSPACE);   // workspace too small for this layout
        }
        g += i1 - i0;
        i0 = 0;
        if (++kvh == p.heads_kv && g < g1) {   // next sequence (one with blocks: g < g1 <= N)
            kvh = 0;
            start_b += H * nb;
            do {
                if (++lane == 64) {
                    c0 += 64;
                    if (c0 >= p.batch) return;   // (not reached)
                    load_chunk();
                    lane = 0;
                }
                nb = at(nb_l);
            } while (nb == 0);
        }
    }
}

}  // namespace fast

// Entry used by nsn_decode_attention for NSN_ATTN_FAST (nsn_attn.hip).
int launch_attn_fast(const nsn_attn_args *a, hipStream_t st) {
    using namespace fast;
    const bool scores = a->k_mode == NSN_KV_SCORES;
    const int64_t G = a->heads_q / a->heads_kv;
    if (G < 1 || G > kMaxGroup) return NSN_EINVAL;
    if (a->bits != 3 && a->bits != 5) return NSN_EINVAL;
    if (a->q_dtype != NSN_DTYPE_BF16 && a->q_dtype != NSN_DTYPE_F16) return NSN_EINVAL;
    auto side_ok = [](const nsn_kv_side &s) {
        if (s.blocks && (!s.codes || !s.mins || !s.scales || !s.factors)) return false;
        if (s.codes && (reinterpret_cast<uintptr_t>(s.codes) & 15u)) return false;
        if (s.mins && (reinterpret_cast<uintptr_t>(s.mins) & 15u)) return false;
        if (s.scales && (reinterpret_cast<uintptr_t>(s.scales) & 15u)) return false;
        if (s.factors && (reinterpret_cast<uintptr_t>(s.factors) & 15u)) return false;
        if (s.tail && ((s.tail_dtype != NSN_DTYPE_F16 && s.tail_dtype != NSN_DTYPE_BF16) ||
                       (reinterpret_cast<uintptr_t>(s.tail) & 15u)))
            return false;
        return true;
    };
    if (!side_ok(a->v) || (!scores && !side_ok(a->k))) return NSN_EINVAL;
    // one tail dtype per launch (a kernel variant each): both sides' tails, when present, agree
    const bool vtail_bf = a->v.tail && a->v.tail_dtype == NSN_DTYPE_BF16;
    const bool ktail_bf = !scores && a->k.tail && a->k.tail_dtype == NSN_DTYPE_BF16;
    if (!scores && a->k.tail && a->v.tail && ktail_bf != vtail_bf) return NSN_EINVAL;
    const bool tbf = vtail_bf || ktail_bf;
    if (a->q && (reinterpret_cast<uintptr_t>(a->q) & 1u)) return NSN_EINVAL;
    if (a->n_splits < 2 || a->max_seq_len <= 0) return NSN_EINVAL;
    FastParams p{};
    p.q = a->q;
    p.batch = a->batch;
    p.heads_q = a->heads_q;
    p.heads_kv = a->heads_kv;
    p.group = static_cast<int>(G);
    p.scale = a->scale;
    p.seq_len = a->seq_len;
    p.n_splits = a->n_splits;
    // a stream of n blocks touches at most ceil(n / P) + 1 waves
    const int64_t nb_max = (static_cast<int64_t>(a->max_seq_len) + kBlockTok - 1) / kBlockTok;
    p.min_blocks = (nb_max + a->n_splits - 2) / (a->n_splits - 1);
    auto side = [](const nsn_kv_side &s) {
        return FastSide{s.codes, s.mins, s.scales, s.factors, s.blocks, s.block_cap,
                        static_cast<const uint16_t *>(s.tail), s.tail_cap};
    };
    if (!scores) p.k = side(a->k);
    p.v = side(a->v);
    p.scores = a->scores;
    p.scores_cap = a->scores_cap;
    p.partials = a->partials;
    p.status = a->status;
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return NSN_ELAUNCH;
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return NSN_ELAUNCH;
    // 3-bit: two resident waves per SIMD, one per (CU, SIMD, slot).  5-bit:
    // the double-buffered 5 KB stages (26.8 KB of LDS per wave) leave room
    // for 6 waves per CU, so a grid of 8 per CU would run its last quarter
    // as a second, mostly idle round.
    // (Measured on C3: 6 per CU 84 us, 4 or 5 per CU 87 us, 8 per CU 100 us.)
    const int per_cu = (a->bits == 3) ? 8 : 6;
    p.weighted = per_cu == 8 ? 1 : (per_cu == 6 ? 2 : 0);
    const dim3 grid(static_cast<unsigned>(per_cu * (cus[dev] > 0 ? cus[dev] : 256)));
    const bool bf = a->q_dtype == NSN_DTYPE_BF16;
#define NSN_FAST_LAUNCH2(B_, Q_, S_, G_, T_) \
    hipLaunchKernelGGL((attn_fast_kernel<B_, Q_, S_, G_, T_>), grid, dim3(64), 0, st, p)
#define NSN_FAST_LAUNCH1(B_, Q_, S_, G_)                              \
    do {                                                              \
        if (tbf) NSN_FAST_LAUNCH2(B_, Q_, S_, G_, true);              \
        else NSN_FAST_LAUNCH2(B_, Q_, S_, G_, false);                 \
    } while (0)
#define NSN_FAST_LAUNCH(B_, Q_, S_)                                   \
    do {                                                              \
        if (G <= 4) NSN_FAST_LAUNCH1(B_, Q_, S_, 4);                  \
        else NSN_FAST_LAUNCH1(B_, Q_, S_, 8);                         \
    } while (0)
    if (a->bits == 3) {
        if (bf) { if (scores) NSN_FAST_LAUNCH(3, NSN_DTYPE_BF16, true); else NSN_FAST_LAUNCH(3, NSN_DTYPE_BF16, false); }
        else { if (scores) NSN_FAST_LAUNCH(3, NSN_DTYPE_F16, true); else NSN_FAST_LAUNCH(3, NSN_DTYPE_F16, false); }
    } else {
        if (bf) { if (scores) NSN_FAST_LAUNCH(5, NSN_DTYPE_BF16, true); else NSN_FAST_LAUNCH(5, NSN_DTYPE_BF16, false); }
        else { if (scores) NSN_FAST_LAUNCH(5, NSN_DTYPE_F16, true); else NSN_FAST_LAUNCH(5, NSN_DTYPE_F16, false); }
    }
#undef NSN_FAST_LAUNCH
#undef NSN_FAST_LAUNCH1
#undef NSN_FAST_LAUNCH2
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

}  // namespace nsn
