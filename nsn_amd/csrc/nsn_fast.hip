// Fast single-query decode attention over NSN-packed K/V for gfx950 (MFMA).
//
// Same work decomposition and partial format as the exact-order kernel in
// nsn_attn.hip (work unit = sequence x kv-head x context split, all G query
// heads of the kv-head served by one pass over its blocks; log-sum-exp merge
// of the splits).  One wave per work unit; per 64-token packed block:
//
//   scores   S[h,t] = scale * f_K[t] * (q_h.m_K + sum_c (q_h[c] s_K[c]) z_K[t,c])
//            The contraction over channels runs on v_mfma_f32_16x16x32_f16:
//            B = raw codes z as fp16 subnormals (z * 2^-24, exact), A = the
//            coefficient rows q_h (.) s_K split into fp16 hi + lo parts.
//   softmax  online (running max / sum per head), exp2 with log2(e) folded.
//   output   acc[h,c] += s_V[c] * sum_t p'[h,t] z_V[t,c] + m_V[c] * sum_t p'[h,t]
//            with p' = p * f_V.  The V codes are transposed (tokens onto the
//            contraction axis) by an MFMA against an identity fragment, then
//            P' (fp16 hi/lo rows) x Z_V runs on MFMA.
//
// f_K, f_V are the per-token decode factors n / |m + s*z| of each packed block
// (nsn_block_factors): constant once a block is encoded, so they are read, not
// recomputed.  Reconstruction therefore equals nsn_decode's up to rounding
// (loop_kv_pilot.py:216-225); results match the fp64 oracle within the stated
// tolerance, not bit for bit.  Tokens past the packed prefix (the fp16 tail,
// or a fully dense fp16 K/V for the fp16 baseline) take the same MFMA path
// with the fp16 values themselves as operands.
//
// Reference routes replaced: experiments/ac08/source/loop_kv_vf01_kernel.py:56-139
// (fused readout), experiments/nb06/source/loop_kv_nb06_kernel.py:54-154 (GQA),
// experiments/ac08/source/loop_kv_af01_kernel.py:13-68 (score-input readout).
#include "nsn_common.hpp"

namespace nsn {
namespace fast {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __fp16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kPartStride = 132;
constexpr int kMaxGroup = 8;
constexpr float kTwo24 = 16777216.0f;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// Two fp32 -> packed fp16 pair, round toward zero (v_cvt_pkrtz_f16_f32).
__device__ __forceinline__ uint32_t pkrtz(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ float lo_f32(uint32_t p) { return static_cast<float>(__builtin_bit_cast(half2_t, p)[0]); }
__device__ __forceinline__ float hi_f32(uint32_t p) { return static_cast<float>(__builtin_bit_cast(half2_t, p)[1]); }

// Split 8 fp32 values into fp16 hi (round toward zero) and lo = rn(x - hi):
// hi + lo carries ~22 significant bits.
__device__ __forceinline__ void split_hilo(const float (&x)[8], u32x4 &hi, u32x4 &lo) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t h = pkrtz(x[2 * k], x[2 * k + 1]);
        const float r0 = x[2 * k] - lo_f32(h), r1 = x[2 * k + 1] - hi_f32(h);
        hi[k] = h;
        lo[k] = pkrtz(r0, r1);
    }
}

// ---------------------------------------------------------------------------
// Channel order of the MFMA contraction.  A lane owns a 32-channel chunk of
// one token (chunk = lane / 16); its codes are unpacked into 16 dwords
// D[j] = code(lo_j) | code(hi_j) << 16 (two fp16 subnormals), pair j covering
// local channels (j, j+16) -- or (j+16, j) for j = 6..9 at 3 bits, where that
// order is the cheaper one to extract.  K-step kk feeds D[4kk .. 4kk+3].
// ---------------------------------------------------------------------------
template <int BITS>
__host__ __device__ constexpr bool pair_reversed(int j) { return BITS == 3 && j >= 6 && j <= 9; }
template <int BITS>
__host__ __device__ constexpr int pi_channel(int kk, int e) {   // local channel of fragment element e
    const int j = 4 * kk + e / 2;
    const bool second = (e & 1) != pair_reversed<BITS>(j);
    return second ? j + 16 : j;
}

__device__ __forceinline__ uint32_t bfi16(uint32_t lo_src, uint32_t hi_src) {   // low half of a, high half of b
    return (lo_src & 0xffffu) | (hi_src & 0xffff0000u);
}
__device__ __forceinline__ uint32_t alignbit(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbit(hi, lo, s);
}

// 3-bit chunk: 96 bits (u0, u1, u2), code j at bits 3j .. 3j+2.
__device__ __forceinline__ void unpack3(uint32_t u0, uint32_t u1, uint32_t u2, uint32_t (&D)[16]) {
    constexpr uint32_t M = 0x00070007u;
    const uint32_t x = bfi16(u0, u1);
    D[0] = x & M;
    D[1] = (x >> 3) & M;
    D[2] = (x >> 6) & M;
    D[3] = (x >> 9) & M;
    D[4] = (x >> 12) & M;
    D[5] = ((u0 >> 15) & 7u) | ((alignbit(u2, u1, 31) & 7u) << 16);
    const uint32_t y = bfi16(u2, u0);
    D[6] = (y >> 2) & M;
    D[7] = (y >> 5) & M;
    D[8] = (y >> 8) & M;
    D[9] = (y >> 11) & M;
    D[10] = (alignbit(u1, u0, 30) & 7u) | (((u2 >> 14) & 7u) << 16);
    const uint32_t z = bfi16(u1, u2);
    D[11] = (z >> 1) & M;
    D[12] = (z >> 4) & M;
    D[13] = (z >> 7) & M;
    D[14] = (z >> 10) & M;
    D[15] = (z >> 13) & M;
}

// Generic chunk of 32 codes at BITS bits (BITS dwords).
template <int BITS>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&u)[BITS], int i) {
    const int pos = i * BITS, w = pos >> 5, sh = pos & 31;
    uint32_t v;
    if (sh + BITS <= 32) v = u[w] >> sh;
    else v = alignbit(u[w + 1], u[w], sh);
    return v & ((1u << BITS) - 1u);
}

template <int BITS>
__device__ __forceinline__ void unpack_chunk(const uint32_t (&u)[BITS], uint32_t (&D)[16]) {
    if constexpr (BITS == 3) {
        unpack3(u[0], u[1], u[2], D);
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int a = pair_reversed<BITS>(j) ? j + 16 : j, b = pair_reversed<BITS>(j) ? j : j + 16;
            D[j] = code_at<BITS>(u, a) | (code_at<BITS>(u, b) << 16);
        }
    }
}

// Dense fp16 chunk (32 halves in natural order, as 16 dwords) -> pair order.
template <int BITS>
__device__ __forceinline__ void pair_dense(const uint32_t (&h)[16], uint32_t (&D)[16]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int a = pair_reversed<BITS>(j) ? j + 16 : j, b = pair_reversed<BITS>(j) ? j : j + 16;
        const uint32_t ha = (a & 1) ? (h[a >> 1] >> 16) : (h[a >> 1] & 0xffffu);
        const uint32_t hb = (b & 1) ? (h[b >> 1] & 0xffff0000u) : (h[b >> 1] << 16);
        D[j] = ha | hb;
    }
}

template <int QDT>
__device__ __forceinline__ float load_q(const void *q, int64_t idx) {
    return Elem<QDT>::load(static_cast<const uint16_t *>(q)[idx]);
}

struct FastSide {
    const uint8_t *codes;
    const uint16_t *mins, *scales;
    const float *factors;
    const int32_t *blocks;
    int64_t block_cap;
    const uint16_t *tail;   // fp16
    int64_t tail_cap;
};

struct FastParams {
    const void *q;
    int64_t heads_q, heads_kv;
    int group;
    float scale;
    const int32_t *seq_len;
    int split_tokens, n_splits;
    FastSide k, v;
    const float *scores;
    int64_t scores_cap;
    float *partials;
    int32_t *status;
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

// LDS hand-off inside the single wave of a workgroup: the wave's LDS accesses
// complete in order, so waiting for them (and stopping the compiler from
// moving memory accesses across) is enough -- no s_barrier, and prefetched
// global loads stay in flight.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Load the lane's 32-channel fp16 chunk of one dense token (64 bytes).
__device__ __forceinline__ void load_dense_chunk(const uint16_t *row, int grp, uint32_t (&h)[16]) {
    const uint4 *src = reinterpret_cast<const uint4 *>(row + 32 * grp);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint4 v = src[k];
        h[4 * k] = v.x; h[4 * k + 1] = v.y; h[4 * k + 2] = v.z; h[4 * k + 3] = v.w;
    }
}

// K-side data of a packed block (needed first; issued one block ahead).
template <int BITS>
struct KLoads {
    uint32_t kc[4][BITS];   // K codes: token 16*nt + row, chunk grp
    uint2 ks[2], km[2];     // K scale / min at the coefficient-prep channels (two runs of 4)
    float fk[4];            // K decode factors at tokens 16*nt + row
};
// V-side data (needed after the scores; issued when the block starts).
template <int BITS>
struct VLoads {
    uint32_t vc[4][BITS];   // V codes
    float fv[4];            // V decode factors
    uint32_t vsm[8];        // V scale | min << 16 at the output channels cch[n2]
};

template <int BITS>
__device__ __forceinline__ void issue_k_loads(const FastParams &p, int64_t ibk, int row, int grp, int wch,
                                              KLoads<BITS> &f) {
    constexpr int NB = packed_block_bytes(BITS);
    {
        const uint32_t *cb = reinterpret_cast<const uint32_t *>(p.k.codes + ibk * NB);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int w = 0; w < BITS; ++w) f.kc[nt][w] = cb[(16 * nt + row) * (4 * BITS) + grp * BITS + w];
        const uint16_t *sb = p.k.scales + ibk * kDim + wch;
        const uint16_t *mb = p.k.mins + ibk * kDim + wch;
        f.ks[0] = *reinterpret_cast<const uint2 *>(sb);
        f.ks[1] = *reinterpret_cast<const uint2 *>(sb + 16);
        f.km[0] = *reinterpret_cast<const uint2 *>(mb);
        f.km[1] = *reinterpret_cast<const uint2 *>(mb + 16);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) f.fk[nt] = p.k.factors[ibk * kBlockTok + 16 * nt + row];
    }
}

template <int BITS>
__device__ __forceinline__ void issue_v_loads(const FastParams &p, int64_t ibv, int row, int grp, const int (&cch)[8],
                                              VLoads<BITS> &f) {
    constexpr int NB = packed_block_bytes(BITS);
    const uint32_t *cb = reinterpret_cast<const uint32_t *>(p.v.codes + ibv * NB);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int w = 0; w < BITS; ++w) f.vc[nt][w] = cb[(16 * nt + row) * (4 * BITS) + grp * BITS + w];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) f.fv[nt] = p.v.factors[ibv * kBlockTok + 16 * nt + row];
#pragma unroll
    for (int n2 = 0; n2 < 8; ++n2)
        f.vsm[n2] = static_cast<uint32_t>(p.v.scales[ibv * kDim + cch[n2]]) |
                    (static_cast<uint32_t>(p.v.mins[ibv * kDim + cch[n2]]) << 16);
}

template <int BITS, int QDT, bool SCORES, int GRP>
__global__ __launch_bounds__(64) void attn_fast_kernel(FastParams p) {
    constexpr int NJ = GRP > 4 ? 2 : 1;  // coefficient-prep heads per lane (GRP >= group)
    const int G = p.group;                 // query heads per kv-head
    // A-operand fragments: [set 0 = packed coefficients (q.s), set 1 = dense (q)][row][chunk][kstep]
    __shared__ u32x4 afrag_s[2][16][4][4];
    __shared__ float pbuf[kMaxGroup][kBlockTok];
    __shared__ float qm_s[kMaxGroup];

    const int l = threadIdx.x;
    const int row = l & 15, grp = l >> 4;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int64_t seqrow = static_cast<int64_t>(b) * p.heads_kv + kvh;
    const int64_t T = p.seq_len[b];
    const int64_t t_begin = static_cast<int64_t>(split) * p.split_tokens;
    const int64_t t_end = t_begin + p.split_tokens < T ? t_begin + p.split_tokens : T;
    const int64_t hq0 = static_cast<int64_t>(kvh) * G;
    const float sc2 = p.scale * kLog2e;

    // coefficient-prep role: head (l>>4) [+4], chunk (l>>2)&3, kstep l&3 -> 8 channels
    const int wgq = (l >> 2) & 3, wkk = l & 3;
    const int wch = 32 * wgq + 4 * wkk;      // first channel of the lane's two runs of 4
    float qv[NJ][8];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int h = grp + 4 * j;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            qv[j][e] = (h < G) ? load_q<QDT>(p.q, (static_cast<int64_t>(b) * p.heads_q + hq0 + h) * kDim + 32 * wgq +
                                                       pi_channel<BITS>(wkk, e))
                               : 0.f;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int h = grp + 4 * j;
        if (h < G) {
            u32x4 hi, lo;
            split_hilo(qv[j], hi, lo);
            afrag_s[1][2 * h][wgq][wkk] = hi;
            afrag_s[1][2 * h + 1][wgq][wkk] = lo;
        }
    }
    // identity fragments for the token<->channel transposition: B[k=8*grp+e][j=row] = 1
    // iff grp == row/4 and e == 2*(row%4) + b  (b = 0, 1)
    u32x4 ident[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const bool on = (grp == (row >> 2)) && (k == (row & 3));
            ident[bb][k] = on ? (bb ? 0x3c000000u : 0x00003c00u) : 0u;
        }
    }
    // channel of PV output column `row` in N-tile n2 (kk = n2/2, half = n2%2)
    int cch[8];
#pragma unroll
    for (int n2 = 0; n2 < 8; ++n2) cch[n2] = 32 * (row >> 2) + pi_channel<BITS>(n2 >> 1, 2 * (row & 3) + (n2 & 1));

    // per-lane output heads (rows 4*grp .. 4*grp+3 = hA hi, hA lo, hB hi, hB lo)
    const int hA = 2 * grp, hB = 2 * grp + 1;
    const bool vA = hA < G, vB = hB < G;
    float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
    float acc[2][8];
#pragma unroll
    for (int n2 = 0; n2 < 8; ++n2) acc[0][n2] = acc[1][n2] = 0.f;
    bool bad = false;

    const int64_t nbk = (!SCORES && p.k.blocks) ? p.k.blocks[b] : 0;
    const int64_t nbv = p.v.blocks ? p.v.blocks[b] : 0;
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    const f32x4 zf = {0.f, 0.f, 0.f, 0.f};
    lds_sync();

    KLoads<BITS> cur;
    if (!SCORES && t_begin < t_end && t_begin < nbk * kBlockTok)
        issue_k_loads<BITS>(p, seqrow * p.k.block_cap + t_begin / kBlockTok, row, grp, wch, cur);

    for (int64_t t0 = t_begin; t0 < t_end; t0 += kBlockTok) {
        const int valid = static_cast<int>(t_end - t0 < kBlockTok ? t_end - t0 : kBlockTok);
        const bool kpacked = !SCORES && (t0 < nbk * kBlockTok);
        const bool vpacked = t0 < nbv * kBlockTok;
        const int64_t ibk = seqrow * p.k.block_cap + t0 / kBlockTok;
        const int64_t ibv = seqrow * p.v.block_cap + t0 / kBlockTok;
        // ---- this block's V loads, then the next block's K loads, before any compute
        VLoads<BITS> vl;
        if (vpacked) issue_v_loads<BITS>(p, ibv, row, grp, cch, vl);
        KLoads<BITS> nxt;
        const int64_t t1 = t0 + kBlockTok;
        if (!SCORES && t1 < t_end && t1 < nbk * kBlockTok) issue_k_loads<BITS>(p, ibk + 1, row, grp, wch, nxt);
        float s[2][4];   // scores (log2 domain) for heads hA, hB at tokens 16*nt + row

        // ------------------------------------------------------------ scores
        if constexpr (SCORES) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const int tt = 16 * nt + row;
                const bool ok = tt < valid;
                const float *sa = p.scores + (static_cast<int64_t>(b) * p.heads_q + hq0) * p.scores_cap + t0 + tt;
                s[0][nt] = (ok && vA) ? sa[hA * p.scores_cap] * kLog2e : -INFINITY;
                s[1][nt] = (ok && vB) ? sa[hB * p.scores_cap] * kLog2e : -INFINITY;
            }
        } else {
            u32x4 af[4];
            f32x4 C[4];
            if (kpacked) {
                // coefficient rows W = q (.) s_K (fp16 hi, lo) and q.m_K for head grp (+4)
                float sv[8], mv[8];
                {
                    const uint32_t sw[4] = {cur.ks[0].x, cur.ks[0].y, cur.ks[1].x, cur.ks[1].y};
                    const uint32_t mw[4] = {cur.km[0].x, cur.km[0].y, cur.km[1].x, cur.km[1].y};
                    float sa_[4], sb_[4], ma_[4], mb_[4];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        sa_[2 * i] = lo_f32(sw[i]); sa_[2 * i + 1] = hi_f32(sw[i]);
                        sb_[2 * i] = lo_f32(sw[2 + i]); sb_[2 * i + 1] = hi_f32(sw[2 + i]);
                        ma_[2 * i] = lo_f32(mw[i]); ma_[2 * i + 1] = hi_f32(mw[i]);
                        mb_[2 * i] = lo_f32(mw[2 + i]); mb_[2 * i + 1] = hi_f32(mw[2 + i]);
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool rev = pair_reversed<BITS>(4 * wkk + i);
                        sv[2 * i] = rev ? sb_[i] : sa_[i];
                        sv[2 * i + 1] = rev ? sa_[i] : sb_[i];
                        mv[2 * i] = rev ? mb_[i] : ma_[i];
                        mv[2 * i + 1] = rev ? ma_[i] : mb_[i];
                    }
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int h = grp + 4 * j;
                    float w[8], qm = 0.f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        w[e] = qv[j][e] * sv[e];
                        qm = __builtin_fmaf(qv[j][e], mv[e], qm);
                    }
                    qm = red16_sum(qm);
                    if (h < G) {
                        u32x4 hi, lo;
                        split_hilo(w, hi, lo);
                        afrag_s[0][2 * h][wgq][wkk] = hi;
                        afrag_s[0][2 * h + 1][wgq][wkk] = lo;
                        if (row == 0) qm_s[h] = qm;
                    }
                }
                lds_sync();
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) af[kk] = (row < 2 * G) ? afrag_s[0][row][grp][kk] : zero4;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    uint32_t D[16];
                    unpack_chunk<BITS>(cur.kc[nt], D);
                    C[nt] = zf;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const u32x4 bz = {D[4 * kk], D[4 * kk + 1], D[4 * kk + 2], D[4 * kk + 3]};
                        C[nt] = mfma(af[kk], bz, C[nt]);
                    }
                }
                const float qmA = vA ? qm_s[hA] : 0.f, qmB = vB ? qm_s[hB] : 0.f;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const float f = cur.fk[nt] * sc2;
                    s[0][nt] = vA ? (qmA + (C[nt][0] + C[nt][1]) * kTwo24) * f : -INFINITY;
                    s[1][nt] = vB ? (qmB + (C[nt][2] + C[nt][3]) * kTwo24) * f : -INFINITY;
                }
            } else {
                // dense fp16 keys: tokens t0 - 64*nbk + tt of the tail buffer
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) af[kk] = (row < 2 * G) ? afrag_s[1][row][grp][kk] : zero4;
                const int64_t base = t0 - nbk * kBlockTok;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const int tt = 16 * nt + row;
                    uint32_t h[16], D[16];
                    if (tt < valid) {
                        load_dense_chunk(p.k.tail + (seqrow * p.k.tail_cap + base + tt) * kDim, grp, h);
                    } else {
#pragma unroll
                        for (int k = 0; k < 16; ++k) h[k] = 0u;
                    }
                    pair_dense<BITS>(h, D);
                    C[nt] = zf;
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        const u32x4 bz = {D[4 * kk], D[4 * kk + 1], D[4 * kk + 2], D[4 * kk + 3]};
                        C[nt] = mfma(af[kk], bz, C[nt]);
                    }
                }
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    const bool ok = 16 * nt + row < valid;
                    s[0][nt] = (vA && ok) ? (C[nt][0] + C[nt][1]) * sc2 : -INFINITY;
                    s[1][nt] = (vB && ok) ? (C[nt][2] + C[nt][3]) * sc2 : -INFINITY;
                }
            }
        }

        // ------------------------------------------------------------ softmax
        float alpha[2], psum[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float bm = fmaxf(fmaxf(s[hh][0], s[hh][1]), fmaxf(s[hh][2], s[hh][3]));
            bm = red16_max(bm);
            const float mnew = fmaxf(m_run[hh], bm);
            const float msafe = (mnew == -INFINITY) ? 0.f : mnew;
            alpha[hh] = (m_run[hh] == -INFINITY) ? 0.f : exp2f(m_run[hh] - msafe);
            float ls = 0.f, ps = 0.f;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const float pw = (s[hh][nt] == -INFINITY) ? 0.f : exp2f(s[hh][nt] - msafe);
                ls += pw;
                const float pp = vpacked ? pw * vl.fv[nt] : pw;
                ps += pp;
                s[hh][nt] = pp;
            }
            ls = red16_sum(ls);
            psum[hh] = red16_sum(ps);
            l_run[hh] = l_run[hh] * alpha[hh] + ls;
            m_run[hh] = mnew;
        }
        if (vA) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) pbuf[hA][16 * nt + row] = s[0][nt];
        }
        if (vB) {
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) pbuf[hB][16 * nt + row] = s[1][nt];
        }
        lds_sync();

        // ------------------------------------------------------------ P'.V
        u32x4 pa[2];
        {
            const int h = row >> 1, part = row & 1;
#pragma unroll
            for (int kk2 = 0; kk2 < 2; ++kk2) {
                if (h < G) {
                    const float4 x0 = *reinterpret_cast<const float4 *>(&pbuf[h][32 * kk2 + 4 * grp]);
                    const float4 x1 = *reinterpret_cast<const float4 *>(&pbuf[h][32 * kk2 + 16 + 4 * grp]);
                    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                    u32x4 hi, lo;
                    split_hilo(x, hi, lo);
                    pa[kk2] = part ? lo : hi;
                } else {
                    pa[kk2] = zero4;
                }
            }
        }
        f32x4 O[8];
#pragma unroll
        for (int n2 = 0; n2 < 8; ++n2) O[n2] = zf;
#pragma unroll
        for (int kk2 = 0; kk2 < 2; ++kk2) {
            uint32_t Da[16], Db[16];
            if (vpacked) {
                unpack_chunk<BITS>(vl.vc[2 * kk2], Da);
                unpack_chunk<BITS>(vl.vc[2 * kk2 + 1], Db);
            } else {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int tt = 16 * (2 * kk2 + half) + row;
                    uint32_t h[16];
                    if (tt < valid) {
                        load_dense_chunk(p.v.tail + (seqrow * p.v.tail_cap + t0 - nbv * kBlockTok + tt) * kDim, grp, h);
                    } else {
#pragma unroll
                        for (int k = 0; k < 16; ++k) h[k] = 0u;
                    }
                    if (half) pair_dense<BITS>(h, Db);
                    else pair_dense<BITS>(h, Da);
                }
            }
#pragma unroll
            for (int n2 = 0; n2 < 8; ++n2) {
                const int kk = n2 >> 1, bb = n2 & 1;
                const u32x4 aA = {Da[4 * kk], Da[4 * kk + 1], Da[4 * kk + 2], Da[4 * kk + 3]};
                const u32x4 aB = {Db[4 * kk], Db[4 * kk + 1], Db[4 * kk + 2], Db[4 * kk + 3]};
                const f32x4 Ta = mfma(aA, ident[bb], zf);
                const f32x4 Tb = mfma(aB, ident[bb], zf);
                const u32x4 bz = {pkrtz(Ta[0], Ta[1]), pkrtz(Ta[2], Ta[3]), pkrtz(Tb[0], Tb[1]), pkrtz(Tb[2], Tb[3])};
                O[n2] = mfma(pa[kk2], bz, O[n2]);
            }
        }
        // ------------------------------------------------------------ epilogue
        if (vpacked) {
#pragma unroll
            for (int n2 = 0; n2 < 8; ++n2) {
                const float sc = f16_bits_to_f32(static_cast<uint16_t>(vl.vsm[n2] & 0xffffu)) * kTwo24;
                const float mc = f16_bits_to_f32(static_cast<uint16_t>(vl.vsm[n2] >> 16));
                acc[0][n2] = acc[0][n2] * alpha[0] + (sc * (O[n2][0] + O[n2][1]) + mc * psum[0]);
                acc[1][n2] = acc[1][n2] * alpha[1] + (sc * (O[n2][2] + O[n2][3]) + mc * psum[1]);
            }
        } else {
#pragma unroll
            for (int n2 = 0; n2 < 8; ++n2) {
                acc[0][n2] = acc[0][n2] * alpha[0] + (O[n2][0] + O[n2][1]);
                acc[1][n2] = acc[1][n2] * alpha[1] + (O[n2][2] + O[n2][3]);
            }
        }
        cur = nxt;
        lds_sync();   // pbuf / afrag_s are rewritten by the next block
    }

    // ---------------------------------------------------------------- partials
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const int h = hh ? hB : hA;
        const bool v = hh ? vB : vA;
        if (!v) continue;
        float *dst = p.partials + ((static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.n_splits + split) * kPartStride;
        if (row == 0) {
            dst[0] = (m_run[hh] == -INFINITY) ? -INFINITY : m_run[hh] * kLn2;
            dst[1] = l_run[hh];
            dst[2] = 0.f;
            dst[3] = 0.f;
            bad |= !finite(l_run[hh]);
        }
#pragma unroll
        for (int n2 = 0; n2 < 8; ++n2) {
            dst[4 + cch[n2]] = acc[hh][n2];
            bad |= !finite(acc[hh][n2]);
        }
    }
    if (bad) raise_status(p.status, NSN_ST_NONFINITE_ATTN);
}

}  // namespace fast

// Entry used by nsn_decode_attention for NSN_ATTN_FAST (nsn_attn.hip).
int launch_attn_fast(const nsn_attn_args *a, hipStream_t st) {
    using namespace fast;
    const bool scores = a->k_mode == NSN_KV_SCORES;
    const int64_t G = a->heads_q / a->heads_kv;
    if (G > kMaxGroup) return NSN_EINVAL;
    if (a->bits != 3 && a->bits != 5) return NSN_EINVAL;
    if (a->q_dtype != NSN_DTYPE_BF16 && a->q_dtype != NSN_DTYPE_F16) return NSN_EINVAL;
    auto side_ok = [](const nsn_kv_side &s) {
        if (s.blocks && (!s.codes || !s.mins || !s.scales || !s.factors)) return false;
        if (s.codes && (reinterpret_cast<uintptr_t>(s.codes) & 15u)) return false;
        if (s.tail && (s.tail_dtype != NSN_DTYPE_F16 || (reinterpret_cast<uintptr_t>(s.tail) & 15u))) return false;
        return true;
    };
    if (!side_ok(a->v) || (!scores && !side_ok(a->k))) return NSN_EINVAL;
    FastParams p{};
    p.q = a->q;
    p.heads_q = a->heads_q;
    p.heads_kv = a->heads_kv;
    p.group = static_cast<int>(G);
    p.scale = a->scale;
    p.seq_len = a->seq_len;
    p.split_tokens = a->split_tokens;
    p.n_splits = a->n_splits;
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
    const dim3 grid(static_cast<unsigned>(a->n_splits), static_cast<unsigned>(a->heads_kv),
                    static_cast<unsigned>(a->batch));
    const bool bf = a->q_dtype == NSN_DTYPE_BF16;
    if (G < 1 || G > 8) return NSN_EINVAL;
#define NSN_FAST_LAUNCH1(B_, Q_, S_, G_) hipLaunchKernelGGL((attn_fast_kernel<B_, Q_, S_, G_>), grid, dim3(64), 0, st, p)
#define NSN_FAST_LAUNCH(B_, Q_, S_)                                   \
    do {                                                              \
        if (G == 1) NSN_FAST_LAUNCH1(B_, Q_, S_, 1);                  \
        else if (G == 2) NSN_FAST_LAUNCH1(B_, Q_, S_, 2);             \
        else if (G <= 4) NSN_FAST_LAUNCH1(B_, Q_, S_, 4);             \
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
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

}  // namespace nsn
