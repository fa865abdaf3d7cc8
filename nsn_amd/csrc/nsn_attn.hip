// Single-query decode attention over NSN-packed K/V for gfx950.
//
// Work unit = (sequence b, kv-head, context split).  Each unit serves all
// G = Hq/Hkv query heads of its kv-head, so every packed block is read and
// reconstructed once per kv-head (the reference's GQA kernel reconstructs it
// once per query head, experiments/nb06/source/loop_kv_nb06_kernel.py:56).
// Each unit writes per-head softmax partials (running max, sum, weighted V);
// a merge kernel combines the splits (log-sum-exp), as the reference's AF01
// merge does (experiments/ac08/source/loop_kv_af01_kernel.py:70-82).
//
// This file holds the exact-order ("reference") kernel: K and V tiles are
// reconstructed with nsn_decode's arithmetic (loop_kv_pilot.py:216-225),
// rounded to the attention dtype as the reference's read_v does
// (loop_kv_vf01_kernel.py:34), and QK / softmax / PV run in fp32 with
// unfused multiply-add.  Because a restored tile and the same values read
// back from HBM go through identical arithmetic, the bridge route (restore V
// to HBM, then attend) and the fused route give bitwise-equal outputs -- the
// reference's route-equality property (AC/verify_loop_kv_vf01.py:41-50).
#include <mutex>

#include "nsn_common.hpp"

namespace nsn {

constexpr int kPartStride = 132;  // floats per (b, hq, split) partial: m, l, pad, pad, acc[128]
constexpr int kMaxGroup = 16;

struct SideParams {
    const uint8_t *codes;
    const uint16_t *norms, *mins, *scales;
    const int32_t *blocks;
    int64_t block_cap;
    const void *tail;
    int64_t tail_cap;
};

struct AttnParams {
    const void *q;
    int64_t heads_q, heads_kv;
    int group;
    float scale;
    const int32_t *seq_len;
    int64_t batch;
    int split_tokens, n_splits;
    SideParams k, v;
    const float *scores;
    int64_t scores_cap;
    float *partials;
    int32_t *status;
    float *trace_scores, *trace_v;   // nullable: the kernel's own scores and V rows
    int64_t trace_cap;
};

template <int DT>
__device__ __forceinline__ float load_elem(const void *base, int64_t idx) {
    return Elem<DT>::load(static_cast<const typename Elem<DT>::T *>(base)[idx]);
}

// Flags returned by the tile loaders.
constexpr int kBadRestore = 1;   // a reconstructed value is nonfinite
constexpr int kBadInput = 2;     // a raw input (block metadata, tail token) is nonfinite

// Reconstruct packed block `blk` of row `row` (= b*Hkv + kvh) into tile[64][kXP]
// as fp32 values already rounded to RDT.  Returns kBad* flags.
template <int BITS, int RDT>
__device__ int restore_tile(const SideParams &sd, int64_t row, int64_t blk, float *tile, uint32_t *codes_s,
                             float *m_s, float *s_s, float *n_s, double *rden_s) {
    constexpr int kXP = kDim + 4;
    const int tid = threadIdx.x;
    const int64_t ib = row * sd.block_cap + blk;
    bool bad_in = false;   // the grouped finite check of the metadata, fused here
    if (tid < kDim) {
        m_s[tid] = f16_bits_to_f32(sd.mins[ib * kDim + tid]);
        s_s[tid] = f16_bits_to_f32(sd.scales[ib * kDim + tid]);
        bad_in = !finite(m_s[tid]) || !finite(s_s[tid]);
    } else if (tid < kDim + kBlockTok) {
        n_s[tid - kDim] = f16_bits_to_f32(sd.norms[ib * kBlockTok + tid - kDim]);
        bad_in = !finite(n_s[tid - kDim]);
    }
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(sd.codes + ib * packed_block_bytes(BITS)) + tid * BITS;
        uint32_t w[BITS];
#pragma unroll
        for (int k = 0; k < BITS; ++k) w[k] = src[k];
        constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 4 * k + e, pos = i * BITS, d = pos >> 5, sh = pos & 31;
                uint32_t v = w[d] >> sh;
                if (sh + BITS > 32) v |= w[d + 1] << (32 - sh);
                word |= (v & mask) << (8 * e);
            }
            codes_s[tid * 8 + k] = word;
        }
    }
    __syncthreads();
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
    bool bad = false;
    const int cg = tid & 15, r0 = tid >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + 16 * j;
        const uint8_t *cr = reinterpret_cast<const uint8_t *>(codes_s) + r * kDim;
        const float n = n_s[r];
        const double rd = rden_s[r];
        float *dst = tile + r * kXP + 8 * cg;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int c = 8 * cg + e;
            const float prod = s_s[c] * static_cast<float>(cr[c]);
            const float d = m_s[c] + prod;
            const float val = n * div_by_recip(d, rd);
            float y = (n == 0.f) ? 0.f : val;
            y = Elem<RDT>::load(Elem<RDT>::store(y));
            bad |= !finite(y);
            dst[e] = y;
        }
    }
    return (bad ? kBadRestore : 0) | (bad_in ? kBadInput : 0);
}

// Dense tile: tokens [t0, t0 + valid) of the tail buffer row, zero beyond.
// A nonfinite tail token is a raw-input failure.
template <int TDT>
__device__ int dense_tile(const SideParams &sd, int64_t row, int64_t t0, int valid, float *tile) {
    constexpr int kXP = kDim + 4;
    const int tid = threadIdx.x;
    const int cg = tid & 15, r0 = tid >> 4;
    bool bad = false;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int r = r0 + 16 * j;
        float *dst = tile + r * kXP + 8 * cg;
        if (r < valid) {
            const int64_t base = (row * sd.tail_cap + t0 + r) * kDim + 8 * cg;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                dst[e] = load_elem<TDT>(sd.tail, base + e);
                bad |= !finite(dst[e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) dst[e] = 0.f;
        }
    }
    return bad ? kBadInput : 0;
}

template <int BITS, int RDT, int TDT>
__device__ int load_tile(const SideParams &sd, int64_t row, int b, int64_t t0, int valid, float *tile,
                          uint32_t *codes_s, float *m_s, float *s_s, float *n_s, double *rden_s) {
    const int64_t nb = sd.blocks ? sd.blocks[b] : 0;
    if (t0 < nb * kBlockTok)
        return restore_tile<BITS, RDT>(sd, row, t0 / kBlockTok, tile, codes_s, m_s, s_s, n_s, rden_s);
    return dense_tile<TDT>(sd, row, t0 - nb * kBlockTok, valid, tile);
}

template <int BITS, int QDT, int RDT, int TDT, bool SCORES>
__global__ __launch_bounds__(256) void attn_reference_kernel(AttnParams p) {
    constexpr int kXP = kDim + 4;
    __shared__ float tile[kBlockTok * kXP];
    __shared__ uint32_t codes_s[kBlockTok * kDim / 4];
    __shared__ float m_s[kDim], s_s[kDim], n_s[kBlockTok];
    __shared__ double rden_s[kBlockTok];
    __shared__ float q_s[kMaxGroup * kDim];
    __shared__ float sc_s[kMaxGroup * kBlockTok];
    __shared__ float run_m[kMaxGroup], run_l[kMaxGroup], alpha_s[kMaxGroup];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int G = p.group;
    const int64_t row = static_cast<int64_t>(b) * p.heads_kv + kvh;
    // The usable length.  One whose blocks or tail lie past the cache's
    // capacity, or past the splits' reach, is possible only with the host
    // checks skipped (device lengths): nothing of that sequence is read, the
    // status word says why, and the merge sees a partial count of 0.
    int64_t T = p.seq_len[b];
    {
        auto fits = [&](const SideParams &sd) {
            const int64_t nb = sd.blocks ? sd.blocks[b] : 0;
            if (nb < 0 || nb > (sd.blocks ? sd.block_cap : 0)) return false;
            const int64_t rest = T - nb * kBlockTok;
            return rest <= 0 || (sd.tail != nullptr && rest <= sd.tail_cap);
        };
        const bool cap_ok = T >= 0 && (SCORES ? T <= p.scores_cap : fits(p.k)) && fits(p.v);
        const bool ws_ok = T <= static_cast<int64_t>(p.n_splits) * p.split_tokens;
        if (!cap_ok || !ws_ok) {
            if (tid == 0 && split == 0 && kvh == 0)
                raise_status(p.status, !cap_ok ? NSN_ST_CAPACITY : NSN_ST_WORKSPACE);
            T = 0;
        }
    }
    const int64_t t_begin = static_cast<int64_t>(split) * p.split_tokens;
    const int64_t t_end = t_begin + p.split_tokens < T ? t_begin + p.split_tokens : T;
    const int64_t hq0 = static_cast<int64_t>(kvh) * G;

    // thread -> accumulator slots: heads wave, wave+4, ...; channels 2*lane, 2*lane+1
    float acc[kMaxGroup / 4][2];
#pragma unroll
    for (int k = 0; k < kMaxGroup / 4; ++k) acc[k][0] = acc[k][1] = 0.f;

    bool bad_in = false;   // raw inputs: q, block metadata, tail tokens (the fused finite check)
    for (int i = tid; i < G * kDim; i += 256) {
        const int h = i / kDim, c = i - h * kDim;
        q_s[i] = load_elem<QDT>(p.q, (static_cast<int64_t>(b) * p.heads_q + hq0 + h) * kDim + c);
        bad_in |= !finite(q_s[i]);
    }
    if (tid < G) { run_m[tid] = -INFINITY; run_l[tid] = 0.f; }
    bool bad_attn = false, bad_restore = false;
    __syncthreads();

    for (int64_t t0 = t_begin; t0 < t_end; t0 += kBlockTok) {
        const int valid = static_cast<int>(t_end - t0 < kBlockTok ? t_end - t0 : kBlockTok);
        // ---- scores [G][64] ----
        if constexpr (SCORES) {
            for (int i = tid; i < G * kBlockTok; i += 256) {
                const int h = i / kBlockTok, t = i - h * kBlockTok;
                float s = -INFINITY;
                if (t < valid) {
                    s = p.scores[(static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.scores_cap + t0 + t];
                    bad_attn |= !finite(s);
                    if (p.trace_scores && t0 + t < p.trace_cap)
                        p.trace_scores[(static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.trace_cap + t0 + t] = s;
                }
                sc_s[i] = s;
            }
        } else {
            const int fl = load_tile<BITS, RDT, TDT>(p.k, row, b, t0, valid, tile, codes_s, m_s, s_s, n_s, rden_s);
            bad_restore |= (fl & kBadRestore) != 0;
            bad_in |= (fl & kBadInput) != 0;
            __syncthreads();
            const int r = tid >> 2, qq = tid & 3;
            for (int h = 0; h < G; ++h) {
                float part = 0.f;
                const float *kr = tile + r * kXP + 32 * qq;
                const float *qh = q_s + h * kDim + 32 * qq;
#pragma unroll 8
                for (int c = 0; c < 32; ++c) {
                    const float prod = kr[c] * qh[c];
                    part = part + prod;
                }
                const float o1 = __shfl_down(part, 1), o2 = __shfl_down(part, 2), o3 = __shfl_down(part, 3);
                if (qq == 0) {
                    float s = ((part + o1) + o2) + o3;
                    s = s * p.scale;
                    if (r < valid) bad_attn |= !finite(s);
                    if (r < valid && p.trace_scores && t0 + r < p.trace_cap)
                        p.trace_scores[(static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.trace_cap + t0 + r] = s;
                    sc_s[h * kBlockTok + r] = (r < valid) ? s : -INFINITY;
                }
            }
        }
        __syncthreads();
        // ---- online softmax per head: wave w handles heads w, w+4, ... ----
        for (int h = wave; h < G; h += 4) {
            const float s = sc_s[h * kBlockTok + lane];
            float mx = s;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                const float o = __shfl_xor(mx, off);
                mx = o > mx ? o : mx;
            }
            const float m_old = run_m[h];
            const float m_new = m_old > mx ? m_old : mx;
            const float pw = (lane < valid) ? expf(s - m_new) : 0.f;
            float sum = pw;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) sum = sum + __shfl_xor(sum, off);
            sc_s[h * kBlockTok + lane] = pw;
            if (lane == 0) {
                const float alpha = (m_old == -INFINITY) ? 0.f : expf(m_old - m_new);
                alpha_s[h] = alpha;
                run_m[h] = m_new;
                run_l[h] = run_l[h] * alpha + sum;
                if (!finite(sum) || !finite(m_new)) bad_attn = true;
            }
        }
        __syncthreads();
        // ---- V tile and P.V ----
        {
            const int fl = load_tile<BITS, RDT, TDT>(p.v, row, b, t0, valid, tile, codes_s, m_s, s_s, n_s, rden_s);
            bad_restore |= (fl & kBadRestore) != 0;
            bad_in |= (fl & kBadInput) != 0;
        }
        __syncthreads();
        if (p.trace_v)   // the V rows this block multiplies (row = b * Hkv + kv-head)
            for (int i = tid; i < valid * kDim; i += 256) {
                const int t = i / kDim, c = i - t * kDim;
                if (t0 + t < p.trace_cap) p.trace_v[(row * p.trace_cap + t0 + t) * kDim + c] = tile[t * kXP + c];
            }
#pragma unroll
        for (int k = 0; k < kMaxGroup / 4; ++k) {
            const int h = wave + 4 * k;
            if (h < G) {
                const float alpha = alpha_s[h];
                float a0 = acc[k][0] * alpha, a1 = acc[k][1] * alpha;
                const float *ph = sc_s + h * kBlockTok;
                for (int t = 0; t < valid; ++t) {
                    const float w = ph[t];
                    const float2 vv = *reinterpret_cast<const float2 *>(tile + t * kXP + 2 * lane);
                    const float p0 = w * vv.x, p1 = w * vv.y;
                    a0 = a0 + p0;
                    a1 = a1 + p1;
                }
                acc[k][0] = a0;
                acc[k][1] = a1;
            }
        }
        __syncthreads();
    }

    // ---- partials ----
#pragma unroll
    for (int k = 0; k < kMaxGroup / 4; ++k) {
        const int h = wave + 4 * k;
        if (h < G) {
            float *dst = p.partials + ((static_cast<int64_t>(b) * p.heads_q + hq0 + h) * p.n_splits + split) * kPartStride;
            if (lane == 0) {
                dst[0] = run_m[h]; dst[1] = run_l[h]; dst[2] = 0.f; dst[3] = 0.f;
                if (split == 0)   // every split writes a slot: the merge reads all n_splits (none: no token)
                    reinterpret_cast<int32_t *>(p.partials + p.batch * p.heads_q * p.n_splits * kPartStride)
                        [static_cast<int64_t>(b) * p.heads_q + hq0 + h] = (T > 0) ? p.n_splits : 0;
            }
            *reinterpret_cast<float2 *>(dst + 4 + 2 * lane) = make_float2(acc[k][0], acc[k][1]);
            bad_attn |= !finite(acc[k][0]) || !finite(acc[k][1]);
        }
    }
    int st = (bad_attn ? NSN_ST_NONFINITE_ATTN : 0) | (bad_restore ? NSN_ST_NONFINITE_RESTORE : 0) |
             (bad_in ? NSN_ST_NONFINITE_ATTN_INPUT : 0);
    if (__any(st != 0)) {
        if (st) raise_status(p.status, st);
    }
}

// Merge splits: one 256-thread block (4 waves) per (b, hq).  Wave w sums
// splits w, w+4, ... (all its loads in flight together), lane c owns channels
// 2c, 2c+1; the four wave partials are combined in LDS.
constexpr int kMergeSlots = 16;   // partial slots per wave the merge holds in registers (64 per (b, hq))
template <int ODT>
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *partials, const int32_t *counts, int n_splits,
                                                         float *ctx, void *out, int32_t *status) {
    __shared__ float red_m[4], red_z[4];
    __shared__ float2 red_u[4][64];
    const int64_t bh = blockIdx.x;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const float *base = partials + bh * n_splits * kPartStride;
    // partial slots written for this (b, hq): both decode kernels write the
    // count, 0 for a (b, hq) that attended no token -- zero output, flagged
    int used = counts[bh];
    if (used <= 0) {   // (uniform across the block)
        if (w == 0) {
            const int64_t c = bh * kDim + 2 * lane;
            if (ctx) ctx[c] = ctx[c + 1] = 0.f;
            static_cast<typename Elem<ODT>::T *>(out)[c] = Elem<ODT>::store(0.f);
            static_cast<typename Elem<ODT>::T *>(out)[c + 1] = Elem<ODT>::store(0.f);
            if (lane == 0) raise_status(status, NSN_ST_EMPTY);
        }
        return;
    }
    used = used > n_splits ? n_splits : used;   // (in bounds whatever the count)
    n_splits = used;
    float z = 0.f, u0 = 0.f, u1 = 0.f;
    if (n_splits <= 4 * kMergeSlots) {
        // Wave w's slots w, w+4, ... all loaded at once (one round trip after
        // the count), the maximum exchanged through LDS; then the same sums
        // in the same order as the loop below.
        float pm[kMergeSlots], pz[kMergeSlots];
        float2 pu[kMergeSlots];
#pragma unroll
        for (int i = 0; i < kMergeSlots; ++i) {
            const int s = w + 4 * i;
            pm[i] = -INFINITY;
            pz[i] = 0.f;
            pu[i] = make_float2(0.f, 0.f);
            if (s < n_splits) {
                const float *ps = base + static_cast<int64_t>(s) * kPartStride;
                pm[i] = ps[0];
                pz[i] = ps[1];
                pu[i] = *reinterpret_cast<const float2 *>(ps + 4 + 2 * lane);
            }
        }
        float lw = -INFINITY;
#pragma unroll
        for (int i = 0; i < kMergeSlots; ++i) lw = fmaxf(lw, pm[i]);
        if (lane == 0) red_m[w] = lw;
        __syncthreads();
        const float L = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
#pragma unroll
        for (int i = 0; i < kMergeSlots; ++i) {
            if (w + 4 * i < n_splits) {
                const float a = (pm[i] == -INFINITY) ? 0.f : expf(pm[i] - L);
                z = z + pz[i] * a;
                u0 = u0 + pu[i].x * a;
                u1 = u1 + pu[i].y * a;
            }
        }
    } else {
        float L = -INFINITY;
        for (int s = lane; s < n_splits; s += 64) L = fmaxf(L, base[static_cast<int64_t>(s) * kPartStride]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) L = fmaxf(L, __shfl_xor(L, off));
#pragma unroll 4
        for (int s = w; s < n_splits; s += 4) {
            const float *ps = base + static_cast<int64_t>(s) * kPartStride;
            const float m = ps[0];
            const float a = (m == -INFINITY) ? 0.f : expf(m - L);
            z = z + ps[1] * a;
            const float2 u = *reinterpret_cast<const float2 *>(ps + 4 + 2 * lane);
            u0 = u0 + u.x * a;
            u1 = u1 + u.y * a;
        }
    }
    if (lane == 0) red_z[w] = z;
    red_u[w][lane] = make_float2(u0, u1);
    __syncthreads();
    if (w != 0) return;
    const float den = (red_z[0] + red_z[1]) + (red_z[2] + red_z[3]);
    const float n0 = (red_u[0][lane].x + red_u[1][lane].x) + (red_u[2][lane].x + red_u[3][lane].x);
    const float n1 = (red_u[0][lane].y + red_u[1][lane].y) + (red_u[2][lane].y + red_u[3][lane].y);
    const float cx0 = n0 / den, cx1 = n1 / den;
    const typename Elem<ODT>::T o0 = Elem<ODT>::store(cx0), o1 = Elem<ODT>::store(cx1);
    const int64_t c = bh * kDim + 2 * lane;
    if (ctx) {
        ctx[c] = cx0;
        ctx[c + 1] = cx1;
    }
    static_cast<typename Elem<ODT>::T *>(out)[c] = o0;
    static_cast<typename Elem<ODT>::T *>(out)[c + 1] = o1;
    const bool bad = !finite(cx0) || !finite(cx1) || !finite(Elem<ODT>::load(o0)) || !finite(Elem<ODT>::load(o1)) ||
                     !(den > 0.f);
    if (bad) raise_status(status, NSN_ST_NONFINITE_OUTPUT);
}

}  // namespace nsn

using namespace nsn;

namespace {

bool side_ok(const nsn_kv_side &s, int bits) {
    (void)bits;
    if (s.blocks && (!s.codes || !s.norms || !s.mins || !s.scales)) return false;
    if (s.codes && (reinterpret_cast<uintptr_t>(s.codes) & 15u)) return false;
    return true;
}

SideParams to_side(const nsn_kv_side &s) {
    return SideParams{s.codes, s.norms, s.mins, s.scales, s.blocks, s.block_cap, s.tail, s.tail_cap};
}

template <int BITS, int QDT, int RDT, int TDT>
int launch_reference_scores(bool scores, dim3 grid, hipStream_t st, const AttnParams &p) {
    if (scores) hipLaunchKernelGGL((attn_reference_kernel<BITS, QDT, RDT, TDT, true>), grid, dim3(256), 0, st, p);
    else hipLaunchKernelGGL((attn_reference_kernel<BITS, QDT, RDT, TDT, false>), grid, dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

template <int BITS, int QDT, int RDT>
int dispatch_tail(int tdt, bool scores, dim3 grid, hipStream_t st, const AttnParams &p) {
    if (tdt == NSN_DTYPE_F16) return launch_reference_scores<BITS, QDT, RDT, NSN_DTYPE_F16>(scores, grid, st, p);
    if (tdt == NSN_DTYPE_BF16) return launch_reference_scores<BITS, QDT, RDT, NSN_DTYPE_BF16>(scores, grid, st, p);
    return NSN_EINVAL;
}

template <int BITS, int QDT>
int dispatch_round(int rdt, int tdt, bool scores, dim3 grid, hipStream_t st, const AttnParams &p) {
    if (rdt == NSN_DTYPE_F16) return dispatch_tail<BITS, QDT, NSN_DTYPE_F16>(tdt, scores, grid, st, p);
    if (rdt == NSN_DTYPE_BF16) return dispatch_tail<BITS, QDT, NSN_DTYPE_BF16>(tdt, scores, grid, st, p);
    return dispatch_tail<BITS, QDT, NSN_DTYPE_F32>(tdt, scores, grid, st, p);
}

template <int BITS>
int dispatch_q(int qdt, int rdt, int tdt, bool scores, dim3 grid, hipStream_t st, const AttnParams &p) {
    if (qdt == NSN_DTYPE_BF16) return dispatch_round<BITS, NSN_DTYPE_BF16>(rdt, tdt, scores, grid, st, p);
    if (qdt == NSN_DTYPE_F16) return dispatch_round<BITS, NSN_DTYPE_F16>(rdt, tdt, scores, grid, st, p);
    return dispatch_round<BITS, NSN_DTYPE_F32>(rdt, tdt, scores, grid, st, p);
}

}  // namespace

extern "C" {

int64_t nsn_attention_workspace_floats(int64_t batch, int64_t heads_q, int n_splits) {
    // partials, then one int32 partial count per (b, hq)
    return batch * heads_q * (static_cast<int64_t>(n_splits) * kPartStride + 1);
}

int nsn_decode_attention(const nsn_attn_args *a, nsn_stream_t stream) {
    if (!a) return NSN_EINVAL;
    if (a->batch <= 0 || a->heads_kv <= 0 || a->heads_q <= 0 || a->heads_q % a->heads_kv) return NSN_EINVAL;
    const int64_t G = a->heads_q / a->heads_kv;
    if (G > kMaxGroup) return NSN_EINVAL;
    if (a->bits != 3 && a->bits != 4 && a->bits != 5) return NSN_EINVAL;
    if (!a->q || !a->seq_len || !a->partials || !a->out) return NSN_EINVAL;
    if (a->split_tokens <= 0 || a->split_tokens % kBlockTok || a->n_splits <= 0) return NSN_EINVAL;
    if (static_cast<int64_t>(a->n_splits) * a->split_tokens < a->max_seq_len) return NSN_EINVAL;
    const bool scores = a->k_mode == NSN_KV_SCORES;
    if (!scores && a->k_mode != NSN_KV_PACKED) return NSN_EINVAL;
    if (scores && !a->scores) return NSN_EINVAL;
    if (!scores && (!side_ok(a->k, a->bits) || a->k.tail_dtype != a->v.tail_dtype)) return NSN_EINVAL;
    if (!side_ok(a->v, a->bits)) return NSN_EINVAL;
    if (a->out_dtype != NSN_DTYPE_BF16 && a->out_dtype != NSN_DTYPE_F16 && a->out_dtype != NSN_DTYPE_F32) return NSN_EINVAL;
    if (a->batch > 65535 || a->heads_kv > 65535) return NSN_EINVAL;

    AttnParams p{};
    p.q = a->q;
    p.heads_q = a->heads_q;
    p.heads_kv = a->heads_kv;
    p.group = static_cast<int>(G);
    p.scale = a->scale;
    p.seq_len = a->seq_len;
    p.split_tokens = a->split_tokens;
    p.batch = a->batch;
    p.n_splits = a->n_splits;
    p.k = to_side(a->k);
    p.v = to_side(a->v);
    p.scores = a->scores;
    p.scores_cap = a->scores_cap;
    p.partials = a->partials;
    p.status = a->status;
    const bool trace = a->trace_scores || a->trace_v;
    if (trace && (a->kernel != NSN_ATTN_REFERENCE || a->trace_cap < a->max_seq_len)) return NSN_EINVAL;
    p.trace_scores = a->trace_scores;
    p.trace_v = a->trace_v;
    p.trace_cap = a->trace_cap;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(a->n_splits), static_cast<unsigned>(a->heads_kv),
                    static_cast<unsigned>(a->batch));
    int rc;
    if (a->kernel == NSN_ATTN_FAST) {
        rc = launch_attn_fast(a, st);
        if (rc != NSN_OK) return rc;
        if (!a->merge) return NSN_OK;
        return nsn_attention_merge(a->partials, a->batch, a->heads_q, a->n_splits, a->ctx, a->out, a->out_dtype,
                                   a->status, stream);
    }
    if (a->kernel != NSN_ATTN_REFERENCE) return NSN_EINVAL;
    if (a->bits == 3) rc = dispatch_q<3>(a->q_dtype, a->kv_round_dtype, a->v.tail_dtype, scores, grid, st, p);
    else if (a->bits == 4) rc = dispatch_q<4>(a->q_dtype, a->kv_round_dtype, a->v.tail_dtype, scores, grid, st, p);
    else rc = dispatch_q<5>(a->q_dtype, a->kv_round_dtype, a->v.tail_dtype, scores, grid, st, p);
    if (rc != NSN_OK) return rc;
    if (!a->merge) return NSN_OK;
    return nsn_attention_merge(a->partials, a->batch, a->heads_q, a->n_splits, a->ctx, a->out, a->out_dtype,
                               a->status, stream);
}

int nsn_attention_merge(const float *partials, int64_t batch, int64_t heads_q, int n_splits, float *ctx, void *out,
                        int out_dtype, int32_t *status, nsn_stream_t stream) {
    if (!partials || !out || batch <= 0 || heads_q <= 0 || n_splits <= 0) return NSN_EINVAL;
    if (batch * heads_q > 0x7fffffff) return NSN_EINVAL;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const dim3 mgrid(static_cast<unsigned>(batch * heads_q));
    const int32_t *counts = reinterpret_cast<const int32_t *>(partials + batch * heads_q * n_splits * kPartStride);
    if (out_dtype == NSN_DTYPE_BF16)
        hipLaunchKernelGGL(attn_merge_kernel<NSN_DTYPE_BF16>, mgrid, dim3(256), 0, st, partials, counts, n_splits, ctx, out, status);
    else if (out_dtype == NSN_DTYPE_F16)
        hipLaunchKernelGGL(attn_merge_kernel<NSN_DTYPE_F16>, mgrid, dim3(256), 0, st, partials, counts, n_splits, ctx, out, status);
    else if (out_dtype == NSN_DTYPE_F32)
        hipLaunchKernelGGL(attn_merge_kernel<NSN_DTYPE_F32>, mgrid, dim3(256), 0, st, partials, counts, n_splits, ctx, out, status);
    else
        return NSN_EINVAL;
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free decode attention: the partials workspace is a file-scope
// device array instead of caller memory.  Each device holds its own copy; its
// address is looked up once per device (with that device current) and used
// for every launch -- the array's name is a host-side stand-in and is never
// passed to a kernel.
static __device__ __align__(256) float scratch[NSN_STATIC_SCRATCH_FLOATS];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float *g_scratch[kMaxDevices] = {};

int scratch_ptr(float **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return NSN_ELAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return NSN_ELAUNCH;
        g_scratch[dev] = static_cast<float *>(ptr);
    }
    *out = g_scratch[dev];
    return NSN_OK;
}
}  // namespace

extern "C" int nsn_decode_attention_static(const nsn_attn_args *a, nsn_stream_t stream) {
    if (!a || a->batch <= 0 || a->heads_q <= 0 || a->n_splits <= 0) return NSN_EINVAL;
    if (nsn_attention_workspace_floats(a->batch, a->heads_q, a->n_splits) > NSN_STATIC_SCRATCH_FLOATS)
        return NSN_ENOSPC;
    float *ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc != NSN_OK) return rc;
    nsn_attn_args b = *a;
    b.partials = ws;
    return nsn_decode_attention(&b, stream);
}

