// K-score decode kernel for gfx950: one decode query per sequence against a
// quantised K cache, scores only (the K side of attention, where the KIVI and
// NSN recipes differ).  Replaces the reference's fused dequant-then-score
// kernel, experiments/kernels/phase_k1c_triton_fused_kernel.py:207-249
// (`_fused_score_kernel`) and its launcher `triton_decode_scores` (:252-281).
//
//   score[b, h, t] = scale * en[b, hkv, t] * sum_d q[b, h, d] * (code[b, t, hkv*D + d] * step[b, hkv*D + d]
//                                                                + min[b, hkv*D + d])
//   hkv = h / (Hq / Hkv)      (GQA); en = 1 for KIVI; code * step + min -> K itself for fp16.
//
// The per-channel step and min factor out of the token loop:
//   score = scale * en_t * (sum_d W[h, d] z[t, d] + c0[h]),  W = q * step,  c0 = q . min
// so the token loop is a [2G x D] x [D x 16 tokens] product per tile on
// v_mfma_f32_16x16x32_f16.  The codes enter as fp16 subnormals z * 2^-24
// (exact); the A rows hold W * 2^sigma split into fp16 hi (toward zero) + lo
// (~22 significant bits); sigma puts max|W| in [2^13, 2^14).  For fp16 K the A
// rows are q itself (exact) and B the K values.
//
// Storage (the reference's K1c layout): codes u8 [B, T, Hkv*D] -- or the same
// codes bit-packed LSB-first along each token row, [B, T, Hkv*D*bits/8] --
// min / step fp16 [B, Hkv*D], en fp16 [B, Hkv, T], q fp16 [B, Hq, D], scores
// fp32 [B, Hq, T].
//
// Work: one wave per (sequence, kv-head, chunk of 16-token tiles); lane l
// owns token column l % 16 and the contiguous channel block g*D/4 .. of lane
// group g = l / 16 (the MFMA k order is permuted to match, in A and B alike),
// so each lane reads D/4 consecutive codes of its token per tile.  Four tiles
// are in flight per wave; the kv-heads of one chunk are consecutive waves.
#include "nsn_common.hpp"
#include "nsn_unpack.hpp"

namespace nsn {
namespace ks {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum { MODE_U8 = 0, MODE_PACKED = 1, MODE_FP16 = 2 };

struct KsParams {
    const uint16_t *q;
    int64_t batch, heads_q, heads_kv, T;
    int group;
    const uint8_t *codes;
    int64_t row_bytes;    // bytes per token row (all kv-heads)
    const uint16_t *mins, *steps, *en;
    float scale;
    float *out;
    int64_t chunk_tiles;  // 16-token tiles per wave
    int64_t n_chunks;     // chunks per (sequence, kv-head) stream
};

__device__ __forceinline__ f32x4 mfma(const u32x4 &a, const u32x4 &b, const f32x4 &c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pkrtz(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ float h2f(uint16_t h) { return f16_bits_to_f32(h); }

template <int D, int MODE, int BITS>
struct Shape {
    static constexpr int CPL = D / 4;                                   // channels per lane
    static constexpr int NK = D / 32;                                   // MFMA k-steps
    static constexpr int LANE_BYTES = MODE == MODE_FP16 ? 2 * CPL : (MODE == MODE_U8 ? CPL : CPL * BITS / 8);
    static constexpr int NW = LANE_BYTES / 4;                           // code dwords per lane per tile
    static constexpr int PF = NW <= 16 ? 4 : 2;                         // tiles in flight
};

template <int D, int MODE, int BITS>
struct Tile {
    uint32_t w[Shape<D, MODE, BITS>::NW];
    uint32_t en;   // fp16 bits of en[t] (NSN)
};

// Element order of a K-step's B operand: element e holds channel 8kk + ch(e)
// of the lane's block, at bit k(e) of its half (identity and 0 for u8 codes
// and fp16 K; the unpack's windows for bit-packed codes).
template <int MODE, int BITS, bool PACKED = (MODE == MODE_PACKED)>
struct Elems {
    static constexpr int ch(int e) { return e; }
    static constexpr int k(int) { return 0; }
};
template <int MODE, int BITS>
struct Elems<MODE, BITS, true> {
    static constexpr int ch(int e) { return unpack::Layout<BITS>::chE[e]; }
    static constexpr int k(int e) { return unpack::Layout<BITS>::kE[e]; }
};

// B operands (NK k-steps) of one tile from the lane's raw code dwords.
template <int D, int MODE, int BITS>
__device__ __forceinline__ void b_frags(const Tile<D, MODE, BITS> &r, u32x4 (&B)[Shape<D, MODE, BITS>::NK]) {
    constexpr int NK = Shape<D, MODE, BITS>::NK;
    if constexpr (MODE == MODE_FP16) {
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) B[kk] = u32x4{r.w[4 * kk], r.w[4 * kk + 1], r.w[4 * kk + 2], r.w[4 * kk + 3]};
    } else if constexpr (MODE == MODE_U8) {
        // bytes b0..b7 of a k-step -> halves (b0, b1), (b2, b3), ...: each code an fp16 subnormal z * 2^-24
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) {
            const uint32_t x = r.w[2 * kk], y = r.w[2 * kk + 1];
            B[kk] = u32x4{__builtin_amdgcn_perm(x, x, 0x0C010C00u), __builtin_amdgcn_perm(x, x, 0x0C030C02u),
                          __builtin_amdgcn_perm(y, y, 0x0C010C00u), __builtin_amdgcn_perm(y, y, 0x0C030C02u)};
        }
    } else {
        // 32 codes per BITS dwords: byte windows and one AND per pair of codes
#pragma unroll
        for (int g = 0; g < NK / 4; ++g) {
            uint32_t u[BITS];
#pragma unroll
            for (int k = 0; k < BITS; ++k) u[k] = r.w[g * BITS + k];
            u32x4 Bg[4];
            unpack::kunpack(u, Bg);
#pragma unroll
            for (int k = 0; k < 4; ++k) B[4 * g + k] = Bg[k];
        }
    }
}

template <int D, int MODE, int BITS, bool NSN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 128 ? 4 : 2))) void kscore_kernel(KsParams p) {
    using SH = Shape<D, MODE, BITS>;
    constexpr int CPL = SH::CPL, NK = SH::NK, NW = SH::NW, PF = SH::PF;
    const int l = threadIdx.x & 63;
    // wave -> (sequence, chunk, kv-head), kv-head fastest: the waves of one
    // chunk read the same token rows, each its kv-head's slice, together whole rows
    const int64_t wid = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t sc = wid / p.heads_kv;
    const int hkv = static_cast<int>(wid - sc * p.heads_kv);
    const int64_t b = sc / p.n_chunks, chunk = sc - b * p.n_chunks;
    if (b >= p.batch) return;   // (whole wave)
    const int G = p.group;
    const int row = l & 15, grp = l >> 4;
    const int64_t T = p.T;
    const int64_t ntiles_all = (T + 15) / 16;
    const int64_t it0 = chunk * p.chunk_tiles;
    const int64_t it1 = (it0 + p.chunk_tiles < ntiles_all) ? it0 + p.chunk_tiles : ntiles_all;
    if (it0 >= it1) return;

    // ---- A rows: row 2h + part holds head h's W * 2^sigma, hi (part 0) or lo (part 1)
    const int h_a = row >> 1, part = row & 1;
    const bool arow = h_a < G && (MODE != MODE_FP16 || part == 0);
    const int64_t hq0 = static_cast<int64_t>(hkv) * G;
    const int ch0 = grp * CPL;   // the lane's channel block
    float wv[CPL];
    float mx = 0.f, c0p = 0.f;
    const uint16_t *qrow = p.q + ((b * p.heads_q + hq0 + (h_a < G ? h_a : 0)) * D);
    const int64_t cbase = b * p.heads_kv * D + static_cast<int64_t>(hkv) * D;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const float qv = (h_a < G) ? h2f(qrow[ch0 + i]) : 0.f;
        float w = qv;
        if constexpr (MODE != MODE_FP16) {
            w = qv * h2f(p.steps[cbase + ch0 + i]);
            c0p = __builtin_fmaf(qv, h2f(p.mins[cbase + ch0 + i]), c0p);
        }
        wv[i] = w;
        mx = fmaxf(mx, fabsf(w));
    }
    // the row's maximum and the min term over all D channels (the 4 lane groups)
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    c0p += __shfl_xor(c0p, 16);
    c0p += __shfl_xor(c0p, 32);
    int sigma = 0;
    if constexpr (MODE != MODE_FP16) {
        int e2 = 0;
        (void)frexpf(mx, &e2);
        sigma = (mx > 0.f && finite(mx)) ? 14 - e2 : 0;
        sigma = sigma < -100 ? -100 : (sigma > 100 ? 100 : sigma);
    }
    u32x4 A[NK];
    {
        const float pw = ldexpf(1.f, sigma);
        using EL = Elems<MODE, BITS>;
#pragma unroll
        for (int kk = 0; kk < NK; ++kk)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // (the code of element e sits at bit k(e): its coefficient carries 2^-k(e))
                const float a = wv[8 * kk + EL::ch(2 * j)] * ldexpf(pw, -EL::k(2 * j));
                const float c = wv[8 * kk + EL::ch(2 * j + 1)] * ldexpf(pw, -EL::k(2 * j + 1));
                uint32_t v;
                if constexpr (MODE == MODE_FP16) {
                    v = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, c));   // q is fp16: exact
                } else {
                    const uint32_t hi = pkrtz(a, c);
                    const float ah = static_cast<float>(__builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), hi)[0]);
                    const float ch = static_cast<float>(__builtin_bit_cast(__fp16 __attribute__((ext_vector_type(2))), hi)[1]);
                    v = part ? pkrtz(a - ah, c - ch) : hi;
                }
                A[kk][j] = arow ? v : 0u;
            }
    }
    // The lane's output heads are 2*grp and 2*grp + 1 (C rows 4*grp .. 4*grp + 3):
    // their sigma and min term come from the lanes holding rows 4*grp and 4*grp + 2.
    const int hA = 2 * grp, hB = 2 * grp + 1;
    const int sgA = __shfl(sigma, 4 * grp), sgB = __shfl(sigma, 4 * grp + 2);
    const float c0A = __shfl(c0p, 4 * grp), c0B = __shfl(c0p, 4 * grp + 2);
    const float kA = (MODE == MODE_FP16) ? 1.f : ldexpf(1.f, 24 - sgA);
    const float kB = (MODE == MODE_FP16) ? 1.f : ldexpf(1.f, 24 - sgB);
    float *const outA = p.out + (b * p.heads_q + hq0 + hA) * T;
    float *const outB = p.out + (b * p.heads_q + hq0 + hB) * T;
    const bool stA = hA < G, stB = hB < G;

    // ---- tiles: lane loads its token's channel block, PF tiles ahead
    const uint8_t *const cl = p.codes + b * T * p.row_bytes + static_cast<int64_t>(hkv) * (D * SH::LANE_BYTES / CPL) +
                              grp * SH::LANE_BYTES;
    const uint16_t *const enl = NSN ? p.en + (b * p.heads_kv + hkv) * T : nullptr;
    auto load = [&](int64_t it) {
        Tile<D, MODE, BITS> r;
        int64_t t = it * 16 + row;
        t = t < T ? t : T - 1;
        const uint8_t *src = cl + t * p.row_bytes;
        if constexpr (NW % 4 == 0) {
#pragma unroll
            for (int k = 0; k < NW / 4; ++k) {
                const uint4 v = reinterpret_cast<const uint4 *>(src)[k];
                r.w[4 * k] = v.x; r.w[4 * k + 1] = v.y; r.w[4 * k + 2] = v.z; r.w[4 * k + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < NW; ++k) r.w[k] = reinterpret_cast<const uint32_t *>(src)[k];
        }
        r.en = NSN ? enl[t] : 0u;
        return r;
    };
    auto process = [&](const Tile<D, MODE, BITS> &r, int64_t it) {
        u32x4 Bf[NK];
        b_frags<D, MODE, BITS>(r, Bf);
        f32x4 C = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NK; ++kk) C = mfma(A[kk], Bf[kk], C);
        const int64_t t = it * 16 + row;
        if (t < T) {
            const float f = NSN ? h2f(static_cast<uint16_t>(r.en)) * p.scale : p.scale;
            if (stA) outA[t] = ((C[0] + C[1]) * kA + c0A) * f;
            if (stB) outB[t] = ((C[2] + C[3]) * kB + c0B) * f;
        }
    };
    Tile<D, MODE, BITS> buf[PF];
#pragma unroll
    for (int u = 0; u < PF; ++u)
        if (it0 + u < it1) buf[u] = load(it0 + u);
    for (int64_t base = it0; base < it1; base += PF) {
#pragma unroll
        for (int u = 0; u < PF; ++u) {
            const int64_t it = base + u;
            if (it < it1) {
                const Tile<D, MODE, BITS> r = buf[u];
                if (it + PF < it1) buf[u] = load(it + PF);
                process(r, it);
            }
        }
    }
}

}  // namespace ks
}  // namespace nsn

using namespace nsn;

namespace {

template <int D, int MODE, int BITS>
void ks_launch_nsn(bool nsn, dim3 grid, hipStream_t s, const ks::KsParams &p) {
    if (nsn) hipLaunchKernelGGL((ks::kscore_kernel<D, MODE, BITS, true>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((ks::kscore_kernel<D, MODE, BITS, false>), grid, dim3(256), 0, s, p);
}

template <int D>
void ks_launch_d(int mode, int bits, bool nsn, dim3 grid, hipStream_t s, const ks::KsParams &p) {
    if (mode == NSN_KS_FP16) ks_launch_nsn<D, ks::MODE_FP16, 16>(false, grid, s, p);
    else if (mode == NSN_KS_U8) ks_launch_nsn<D, ks::MODE_U8, 8>(nsn, grid, s, p);
    else if (bits == 3) ks_launch_nsn<D, ks::MODE_PACKED, 3>(nsn, grid, s, p);
    else if (bits == 4) ks_launch_nsn<D, ks::MODE_PACKED, 4>(nsn, grid, s, p);
    else ks_launch_nsn<D, ks::MODE_PACKED, 5>(nsn, grid, s, p);
}

}  // namespace

extern "C" int nsn_kscore(const nsn_kscore_args *a, nsn_stream_t stream) {
    if (!a) return NSN_EINVAL;
    if (a->batch < 0 || a->T < 0 || a->heads_kv <= 0 || a->heads_q <= 0) return NSN_EINVAL;
    if (a->head_dim != 128 && a->head_dim != 256) return NSN_EINVAL;
    if (a->heads_q % a->heads_kv) return NSN_EINVAL;
    const int64_t G = a->heads_q / a->heads_kv;
    if (G < 1 || G > 8) return NSN_EINVAL;
    if (a->mode != NSN_KS_U8 && a->mode != NSN_KS_PACKED && a->mode != NSN_KS_FP16) return NSN_EINVAL;
    if (a->mode == NSN_KS_PACKED && a->bits != 3 && a->bits != 4 && a->bits != 5) return NSN_EINVAL;
    if (a->batch == 0 || a->T == 0) return NSN_OK;
    if (!a->q || !a->codes || !a->out) return NSN_EINVAL;
    if (a->mode != NSN_KS_FP16 && (!a->mins || !a->steps)) return NSN_EINVAL;
    const int64_t D = a->head_dim, hidden = a->heads_kv * D;
    const int64_t row_bytes = a->mode == NSN_KS_FP16 ? 2 * hidden
                            : a->mode == NSN_KS_U8 ? hidden : hidden * a->bits / 8;
    const int64_t lane_bytes = a->mode == NSN_KS_FP16 ? D / 2 : a->mode == NSN_KS_U8 ? D / 4 : D / 4 * a->bits / 8;
    const uintptr_t need = (lane_bytes % 16 == 0) ? 16 : 4;
    if ((reinterpret_cast<uintptr_t>(a->codes) & (need - 1)) || (row_bytes % static_cast<int64_t>(need))) return NSN_EINVAL;
    if ((reinterpret_cast<uintptr_t>(a->q) & 1u) || (reinterpret_cast<uintptr_t>(a->out) & 3u)) return NSN_EINVAL;
    const int64_t streams = a->batch * a->heads_kv;
    const int64_t tiles = (a->T + 15) / 16;
    // about 16 waves per CU over 256 CUs, each a contiguous run of tiles
    int64_t chunk = (streams * tiles + 4095) / 4096;
    chunk = chunk < 1 ? 1 : (chunk > 64 ? 64 : chunk);
    const int64_t n_chunks = (tiles + chunk - 1) / chunk;
    const int64_t waves = streams * n_chunks;
    if ((waves + 3) / 4 > 0x7fffffff) return NSN_EINVAL;
    ks::KsParams p{};
    p.q = static_cast<const uint16_t *>(a->q);
    p.batch = a->batch;
    p.heads_q = a->heads_q;
    p.heads_kv = a->heads_kv;
    p.T = a->T;
    p.group = static_cast<int>(G);
    p.codes = static_cast<const uint8_t *>(a->codes);
    p.row_bytes = row_bytes;
    p.mins = static_cast<const uint16_t *>(a->mins);
    p.steps = static_cast<const uint16_t *>(a->steps);
    p.en = static_cast<const uint16_t *>(a->eff_norm);
    p.scale = a->scale;
    p.out = a->out;
    p.chunk_tiles = chunk;
    p.n_chunks = n_chunks;
    const bool nsn = a->eff_norm != nullptr && a->mode != NSN_KS_FP16;
    const dim3 grid(static_cast<unsigned>((waves + 3) / 4));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (D == 128) ks_launch_d<128>(a->mode, a->bits, nsn, grid, s, p);
    else ks_launch_d<256>(a->mode, a->bits, nsn, grid, s, p);
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}
