// Streaming-cache kernels: append new K/V tokens to the tail in place.
//
// The reference appends by concatenation (a new tensor per update,
// loop_kv_pk01_cache.py:101-102); here the tail is preallocated and both
// sides' new tokens are copied into it by one launch.
#include "nsn_common.hpp"

namespace nsn {
namespace {

// One thread per 16-byte chunk of a new token row, for K and V at once.
__global__ __launch_bounds__(256) void tail_append_kernel(const uint4 *k_new, const uint4 *v_new, int64_t rows,
                                                          int64_t n, int64_t new_row_stride, uint4 *k_tail,
                                                          uint4 *v_tail, int64_t tail_cap, int64_t offset,
                                                          int chunks) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = rows * n * chunks;
    if (i >= total) return;
    const int64_t c = i % chunks, tok = (i / chunks) % n, r = i / (chunks * n);
    const int64_t src = (r * new_row_stride + tok) * chunks + c;
    const int64_t dst = (r * tail_cap + offset + tok) * chunks + c;
    k_tail[dst] = k_new[src];
    v_tail[dst] = v_new[src];
}

// The same copy with the destination taken from device memory: the new
// tokens go to [*tail_end - n, *tail_end) of every row.  An end outside
// [n, tail_cap] writes nothing and raises NSN_ST_TAIL_RANGE.
__global__ __launch_bounds__(256) void tail_append_to_kernel(const uint4 *k_new, const uint4 *v_new, int64_t rows,
                                                             int64_t n, int64_t new_row_stride, uint4 *k_tail,
                                                             uint4 *v_tail, int64_t tail_cap,
                                                             const int32_t *tail_end, int chunks, int32_t *status) {
    const int64_t end = *tail_end;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (end < n || end > tail_cap) {
        if (i == 0) raise_status(status, NSN_ST_TAIL_RANGE);
        return;
    }
    const int64_t total = rows * n * chunks;
    if (i >= total) return;
    const int64_t c = i % chunks, tok = (i / chunks) % n, r = i / (chunks * n);
    const int64_t src = (r * new_row_stride + tok) * chunks + c;
    const int64_t dst = (r * tail_cap + end - n + tok) * chunks + c;
    k_tail[dst] = k_new[src];
    v_tail[dst] = v_new[src];
}

// The copy with a dtype conversion: one thread per 8 elements of a new token
// row (16 bytes of a 16-bit tail), each element read as SDT, rounded to DDT
// (round to nearest even; what torch's Tensor.to does).
template <int SDT, int DDT>
__global__ __launch_bounds__(256) void tail_append_cast_kernel(const void *k_new, const void *v_new, int64_t rows,
                                                               int64_t n, int64_t new_row_stride, uint4 *k_tail,
                                                               uint4 *v_tail, int64_t tail_cap, int64_t offset) {
    using S = Elem<SDT>;
    using D = Elem<DDT>;
    constexpr int G = kDim / 8;   // 8-element groups per row
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= rows * n * G) return;
    const int64_t c = i % G, tok = (i / G) % n, r = i / (G * n);
    const int64_t src = (r * new_row_stride + tok) * kDim + 8 * c;
    const int64_t dst = (r * tail_cap + offset + tok) * G + c;
#pragma unroll
    for (int side = 0; side < 2; ++side) {
        const typename S::T *x = static_cast<const typename S::T *>(side ? v_new : k_new) + src;
        typename S::T v[8];
        if constexpr (SDT == NSN_DTYPE_F32) {
            const float4 a = reinterpret_cast<const float4 *>(x)[0], b = reinterpret_cast<const float4 *>(x)[1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 a = *reinterpret_cast<const uint4 *>(x);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        }
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            o[e] = static_cast<uint32_t>(D::store(S::load(v[2 * e]))) |
                   (static_cast<uint32_t>(D::store(S::load(v[2 * e + 1]))) << 16);
        (side ? v_tail : k_tail)[dst] = uint4{o[0], o[1], o[2], o[3]};
    }
}

struct RopeParams {
    const uint16_t *q, *k, *v, *cos, *sin;
    int64_t cs_stride;   // elements between the cos/sin rows of two sequences (0: one row for all)
    int64_t q_stride, kv_stride;   // elements between two sequences' rows of q, and of k and v
    int64_t batch, heads_q, heads_kv;
    uint16_t *q_out, *k_tail, *v_tail;
    int64_t tail_cap;
    const int32_t *tail_end;
    int64_t offset;
    int32_t *status;
    int tail_bf16;   // tails hold bf16 (else fp16)
};

// One decode token per sequence: rotary embedding of q and k as transformers'
// apply_rotary_pos_emb computes it in the model dtype DT (x*cos and
// rotate_half(x)*sin each rounded to DT, then their sum rounded to DT), the
// rotated q written out, and the rotated k and the plain v converted to the
// tails' fp16 or bf16 and appended to them.  16 threads per row (q rows, then k rows, then v
// rows); thread j owns the channel pairs (c, c + 64) for c = 4j .. 4j + 3.
template <int DT>
__global__ __launch_bounds__(256) void rope_append_kernel(RopeParams p) {
    using E = Elem<DT>;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t nq = p.batch * p.heads_q, nk = p.batch * p.heads_kv;
    if (i >= (nq + 2 * nk) * 16) return;
    const int64_t row = i >> 4;
    const int c0 = 4 * static_cast<int>(i & 15);
    const int kind = row < nq ? 0 : (row < nq + nk ? 1 : 2);
    int64_t off = p.offset;
    if (p.tail_end) {
        const int64_t end = *p.tail_end;
        if (end < 1 || end > p.tail_cap) {   // the rotated q is still written; the tails are not
            if (i == 0) raise_status(p.status, NSN_ST_TAIL_RANGE);
            if (kind != 0) return;
        }
        off = end - 1;
    }
    const int64_t r = kind == 0 ? row : (kind == 1 ? row - nq : row - nq - nk);   // (b, h) row of its tensor
    const int64_t heads = kind == 0 ? p.heads_q : p.heads_kv;
    const int64_t b = r / heads;
    const uint16_t *src = (kind == 0 ? p.q : (kind == 1 ? p.k : p.v)) + b * (kind == 0 ? p.q_stride : p.kv_stride) +
                          (r - b * heads) * kDim;
    const uint2 a = *reinterpret_cast<const uint2 *>(src + c0);
    const uint2 z = *reinterpret_cast<const uint2 *>(src + 64 + c0);
    const uint16_t x1[4] = {static_cast<uint16_t>(a.x), static_cast<uint16_t>(a.x >> 16), static_cast<uint16_t>(a.y),
                            static_cast<uint16_t>(a.y >> 16)};
    const uint16_t x2[4] = {static_cast<uint16_t>(z.x), static_cast<uint16_t>(z.x >> 16), static_cast<uint16_t>(z.y),
                            static_cast<uint16_t>(z.y >> 16)};
    float o1[4], o2[4];
    if (kind < 2) {
        auto rd = [](float x) { return E::load(E::store(x)); };
        const uint16_t *cs = p.cos + b * p.cs_stride, *sn = p.sin + b * p.cs_stride;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float u = E::load(x1[j]), w = E::load(x2[j]);
            const float c1 = E::load(cs[c0 + j]), c2 = E::load(cs[64 + c0 + j]);
            const float s1 = E::load(sn[c0 + j]), s2 = E::load(sn[64 + c0 + j]);
            o1[j] = rd(rd(u * c1) + rd(-w * s1));
            o2[j] = rd(rd(w * c2) + rd(u * s2));
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            o1[j] = E::load(x1[j]);
            o2[j] = E::load(x2[j]);
        }
    }
    uint16_t *dst;
    uint16_t h1[4], h2[4];
    if (kind == 0) {
        dst = p.q_out + r * kDim;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h1[j] = E::store(o1[j]);
            h2[j] = E::store(o2[j]);
        }
    } else {
        dst = (kind == 1 ? p.k_tail : p.v_tail) + (r * p.tail_cap + off) * kDim;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h1[j] = p.tail_bf16 ? f32_to_bf16_bits(o1[j]) : f32_to_f16_bits(o1[j]);
            h2[j] = p.tail_bf16 ? f32_to_bf16_bits(o2[j]) : f32_to_f16_bits(o2[j]);
        }
    }
    *reinterpret_cast<uint2 *>(dst + c0) = make_uint2(h1[0] | (static_cast<uint32_t>(h1[1]) << 16),
                                                      h1[2] | (static_cast<uint32_t>(h1[3]) << 16));
    *reinterpret_cast<uint2 *>(dst + 64 + c0) = make_uint2(h2[0] | (static_cast<uint32_t>(h2[1]) << 16),
                                                           h2[2] | (static_cast<uint32_t>(h2[3]) << 16));
}

}  // namespace
}  // namespace nsn

using namespace nsn;

extern "C" int nsn_tail_append(const void *k_new, const void *v_new, int64_t rows, int64_t n, int64_t new_row_stride,
                               void *k_tail, void *v_tail, int64_t tail_cap, int64_t offset, int dtype,
                               nsn_stream_t stream) {
    if (rows < 0 || n < 0 || offset < 0 || new_row_stride < n || tail_cap < offset + n) return NSN_EINVAL;
    if (dtype != NSN_DTYPE_F16 && dtype != NSN_DTYPE_BF16 && dtype != NSN_DTYPE_F32) return NSN_EINVAL;
    if (rows == 0 || n == 0) return NSN_OK;
    if (!k_new || !v_new || !k_tail || !v_tail) return NSN_EINVAL;
    for (const void *ptr : {k_new, v_new, static_cast<const void *>(k_tail), static_cast<const void *>(v_tail)})
        if (reinterpret_cast<uintptr_t>(ptr) & 15u) return NSN_EINVAL;
    const int chunks = kDim * (dtype == NSN_DTYPE_F32 ? 4 : 2) / 16;
    const int64_t total = rows * n * chunks;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return NSN_EINVAL;
    hipLaunchKernelGGL(tail_append_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const uint4 *>(k_new),
                       static_cast<const uint4 *>(v_new), rows, n, new_row_stride, static_cast<uint4 *>(k_tail),
                       static_cast<uint4 *>(v_tail), tail_cap, offset, chunks);
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

extern "C" int nsn_tail_append_cast(const void *k_new, const void *v_new, int src_dtype, int64_t rows, int64_t n,
                                    int64_t new_row_stride, void *k_tail, void *v_tail, int64_t tail_cap,
                                    int64_t offset, int dtype, nsn_stream_t stream) {
    if (rows < 0 || n < 0 || offset < 0 || new_row_stride < n || tail_cap < offset + n) return NSN_EINVAL;
    if (src_dtype != NSN_DTYPE_F16 && src_dtype != NSN_DTYPE_BF16 && src_dtype != NSN_DTYPE_F32) return NSN_EINVAL;
    if (dtype != NSN_DTYPE_F16 && dtype != NSN_DTYPE_BF16) return NSN_EINVAL;
    if (rows == 0 || n == 0) return NSN_OK;
    if (!k_new || !v_new || !k_tail || !v_tail) return NSN_EINVAL;
    for (const void *ptr : {k_new, v_new, static_cast<const void *>(k_tail), static_cast<const void *>(v_tail)})
        if (reinterpret_cast<uintptr_t>(ptr) & 15u) return NSN_EINVAL;
    const int64_t total = rows * n * (kDim / 8);
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return NSN_EINVAL;
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    uint4 *kt = static_cast<uint4 *>(k_tail), *vt = static_cast<uint4 *>(v_tail);
#define NSN_CAST_LAUNCH(S_, D_)                                                                                     \
    hipLaunchKernelGGL((tail_append_cast_kernel<S_, D_>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, k_new, \
                       v_new, rows, n, new_row_stride, kt, vt, tail_cap, offset)
    if (dtype == NSN_DTYPE_F16) {
        if (src_dtype == NSN_DTYPE_F16) NSN_CAST_LAUNCH(NSN_DTYPE_F16, NSN_DTYPE_F16);
        else if (src_dtype == NSN_DTYPE_BF16) NSN_CAST_LAUNCH(NSN_DTYPE_BF16, NSN_DTYPE_F16);
        else NSN_CAST_LAUNCH(NSN_DTYPE_F32, NSN_DTYPE_F16);
    } else {
        if (src_dtype == NSN_DTYPE_F16) NSN_CAST_LAUNCH(NSN_DTYPE_F16, NSN_DTYPE_BF16);
        else if (src_dtype == NSN_DTYPE_BF16) NSN_CAST_LAUNCH(NSN_DTYPE_BF16, NSN_DTYPE_BF16);
        else NSN_CAST_LAUNCH(NSN_DTYPE_F32, NSN_DTYPE_BF16);
    }
#undef NSN_CAST_LAUNCH
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

extern "C" int nsn_tail_append_to(const void *k_new, const void *v_new, int64_t rows, int64_t n,
                                  int64_t new_row_stride, void *k_tail, void *v_tail, int64_t tail_cap,
                                  const int32_t *tail_end, int dtype, int32_t *status, nsn_stream_t stream) {
    if (rows < 0 || n < 0 || new_row_stride < n || tail_cap < n) return NSN_EINVAL;
    if (dtype != NSN_DTYPE_F16 && dtype != NSN_DTYPE_BF16 && dtype != NSN_DTYPE_F32) return NSN_EINVAL;
    if (rows == 0 || n == 0) return NSN_OK;
    if (!k_new || !v_new || !k_tail || !v_tail || !tail_end || !status) return NSN_EINVAL;
    for (const void *ptr : {k_new, v_new, static_cast<const void *>(k_tail), static_cast<const void *>(v_tail)})
        if (reinterpret_cast<uintptr_t>(ptr) & 15u) return NSN_EINVAL;
    const int chunks = kDim * (dtype == NSN_DTYPE_F32 ? 4 : 2) / 16;
    const int64_t total = rows * n * chunks;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return NSN_EINVAL;
    hipLaunchKernelGGL(tail_append_to_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), static_cast<const uint4 *>(k_new),
                       static_cast<const uint4 *>(v_new), rows, n, new_row_stride, static_cast<uint4 *>(k_tail),
                       static_cast<uint4 *>(v_tail), tail_cap, tail_end, chunks, status);
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}

extern "C" int nsn_rope_append(const void *q, const void *k, const void *v, int64_t q_stride, int64_t kv_stride,
                               const void *cos, const void *sin, int64_t cs_stride, int64_t batch, int64_t heads_q,
                               int64_t heads_kv, void *q_out, void *k_tail,
                               void *v_tail, int64_t tail_cap, const int32_t *tail_end, int64_t offset, int dtype,
                               int tail_dtype, int32_t *status, nsn_stream_t stream) {
    if (batch < 0 || heads_q < 0 || heads_kv < 0 || tail_cap < 1 || (cs_stride != 0 && cs_stride < kDim))
        return NSN_EINVAL;
    if (q_stride < heads_q * kDim || kv_stride < heads_kv * kDim || (q_stride & 3) || (kv_stride & 3))
        return NSN_EINVAL;
    if (dtype != NSN_DTYPE_F16 && dtype != NSN_DTYPE_BF16) return NSN_EINVAL;
    if (tail_dtype != NSN_DTYPE_F16 && tail_dtype != NSN_DTYPE_BF16) return NSN_EINVAL;
    if (!tail_end && (offset < 0 || offset >= tail_cap)) return NSN_EINVAL;
    if (batch == 0 || heads_q + heads_kv == 0) return NSN_OK;
    if (!q || !k || !v || !cos || !sin || !q_out || !k_tail || !v_tail || !status) return NSN_EINVAL;
    for (const void *ptr : {q, k, v, static_cast<const void *>(q_out), static_cast<const void *>(k_tail),
                            static_cast<const void *>(v_tail)})
        if (reinterpret_cast<uintptr_t>(ptr) & 7u) return NSN_EINVAL;
    const int64_t threads = batch * (heads_q + 2 * heads_kv) * 16;
    const int64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffff) return NSN_EINVAL;
    RopeParams p{static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v),
                 static_cast<const uint16_t *>(cos), static_cast<const uint16_t *>(sin), cs_stride, q_stride, kv_stride,
                 batch, heads_q, heads_kv,
                 static_cast<uint16_t *>(q_out), static_cast<uint16_t *>(k_tail), static_cast<uint16_t *>(v_tail),
                 tail_cap, tail_end, offset, status, tail_dtype == NSN_DTYPE_BF16 ? 1 : 0};
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dtype == NSN_DTYPE_BF16) hipLaunchKernelGGL(rope_append_kernel<NSN_DTYPE_BF16>, dim3(blocks), dim3(256), 0, st, p);
    else hipLaunchKernelGGL(rope_append_kernel<NSN_DTYPE_F16>, dim3(blocks), dim3(256), 0, st, p);
    return hipGetLastError() == hipSuccess ? NSN_OK : NSN_ELAUNCH;
}
