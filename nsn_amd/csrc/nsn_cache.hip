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
