// Device helpers shared by the NSN kernels (gfx950 / CDNA4, wave64).
//
// Arithmetic that must reproduce the reference bit-for-bit (the codec) uses
// only IEEE-exact building blocks: explicit fmaf where torch fuses, unfused
// multiply/add elsewhere (the library is built with -ffp-contract=off),
// correctly rounded division and square root, round-half-even, and RNE
// conversions to fp16/bf16.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/nsn_hip.h"

namespace nsn {

constexpr int kDim = 128;       // channels per token row (head_dim)
constexpr int kBlockTok = 64;   // tokens per packed block
constexpr float kEps = 1e-12f;  // clamp_min of the norms

__host__ __device__ constexpr int packed_block_bytes(int bits) { return kBlockTok * kDim * bits / 8; }

// ------------------------------------------------------------ conversions

// Materialise an fp32 value in a VGPR.  Without it the backend may fold
// "fp32 multiply, then convert to fp16" into one v_fma_mixlo_f16, which rounds
// the exact product straight to fp16 and skips the fp32 rounding the
// reference performs -- a different result at fp16 ties.
__device__ __forceinline__ float keep_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __half_as_ushort(__float2half_rn(keep_f32(f)));   // v_cvt_f16_f32, round to nearest even
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

template <int DT> struct Elem;
template <> struct Elem<NSN_DTYPE_F16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return f16_bits_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_f16_bits(f); }
};
template <> struct Elem<NSN_DTYPE_BF16> {
    using T = uint16_t;
    static __device__ __forceinline__ float load(T v) { return bf16_bits_to_f32(v); }
    static __device__ __forceinline__ T store(float f) { return f32_to_bf16_bits(f); }
};
template <> struct Elem<NSN_DTYPE_F32> {
    using T = float;
    static __device__ __forceinline__ float load(T v) { return v; }
    static __device__ __forceinline__ T store(float f) { return f; }
};

// ------------------------------------------------------ exact arithmetic

// Correctly rounded fp32 square root: the double square root is correctly
// rounded, and rounding a correctly rounded 53-bit square root to 24 bits is
// again correctly rounded (53 >= 2*24 + 2).
__device__ __forceinline__ float sqrt_rn(float x) {
    return static_cast<float>(__dsqrt_rn(static_cast<double>(x)));
}

// a / b for fp32 a, b given rb = 1.0 / (double)b (correctly rounded double).
// The fp64 product is within 2^-52 (relative) of a/b, while a quotient of two
// 24-bit significands is never closer than 2^-49 (relative) to a rounding
// midpoint of fp32 unless it is exact; so the final rounding to fp32 equals
// IEEE division.  Costs one fp64 multiply per element instead of the ~10
// instruction fp32 division sequence.
__device__ __forceinline__ float div_by_recip(float a, double rb) {
    return static_cast<float>(static_cast<double>(a) * rb);
}

__device__ __forceinline__ double recip_rn(float b) { return __ddiv_rn(1.0, static_cast<double>(b)); }

// torch's clamp_min(1e-12): NaN propagates.
__device__ __forceinline__ float clamp_eps(float n) { return (n > kEps || n != n) ? n : kEps; }

__device__ __forceinline__ bool finite(float x) { return __builtin_isfinite(x); }

// Lane-ordered accumulation of squares that reproduces torch-CPU's
// vector_norm over a contiguous row of 128 fp32 values: lane j (0..7) holds
// fma-chained squares of elements j, j+8, ..., then the lanes are summed in
// order 0..7.
__device__ __forceinline__ float lane8_sum(const float (&acc)[8]) {
    float s = acc[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) s = s + acc[j];
    return s;
}

// Fast (MFMA) decode attention launcher, defined in nsn_fast.hip.
int launch_attn_fast(const nsn_attn_args *a, hipStream_t st);

// ------------------------------------------------------------ status word

__device__ __forceinline__ void raise_status(int32_t* status, int bits) {
    if (status && bits) atomicOr(status, bits);
}

}  // namespace nsn
