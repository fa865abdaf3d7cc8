// Bit-packed K codes -> fp16-subnormal MFMA B operands (gfx950), shared by
// the fast decode kernel (nsn_fast.hip) and the K-score kernel
// (nsn_kscore.hip).
//
// A lane holds 32 consecutive codes of one token (BITS dwords of the
// LSB-first bitstream, starting on a 32-code boundary).  kunpack turns them
// into the B operands of 4 K-steps of v_mfma_f32_16x16x32_f16: K-step kk
// covers codes 8kk .. 8kk+7, element e (dword e/2, half e%2) = code
// 8kk + chE[e], left at bit kE[e] of its half -- an fp16 subnormal of value
// z * 2^(kE[e]-24), exact.  The A operand pairs element e with the matching
// coefficient times 2^-kE[e].
#pragma once

#include "nsn_common.hpp"

namespace nsn {
namespace unpack {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// v_perm_b32: byte i of the result = byte sel[i] of {hi:lo} (0..3 = lo, 4..7 = hi, 0x0c = 0).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// ---------------------------------------------------------------------------
// Code layouts.  A lane's B operand for one MFMA K-step is 8 codes as fp16
// halves e = 0..7 (dword e/2, half e%2).
//
// K side: the lane owns one token and a 32-channel chunk; K-step kk takes the
// chunk's channels 8kk .. 8kk+7 (3 bytes at 3 bits), element e = channel
// chE[e], its code left at bit kE[e] of the half (value z * 2^(kE-24)).
// V side: the lane owns channels 8*row .. 8*row+7 of 16 tokens; tile m is
// channel 8*row + m, its code at bit kV[m] of every half.
// ---------------------------------------------------------------------------
template <int BITS> struct Layout;
template <> struct Layout<3> {
    static constexpr int chE[8] = {0, 3, 1, 4, 2, 5, 6, 7};
    static constexpr int kE[8] = {0, 1, 3, 4, 6, 7, 2, 5};
    static constexpr int kV[8] = {0, 3, 6, 1, 4, 7, 2, 5};
};
template <> struct Layout<5> {
    static constexpr int chE[8] = {0, 1, 2, 4, 5, 7, 3, 6};
    static constexpr int kE[8] = {0, 5, 2, 4, 1, 3, 1, 0};
    static constexpr int kV[8] = {0, 5, 2, 1, 4, 1, 0, 3};
};

// 3-bit K chunk (u0, u1, u2 = 12 bytes, 32 codes) -> 4 K-step B operands.
// Group kk spans bytes g0 g1 g2 = 3kk .. 3kk+2.  P = (g0 g1 | g1 g2) holds the
// 16-bit windows starting at g0 and g1; Q = (g2 | g2).  Every code then sits
// at bit 0..7 of one window and is isolated by a single AND.
__device__ __forceinline__ void kgroup3(uint32_t P, uint32_t Q, u32x4 &B) {
    B[0] = P & 0x000E0007u;   // ch0 @0 | ch3 @1
    B[1] = P & 0x00700038u;   // ch1 @3 | ch4 @4
    B[2] = P & 0x038001C0u;   // ch2 @6 | ch5 @7
    B[3] = Q & 0x00E0001Cu;   // ch6 @2 | ch7 @5
}
__device__ __forceinline__ void kunpack(const uint32_t (&u)[3], u32x4 (&B)[4]) {
    kgroup3(perm(u[0], u[0], 0x02010100u), perm(u[0], u[0], 0x0C020C02u), B[0]);
    kgroup3(perm(u[1], u[0], 0x05040403u), perm(u[1], u[0], 0x0C050C05u), B[1]);
    kgroup3(perm(u[2], u[1], 0x04030302u), perm(u[2], u[1], 0x0C040C04u), B[2]);
    kgroup3(perm(u[2], u[2], 0x03020201u), perm(u[2], u[2], 0x0C030C03u), B[3]);
}
// 5-bit K chunk (u0..u4 = 20 bytes, 32 codes) -> 4 K-step B operands.  Group
// g = bytes b0..b4 = 5g..5g+4 (8 codes at bits 5k).  Byte windows hold codes
// 0/1 (b0 b1: bits 0, 5), 2 (b1 b2: bit 2), 4 (b2 b3: bit 4), 5 (b3 b4: bit
// 1), 7 (b4: bit 3); codes 3 and 6 straddle bytes at bits 15 and 30 and come
// from the group shifted by 14 bits (bit 1 of the low half, bit 0 of the high
// half).  One AND per pair of codes, 3 perms and 1 funnel shift per group.
__device__ __forceinline__ constexpr uint32_t sel4(int a, int b, int c, int d) {
    return static_cast<uint32_t>(a | (b << 8) | (c << 16) | (d << 24));
}
__device__ __forceinline__ void kunpack(const uint32_t (&u)[5], u32x4 (&B)[4]) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int w = (5 * g) / 4, o = 5 * g - 4 * w;           // group bytes at o .. o+4 of (u[w+1]:u[w])
        const uint32_t lo = u[w], hi = u[w + 1 < 5 ? w + 1 : 4];
        const uint32_t P0 = perm(hi, lo, sel4(o, o + 1, o, o + 1));
        const uint32_t P1 = perm(hi, lo, sel4(o + 1, o + 2, o + 2, o + 3));
        const uint32_t P2 = perm(hi, lo, sel4(o + 3, o + 4, o + 4, o + 4));
        const int bit = 40 * g + 14, aw = bit / 32;
        const uint32_t A = __builtin_amdgcn_alignbit(u[aw + 1 < 5 ? aw + 1 : 4], u[aw], bit % 32);
        B[g][0] = P0 & 0x03E0001Fu;   // ch0 @0 | ch1 @5
        B[g][1] = P1 & 0x01F0007Cu;   // ch2 @2 | ch4 @4
        B[g][2] = P2 & 0x00F8003Eu;   // ch5 @1 | ch7 @3
        B[g][3] = A & 0x001F003Eu;    // ch3 @1 | ch6 @0
    }
}

// 4-bit: two codes per byte.  Bytes b0, b1 of each dword go to the low and
// high halves (P), b2, b3 likewise (Q); one AND keeps the low nibbles (bit 0),
// another the high nibbles (bit 4).
template <> struct Layout<4> {
    static constexpr int chE[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    static constexpr int kE[8] = {0, 0, 4, 4, 0, 0, 4, 4};
};
__device__ __forceinline__ void kunpack(const uint32_t (&u)[4], u32x4 (&B)[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const uint32_t x = u[kk];
        const uint32_t P = perm(x, x, 0x0C010C00u), Q = perm(x, x, 0x0C030C02u);
        B[kk][0] = P & 0x000F000Fu;   // ch0 @0 | ch2 @0
        B[kk][1] = P & 0x00F000F0u;   // ch1 @4 | ch3 @4
        B[kk][2] = Q & 0x000F000Fu;   // ch4 @0 | ch6 @0
        B[kk][3] = Q & 0x00F000F0u;   // ch5 @4 | ch7 @4
    }
}

}  // namespace unpack
}  // namespace nsn
