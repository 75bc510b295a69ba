/*
 * attn_planes.h - integers of the engine's int8 / int16 caches as exact f16
 * planes, by byte permutes and packed f16 arithmetic: shared by the split
 * and wide kernels (staging a chunk) and the exact prefill's copy pass.
 * Internal, device code only.
 *
 * A byte b under the exponent byte 0x64 is the half 1024 + b: halves in
 * [1024, 2048) step by 1, so one byte permute and one packed subtraction
 * give two bytes as exact halves.
 */
#ifndef JANAS_AMD_ATTN_PLANES_H
#define JANAS_AMD_ATTN_PLANES_H

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace janas {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef int i4 __attribute__((ext_vector_type(4)));   /* 16 bytes as int8 operands */

/* 4 signed bytes (a word, the first in the low byte) to 4 halves, exactly:
   b ^ 0x80 = b + 128 under 0x64 is the half 1152 + b, less 1152 is b - one
   xor, two byte permutes and two packed subtractions for the 4 */
__device__ __forceinline__ void i8_widen4(uint32_t x, h2 &a, h2 &b)
{
    const uint32_t u = x ^ 0x80808080u;
    const uint32_t pa = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t pb = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    a = __builtin_bit_cast(h2, pa) - off;
    b = __builtin_bit_cast(h2, pb) - off;
}

/* 8 signed bytes (lo: the first 4) to 8 halves */
__device__ __forceinline__ h8 i8_widen8(uint32_t lo, uint32_t hi)
{
    h2 p[4];
    i8_widen4(lo, p[0], p[1]);
    i8_widen4(hi, p[2], p[3]);
    return h8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

/* 4 int16 numbers (two words, the first in the low half) as the f16 planes
   256 (x >> 8) and x & 255, both exact: the low bytes less 1024 are x & 255;
   the high bytes, flipped to b + 128, less 1152 are x >> 8, times 256 - two
   byte permutes and six packed f16 operations for the 4, the same numbers
   as converting each through f32 */
__device__ __forceinline__ void i16_planes4(uint32_t w0, uint32_t w1, h4 &hi, h4 &lo)
{
    const h2 k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const h2 k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 k256 = {(_Float16)256.0f, (_Float16)256.0f};
    const h2 l0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w0, 0x04020400u)) - k1024;
    const h2 l1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w1, 0x04020400u)) - k1024;
    const h2 h0 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w0 ^ 0x80808080u,
                                                                0x04030401u)) - k1152) * k256;
    const h2 h1 = (__builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, w1 ^ 0x80808080u,
                                                                0x04030401u)) - k1152) * k256;
    lo = h4{l0[0], l0[1], l1[0], l1[1]};
    hi = h4{h0[0], h0[1], h1[0], h1[1]};
}

/* 8 int16 numbers (four words) as the two planes */
__device__ __forceinline__ void i16_planes8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3,
                                            h8 &hi, h8 &lo)
{
    h4 h0, l0, h1, l1;
    i16_planes4(w0, w1, h0, l0);
    i16_planes4(w2, w3, h1, l1);
    hi = h8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
    lo = h8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
}

}  // namespace
}  // namespace janas

#endif
