/*
 * attn_elem.h - device helpers shared by the split kernels (attn_split.hip,
 * attn_wide.hip): vector types, the MFMA and transposed-LDS wrappers, how a
 * cached element type becomes exact f16 planes, the XCD-aware workgroup
 * order and a token's first visible position. Internal, device code only.
 */
#ifndef JANAS_AMD_ATTN_ELEM_H
#define JANAS_AMD_ATTN_ELEM_H

#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_kernels.h"
#include "attn_planes.h"

namespace janas {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
/* 16 bytes as a native vector (HIP's uint4 is a struct, which keeps large
   arrays of it out of registers) */
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;     /* query rows a workgroup */

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

/*
 * ds_read_b64_tr_b16: within each group of 16 lanes, lane k supplies the
 * address of 4 halves; lane l receives half l % 4 of the 8-byte pieces of
 * lanes (l % 16) / 4 + 4 i, i = 0..3. With lane k pointing at
 * row base + k / 4, column c0 + 4 (k % 4) of a row-major tile, lane l gets
 * rows base .. base + 3 of column c0 + l % 16: four positions of one value
 * column, the B layout of the PV product.
 */
__device__ __forceinline__ h4 lds_read_tr(const _Float16 *p)
{
    s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4 *)p);
    return __builtin_bit_cast(h4, v);
}

/* x = hi + lo, both f16; x already scaled into f16's normal range. x is
   pinned as the f32 number it is: left free, the compiler may form hi from
   the product that made x, rounded once to f16 (v_fma_mixlo_f16), in one
   kernel instance and from x in another - different bits for one row in
   two instances, and hi + lo no longer x. */
__device__ __forceinline__ void split_hl(float x, _Float16 &hi, _Float16 &lo)
{
    asm volatile("" : "+v"(x));
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

/* ---- element types of the cache -------------------------------------- */

/*
 * Elem<T>: how 8 consecutive numbers of a cached row become f16 planes
 * whose sum is the number exactly (planes8).
 */
template <int T> struct Elem;

template <> struct Elem<kF16> {
    static constexpr int bytes = 2, planes = 1;
    struct Raw { uint4 a; };
    __device__ static Raw load8(const void *b, size_t i)
    {
        return Raw{*(const uint4 *)((const uint16_t *)b + i)};
    }
    __device__ static void planes8(const Raw &r, h8 *p)
    {
        p[0] = __builtin_bit_cast(h8, r.a);
    }
};

template <> struct Elem<kI8> {
    static constexpr int bytes = 1, planes = 1;
    struct Raw { uint2 a; };
    __device__ static Raw load8(const void *b, size_t i)
    {
        return Raw{*(const uint2 *)((const int8_t *)b + i)};
    }
    /* 8 signed bytes to 8 halves, exactly (i8_widen8) */
    __device__ static h8 widen(uint32_t lo, uint32_t hi) { return i8_widen8(lo, hi); }
    __device__ static void planes8(const Raw &r, h8 *p)
    {
        p[0] = widen(r.a.x, r.a.y);
    }
};

template <> struct Elem<kI16> {
    static constexpr int bytes = 2, planes = 2;
    struct Raw { uint4 a; };
    __device__ static Raw load8(const void *b, size_t i)
    {
        return Raw{*(const uint4 *)((const int16_t *)b + i)};
    }
    /* x = 256 (x >> 8) + (x & 255): both parts exact in f16 */
    __device__ static void split(uint4 u, h8 &hi, h8 &lo) { i16_planes8(u.x, u.y, u.z, u.w, hi, lo); }
    __device__ static void planes8(const Raw &r, h8 *p) { split(r.a, p[0], p[1]); }
};

template <> struct Elem<kF32> {
    static constexpr int bytes = 4, planes = 2;
    struct Raw { uint4 a, b; };
    __device__ static Raw load8(const void *b, size_t i)
    {
        const uint4 *s = (const uint4 *)((const float *)b + i);
        return Raw{s[0], s[1]};
    }
    __device__ static void planes8(const Raw &r, h8 *p)
    {
        uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 hi, lo;
            split_hl(__builtin_bit_cast(float, w[e]), hi, lo);
            p[0][e] = hi;
            p[1][e] = lo;
        }
    }
};

/* Which plane pairs enter a product: the low parts of both sides are
   dropped only when both are true residuals (f32 against the split query
   or weights), where their product is below 2^-22 of the sum. */
template <int T> __device__ constexpr bool use_pair(int data_plane, int x_plane)
{
    return !(T == kF32 && data_plane == 1 && x_plane == 1);
}

__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n)
{
    /* blocks are dealt to the 8 XCDs round robin: give each XCD a
       contiguous run of logical ids, so that the row tiles of one chunk
       (consecutive ids) share an L2 */
    /* XCD x (of 8) holds ids x q + min(x, r) .. : n = 8 q + r, the first r
       XCDs one more; branch-free, so the argument loads after it are not
       split across branches. n comes from the arguments (n_wg), loaded with
       the rest, not from the dispatch's grid size */
    const uint32_t x = bid % 8, k = bid / 8, q = n / 8, r = n % 8;
    return x * q + (x < r ? x : r) + k;
}

constexpr int kBlk = 1024 + 32;  /* LDS bytes of a kilobyte of rows */

/* LDS byte offset of byte b of rows stored a kilobyte at a time, each
   followed by 32 bytes of padding (spreads the rows over the banks) */
__device__ __forceinline__ uint32_t blk_off(uint32_t b)
{
    return (b >> 10) * kBlk + (b & 1023);
}

/*
 * The 16-byte unit of a cached row that starts at byte cb (units past the
 * row's rowb bytes read its first unit). An int8 row of 8 mod 16 bytes ends
 * inside its last unit: that unit is read 8 bytes earlier (back), so the
 * load stays inside the row - and inside the buffer at the cache's last
 * row - and unit_fix() swaps its halves into place: the first 8 bytes are
 * the row's last 8, the other 8 are finite numbers of the same row that
 * land in columns past hd (multiplied by zero query columns, or not stored).
 */
__device__ __forceinline__ uint32_t unit_at(uint32_t cb, uint32_t rowb, bool &back)
{
    const uint32_t c = cb < rowb ? cb : 0;
    back = c + 16 > rowb;
    return back ? c - 8 : c;
}

__device__ __forceinline__ u4 unit_fix(u4 x, bool back)
{
    return back ? u4{x.z, x.w, x.x, x.y} : x;
}

/* ---- cross-lane reductions without LDS: v_permlane16_swap /
   v_permlane32_swap exchange rows of 16 (lanes l ^ 16) and halves of the
   wave (l ^ 32); the pair they return holds a value and its partner's, in
   lane order, so both lanes of a pair see the same operands ---- */
__device__ __forceinline__ float max_x16(float a)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float a)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float a)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float a)
{
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
/* the largest over each row of 16 lanes, in every lane of it: DPP
   quad_perm [1, 0, 3, 2] and [2, 3, 0, 1], then row_ror 4 and 8 (a maximum
   does not depend on the order it is taken in, so this is the same number
   as lane-by-lane shuffles give, without their LDS round trips) */
__device__ __forceinline__ float max_row16(float a)
{
    a = fmaxf(a, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(a), 0xB1, 0xf, 0xf, false)));
    a = fmaxf(a, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(a), 0x4E, 0xf, 0xf, false)));
    a = fmaxf(a, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(a), 0x124, 0xf, 0xf, false)));
    a = fmaxf(a, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(a), 0x128, 0xf, 0xf, false)));
    return a;
}
/* lane l ^ 1's value (DPP quad_perm [1, 0, 3, 2]) */
__device__ __forceinline__ float from_x1(float a)
{
    return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(a), 0xB1, 0xf, 0xf, false));
}

/* log2(e), and the reference's weight cutoff e^-80 (attention.c:580) in
   powers of two: 80 / ln 2 */
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kCut2 = -115.41560327111707f;

/* ---- the reference's INT16 way (int8 caches): every float operation
   rounds where the reference's does - no multiply-add is fused unless
   written as one - so the scores, weights and quantized numbers are its
   own, bit for bit ---- */

/* janas_exp_det (vmath.h:36-52): e^x by the Cephes expf polynomial on
   x - n ln 2, ln 2 in two parts, 2^n put into the exponent. A restatement
   of the reference's function, step for step and with its constants, so
   that the INT16 way's weights are its bits: from Janas-LLM
   (prabanta-dev/janas, src/llm/vmath.h), GPL-3.0-or-later; the
   polynomial is Cephes' expf (Stephen L. Moshier). */
__device__ __forceinline__ float exp_det(float x)
{
#pragma clang fp contract(off)
    x = fminf(fmaxf(x, -88.0f), 88.0f);
    const float n = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(-n, 0.693359375f, x);
    r = __builtin_fmaf(-n, -2.12194440e-4f, r);
    float y = 1.9875691500e-4f;
    y = __builtin_fmaf(y, r, 1.3981999507e-3f);
    y = __builtin_fmaf(y, r, 8.3334519073e-3f);
    y = __builtin_fmaf(y, r, 4.1665795894e-2f);
    y = __builtin_fmaf(y, r, 1.6666665459e-1f);
    y = __builtin_fmaf(y, r, 5.0000001201e-1f);
    y = __builtin_fmaf(y, r * r, r);
    y = y + 1.0f;
    return y * __uint_as_float((uint32_t)((int32_t)n + 127) << 23);
}

/* a score from the exact sums of the query's high (x >> 8) and low
   (x & 255) planes against int8 keys: the int32 sum, then times the query
   scale, the score scale and the key scale (attention_scores.h:73-81). The
   high sum times 256 may pass 2^31 on its own: unsigned, it wraps back
   into the int32 sum, which the reference's bound keeps below 2^31 */
__device__ __forceinline__ float q16_scale(int32_t s, float qsc, float scale, float ks)
{
#pragma clang fp contract(off)
    return (float)s * qsc * scale * ks;
}
__device__ __forceinline__ float q16_score(float hi, float lo, float qsc, float scale,
                                           float ks)
{
    const int32_t s = (int32_t)((uint32_t)(int32_t)hi * 256u + (uint32_t)(int32_t)lo);
    return q16_scale(s, qsc, scale, ks);
}

/* a weight (att_weights_ref, attention.c:574-588): 0 below e^-80 of the
   row's largest score m (finite) and for masked scores (-inf) */
__device__ __forceinline__ float det_weight(float s, float m)
{
#pragma clang fp contract(off)
    const float d = s - m;
    return d < -80.0f ? 0.0f : exp_det(d);
}

/* 32767 / mx, or 0 (quant_worker / att_wquant_ref): a quantization's
   multiplier */
__device__ __forceinline__ float q16_inv(float mx)
{
    return mx > 0.0f ? 32767.0f / mx : 0.0f;
}

/* x * inv rounded to the nearest integer, ties to even (lrintf) */
__device__ __forceinline__ int32_t q16_round(float x, float inv)
{
#pragma clang fp contract(off)
    return (int32_t)__builtin_rintf(x * inv);
}

__device__ __forceinline__ uint32_t row_lo(const SplitArgs &A, uint32_t pos)
{
    return A.window && pos + 1 > A.window ? pos + 1 - A.window : 0;
}

}  // namespace
}  // namespace janas

#endif
