/*
 * attn_q8k.h - one Q8_K block (struct janas_block_q8k, src/llm/quant.h:
 * 283-300) from 256 numbers held one a thread by a workgroup of 256, as
 * q8k_quantize_ref does it (src/llm/quant.c:174-200, q8_32_ref :150-172):
 * d = amax / 127 and its reciprocal, rint and clamp to +-127, the sums of
 * 16 and of 32, and the same numbers again in 8 blocks of 32 with scales of
 * their own. Shared by the Q8_K pass (attn_cache.hip), the merge that
 * quantizes its own output (attn_split.hip) and the prefill kernels' output
 * and segment merge (attn_prefill.hip), each with its own way of holding a
 * block's numbers. Internal, device code only.
 */
#ifndef JANAS_AMD_ATTN_Q8K_H
#define JANAS_AMD_ATTN_Q8K_H

#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_kernels.h"

namespace janas {

/* the workgroup's LDS for a block */
struct Q8kLds {
    float red[8];
    int sum[16];
    __attribute__((aligned(16))) uint8_t blk[kQ8kBytes];
};

/* a block's (or a 32's) scale from its largest magnitude, and the
   reciprocal it quantizes with (quant.c:150-200) */
__device__ __forceinline__ void q8k_scale(float amax, float &d, float &id)
{
#pragma clang fp contract(off)
    d = amax / 127.0f;
    id = d > 0.0f ? 1.0f / d : 0.0f;
}

/* one number quantized: rint(x id), clamped to +-127 */
__device__ __forceinline__ int q8k_round(float x, float id)
{
#pragma clang fp contract(off)
    float q = rintf(x * id);
    q = q > 127.0f ? 127.0f : q < -127.0f ? -127.0f : q;
    return (int)q;
}

/*
 * Thread t (of 256, all of them calling) holds number t of the block; the
 * block's 628 bytes go to dst. Block layout: d @0, qs @4, bsums @260,
 * d32 @292, qs32 @324, bsums32 @580, bsums2 @612.
 */
__device__ __forceinline__ void q8k_block(float x, uint32_t t, uint8_t *dst, Q8kLds &S)
{
#pragma clang fp contract(off)
    const uint32_t w = t >> 6, lane = t & 63;
    /* the 256's largest magnitude (waves, then across) and the 32's */
    float m = fabsf(x);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        m = fmaxf(m, __shfl_xor(m, o, 64));
    float m32 = fabsf(x);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1)
        m32 = fmaxf(m32, __shfl_xor(m32, o, 64));
    if (lane == 0)
        S.red[w] = m;
    __syncthreads();
    const float amax = fmaxf(fmaxf(S.red[0], S.red[1]), fmaxf(S.red[2], S.red[3]));
    float d, id, d32, id32;
    q8k_scale(amax, d, id);
    q8k_scale(m32, d32, id32);
    const int q = q8k_round(x, id), q32 = q8k_round(x, id32);
    S.blk[4 + t] = (uint8_t)(int8_t)q;
    S.blk[324 + t] = (uint8_t)(int8_t)q32;
    if (t == 0)
        *(float *)&S.blk[0] = d;
    if ((t & 31) == 0)
        *(float *)&S.blk[292 + 4 * (t / 32)] = d32;
    /* sums of 16: integers, exact in any order */
    int s = q, s32 = q32;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
        s += __shfl_xor(s, o, 64);
        s32 += __shfl_xor(s32, o, 64);
    }
    if ((t & 15) == 0) {
        *(int16_t *)&S.blk[260 + 2 * (t / 16)] = (int16_t)s;
        *(int16_t *)&S.blk[580 + 2 * (t / 16)] = (int16_t)s32;
        S.sum[t / 16] = s;
    }
    __syncthreads();
    if (t < 8)
        *(int16_t *)&S.blk[612 + 2 * t] = (int16_t)(S.sum[2 * t] + S.sum[2 * t + 1]);
    __syncthreads();
    if (t < kQ8kBytes / 4)
        *(uint32_t *)(dst + 4 * t) = *(const uint32_t *)&S.blk[4 * t];
}

/*
 * Q8_K blocks of numbers spread over a wave four to a lane, one block a
 * wave: lane k holds numbers 4 k .. 4 k + 3 of the block (x[0..3]) - the
 * prefill's segment merge, whose threads take 4 columns of a row each. The
 * operations are q8k_block's; the reductions go across lanes. store: the
 * wave's block exists (all lanes of a wave agree).
 */
__device__ __forceinline__ void q8k_wave4(const float x[4], uint8_t *dst, bool store)
{
#pragma clang fp contract(off)
    const uint32_t k = threadIdx.x & 63;
    float m32 = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
#pragma unroll
    for (int o = 1; o < 8; o <<= 1)
        m32 = fmaxf(m32, __shfl_xor(m32, o, 64));
    float m = m32;
#pragma unroll
    for (int o = 8; o < 64; o <<= 1)
        m = fmaxf(m, __shfl_xor(m, o, 64));
    float d, id, d32, id32;
    q8k_scale(m, d, id);
    q8k_scale(m32, d32, id32);
    uint32_t qw = 0, qw32 = 0;
    int s = 0, s32 = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int q = q8k_round(x[e], id), q32 = q8k_round(x[e], id32);
        qw |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
        qw32 |= (uint32_t)(uint8_t)(int8_t)q32 << (8 * e);
        s += q;
        s32 += q32;
    }
    /* sums of 16 (4 lanes) and of 32 (8 lanes): integers, exact */
#pragma unroll
    for (int o = 1; o < 4; o <<= 1) {
        s += __shfl_xor(s, o, 64);
        s32 += __shfl_xor(s32, o, 64);
    }
    const int s2 = s + __shfl_xor(s, 4, 64);
    if (!store)
        return;
    *(uint32_t *)(dst + 4 + 4 * k) = qw;
    *(uint32_t *)(dst + 324 + 4 * k) = qw32;
    if ((k & 3) == 0) {
        *(int16_t *)(dst + 260 + 2 * (k / 4)) = (int16_t)s;
        *(int16_t *)(dst + 580 + 2 * (k / 4)) = (int16_t)s32;
    }
    if ((k & 7) == 0) {
        *(float *)(dst + 292 + 4 * (k / 8)) = d32;
        *(int16_t *)(dst + 612 + 2 * (k / 8)) = (int16_t)s2;
    }
    if (k == 0)
        *(float *)dst = d;
}

/*
 * Q8_K blocks of the rows a prefill wave holds: lane l's row is l % 32,
 * x[c][4 m + e] its column 32 c + 8 m + 4 (l / 32) + e (c < CT, a row of
 * 32 CT numbers), RB rows a block (RB = 256 / (32 CT), lanes differing in
 * their low log2(RB) bits). q8k_block's operations; the reductions go
 * across the block's lanes. dst: the lane's block; store: its row exists
 * (all rows of a block agree).
 */
template <int CT, class Rows>
__device__ __forceinline__ void q8k_rows(const Rows &x, uint8_t *dst, bool store)
{
#pragma clang fp contract(off)
    constexpr uint32_t HD = 32 * CT, RB = 256 / HD;
    static_assert(RB * HD == 256, "a block is whole rows");
    const uint32_t lane = threadIdx.x & 63, g = lane >> 5, hb = lane & (RB - 1);
    float m32[CT], m = 0.0f;
#pragma unroll
    for (int c = 0; c < CT; c++) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++)
            t = fmaxf(t, fabsf(x[c][i]));
        m32[c] = fmaxf(t, __shfl_xor(t, 32, 64));
        m = fmaxf(m, m32[c]);
    }
#pragma unroll
    for (uint32_t o = 1; o < RB; o <<= 1)
        m = fmaxf(m, __shfl_xor(m, o, 64));
    float d, id;
    q8k_scale(m, d, id);
#pragma unroll
    for (int c = 0; c < CT; c++) {
        float d32, id32;
        q8k_scale(m32[c], d32, id32);
        uint32_t qw[4], qw32[4];
        int s[2] = {0, 0}, s32[2] = {0, 0};
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            qw[mm] = qw32[mm] = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int q = q8k_round(x[c][4 * mm + e], id);
                const int q32 = q8k_round(x[c][4 * mm + e], id32);
                qw[mm] |= (uint32_t)(uint8_t)(int8_t)q << (8 * e);
                qw32[mm] |= (uint32_t)(uint8_t)(int8_t)q32 << (8 * e);
                s[mm / 2] += q;
                s32[mm / 2] += q32;
            }
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            s[h] += __shfl_xor(s[h], 32, 64);
            s32[h] += __shfl_xor(s32[h], 32, 64);
        }
        if (!store)
            continue;
        const uint32_t pos = hb * HD + 32 * c + 4 * g;
#pragma unroll
        for (int mm = 0; mm < 4; mm++) {
            *(uint32_t *)(dst + 4 + pos + 8 * mm) = qw[mm];
            *(uint32_t *)(dst + 324 + pos + 8 * mm) = qw32[mm];
        }
        if (g == 0) {
            const uint32_t b32 = hb * CT + c;
            *(float *)(dst + 292 + 4 * b32) = d32;
            *(int16_t *)(dst + 612 + 2 * b32) = (int16_t)(s[0] + s[1]);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                *(int16_t *)(dst + 260 + 2 * (2 * b32 + h)) = (int16_t)s[h];
                *(int16_t *)(dst + 580 + 2 * (2 * b32 + h)) = (int16_t)s32[h];
            }
        }
    }
    if (store && g == 0 && hb == 0)
        *(float *)dst = d;
}

}  // namespace janas

#endif
