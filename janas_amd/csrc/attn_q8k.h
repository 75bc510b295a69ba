/*
 * attn_q8k.h - one Q8_K block (struct janas_block_q8k, src/llm/quant.h:
 * 283-300) from 256 numbers held one a thread by a workgroup of 256, as
 * q8k_quantize_ref does it (src/llm/quant.c:174-200, q8_32_ref :150-172):
 * d = amax / 127 and its reciprocal, rint and clamp to +-127, the sums of
 * 16 and of 32, and the same numbers again in 8 blocks of 32 with scales of
 * their own. Shared by the Q8_K pass (attn_cache.hip) and the merge that
 * quantizes its own output (attn_split.hip). Internal, device code only.
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
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    float q = rintf(x * id);
    q = q > 127.0f ? 127.0f : q < -127.0f ? -127.0f : q;
    const float d32 = m32 / 127.0f;
    const float id32 = d32 > 0.0f ? 1.0f / d32 : 0.0f;
    float q32 = rintf(x * id32);
    q32 = q32 > 127.0f ? 127.0f : q32 < -127.0f ? -127.0f : q32;
    S.blk[4 + t] = (uint8_t)(int8_t)q;
    S.blk[324 + t] = (uint8_t)(int8_t)q32;
    if (t == 0)
        *(float *)&S.blk[0] = d;
    if ((t & 31) == 0)
        *(float *)&S.blk[292 + 4 * (t / 32)] = d32;
    /* sums of 16: integers, exact in any order */
    int s = (int)q, s32 = (int)q32;
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

}  // namespace janas

#endif
