/*
 * attn_cache.hip - the device side of the rules around the KV-cache
 * attention: writing new K/V rows into the cache, preparing the queries,
 * turning cached keys back on a context shift, and putting the attention
 * output into Q8_K blocks for the next product. Each kernel follows the
 * reference's arithmetic operation for operation, so that its bits are the
 * reference's:
 *
 *   rows_kernel    qkv_item (src/llm/model_attn.c:75-146): per (token, head)
 *                  row, the rms norm (model_impl.h:635-644: a double sum of
 *                  squares in order, 1 / sqrtf(mean + eps), x * s * w), the
 *                  NeoX rotation of the first n_rot dimensions
 *                  (model_attn.c:30-39), for values optionally the weightless
 *                  norm (model_attn.c:106-113), then 8 or 16 bits with a scale
 *                  of the row's own (the largest magnitude becomes 127 or
 *                  32767, lrintf), or f16 / f32 as they are.
 *   unrotate       unrotate_row (model.c:263-290): dequantize, rotate back,
 *                  find the largest magnitude anew, requantize.
 *   q8k_kernel     q8k_quantize_ref (quant.c:174-200, q8_32_ref :150-172):
 *                  d = amax / 127, 1 / d, rint, sums of 16 and of 32.
 *
 * A row is one wave: its numbers sit in LDS, the lanes take the elementwise
 * steps and the rotation's pairs, a wave reduction (exact: a maximum) finds
 * the largest magnitude, and lane 0 alone adds the squares in the reference's
 * order - the one step whose rounding depends on order. No multiply-add is
 * fused in this file, as in the reference's build (-ffp-contract=off).
 */
#pragma clang fp contract(off)

#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_kernels.h"
#include "attn_q8k.h"

namespace janas {
namespace {

constexpr int kRowWaves = 4;    /* rows (waves) a workgroup */
constexpr int kMaxHd = 512;

__device__ __forceinline__ float wave_max(float x)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

/* 1 / sqrtf(mean of squares + eps), the sum of squares in double in the
   order of the row (model_impl.h:638-641); lane 0 computes, all get it */
__device__ float inv_rms(const float *r, uint32_t n, float eps, uint32_t lane,
                         float *slot)
{
    if (lane == 0) {
        double ss = 0.0;
        for (uint32_t i = 0; i < n; i++)
            ss += (double)r[i] * r[i];
        *slot = 1.0f / sqrtf((float)(ss / n) + eps);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return *slot;
}

/* the NeoX rotation of r[0 .. n_rot) by the token's table (model_attn.c:
   30-39), or turned back by it (back: model.c:273-277) */
__device__ void rotate(float *r, uint32_t n_rot, const float *cs,
                       const float *sn, uint32_t lane, bool back)
{
    const uint32_t half = n_rot / 2;
    for (uint32_t i = lane; i < half; i += 64) {
        const float a = r[i], b = r[i + half];
        if (!back) {
            r[i] = a * cs[i] - b * sn[i];
            r[i + half] = a * sn[i] + b * cs[i];
        } else {
            r[i] = a * cs[i] + b * sn[i];
            r[i + half] = b * cs[i] - a * sn[i];
        }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

/* r[0 .. hd) at 8 or 16 bits (or f16 / f32) into dst, the scale to *z */
__device__ void quantize_row(const float *r, uint32_t hd, int kv, void *dst,
                             float *z, uint32_t lane)
{
    float mx = 0.0f;
    for (uint32_t i = lane; i < hd; i += 64)
        mx = fmaxf(mx, fabsf(r[i]));
    mx = wave_max(mx);
    if (kv == kI8 || kv == kI16) {
        const float top = kv == kI16 ? 32767.0f : 127.0f;
        const float inv = mx > 0.0f ? top / mx : 0.0f;
        if (lane == 0)
            *z = mx / top;
        for (uint32_t i = lane; i < hd; i += 64) {
            const float q = rintf(r[i] * inv);
            if (kv == kI16)
                ((int16_t *)dst)[i] = (int16_t)q;
            else
                ((int8_t *)dst)[i] = (int8_t)q;
        }
    } else if (kv == kF16) {
        for (uint32_t i = lane; i < hd; i += 64)
            ((_Float16 *)dst)[i] = (_Float16)r[i];
    } else {
        for (uint32_t i = lane; i < hd; i += 64)
            ((float *)dst)[i] = r[i];
    }
}

/*
 * Rows of the write (qkv_item's key and value part) and of the query
 * preparation: row id = j * heads + h. For the cache write a row is a key
 * and a value; for queries the query alone, turned in place.
 */
__global__ __launch_bounds__(64 * kRowWaves) void rows_kernel(const RowArgs A)
{
    __shared__ float sK[kRowWaves][kMaxHd], sV[kRowWaves][kMaxHd];
    __shared__ float sS[kRowWaves];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t id = blockIdx.x * kRowWaves + w;
    if (id >= A.n * A.heads)
        return;
    const uint32_t j = id / A.heads, h = id % A.heads, hd = A.hd;
    const uint32_t half = A.n_rot / 2;
    const float *cs = A.cs + (size_t)j * half, *sn = A.sn + (size_t)j * half;
    float *kr = sK[w], *vr = sV[w];
    const size_t src = (size_t)id * hd;
    for (uint32_t i = lane; i < hd; i += 64)
        kr[i] = A.k[src + i];
    if (A.v)
        for (uint32_t i = lane; i < hd; i += 64)
            vr[i] = A.v[src + i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

    if (A.norm) {
        const float s = inv_rms(kr, hd, A.eps, lane, &sS[w]);
        for (uint32_t i = lane; i < hd; i += 64)
            kr[i] = kr[i] * s * A.norm[i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    rotate(kr, A.n_rot, cs, sn, lane, false);
    if (!A.kc) {
        /* the query: in place */
        for (uint32_t i = lane; i < hd; i += 64)
            A.k[src + i] = kr[i];
        return;
    }
    if (A.v_norm) {
        const float s = inv_rms(vr, hd, A.eps, lane, &sS[w]);
        for (uint32_t i = lane; i < hd; i += 64)
            vr[i] = vr[i] * s;
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    }
    const uint32_t p = A.pos0 + j, row = A.ring ? p % A.cap : p;
    const size_t at = (size_t)h * A.cap + row;
    const size_t eb = A.kv == kI8 ? 1 : A.kv == kF32 ? 4 : 2;
    quantize_row(kr, hd, A.kv, (char *)A.kc + at * hd * eb, A.kz ? A.kz + at : nullptr,
                 lane);
    quantize_row(vr, hd, A.kv, (char *)A.vc + at * hd * eb, A.vz ? A.vz + at : nullptr,
                 lane);
}

/*
 * The shift's rows: moved position i of KV head h is read from the copy
 * (rows src_first + i of the copy, mod cap for a ring), written to its new
 * row, and its key turned back by the shift's angles and quantized anew
 * (model.c:304-377; unrotate_row :263-290).
 */
__global__ __launch_bounds__(64 * kRowWaves) void shift_kernel(const ShiftArgs A)
{
    __shared__ float sK[kRowWaves][kMaxHd];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t id = blockIdx.x * kRowWaves + w;
    if (id >= A.n_kv * A.count)
        return;
    const uint32_t h = id / A.count, i = id % A.count;
    const uint32_t p = A.first + i; /* the position as it was */
    const uint32_t srow = A.ring ? p % A.cap : p - A.copy_first;
    const uint32_t drow = A.ring ? (p - A.drop) % A.cap : p - A.drop;
    const uint32_t hd = A.hd;
    const size_t eb = A.kv == kI16 ? 2 : 1, rowb = hd * eb;
    const size_t sat = (size_t)h * A.copy_rows + srow;
    const size_t dat = (size_t)h * A.cap + drow;
    /* the value row and its scale move as they are */
    for (uint32_t b = lane; b < rowb; b += 64)
        ((uint8_t *)A.v)[dat * rowb + b] = ((const uint8_t *)A.cv)[sat * rowb + b];
    float *kr = sK[w];
    const float z = A.ckz[sat];
    for (uint32_t e = lane; e < hd; e += 64) {
        const float x = A.kv == kI16 ? (float)((const int16_t *)A.ck)[sat * hd + e]
                                     : (float)((const int8_t *)A.ck)[sat * hd + e];
        kr[e] = x * z;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane == 0)
        A.vz[dat] = A.cvz[sat];
    if (A.n_rot / 2 == 0) {
        /* nothing to turn: the key row and its scale move as they are */
        for (uint32_t b = lane; b < rowb; b += 64)
            ((uint8_t *)A.k)[dat * rowb + b] = ((const uint8_t *)A.ck)[sat * rowb + b];
        if (lane == 0)
            A.kz[dat] = z;
        return;
    }
    rotate(kr, A.n_rot, A.cs, A.sn, lane, true);
    quantize_row(kr, hd, A.kv, (char *)A.k + dat * rowb, A.kz + dat, lane);
}

/*
 * One Q8_K block (256 numbers of a token's output) a workgroup of 256:
 * thread t takes number t (quant.c:174-200).
 */
__global__ __launch_bounds__(256) void q8k_kernel(const Q8kArgs A)
{
    __shared__ Q8kLds S;
    const uint32_t t = threadIdx.x, b = blockIdx.x;
    q8k_block(A.x[(size_t)b * 256 + t], t, A.y + (size_t)b * kQ8kBytes, S);
}

/* one 4-byte word a thread: tensor blockIdx.y, word i of its packed rows */
__global__ __launch_bounds__(256) void refresh_kernel(const RefreshArgs A)
{
    const uint32_t t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t w = A.words[t], per_head = A.count * w;
    if (i >= A.n_kv * per_head)
        return;
    const uint32_t h = i / per_head, r = (i % per_head) / w, e = i % w;
    const uint32_t row = (A.lo + r) % A.cap;
    A.dst[t][((size_t)h * A.cap + row) * w + e] = A.src[t][i];
}

}  // namespace

hipError_t launch_refresh(const RefreshArgs &a, hipStream_t s)
{
    uint32_t most = 0;
    for (uint32_t t = 0; t < a.n_t; t++)
        most = a.words[t] > most ? a.words[t] : most;
    const uint64_t words = (uint64_t)a.n_kv * a.count * most;
    if (a.n_t == 0 || words == 0)
        return hipSuccess;
    if (a.n_t > 4 || words > 0xFFFFFFFFull)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(refresh_kernel, dim3((uint32_t)((words + 255) / 256), a.n_t), dim3(256),
                       0, s, a);
    return hipGetLastError();
}

hipError_t launch_rows(const RowArgs &a, hipStream_t s)
{
    const uint32_t rows = a.n * a.heads;
    if (rows == 0)
        return hipSuccess;
    hipLaunchKernelGGL(rows_kernel, dim3((rows + kRowWaves - 1) / kRowWaves),
                       dim3(64 * kRowWaves), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_shift(const ShiftArgs &a, hipStream_t s)
{
    const uint32_t rows = a.n_kv * a.count;
    if (rows == 0)
        return hipSuccess;
    hipLaunchKernelGGL(shift_kernel, dim3((rows + kRowWaves - 1) / kRowWaves),
                       dim3(64 * kRowWaves), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_q8k(const Q8kArgs &a, hipStream_t s)
{
    if (a.blocks == 0)
        return hipSuccess;
    hipLaunchKernelGGL(q8k_kernel, dim3(a.blocks), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace janas
