/*
 * attn_split.hip - split-KV attention over the KV cache for CDNA4 (gfx950):
 * decode, speculative verify and blocks of up to a few dozen tokens.
 *
 * The reference computes one softmax partial per (KV head, chunk of 256
 * positions, token, query head) and merges them in chunk order
 * (src/llm/attention.c:25-36, :631-810, :870-910). This file keeps that
 * contract - chunks at absolute offsets, a partial (largest score, sum of
 * weights, weighted values) per (chunk, token, head), an ordered merge - so a
 * token's result does not depend on the block it runs in, and maps it onto
 * the GPU:
 *
 *   split kernel   one workgroup (4 waves of 64) per (sequence, KV head,
 *                  chunk, tile of 16 query rows); a query row is a (token,
 *                  query head of the KV head's group), so every K/V row of
 *                  the chunk is read once for the whole GQA group. Wave w
 *                  takes positions 64w .. 64w + 63 of the chunk.
 *   merge kernel   one wave per (token, query head, 64 columns): the ordered
 *                  merge of the chunk partials, the output gate
 *                  sigmoid(g) * o (model_attn.c:159-170) fused in.
 *
 * Scores and values run on the matrix cores (v_mfma_f32_16x16x32_f16) at
 * float accuracy: the query and the weights are split into a high and a low
 * f16 part (x = hi + lo, 22 significant bits), each scaled by a power of two
 * first so that neither part loses bits to f16's range; keys and values
 * enter as f16 planes whose sum is the cached number exactly (int8 and f16:
 * one plane; int16: 256 * (x >> 8) and x & 255; f32: hi + lo). Products are
 * exact in the MFMA and summed in f32.
 *
 *   S^T = K . Q^T   A = K rows straight from HBM (16 bytes a lane), B = the
 *                   query planes from LDS; lane l ends with the scores of
 *                   query row l % 16 at positions 4 (l / 16) + i of each
 *                   16-position tile, which is already the A layout P needs.
 *   O   = P . V     A = the weights in registers, B = V rows staged in LDS
 *                   and read back transposed with ds_read_b64_tr_b16.
 */
#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_kernels.h"

namespace janas {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kWavePos = 64;  /* positions a wave */
constexpr int kRows = 16;     /* query rows a workgroup */
constexpr int kPad = 16;      /* halves of padding an LDS row */

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

__device__ __forceinline__ h8 cat(h4 a, h4 b)
{
    return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

/* x = hi + lo, both f16; x already scaled into f16's normal range */
__device__ __forceinline__ void split_hl(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

/* ---- element types of the cache -------------------------------------- */

/*
 * Elem<T>: how 8 consecutive numbers of a K row become the A operand of
 * the score product (load8 / planes8), and how a 16-byte unit of a V row
 * becomes f16 planes in LDS (unit_planes).
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
    /* 8 numbers a unit */
    static constexpr int per_unit = 8;
    __device__ static void unit_planes(uint4 u, h8 *p)
    {
        p[0] = __builtin_bit_cast(h8, u);
    }
};

template <> struct Elem<kI8> {
    static constexpr int bytes = 1, planes = 1;
    struct Raw { uint2 a; };
    __device__ static Raw load8(const void *b, size_t i)
    {
        return Raw{*(const uint2 *)((const int8_t *)b + i)};
    }
    __device__ static h8 widen(uint32_t lo, uint32_t hi)
    {
        h8 r;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            r[e] = (_Float16)(int)(int8_t)(lo >> (8 * e));
            r[4 + e] = (_Float16)(int)(int8_t)(hi >> (8 * e));
        }
        return r;
    }
    __device__ static void planes8(const Raw &r, h8 *p)
    {
        p[0] = widen(r.a.x, r.a.y);
    }
    /* 16 numbers a unit, two groups of 8 halves */
    static constexpr int per_unit = 16;
    __device__ static void unit_planes(uint4 u, h8 *p)
    {
        p[0] = widen(u.x, u.y);
        p[1] = widen(u.z, u.w);
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
    __device__ static void split(uint4 u, h8 &hi, h8 &lo)
    {
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            int x = (int)(int16_t)(w[e / 2] >> (16 * (e % 2)));
            hi[e] = (_Float16)(float)((x >> 8) * 256);
            lo[e] = (_Float16)(x & 255);
        }
    }
    __device__ static void planes8(const Raw &r, h8 *p) { split(r.a, p[0], p[1]); }
    static constexpr int per_unit = 8;
    __device__ static void unit_planes(uint4 u, h8 *p) { split(u, p[0], p[1]); }
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
    /* 4 numbers a unit: the first half of each plane's h8 */
    static constexpr int per_unit = 4;
    __device__ static void unit_planes(uint4 u, h8 *p)
    {
        uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
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
    uint32_t x = bid % 8, k = bid / 8, q = n / 8, r = n % 8;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

__device__ __forceinline__ uint32_t row_lo(const SplitArgs &A, uint32_t pos)
{
    return A.window && pos + 1 > A.window ? pos + 1 - A.window : 0;
}

template <int T, int D> struct Shape {
    static constexpr int P = Elem<T>::planes;
    /* value columns staged at a time */
    static constexpr int VC = P == 1 ? (D < 256 ? D : 256) : (D < 128 ? D : 128);
    static constexpr int NCB = D / VC;
    static constexpr int VPITCH = VC + kPad;
    static constexpr int QPITCH = D + kPad;
    static constexpr int UPR = D * Elem<T>::bytes / 16;  /* 16-byte units a V row */
    static constexpr int NT = D / 16;                    /* output column tiles */
    static constexpr int KS = D / 32;                    /* score k-steps */
    static constexpr size_t lds_q = 2 * kRows * QPITCH * 2;
    static constexpr size_t lds_v = (size_t)kWaves * P * 32 * VPITCH * 2;
    static constexpr size_t lds_acc = (size_t)2 * NT * 64 * 16; /* two buffers */
    static constexpr size_t lds_va = lds_v > lds_acc ? lds_v : lds_acc;
};

template <int T, int D>
__global__ __launch_bounds__(256) void split_kernel(const SplitArgs A)
{
    using E = Elem<T>;
    using S = Shape<T, D>;
    constexpr int P = S::P;
    __shared__ __attribute__((aligned(16))) _Float16 sQ[2][kRows][S::QPITCH];
    /* V planes while the values are summed, then the waves' sums */
    __shared__ __attribute__((aligned(16))) char sVA[S::lds_va];
    __shared__ float sMax[kWaves][kRows], sSum[kWaves][kRows];
    __shared__ int sExp[kWaves][kRows];
    __shared__ uint32_t sLo[kRows], sHi[kRows];
    __shared__ float sQs[kRows];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t id = xcd_remap(blockIdx.x, gridDim.x);
    uint32_t si = 0;
    while (si + 1 < A.n_seqs && A.seq[si + 1].wg0 <= id)
        si++;
    const SeqDesc &sq = A.seq[si];
    const uint32_t G = A.group, hd = A.hd;
    const uint32_t local = id - sq.wg0;
    const uint32_t rt = local % sq.rtiles;
    const uint32_t c = sq.c0 + (local / sq.rtiles) % sq.span;
    const uint32_t kvh = local / sq.rtiles / sq.span;
    const uint32_t R = sq.n * G, r0 = rt * kRows;
    const uint32_t t0 = c * kChunk;

    /* the tile's tokens see [lo(first), last(final)]: nothing of this chunk
       means no partial is needed (the merge does not read it) */
    {
        uint32_t jf = r0 / G, jl = (r0 + kRows < R ? r0 + kRows : R) - 1;
        jl /= G;
        uint32_t lo = row_lo(A, sq.pos0 + jf);
        uint32_t hi = sq.last ? sq.last[jl] : sq.pos0 + jl;
        if (t0 > hi || t0 + kChunk <= lo)
            return;
    }

    /* rows: visible range, and the query planes scaled by 2^e so that the
       largest |q| of the row lies in [2^13, 2^14) */
    if (tid < kRows) {
        uint32_t r = r0 + tid;
        uint32_t lo = 1, hi = 0;
        if (r < R) {
            uint32_t j = r / G;
            lo = row_lo(A, sq.pos0 + j);
            hi = sq.last ? sq.last[j] : sq.pos0 + j;
        }
        sLo[tid] = lo;
        sHi[tid] = hi;
    }
    {
        /* 16 threads a row, hd / 16 numbers each (hd a multiple of 8:
           columns past hd are zero) */
        const uint32_t qr = tid >> 4, ql = tid & 15, r = r0 + qr;
        const float *qrow = nullptr;
        if (r < R) {
            uint32_t j = r / G, h = kvh * G + r % G;
            qrow = sq.q + ((size_t)j * A.n_head + h) * hd;
        }
        constexpr int PER = D / 16;
        float v[PER];
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < PER; e++) {
            uint32_t col = ql * PER + e;
            v[e] = qrow && col < hd ? qrow[col] : 0.0f;
            mx = fmaxf(mx, fabsf(v[e]));
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1)
            mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        int ex = 0;
        if (mx > 0.0f && mx < INFINITY) {
            frexpf(mx, &ex);
            ex = 14 - ex;
        }
        const float up = ldexpf(1.0f, ex);
#pragma unroll
        for (int e = 0; e < PER; e++) {
            _Float16 hi, lo;
            split_hl(v[e] * up, hi, lo);
            sQ[0][qr][ql * PER + e] = hi;
            sQ[1][qr][ql * PER + e] = lo;
        }
        if (ql == 0)
            sQs[qr] = ldexpf(1.0f, -ex);
    }
    __syncthreads();

    const uint32_t p0w = t0 + w * kWavePos;
    /* does any row see a position of this wave? */
    const uint32_t lo_all = sLo[0], hi_all = sHi[(R - r0 < kRows ? R - r0 : kRows) - 1];
    const bool active = p0w < sq.end && p0w <= hi_all && p0w + kWavePos > lo_all;
    const size_t head_row = (size_t)kvh * sq.cap;
    /* rows of the chunk in the cache: contiguous, a ring's too (cap is a
       multiple of the chunk) */
    const size_t crow = head_row + (A.ring ? t0 % sq.cap : t0);
    const uint32_t g16 = lane >> 4, l16 = lane & 15;

    /* ---- loads: the wave's K rows in A layout, its V rows coalesced ---- */
    typename E::Raw kraw[4][S::KS];
    uint4 vraw[S::UPR];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) {
        const uint32_t p = p0w + 16 * mt + l16;
        const bool ok = active && p < sq.end;
        const size_t base = (crow + (p - t0)) * hd;
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            const uint32_t d0 = 32 * s + 8 * g16;
            if (ok && d0 < hd)
                kraw[mt][s] = E::load8(sq.k, base + d0);
            else
                kraw[mt][s] = typename E::Raw{};
        }
    }
#pragma unroll
    for (int i = 0; i < S::UPR; i++) {
        const uint32_t u = i * 64 + lane, row = u / S::UPR, cu = u % S::UPR;
        const uint32_t p = p0w + row, col = cu * E::per_unit;
        vraw[i] = uint4{0, 0, 0, 0};
        if (active && p < sq.end && col < hd) {
            const char *src = (const char *)sq.v +
                              ((crow + (p - t0)) * hd + col) * E::bytes;
            if (col + E::per_unit <= hd) {
                vraw[i] = *(const uint4 *)src;
            } else {
                /* int8 rows of 8 mod 16 numbers: the last unit is half */
                uint2 h = *(const uint2 *)src;
                vraw[i].x = h.x;
                vraw[i].y = h.y;
            }
        }
    }

    /* ---- scores ---- */
    f4 sacc[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
        sacc[mt] = f4{0, 0, 0, 0};
    if (active) {
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            h8 qb[2];
            qb[0] = *(const h8 *)&sQ[0][l16][32 * s + 8 * g16];
            qb[1] = *(const h8 *)&sQ[1][l16][32 * s + 8 * g16];
#pragma unroll
            for (int mt = 0; mt < 4; mt++) {
                h8 ka[P];
                E::planes8(kraw[mt][s], ka);
#pragma unroll
                for (int kp = 0; kp < P; kp++)
#pragma unroll
                    for (int qp = 0; qp < 2; qp++)
                        if (use_pair<T>(kp, qp))
                            sacc[mt] = mfma(ka[kp], qb[qp], sacc[mt]);
            }
        }
    }

    /* scale, mask; lane l holds row l16 at positions 16 mt + 4 g16 + i */
    const uint32_t rlo = sLo[l16], rhi = sHi[l16];
    const float qs = sQs[l16] * A.scale;
    const bool scaled = T == kI8 || T == kI16;
    float sv[4][4];
    float m = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t p = p0w + 16 * mt + 4 * g16 + i;
            float s = -INFINITY;
            if (active && p >= rlo && p <= rhi && p < sq.end) {
                s = sacc[mt][i] * qs;
                if (scaled)
                    s *= sq.ks[crow + (p - t0)];
            }
            sv[mt][i] = s;
            m = fmaxf(m, s);
        }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    if (lane < 16)
        sMax[w][lane] = m;
    __syncthreads();
    const float mc = fmaxf(fmaxf(sMax[0][l16], sMax[1][l16]),
                           fmaxf(sMax[2][l16], sMax[3][l16]));

    /* weights: e^(s - max) of the chunk, 0 when not visible or below
       e^-80 (attention.c:574-590); their sum; then the value scale */
    float lsum = 0.0f, pmax = 0.0f;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = sv[mt][i];
            float pw = 0.0f;
            if (s != -INFINITY && s - mc >= -80.0f)
                pw = expf(s - mc);
            lsum += pw;
            if (scaled && pw != 0.0f) {
                const uint32_t p = p0w + 16 * mt + 4 * g16 + i;
                pw *= sq.vs[crow + (p - t0)];
            }
            sv[mt][i] = pw;
            pmax = fmaxf(pmax, pw);
        }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    pmax = fmaxf(pmax, __shfl_xor(pmax, 16, 64));
    pmax = fmaxf(pmax, __shfl_xor(pmax, 32, 64));
    int pe = 0;
    if (pmax > 0.0f && pmax < INFINITY) {
        frexpf(pmax, &pe);
        pe = 14 - pe;
    }
    if (lane < 16) {
        sSum[w][lane] = lsum;
        sExp[w][lane] = pe;
    }
    /* A operands of the value product: k-slot j of k-step kk is position
       32 kk + 4 g16 + j (j < 4) or 32 kk + 16 + 4 g16 + j - 4 */
    h8 pa[2][2];
    {
        const float up = ldexpf(1.0f, pe);
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                _Float16 hi, lo;
                split_hl(sv[2 * kk + j / 4][j % 4] * up, hi, lo);
                pa[kk][0][j] = hi;
                pa[kk][1][j] = lo;
            }
    }

    /* ---- values ---- */
    f4 o[S::NT];
#pragma unroll
    for (int nt = 0; nt < S::NT; nt++)
        o[nt] = f4{0, 0, 0, 0};
    _Float16 *vw = (_Float16 *)sVA + (size_t)w * P * 32 * S::VPITCH;
    if (active) {
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int cb = 0; cb < S::NCB; cb++) {
                /* the wave's rows 32 kk .. 32 kk + 31, columns of block cb,
                   as f16 planes */
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int i = 0; i < S::UPR; i++) {
                    const uint32_t row = (i * 64) / S::UPR;
                    if ((int)(row / 32) != kk)
                        continue;
                    const uint32_t u = i * 64 + lane, rr = u / S::UPR - 32 * kk;
                    const int col = (int)(u % S::UPR) * E::per_unit - cb * S::VC;
                    if (col < 0 || col >= S::VC)
                        continue;
                    h8 pl[2];
                    E::unit_planes(vraw[i], pl);
#pragma unroll
                    for (int pp = 0; pp < P; pp++) {
                        _Float16 *dst = vw + ((size_t)pp * 32 + rr) * S::VPITCH + col;
                        if (T == kF32) {
                            *(h4 *)dst = h4{pl[pp][0], pl[pp][1], pl[pp][2], pl[pp][3]};
                        } else if (T == kI8) {
                            *(h8 *)dst = pl[0];
                            *(h8 *)(dst + 8) = pl[1];
                        } else {
                            *(h8 *)dst = pl[pp];
                        }
                    }
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int ntl = 0; ntl < S::VC / 16; ntl++) {
                    const int nt = cb * (S::VC / 16) + ntl;
                    if (16 * nt >= (int)hd)
                        continue;
                    const int tc = 16 * ntl + 4 * (l16 & 3);
                    const int tr = 4 * g16 + (l16 >> 2);
#pragma unroll
                    for (int pp = 0; pp < P; pp++) {
                        const _Float16 *src = vw + (size_t)pp * 32 * S::VPITCH;
                        h8 vb = cat(lds_read_tr(src + tr * S::VPITCH + tc),
                                    lds_read_tr(src + (16 + tr) * S::VPITCH + tc));
#pragma unroll
                        for (int ap = 0; ap < 2; ap++)
                            if (use_pair<T>(pp, ap))
                                o[nt] = mfma(pa[kk][ap], vb, o[nt]);
                    }
                }
            }
    }

    /* ---- the waves' sums, (w0 + w1) + (w2 + w3), back to 2^0 ---- */
    float down[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        down[i] = ldexpf(1.0f, -sExp[w][4 * g16 + i]);
#pragma unroll
    for (int nt = 0; nt < S::NT; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            o[nt][i] *= down[i];
    __syncthreads();
    f4 *sacc4 = (f4 *)sVA; /* two buffers of [NT][64] */
    if (w == 1 || w == 3) {
        f4 *dst = sacc4 + (size_t)(w / 2) * S::NT * 64;
#pragma unroll
        for (int nt = 0; nt < S::NT; nt++)
            dst[nt * 64 + lane] = o[nt];
    }
    __syncthreads();
    if (w == 0 || w == 2) {
        const f4 *src = sacc4 + (size_t)(w / 2) * S::NT * 64;
#pragma unroll
        for (int nt = 0; nt < S::NT; nt++)
            o[nt] += src[nt * 64 + lane];
    }
    __syncthreads();
    if (w == 2) {
#pragma unroll
        for (int nt = 0; nt < S::NT; nt++)
            sacc4[nt * 64 + lane] = o[nt];
    }
    __syncthreads();
    if (w != 0)
        return;
#pragma unroll
    for (int nt = 0; nt < S::NT; nt++)
        o[nt] += sacc4[nt * 64 + lane];

    /* ---- the partial of each row that sees the chunk ---- */
    const uint64_t prow = sq.part0 + ((uint64_t)kvh * sq.span + (c - sq.c0)) * R + r0;
    if (lane < kRows && r0 + lane < R) {
        const float l = (sSum[0][lane] + sSum[1][lane]) + (sSum[2][lane] + sSum[3][lane]);
        const float mx = fmaxf(fmaxf(sMax[0][lane], sMax[1][lane]),
                               fmaxf(sMax[2][lane], sMax[3][lane]));
        A.part_ml[(prow + lane) * 2] = mx;
        A.part_ml[(prow + lane) * 2 + 1] = l;
    }
#pragma unroll
    for (int nt = 0; nt < S::NT; nt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 4 * g16 + i, col = 16 * nt + l16;
            if (r0 + row < R && col < hd)
                A.part_acc[(prow + row) * hd + col] = o[nt][i];
        }
}

/* merge of the chunks of (token j, query head h), 64 columns a wave, in
   chunk order (attention.c:870-910); then the gate */
__global__ __launch_bounds__(64) void merge_kernel(const SplitArgs A)
{
    const uint32_t id = blockIdx.x, lane = threadIdx.x;
    uint32_t si = 0;
    while (si + 1 < A.n_seqs && A.seq[si + 1].mg0 <= id)
        si++;
    const SeqDesc &sq = A.seq[si];
    const uint32_t hd = A.hd, G = A.group, nd = (hd + 63) / 64;
    const uint32_t local = id - sq.mg0, db = local % nd;
    const uint32_t h = (local / nd) % A.n_head, j = local / nd / A.n_head;
    const uint32_t kvh = h / G, r = j * G + h % G, R = sq.n * G;
    const uint32_t pos = sq.pos0 + j;
    const uint32_t lo = row_lo(A, pos), hi = sq.last ? sq.last[j] : pos;
    const uint32_t clo = lo / kChunk, chi = hi / kChunk;
    const uint64_t base = sq.part0 + (uint64_t)kvh * sq.span * R + r;
    float mx = -INFINITY;
    for (uint32_t cc = clo; cc <= chi; cc++)
        mx = fmaxf(mx, A.part_ml[(base + (uint64_t)(cc - sq.c0) * R) * 2]);
    const uint32_t col = db * 64 + lane;
    float sum = 0.0f, acc = 0.0f;
    for (uint32_t cc = clo; cc <= chi; cc++) {
        const uint64_t pr = base + (uint64_t)(cc - sq.c0) * R;
        const float wgt = expf(A.part_ml[pr * 2] - mx);
        sum += wgt * A.part_ml[pr * 2 + 1];
        if (col < hd)
            acc = fmaf(wgt, A.part_acc[pr * hd + col], acc);
    }
    if (col >= hd)
        return;
    float o = acc * (1.0f / sum);
    const size_t oi = ((size_t)j * A.n_head + h) * hd + col;
    if (A.gate_mode == kGateElem)
        o *= 1.0f / (1.0f + expf(-sq.gate[oi]));
    else if (A.gate_mode == kGateHead)
        o *= 1.0f / (1.0f + expf(-sq.gate[(size_t)j * A.n_head + h]));
    sq.out[oi] = o;
}

template <int T, int D>
hipError_t launch_t(const SplitArgs &a, hipStream_t s)
{
    hipLaunchKernelGGL((split_kernel<T, D>), dim3(a.n_wg), dim3(256), 0, s, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_d(uint32_t hd, const SplitArgs &a, hipStream_t s)
{
    if (hd <= 64)
        return launch_t<T, 64>(a, s);
    if (hd <= 128)
        return launch_t<T, 128>(a, s);
    if (hd <= 256)
        return launch_t<T, 256>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

int split_supported(int kv, uint32_t hd)
{
    return kv >= kI8 && kv <= kF32 && hd >= 8 && hd % 8 == 0 && hd <= 256;
}

hipError_t launch_split(int kv, const SplitArgs &a, hipStream_t s)
{
    switch (kv) {
    case kI8:
        return launch_d<kI8>(a.hd, a, s);
    case kI16:
        return launch_d<kI16>(a.hd, a, s);
    case kF16:
        return launch_d<kF16>(a.hd, a, s);
    case kF32:
        return launch_d<kF32>(a.hd, a, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_merge(const SplitArgs &a, uint32_t n_wg, hipStream_t s)
{
    hipLaunchKernelGGL(merge_kernel, dim3(n_wg), dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace janas
