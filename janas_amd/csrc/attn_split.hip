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
 *   split kernel   one workgroup (8 waves of 64) per (sequence, KV head,
 *                  chunk, tile of 16 query rows); a query row is a (token,
 *                  query head of the KV head's group), so every K/V row of
 *                  the chunk is read once for the whole GQA group. Wave w
 *                  loads positions 32 w .. 32 w + 31 of K at once, then of V
 *                  as soon as its K is in, with contiguous 16-byte loads,
 *                  stages them through its own LDS region
 *                  into MFMA operand order, and computes a one-shot softmax
 *                  over its 32 positions; the 8 waves' partials are combined
 *                  in LDS in a fixed order into the chunk's exact partial.
 *                  Workgroups are renumbered so each XCD takes a contiguous
 *                  range (neighbouring chunks share an L2).
 *   merge kernel   one workgroup per (token, query head, 32 or 128 columns): the
 *                  ordered merge of the chunk partials (8 groups of chunks in
 *                  parallel, each in batches of 16, combined in a fixed
 *                  tree), the output gate sigmoid(g) * o (model_attn.c:
 *                  159-170) fused in.
 *
 * Scores and values run on the matrix cores (v_mfma_f32_16x16x32_f16) at
 * float accuracy: the query and the weights are split into a high and a low
 * f16 part (x = hi + lo, 22 significant bits), each scaled by a power of two
 * first so that neither part loses bits to f16's range; keys and values
 * enter as f16 planes whose sum is the cached number exactly (int8 and f16:
 * one plane; int16: 256 * (x >> 8) and x & 255; f32: hi + lo). Products are
 * exact in the MFMA and summed in f32; for an f32 cache the product of the
 * two low parts (below 2^-22 of a term) is left out.
 *
 *   S^T = K . Q^T   wave w scores its 32 positions as two 16-position
 *                   tiles (A = K rows from LDS, B = the query planes from
 *                   LDS); lane l holds row l % 16 at positions 4 (l / 16) + i
 *                   of each tile - already the A layout of the value product.
 *   O   = P . V     the weights stay in registers as A operands; V is read
 *                   back transposed with ds_read_b64_tr_b16 (16-bit types,
 *                   and int8 rows widened to f16 as they are staged) or
 *                   gathered (f32 planes); every wave sums all value
 *                   columns over its positions.
 */
#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_elem.h"

namespace janas {
namespace {

/* ---- the split kernel: one shot, every load in flight at once -------- */

/*
 * A workgroup is 8 waves (2 a SIMD); wave w takes positions 32 w .. 32 w + 31
 * of the chunk. Every wave issues its loads in two bursts - the tile's
 * query and its 32 K rows at once, then its 32 V rows as soon as the K rows
 * are in - 16 contiguous bytes a lane (1 KB a wave instruction, the pattern
 * that streams HBM fastest), so the chunk's 128 KB of K (head_dim 256, f16)
 * are in flight from the first microsecond and the scores overlap the V
 * transfer. Asking for V earlier - with K, or right after the query
 * barrier - measured slower (17.8 and 16.4 us against 15.7 us on a 32k
 * decode): K then lands later and the scores no longer overlap anything.
 * K rows pass through a private LDS region to become the MFMA's A operand;
 * the same region then holds the V rows, read back transposed. A wave's
 * softmax is one shot over its 32 positions; the 8 waves' (max, sum,
 * values) are combined at the end. No load goes straight to LDS: with
 * those in flight the compiler makes every barrier and every use of a
 * register load wait for all of them. In a decode K and V are read once,
 * so their loads are nontemporal (15.7 against 16.6 us on the 32k decode);
 * the row tiles of a block of tokens read a chunk each, and plain loads
 * keep it in L2 for them (the NT instance is the decode one: a branch
 * between the two in one kernel cost the decode 6 %).
 */
constexpr int kWaves = 8;
constexpr int kWavePos = kChunk / kWaves; /* 32 */

template <int T, int D> struct Shape {
    static constexpr int EB = Elem<T>::bytes;
    static constexpr int P = Elem<T>::planes;
    static constexpr bool SCALED = T == kI8 || T == kI16;
    static constexpr int RB = D * EB;               /* bytes of a (padded) row */
    static constexpr int WBYTES = kWavePos * RB;    /* a wave's K (or V) rows */
    static constexpr int UNITS = WBYTES / 1024;     /* 16-byte loads a lane */
    static constexpr int KS = D / 32;               /* score k-steps */
    static constexpr int NT = D / 16;               /* output column tiles */
    static constexpr int QV = D / 128 > 0 ? D / 128 : 1; /* q float4 a lane */
    static constexpr int QP = D + 16;               /* halves a q row in LDS */
    /* a wave's region: its rows (int8 values widened to f16: twice the
       bytes), later its sums ([NT][64] f4) */
    static constexpr int RROWS = (T == kI8 ? 2 : 1) * UNITS * kBlk;
    static constexpr int RSUM = NT * 64 * 16;
    static constexpr int REGION = RROWS > RSUM ? RROWS : RSUM;
    static constexpr int VRB = T == kI8 ? 2 * RB : RB; /* bytes of a V row in LDS */
};

/* ONE: a launch of one sequence - its descriptor is read at fixed offsets
   with the rest of the arguments, not after the launch's sequence count (a
   round trip to the arguments earlier for the first loads, 0.4 us a
   decode) */
template <int T, int D, bool NT, bool ONE = false>
__global__ __launch_bounds__(512) void split_kernel(const SplitArgs A)
{
    using E = Elem<T>;
    using S = Shape<T, D>;
    constexpr int P = S::P;
    static_assert(S::UNITS >= 1 && S::WBYTES % 1024 == 0, "whole kilobytes a wave");
    static_assert(2 * S::UNITS + 2 * S::QV + 16 < 63, "the loads fit the wait counter");
    __shared__ __attribute__((aligned(16))) char sW[kWaves * S::REGION];
    __shared__ __attribute__((aligned(16))) _Float16 sQ[2][kRows][S::QP];
    __shared__ float sMax[kWaves][kRows], sSum[kWaves][kRows];
    __shared__ float sQs[kRows];
    __shared__ uint32_t sLo[kRows], sHi[kRows];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t g16 = lane >> 4, l16 = lane & 15;
    const uint32_t id = xcd_remap(blockIdx.x, A.n_wg);
    uint32_t si = 0;
    if constexpr (!ONE)
        si = seq_index(A, &SeqDesc::wg0, id);
    const SeqDesc &sq = A.seq[si];
    const uint32_t G = A.group, hd = A.hd;
    /* the cache and query addresses with the first batch of argument loads
       (otherwise the compiler asks for them just before the big loads, one
       round trip later) */
    asm volatile("" ::"s"(sq.k), "s"(sq.v), "s"(sq.q), "s"(A.n_head));
    const uint32_t local = id - sq.wg0;
    const uint32_t rt = local % sq.rtiles;
    const uint32_t c = sq.c0 + (local / sq.rtiles) % sq.span;
    const uint32_t kvh = local / sq.rtiles / sq.span;
    const uint32_t R = sq.n * G, r0 = rt * kRows;
    const uint32_t t0 = c * kChunk;

    /* the tile's tokens see [lo(first), last(final)]: nothing of this chunk
       means no partial is needed (the merge does not read it) */
    const uint32_t rows_here = R - r0 < kRows ? R - r0 : kRows;
    const uint32_t jf = r0 / G, jl = (r0 + rows_here - 1) / G;
    const uint32_t lo_all = row_lo(A, sq.pos0 + jf);
    const uint32_t hi_all = sq.last ? sq.last[jl] : sq.pos0 + jl;
    if (t0 > hi_all || t0 + kChunk <= lo_all)
        return;
    const uint32_t p0w = t0 + w * kWavePos;
    /* does any row see a position of this wave? (uniform in the wave) */
    const bool active = p0w <= hi_all && p0w + kWavePos > lo_all;
    const uint32_t plast = sq.end - 1;
    /* rows of the chunk in the cache: contiguous, a ring's too (cap is a
       multiple of the chunk) */
    const size_t crow = (size_t)kvh * sq.cap + (A.ring ? t0 % sq.cap : t0);

    /* rows: visible range (read before the big loads, whose count a wait
       for last[] would otherwise include) */
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

    /* ---- every load, unconditional: rows past the call read its last
       row, columns past hd column 0 - valid memory whose numbers are masked
       or multiplied by zero weights ---- */
    /* q: wave w takes rows 2 w and 2 w + 1, lane l row 2 w + l / 32 */
    const uint32_t qrow = 2 * w + (lane >> 5);
    float4 qv[S::QV];
    bool qok[S::QV];
    {
        const uint32_t r = r0 + qrow < R ? r0 + qrow : r0;
        const uint32_t j = r / G, h = kvh * G + r % G;
        const float *src = sq.q + ((size_t)j * A.n_head + h) * hd;
#pragma unroll
        for (int i = 0; i < S::QV; i++) {
            const uint32_t col = 4 * ((lane & 31) + 32 * i);
            qok[i] = r0 + qrow < R && col < hd && col < D;
            qv[i] = *(const float4 *)(src + (col < hd ? col : 0));
        }
    }
    /* K and V: byte 1024 i + 16 lane of the wave's 32 rows */
    /* the chunk's rows start at one address per block; a lane's byte
       offset from it stays below kChunk rows, 32 bits (the loads take the
       base in scalar registers and the offset in one vector register) */
    u4 kraw[S::UNITS], vraw[S::UNITS];
    const uint32_t rbytes = hd * S::EB, rlast = plast - t0;
    const char *const kbase = (const char *)sq.k + crow * rbytes;
    const char *const vbase = (const char *)sq.v + crow * rbytes;
    uint32_t off[S::UNITS];
    bool back[S::UNITS]; /* int8 rows of 8 mod 16 bytes: unit_at() */
#pragma unroll
    for (int i = 0; i < S::UNITS; i++) {
        const uint32_t byte = i * 1024 + lane * 16;
        const uint32_t row = byte / S::RB, cb = byte % S::RB;
        const uint32_t p = w * kWavePos + row; /* from t0 */
        uint32_t at;
        if constexpr (S::EB == 1) {
            at = unit_at(cb, hd, back[i]);
        } else {
            at = cb < hd * S::EB ? cb : 0;
            back[i] = false;
        }
        off[i] = __umul24(p < rlast ? p : rlast, rbytes) + at;
    }
    /* NT: every chunk is read by one row tile (decode), once: nontemporal;
       one that several row tiles read (blocks of tokens) should stay in L2 */
    if constexpr (NT) {
#pragma unroll
        for (int i = 0; i < S::UNITS; i++)
            kraw[i] = __builtin_nontemporal_load((const u4 *)(kbase + off[i]));
    } else {
#pragma unroll
        for (int i = 0; i < S::UNITS; i++)
            kraw[i] = *(const u4 *)(kbase + off[i]);
    }
    /* the scales of the lane's positions 16 mt + 4 g16 + i */
    float ks8[8], vs8[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        ks8[e] = 1.0f;
        vs8[e] = 1.0f;
    }
    if constexpr (S::SCALED) {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t p = w * kWavePos + 16 * (e / 4) + 4 * g16 + e % 4;
            const uint32_t at = p < rlast ? p : rlast;
            ks8[e] = sq.ks[crow + at];
            vs8[e] = sq.vs[crow + at];
        }
    }

    /* ---- q: scaled by 2^e so that the row's largest |q| lies in
       [2^13, 2^14), split into f16 planes, into LDS ---- */
    {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < S::QV; i++)
            if (qok[i])
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(qv[i].x), fabsf(qv[i].y)),
                                     fmaxf(fabsf(qv[i].z), fabsf(qv[i].w))));
#pragma unroll
        for (int o2 = 1; o2 < 32; o2 <<= 1)
            mx = fmaxf(mx, __shfl_xor(mx, o2, 64));
        int ex = 0;
        if (mx > 0.0f && mx < INFINITY) {
            frexpf(mx, &ex);
            ex = 14 - ex;
        }
        const float up = ldexpf(1.0f, ex);
#pragma unroll
        for (int i = 0; i < S::QV; i++) {
            const uint32_t col = 4 * ((lane & 31) + 32 * i);
            if (col >= D)
                continue;
            const float x[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 hi, lo;
                split_hl(qok[i] ? x[e] * up : 0.0f, hi, lo);
                sQ[0][qrow][col + e] = hi;
                sQ[1][qrow][col + e] = lo;
            }
        }
        if ((lane & 31) == 0)
            sQs[qrow] = ldexpf(1.0f, -ex);
    }
    __syncthreads();

    /* ---- K into the wave's region, then the scores of its two tiles of
       16 positions (A = K rows 16 mt + l16, B = the query planes) ---- */
    char *const reg = sW + (size_t)w * S::REGION;
#pragma unroll
    for (int i = 0; i < S::UNITS; i++)
        *(u4 *)(reg + blk_off(i * 1024 + lane * 16)) =
            S::EB == 1 ? unit_fix(kraw[i], back[i]) : kraw[i];
    /* V once the wave's K is in */
    if constexpr (NT) {
#pragma unroll
        for (int i = 0; i < S::UNITS; i++)
            vraw[i] = __builtin_nontemporal_load((const u4 *)(vbase + off[i]));
    } else {
#pragma unroll
        for (int i = 0; i < S::UNITS; i++)
            vraw[i] = *(const u4 *)(vbase + off[i]);
    }
    f4 sacc[2];
    {
        f4 sa[2][2] = {{f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}, {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}};
#pragma unroll
        for (int k = 0; k < S::KS; k++) {
            const h8 qb0 = *(const h8 *)&sQ[0][l16][32 * k + 8 * g16];
            const h8 qb1 = *(const h8 *)&sQ[1][l16][32 * k + 8 * g16];
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const uint32_t bo = (16 * mt + l16) * S::RB + (32 * k + 8 * g16) * S::EB;
                typename E::Raw kr;
                if constexpr (S::EB == 1) {
                    kr.a = *(const uint2 *)(reg + blk_off(bo));
                } else if constexpr (S::EB == 2) {
                    kr.a = *(const uint4 *)(reg + blk_off(bo));
                } else {
                    kr.a = *(const uint4 *)(reg + blk_off(bo));
                    kr.b = *(const uint4 *)(reg + blk_off(bo + 16));
                }
                h8 ka[P];
                E::planes8(kr, ka);
#pragma unroll
                for (int kp = 0; kp < P; kp++) {
                    if (use_pair<T>(kp, 0))
                        sa[mt][0] = mfma(ka[kp], qb0, sa[mt][0]);
                    if (use_pair<T>(kp, 1))
                        sa[mt][1] = mfma(ka[kp], qb1, sa[mt][1]);
                }
            }
        }
        sacc[0] = sa[0][0] + sa[0][1];
        sacc[1] = sa[1][0] + sa[1][1];
    }

    /* ---- the wave's softmax, one shot over its 32 positions: lane l holds
       row l16 at positions 16 mt + 4 g16 + i ---- */
    const uint32_t rlo = sLo[l16], rhi = sHi[l16];
    const float qs = sQs[l16] * A.scale;
    float sv[8];
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const uint32_t p = p0w + 16 * (e / 4) + 4 * g16 + e % 4;
        float x = -INFINITY;
        if (active && p >= rlo && p <= rhi && p <= plast) {
            x = sacc[e / 4][e % 4] * qs;
            if constexpr (S::SCALED)
                x *= ks8[e];
        }
        sv[e] = x;
        m = fmaxf(m, x);
    }
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    /* the weights' power of two: the largest (e^0 times the largest value
       scale of the wave's positions) lands in [2^12, 2^13) */
    int pe = 13;
    if constexpr (S::SCALED) {
        float vm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++)
            vm = fmaxf(vm, vs8[e]);
        vm = fmaxf(vm, __shfl_xor(vm, 16, 64));
        vm = fmaxf(vm, __shfl_xor(vm, 32, 64));
        int ev = 0;
        if (vm > 0.0f && vm < INFINITY)
            frexpf(vm, &ev);
        pe = 13 - ev;
    }
    const float up = ldexpf(1.0f, pe);
    float lsum = 0.0f;
    /* A operand of the value product: k-slot j is position 4 g16 + j (j < 4)
       or 16 + 4 g16 + j - 4 - the scores' own layout */
    h8 pa[2];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float x = sv[e];
        float pw = 0.0f;
        if (x != -INFINITY && x - m >= -80.0f)
            pw = expf(x - m);
        lsum += pw;
        _Float16 hi, lo;
        split_hl(pw * vs8[e] * up, hi, lo);
        pa[0][e] = hi;
        pa[1][e] = lo;
    }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);

    /* ---- V into the same region (the wave's reads of K are done: LDS
       serves a wave in order), then the values ---- */
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if constexpr (T == kI8) {
        /* int8 values widened to f16 rows (exact), read back transposed
           like the 16-bit types */
#pragma unroll
        for (int i = 0; i < S::UNITS; i++) {
            const uint32_t byte = i * 1024 + lane * 16;
            const uint32_t row = byte / S::RB, cb = byte % S::RB;
            const u4 x = unit_fix(vraw[i], back[i]);
            *(h8 *)(reg + blk_off(row * S::VRB + cb * 2)) = Elem<kI8>::widen(x.x, x.y);
            *(h8 *)(reg + blk_off(row * S::VRB + cb * 2 + 16)) = Elem<kI8>::widen(x.z, x.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < S::UNITS; i++)
            *(u4 *)(reg + blk_off(i * 1024 + lane * 16)) =
                S::EB == 1 ? unit_fix(vraw[i], back[i]) : vraw[i];
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    f4 o[S::NT];
#pragma unroll
    for (int t = 0; t < S::NT; t++)
        o[t] = f4{0, 0, 0, 0};
    {
        h8 vbp[S::NT][P];
#pragma unroll
        for (int t = 0; t < S::NT; t++) {
            if constexpr (S::EB == 2 || T == kI8) {
                const uint32_t r1 = 4 * g16 + (l16 >> 2);
                const uint32_t cc = 16 * t + 4 * (l16 & 3);
                const h4 x = lds_read_tr((const _Float16 *)(reg + blk_off(r1 * S::VRB + cc * 2)));
                const h4 y = lds_read_tr((const _Float16 *)(reg + blk_off((r1 + 16) * S::VRB + cc * 2)));
                const h8 xy = h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                if constexpr (T == kF16 || T == kI8)
                    vbp[t][0] = xy;
                else
                    Elem<kI16>::split(__builtin_bit_cast(uint4, xy), vbp[t][0], vbp[t][1]);
            } else {
                /* f32: the 8 positions of one column, one by one */
                const uint32_t cc = 16 * t + l16;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t rv = 16 * (e / 4) + 4 * g16 + e % 4;
                    const uint32_t bo = blk_off(rv * S::RB + cc * S::EB);
                    _Float16 hi, lo;
                    split_hl(*(const float *)(reg + bo), hi, lo);
                    vbp[t][0][e] = hi;
                    vbp[t][1][e] = lo;
                }
            }
        }
        /* columns past hd hold column 0's numbers: their sums are dropped */
#pragma unroll
        for (int ap = 0; ap < 2; ap++)
#pragma unroll
            for (int pp = 0; pp < P; pp++)
                if (use_pair<T>(pp, ap))
#pragma unroll
                    for (int t = 0; t < S::NT; t++)
                        o[t] = mfma(pa[ap], vbp[t][pp], o[t]);
    }

    /* ---- the 8 waves combined: chunk max M, wave w's sums weighted by
       e^(m_w - M) (and back to 2^0), then wave w adds up its column tiles
       over the waves in a fixed order and writes them ---- */
    if (lane < 16) {
        sMax[w][lane] = m;
        sSum[w][lane] = lsum;
    }
    __syncthreads();
    float mc = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ww++)
        mc = fmaxf(mc, sMax[ww][l16]);
    {
        const float f = (m == -INFINITY ? 0.0f : expf(m - mc)) * ldexpf(1.0f, -pe);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float fi = __shfl(f, 4 * g16 + i, 64);
#pragma unroll
            for (int t = 0; t < S::NT; t++)
                o[t][i] *= fi;
        }
    }
    /* the region's V reads are done (in order); sums as [NT][64] f4 */
    f4 *mine = (f4 *)reg;
#pragma unroll
    for (int t = 0; t < S::NT; t++)
        mine[t * 64 + lane] = o[t];
    __syncthreads();
    const uint64_t prow = sq.part0 + ((uint64_t)kvh * sq.span + (c - sq.c0)) * R + r0;
    for (uint32_t t = w; t < (uint32_t)S::NT; t += kWaves) {
        f4 part[kWaves];
#pragma unroll
        for (int ww = 0; ww < kWaves; ww++)
            part[ww] = ((const f4 *)(sW + (size_t)ww * S::REGION))[t * 64 + lane];
        const f4 sum = ((part[0] + part[1]) + (part[2] + part[3])) +
                       ((part[4] + part[5]) + (part[6] + part[7]));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t row = 4 * g16 + i, col = 16 * t + l16;
            if (r0 + row < R && col < hd)
                A.part_acc[(prow + row) * hd + col] = sum[i];
        }
    }
    if (w == 0 && lane < kRows && r0 + lane < R) {
        float l = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kWaves; ww++) {
            const float mw = sMax[ww][lane];
            l += (mw == -INFINITY ? 0.0f : expf(mw - mc)) * sSum[ww][lane];
        }
        A.part_ml[(prow + lane) * 2] = mc;
        A.part_ml[(prow + lane) * 2 + 1] = l;
    }
}

/*
 * Merge of the chunk partials of (token j, query head h), 32 or 128 columns
 * a workgroup (attention.c:870-910). Group g of 8 (32 lanes each, a lane a
 * column) takes chunks g, g + 8, ... of the token's range, 16 at a time in
 * one batch of loads: their largest score M_g, then sum_c e^(m_c - M_g) l_c
 * and acc_c in chunk order. The groups are combined with weights
 * e^(M_g - M) as ((g0 + g1) + (g2 + g3)) + ((g4 + g5) + (g6 + g7)). The
 * order depends only on the token's own chunk range, so a token merges the
 * same way in any block. The gate sigmoid(g) * o is applied on the way out.
 */
constexpr int kMergeGroups = 8;
constexpr int kMergeLanes = 32;            /* lanes a group */
constexpr int kMergeBatch = 16;

/* the 4 columns of a float4, one by one */
__device__ __forceinline__ float &f4e(float4 &v, int e)
{
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

/*
 * CPL columns a lane (1 or 4: 32 or 128 columns a workgroup). Each column's
 * arithmetic is the same in both, so a token's output does not depend on
 * the instance its call takes; 4 when a launch has (token, head) pairs
 * enough to fill the GPU with 4 times fewer workgroups (blocks of tokens),
 * 1 when it has few (a decode spreads its loads over more CUs).
 */
template <int CPL, bool ONE = false>
__global__ __launch_bounds__(256) void merge_kernel(const SplitArgs A)
{
    constexpr uint32_t kCols = kMergeLanes * CPL;
    __shared__ float sM[kMergeGroups], sL[kMergeGroups];
    __shared__ float4 sAcc[kMergeGroups][kMergeLanes];
    const uint32_t id = blockIdx.x, tid = threadIdx.x;
    const uint32_t g = tid / kMergeLanes, cl = tid % kMergeLanes;
    uint32_t si = 0;
    if constexpr (!ONE)
        si = seq_index(A, &SeqDesc::mg0, id);
    const SeqDesc &sq = A.seq[si];
    const uint32_t hd = A.hd, G = A.group, nd = (hd + kCols - 1) / kCols;
    const uint32_t local = id - sq.mg0, db = local % nd;
    const uint32_t h = (local / nd) % A.n_head, j = local / nd / A.n_head;
    const uint32_t kvh = h / G, r = j * G + h % G, R = sq.n * G;
    const uint32_t pos = sq.pos0 + j;
    const uint32_t lo = row_lo(A, pos), hi = sq.last ? sq.last[j] : pos;
    const uint32_t clo = lo / kChunk, nc = hi / kChunk - clo + 1;
    /* partial row of chunk clo + i */
    const uint64_t base = sq.part0 + ((uint64_t)kvh * sq.span + (clo - sq.c0)) * R + r;
    /* the lane's columns col .. col + CPL - 1 (hd is a multiple of 8: all
       are inside the row or none is) */
    const uint32_t col = db * kCols + CPL * cl;
    const bool colok = col < hd;
    /* the gate, asked for with the partials so the loads overlap: branch-
       free (a load under a branch is waited for where the branches join,
       before the partials' loads), from a valid dummy address when unused */
    const size_t oi = ((size_t)j * A.n_head + h) * hd + col;
    const bool gel = A.gate_mode == kGateElem && colok;
    const float *gsrc = gel ? sq.gate + oi : A.part_ml;
    const float *hsrc = A.gate_mode == kGateHead ? sq.gate + (size_t)j * A.n_head + h
                                                 : A.part_ml;
    float4 gv = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (CPL == 4)
        gv = *(const float4 *)gsrc;
    else
        gv.x = *gsrc;
    const float gh = *hsrc;
    float mg = -INFINITY, lg = 0.0f;
    float4 ag = {0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t i0 = g; i0 < nc; i0 += kMergeGroups * kMergeBatch) {
        float2 ml[kMergeBatch];
        float4 v[kMergeBatch];
        /* branch-free: chunks past the range read the last one, weight 0 */
#pragma unroll
        for (int b = 0; b < kMergeBatch; b++) {
            const uint32_t i = i0 + kMergeGroups * b < nc ? i0 + kMergeGroups * b : nc - 1;
            const uint64_t pr = base + (uint64_t)i * R;
            ml[b] = *(const float2 *)(A.part_ml + pr * 2);
            const float *src = A.part_acc + pr * hd + (colok ? col : 0);
            if constexpr (CPL == 4)
                v[b] = *(const float4 *)src;
            else
                v[b].x = *src;
        }
        float mb = mg;
#pragma unroll
        for (int b = 0; b < kMergeBatch; b++)
            if (i0 + kMergeGroups * b < nc)
                mb = fmaxf(mb, ml[b].x);
        /* the batch's sums, against the group's new largest score */
        const float f = mg == -INFINITY ? 0.0f : expf(mg - mb);
        lg *= f;
#pragma unroll
        for (int e = 0; e < CPL; e++)
            f4e(ag, e) *= f;
#pragma unroll
        for (int b = 0; b < kMergeBatch; b++) {
            const float wgt = i0 + kMergeGroups * b < nc ? expf(ml[b].x - mb) : 0.0f;
            lg += wgt * ml[b].y;
#pragma unroll
            for (int e = 0; e < CPL; e++)
                f4e(ag, e) = fmaf(wgt, f4e(v[b], e), f4e(ag, e));
        }
        mg = mb;
    }
    if (cl == 0) {
        sM[g] = mg;
        sL[g] = lg;
    }
    sAcc[g][cl] = ag;
    __syncthreads();
    if (g != 0 || !colok)
        return;
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kMergeGroups; k++)
        mx = fmaxf(mx, sM[k]);
    float wl[kMergeGroups];
    float4 wa[kMergeGroups];
#pragma unroll
    for (int k = 0; k < kMergeGroups; k++) {
        const float wk = sM[k] == -INFINITY ? 0.0f : expf(sM[k] - mx);
        float4 a = sAcc[k][cl];
        wl[k] = wk * sL[k];
#pragma unroll
        for (int e = 0; e < CPL; e++)
            f4e(wa[k], e) = wk * f4e(a, e);
    }
    const float sum = ((wl[0] + wl[1]) + (wl[2] + wl[3])) + ((wl[4] + wl[5]) + (wl[6] + wl[7]));
    const float inv = 1.0f / sum;
    float4 o;
#pragma unroll
    for (int e = 0; e < CPL; e++) {
        float x[kMergeGroups];
#pragma unroll
        for (int k = 0; k < kMergeGroups; k++)
            x[k] = f4e(wa[k], e);
        float y = (((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]))) * inv;
        if (A.gate_mode == kGateElem)
            y *= 1.0f / (1.0f + expf(-f4e(gv, e)));
        else if (A.gate_mode == kGateHead)
            y *= 1.0f / (1.0f + expf(-gh));
        f4e(o, e) = y;
    }
    if constexpr (CPL == 4)
        *(float4 *)(sq.out + oi) = o;
    else
        sq.out[oi] = o.x;
}

template <int T, int D>
hipError_t launch_t(const SplitArgs &a, hipStream_t s)
{
    if (a.once && a.n_seqs == 1)
        hipLaunchKernelGGL((split_kernel<T, D, true, true>), dim3(a.n_wg), dim3(512), 0, s, a);
    else if (a.once)
        hipLaunchKernelGGL((split_kernel<T, D, true>), dim3(a.n_wg), dim3(512), 0, s, a);
    else
        hipLaunchKernelGGL((split_kernel<T, D, false>), dim3(a.n_wg), dim3(512), 0, s, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_d(uint32_t hd, const SplitArgs &a, hipStream_t s)
{
    if (hd <= 64)
        return launch_t<T, 64>(a, s);
    if (hd <= 128)
        return launch_t<T, 128>(a, s);
    if constexpr (T != kF32) {
        if (hd <= 256)
            return launch_t<T, 256>(a, s);
        return launch_wide(T, a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace

int split_supported(int kv, uint32_t hd)
{
    /* f32 rows above 128 numbers would not leave two stages in LDS; 8- and
       16-bit rows above 256 take the wide kernel (attn_wide.hip) */
    return kv >= kI8 && kv <= kF32 && hd >= 8 && hd % 8 == 0 &&
           hd <= (kv == kF32 ? 128u : 512u);
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

uint32_t merge_cols(uint64_t pairs, uint32_t hd)
{
    /* 128 columns a workgroup when that still leaves kMergeFill of them */
    return pairs * ((hd + 127) / 128) >= kMergeFill ? 128 : 32;
}

hipError_t launch_merge(const SplitArgs &a, uint32_t n_wg, hipStream_t s)
{
    const bool one = a.n_seqs == 1;
    if (a.merge_cols == 128 && one)
        hipLaunchKernelGGL((merge_kernel<4, true>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 128)
        hipLaunchKernelGGL(merge_kernel<4>, dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 32 && one)
        hipLaunchKernelGGL((merge_kernel<1, true>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 32)
        hipLaunchKernelGGL(merge_kernel<1>, dim3(n_wg), dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace janas
