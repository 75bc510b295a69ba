/*
 * attn_wide.hip - split-KV attention for head sizes above 256 (up to 512,
 * Gemma 4's int16 cache: src/llm/attention.c:998-1000 admits head_dim up
 * to 512, tests/test_attention.c:253-338 runs it).
 *
 * The contract is the split kernel's (attn_split.hip): one workgroup per
 * (sequence, KV head, chunk of 256 positions, tile of 16 query rows), the
 * same partial (largest score, sum of weights, weighted values) per chunk
 * and query row, merged by the same ordered merge kernel - so a token's
 * result does not depend on the block it runs in. What changes is how a
 * workgroup walks its chunk, because a 512-number row is 1 KB (16-bit
 * types): the split kernel's layout (8 waves each holding 32 rows) would
 * need 256 KB of LDS and 256 registers of loads a lane.
 *
 *   4 waves (one a SIMD), wave w takes positions 64 w .. 64 w + 63 in 4
 *   rounds of 16. A round's 16 rows (16 KB) arrive with contiguous 16-byte
 *   loads a lane (1 KB a wave instruction) and pass through the wave's own
 *   LDS region. The wave keeps two rounds of loads in flight: when round s
 *   is in LDS it asks for round s + 2 and then computes on round s; the 8
 *   rounds are K 0..3 then V 0..3, so V's first loads overlap K's scores.
 *   The softmax is one shot over the wave's 64 positions (the scores of
 *   all 4 K rounds are in registers before any V round is used); the 4
 *   waves' partials are combined in LDS in a fixed order.
 *
 *   S^T = K . Q^T   v_mfma_f32_16x16x32_f16 over the head dimension: A =
 *                   a round's 16 K rows from LDS, B = the query planes from
 *                   LDS; lane l holds query row l % 16 at positions
 *                   4 (l / 16) + i of the round.
 *   O   = P . V     v_mfma_f32_16x16x16_f16 over the round's 16 positions:
 *                   the weights are already its A operand (row l % 16,
 *                   k = 4 (l / 16) + i); V is read back transposed with
 *                   ds_read_b64_tr_b16 - int8 rows are widened to f16 on
 *                   their way into LDS so every type reads the same way.
 *
 * Accuracy is the split kernel's: the query and the weights are split into
 * high and low f16 parts after scaling by a power of two, keys and values
 * enter as f16 planes whose sum is the cached number exactly (int16:
 * 256 (x >> 8) + (x & 255)); products are exact and summed in f32.
 */
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include <hip/hip_runtime.h>

#include "attn_elem.h"

/* One instance or another (one sequence, several), a row is computed with
   the same operations: nothing is fused into multiply-adds but what is
   written as fmaf, so the compiler cannot fuse differently per instance. */
#pragma clang fp contract(off)

namespace janas {
namespace {

constexpr int kWWaves = 4;                  /* waves a workgroup */
constexpr int kWPos = kChunk / kWWaves;     /* 64 positions a wave */
constexpr int kRound = 16;                  /* positions a round */
constexpr int kRounds = kWPos / kRound;     /* 4 K rounds, then 4 V rounds */
constexpr int kWD = 512;                    /* largest head size */
constexpr int kWBuf = 2;                    /* rounds of loads in flight */

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

/* four int16 (as halves' bits) -> exact f16 planes 256 (x >> 8), x & 255 */
__device__ __forceinline__ void split16(h4 raw, h4 &hi, h4 &lo)
{
    const uint2 u = __builtin_bit_cast(uint2, raw);
    i16_planes4(u.x, u.y, hi, lo);
}

template <int T, int D> struct WShape {
    static_assert(T == kI8 || T == kI16 || T == kF16, "8- and 16-bit caches");
    static constexpr int EB = Elem<T>::bytes;
    static constexpr int KP = Elem<T>::planes;      /* K planes */
    static constexpr int VP = T == kI16 ? 2 : 1;    /* V planes (int8 widened) */
    static constexpr bool SCALED = T == kI8 || T == kI16;
    static constexpr int RB = D * EB;               /* bytes of a padded row */
    static constexpr int VB = D * 2;                /* a V row in LDS (16-bit) */
    static constexpr int UNITS = kRound * RB / 1024; /* 16-byte loads a lane a round */
    static constexpr int KS = D / 32;               /* score k-steps */
    static constexpr int NT = D / 16;               /* output column tiles */
    static constexpr int QV = D / 64;               /* q float4 a lane */
    static constexpr int QP = D + 16;               /* halves a q row in LDS */
    /* a wave's region: a round's rows (V as 16-bit: 16 VB bytes), later
       half of its sums ([NT / 2][64] f4, as many bytes) */
    static constexpr int REGION = kRound * VB / 1024 * kBlk;
};

/* ONE: a launch of one sequence, its descriptor read at fixed offsets.
   Q16: the reference's INT16 way over an int8 cache (attn_split.hip's
   split kernel has the same arithmetic): a quantized query, exact integer
   scores, weights quantized per chunk and exact integer value sums */
template <int T, int D, int NB, bool ONE = false, bool Q16 = false>
__global__ __launch_bounds__(256) void wide_kernel(const SplitArgs A)
{
    static_assert(!Q16 || T == kI8, "INT16: int8 caches");
    using E = Elem<T>;
    using S = WShape<T, D>;
    static_assert(S::UNITS * 1024 == kRound * S::RB, "whole kilobytes a round");
    static_assert(NB * S::UNITS + S::QV + 2 < 63, "the loads fit the wait counter");
    static_assert(NB >= 1 && NB <= 2 * kRounds, "rounds in flight");
    static_assert(kRound * S::VB <= S::REGION && S::NT / 2 * 64 * 16 <= S::REGION,
                  "a round of V rows and half the sums fit the region");
    __shared__ __attribute__((aligned(16))) char sW[kWWaves * S::REGION];
    __shared__ __attribute__((aligned(16))) _Float16 sQ[2][kRows][S::QP];
    __shared__ __attribute__((aligned(16))) float sKz[kChunk];
    __shared__ __attribute__((aligned(16))) float sVz[kChunk];
    __shared__ float sMax[kWWaves][kRows], sSum[kWWaves][kRows];
    __shared__ float sQs[kRows];
    __shared__ float sX[kWWaves][kRows];  /* INT16: largest weight x value scale */
    __shared__ uint32_t sLo[kRows], sHi[kRows];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t g16 = lane >> 4, l16 = lane & 15;
    if constexpr (!ONE)
        starts_early(A.n_wg, A.n_wg, A.n_seqs, A.wg0s);
    const uint32_t id = xcd_remap(blockIdx.x, A.n_wg);
    uint32_t si = 0;
    if constexpr (!ONE)
        si = seq_index(A.wg0s, A.n_seqs, id);
    const SeqDesc &sq = A.seq[si];
    const uint32_t G = A.group, hd = A.hd;
    /* the descriptor fields the workgroup starts from (the cache and query
       addresses among them) in one round trip: left to the scheduler,
       a second batch of them went out after a wait for the first */
    asm volatile("" ::"s"(sq.k), "s"(sq.v), "s"(sq.q), "s"(A.n_head), "s"(sq.n),
                 "s"(sq.pos0), "s"(sq.end), "s"(sq.c0), "s"(sq.span), "s"(sq.rtiles),
                 "s"(sq.wg0), "s"(sq.cap), "s"(sq.last));
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
    /* a last[] past the call's end counts as its end */
    uint32_t hi_all = sq.last ? sq.last[jl] : sq.pos0 + jl;
    hi_all = hi_all < sq.end - 1 ? hi_all : sq.end - 1;
    if (t0 > hi_all || t0 + kChunk <= lo_all)
        return;
    const uint32_t p0w = t0 + w * kWPos;
    /* does any row see a position of this wave? (uniform in the wave) */
    const bool active = p0w <= hi_all && p0w + kWPos > lo_all;
    const uint32_t plast = sq.end - 1;
    /* rows of the chunk in the cache: contiguous, a ring's too (cap is a
       multiple of the chunk) */
    const size_t crow = (size_t)kvh * sq.cap + (A.ring ? t0 % sq.cap : t0);
    /* the chunk's rows start at one address per block; a lane's byte
       offset from it stays below kChunk rows, 32 bits (the loads take the
       base in scalar registers and the offset in one vector register) */
    const uint32_t rbytes = hd * S::EB, rlast = plast - t0;
    const char *const kbase = (const char *)sq.k + crow * rbytes;
    const char *const vbase = (const char *)sq.v + crow * rbytes;

    if (tid < kRows) {
        uint32_t r = r0 + tid;
        uint32_t lo = 1, hi = 0;
        if (r < R) {
            uint32_t j = r / G;
            lo = row_lo(A, sq.pos0 + j);
            hi = sq.last ? sq.last[j] : sq.pos0 + j;
            hi = hi < sq.end - 1 ? hi : sq.end - 1;
        }
        sLo[tid] = lo;
        sHi[tid] = hi;
    }

    /* ---- every load unconditional: rows past the call read its last row,
       columns past hd column 0 - valid memory whose numbers are masked or
       multiplied by zero weights ---- */
    /* q: wave w takes rows 4 w .. 4 w + 3, lane l row 4 w + l / 16 */
    const uint32_t qrow = 4 * w + g16;
    float4 qv[S::QV];
    bool qok[S::QV];
    {
        const uint32_t r = r0 + qrow < R ? r0 + qrow : r0;
        const uint32_t j = r / G, h = kvh * G + r % G;
        const float *src = sq.q + ((size_t)j * A.n_head + h) * hd;
#pragma unroll
        for (int i = 0; i < S::QV; i++) {
            const uint32_t col = 4 * (l16 + 16 * i);
            qok[i] = r0 + qrow < R && col < hd;
            qv[i] = *(const float4 *)(src + (col < hd ? col : 0));
        }
    }
    /* the scales of the chunk's positions, one a thread */
    float kz = 1.0f, vz = 1.0f;
    if constexpr (S::SCALED) {
        const uint32_t at = tid < rlast ? tid : rlast;
        kz = sq.ks[crow + at];
        vz = sq.vs[crow + at];
    }
    /* round s (K 0..3, V 0..3): byte 1024 i + 16 lane of its 16 rows */
    auto load_round = [&](u4 *buf, int s) {
        const char *base = s < kRounds ? kbase : vbase;
        const uint32_t p0 = w * kWPos + kRound * (s % kRounds); /* from t0 */
#pragma unroll
        for (int i = 0; i < S::UNITS; i++) {
            const uint32_t byte = i * 1024 + lane * 16;
            const uint32_t row = byte / S::RB, cb = byte % S::RB;
            const uint32_t p = p0 + row;
            uint32_t at;
            if constexpr (S::EB == 1) {
                bool back;
                at = unit_at(cb, hd, back);
            } else {
                at = cb < hd * S::EB ? cb : 0;
            }
            const uint32_t off = __umul24(p < rlast ? p : rlast, rbytes) + at;
            buf[i] = __builtin_nontemporal_load((const u4 *)(base + off));
        }
    };
    u4 buf[NB][S::UNITS];
#pragma unroll
    for (int b = 0; b < NB; b++)
        load_round(buf[b], b);

    /* ---- q: scaled by 2^e so that the row's largest |q| lies in
       [2^13, 2^14), split into f16 planes, into LDS ---- */
    {
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < S::QV; i++)
            if (qok[i])
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(qv[i].x), fabsf(qv[i].y)),
                                     fmaxf(fabsf(qv[i].z), fabsf(qv[i].w))));
        mx = max_row16(mx);
        if constexpr (Q16) {
            /* the row as int16 with one scale (quant_worker,
               attention.c:820-839): planes x >> 8 and x & 255 */
            const float inv = q16_inv(mx);
#pragma unroll
            for (int i = 0; i < S::QV; i++) {
                const uint32_t col = 4 * (l16 + 16 * i);
                const float x[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int32_t qi = qok[i] ? q16_round(x[e], inv) : 0;
                    sQ[0][qrow][col + e] = (_Float16)(qi >> 8);
                    sQ[1][qrow][col + e] = (_Float16)(qi & 255);
                }
            }
            if (l16 == 0)
                sQs[qrow] = mx / 32767.0f;
        } else {
            int ex = 0;
            if (mx > 0.0f && mx < INFINITY) {
                frexpf(mx, &ex);
                ex = 14 - ex;
            }
            const float up = ldexpf(1.0f, ex);
#pragma unroll
            for (int i = 0; i < S::QV; i++) {
                const uint32_t col = 4 * (l16 + 16 * i);
                const float x[4] = {qv[i].x, qv[i].y, qv[i].z, qv[i].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    _Float16 hi, lo;
                    split_hl(qok[i] ? x[e] * up : 0.0f, hi, lo);
                    sQ[0][qrow][col + e] = hi;
                    sQ[1][qrow][col + e] = lo;
                }
            }
            if (l16 == 0)
                sQs[qrow] = ldexpf(1.0f, -ex);
        }
    }
    sKz[tid] = kz;
    sVz[tid] = vz;
    __syncthreads();

    const uint32_t rlo = sLo[l16], rhi = sHi[l16];
    /* scores in powers of two: log2 e folded into the scale */
    const float qs = sQs[l16] * A.scale * kLog2e;
    const float qsc = sQs[l16];
    /* this lane's positions of round r: 16 r + 4 g16 + i of the wave */
    const uint32_t pl = w * kWPos + 4 * g16;
    char *const reg = sW + (size_t)w * S::REGION;

    float sv[4 * kRounds];
    h4 pa[kRounds][2];
    float m = -INFINITY, lsum = 0.0f;
    int pe = 13;
    f4 o[S::NT];
    /* INT16: the low weight plane's sums apart (each plane's sums are
       exact integers in f32; their mix 256 hi + lo would not be) */
    f4 o2[Q16 ? S::NT : 1];
#pragma unroll
    for (int t = 0; t < S::NT; t++)
        o[t] = f4{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < (Q16 ? S::NT : 1); t++)
        o2[t] = f4{0, 0, 0, 0};

    /* step s (a compile-time constant): round s into LDS, round s + NB
       asked for, round s computed on */
    auto step = [&](auto step_no) {
        constexpr int s = decltype(step_no)::value;
        u4 *const b = buf[s % NB];
        /* round s into the region (the wave's reads of the previous round
           are done: LDS serves a wave in order) */
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (T == kI8) {
#pragma unroll
            for (int i = 0; i < S::UNITS; i++) {
                const uint32_t byte = i * 1024 + lane * 16;
                const uint32_t row = byte / S::RB, cb = byte % S::RB;
                bool back;
                (void)unit_at(cb, hd, back);
                const u4 x = unit_fix(b[i], back);
                if constexpr (s >= kRounds) {
                    /* values widened to f16 rows of 1 KB */
                    const h8 lo8 = Elem<kI8>::widen(x.x, x.y);
                    const h8 hi8 = Elem<kI8>::widen(x.z, x.w);
                    *(h8 *)(reg + blk_off(row * S::VB + cb * 2)) = lo8;
                    *(h8 *)(reg + blk_off(row * S::VB + cb * 2 + 16)) = hi8;
                } else {
                    *(u4 *)(reg + blk_off(byte)) = x;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < S::UNITS; i++)
                *(u4 *)(reg + blk_off(i * 1024 + lane * 16)) = b[i];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (s + NB < 2 * kRounds)
            load_round(b, s + NB);

        if constexpr (s < kRounds) {
            /* scores of round s: 4 accumulators (even / odd k-step, high /
               low query plane) so that neighbouring products do not wait
               for each other */
            f4 sa[2][2] = {{f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}, {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}}};
#pragma unroll
            for (int k = 0; k < S::KS; k++) {
                const h8 qb0 = *(const h8 *)&sQ[0][l16][32 * k + 8 * g16];
                const h8 qb1 = *(const h8 *)&sQ[1][l16][32 * k + 8 * g16];
                const uint32_t bo = l16 * S::RB + (32 * k + 8 * g16) * S::EB;
                typename E::Raw kr;
                if constexpr (S::EB == 1)
                    kr.a = *(const uint2 *)(reg + blk_off(bo));
                else
                    kr.a = *(const uint4 *)(reg + blk_off(bo));
                h8 ka[S::KP];
                E::planes8(kr, ka);
#pragma unroll
                for (int kp = 0; kp < S::KP; kp++) {
                    sa[k & 1][0] = mfma(ka[kp], qb0, sa[k & 1][0]);
                    sa[k & 1][1] = mfma(ka[kp], qb1, sa[k & 1][1]);
                }
            }
            const f4 acc = (sa[0][0] + sa[1][0]) + (sa[0][1] + sa[1][1]);
            /* INT16: the planes' exact sums apart */
            const f4 ahi = sa[0][0] + sa[1][0], alo = sa[0][1] + sa[1][1];
            /* the key scales of the lane's 4 positions, one read (read
               under the mask, each was a branch and a wait of its own) */
            f4 kz = f4{1.0f, 1.0f, 1.0f, 1.0f};
            if constexpr (S::SCALED)
                kz = *(const f4 *)&sKz[pl + kRound * s];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t pc = pl + kRound * s + i; /* chunk-relative */
                const uint32_t p = t0 + pc;
                float x = -INFINITY;
                if (active && p >= rlo && p <= rhi && p <= plast) {
                    if constexpr (Q16) {
                        x = q16_score(ahi[i], alo[i], qsc, A.scale, kz[i]);
                    } else {
                        x = acc[i] * qs;
                        if constexpr (S::SCALED)
                            x *= kz[i];
                    }
                }
                sv[4 * s + i] = x;
                m = fmaxf(m, x);
            }
        } else {
            const int r = s - kRounds;
            /* values of round r, 8 column tiles at a time */
#pragma unroll
            for (int t8 = 0; t8 < S::NT; t8 += 8) {
                h4 vb[8][S::VP];
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint32_t r1 = 4 * g16 + (l16 >> 2);
                    const uint32_t cc = 16 * (t8 + t) + 4 * (l16 & 3);
                    const h4 x = lds_read_tr((const _Float16 *)(reg + blk_off(r1 * S::VB + cc * 2)));
                    if constexpr (T == kI16)
                        split16(x, vb[t][0], vb[t][1]);
                    else
                        vb[t][0] = x;
                }
                if constexpr (Q16) {
#pragma unroll
                    for (int t = 0; t < 8; t++) {
                        o[t8 + t] = mfma16(pa[r][0], vb[t][0], o[t8 + t]);
                        o2[t8 + t] = mfma16(pa[r][1], vb[t][0], o2[t8 + t]);
                    }
                } else {
#pragma unroll
                    for (int ap = 0; ap < 2; ap++)
#pragma unroll
                        for (int vp = 0; vp < S::VP; vp++)
#pragma unroll
                            for (int t = 0; t < 8; t++)
                                o[t8 + t] = mfma16(pa[r][ap], vb[t][vp], o[t8 + t]);
                }
            }
        }

        if constexpr (s == kRounds - 1 && Q16) {
            /* INT16: the chunk's largest score over the 4 waves, the
               weights e^(s - M) times the value scales, their largest over
               the chunk, and the weights quantized against it to
               0 .. 32767, planes w >> 8 and w & 255 (att_weights_ref,
               att_wquant_ref, attention.c:158-176, :574-588, :761-772) */
            m = max_x32(max_x16(m));
            if (lane < 16)
                sMax[w][lane] = m;
            __syncthreads();
            m = fmaxf(fmaxf(sMax[0][l16], sMax[1][l16]), fmaxf(sMax[2][l16], sMax[3][l16]));
            const float mm = m == -INFINITY ? 0.0f : m;
            float pv[4 * kRounds];
            float vmx = 0.0f;
            f4 vz[kRounds];
#pragma unroll
            for (int r = 0; r < kRounds; r++)
                vz[r] = *(const f4 *)&sVz[pl + kRound * r];
#pragma unroll
            for (int e = 0; e < 4 * kRounds; e++) {
                const float wt = det_weight(sv[e], mm);
                lsum += wt;
                pv[e] = wt * vz[e / 4][e % 4];
                vmx = fmaxf(vmx, pv[e]);
            }
            vmx = max_x32(max_x16(vmx));
            lsum = sum_x32(sum_x16(lsum));
            if (lane < 16)
                sX[w][lane] = vmx;
            __syncthreads();
            const float inv = q16_inv(fmaxf(fmaxf(sX[0][l16], sX[1][l16]), fmaxf(sX[2][l16], sX[3][l16])));
#pragma unroll
            for (int e = 0; e < 4 * kRounds; e++) {
                const int32_t q = q16_round(pv[e], inv);
                pa[e / 4][0][e % 4] = (_Float16)(q >> 8);
                pa[e / 4][1][e % 4] = (_Float16)(q & 255);
            }
        } else if constexpr (s == kRounds - 1) {
            /* the wave's softmax over its 64 positions, one shot */
            m = max_x32(max_x16(m));
            /* the weights' power of two: the largest (e^0 times the largest
               value scale of the wave's positions) lands in [2^12, 2^13) */
            float vsc[4 * kRounds];
#pragma unroll
            for (int r = 0; r < kRounds; r++) {
                const f4 z = S::SCALED ? *(const f4 *)&sVz[pl + kRound * r] : f4{1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
                for (int i = 0; i < 4; i++)
                    vsc[4 * r + i] = z[i];
            }
            if constexpr (S::SCALED) {
                float vm = 0.0f;
#pragma unroll
                for (int e = 0; e < 4 * kRounds; e++)
                    vm = fmaxf(vm, vsc[e]);
                vm = max_x32(max_x16(vm));
                int ev = 0;
                if (vm > 0.0f && vm < INFINITY)
                    frexpf(vm, &ev);
                pe = 13 - ev;
            }
            const float up = ldexpf(1.0f, pe);
#pragma unroll
            for (int e = 0; e < 4 * kRounds; e++) {
                const float x = sv[e];
                float pw = 0.0f;
                if (x != -INFINITY && x - m >= kCut2)
                    pw = __builtin_amdgcn_exp2f(x - m);
                lsum += pw;
                _Float16 hi, lo;
                split_hl(pw * vsc[e] * up, hi, lo);
                pa[e / 4][0][e % 4] = hi;
                pa[e / 4][1][e % 4] = lo;
            }
            lsum = sum_x32(sum_x16(lsum));
        }
    };
    static_assert(2 * kRounds == 8, "eight steps");
    step(std::integral_constant<int, 0>());
    step(std::integral_constant<int, 1>());
    step(std::integral_constant<int, 2>());
    step(std::integral_constant<int, 3>());
    step(std::integral_constant<int, 4>());
    step(std::integral_constant<int, 5>());
    step(std::integral_constant<int, 6>());
    step(std::integral_constant<int, 7>());

    /* ---- the 4 waves combined: chunk max M, wave w's sums weighted by
       2^(m_w - M) (and back to 2^0), then summed over the waves in a fixed
       order, half the column tiles at a time ---- */
    if (lane < 16) {
        if constexpr (!Q16)
            sMax[w][lane] = m;  /* INT16: the waves' maxima are there */
        sSum[w][lane] = lsum;
    }
    __syncthreads();
    float mc = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWWaves; ww++)
        mc = fmaxf(mc, sMax[ww][l16]);
    if constexpr (Q16) {
        /* exact integer sums, 256 hi + lo as int32 bits (at most 64
           positions of 32767 x 128: no overflow) */
#pragma unroll
        for (int t = 0; t < S::NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[t][i] = __int_as_float((int32_t)o[t][i] * 256 + (int32_t)o2[t][i]);
    } else {
        const float f = (m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mc)) * ldexpf(1.0f, -pe);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float fi = __shfl(f, 4 * g16 + i, 64);
#pragma unroll
            for (int t = 0; t < S::NT; t++)
                o[t][i] *= fi;
        }
    }
    /* INT16: the weights' scale of row 4 g16 + i, mx / 32767 */
    float wsc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (Q16) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t rr = 4 * g16 + i;
            wsc[i] = fmaxf(fmaxf(sX[0][rr], sX[1][rr]), fmaxf(sX[2][rr], sX[3][rr])) / 32767.0f;
        }
    }
    const uint64_t prow = sq.part0 + ((uint64_t)kvh * sq.span + (c - sq.c0)) * R + r0;
    f4 *const mine = (f4 *)reg;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        if (half)
            __syncthreads(); /* every wave has read the first half */
        /* the region's V reads are done (in order); sums as [NT / 2][64] f4 */
#pragma unroll
        for (int t = 0; t < S::NT / 2; t++)
            mine[t * 64 + lane] = o[half * (S::NT / 2) + t];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < S::NT / 2 / kWWaves; j++) {
            const uint32_t t = w + kWWaves * j;
            f4 part[kWWaves];
#pragma unroll
            for (int ww = 0; ww < kWWaves; ww++)
                part[ww] = ((const f4 *)(sW + (size_t)ww * S::REGION))[t * 64 + lane];
            f4 sum;
            if constexpr (Q16) {
                /* the chunk's exact int32 sum, then one multiply
                   (att_values_i16_ref, attention.c:178-193) */
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t acc = (__float_as_int(part[0][i]) + __float_as_int(part[1][i])) +
                                        (__float_as_int(part[2][i]) + __float_as_int(part[3][i]));
                    sum[i] = (float)acc * wsc[i];
                }
            } else {
                sum = (part[0] + part[1]) + (part[2] + part[3]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t row = 4 * g16 + i;
                const uint32_t col = 16 * (half * (S::NT / 2) + t) + l16;
                if (r0 + row < R && col < hd)
                    A.part_acc[(prow + row) * hd + col] = sum[i];
            }
        }
    }
    if (w == 0 && lane < kRows && r0 + lane < R) {
        float l = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kWWaves; ww++) {
            const float mw = sMax[ww][lane];
            if constexpr (Q16)
                l += sSum[ww][lane]; /* already against the chunk's M */
            else
                l += (mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mc)) * sSum[ww][lane];
        }
        /* INT16's largest score is in natural units: to powers of two for
           the merge */
        A.part_ml[(prow + lane) * 2] = Q16 ? mc * kLog2e : mc;
        A.part_ml[(prow + lane) * 2 + 1] = l;
    }
}

template <int T, int D, int NB>
hipError_t launch_w(const SplitArgs &a, hipStream_t s)
{
    if constexpr (T == kI8) {
        if (a.int16) {
            if (a.n_seqs == 1)
                hipLaunchKernelGGL((wide_kernel<T, D, NB, true, true>), dim3(a.n_wg), dim3(256), 0, s, a);
            else
                hipLaunchKernelGGL((wide_kernel<T, D, NB, false, true>), dim3(a.n_wg), dim3(256), 0, s, a);
            return hipGetLastError();
        }
    }
    if (a.n_seqs == 1)
        hipLaunchKernelGGL((wide_kernel<T, D, NB, true>), dim3(a.n_wg), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((wide_kernel<T, D, NB>), dim3(a.n_wg), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_wide(int kv, const SplitArgs &a, hipStream_t s)
{
    if (a.hd > (uint32_t)kWD || a.hd % 8)
        return hipErrorInvalidValue;
    switch (kv) {
    case kI8:
        return launch_w<kI8, kWD, kWBuf>(a, s);
    case kI16:
        return launch_w<kI16, kWD, kWBuf>(a, s);
    case kF16:
        return launch_w<kF16, kWD, kWBuf>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace janas
