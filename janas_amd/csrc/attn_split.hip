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
 *   split kernel   one workgroup (4 waves of 64, one a SIMD) per (sequence,
 *                  KV head, chunk, one or two tiles of 8 query rows); a
 *                  query row is a (token, query head of the KV head's
 *                  group), so every K/V row of the chunk is read once for
 *                  the whole GQA group (and its operands once for both
 *                  tiles).
 *                  Wave w streams positions 64 w .. 64 w + 63 in groups of
 *                  16 with two groups in flight, scores each K group as it
 *                  lands, takes a one-shot softmax over its 64 positions and
 *                  the value product of each V group as it lands; the 4
 *                  waves' partials are combined in LDS in a fixed order into
 *                  the chunk's exact partial. Workgroups are renumbered so
 *                  each XCD takes a contiguous range (neighbouring chunks
 *                  share an L2).
 *   merge kernel   one workgroup per (token, query head, 32 or 128 columns): the
 *                  ordered merge of the chunk partials (8 groups of chunks in
 *                  parallel, each in batches of 2 to 16 by the
 *                  launch's longest span, combined in a fixed
 *                  tree), the output gate sigmoid(g) * o (model_attn.c:
 *                  159-170) fused in.
 *
 * Scores and values run on the matrix cores at float accuracy: the query
 * and the weights are split into a high and a low f16 part (x = hi + lo, 22
 * significant bits), each scaled by a power of two first so that neither
 * part loses bits to f16's range; keys and values enter as f16 planes whose
 * sum is the cached number exactly (int8 and f16: one plane; int16:
 * 256 * (x >> 8) and x & 255; f32: hi + lo). The two query (weight) planes
 * of a row are neighbouring MFMA rows, so one product takes both. Products
 * are exact in the MFMA and summed in f32. Scores, the partials' largest
 * scores and the merge work in powers of two (log2 e folded into the score
 * scale), so each exponential is one v_exp_f32.
 */
#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_elem.h"
#include "attn_q8k.h"

/* A token's result must not depend on the instance its call takes (one or
   two row tiles, one sequence or several, 32, 128 or 256 merge columns):
   each computes a row with the same operations, but left free the compiler
   fuses a different product of a sum like a b + c d into a multiply-add in
   each instance. So nothing is fused here but what is written as fmaf. */
#pragma clang fp contract(off)

namespace janas {
namespace {

/* ---- the split kernel: four waves, each streaming its positions ------- */

/*
 * A workgroup is 4 waves, one a SIMD; wave w takes positions 64 w .. 64 w +
 * 63 of the chunk as 4 groups of 16. The memory pipe of a SIMD serves its
 * loads in issue order and only so many at once (an instruction that asks
 * for more waits until earlier data lands), so a wave keeps two groups (its
 * K, then its V) in flight: when group s has landed it asks for group s + 2
 * and then computes on s - K groups 0..3, then V groups 0..3, 1 KB a load
 * instruction. The scores of a group are computed as soon as its K is in;
 * the softmax is one shot over the wave's 64 positions once all four K
 * groups are scored; the value product takes each V group as it lands. The
 * query's two planes are staged in LDS once, before the big loads are
 * issued, so no score waits for a load queued behind the chunk.
 *
 * Query rows come in tiles of 8 (row r = token j x group + head): MFMA row
 * 2 i is tile row i's high plane, 2 i + 1 its low plane, so a lane's two
 * neighbours hold one query row's two partial sums (added across lanes l
 * and l ^ 1 for the scores, and inside a lane for the values: output rows
 * 2 i and 2 i + 1 land in the same lane). The two lanes of a row split
 * its work: lane l takes positions 2 (l & 1) and 2 (l & 1) + 1 of its four
 * a group - their masks, softmax and both weight planes - and the pair
 * swaps the plane each needs, so nothing is made twice.
 *
 *   S^T = K . Q^T   v_mfma_f32_16x16x32_f16 over the head dimension: A = a
 *                   group's 16 K rows (LDS), B = the query planes (LDS);
 *                   lane l holds MFMA row l % 16 at positions 4 (l / 16) + i.
 *   O   = P . V     v_mfma_f32_16x16x16_f16 over the group's 16 positions:
 *                   the weights are already its A operand; V is read back
 *                   transposed (ds_read_b64_tr_b16).
 *
 * Every wave's (largest score, sum of weights, weighted values) is combined
 * in LDS in a fixed order into the chunk's partial. Scores are kept in
 * powers of two (log2 e folded into the score scale; the partial's largest
 * score too), so every exponential is one v_exp_f32.
 *
 * Element types: f16 and int16 rows are staged as they are (int16 is split
 * into 256 (x >> 8) and x & 255 when read), int8 rows are widened to f16
 * (the INT16 way's keys from head size 128 stay bytes, for the integer
 * matrix cores),
 * f32 rows are split into two f16 planes; every LDS row is head size x 16
 * bits, its 16-byte units swizzled (unit u of row r in slot u ^ swz(r)) so
 * that both operand reads are free of bank conflicts.
 */
constexpr int kSW = 4;              /* waves a workgroup */
constexpr int kSWP = kChunk / kSW;  /* positions a wave */
constexpr int kSG = 16;             /* positions a group */
constexpr int kSNG = kSWP / kSG;    /* groups a wave */

template <int T, int D> struct SS {
    static constexpr int EB = Elem<T>::bytes;
    static constexpr int MRB = D * EB;               /* bytes of a padded row in memory */
    static constexpr int LG = kSG * MRB / 1024;      /* 1 KB loads a group */
    static constexpr int LRB = 2 * D;                /* bytes of an LDS row */
    static constexpr int NPL = T == kF32 ? 2 : 1;    /* LDS planes */
    static constexpr int PLB = kSG * LRB;            /* bytes of a plane */
    static constexpr int REG = PLB * NPL;            /* a wave's region */
    static constexpr int KS = D / 32;                /* score k-steps */
    static constexpr int NT = D / 16;                /* value column tiles */
    static constexpr int DP = Elem<T>::planes;       /* data planes a product */
    static constexpr bool SCALED = T == kI8 || T == kI16;
    /* groups in flight a wave (deeper measured no faster: int8 rows
       with 4 in flight took 8% longer at config 4's shape) */
    static constexpr int NF = 2;
    static_assert(LG >= 1 && kSG * MRB % 1024 == 0, "whole kilobytes a group");
    static_assert(REG >= 32 * D, "the region holds the wave's sums");
};

/* the LDS slot of unit u of a row r (the units of a row: D / 8) */
template <int D> __device__ __forceinline__ uint32_t slot(uint32_t u, uint32_t r)
{
    if constexpr (D >= 128)
        return u ^ (((r << 1) | ((r >> 3) & 1)) & 15);
    else
        return u ^ ((r >> 1) & 7);
}

/* ONE: a launch of one sequence - its descriptor is read at fixed offsets
   with the rest of the arguments, not after the launch's sequence count.
   Head sizes up to 128 over 8- and 16-bit caches ask for 3 waves a SIMD
   (at most 168 registers): the f16 instance otherwise takes 176 and holds
   two workgroups a CU, where calls of several row tiles (a verify) or many
   chunks (a ragged decode) want more in flight. NT: every chunk is read by
   one workgroup (decode, or a verify whose rows are all one workgroup's):
   nontemporal loads; the workgroups of a block of tokens read a chunk
   each, and plain loads keep it in L2 for them.
   MT: row tiles of 8 a workgroup (1, or 2 at head sizes up to 128 over 8-
   and 16-bit caches). Every K and V operand read from LDS feeds MT
   products, one a tile, so a verify's or a block's rows read a chunk once
   per two tiles. A row's arithmetic - its products, softmax, combine - is
   the same in either, so its partial is the same bits whichever instance
   its call takes. */
template <int T, int D, bool NT, bool ONE = false, bool Q16 = false, int MT = 1>
__global__ __launch_bounds__(kSW * 64) __attribute__((amdgpu_waves_per_eu(D <= 128 && T != kF32 ? 3 : 1))) void split_kernel(const SplitArgs A)
{
    static_assert(!Q16 || (T == kI8 && D % 16 == 0), "INT16: int8 caches");
    static_assert(MT == 1 || (MT == 2 && D <= 128 && T != kF32),
                  "two row tiles: 8- and 16-bit rows up to 128");
    using S = SS<T, D>;
    constexpr int KS = S::KS, NT_ = S::NT, LG = S::LG, DP = S::DP;
    constexpr uint32_t TR = kTileRows * MT;      /* query rows a workgroup */
    /* a wave's LDS region: its staged groups, then its sums (32 D bytes a
       tile) for the combine */
    constexpr int CR = S::REG > 32 * D * MT ? S::REG : 32 * D * MT;
    __shared__ __attribute__((aligned(1024))) char sR[kSW * CR];
    __shared__ __attribute__((aligned(16))) _Float16 sQ[2 * TR][D + 8];
    /* INT16 over int8 keys, head sizes from 128: the scores are integer
       products (v_mfma_i32_16x16x64_i8) of the keys as they are in memory
       and the query's planes as bytes, x >> 8 and (x & 255) - 128; the
       second plane's offset is given back as 128 times the key's sum, a
       product of the keys with ones. The keys skip the widening to f16 */
    constexpr bool RAWK = Q16 && D >= 128;
    constexpr int KS8 = D / 64;   /* integer k-steps */
    __shared__ __attribute__((aligned(16))) int8_t sQ8[RAWK ? 2 * TR : 1][RAWK ? D + 16 : 16];
    __shared__ float sQs[TR];
    __shared__ __attribute__((aligned(16))) float sM[kSW][TR];
    __shared__ __attribute__((aligned(16))) float sL[kSW][TR];
    __shared__ float sPe[kSW];
    __shared__ float sX[kSW][TR];   /* INT16: largest weight x value scale */
    __shared__ __attribute__((aligned(16))) float sKs[kSW][kSWP];
    __shared__ __attribute__((aligned(16))) float sVs[kSW][kSWP];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t g = lane >> 4, l16 = lane & 15;
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
    const uint32_t R = sq.n * G, r0 = rt * TR;
    const uint32_t t0 = c * kChunk, plast = sq.end - 1;

    /* the workgroup's tokens see [lo(first), last(final)]: nothing of this
       chunk means no partial is needed (the merge does not read it) */
    const uint32_t rows_here = R - r0 < TR ? R - r0 : TR;
    const uint32_t jf = r0 / G, jl = (r0 + rows_here - 1) / G;
    const uint32_t lo_all = row_lo(A, sq.pos0 + jf);
    uint32_t hi_all = sq.last ? sq.last[jl] : sq.pos0 + jl;
    hi_all = hi_all < plast ? hi_all : plast;
    if (t0 > hi_all || t0 + kChunk <= lo_all)
        return;
    const uint32_t rlast = plast - t0;
    const size_t crow = (size_t)kvh * sq.cap + (A.ring ? t0 % sq.cap : t0);
    const uint32_t rbytes = hd * S::EB;
    const char *const kbase = (const char *)sq.k + crow * rbytes;
    const char *const vbase = (const char *)sq.v + crow * rbytes;

    /* the lane's MFMA row in tile mt: row qr = l16 / 2 of the tile, plane
       l16 & 1; its visible positions [rlo, rhi] */
    const uint32_t qr = l16 >> 1;
    uint32_t rlo[MT], rhi[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const uint32_t rq = r0 + kTileRows * mt + qr;
        rlo[mt] = 1;
        rhi[mt] = 0;
        if (rq < R) {
            const uint32_t j = rq / G;
            rlo[mt] = row_lo(A, sq.pos0 + j);
            uint32_t hi = sq.last ? sq.last[j] : sq.pos0 + j;
            rhi[mt] = hi < plast ? hi : plast;
        }
    }

    /* ---- the query: wave w loads rows 2 w, 2 w + 1 of every tile (D / 4
       lanes a row, a float4 each; columns past hd read column 0) ---- */
    constexpr int QL = D / 4;                  /* lanes a query row */
    constexpr int QN = QL >= 64 ? 2 : 1;        /* loads a lane a tile */
    float4 qv[MT][QN];
    uint32_t qrow[QN], qcol[QN];
    /* lanes past the wave's two rows (head size 64) take none */
    const bool qlane = QN == 2 || lane / QL < 2;
#pragma unroll
    for (int h = 0; h < QN; h++) {
        const uint32_t e = QN == 2 ? lane : lane % QL;
        qrow[h] = qlane ? 2 * w + (QN == 2 ? h : lane / QL) : kTileRows;
        qcol[h] = 4 * e;
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int h = 0; h < QN; h++) {
            const uint32_t rr = r0 + kTileRows * mt + qrow[h];
            const uint32_t r = rr < R ? rr : r0;
            const uint32_t j = r / G, hh = kvh * G + r % G;
            const float *src = sq.q + ((size_t)j * A.n_head + hh) * hd;
            qv[mt][h] = *(const float4 *)(src + (qcol[h] < hd ? qcol[h] : 0));
        }
    /* the value and key scales of the wave's 64 positions, a lane each */
    float ksv = 1.0f, vsv = 1.0f;
    if constexpr (S::SCALED) {
        const uint32_t p = w * kSWP + lane;
        const uint32_t at = p < rlast ? p : rlast;
        ksv = sq.ks[crow + at];
        vsv = sq.vs[crow + at];
    }
    __builtin_amdgcn_sched_barrier(0);

    /* ---- K and V, 1 KB a load: load l of group s covers padded bytes
       1024 l + 16 lane of the group's 16 rows ---- */
    u4 kr[kSNG][LG], vr[kSNG][LG];
    uint32_t off[LG];
    bool back[LG];
#pragma unroll
    for (int l = 0; l < LG; l++) {
        const uint32_t b = 1024 * l + 16 * lane;
        const uint32_t row = b / S::MRB, cb = b % S::MRB;
        uint32_t at;
        if constexpr (S::EB == 1) {
            at = unit_at(cb, hd, back[l]);
        } else {
            at = cb < rbytes ? cb : 0;
            back[l] = false;
        }
        off[l] = row * 0x10000u + at; /* row in the high half */
    }
    auto addr = [&](int s, int l) -> uint32_t {
        const uint32_t p = w * kSWP + kSG * s + (off[l] >> 16);
        return __umul24(p < rlast ? p : rlast, rbytes) + (off[l] & 0xFFFF);
    };
    auto kload = [&](int s) {
#pragma unroll
        for (int l = 0; l < LG; l++)
            kr[s][l] = NT ? __builtin_nontemporal_load((const u4 *)(kbase + addr(s, l)))
                          : *(const u4 *)(kbase + addr(s, l));
    };
    auto vload = [&](int s) {
#pragma unroll
        for (int l = 0; l < LG; l++)
            vr[s][l] = NT ? __builtin_nontemporal_load((const u4 *)(vbase + addr(s, l)))
                          : *(const u4 *)(vbase + addr(s, l));
    };
    /* group i of the wave's 8: K groups 0..3, then V groups 0..3 */
    auto issue = [&](int i) {
        if (i < kSNG)
            kload(i);
        else if (i < 2 * kSNG)
            vload(i - kSNG);
    };
    constexpr int NF = S::NF;
    issue(0);
    __builtin_amdgcn_sched_barrier(0);
    issue(1);
    __builtin_amdgcn_sched_barrier(0);

    /* ---- the query planes: scaled by 2^e so that the row's largest |q|
       lies in [2^13, 2^14), split into f16 hi + lo, into LDS ---- */
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int h = 0; h < QN; h++) {
        const uint32_t tr = kTileRows * mt + qrow[h];   /* row of the workgroup */
        const bool ok = r0 + tr < R && qrow[h] < kTileRows;
        const float4 qq = qv[mt][h];
        const float x[4] = {qq.x, qq.y, qq.z, qq.w};
        float mx = 0.0f;
        if (ok && qcol[h] < hd)
            mx = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        /* over the row's QL lanes (16, 32 or 64) */
        static_assert(QL == 16 || QL == 32 || QL == 64, "rows of whole 16-lane groups");
        mx = max_row16(mx);
        if constexpr (QL >= 32)
            mx = max_x16(mx);
        if constexpr (QL >= 64)
            mx = max_x32(mx);
        if constexpr (Q16) {
            /* INT16: the row as int16 with one scale (quant_worker,
               attention.c:820-839), planes x >> 8 and x & 255 */
            const float inv = q16_inv(mx);
            if (qrow[h] < kTileRows) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int32_t qi = ok && qcol[h] < hd ? q16_round(x[e], inv) : 0;
                    if constexpr (RAWK) {
                        sQ8[2 * tr][qcol[h] + e] = (int8_t)(qi >> 8);
                        sQ8[2 * tr + 1][qcol[h] + e] = (int8_t)((qi & 255) - 128);
                    } else {
                        sQ[2 * tr][qcol[h] + e] = (_Float16)(qi >> 8);
                        sQ[2 * tr + 1][qcol[h] + e] = (_Float16)(qi & 255);
                    }
                }
                if (qcol[h] == 0)
                    sQs[tr] = mx / 32767.0f;
            }
            continue;
        }
        int ex = 0;
        if (mx > 0.0f && mx < INFINITY) {
            frexpf(mx, &ex);
            ex = 14 - ex;
        }
        const float up = ldexpf(1.0f, ex);
        if (qrow[h] < kTileRows) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 hi, lo;
                split_hl(ok && qcol[h] < hd ? x[e] * up : 0.0f, hi, lo);
                sQ[2 * tr][qcol[h] + e] = hi;
                sQ[2 * tr + 1][qcol[h] + e] = lo;
            }
            if (qcol[h] == 0)
                sQs[tr] = ldexpf(1.0f, -ex);
        }
    }
    if constexpr (S::SCALED) {
        sKs[w][lane] = ksv;
        sVs[w][lane] = vsv;
    }
    __builtin_amdgcn_sched_barrier(0);
    /* the rest of the groups in flight, now that the query is in */
#pragma unroll
    for (int i = 2; i < NF; i++) {
        issue(i);
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
    h8 qb[MT][KS];
    i4 qb8[MT][KS8];
    float qs2[MT], qsc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        if constexpr (RAWK) {
#pragma unroll
            for (int ks = 0; ks < KS8; ks++)
                qb8[mt][ks] = *(const i4 *)&sQ8[16 * mt + l16][64 * ks + 16 * g];
        } else {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                qb[mt][ks] = *(const h8 *)&sQ[16 * mt + l16][32 * ks + 8 * g];
        }
        qsc[mt] = sQs[kTileRows * mt + qr];
        qs2[mt] = qsc[mt] * A.scale * kLog2e;
    }

    char *const myR = sR + w * CR;
    /* the group's 16 B of row `row`, byte cb of the padded row, into the
       region (16-bit units; int8 widened, f32 split into two planes) */
    auto stage = [&](const u4 &x0, int l) {
        const uint32_t row = off[l] >> 16;
        const uint32_t cb = (1024 * l + 16 * lane) % S::MRB;
        char *rb = myR + row * S::LRB;
        if constexpr (T == kF16 || T == kI16) {
            *(u4 *)(rb + 16 * slot<D>(cb / 16, row)) = x0;
        } else if constexpr (T == kI8) {
            const u4 x = unit_fix(x0, back[l]);
            *(h8 *)(rb + 16 * slot<D>(cb / 8, row)) = Elem<kI8>::widen(x.x, x.y);
            *(h8 *)(rb + 16 * slot<D>(cb / 8 + 1, row)) = Elem<kI8>::widen(x.z, x.w);
        } else {
            h4 hi, lo;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                _Float16 a, b;
                split_hl(__uint_as_float(x0[e]), a, b);
                hi[e] = a;
                lo[e] = b;
            }
            const uint32_t u = cb / 32, half = (cb / 16) & 1;
            *(h4 *)(rb + 16 * slot<D>(u, row) + 8 * half) = hi;
            *(h4 *)(rb + S::PLB + 16 * slot<D>(u, row) + 8 * half) = lo;
        }
    };

    /* a K group's 16 B as they are (RAWK): rows of D bytes, D / 16 units
       swizzled as an f16 row of D / 2 numbers */
    auto stage_raw = [&](const u4 &x0, int l) {
        const uint32_t row = off[l] >> 16;
        const uint32_t cb = (1024 * l + 16 * lane) % S::MRB;
        *(u4 *)(myR + row * D + 16 * slot<D / 2>(cb / 16, row)) = x0;
    };

    /* ---- scores, a group at a time as its K lands (lane: MFMA row l16 at
       positions 16 s + 4 g + i), each K operand read once for the MT
       tiles ---- */
    const uint32_t p0w = t0 + w * kSWP;
    /* whether every row of the tiles that exists sees all 64 positions of
       the wave (a chunk inside every row's range), so that its scores take
       no mask. A row past R is left out; its numbers are never stored. The
       test is the same for the whole wave (a vote), so the branch below is
       a scalar one */
    bool full = false;
    {
        bool seen = true;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            seen = seen && (r0 + kTileRows * mt + qr >= R ||
                            (rlo[mt] <= p0w && p0w + kSWP - 1 <= rhi[mt]));
        full = __builtin_amdgcn_ballot_w64(!seen) == 0;
    }
    /* the scores of the lane's two positions of each group (its row's
       other lane has the other two) */
    float sv[MT][kSNG][2];
    float m[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        m[mt] = -INFINITY;
#pragma unroll
    for (int s = 0; s < kSNG; s++) {
        {
            u4 t[LG];
#pragma unroll
            for (int l = 0; l < LG; l++)
                t[l] = kr[s][l];
            __builtin_amdgcn_sched_barrier(0);
            issue(s + NF);
            __builtin_amdgcn_sched_barrier(0);
            if (s > 0)
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int l = 0; l < LG; l++) {
                if constexpr (RAWK)
                    stage_raw(t[l], l);
                else
                    stage(t[l], l);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (RAWK) {
            /* INT16 on the integer matrix cores: the planes' sums and the
               keys' sums, then the same exact score as below */
            i4 si[MT], sk = i4{0, 0, 0, 0};
            const i4 ones = i4{0x01010101, 0x01010101, 0x01010101, 0x01010101};
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                si[mt] = i4{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < KS8; ks++) {
                const i4 ka = *(const i4 *)(myR + l16 * D + 16 * slot<D / 2>(4 * ks + g, l16));
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    si[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, qb8[mt][ks], si[mt], 0, 0, 0);
                sk = __builtin_amdgcn_mfma_i32_16x16x64_i8(ka, ones, sk, 0, 0, 0);
            }
            const uint32_t b = l16 & 1;
            const float2 kz2 = *(const float2 *)&sKs[w][kSG * s + 4 * g + 2 * b];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t own = (uint32_t)(b ? si[mt][2 + j] : si[mt][j]);
                    const uint32_t nbr = __builtin_amdgcn_update_dpp(
                        0u, (uint32_t)(b ? si[mt][j] : si[mt][2 + j]), 0xB1, 0xf, 0xf, false);
                    const uint32_t ks1 = (uint32_t)(b ? sk[2 + j] : sk[j]);
                    /* 256 hi + (lo - 128) + 128 x the keys' sum, as unsigned
                       words (the int32 sum wraps back into range) */
                    const uint32_t hi = b ? nbr : own, lo = b ? own : nbr;
                    float x = q16_scale((int32_t)(hi * 256u + lo + ks1 * 128u), qsc[mt],
                                        A.scale, j ? kz2.y : kz2.x);
                    const uint32_t p = p0w + kSG * s + 4 * g + 2 * b + j;
                    const bool vis = (p >= rlo[mt]) & (p <= rhi[mt]);
                    sv[mt][s][j] = vis ? x : -INFINITY;
                    m[mt] = fmaxf(m[mt], sv[mt][s][j]);
                }
            continue;
        }
        f4 sa[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            sa[mt] = f4{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            h8 ka[DP];
            const uint32_t sl = 16 * slot<D>(4 * ks + g, l16);
            if constexpr (T == kI16) {
                const uint4 raw = *(const uint4 *)(myR + l16 * S::LRB + sl);
                Elem<kI16>::split(raw, ka[0], ka[1]);
            } else {
                ka[0] = *(const h8 *)(myR + l16 * S::LRB + sl);
                if constexpr (T == kF32)
                    ka[1] = *(const h8 *)(myR + S::PLB + l16 * S::LRB + sl);
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int dp = 0; dp < DP; dp++)
                    sa[mt] = mfma(ka[dp], qb[mt][ks], sa[mt]);
        }
        /* the key scales of the lane's 4 positions, one read for all of
           them (read under the mask below, each was a branch and a wait of
           its own) */
        if constexpr (Q16) {
            /* INT16: lane l16 & 1 = b makes the scores of positions 2 b and
               2 b + 1 of its four, its neighbour (the row's other plane) the
               other two: from its own plane's sum and the neighbour's, in
               natural units, the reference's score bit for bit. So each
               score, weight and quantized weight is made once, not in both
               lanes of a row */
            const uint32_t b = l16 & 1;
            const float2 kz2 = *(const float2 *)&sKs[w][kSG * s + 4 * g + 2 * b];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float own = b ? sa[mt][2 + j] : sa[mt][j];
                    const float nbr = from_x1(b ? sa[mt][j] : sa[mt][2 + j]);
                    float x = q16_score(b ? nbr : own, b ? own : nbr, qsc[mt], A.scale,
                                        j ? kz2.y : kz2.x);
                    const uint32_t p = p0w + kSG * s + 4 * g + 2 * b + j;
                    const bool vis = (p >= rlo[mt]) & (p <= rhi[mt]);
                    sv[mt][s][j] = vis ? x : -INFINITY;
                    m[mt] = fmaxf(m[mt], sv[mt][s][j]);
                }
            continue;
        }
        /* FLOAT: the same split of a row's four positions between its two
           lanes; a score is (high plane's sum + low plane's) x scale, the
           same in both lanes */
        const uint32_t b = l16 & 1;
        float2 kz2 = make_float2(1.0f, 1.0f);
        if constexpr (S::SCALED)
            kz2 = *(const float2 *)&sKs[w][kSG * s + 4 * g + 2 * b];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float y0 = sa[mt][j] + from_x1(sa[mt][j]);
                const float y1 = sa[mt][2 + j] + from_x1(sa[mt][2 + j]);
                float x = (b ? y1 : y0) * qs2[mt];
                if constexpr (S::SCALED)
                    x *= j ? kz2.y : kz2.x;
                sv[mt][s][j] = x;
            }
        /* both bounds tested, then one select: no part of the score under a
           branch of its own; with two row tiles only where a row does not
           see all of the wave's positions */
        if (!full) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t p = p0w + kSG * s + 4 * g + 2 * b + j;
                    const bool vis = (p >= rlo[mt]) & (p <= rhi[mt]);
                    sv[mt][s][j] = vis ? sv[mt][s][j] : -INFINITY;
                }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                m[mt] = fmaxf(m[mt], sv[mt][s][j]);
    }
    /* over the row's two lanes, then its 4 lane groups */
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        m[mt] = max_x32(max_x16(fmaxf(m[mt], from_x1(m[mt]))));
    /* the lane's two positions of each group (2 b, 2 b + 1) and their value
       scales, in registers */
    const uint32_t b = l16 & 1;
    float2 vz2[kSNG];
#pragma unroll
    for (int s = 0; s < kSNG; s++)
        vz2[s] = S::SCALED ? *(const float2 *)&sVs[w][kSG * s + 4 * g + 2 * b] : make_float2(1.0f, 1.0f);
    h4 pa[MT][kSNG];
    if constexpr (Q16) {
        /* INT16: the chunk's largest score over the 4 waves, the weights
           e^(s - M) times the value scales, their largest over the chunk,
           and the weights quantized against it to 0 .. 32767, planes
           w >> 8 and w & 255 (att_weights_ref, att_wquant_ref,
           attention.c:158-176, :574-588, :761-772) */
        if (lane < 16 && !(lane & 1))
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                sM[w][kTileRows * mt + (lane >> 1)] = m[mt];
        __syncthreads();
        float pv[MT][kSNG][2];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t rr = kTileRows * mt + qr;
            m[mt] = fmaxf(fmaxf(sM[0][rr], sM[1][rr]), fmaxf(sM[2][rr], sM[3][rr]));
            const float mm = m[mt] == -INFINITY ? 0.0f : m[mt];
            float lsum = 0.0f, vmx = 0.0f;
#pragma unroll
            for (int s = 0; s < kSNG; s++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float wt = det_weight(sv[mt][s][j], mm);
                    lsum += wt;
                    pv[mt][s][j] = wt * (j ? vz2[s].y : vz2[s].x);
                    vmx = fmaxf(vmx, pv[mt][s][j]);
                }
            vmx = max_x32(max_x16(fmaxf(vmx, from_x1(vmx))));
            lsum = sum_x32(sum_x16(lsum + from_x1(lsum)));
            if (lane < 16 && !(lane & 1)) {
                sX[w][kTileRows * mt + (lane >> 1)] = vmx;
                sL[w][kTileRows * mt + (lane >> 1)] = lsum;
            }
        }
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t rr = kTileRows * mt + qr;
            const float inv = q16_inv(fmaxf(fmaxf(sX[0][rr], sX[1][rr]), fmaxf(sX[2][rr], sX[3][rr])));
            /* the lane's plane (b = 0: w >> 8, 1: w & 255) of all four
               positions: its own two quantized weights and its neighbour's */
            const uint32_t sh = b ? 0 : 8;
#pragma unroll
            for (int s = 0; s < kSNG; s++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const uint32_t q = (uint32_t)q16_round(pv[mt][s][j], inv);
                    const uint32_t r = __builtin_amdgcn_update_dpp(0u, q, 0xB1, 0xf, 0xf, false);
                    pa[mt][s][j] = (_Float16)(float)(((b ? r : q) >> sh) & 255);
                    pa[mt][s][2 + j] = (_Float16)(float)(((b ? q : r) >> sh) & 255);
                }
        }
    }

    /* ---- the wave's softmax (powers of two); the weights' power of two
       puts their largest (times the largest value scale) in [2^12, 2^13) */
    int pe = 13;
    if constexpr (S::SCALED && !Q16) {
        float vm = 0.0f;
#pragma unroll
        for (int s = 0; s < kSNG; s++)
            vm = fmaxf(vm, fmaxf(vz2[s].x, vz2[s].y));
        vm = max_x32(max_x16(fmaxf(vm, from_x1(vm))));
        int ev = 0;
        if (vm > 0.0f && vm < INFINITY)
            frexpf(vm, &ev);
        pe = 13 - ev;
    }
    if constexpr (!Q16) {
        const float up = ldexpf(1.0f, pe);
        /* a lane makes both f16 planes of its own two weights, hi = f16(pv)
           and lo = f16(pv - hi), each as one multiply-add rounded once to
           f16 (pv - 0 hi is pv, and pv - hi is exact in f32: split_hl's
           planes); it keeps its row plane's (b = 0: hi, 1: lo) and swaps the
           other for its neighbour's, so it holds its plane of all four */
        const float keepf = b ? -1.0f : -0.0f, sendf = b ? 0.0f : -1.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float mm = m[mt] == -INFINITY ? 0.0f : m[mt];
            float lsum = 0.0f;
#pragma unroll
            for (int s = 0; s < kSNG; s++) {
                h2 keep, send;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    /* the reference's cutoff (a weight below e^-80 is 0,
                       attention.c:580) needs no test here: such a weight is
                       below 2^-115, its planes are f16 zeros (pv is below
                       2^-102), and it cannot change a sum that holds the
                       wave's largest weight, 1 (a masked score gives
                       exp2(-inf) = 0) */
                    const float d = sv[mt][s][j] - mm;
                    const float pw = __builtin_amdgcn_exp2f(d);
                    lsum += pw;
                    float pv = pw * up;
                    if constexpr (S::SCALED)
                        pv *= j ? vz2[s].y : vz2[s].x;
                    /* pv as rounded (no product fused into the conversion) */
                    asm volatile("" : "+v"(pv));
                    const float hi = (float)(_Float16)pv;
                    keep[j] = (_Float16)__builtin_fmaf(keepf, hi, pv);
                    send[j] = (_Float16)__builtin_fmaf(sendf, hi, pv);
                }
                const uint32_t kept = __builtin_bit_cast(uint32_t, keep);
                const uint32_t got = __builtin_amdgcn_update_dpp(
                    0u, __builtin_bit_cast(uint32_t, send), 0xB1, 0xf, 0xf, false);
                pa[mt][s] = __builtin_bit_cast(h4, make_uint2(b ? got : kept, b ? kept : got));
            }
            lsum = sum_x32(sum_x16(lsum + from_x1(lsum)));
            if (lane < 16 && !(lane & 1)) {
                sM[w][kTileRows * mt + (lane >> 1)] = m[mt];
                sL[w][kTileRows * mt + (lane >> 1)] = lsum;
            }
        }
        if (lane == 0)
            sPe[w] = ldexpf(1.0f, -pe);
    }

    /* ---- values, a group at a time as its V lands, each V operand read
       once for the MT tiles ---- */
    f4 o[MT][NT_];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NT_; t++)
            o[mt][t] = f4{0, 0, 0, 0};
    const uint32_t r1 = 4 * g + (l16 >> 2);
#pragma unroll
    for (int s = 0; s < kSNG; s++) {
        {
            u4 t[LG];
#pragma unroll
            for (int l = 0; l < LG; l++)
                t[l] = vr[s][l];
            __builtin_amdgcn_sched_barrier(0);
            issue(kSNG + s + NF);
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int l = 0; l < LG; l++)
                stage(t[l], l);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        h4 vb[NT_][DP];
#pragma unroll
        for (int t = 0; t < NT_; t++) {
            const uint32_t cc = 16 * t + 4 * (l16 & 3);
            const uint32_t a = r1 * S::LRB + 16 * slot<D>(cc / 8, r1) + (cc % 8) * 2;
            if constexpr (T == kI16) {
                const h4 x = lds_read_tr((const _Float16 *)(myR + a));
                const uint2 u = __builtin_bit_cast(uint2, x);
                i16_planes4(u.x, u.y, vb[t][0], vb[t][1]);
            } else {
                vb[t][0] = lds_read_tr((const _Float16 *)(myR + a));
                if constexpr (T == kF32)
                    vb[t][1] = lds_read_tr((const _Float16 *)(myR + S::PLB + a));
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int t = 0; t < NT_; t++)
#pragma unroll
                for (int dp = 0; dp < DP; dp++)
                    o[mt][t] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[mt][s], vb[t][dp], o[mt][t], 0, 0, 0);
    }

    /* ---- the waves combined: tile row 2 g + h's sums are o[t][2 h] +
       o[t][2 h + 1] (high and low weights); into the region, then wave w
       sums its column tiles over the waves with weights 2^(m_w - M)
       2^-pe_w ---- */
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float2 *mine = (float2 *)myR;
    const uint64_t prow0 = sq.part0 + ((uint64_t)kvh * sq.span + (c - sq.c0)) * R + r0;
    /* lane jj of a tile: source lanes 2 jj, 2 jj + 1 - tile rows 2 gs,
       2 gs + 1 of columns cs, cs + 1 */
    const uint32_t jj = lane & 31, gs = jj >> 3;
    {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NT_; t++) {
            if constexpr (Q16) {
                /* exact integer sums, 256 hi + lo as int32 bits (at most 64
                   positions of 32767 x 128: no overflow) */
                const int32_t a0 = (int32_t)o[mt][t][0] * 256 + (int32_t)o[mt][t][1];
                const int32_t a1 = (int32_t)o[mt][t][2] * 256 + (int32_t)o[mt][t][3];
                mine[(mt * NT_ + t) * 64 + lane] = make_float2(__int_as_float(a0), __int_as_float(a1));
            } else {
                mine[(mt * NT_ + t) * 64 + lane] =
                    make_float2(o[mt][t][0] + o[mt][t][1], o[mt][t][2] + o[mt][t][3]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const uint32_t rb = kTileRows * mt;   /* the tile's first row */
            float fw[kSW][2], wsc[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t rr = rb + 2 * gs + h;
                if constexpr (Q16) {
                    /* the weights' scale, mx / 32767 (att_wquant_ref) */
                    wsc[h] = fmaxf(fmaxf(sX[0][rr], sX[1][rr]), fmaxf(sX[2][rr], sX[3][rr])) / 32767.0f;
                    continue;
                }
                float mx = -INFINITY;
#pragma unroll
                for (int ww = 0; ww < kSW; ww++)
                    mx = fmaxf(mx, sM[ww][rr]);
#pragma unroll
                for (int ww = 0; ww < kSW; ww++) {
                    const float mw = sM[ww][rr];
                    fw[ww][h] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mx) * sPe[ww];
                }
            }
            constexpr int TPW = NT_ / kSW;   /* column tiles a wave: 1, 2 or 4 */
#pragma unroll
            for (int tt = 0; tt < (TPW + 1) / 2; tt++) {
                const uint32_t t = TPW * w + 2 * tt + (lane >> 5);
                if (TPW == 1 && lane >= 32)
                    break;
                const uint32_t cs = 16 * t + ((2 * jj) & 15);
                f4 part[kSW];
#pragma unroll
                for (int ww = 0; ww < kSW; ww++)
                    part[ww] = ((const f4 *)(sR + ww * CR))[(mt * NT_ + t) * 32 + jj];
                float res[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if constexpr (Q16) {
                        /* the chunk's exact int32 sum, then one multiply
                           (att_values_i16_ref, attention.c:178-193) */
                        const int32_t acc = (__float_as_int(part[0][i]) + __float_as_int(part[1][i])) +
                                            (__float_as_int(part[2][i]) + __float_as_int(part[3][i]));
                        res[i] = (float)acc * wsc[i % 2];
                    } else {
                        res[i] = (part[0][i] * fw[0][i % 2] + part[1][i] * fw[1][i % 2]) +
                                 (part[2][i] * fw[2][i % 2] + part[3][i] * fw[3][i % 2]);
                    }
                }
                if (cs < hd) {
                    const uint32_t ra = rb + 2 * gs;
                    if (r0 + ra < R)
                        *(float2 *)&A.part_acc[(prow0 + ra) * hd + cs] = make_float2(res[0], res[2]);
                    if (r0 + ra + 1 < R)
                        *(float2 *)&A.part_acc[(prow0 + ra + 1) * hd + cs] = make_float2(res[1], res[3]);
                }
            }
        }
    }
    if (w == 0 && lane < TR && r0 + lane < R) {
        float mc = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < kSW; ww++)
            mc = fmaxf(mc, sM[ww][lane]);
        float l[kSW];
#pragma unroll
        for (int ww = 0; ww < kSW; ww++) {
            const float mw = sM[ww][lane];
            if constexpr (Q16)
                l[ww] = sL[ww][lane]; /* already against the chunk's M */
            else
                l[ww] = (mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mc)) * sL[ww][lane];
        }
        /* INT16's largest score is in natural units: to powers of two for
           the merge */
        if constexpr (Q16)
            mc *= kLog2e;
        *(float2 *)&A.part_ml[(prow0 + lane) * 2] = make_float2(mc, (l[0] + l[1]) + (l[2] + l[3]));
    }
}

/*
 * Merge of the chunk partials of (token j, query head h), 32 or 128 columns
 * a workgroup (attention.c:870-910). Group g of 8 (32 lanes each, a lane
 * CPL columns) takes chunks g, g + 8, ... of the token's range, 16 at a
 * time in one batch of loads: their largest score M_g, then
 * sum_c e^(m_c - M_g) l_c and acc_c in chunk order. The groups are combined
 * with weights e^(M_g - M) as ((g0 + g1) + (g2 + g3)) + ((g4 + g5) +
 * (g6 + g7)). The order depends only on the token's own chunk range, so a
 * token merges the same way in any block. The gate sigmoid(g) * o is
 * applied on the way out.
 *
 * Q8K: a workgroup takes one block of 256 of the token's n_head x hd
 * outputs instead (a lane 8 consecutive ones, of one head since hd is a
 * multiple of 8), merges them with the same arithmetic column by column -
 * so the outputs are the same bits - and quantizes them into the block's
 * Q8_K (attn_merge.comp:78-138 does the same in the reference's GPU path):
 * no pass of its own for the quantization.
 */
constexpr int kMergeGroups = 8;
constexpr int kMergeLanes = 32;            /* lanes a group */

/* the 4 columns of a float4, one by one */
__device__ __forceinline__ float &f4e(float4 &v, int e)
{
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

/*
 * CPL columns a lane (1, 4 or 8: 32, 128 or 256 columns a workgroup). Each
 * column's arithmetic is the same in all, so a token's output does not
 * depend on the instance its call takes; 4 when a launch has (token, head)
 * pairs enough to fill the GPU with 4 times fewer workgroups (blocks of
 * tokens), 1 when it has few (a decode spreads its loads over more CUs), 8
 * with Q8K.
 *
 * NB chunks a group's batch (2, 3, 4, 6, 8, 12 or 16): every load of a batch is issued
 * at once, and chunks past the row's range load its last chunk again and
 * enter with weight 0. Those are exact no-ops (the sums start at +0 and
 * never become -0, so adding 0 x v or 0 x l leaves them as they are), so
 * a row whose chunks fit one batch gets the same bits from any NB; the
 * launch takes the smallest NB whose batch holds its longest span, and a
 * short context does not issue 16 loads a group for a few chunks.
 */
template <int CPL, bool ONE = false, bool Q8K = false, int NB = 16>
__global__ __launch_bounds__(256) void merge_kernel(const SplitArgs A)
{
    static_assert(CPL == 1 || CPL == 4 || CPL == 8, "1, 4 or 8 columns a lane");
    static_assert(!Q8K || CPL == 8, "a Q8_K block: 256 columns");
    constexpr int NV = CPL >= 4 ? CPL / 4 : 1;  /* float4s a lane */
    constexpr uint32_t kCols = kMergeLanes * CPL;
    /* a lane's own largest score and sum (with Q8K the lanes of a
       workgroup may belong to different heads) */
    __shared__ float sM[kMergeGroups][kMergeLanes], sL[kMergeGroups][kMergeLanes];
    __shared__ float4 sAcc[kMergeGroups][NV][kMergeLanes];
    __shared__ float sOut[Q8K ? 256 : 1];
    __shared__ Q8kLds sQ;
    if constexpr (!ONE)
        starts_early(A.n_wg, A.n_wg, A.n_seqs, A.mg0s);
    const uint32_t id = blockIdx.x, tid = threadIdx.x;
    const uint32_t g = tid / kMergeLanes, cl = tid % kMergeLanes;
    uint32_t si = 0;
    if constexpr (!ONE)
        si = seq_index(A.mg0s, A.n_seqs, id);
    const SeqDesc &sq = A.seq[si];
    const uint32_t hd = A.hd, G = A.group;
    const uint32_t local = id - sq.mg0;
    /* the lane's token j, head h and columns col .. col + CPL - 1 (hd is a
       multiple of 8: all are inside the row or none is) */
    uint32_t j, h, col, blk = 0;
    if constexpr (Q8K) {
        const uint32_t nb = A.n_head * hd / 256;   /* blocks a token */
        j = local / nb;
        blk = local % nb;
        const uint32_t e0 = 256 * blk + CPL * cl;
        h = e0 / hd;
        col = e0 % hd;
    } else {
        const uint32_t nd = (hd + kCols - 1) / kCols, db = local % nd;
        h = (local / nd) % A.n_head;
        j = local / nd / A.n_head;
        col = db * kCols + CPL * cl;
    }
    const uint32_t kvh = h / G, r = j * G + h % G, R = sq.n * G;
    const uint32_t pos = sq.pos0 + j;
    /* last[] past the call's end would read partials of other rows */
    uint32_t hi = sq.last ? sq.last[j] : pos;
    hi = hi < sq.end - 1 ? hi : sq.end - 1;
    const uint32_t lo = row_lo(A, pos);
    const uint32_t clo = lo / kChunk, nc = hi / kChunk - clo + 1;
    /* partial row of chunk clo + i */
    const uint64_t base = sq.part0 + ((uint64_t)kvh * sq.span + (clo - sq.c0)) * R + r;
    const bool colok = col < hd;
    /* the gate, asked for with the partials so the loads overlap: branch-
       free (a load under a branch is waited for where the branches join,
       before the partials' loads), from a valid dummy address when unused */
    const size_t oi = ((size_t)j * A.n_head + h) * hd + col;
    const bool gel = A.gate_mode == kGateElem && colok;
    const float *gsrc = gel ? sq.gate + oi : A.part_ml;
    const float *hsrc = A.gate_mode == kGateHead ? sq.gate + (size_t)j * A.n_head + h
                                                 : A.part_ml;
    float4 gv[NV];
#pragma unroll
    for (int u = 0; u < NV; u++)
        gv[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (CPL >= 4) {
#pragma unroll
        for (int u = 0; u < NV; u++)
            gv[u] = ((const float4 *)gsrc)[gel ? u : 0];
    } else {
        gv[0].x = *gsrc;
    }
    /* the same for the per-head gate: its address is the same in every
       lane, and the compiler would make it a scalar load, for which the
       partials' loads then wait (their addresses need the scalar counter
       at zero); an opaque zero offset keeps it a vector load like the
       others */
    uint32_t z0;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z0));
    const float gh = hsrc[z0];
    float mg = -INFINITY, lg = 0.0f;
    float4 ag[NV];
#pragma unroll
    for (int u = 0; u < NV; u++)
        ag[u] = float4{0.0f, 0.0f, 0.0f, 0.0f};
    /* the lane's addresses in chunk clo; a chunk's rows are R further on
       (one multiply-add a load) */
    const char *const ml0 = (const char *)((const float2 *)A.part_ml + base);
    const char *const acc0 = (const char *)(A.part_acc + base * hd + (colok ? col : 0));
    const uint32_t rml = R * 8, racc = R * hd * 4;   /* bytes a chunk */
    for (uint32_t i0 = g; i0 < nc; i0 += kMergeGroups * NB) {
        float2 ml[NB];
        float4 v[NB][NV];
        /* branch-free: chunks past the range read the last one, weight 0 */
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t i = i0 + kMergeGroups * b < nc ? i0 + kMergeGroups * b : nc - 1;
            ml[b] = *(const float2 *)(ml0 + (uint64_t)i * rml);
            const float *src = (const float *)(acc0 + (uint64_t)i * racc);
            if constexpr (CPL >= 4) {
#pragma unroll
                for (int u = 0; u < NV; u++)
                    v[b][u] = ((const float4 *)src)[u];
            } else {
                v[b][0].x = *src;
            }
        }
        float mb = mg;
#pragma unroll
        for (int b = 0; b < NB; b++)
            if (i0 + kMergeGroups * b < nc)
                mb = fmaxf(mb, ml[b].x);
        /* the batch's sums, against the group's new largest score (scores
           in powers of two) */
        const float f = mg == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mg - mb);
        lg *= f;
#pragma unroll
        for (int e = 0; e < CPL; e++)
            f4e(ag[e / 4], e % 4) *= f;
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const float wgt = i0 + kMergeGroups * b < nc ? __builtin_amdgcn_exp2f(ml[b].x - mb) : 0.0f;
            lg += wgt * ml[b].y;
#pragma unroll
            for (int e = 0; e < CPL; e++)
                f4e(ag[e / 4], e % 4) = fmaf(wgt, f4e(v[b][e / 4], e % 4), f4e(ag[e / 4], e % 4));
        }
        mg = mb;
    }
    /* the gate's sigmoid, made by group 0 while the other groups finish
       (not after the barrier, on the way to the store) */
    float sig[CPL];
#pragma unroll
    for (int e = 0; e < CPL; e++) {
        sig[e] = 1.0f;
        if (g == 0) {
            if (A.gate_mode == kGateElem)
                sig[e] = 1.0f / (1.0f + expf(-f4e(gv[e / 4], e % 4)));
            else if (A.gate_mode == kGateHead)
                sig[e] = 1.0f / (1.0f + expf(-gh));
        }
    }
    sM[g][cl] = mg;
    sL[g][cl] = lg;
#pragma unroll
    for (int u = 0; u < NV; u++)
        sAcc[g][u][cl] = ag[u];
    __syncthreads();
    if (g == 0 && colok) {
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kMergeGroups; k++)
            mx = fmaxf(mx, sM[k][cl]);
        float wl[kMergeGroups], wk[kMergeGroups];
#pragma unroll
        for (int k = 0; k < kMergeGroups; k++) {
            wk[k] = sM[k][cl] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sM[k][cl] - mx);
            wl[k] = wk[k] * sL[k][cl];
        }
        if (A.skip && col == 0) {
            /* JANAS_ATTN_SKIPSTAT: how many of the row's chunks lie more
               than 8, 16 or 32 (natural units; m is in powers of two) below
               its largest score, as merge_one counts them
               (attention.c:883-898): from the call's first chunk, so the
               chunks before the token's own window count as below, and n
               counts from chunk 0 */
            unsigned long long k[3] = {clo - sq.c0, clo - sq.c0, clo - sq.c0};
            for (uint32_t i = 0; i < nc; i++) {
                const float mi = A.part_ml[(base + (uint64_t)i * R) * 2];
                k[0] += mi < mx - 8.0f * kLog2e;
                k[1] += mi < mx - 16.0f * kLog2e;
                k[2] += mi < mx - 32.0f * kLog2e;
            }
            for (int wq = 0; wq < 2; wq++) {
                if (wq == 1 && pos < 16384)
                    break;
                atomicAdd(&A.skip[wq], (unsigned long long)(hi / kChunk + 1));
#pragma unroll
                for (int t = 0; t < 3; t++)
                    atomicAdd(&A.skip[2 + 3 * wq + t], k[t]);
            }
        }
        const float sum = ((wl[0] + wl[1]) + (wl[2] + wl[3])) + ((wl[4] + wl[5]) + (wl[6] + wl[7]));
        const float inv = 1.0f / sum;
        float4 o[NV];
#pragma unroll
        for (int e = 0; e < CPL; e++) {
            float x[kMergeGroups];
#pragma unroll
            for (int k = 0; k < kMergeGroups; k++) {
                float4 a = sAcc[k][e / 4][cl];
                x[k] = wk[k] * f4e(a, e % 4);
            }
            float y = (((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]))) * inv;
            if (A.gate_mode != kGateNone)
                y *= sig[e];
            f4e(o[e / 4], e % 4) = y;
            if constexpr (Q8K)
                sOut[CPL * cl + e] = y;
        }
        if constexpr (CPL >= 4) {
#pragma unroll
            for (int u = 0; u < NV; u++)
                ((float4 *)(sq.out + oi))[u] = o[u];
        } else {
            sq.out[oi] = o[0].x;
        }
    }
    if constexpr (Q8K) {
        /* every thread: the block's number tid, quantized (the same bits
           as the Q8_K pass over the output) */
        if (sq.q8k == nullptr)
            return;  /* a sequence of the launch that asked for none */
        __syncthreads();
        const uint32_t nb = A.n_head * hd / 256;
        q8k_block(sOut[tid], tid, (uint8_t *)sq.q8k + ((size_t)j * nb + blk) * kQ8kBytes, sQ);
    }
}

template <int T, int D, bool Q16, int MT>
hipError_t launch_m(const SplitArgs &a, hipStream_t s)
{
    /* one sequence: its descriptor with the first arguments (a verify or a
       64-token block 3 % faster than reading it after the count) */
    const bool one = a.n_seqs == 1;
    if (a.once && one)
        hipLaunchKernelGGL((split_kernel<T, D, true, true, Q16, MT>), dim3(a.n_wg), dim3(kSW * 64), 0, s, a);
    else if (a.once)
        hipLaunchKernelGGL((split_kernel<T, D, true, false, Q16, MT>), dim3(a.n_wg), dim3(kSW * 64), 0, s, a);
    else if (one)
        hipLaunchKernelGGL((split_kernel<T, D, false, true, Q16, MT>), dim3(a.n_wg), dim3(kSW * 64), 0, s, a);
    else
        hipLaunchKernelGGL((split_kernel<T, D, false, false, Q16, MT>), dim3(a.n_wg), dim3(kSW * 64), 0, s, a);
    return hipGetLastError();
}

template <int T, int D, bool Q16>
hipError_t launch_q(const SplitArgs &a, hipStream_t s)
{
    if constexpr (D <= 128 && T != kF32) {
        if (a.mt == 2)
            return launch_m<T, D, Q16, 2>(a, s);
    }
    if (a.mt != 1)
        return hipErrorInvalidValue;
    return launch_m<T, D, Q16, 1>(a, s);
}

template <int T, int D>
hipError_t launch_t(const SplitArgs &a, hipStream_t s)
{
    if constexpr (T == kI8 && D % 16 == 0) {
        if (a.int16)
            return launch_q<T, D, true>(a, s);
    }
    return launch_q<T, D, false>(a, s);
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
       16-bit rows above 256 take the wide kernel (attn_wide.hip). An int8
       row is read 16 bytes at a time, so it needs 16 bytes at least. */
    return kv >= kI8 && kv <= kF32 && hd >= (kv == kI8 ? 16u : 8u) && hd % 8 == 0 &&
           hd <= (kv == kF32 ? 128u : 512u);
}

uint32_t split_mt(int kv, uint32_t hd, uint32_t tiles)
{
    /* row tiles a workgroup: two when a KV head's rows fill them, for 8-
       and 16-bit rows up to 128 numbers. Four (one workgroup for a verify's
       32 rows) measured slower than two: each wave's chain of products and
       softmax grows with its tiles, and this kernel is bound by that chain,
       not by the matrix cores' rate (8 drafts over 8k positions, 32 / 8 /
       128: one tile 15.1 us, two 14.1, four 16.2). Four for blocks of 16
       tokens or more only was no better: at one wave a SIMD (215 + 192
       registers) 64 tokens at 4096 positions took 67.7 us against 47.5,
       the same bits. Above 128 the sums of two tiles would not fit beside
       the staged rows. */
    if (kv == kF32 || hd > 128)
        return 1;
    uint32_t mt = 1;
    while (mt < tiles && mt < kSplitMaxMt)
        mt *= 2;
    return mt;
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

template <int NB>
hipError_t launch_merge_nb(const SplitArgs &a, uint32_t n_wg, hipStream_t s)
{
    const bool one = a.n_seqs == 1;
    if (a.merge_cols == kMergeQ8k && one)
        hipLaunchKernelGGL((merge_kernel<8, true, true, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == kMergeQ8k)
        hipLaunchKernelGGL((merge_kernel<8, false, true, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 128 && one)
        hipLaunchKernelGGL((merge_kernel<4, true, false, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 128)
        hipLaunchKernelGGL((merge_kernel<4, false, false, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 32 && one)
        hipLaunchKernelGGL((merge_kernel<1, true, false, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else if (a.merge_cols == 32)
        hipLaunchKernelGGL((merge_kernel<1, false, false, NB>), dim3(n_wg), dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_merge(const SplitArgs &a, uint32_t n_wg, hipStream_t s)
{
    /* a row reads at most its sequence's span of chunks: the batch that
       holds the launch's longest span in one round */
    uint32_t span = 0;
    for (uint32_t i = 0; i < a.n_seqs && i < kMaxSeqs; i++)
        span = a.seq[i].span > span ? a.seq[i].span : span;
    if (span <= kMergeGroups * 2)
        return launch_merge_nb<2>(a, n_wg, s);
    if (span <= kMergeGroups * 3)
        return launch_merge_nb<3>(a, n_wg, s);
    if (span <= kMergeGroups * 4)
        return launch_merge_nb<4>(a, n_wg, s);
    if (span <= kMergeGroups * 6)
        return launch_merge_nb<6>(a, n_wg, s);
    if (span <= kMergeGroups * 8)
        return launch_merge_nb<8>(a, n_wg, s);
    if (span <= kMergeGroups * 12)
        return launch_merge_nb<12>(a, n_wg, s);
    return launch_merge_nb<16>(a, n_wg, s);
}

}  // namespace janas
