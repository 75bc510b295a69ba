/*
 * attn_prefill.hip - causal attention of whole prompts over the KV cache on
 * CDNA4 (gfx950): prefill and chunked prefill, where the work is matrix
 * products rather than bandwidth.
 *
 * The reference runs a prompt as calls of up to 64 tokens through the same
 * chunked attention as decoding (model_attn.c:284-294, attention.c:25-36);
 * this kernel computes the same function - token j of a call sees positions
 * lo_j .. hi_j (window start, its own position or set_last's last[j]) - as
 * one pass of an online softmax over key tiles, which is what keeps the
 * matrix cores busy:
 *
 *   workgroup   8 waves, 256 query rows = 64 tokens x the 4 (or G) query
 *               heads of one KV head, so each K/V tile is read once for the
 *               whole GQA group (head size 256: 4 waves, 128 rows, one wave
 *               a SIMD with 512 registers, and 64-position key tiles; head
 *               size 512: 4 waves as 2 row groups x 2 column halves, 64
 *               rows, 32-position tiles). Row blocks of later tokens (more
 *               keys to see) are dispatched first; a KV head's blocks go to
 *               one group of XCDs (they share its L2s), dealt round robin
 *               among them so that each XCD gets long and short blocks.
 *               Calls too small to fill the GPU take prefill_half_kernel:
 *               128 rows a workgroup as two key groups of 4 waves, each
 *               over half of the key tiles, combined in LDS at the end.
 *   key tiles   128 positions of K and V in LDS, two buffers; the next
 *               tile is loaded while this one is computed. 128 rather than
 *               64 positions: the tile's fixed costs (barriers, the row
 *               maximum's exchange) spread over twice the products (+3 %).
 *               Two kernels differ only in how a tile reaches LDS:
 *               prefill_dma_kernel (f16, head sizes up to 256) loads it
 *               straight from memory into XOR-swizzled LDS rows
 *               (global_load_lds_dwordx4; one barrier a tile) and keeps its
 *               operand reads a k-step ahead of the products;
 *               prefill_kernel (int8 / int16, dequantized with their scales
 *               as they are staged, and head sizes up to 64) goes through
 *               registers into padded rows.
 *   scores      S^T = K . Q^T on v_mfma_f32_32x32x16_f16: A = K rows from
 *               LDS, B = the query in f16, scaled by the score scale times
 *               log2(e) so that the weights are exp2(s - m). Lane l holds
 *               32 positions of row l % 32 - already the B layout of the
 *               value product.
 *   softmax     one lane's row state (maximum m, sum) with a lazy maximum:
 *               m moves only when a score passes it by more than 8, which
 *               keeps the weights inside f16 and skips almost every
 *               rescaling; the accumulators start at -m, so no subtraction.
 *   values      O^T += V^T . P^T with the weights in f16 as they are, V rows
 *               read back transposed (ds_read_b64_tr_b16); a row's output
 *               stays in the lane that holds its softmax state.
 *   masks       only the tiles a row's range cuts; tiles wholly outside
 *               every row's range are not visited.
 *   segments    a call whose row blocks alone would leave compute units
 *               idle (a short prompt, a 512-token chunk of a long one)
 *               splits each block's key tiles into nseg contiguous
 *               segments, one workgroup each; a segment leaves its rows'
 *               partials (m, sum, unnormalised values) and pmerge_kernel
 *               folds them in segment order. nseg is the host's choice per
 *               sequence (attn_api.cpp), from the sequence and the
 *               device's compute units alone.
 *   epilogue    O / sum, the output gate sigmoid(g) * o (model_attn.c:
 *               159-170) fused in.
 *
 * The query and the weights enter the products as f16 (11 significant bits)
 * - the f16 cache's own precision; the error stays within the 2e-3 bar the
 * f16 paths are held to.
 */
#include <math.h>
#include <stdint.h>

#include <hip/hip_runtime.h>

#include "attn_kernels.h"
#include "attn_planes.h"
#include "attn_q8k.h"

namespace janas {
namespace {

typedef float f16x __attribute__((ext_vector_type(16)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kPRows = 32;                 /* query rows a wave */

/* waves a workgroup and key positions a tile: 8 and 128 up to head size
   128; 4 (one a SIMD, 512 registers: a 256-column row's output alone is
   128 of them) and 64 (LDS) at 256; at 512 the 4 waves are 2 row groups of
   2 column halves (CS): both waves of a row group take its scores and
   softmax, each the value product and the output of 256 columns, over
   32-position tiles; each takes the score product over its own 256 columns
   of the head and the two partial scores meet in LDS */
/* HV (halves, head sizes 72..128, calls whose row blocks would leave
   compute units idle): the 8 waves are two key groups of 4 over the same
   128 rows, each taking half of the block's key tiles of 64 positions; the
   two halves' states are combined in LDS at the end */
/* EX (the exact kernel over an int8 / int16 cache, prefill_exact_kernel):
   the planes each key and value row enters the products as, 1 (int8) or 2
   (int16); 64-position tiles (32 at head size 256 with two planes, for
   LDS), and 4 waves, one a SIMD, where two planes' operands would not fit
   two waves' registers */
template <int D, bool HV = false, int EX = 0> struct PCfg {
    static_assert(!HV || D == 128, "halves: head sizes 72..128");
    static_assert(!HV || !EX, "halves: f16 only");
    static constexpr int W = D > 128 || (EX == 2 && D > 64) ? 4 : 8;
    static constexpr int GW = HV ? 4 : W;   /* waves a key group */
    static constexpr int TILE = EX == 2 && D == 256 ? 32
                              : HV || EX ? 64 : D > 256 ? 32 : D > 128 ? 64 : 128;
    static constexpr int NPB = TILE / 32;   /* blocks of 32 positions a tile */
    static constexpr int CS = D > 256 ? 2 : 1;  /* column splits of a row */
    static constexpr int OC = D / CS;       /* output columns a wave */
    static constexpr int BLOCK = GW / CS * kPRows; /* query rows a workgroup */
};
constexpr float kLog2e = 1.4426950408889634f;
/* a row's weights are exp2(s - m) against a maximum m that is only moved
   when a score passes it by more than this (so weights stay below 2^8,
   well inside f16) - most tiles then need no rescaling */
constexpr float kSlack = 8.0f;

/* v_mfma_f32_32x32x16_f16: lane l holds A[l % 32][8 (l / 32) .. + 7],
   B[8 (l / 32) .. + 7][l % 32] and D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32] */
__device__ __forceinline__ f16x mfma(h8 a, h8 b, f16x c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

/* ds_read_b64_tr_b16 (see attn_split.hip): lane k of a 16-lane group
   points at row base + k / 4, column c0 + 4 (k % 4); lane l receives rows
   base .. base + 3 of column c0 + l % 16 */
__device__ __forceinline__ h4 lds_read_tr(const _Float16 *p)
{
    s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s4 *)p);
    return __builtin_bit_cast(h4, v);
}

/*
 * Workgroup ids for the 8 XCDs (blocks are dealt to them round robin) in
 * groups of S (1, 2, 4 or 8): group j takes a contiguous run of logical
 * ids, dealt round robin among its S XCDs (S = 1: each XCD a contiguous
 * run; S = 8: the hardware's own order). Block bid = 8 k + x, x = S j + m,
 * is the group's block k S + m; the groups before j hold j S q + min(r, j S)
 * blocks (n = 8 q + r). A run of ids whose lengths fall from first to last
 * (the prefill's row blocks of a KV head) is then shared evenly by the
 * group's XCDs, which still see one KV head's keys.
 */
__device__ __forceinline__ uint32_t xcd_remap_striped(uint32_t bid, uint32_t n, uint32_t S)
{
    const uint32_t x = bid % 8, k = bid / 8, q = n / 8, r = n % 8;
    const uint32_t j = x / S, m = x % S, js = j * S;
    return js * q + (js < r ? js : r) + k * S + m;
}

__device__ __forceinline__ uint32_t row_lo(const PrefillArgs &A, uint32_t pos)
{
    return A.window && pos + 1 > A.window ? pos + 1 - A.window : 0;
}

/*
 * The cache's element types as the kernel stages them: 8 consecutive numbers
 * of a row (a 16-byte LDS store of f16) from their raw bytes. f16 is stored
 * as it is; int8 and int16 are dequantized with the position's scale into
 * f16 - the number the cache stands for, at f16's 11 bits.
 */
template <int T> struct PElem;
template <> struct PElem<kF16> {
    typedef u4 Raw;
    static constexpr bool SCALED = false;
    static constexpr uint32_t EB = 2;
    __device__ static Raw load(const char *b, uint32_t off)
    {
        return *(const u4 *)(b + off);
    }
    __device__ static u4 to_f16(const Raw &r, float) { return r; }
};
template <> struct PElem<kI8> {
    typedef uint2 Raw;
    static constexpr bool SCALED = true;
    static constexpr uint32_t EB = 1;
    __device__ static Raw load(const char *b, uint32_t off)
    {
        return *(const uint2 *)(b + off);
    }
    __device__ static u4 to_f16(const Raw &r, float z)
    {
        h8 h;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = (_Float16)((float)(int8_t)(r.x >> (8 * e)) * z);
            h[4 + e] = (_Float16)((float)(int8_t)(r.y >> (8 * e)) * z);
        }
        return __builtin_bit_cast(u4, h);
    }
};
template <> struct PElem<kI16> {
    typedef u4 Raw;
    static constexpr bool SCALED = true;
    static constexpr uint32_t EB = 2;
    __device__ static Raw load(const char *b, uint32_t off)
    {
        return *(const u4 *)(b + off);
    }
    __device__ static u4 to_f16(const Raw &r, float z)
    {
        h8 h;
#pragma unroll
        for (int e = 0; e < 8; e++)
            h[e] = (_Float16)((float)(int16_t)(r[e / 2] >> (16 * (e % 2))) * z);
        return __builtin_bit_cast(u4, h);
    }
};

template <int D> struct PShape {
    static constexpr int KP = D + 8;   /* halves a K row in LDS (pitch) */
    static constexpr int VP = D + 16;  /* halves a V row in LDS */
    static constexpr int KS = D / 16 / PCfg<D>::CS;  /* a wave's score k-steps */
    static constexpr int CT = PCfg<D>::OC / 32;  /* a wave's output column tiles */
    /* a tile's 16-byte units of K (and of V), and a thread's share */
    static constexpr int UNITS = PCfg<D>::TILE * D * 2 / 16;
    static constexpr int UPT = UNITS / (PCfg<D>::W * 64);
    static constexpr int UPR = D * 2 / 16;  /* units a row */
};

/*
 * What a workgroup and a lane work on (shared by both kernels below).
 * Lane l of wave w owns query row r0 + 32 w + l % 32 (half its scores sit
 * in lane l ^ 32). Scores S^T = K . Q^T: element i of sacc[b] is position
 * p0 + 32 b + 8 (i / 4) + 4 (l / 32) + i % 4. Outputs O^T = V^T . P^T:
 * element i of o[c] is column 32 c + 8 (i / 4) + 4 (l / 32) + i % 4 of the
 * lane's row - so the softmax state and the output of a row share a lane.
 */
struct PBlock {
    const SeqDesc *sq;
    uint32_t lo_all, hi_all;   /* positions any row of the block sees */
    uint32_t tfirst, tlast;    /* key tiles visited (the segment's) */
    uint32_t seg, nseg;        /* the key segment, of nseg (1: not split) */
    size_t head_row;           /* the KV head's first cache row */
    uint32_t kvh;              /* the KV head */
    bool rok;                  /* the lane's row exists */
    uint32_t rj, rh;           /* its token and query head */
    uint32_t rlo, rhi;         /* the positions it sees */
    uint32_t col0;             /* the wave's first output column */
};

/* ONE: a launch of one sequence - its descriptor is read at fixed
   offsets with the rest of the arguments, not after the launch's sequence
   count (a round trip less before the first loads: a 1024-token prompt
   29.8 -> 29.0 us) */
template <int D, bool HV = false, int EX = 0, bool ONE = false>
__device__ __forceinline__ PBlock block_of(const PrefillArgs &A)
{
    constexpr int kPBlock = PCfg<D, HV, EX>::BLOCK, kTile = PCfg<D, HV, EX>::TILE;
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t l32 = lane & 31;
    /* the XCDs in groups of 8 / gcd(n_kv, 8): each group takes whole KV
       heads (their keys stay in its L2s) and deals their row blocks, longest
       first, round robin among its XCDs, so every XCD gets long and short
       blocks alike. With contiguous runs a XCD alone (16 / 2 / 256 at 8k:
       one KV head over 4 XCDs) took either the longest blocks or the
       shortest: 1345 against 895 us. */
    if constexpr (!ONE)
        starts_early(A.n_wg, A.n_kv, A.n_seqs, A.wg0s);
    const uint32_t S = 8u >> min(__builtin_ctz(A.n_kv | 8u), 3);
    /* the launch's grid is n_wg workgroups (read with the other arguments:
       the grid size is an implicit argument past them, in a cache line of
       its own) */
    const uint32_t id = xcd_remap_striped(blockIdx.x, A.n_wg, S);
    const uint32_t si = ONE ? 0 : seq_index(A.wg0s, A.n_seqs, id);
    PBlock P;
    P.sq = &A.seq[si];
    const SeqDesc &sq = *P.sq;
    /* the descriptor fields the block starts from in one round trip */
    asm volatile("" ::"s"(sq.n), "s"(sq.nseg), "s"(sq.wg0), "s"(sq.pos0), "s"(sq.end),
                 "s"(sq.cap), "s"(sq.last), "s"(sq.q), "s"(sq.k), "s"(sq.v));
    const uint32_t G = A.group;
    const uint32_t R = sq.n * G;
    const uint32_t nrb = (R + kPBlock - 1) / kPBlock;
    /* a KV head's workgroups: row blocks, the longest rows first, each
       split into nseg key segments */
    const uint32_t nseg = sq.nseg;
    const uint32_t local = id - sq.wg0;
    const uint32_t kvh = local / (nrb * nseg);
    const uint32_t rem = local % (nrb * nseg);
    const uint32_t rb = nrb - 1 - rem / nseg;
    const uint32_t r0 = rb * kPBlock;

    /* the block's rows see [lo(first token), hi(last token)] */
    const uint32_t rows_here = R - r0 < kPBlock ? R - r0 : kPBlock;
    const uint32_t jf = r0 / G, jl = (r0 + rows_here - 1) / G;
    P.lo_all = row_lo(A, sq.pos0 + jf);
    /* with set_last's bounds any token may see up to the call's end */
    P.hi_all = sq.last ? sq.end - 1 : sq.pos0 + jl;
    P.tfirst = P.lo_all / kTile;
    P.tlast = P.hi_all / kTile;
    /* segment seg: tiles tfirst + [seg nt / nseg, (seg + 1) nt / nseg). An
       empty one (a block with fewer tiles than segments) runs its first
       tile with every row masked, which leaves the neutral partial
       (m = -inf, no weight) - no branch around the tile loop */
    P.seg = rem % nseg;
    P.nseg = nseg;
    bool empty = false;
    if (nseg > 1) {
        const uint64_t nt = P.tlast - P.tfirst + 1;
        const uint32_t a = P.tfirst + (uint32_t)(P.seg * nt / nseg);
        const uint32_t b = P.tfirst + (uint32_t)((P.seg + 1) * nt / nseg);
        empty = a == b;
        P.tfirst = a;
        P.tlast = empty ? a : b - 1;
    }
    P.head_row = (size_t)kvh * sq.cap;
    P.kvh = kvh;

    const uint32_t r = r0 + kPRows * ((w % PCfg<D, HV, EX>::GW) / PCfg<D>::CS) + l32;
    P.col0 = (w % PCfg<D>::CS) * PCfg<D>::OC;
    P.rok = r < R;
    P.rj = (P.rok ? r : r0) / G;
    P.rh = kvh * G + (P.rok ? r : r0) % G;
    P.rlo = P.rok && !empty ? row_lo(A, sq.pos0 + P.rj) : 1;
    /* set_last's bound, clamped to the call's end as the split path
       clamps it (a last[] past last_max sees up to last_max) */
    const uint32_t rl = sq.last ? min(sq.last[P.rj], sq.end - 1) : sq.pos0 + P.rj;
    P.rhi = P.rok && !empty ? rl : 0;
    return P;
}

/* the lane's query row in f16, scaled by the score scale times log2(e):
   the B operands of the score product (the wave's columns P.col0 .. when
   the row is split) */
template <int D>
__device__ __forceinline__ void load_query(const PrefillArgs &A, const PBlock &P,
                                           h8 *qb)
{
    const uint32_t g = (threadIdx.x & 63) >> 5, hd = A.hd;
    const float *qrow = P.sq->q + ((size_t)P.rj * A.n_head + P.rh) * hd;
    const float f = A.scale * kLog2e;
#pragma unroll
    for (int s = 0; s < D / 16 / PCfg<D>::CS; s++) {
        const uint32_t c = P.col0 + 16 * s + 8 * g;
        const bool cok = P.rok && c < hd;
        const float4 x0 = *(const float4 *)(qrow + (cok ? c : 0));
        const float4 x1 = *(const float4 *)(qrow + (cok ? c + 4 : 0));
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; e++)
            qb[s][e] = (_Float16)(cok ? xs[e] * f : 0.0f);
    }
}

/*
 * One key tile (PCfg::TILE positions) from p0 for the lane's row: the scores,
 * the masks, the lazy-maximum softmax and the value product. kop(s, b) is
 * the A operand of score k-step s for positions 32 b .. 32 b + 31 (K rows
 * 32 b + l % 32, columns 16 s + 8 (l / 32) .. + 7); vop(ks, c) the A operand
 * of value k-step ks for columns 32 c .. 32 c + 31 (positions 16 ks +
 * 4 (l / 32) + 0..3 and + 8 of column 32 c + l % 32).
 */
struct NoExchange {
    template <class T> __device__ void operator()(T *) const {}
};
struct NoLoads {
    __device__ void operator()(int) const {}
};

/* lop(s): called at the start of score k-step s (the DMA kernel issues one
   load instruction of the next tile there) */
template <int D, bool PIPE, bool HV = false, class KOp, class VOp, class XOp = NoExchange,
          class LOp = NoLoads>
__device__ __forceinline__ void tile_pass(uint32_t p0, const PBlock &P, const h8 *qb,
                                          float &m, float &lsum, f16x *o,
                                          KOp kop, VOp vop, XOp xop = XOp(), LOp lop = LOp())
{
    constexpr int kNPB = PCfg<D, HV>::NPB, kTile = PCfg<D, HV>::TILE;
    constexpr int KS = D / 16 / PCfg<D>::CS, CT = PCfg<D>::OC / 32;
    const uint32_t g = (threadIdx.x & 63) >> 5;
    /* scores less the row's maximum so far (the accumulators start at
       -m; a split row's second half starts at 0): kNPB blocks of 32
       positions */
    const float mref = m == -INFINITY ? 0.0f : m;
    f16x sacc[kNPB];
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            sacc[b][i] = P.col0 == 0 ? -mref : 0.0f;
    /* PIPE: the operands of k-step s + 1 are asked for before the products
       of step s, so the LDS latency hides behind them (32 more registers) */
    if constexpr (!PIPE) {
#pragma unroll
        for (int s = 0; s < KS; s++) {
            lop(s);
#pragma unroll
            for (int b = 0; b < kNPB; b++)
                sacc[b] = mfma(kop(s, b), qb[s], sacc[b]);
        }
    } else {
    h8 ka[2][kNPB];
#pragma unroll
    for (int b = 0; b < kNPB; b++)
        ka[0][b] = kop(0, b);
#pragma unroll
    for (int s = 0; s < KS; s++) {
        lop(s);
        if (s + 1 < KS)
#pragma unroll
            for (int b = 0; b < kNPB; b++)
                ka[(s + 1) & 1][b] = kop(s + 1, b);
#pragma unroll
        for (int b = 0; b < kNPB; b++)
            sacc[b] = mfma(ka[s & 1][b], qb[s], sacc[b]);
    }
    /* keep that order: the scheduler would otherwise sink every read to
       just before its product (and the loads of lop to the end) */
    constexpr bool kLoads = !__is_same(LOp, NoLoads);
    __builtin_amdgcn_sched_group_barrier(0x100, kNPB, 0);
#pragma unroll
    for (int s = 0; s < KS; s++) {
        if (kLoads)
            __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
        if (s + 1 < KS)
            __builtin_amdgcn_sched_group_barrier(0x100, kNPB, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, kNPB, 0);
    }
    }

    /* a split row: the two partial scores summed (the same sum in both
       waves) */
    xop(sacc);

    /* masks, only where a row of the wave sees part of the tile */
    const bool partial = !(P.rlo <= p0 && P.rhi >= p0 + kTile - 1);
    if (__any(partial)) {
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t p = p0 + 32 * b + 8 * (i / 4) + 4 * g + i % 4;
                if (p < P.rlo || p > P.rhi)
                    sacc[b][i] = -INFINITY;
            }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            mx = fmaxf(mx, sacc[b][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    /* move m when the row has none yet, or a score passed it by more than
       the slack */
    const bool move = m == -INFINITY ? mx != -INFINITY : mx > kSlack;
    if (__any(move)) {
        const float sh = move ? mx : 0.0f;
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(-sh);
        m = move ? mref + mx : m;
        lsum *= alpha;
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                sacc[b][i] -= sh;
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                o[c][i] *= alpha;
    }

    /* weights in f16, the PV operands: k-step ks holds positions
       32 (ks / 2) + 16 (ks % 2) + 8 (e / 4) + 4 (l / 32) + e % 4 */
    h8 pa[2 * kNPB];
    float ls = 0.0f;
    auto weights = [&](int ks) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            pa[ks][e] = (_Float16)__builtin_amdgcn_exp2f(sacc[ks / 2][8 * (ks % 2) + e]);
        /* the sum from the operand's own registers (pairs rebuilt from its
           elements are converted a second time) */
        const uint4 pw = __builtin_bit_cast(uint4, pa[ks]);
        const uint32_t pws[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
            ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, pws[e]),
                                        h2{(_Float16)1.0f, (_Float16)1.0f},
                                        ls, false);
    };

    /* O^T += V^T . P^T (PIPE: operands one k-step ahead, except at head
       size 512, whose 8 column tiles of read-ahead would not fit) */
    if constexpr (!PIPE || D > 256) {
#pragma unroll
        for (int ks = 0; ks < 2 * kNPB; ks++)
            weights(ks);
        lsum += ls;
#pragma unroll
        for (int ks = 0; ks < 2 * kNPB; ks++)
#pragma unroll
            for (int c = 0; c < CT; c++)
                o[c] = mfma(vop(ks, c), pa[ks], o[c]);
        return;
    }
    /* PIPE: k-step ks + 1's operands and weights are made while k-step
       ks's products run */
    h8 va[2][CT];
#pragma unroll
    for (int c = 0; c < CT; c++)
        va[0][c] = vop(0, c);
    weights(0);
#pragma unroll
    for (int ks = 0; ks < 2 * kNPB; ks++) {
        if (ks + 1 < 2 * kNPB) {
#pragma unroll
            for (int c = 0; c < CT; c++)
                va[(ks + 1) & 1][c] = vop(ks + 1, c);
            weights(ks + 1);
        }
#pragma unroll
        for (int c = 0; c < CT; c++)
            o[c] = mfma(va[ks & 1][c], pa[ks], o[c]);
    }
    lsum += ls;
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * CT, 1);
#pragma unroll
    for (int ks = 0; ks < 2 * kNPB; ks++) {
        if (ks + 1 < 2 * kNPB) {
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * CT, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, CT, 1);
    }
}

/* write_out for a sequence that asks for Q8_K when the kernel writes its
   blocks (A.q8k_fused: head size D exactly, 64, 128 or 256, a block's rows
   in one wave): the output and its blocks from the same numbers */
template <int D>
__device__ __forceinline__ void write_out_q8k(const PrefillArgs &A, const PBlock &P, float lt,
                                           f16x *x)
{
    constexpr int CT = D / 32;
    const uint32_t g = (threadIdx.x & 63) >> 5, hd = A.hd;
    const SeqDesc &sq = *P.sq;
    const float inv = 1.0f / lt;
    const size_t obase = ((size_t)P.rj * A.n_head + P.rh) * hd;
    /* the sums become the outputs in place */
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t col = 32 * c + 8 * (i / 4) + 4 * g + i % 4;
            float v = x[c][i] * inv;
            if (A.gate_mode == kGateElem)
                v *= 1.0f / (1.0f + expf(-sq.gate[P.rok ? obase + col : 0]));
            else if (A.gate_mode == kGateHead)
                v *= 1.0f / (1.0f + expf(-sq.gate[P.rok ? (size_t)P.rj * A.n_head + P.rh : 0]));
            x[c][i] = P.rok ? v : 0.0f;
        }
    if (P.rok)
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++)
                *(float4 *)(sq.out + obase + 32 * c + 8 * q4 + 4 * g) =
                    float4{x[c][4 * q4], x[c][4 * q4 + 1], x[c][4 * q4 + 2], x[c][4 * q4 + 3]};
    uint8_t *dst = (uint8_t *)sq.q8k +
                   ((size_t)P.rj * (A.n_head * D / 256) + P.rh / (256 / D)) * kQ8kBytes;
    q8k_rows<CT>(x, dst, P.rok);
}

/* out = sums / weights, gated (and its Q8_K blocks: write_out_q8k, which
   turns o into the outputs in place; QF false: not compiled in, the
   host leaves those blocks to a pass) */
template <int D, bool QF = true>
__device__ __forceinline__ void write_out(const PrefillArgs &A, const PBlock &P,
                                          float lsum, f16x *o)
{
    const uint32_t g = (threadIdx.x & 63) >> 5, hd = A.hd;
    const SeqDesc &sq = *P.sq;
    const float lt = lsum + __shfl_xor(lsum, 32, 64);
    if constexpr (QF && (D == 64 || D == 128 || D == 256)) {
        if (A.q8k_fused && sq.q8k) {
            write_out_q8k<D>(A, P, lt, o);
            return;
        }
    }
    if (!P.rok)
        return;
    const float inv = 1.0f / lt;
    const size_t obase = ((size_t)P.rj * A.n_head + P.rh) * hd;
#pragma unroll
    for (int c = 0; c < PCfg<D>::OC / 32; c++)
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint32_t col = P.col0 + 32 * c + 8 * q4 + 4 * g;
            if (col >= hd)
                continue;
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[e] = o[c][4 * q4 + e] * inv;
                if (A.gate_mode == kGateElem)
                    x[e] *= 1.0f / (1.0f + expf(-sq.gate[obase + col + e]));
                else if (A.gate_mode == kGateHead)
                    x[e] *= 1.0f / (1.0f + expf(-sq.gate[(size_t)P.rj * A.n_head + P.rh]));
            }
            *(float4 *)(sq.out + obase + col) = float4{x[0], x[1], x[2], x[3]};
        }
}

/* the lane's row when its row block is split into key segments: the
   segment's partial - largest score m (log2 units, -inf when the row saw
   nothing of it), sum of weights, unnormalised weighted values - for the
   ordered merge (pmerge_kernel); otherwise the output itself */
template <int D, bool QF = true>
__device__ __forceinline__ void finish(const PrefillArgs &A, const PBlock &P,
                                       float m, float lsum, f16x *o)
{
    if (P.nseg == 1) {
        write_out<D, QF>(A, P, lsum, o);
        return;
    }
    const uint32_t g = (threadIdx.x & 63) >> 5, hd = A.hd;
    const float lt = lsum + __shfl_xor(lsum, 32, 64);
    if (!P.rok)
        return;
    const size_t pr = P.sq->part0 + ((size_t)P.rj * A.n_head + P.rh) * P.nseg + P.seg;
    if (g == 0 && P.col0 == 0)
        *(float2 *)(A.part_ml + 2 * pr) = float2{m, lt};
    float *dst = A.part_acc + pr * hd;
#pragma unroll
    for (int c = 0; c < PCfg<D>::OC / 32; c++)
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint32_t col = P.col0 + 32 * c + 8 * q4 + 4 * g;
            if (col < hd)
                *(float4 *)(dst + col) = float4{o[c][4 * q4], o[c][4 * q4 + 1],
                                                o[c][4 * q4 + 2], o[c][4 * q4 + 3]};
        }
}

/*
 * The kernel for int8 / int16 caches (dequantized with their scales as
 * tiles are staged) and head sizes up to 64: each thread loads its units
 * of the next tile into registers while this tile is computed, then stores
 * them into padded LDS rows (K pitch D + 8, V pitch D + 16 halves).
 */
template <int T, int D, bool ONE>
__global__ __launch_bounds__(PCfg<D>::W * 64) void prefill_kernel(const PrefillArgs A)
{
    using S = PShape<D>;
    using E = PElem<T>;
    constexpr int kPWaves = PCfg<D>::W, kTile = PCfg<D>::TILE;
    static_assert(S::UPT >= 1 && S::UNITS % (kPWaves * 64) == 0, "tile loads");
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][kTile][S::KP];
    __shared__ __attribute__((aligned(16))) _Float16 sV[2][kTile][S::VP];
    /* the partial scores of split rows, a wave's 64 lanes x 16 x kNPB */
    constexpr int kCS = PCfg<D>::CS;
    __shared__ __attribute__((aligned(16))) float sX[kCS > 1 ? kPWaves : 1][64][16 * PCfg<D>::NPB];

    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t g = lane >> 5, l32 = lane & 31, l16 = lane & 15;
    const PBlock P = block_of<D, false, 0, ONE>(A);
    const SeqDesc &sq = *P.sq;
    const uint32_t hd = A.hd;
    const bool ring = A.ring != 0;
    h8 qb[S::KS];
    load_query<D>(A, P, qb);

    /* ---- a tile's K and V: thread t's units t + 512 u; columns past hd
       read column 0 (their products meet zero query columns, or are not
       stored). One base row a tile and 32-bit offsets, as in the DMA
       kernel: rows outside [lo_all, hi_all] read the nearest row inside,
       which lies in the same tile ---- */
    const uint32_t rbytes = hd * E::EB;
    auto load = [&](uint32_t tile, typename E::Raw *kr, typename E::Raw *vr,
                    float *kz, float *vz) {
        const uint32_t t0 = tile * kTile;
        const size_t brow = P.head_row + (ring ? t0 % sq.cap : t0);
        const char *const kb = (const char *)sq.k + brow * rbytes;
        const char *const vb = (const char *)sq.v + brow * rbytes;
#pragma unroll
        for (int u = 0; u < S::UPT; u++) {
            const uint32_t unit = tid + u * (kPWaves * 64);
            const uint32_t row = unit / S::UPR, cu = unit % S::UPR;
            uint32_t p = t0 + row;
            p = p < P.lo_all ? P.lo_all : p > P.hi_all ? P.hi_all : p;
            const uint32_t rel = p - t0;
            const uint32_t col = cu * 8 < hd ? cu * 8 : 0;
            const uint32_t off = __umul24(rel, rbytes) + col * E::EB;
            kr[u] = E::load(kb, off);
            vr[u] = E::load(vb, off);
            if constexpr (E::SCALED) {
                kz[u] = sq.ks[brow + rel];
                vz[u] = sq.vs[brow + rel];
            }
        }
    };
    auto store = [&](int b, const typename E::Raw *kr, const typename E::Raw *vr,
                     const float *kz, const float *vz) {
#pragma unroll
        for (int u = 0; u < S::UPT; u++) {
            const uint32_t unit = tid + u * (kPWaves * 64);
            const uint32_t row = unit / S::UPR, cu = unit % S::UPR;
            *(u4 *)&sK[b][row][cu * 8] = E::to_f16(kr[u], E::SCALED ? kz[u] : 1.0f);
            *(u4 *)&sV[b][row][cu * 8] = E::to_f16(vr[u], E::SCALED ? vz[u] : 1.0f);
        }
    };

    /* running state of the lane's row: weights are exp2(s - m) */
    float m = -INFINITY, lsum = 0.0f;
    f16x o[S::CT];
#pragma unroll
    for (int c = 0; c < S::CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[c][i] = 0.0f;

    typename E::Raw kr[S::UPT], vr[S::UPT];
    float kz[S::UPT], vz[S::UPT];
    load(P.tfirst, kr, vr, kz, vz);
    store(0, kr, vr, kz, vz);
    __syncthreads();

    for (uint32_t tile = P.tfirst; tile <= P.tlast; tile++) {
        const int buf = (tile - P.tfirst) & 1;
        if (tile < P.tlast)
            load(tile + 1, kr, vr, kz, vz);
        tile_pass<D, (D > 256)>(
            tile * kTile, P, qb, m, lsum, o,
            [&](int s, int b) {
                return *(const h8 *)&sK[buf][32 * b + l32][P.col0 + 16 * s + 8 * g];
            },
            [&](int ks, int c) {
                const uint32_t tr = 16 * ks + 4 * g + (l16 >> 2);
                const uint32_t tc = P.col0 + 32 * c + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
                const h4 x = lds_read_tr(&sV[buf][tr][tc]);
                const h4 y = lds_read_tr(&sV[buf][tr + 8][tc]);
                return h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
            },
            [&](f16x *sacc) {
                if constexpr (kCS > 1) {
                    const uint32_t w = tid >> 6;
#pragma unroll
                    for (int b = 0; b < PCfg<D>::NPB; b++)
#pragma unroll
                        for (int i = 0; i < 16; i += 4)
                            *(float4 *)&sX[w][lane][16 * b + i] =
                                float4{sacc[b][i], sacc[b][i + 1], sacc[b][i + 2], sacc[b][i + 3]};
                    __syncthreads();
#pragma unroll
                    for (int b = 0; b < PCfg<D>::NPB; b++)
#pragma unroll
                        for (int i = 0; i < 16; i += 4) {
                            const float4 x = *(const float4 *)&sX[w ^ 1][lane][16 * b + i];
                            /* half 0's partial first, in both waves */
                            const bool h0 = P.col0 == 0;
                            sacc[b][i] = h0 ? sacc[b][i] + x.x : x.x + sacc[b][i];
                            sacc[b][i + 1] = h0 ? sacc[b][i + 1] + x.y : x.y + sacc[b][i + 1];
                            sacc[b][i + 2] = h0 ? sacc[b][i + 2] + x.z : x.z + sacc[b][i + 2];
                            sacc[b][i + 3] = h0 ? sacc[b][i + 3] + x.w : x.w + sacc[b][i + 3];
                        }
                    /* the next tile's writes come after its barriers */
                }
            });
        if (tile < P.tlast) {
            __syncthreads(); /* every wave is done with the other buffer */
            store(buf ^ 1, kr, vr, kz, vz);
            __syncthreads();
        }
    }
    finish<D>(A, P, m, lsum, o);
}

/*
 * The f16 kernel for head sizes up to 256: the next tile goes straight
 * from HBM (or L2) into LDS with global_load_lds_dwordx4 while this tile is
 * computed - no staging registers, no LDS stores, one barrier a tile.
 *
 * A tile is 128 rows of 128 or 256 bytes (head size 64 or 128; 8 waves) or
 * 64 rows of 512 (256; 4 waves, one a SIMD), unpadded; the 16-byte unit u
 * of row r is kept in slot u ^ swz(r), which changes the unit's low 4 (3)
 * bits only. A load instruction fills 1 KB (8, 4 or 2 rows) contiguously,
 * so lane i fetches the unit that belongs in its slot. At head sizes 128
 * and 256 a row is a whole number of 256-byte bank rounds, so a slot's
 * banks depend on slot mod 16 alone, and the swizzle keeps both operand
 * reads free of bank conflicts (at 64 two rows share a round: swz<64>):
 *   - a score operand read takes one unit of 16 consecutive rows a
 *     16-lane pass: swz is a bijection on r mod 16;
 *   - a transposed value read takes units 4 c .. 4 c + 3 of 4 consecutive
 *     rows 4 k .. 4 k + 3 a 32-lane pass (256 bytes): swz(r) = the two
 *     2-bit halves of r mod 16 swapped, so those 4 rows differ in the
 *     slot's bits 2-3 and the 16 units fill 16 slots. (rotl4(r mod 16)
 *     left rows r and r + 1 on the same 8 slots: SQ_LDS_BANK_CONFLICT
 *     counted 2 cycles a value read, a third of the LDS-active cycles;
 *     with this swizzle it counts none, at the same kernel time.)
 *
 * Two buffer pairs, as distinct arrays, and the tile loop unrolled by two.
 */
/* a value the same in every lane, said so (the compiler cannot always
   prove it, and a scalar operand needs it); the builtin returns int, so
   each half is widened unsigned */
__device__ __forceinline__ uint64_t uniform_u64(uint64_t b)
{
    return (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32;
}
template <class T> __device__ __forceinline__ T *uniform_ptr(T *p)
{
    return (T *)(uintptr_t)uniform_u64((uint64_t)(uintptr_t)p);
}

/*
 * One 16-byte-a-lane load from global memory straight into LDS
 * (global_load_lds_dwordx4: lane l's 16 bytes at gbase + voff land at LDS
 * address m0 + 16 l), written out rather than through the builtin. The
 * compiler's wait counting takes a load into LDS as outstanding work of the
 * LDS counter too, so with one in flight it makes every LDS operand wait
 * drain all reads (lgkmcnt(0)), and the operand reads issued a k-step
 * ahead no longer overlap the products. The hardware counts these loads in
 * the vector-memory counter only (measured: after one such load and one LDS
 * read, lgkmcnt(0) returns with the read while vmcnt(0) waits for the load),
 * so they are kept out of the compiler's sight, and every wave waits for its
 * own (s_waitcnt vmcnt(0)) before the barrier that publishes the tile. M0 is
 * set here; nothing else in these kernels reads it (the compiler sets it
 * before each use of its own).
 */
__device__ __forceinline__ void dma16(const char *gbase, uint32_t voff, char *lds)
{
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(voff),
                    "s"(uniform_ptr(gbase)));
}

template <int D> __device__ __forceinline__ uint32_t swz(uint32_t r)
{
    r &= 15;
    if constexpr (D == 64) {
        /* rows of 128 bytes: rows r and r + 1 share a bank round, so each
           parity of r must fill the 8 slots (score reads), and rows 4 k
           and 4 k + 2 must differ in the slot's bit 2 (value reads) */
        return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    } else {
        return ((r & 3) << 2) | (r >> 2);
    }
}

template <int D, bool ONE>
__global__ __launch_bounds__(PCfg<D>::W * 64) void prefill_dma_kernel(const PrefillArgs A)
{
    static_assert(D == 64 || D == 128 || D == 256, "rows of 8, 16 or 32 units");
    constexpr uint32_t kW = PCfg<D>::W, kTile = PCfg<D>::TILE;
    constexpr uint32_t RB = D * 2;              /* bytes a row */
    constexpr uint32_t UPR = RB / 16;           /* 16-byte units a row */
    constexpr uint32_t RPI = 64 / UPR;          /* rows a load instruction */
    constexpr uint32_t NJ = kTile / (RPI * kW); /* load instructions a wave */
    constexpr uint32_t TB = kTile * RB;         /* bytes a tile */
    constexpr int CT = D / 32;
    static_assert(NJ * RPI * kW == kTile, "a tile is whole load rounds");
    __shared__ __attribute__((aligned(1024))) char sK0[TB];
    __shared__ __attribute__((aligned(1024))) char sV0[TB];
    __shared__ __attribute__((aligned(1024))) char sK1[TB];
    __shared__ __attribute__((aligned(1024))) char sV1[TB];

    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t g = lane >> 5, l32 = lane & 31, l16 = lane & 15;
    const PBlock P = block_of<D, false, 0, ONE>(A);
    const SeqDesc &sq = *P.sq;
    const uint32_t hd = A.hd;
    const bool ring = A.ring != 0;
    h8 qb[D / 16];
    load_query<D>(A, P, qb);

    /* loads: instruction j of wave w fills the RPI rows from
       RPI (w + W j) (1 KB), lane i row RPI (w + W j) + i / UPR, slot
       i % UPR (the unit slot ^ swz<D>(row)); columns past hd read column 0
       (their products meet zero query columns, or are not stored) */
    const uint32_t drow = RPI * w + lane / UPR;
    uint32_t dcol[NJ];
#pragma unroll
    for (int j = 0; j < (int)NJ; j++) {
        const uint32_t unit = (lane % UPR) ^ swz<D>(drow + RPI * kW * j);
        dcol[j] = unit * 8 < hd ? unit * 8 : 0;
    }
    /* held in registers: read through P.sq inside the loop they would be
       reloaded after every load into LDS, and a pending scalar load makes
       each LDS operand wait drain the whole queue */
    const char *const kg = uniform_ptr((const char *)sq.k);
    const char *const vg = uniform_ptr((const char *)sq.v);
    const uint32_t cap = __builtin_amdgcn_readfirstlane(sq.cap), rbytes = hd * 2;
    const size_t head_row = uniform_u64(P.head_row);
    const uint32_t wu = __builtin_amdgcn_readfirstlane(w);
    /* a tile's rows are contiguous in the cache (a ring's capacity is a
       multiple of 256 positions): one base a tile, in scalar registers, and
       a 32-bit offset a lane. Rows outside the block's positions read the
       nearest one inside [lo_all, hi_all], which lies in the same tile */
    auto tbase = [&](uint32_t tile) -> size_t {
        const uint32_t t0 = tile * kTile;
        return (head_row + (ring ? t0 % cap : t0)) * rbytes;
    };
    /* the lane's byte offsets in tile `tile` for its NJ load rows */
    auto offsets = [&](uint32_t tile, uint32_t *off) {
        const uint32_t t0 = tile * kTile;
#pragma unroll
        for (int j = 0; j < (int)NJ; j++) {
            uint32_t p = t0 + drow + RPI * kW * j;
            p = p < P.lo_all ? P.lo_all : p > P.hi_all ? P.hi_all : p;
            off[j] = __umul24(p - t0, rbytes) + 2 * dcol[j];
        }
    };
    /* load instruction i of the wave's 2 NJ: rows RPI (w + W (i / 2)) ..,
       of K (i even) or V (i odd) */
    auto fetch_one = [&](size_t base, const uint32_t *off, int i, char *dk, char *dv) {
        const int j = i >> 1;
        const uint32_t at = (wu + kW * j) * 1024;
        if (i & 1)
            dma16(vg + base, off[j], dv + at);
        else
            dma16(kg + base, off[j], dk + at);
    };
    auto fetch = [&](uint32_t tile, char *dk, char *dv) {
        const size_t base = tbase(tile);
        uint32_t off[NJ];
        offsets(tile, off);
#pragma unroll
        for (int i = 0; i < 2 * (int)NJ; i++)
            fetch_one(base, off, i, dk, dv);
    };
    static_assert(2 * NJ == D / 16, "a load instruction a score k-step");
    /* operand addresses: the lane's score rows are 32 b + l % 32 (row mod
       16 = l % 16), its value rows 16 ks + 4 (l / 32) + (l % 16) / 4 and 8
       further */
    uint32_t koff[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; s++)
        koff[s] = l32 * RB + (((2 * s + g) ^ swz<D>(l16)) * 16);
    const uint32_t vrow = 4 * g + (l16 >> 2);
    const uint32_t u0 = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1);
    uint32_t vxo[CT], vyo[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) {
        vxo[c] = vrow * RB + (((4 * c + u0) ^ swz<D>(vrow)) * 16) + (l16 & 1) * 8;
        vyo[c] = (vrow + 8) * RB + (((4 * c + u0) ^ swz<D>(vrow + 8)) * 16) + (l16 & 1) * 8;
    }

    float m = -INFINITY, lsum = 0.0f;
    f16x o[CT];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[c][i] = 0.0f;

    /* tile t from (ck, cv) while t + 1 is loaded into (nk, nv), one load
       instruction a score k-step: all of a tile's loads at once would hold
       each wave at the issue until the CU's load path had taken the lot
       (64 KB at 64 bytes a clock). The block's last tile loads itself again
       into the other buffer (not read again): a branch per load would cut
       the score loop's schedule into pieces */
    auto step = [&](uint32_t tile, const char *ck, const char *cv, char *nk, char *nv) {
        const uint32_t nt = tile < P.tlast ? tile + 1 : tile;
        const size_t nbase = tbase(nt);
        uint32_t noff[NJ];
        offsets(nt, noff);
        tile_pass<D, true>(
            tile * kTile, P, qb, m, lsum, o,
            [&](int s, int b) { return *(const h8 *)(ck + 32 * b * RB + koff[s]); },
            [&](int ks, int c) {
                const char *base = cv + 16 * ks * RB;
                const h4 x = lds_read_tr((const _Float16 *)(base + vxo[c]));
                const h4 y = lds_read_tr((const _Float16 *)(base + vyo[c]));
                return h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
            },
            NoExchange(), [&](int s) { fetch_one(nbase, noff, s, nk, nv); });
        /* the wave's loads of the next tile are in (the last tile's, of
           itself again: no load into LDS outlives the wave) */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (tile < P.tlast)
            __syncthreads(); /* the whole next tile is in; this one is read */
    };

    fetch(P.tfirst, sK0, sV0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (uint32_t tile = P.tfirst;; tile += 2) {
        step(tile, sK0, sV0, sK1, sV1);
        if (tile + 1 > P.tlast)
            break;
        step(tile + 1, sK1, sV1, sK0, sV0);
        if (tile + 2 > P.tlast)
            break;
    }
    finish<D>(A, P, m, lsum, o);
}

/*
 * ---- The exact kernel: int8 / int16 caches at float accuracy ----------
 *
 * The reference's FLOAT way (attention.c:107-118, :574-627, :761-763,
 * :135-145) holds int8 keys and values exact and computes in f32, and so
 * does this pass: the cache's integers enter the products as they are, in
 * f16 planes whose sum is the cached number exactly (int8: one plane; int16:
 * x with its low byte cleared, and the low byte), and the query and the
 * weights as two f16 planes each (x = hi + lo, 22 significant bits), so each
 * product is exact in the matrix core and summed in f32. The scales stay f32:
 *   score   s = (sum_i q'_i k_i) * ks[p] * 2^-e,  q' = q * scale * log2(e) * 2^e
 *           (e puts the row's largest |q'| in [2^13, 2^14): neither plane
 *           loses bits to f16's range)
 *   value   o = sum_p (w_p * vs[p]) v_p / sum_p w_p,  the weight and the value
 *           scale multiplied in f32 before the split into planes
 * The weights carry a fixed power of two, 2^6 over an int8 cache and 2^14
 * over int16 (XBias), so that w * vs = w 2^6 max|v| / 127 (or 2^14 max|v| /
 * 32767) keeps its low plane inside f16's normal range for every weight
 * that matters (the high plane from 2^-3 up: weights from about 2^-9 of
 * the row's largest at a value row's largest magnitude of 1); the power
 * cancels between the sums. A value row's largest magnitude must stay
 * below 500 (w * vs below f16's 65504 at the lazy maximum's 2^8).
 *
 * The keys and values come from a copy of the call's visible rows in those
 * planes (xcopy_kernel: the integers widened, linear in the positions, laid
 * out per KV head from the call's first chunk), tiles straight into LDS as in
 * prefill_dma_kernel, with the same swizzle; the scales of a tile come from
 * the cache itself (a 4-byte load into LDS a lane, every position clamped to
 * the rows the block sees, so nothing outside them is read).
 */
/* x = hi + lo in f16 (22 significant bits). x is pinned in a register
   first (an empty asm): left free, the compiler made hi from the f32
   product x = w * vs for the products, but made it again for lo straight
   from the exact product (v_fma_mixlo_f16 w, vs, 0: one rounding instead of
   two) - at a rounding tie the two differ by an f16 unit, and hi + lo
   missed the weight by twice lo (an error of 2^-10 on one weight in a
   hundred rows). */
__device__ __forceinline__ void split_hl(float x, _Float16 &hi, _Float16 &lo)
{
    asm volatile("" : "+v"(x));
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

template <int EX> struct XBias {
    static constexpr float value = EX == 2 ? 14.0f : 6.0f;
};

/* the loads into LDS of score k-step s when NL are spread over KS steps
   (load i at step i mod KS), plus the tile's scales at step 0 */
template <int NL, int KS> constexpr int xloads_at(int s)
{
    return (s < NL ? (NL - 1 - s) / KS + 1 : 0) + (s == 0 ? 1 : 0);
}

/* a scheduling group of n loads (n a constant once the caller's loop is
   unrolled) */
__device__ __forceinline__ void sgb_vmem(int n)
{
    switch (n) {
    case 1: __builtin_amdgcn_sched_group_barrier(0x010, 1, 0); break;
    case 2: __builtin_amdgcn_sched_group_barrier(0x010, 2, 0); break;
    case 3: __builtin_amdgcn_sched_group_barrier(0x010, 3, 0); break;
    case 4: __builtin_amdgcn_sched_group_barrier(0x010, 4, 0); break;
    default: break;
    }
}

/* One 4-byte-a-lane load from a 64-bit address straight into LDS
   (global_load_lds_dword: lane l's 4 bytes land at LDS address m0 + 4 l),
   written out for the reasons given at dma16. */
__device__ __forceinline__ void dma4(const void *g, char *lds)
{
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
                 :: "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(g));
}

/* the lane's query row times the score scale, log2(e) and 2^e (its largest
   magnitude in [2^13, 2^14)) as two f16 planes; returns 2^-e */
template <int D>
__device__ __forceinline__ float load_query_x(const PrefillArgs &A, const PBlock &P, h8 *qh,
                                              h8 *ql)
{
#pragma clang fp contract(off)
    const uint32_t g = (threadIdx.x & 63) >> 5, hd = A.hd;
    const float *qrow = P.sq->q + ((size_t)P.rj * A.n_head + P.rh) * hd;
    const float f = A.scale * kLog2e;
    float mx = 0.0f;
#pragma unroll
    for (int s = 0; s < D / 16; s++) {
        const uint32_t c = 16 * s + 8 * g;
        if (P.rok && c < hd) {
            const float4 x0 = *(const float4 *)(qrow + c);
            const float4 x1 = *(const float4 *)(qrow + c + 4);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x0.x * f), fabsf(x0.y * f)),
                                 fmaxf(fabsf(x0.z * f), fabsf(x0.w * f))));
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x1.x * f), fabsf(x1.y * f)),
                                 fmaxf(fabsf(x1.z * f), fabsf(x1.w * f))));
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    int ex = 0;
    if (mx > 0.0f && mx < INFINITY) {
        frexpf(mx, &ex);
        ex = 14 - ex;
        ex = ex > 100 ? 100 : ex < -100 ? -100 : ex;
    }
    const float up = ldexpf(1.0f, ex);
#pragma unroll
    for (int s = 0; s < D / 16; s++) {
        const uint32_t c = 16 * s + 8 * g;
        const bool cok = P.rok && c < hd;
        const float4 x0 = *(const float4 *)(qrow + (cok ? c : 0));
        const float4 x1 = *(const float4 *)(qrow + (cok ? c + 4 : 0));
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            _Float16 hi, lo;
            split_hl(cok ? (xs[e] * f) * up : 0.0f, hi, lo);
            qh[s][e] = hi;
            ql[s][e] = lo;
        }
    }
    return ldexpf(1.0f, -ex);
}

/*
 * One key tile of the exact kernel for the lane's row: the tile pass of
 * tile_pass with planes. kop(s, b, p): plane p of the score operand (K rows
 * 32 b + l % 32, columns 16 s + 8 (l / 32) ..); vop(ks, c, p): plane p of the
 * value operand; sop(which, b, j): the key (which 0) or value (1) scales of
 * positions 32 b + 8 j + 4 (l / 32) + 0..3 of the tile; lop(s): the loads
 * of score k-step s. Operands are read one k-step ahead of the products.
 */
template <int D, int EX, int NL, class KOp, class VOp, class SOp, class LOp>
__device__ __forceinline__ void tile_pass_x(uint32_t p0, const PBlock &P, const h8 *qh,
                                            const h8 *ql, float qsc, float &m, float &lsum,
                                            f16x *o, KOp kop, VOp vop, SOp sop, LOp lop)
{
#pragma clang fp contract(off)
    using C = PCfg<D, false, EX>;
    constexpr int kNPB = C::NPB, kTile = C::TILE, NP = EX;
    constexpr int KS = D / 16, CT = D / 32;
    constexpr float kB = XBias<EX>::value;
    const uint32_t g = (threadIdx.x & 63) >> 5;
    const float mref = m == -INFINITY ? 0.0f : m;

    f16x sacc[kNPB];
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            sacc[b][i] = 0.0f;
    h8 ka[2][kNPB][NP];
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int p = 0; p < NP; p++)
            ka[0][b][p] = kop(0, b, p);
#pragma unroll
    for (int s = 0; s < KS; s++) {
        lop(s);
        if (s + 1 < KS)
#pragma unroll
            for (int b = 0; b < kNPB; b++)
#pragma unroll
                for (int p = 0; p < NP; p++)
                    ka[(s + 1) & 1][b][p] = kop(s + 1, b, p);
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int p = 0; p < NP; p++) {
                sacc[b] = mfma(ka[s & 1][b][p], qh[s], sacc[b]);
                sacc[b] = mfma(ka[s & 1][b][p], ql[s], sacc[b]);
            }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kNPB * NP, 0);
#pragma unroll
    for (int s = 0; s < KS; s++) {
        sgb_vmem(xloads_at<NL, KS>(s));
        if (s + 1 < KS)
            __builtin_amdgcn_sched_group_barrier(0x100, kNPB * NP, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * kNPB * NP, 0);
    }

    /* the key scales, the query's 2^-e, and the weights' 2^kB less the
       row's maximum so far */
    const float bm = kB - mref;
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 z = sop(0, b, j);
            const float zs[4] = {z.x, z.y, z.z, z.w};
#pragma unroll
            for (int e = 0; e < 4; e++)
                sacc[b][4 * j + e] = fmaf(sacc[b][4 * j + e], zs[e] * qsc, bm);
        }

    const bool partial = !(P.rlo <= p0 && P.rhi >= p0 + kTile - 1);
    if (__any(partial)) {
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const uint32_t p = p0 + 32 * b + 8 * (i / 4) + 4 * g + i % 4;
                if (p < P.rlo || p > P.rhi)
                    sacc[b][i] = -INFINITY;
            }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < kNPB; b++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            mx = fmaxf(mx, sacc[b][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const bool move = m == -INFINITY ? mx != -INFINITY : mx > kSlack + kB;
    if (__any(move)) {
        const float sh = move ? mx - kB : 0.0f;
        const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(-sh);
        m = move ? mref + sh : m;
        lsum *= alpha;
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                sacc[b][i] -= sh;
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                o[c][i] *= alpha;
    }

    /* weights of value k-step ks (positions 32 (ks / 2) + 16 (ks % 2) +
       8 (e / 4) + 4 (l / 32) + e % 4), times their value scales, as two
       planes; the sum of the weights in f32 */
    float ls = 0.0f;
    auto weights = [&](int ks, h8 &ph, h8 &pl) {
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
            const float4 z = sop(1, ks / 2, 2 * (ks % 2) + jj);
            const float zs[4] = {z.x, z.y, z.z, z.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float w = __builtin_amdgcn_exp2f(sacc[ks / 2][8 * (ks % 2) + 4 * jj + e]);
                ls += w;
                _Float16 hi, lo;
                split_hl(w * zs[e], hi, lo);
                ph[4 * jj + e] = hi;
                pl[4 * jj + e] = lo;
            }
        }
    };
    h8 va[2][CT][NP];
    h8 ph[2], pl[2];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int p = 0; p < NP; p++)
            va[0][c][p] = vop(0, c, p);
    weights(0, ph[0], pl[0]);
#pragma unroll
    for (int ks = 0; ks < 2 * kNPB; ks++) {
        if (ks + 1 < 2 * kNPB) {
#pragma unroll
            for (int c = 0; c < CT; c++)
#pragma unroll
                for (int p = 0; p < NP; p++)
                    va[(ks + 1) & 1][c][p] = vop(ks + 1, c, p);
            weights(ks + 1, ph[(ks + 1) & 1], pl[(ks + 1) & 1]);
        }
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int p = 0; p < NP; p++) {
                o[c] = mfma(va[ks & 1][c][p], ph[ks & 1], o[c]);
                o[c] = mfma(va[ks & 1][c][p], pl[ks & 1], o[c]);
            }
    }
    lsum += ls;
}

/* the kernel over the exact copy: loads and layout as prefill_dma_kernel,
   one buffer pair holding EX planes of K and of V, and each tile's scales */
template <int T, int D, bool ONE>
__global__ __launch_bounds__((PCfg<D, false, (T == kI16 ? 2 : 1)>::W) * 64) void prefill_exact_kernel(
    const PrefillArgs A)
{
    static_assert(D == 64 || D == 128 || D == 256, "rows of 8, 16 or 32 units");
    constexpr int EX = T == kI16 ? 2 : 1, NP = EX;
    using C = PCfg<D, false, EX>;
    constexpr uint32_t kW = C::W, kTile = C::TILE;
    constexpr uint32_t RB = D * 2;              /* bytes a row of a plane */
    constexpr uint32_t UPR = RB / 16;           /* 16-byte units a row */
    constexpr uint32_t RPI = 64 / UPR;          /* rows a load instruction */
    constexpr uint32_t NJ = kTile / (RPI * kW); /* load instructions a wave a plane */
    constexpr uint32_t TB = kTile * RB;         /* bytes a plane's tile */
    constexpr int CT = D / 32, KS = D / 16;
    constexpr int NL = 2 * NP * NJ;             /* K and V loads a wave a tile */
    static_assert(NJ >= 1 && NJ * RPI * kW == kTile, "a tile is whole load rounds");
    static_assert(2 * kTile <= 64 * kW, "a tile's scales are one load a wave");
    __shared__ __attribute__((aligned(1024))) char sK0[NP * TB];
    __shared__ __attribute__((aligned(1024))) char sV0[NP * TB];
    __shared__ __attribute__((aligned(1024))) char sK1[NP * TB];
    __shared__ __attribute__((aligned(1024))) char sV1[NP * TB];
    /* a tile's scales: ks of its positions, then vs; wave w's load fills
       floats 64 w .. 64 w + 63 (past 2 TILE they repeat) */
    __shared__ __attribute__((aligned(16))) float sS0[64 * kW];
    __shared__ __attribute__((aligned(16))) float sS1[64 * kW];

    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t g = lane >> 5, l32 = lane & 31, l16 = lane & 15;
    const PBlock P = block_of<D, false, EX, ONE>(A);
    const SeqDesc &sq = *P.sq;
    const uint32_t hd = A.hd;
    const bool ring = A.ring != 0;
    h8 qh[KS], ql[KS];
    const float qsc = load_query_x<D>(A, P, qh, ql);

    /* the copy: per KV head the positions pb .. end - 1, plane after plane */
    const uint32_t pb = sq.c0 * kChunk, np = sq.end - pb;
    const uint32_t rbytes = hd * 2;
    const size_t pstride = (size_t)A.n_kv * np * rbytes;
    const char *const kg = uniform_ptr((const char *)sq.k);
    const char *const vg = uniform_ptr((const char *)sq.v);
    const uint32_t wu = __builtin_amdgcn_readfirstlane(w);
    const uint32_t drow = RPI * w + lane / UPR;
    uint32_t dcol[NJ];
#pragma unroll
    for (int j = 0; j < (int)NJ; j++) {
        const uint32_t unit = (lane % UPR) ^ swz<D>(drow + RPI * kW * j);
        dcol[j] = unit * 8 < hd ? unit * 8 : 0;
    }
    auto tbase = [&](uint32_t tile) -> size_t {
        return ((size_t)P.kvh * np + (tile * kTile - pb)) * rbytes;
    };
    auto offsets = [&](uint32_t tile, uint32_t *off) {
        const uint32_t t0 = tile * kTile;
#pragma unroll
        for (int j = 0; j < (int)NJ; j++) {
            uint32_t p = t0 + drow + RPI * kW * j;
            p = p < P.lo_all ? P.lo_all : p > P.hi_all ? P.hi_all : p;
            off[j] = __umul24(p - t0, rbytes) + 2 * dcol[j];
        }
    };
    /* load i of a tile: K (i even) or V, plane (i / 2) / NJ, round (i / 2) % NJ */
    auto fetch_one = [&](size_t base, const uint32_t *off, int i, char *dk, char *dv) {
        const int r = i >> 1, p = r / (int)NJ, j = r % (int)NJ;
        const uint32_t at = p * TB + (wu + kW * j) * 1024;
        if (i & 1)
            dma16(vg + base + p * pstride, off[j], dv + at);
        else
            dma16(kg + base + p * pstride, off[j], dk + at);
    };
    /* the lane's scale of tile `tile`: ks, then vs, of the position clamped
       to the block's rows (the cache's own rows, ring-aware) */
    const uint32_t si = (64 * w + lane) % (2 * kTile);
    const float *const zarr = si < kTile ? sq.ks : sq.vs;
    auto saddr = [&](uint32_t tile) -> const float * {
        const uint32_t t0 = tile * kTile;
        uint32_t p = t0 + si % kTile;
        p = p < P.lo_all ? P.lo_all : p > P.hi_all ? P.hi_all : p;
        return zarr + P.head_row + (ring ? t0 % sq.cap : t0) + (p - t0);
    };
    auto fetch = [&](uint32_t tile, char *dk, char *dv, float *ds) {
        const size_t base = tbase(tile);
        uint32_t off[NJ];
        offsets(tile, off);
#pragma unroll
        for (int i = 0; i < NL; i++)
            fetch_one(base, off, i, dk, dv);
        dma4(saddr(tile), (char *)ds + 256 * wu);
    };
    uint32_t koff[KS];
#pragma unroll
    for (int s = 0; s < KS; s++)
        koff[s] = l32 * RB + (((2 * s + g) ^ swz<D>(l16)) * 16);
    const uint32_t vrow = 4 * g + (l16 >> 2);
    const uint32_t u0 = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1);
    uint32_t vxo[CT], vyo[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) {
        vxo[c] = vrow * RB + (((4 * c + u0) ^ swz<D>(vrow)) * 16) + (l16 & 1) * 8;
        vyo[c] = (vrow + 8) * RB + (((4 * c + u0) ^ swz<D>(vrow + 8)) * 16) + (l16 & 1) * 8;
    }

    float m = -INFINITY, lsum = 0.0f;
    f16x o[CT];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[c][i] = 0.0f;

    auto step = [&](uint32_t tile, const char *ck, const char *cv, const float *cs, char *nk,
                    char *nv, float *ns) {
        const uint32_t nt = tile < P.tlast ? tile + 1 : tile;
        const size_t nbase = tbase(nt);
        uint32_t noff[NJ];
        offsets(nt, noff);
        const float *const nz = saddr(nt);
        tile_pass_x<D, EX, NL>(
            tile * kTile, P, qh, ql, qsc, m, lsum, o,
            [&](int s, int b, int p) {
                return *(const h8 *)(ck + p * TB + 32 * b * RB + koff[s]);
            },
            [&](int ks, int c, int p) {
                const char *base = cv + p * TB + 16 * ks * RB;
                const h4 x = lds_read_tr((const _Float16 *)(base + vxo[c]));
                const h4 y = lds_read_tr((const _Float16 *)(base + vyo[c]));
                return h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
            },
            [&](int which, int b, int j) {
                return *(const float4 *)(cs + which * kTile + 32 * b + 8 * j + 4 * g);
            },
            [&](int s) {
#pragma unroll
                for (int i = s; i < NL; i += KS)
                    fetch_one(nbase, noff, i, nk, nv);
                if (s == 0)
                    dma4(nz, (char *)ns + 256 * wu);
            });
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (tile < P.tlast)
            __syncthreads();
    };

    fetch(P.tfirst, sK0, sV0, sS0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (uint32_t tile = P.tfirst;; tile += 2) {
        step(tile, sK0, sV0, sS0, sK1, sV1, sS1);
        if (tile + 1 > P.tlast)
            break;
        step(tile + 1, sK1, sV1, sS1, sK0, sV0, sS0);
        if (tile + 2 > P.tlast)
            break;
    }
    /* head size 256: the Q8_K epilogue's registers would spill into the
       tile loop of this one-wave-a-SIMD kernel; a pass does it */
    finish<D, (D < 256)>(A, P, m, lsum, o);
}

/*
 * The exact copy of an int8 / int16 cache's rows of positions p0 .. p0 +
 * np - 1: the integers as f16 planes whose sum is the number exactly - int8
 * one plane, int16 two (x with its low byte cleared, and the low byte) -
 * row kvh np + (p - p0) of each plane (the cache's row kvh cap + p, or p
 * mod cap on a ring). A thread takes 8 numbers of one row.
 */
template <int T>
__global__ __launch_bounds__(256) void xcopy_kernel(const XcopyArgs A)
{
    const uint32_t upr = A.hd / 8;
    const uint64_t u = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (u >= (uint64_t)A.n_kv * A.np * upr)
        return;
    const uint64_t row = u / upr;
    const uint32_t cu = (uint32_t)(u - row * upr);
    const uint32_t kvh = (uint32_t)(row / A.np), p = A.p0 + (uint32_t)(row % A.np);
    const size_t r = (size_t)kvh * A.cap + (A.ring ? p % A.cap : p);
    const size_t dst = row * A.hd + cu * 8;
    const size_t plane = (size_t)A.n_kv * A.np * A.hd;
    if constexpr (T == kI8) {
        const uint2 kx = *(const uint2 *)((const char *)A.k + r * A.hd + cu * 8);
        const uint2 vx = *(const uint2 *)((const char *)A.v + r * A.hd + cu * 8);
        *(h8 *)(A.k16 + dst) = i8_widen8(kx.x, kx.y);
        *(h8 *)(A.v16 + dst) = i8_widen8(vx.x, vx.y);
    } else {
        /* x & ~255 = 256 (x >> 8), and x & 255 */
        const u4 kx = *(const u4 *)((const char *)A.k + 2 * (r * A.hd + cu * 8));
        const u4 vx = *(const u4 *)((const char *)A.v + 2 * (r * A.hd + cu * 8));
        h8 k0, k1, v0, v1;
        i16_planes8(kx[0], kx[1], kx[2], kx[3], k0, k1);
        i16_planes8(vx[0], vx[1], vx[2], vx[3], v0, v1);
        *(h8 *)(A.k16 + dst) = k0;
        *(h8 *)(A.k16 + plane + dst) = k1;
        *(h8 *)(A.v16 + dst) = v0;
        *(h8 *)(A.v16 + plane + dst) = v1;
    }
}

/* a group index as a type: the two key groups' loops use distinct LDS
   arrays, so the compiler still sees that one buffer's reads never touch
   the loads in flight into the other */
template <int N> struct GroupId {
    static constexpr int value = N;
};

/*
 * The f16 kernel for head sizes 72..128 in calls whose 256-row blocks would
 * leave compute units idle (a prompt of about a thousand tokens, a chunk of
 * a chunked prefill): 128 rows a workgroup, and the 8 waves are two key
 * groups of 4 (waves w and w + 4 take the same 32 rows). Group k walks the
 * k-th half of the block's (or segment's) key tiles of 64 positions - the
 * first ceil(nt / 2), the rest - with the DMA kernel's loads, swizzle and
 * tile pass, each group through its own two buffer pairs; group 1's step
 * past the last tile (nt odd) runs the last tile with every row masked,
 * which adds nothing. Both groups meet at every tile's barrier. At the end
 * group 1 puts each row's state (largest score m, sum of weights, values)
 * into LDS and group 0 combines it with its own - o = 2^(m0 - M) o0 +
 * 2^(m1 - M) o1, the same for the sum, M = max(m0, m1) - and writes the
 * output (or the segment's partial). A block's longest chain of tiles is
 * then half as long as in the DMA kernel, with no partials through memory.
 */
template <int D, bool ONE>
__global__ __launch_bounds__((PCfg<D, true>::W) * 64) void prefill_half_kernel(const PrefillArgs A)
{
    using C = PCfg<D, true>;
    constexpr uint32_t kGW = C::GW, kTile = C::TILE;
    constexpr uint32_t RB = D * 2;              /* bytes a row */
    constexpr uint32_t UPR = RB / 16;           /* 16-byte units a row */
    constexpr uint32_t RPI = 64 / UPR;          /* rows a load instruction */
    constexpr uint32_t NJ = kTile / (RPI * kGW); /* load instructions a wave */
    constexpr uint32_t TB = kTile * RB;         /* bytes a tile */
    constexpr int CT = D / 32;
    static_assert(NJ * RPI * kGW == kTile, "a tile is whole load rounds");
    static_assert(TB >= 64 * 16 * CT * 4, "a buffer holds a wave's values");
    __shared__ __attribute__((aligned(1024))) char sK00[TB];
    __shared__ __attribute__((aligned(1024))) char sV00[TB];
    __shared__ __attribute__((aligned(1024))) char sK01[TB];
    __shared__ __attribute__((aligned(1024))) char sV01[TB];
    __shared__ __attribute__((aligned(1024))) char sK10[TB];
    __shared__ __attribute__((aligned(1024))) char sV10[TB];
    __shared__ __attribute__((aligned(1024))) char sK11[TB];
    __shared__ __attribute__((aligned(1024))) char sV11[TB];
    __shared__ float2 sML[kGW][64];

    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t g = lane >> 5, l32 = lane & 31, l16 = lane & 15;
    const uint32_t grp = __builtin_amdgcn_readfirstlane(w / kGW);
    const uint32_t wu = __builtin_amdgcn_readfirstlane(w % kGW);
    const PBlock P = block_of<D, true, 0, ONE>(A);
    const SeqDesc &sq = *P.sq;
    const uint32_t hd = A.hd;
    const bool ring = A.ring != 0;
    h8 qb[D / 16];
    load_query<D>(A, P, qb);

    /* the group's tiles: half = ceil(nt / 2) steps from tfirst + grp half */
    const uint32_t nt = P.tlast - P.tfirst + 1;
    const uint32_t half = (nt + 1) / 2;
    const uint32_t gt0 = P.tfirst + grp * half;
    /* group 1's step past tlast: the last tile, every row masked */
    PBlock PM = P;
    PM.rlo = 1;
    PM.rhi = 0;

    /* loads as in the DMA kernel, over the group's 4 waves */
    const uint32_t drow = RPI * wu + lane / UPR;
    uint32_t dcol[NJ];
#pragma unroll
    for (int j = 0; j < (int)NJ; j++) {
        const uint32_t unit = (lane % UPR) ^ swz<D>(drow + RPI * kGW * j);
        dcol[j] = unit * 8 < hd ? unit * 8 : 0;
    }
    const char *const kg = uniform_ptr((const char *)sq.k);
    const char *const vg = uniform_ptr((const char *)sq.v);
    const uint32_t cap = __builtin_amdgcn_readfirstlane(sq.cap), rbytes = hd * 2;
    const size_t head_row = uniform_u64(P.head_row);
    auto fetch = [&](uint32_t tile, char *dk, char *dv) __attribute__((always_inline)) {
        const uint32_t t0 = tile * kTile;
        const size_t base = (head_row + (ring ? t0 % cap : t0)) * rbytes;
#pragma unroll
        for (int j = 0; j < (int)NJ; j++) {
            uint32_t p = t0 + drow + RPI * kGW * j;
            p = p < P.lo_all ? P.lo_all : p > P.hi_all ? P.hi_all : p;
            const uint32_t off = __umul24(p - t0, rbytes) + 2 * dcol[j];
            const uint32_t at = (wu + kGW * j) * 1024;
            dma16(kg + base, off, dk + at);
            dma16(vg + base, off, dv + at);
        }
    };
    uint32_t koff[D / 16];
#pragma unroll
    for (int s = 0; s < D / 16; s++)
        koff[s] = l32 * RB + (((2 * s + g) ^ swz<D>(l16)) * 16);
    const uint32_t vrow = 4 * g + (l16 >> 2);
    const uint32_t u0 = 2 * ((lane >> 4) & 1) + ((l16 & 3) >> 1);
    uint32_t vxo[CT], vyo[CT];
#pragma unroll
    for (int c = 0; c < CT; c++) {
        vxo[c] = vrow * RB + (((4 * c + u0) ^ swz<D>(vrow)) * 16) + (l16 & 1) * 8;
        vyo[c] = (vrow + 8) * RB + (((4 * c + u0) ^ swz<D>(vrow + 8)) * 16) + (l16 & 1) * 8;
    }

    float m = -INFINITY, lsum = 0.0f;
    f16x o[CT];
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[c][i] = 0.0f;

    /* step i of the group from (ck, cv) while step i + 1's tile is loaded
       into (nk, nv) */
    auto step = [&](uint32_t i, const char *ck, const char *cv, char *nk, char *nv) __attribute__((always_inline)) {
        const uint32_t t = gt0 + i;
        if (i + 1 < half)
            fetch(t + 1 < P.tlast ? t + 1 : P.tlast, nk, nv);
        __builtin_amdgcn_sched_barrier(0);
        tile_pass<D, true, true>(
            (t < P.tlast ? t : P.tlast) * kTile, t > P.tlast ? PM : P, qb, m, lsum, o,
            [&](int s, int b) { return *(const h8 *)(ck + 32 * b * RB + koff[s]); },
            [&](int ks, int c) {
                const char *base = cv + 16 * ks * RB;
                const h4 x = lds_read_tr((const _Float16 *)(base + vxo[c]));
                const h4 y = lds_read_tr((const _Float16 *)(base + vyo[c]));
                return h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
            });
        /* the wave's loads of the next tile are in (dma16) */
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (i + 1 < half)
            __syncthreads(); /* the next tiles are in; these are read */
    };
    auto run = [&](auto gid) __attribute__((always_inline)) {
        constexpr int G = decltype(gid)::value;
        char *const k0 = G ? sK10 : sK00, *const v0 = G ? sV10 : sV00;
        char *const k1 = G ? sK11 : sK01, *const v1 = G ? sV11 : sV01;
        fetch(gt0 < P.tlast ? gt0 : P.tlast, k0, v0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (uint32_t i = 0;; i += 2) {
            step(i, k0, v0, k1, v1);
            if (i + 1 >= half)
                break;
            step(i + 1, k1, v1, k0, v0);
            if (i + 2 >= half)
                break;
        }
    };
    if (grp == 0)
        run(GroupId<0>());
    else
        run(GroupId<1>());

    /* the halves combined: group 1's state through LDS (the tile buffers,
       every load landed and every read done at the barrier) */
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float *const xo = (float *)(wu == 0 ? sK00 : wu == 1 ? sV00 : wu == 2 ? sK01 : sV01);
    if (grp == 1) {
#pragma unroll
        for (int c = 0; c < CT; c++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                xo[(16 * c + i) * 64 + lane] = o[c][i];
        sML[wu][lane] = float2{m, lsum};
    }
    __syncthreads();
    if (grp == 1)
        return;
    const float2 ml = sML[wu][lane];
    const float M = fmaxf(m, ml.x);
    const float a0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
    const float a1 = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
    lsum = lsum * a0 + ml.y * a1;
#pragma unroll
    for (int c = 0; c < CT; c++)
#pragma unroll
        for (int i = 0; i < 16; i++)
            o[c][i] = o[c][i] * a0 + xo[(16 * c + i) * 64 + lane] * a1;
    finish<D>(A, P, M, lsum, o);
}

/*
 * The ordered merge of split rows: thread t of workgroup b takes 4 columns
 * of one row of its sequence (a row is one (token, head)), the pair
 * kPMergeThreads b + t in row-major order. Up to kPMergeBatch segments'
 * (m, l) and values are asked for at once (more, one after another), then
 * folded in segment order against the largest m: out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s, then the gate as
 * in write_out.
 */
constexpr uint32_t kPMergeBatch = 4;

template <bool ONE>
__global__ __launch_bounds__(kPMergeThreads) void pmerge_kernel(const PrefillArgs A)
{
    if constexpr (!ONE)
        starts_early(A.n_wg, A.n_wg, A.n_seqs, A.mg0s);
    const uint32_t id = blockIdx.x;
    const uint32_t si = ONE ? 0 : seq_index(A.mg0s, A.n_seqs, id);
    const SeqDesc &sq = A.seq[si];
    const uint32_t hd = A.hd, nseg = sq.nseg, c4 = hd / 4;
    const uint64_t pair = (uint64_t)(id - sq.mg0) * kPMergeThreads + threadIdx.x;
    const uint32_t row = (uint32_t)(pair / c4), col = (uint32_t)(pair % c4) * 4;
    /* past the sequence's rows: whole waves, since with Q8_K its outputs
       are whole blocks of 64 pairs */
    if (row >= sq.n * A.n_head)
        return;
    const uint32_t j = row / A.n_head, h = row % A.n_head;
    const size_t pr0 = sq.part0 + (size_t)row * nseg;
    float l = 0.0f;
    float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    /* segment s's weight against the largest m, folded in order */
    auto fold = [&](float mx, float2 ml, float4 v) {
        const float wt = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - mx);
        l += wt * ml.y;
        acc.x += wt * v.x;
        acc.y += wt * v.y;
        acc.z += wt * v.z;
        acc.w += wt * v.w;
    };
    if (nseg <= kPMergeBatch) {
        /* the common case: every segment's loads at once (past nseg the
           last one again, not used) */
        float2 ml[kPMergeBatch];
        float4 v[kPMergeBatch];
#pragma unroll
        for (uint32_t s = 0; s < kPMergeBatch; s++) {
            const size_t pr = pr0 + (s < nseg ? s : nseg - 1);
            ml[s] = *(const float2 *)(A.part_ml + 2 * pr);
            v[s] = *(const float4 *)(A.part_acc + pr * hd + col);
        }
        float mx = -INFINITY;
#pragma unroll
        for (uint32_t s = 0; s < kPMergeBatch; s++)
            if (s < nseg)
                mx = fmaxf(mx, ml[s].x);
#pragma unroll
        for (uint32_t s = 0; s < kPMergeBatch; s++)
            if (s < nseg)
                fold(mx, ml[s], v[s]);
    } else {
        float mx = -INFINITY;
        for (uint32_t s = 0; s < nseg; s++)
            mx = fmaxf(mx, A.part_ml[2 * (pr0 + s)]);
        for (uint32_t s = 0; s < nseg; s++)
            fold(mx, *(const float2 *)(A.part_ml + 2 * (pr0 + s)),
                 *(const float4 *)(A.part_acc + (pr0 + s) * hd + col));
    }
    const float inv = 1.0f / l;
    const size_t oi = ((size_t)j * A.n_head + h) * hd + col;
    float x[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (A.gate_mode == kGateElem)
            x[e] *= 1.0f / (1.0f + expf(-sq.gate[oi + e]));
        else if (A.gate_mode == kGateHead)
            x[e] *= 1.0f / (1.0f + expf(-sq.gate[(size_t)j * A.n_head + h]));
    }
    *(float4 *)(sq.out + oi) = float4{x[0], x[1], x[2], x[3]};
    /* the output's Q8_K blocks: a thread's 4 numbers are 4 of a block, a
       wave's 64 threads one whole block (the pairs run through the output
       in order, 4 numbers a pair, and every wave's first pair is a multiple
       of 64) */
    if (sq.q8k)
        q8k_wave4(x, (uint8_t *)sq.q8k + (pair / 64) * kQ8kBytes, true);
}

template <int T, int D>
hipError_t launch_d(const PrefillArgs &a, hipStream_t s)
{
    /* int8 / int16 up to head size 256: the exact kernel only */
    if constexpr ((T == kI8 || T == kI16) && D <= 256) {
        constexpr int EX = T == kI16 ? 2 : 1;
        if (a.halves || a.exact != EX)
            return hipErrorInvalidValue;
        if (a.n_seqs == 1)
            hipLaunchKernelGGL((prefill_exact_kernel<T, D, true>), dim3(a.n_wg),
                               dim3(PCfg<D, false, EX>::W * 64), 0, s, a);
        else
            hipLaunchKernelGGL((prefill_exact_kernel<T, D, false>), dim3(a.n_wg),
                               dim3(PCfg<D, false, EX>::W * 64), 0, s, a);
        return hipGetLastError();
    }
    if (a.exact)
        return hipErrorInvalidValue;
    if constexpr (T == kF16 && D == 128) {
        if (a.halves) {
            if (a.n_seqs == 1)
                hipLaunchKernelGGL((prefill_half_kernel<D, true>), dim3(a.n_wg), dim3((PCfg<D, true>::W) * 64), 0, s, a);
            else
                hipLaunchKernelGGL((prefill_half_kernel<D, false>), dim3(a.n_wg), dim3((PCfg<D, true>::W) * 64), 0, s, a);
            return hipGetLastError();
        }
    }
    if (a.halves)
        return hipErrorInvalidValue;
    if constexpr (T == kF16 && (D == 64 || D == 128 || D == 256)) {
        if (a.n_seqs == 1)
            hipLaunchKernelGGL((prefill_dma_kernel<D, true>), dim3(a.n_wg), dim3(PCfg<D>::W * 64), 0, s, a);
        else
            hipLaunchKernelGGL((prefill_dma_kernel<D, false>), dim3(a.n_wg), dim3(PCfg<D>::W * 64), 0, s, a);
    } else if constexpr (D > 256) {
        if (a.n_seqs == 1)
            hipLaunchKernelGGL((prefill_kernel<T, D, true>), dim3(a.n_wg), dim3(PCfg<D>::W * 64), 0, s, a);
        else
            hipLaunchKernelGGL((prefill_kernel<T, D, false>), dim3(a.n_wg), dim3(PCfg<D>::W * 64), 0, s, a);
    }
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(const PrefillArgs &a, hipStream_t s)
{
    if (a.hd <= 64)
        return launch_d<T, 64>(a, s);
    if (a.hd <= 128)
        return launch_d<T, 128>(a, s);
    if (a.hd <= 256)
        return launch_d<T, 256>(a, s);
    if (a.hd <= 512)
        return launch_d<T, 512>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

int prefill_supported(int kv, uint32_t hd)
{
    return (kv == kF16 || kv == kI8 || kv == kI16) && hd >= 8 && hd % 8 == 0 &&
           hd <= 512;
}

uint32_t prefill_tile(uint32_t hd, bool halves, int exact)
{
    if (halves)
        return PCfg<128, true>::TILE;
    if (exact == 1)
        return hd > 128 ? PCfg<256, false, 1>::TILE : PCfg<128, false, 1>::TILE;
    if (exact == 2)
        return hd > 128 ? PCfg<256, false, 2>::TILE : PCfg<128, false, 2>::TILE;
    return hd > 256 ? PCfg<512>::TILE : hd > 128 ? PCfg<256>::TILE : PCfg<128>::TILE;
}

hipError_t launch_xcopy(int kv, const XcopyArgs &a, hipStream_t s)
{
    const uint64_t n = (uint64_t)a.n_kv * a.np * (a.hd / 8);
    if (n == 0 || a.hd % 8)
        return hipErrorInvalidValue;
    const dim3 grid((uint32_t)((n + 255) / 256));
    if (kv == kI8)
        hipLaunchKernelGGL(xcopy_kernel<kI8>, grid, dim3(256), 0, s, a);
    else if (kv == kI16)
        hipLaunchKernelGGL(xcopy_kernel<kI16>, grid, dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

int prefill_halves_supported(int kv, uint32_t hd)
{
    /* the DMA kernel's f16 rows at head sizes 72..128 */
    return kv == kF16 && hd > 64 && hd <= 128;
}

hipError_t launch_prefill_merge(const PrefillArgs &a, uint32_t n_wg, hipStream_t s)
{
    if (a.n_seqs == 1)
        hipLaunchKernelGGL(pmerge_kernel<true>, dim3(n_wg), dim3(kPMergeThreads), 0, s, a);
    else
        hipLaunchKernelGGL(pmerge_kernel<false>, dim3(n_wg), dim3(kPMergeThreads), 0, s, a);
    return hipGetLastError();
}

uint32_t prefill_row_blocks(uint32_t n, uint32_t group, uint32_t hd, bool halves, int exact)
{
    /* a workgroup takes PCfg::BLOCK of a KV head's n x group rows */
    const uint64_t block = halves ? PCfg<128, true>::BLOCK
                         : hd > 256 ? PCfg<512>::BLOCK
                         : hd > 128 ? PCfg<256>::BLOCK
                         : exact == 2 && hd > 64 ? PCfg<128, false, 2>::BLOCK
                         : exact == 2 ? PCfg<64, false, 2>::BLOCK : PCfg<128>::BLOCK;
    return (uint32_t)(((uint64_t)n * group + block - 1) / block);
}

hipError_t launch_prefill(int kv, const PrefillArgs &a, hipStream_t s)
{
    switch (kv) {
    case kF16:
        return launch_t<kF16>(a, s);
    case kI8:
        return launch_t<kI8>(a, s);
    case kI16:
        return launch_t<kI16>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace janas
