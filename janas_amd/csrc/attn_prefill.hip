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
 *               whole GQA group. Row blocks of later tokens (more keys to
 *               see) are dispatched first; consecutive workgroups share a KV
 *               head, so they share an XCD's L2.
 *   key tiles   128 positions of K and V in LDS (f16; int8 / int16 caches
 *               dequantized with their scales as they are staged), two
 *               buffers; the next tile is loaded into registers while this
 *               one is computed. 128 rather than 64 positions: the tile's
 *               fixed costs (barriers, the row maximum's exchange, the
 *               stores) spread over twice the products (+3 %).
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

namespace janas {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kPWaves = 8;                 /* waves a workgroup */
constexpr int kPRows = 32;                 /* query rows a wave */
constexpr int kPBlock = kPWaves * kPRows;  /* query rows a workgroup */
constexpr int kTile = 128;                 /* key positions a tile */
constexpr int kNPB = kTile / 32;           /* blocks of 32 positions a tile */
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

__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n)
{
    uint32_t x = bid % 8, k = bid / 8, q = n / 8, r = n % 8;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
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
    __device__ static Raw load(const void *b, size_t i)
    {
        return *(const u4 *)((const uint16_t *)b + i);
    }
    __device__ static u4 to_f16(const Raw &r, float) { return r; }
};
template <> struct PElem<kI8> {
    typedef uint2 Raw;
    static constexpr bool SCALED = true;
    __device__ static Raw load(const void *b, size_t i)
    {
        return *(const uint2 *)((const int8_t *)b + i);
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
    __device__ static Raw load(const void *b, size_t i)
    {
        return *(const u4 *)((const int16_t *)b + i);
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
    static constexpr int KS = D / 16;  /* score k-steps */
    static constexpr int CT = D / 32;  /* output column tiles */
    /* a tile's 16-byte units of K (and of V), and a thread's share */
    static constexpr int UNITS = kTile * D * 2 / 16;
    static constexpr int UPT = UNITS / (kPWaves * 64);
    static constexpr int UPR = D * 2 / 16;  /* units a row */
};

/*
 * Lane l of wave w owns query row r0 + 32 w + l % 32 (half its scores sit
 * in lane l ^ 32). Scores S^T = K . Q^T: element i of sacc[b] is position
 * p0 + 32 b + 8 (i / 4) + 4 (l / 32) + i % 4. Outputs O^T = V^T . P^T:
 * element i of o[c] is column 32 c + 8 (i / 4) + 4 (l / 32) + i % 4 of the
 * lane's row - so the softmax state and the output of a row share a lane.
 */
template <int T, int D>
__global__ __launch_bounds__(512) void prefill_kernel(const PrefillArgs A)
{
    using S = PShape<D>;
    using E = PElem<T>;
    static_assert(S::UPT >= 1 && S::UNITS % (kPWaves * 64) == 0, "tile loads");
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][kTile][S::KP];
    __shared__ __attribute__((aligned(16))) _Float16 sV[2][kTile][S::VP];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t g = lane >> 5, l32 = lane & 31, l16 = lane & 15;
    const uint32_t id = xcd_remap(blockIdx.x, gridDim.x);
    uint32_t si = 0;
    while (si + 1 < A.n_seqs && A.seq[si + 1].wg0 <= id)
        si++;
    const SeqDesc &sq = A.seq[si];
    const uint32_t G = A.group, hd = A.hd;
    const uint32_t R = sq.n * G;
    const uint32_t nrb = (R + kPBlock - 1) / kPBlock;
    const uint32_t local = id - sq.wg0;
    const uint32_t kvh = local / nrb;
    const uint32_t rb = nrb - 1 - local % nrb; /* the longest rows first */
    const uint32_t r0 = rb * kPBlock;

    /* the block's rows see [lo(first token), hi(last token)] */
    const uint32_t rows_here = R - r0 < kPBlock ? R - r0 : kPBlock;
    const uint32_t jf = r0 / G, jl = (r0 + rows_here - 1) / G;
    const uint32_t lo_all = row_lo(A, sq.pos0 + jf);
    /* with set_last's bounds any token may see up to the call's end */
    const uint32_t hi_all = sq.last ? sq.end - 1 : sq.pos0 + jl;
    const uint32_t tfirst = lo_all / kTile, tlast = hi_all / kTile;
    const size_t head_row = (size_t)kvh * sq.cap;
    const bool ring = A.ring != 0;

    /* ---- the lane's row ---- */
    const uint32_t r = r0 + kPRows * w + l32;
    const bool rok = r < R;
    const uint32_t rj = (rok ? r : r0) / G;
    const uint32_t rh = kvh * G + (rok ? r : r0) % G;
    const uint32_t rlo = rok ? row_lo(A, sq.pos0 + rj) : 1;
    const uint32_t rhi = rok ? (sq.last ? sq.last[rj] : sq.pos0 + rj) : 0;
    h8 qb[S::KS];
    {
        const float *qrow = sq.q + ((size_t)rj * A.n_head + rh) * hd;
        const float f = A.scale * kLog2e;
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            const uint32_t c = 16 * s + 8 * g;
            const bool cok = rok && c < hd;
            const float4 x0 = *(const float4 *)(qrow + (cok ? c : 0));
            const float4 x1 = *(const float4 *)(qrow + (cok ? c + 4 : 0));
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                qb[s][e] = (_Float16)(cok ? xs[e] * f : 0.0f);
        }
    }

    /* ---- a tile's K and V: thread t's units t + 512 u. Positions outside
       [lo_all, hi_all] read the nearest of the two (masked, but never a row
       the caller has not written); columns past hd read column 0 (their
       products meet zero query columns, or are not stored) ---- */
    auto load = [&](uint32_t tile, typename E::Raw *kr, typename E::Raw *vr,
                    float *kz, float *vz) {
#pragma unroll
        for (int u = 0; u < S::UPT; u++) {
            const uint32_t unit = tid + u * (kPWaves * 64);
            const uint32_t row = unit / S::UPR, cu = unit % S::UPR;
            uint32_t p = tile * kTile + row;
            p = p < lo_all ? lo_all : p > hi_all ? hi_all : p;
            if (ring)
                p %= sq.cap;
            const size_t cr = head_row + p;
            const uint32_t col = cu * 8 < hd ? cu * 8 : 0;
            kr[u] = E::load(sq.k, cr * hd + col);
            vr[u] = E::load(sq.v, cr * hd + col);
            if constexpr (E::SCALED) {
                kz[u] = sq.ks[cr];
                vz[u] = sq.vs[cr];
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
    load(tfirst, kr, vr, kz, vz);
    store(0, kr, vr, kz, vz);
    __syncthreads();

    for (uint32_t tile = tfirst; tile <= tlast; tile++) {
        const int buf = (tile - tfirst) & 1;
        if (tile < tlast)
            load(tile + 1, kr, vr, kz, vz);
        const uint32_t p0 = tile * kTile;

        /* scores less the row's maximum so far (the accumulators start at
           -m): 2 blocks of 32 positions */
        const float mref = m == -INFINITY ? 0.0f : m;
        f16x sacc[kNPB];
#pragma unroll
        for (int b = 0; b < kNPB; b++)
#pragma unroll
            for (int i = 0; i < 16; i++)
                sacc[b][i] = -mref;
#pragma unroll
        for (int s = 0; s < S::KS; s++)
#pragma unroll
            for (int b = 0; b < kNPB; b++) {
                const h8 ka = *(const h8 *)&sK[buf][32 * b + l32][16 * s + 8 * g];
                sacc[b] = mfma(ka, qb[s], sacc[b]);
            }

        /* masks, only where a row of the wave sees part of the tile */
        const bool partial = !(rlo <= p0 && rhi >= p0 + kTile - 1);
        if (__any(partial)) {
#pragma unroll
            for (int b = 0; b < kNPB; b++)
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const uint32_t p = p0 + 32 * b + 8 * (i / 4) + 4 * g + i % 4;
                    if (p < rlo || p > rhi)
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
        /* move m when the row has none yet, or a score passed it by more
           than the slack */
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
            for (int c = 0; c < S::CT; c++)
#pragma unroll
                for (int i = 0; i < 16; i++)
                    o[c][i] *= alpha;
        }

        /* weights in f16, the PV operands: k-step ks holds positions
           32 (ks / 2) + 16 (ks % 2) + 8 (e / 4) + 4 (l / 32) + e % 4 */
        h8 pa[2 * kNPB];
        float ls = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2 * kNPB; ks++) {
#pragma unroll
            for (int e = 0; e < 8; e++)
                pa[ks][e] = (_Float16)__builtin_amdgcn_exp2f(sacc[ks / 2][8 * (ks % 2) + e]);
#pragma unroll
            for (int e = 0; e < 8; e += 2)
                ls = __builtin_amdgcn_fdot2(h2{pa[ks][e], pa[ks][e + 1]},
                                            h2{(_Float16)1.0f, (_Float16)1.0f},
                                            ls, false);
        }
        lsum += ls;

        /* O^T += V^T . P^T */
#pragma unroll
        for (int ks = 0; ks < 2 * kNPB; ks++) {
            const uint32_t tr = 16 * ks + 4 * g + (l16 >> 2);
#pragma unroll
            for (int c = 0; c < S::CT; c++) {
                const uint32_t tc = 32 * c + 16 * ((lane >> 4) & 1) + 4 * (l16 & 3);
                const h4 x = lds_read_tr(&sV[buf][tr][tc]);
                const h4 y = lds_read_tr(&sV[buf][tr + 8][tc]);
                const h8 va = h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                o[c] = mfma(va, pa[ks], o[c]);
            }
        }
        if (tile < tlast) {
            __syncthreads(); /* every wave is done with the other buffer */
            store(buf ^ 1, kr, vr, kz, vz);
            __syncthreads();
        }
    }

    /* ---- out = sums / weights, gated ---- */
    const float lt = lsum + __shfl_xor(lsum, 32, 64);
    if (!rok)
        return;
    const float inv = 1.0f / lt;
    const size_t obase = ((size_t)rj * A.n_head + rh) * hd;
#pragma unroll
    for (int c = 0; c < S::CT; c++)
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const uint32_t col = 32 * c + 8 * q4 + 4 * g;
            if (col >= hd)
                continue;
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[e] = o[c][4 * q4 + e] * inv;
                if (A.gate_mode == kGateElem)
                    x[e] *= 1.0f / (1.0f + expf(-sq.gate[obase + col + e]));
                else if (A.gate_mode == kGateHead)
                    x[e] *= 1.0f / (1.0f + expf(-sq.gate[(size_t)rj * A.n_head + rh]));
            }
            *(float4 *)(sq.out + obase + col) = float4{x[0], x[1], x[2], x[3]};
        }
}

template <int T, int D>
hipError_t launch_d(const PrefillArgs &a, hipStream_t s)
{
    hipLaunchKernelGGL((prefill_kernel<T, D>), dim3(a.n_wg), dim3(512), 0, s, a);
    return hipGetLastError();
}

template <int T>
hipError_t launch_t(const PrefillArgs &a, hipStream_t s)
{
    if (a.hd <= 64)
        return launch_d<T, 64>(a, s);
    if (a.hd <= 128)
        return launch_d<T, 128>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace

int prefill_supported(int kv, uint32_t hd)
{
    return (kv == kF16 || kv == kI8 || kv == kI16) && hd >= 8 && hd % 8 == 0 &&
           hd <= 128;
}

uint32_t prefill_row_blocks(uint32_t n, uint32_t group)
{
    /* a workgroup takes kPBlock of a KV head's n x group rows */
    return (uint32_t)(((uint64_t)n * group + kPBlock - 1) / kPBlock);
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
