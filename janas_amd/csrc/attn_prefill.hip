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
 *   key tiles   64 positions of K and V in LDS, two buffers; the next tile
 *               is loaded into registers while this one is computed.
 *   scores      S^T = K . Q^T, v_mfma_f32_16x16x32_f16: A = K rows from LDS,
 *               B = the query in f16, scaled by the score scale times
 *               log2(e) so the weights are exp2(s - max); lane l ends with
 *               row l % 16 at positions 4 (l / 16) + i, the A layout of the
 *               value product.
 *   values      O = P . V with the weights in f16 as they are, V rows read
 *               back transposed with ds_read_b64_tr_b16; f32 accumulation.
 *   masks       only the tiles a row's range cuts; tiles wholly outside
 *               every row's range are skipped.
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
typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kPWaves = 8;                 /* waves a workgroup */
constexpr int kPRows = 32;                 /* query rows a wave */
constexpr int kPBlock = kPWaves * kPRows;  /* query rows a workgroup */
constexpr int kTile = 64;                  /* key positions a tile */
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f4 mfma(h8 a, h8 b, f4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
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

template <int D> struct PShape {
    static constexpr int KP = D + 8;   /* halves a K row in LDS (pitch) */
    static constexpr int VP = D + 16;  /* halves a V row in LDS */
    static constexpr int KS = D / 32;  /* score k-steps */
    static constexpr int NT = D / 16;  /* output column tiles */
    /* a tile's 16-byte units of K (and of V), and a thread's share */
    static constexpr int UNITS = kTile * D * 2 / 16;
    static constexpr int UPT = UNITS / (kPWaves * 64);
    static constexpr int UPR = D * 2 / 16;  /* units a row */
};

template <int D>
__global__ __launch_bounds__(512) void prefill_kernel(const PrefillArgs A)
{
    using S = PShape<D>;
    static_assert(S::UPT >= 1 && S::UNITS % (kPWaves * 64) == 0, "tile loads");
    __shared__ __attribute__((aligned(16))) _Float16 sK[2][kTile][S::KP];
    __shared__ __attribute__((aligned(16))) _Float16 sV[2][kTile][S::VP];

    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint32_t g16 = lane >> 4, l16 = lane & 15;
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
    /* the first tile of the ring's or the cache's rows */
    const size_t head_row = (size_t)kvh * sq.cap;

    /* ---- the wave's rows: row-tile rt covers rows 32 w + 16 rt + l16 ---- */
    uint32_t rlo[2], rhi[2];
    h8 qb[2][S::KS];
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        const uint32_t r = r0 + kPRows * w + 16 * rt + l16;
        const bool ok = r < R;
        const uint32_t rr = ok ? r : r0;
        const uint32_t j = rr / G, h = kvh * G + rr % G;
        rlo[rt] = ok ? row_lo(A, sq.pos0 + j) : 1;
        rhi[rt] = ok ? (sq.last ? sq.last[j] : sq.pos0 + j) : 0;
        const float *qrow = sq.q + ((size_t)j * A.n_head + h) * hd;
        const float f = A.scale * kLog2e;
#pragma unroll
        for (int s = 0; s < S::KS; s++) {
            const uint32_t c = 32 * s + 8 * g16;
            const bool cok = ok && c < hd;
            const float4 x0 = *(const float4 *)(qrow + (cok ? c : 0));
            const float4 x1 = *(const float4 *)(qrow + (cok ? c + 4 : 0));
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; e++)
                qb[rt][s][e] = (_Float16)(cok ? xs[e] * f : 0.0f);
        }
    }

    /* ---- a tile's K and V: thread t's units t + 512 u. Positions outside
       [lo_all, hi_all] read the nearest of the two (masked, but never a row
       the caller has not written); columns past hd read column 0 (their
       products meet zero query columns, or are not stored) ---- */
    auto load = [&](uint32_t tile, u4 *kr, u4 *vr) {
#pragma unroll
        for (int u = 0; u < S::UPT; u++) {
            const uint32_t unit = tid + u * (kPWaves * 64);
            const uint32_t row = unit / S::UPR, cu = unit % S::UPR;
            uint32_t p = tile * kTile + row;
            p = p < lo_all ? lo_all : p > hi_all ? hi_all : p;
            const size_t cr = head_row + (A.ring ? p % sq.cap : p);
            const uint32_t col = cu * 8 < hd ? cu * 8 : 0;
            kr[u] = *(const u4 *)((const uint16_t *)sq.k + cr * hd + col);
            vr[u] = *(const u4 *)((const uint16_t *)sq.v + cr * hd + col);
        }
    };
    auto store = [&](int b, const u4 *kr, const u4 *vr) {
#pragma unroll
        for (int u = 0; u < S::UPT; u++) {
            const uint32_t unit = tid + u * (kPWaves * 64);
            const uint32_t row = unit / S::UPR, cu = unit % S::UPR;
            *(u4 *)&sK[b][row][cu * 8] = kr[u];
            *(u4 *)&sV[b][row][cu * 8] = vr[u];
        }
    };

    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    f4 o[2][S::NT];
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int t = 0; t < S::NT; t++)
            o[rt][t] = f4{0, 0, 0, 0};

    u4 kr[S::UPT], vr[S::UPT];
    load(tfirst, kr, vr);
    store(0, kr, vr);
    __syncthreads();

    for (uint32_t tile = tfirst; tile <= tlast; tile++) {
        const int b = (tile - tfirst) & 1;
        if (tile < tlast)
            load(tile + 1, kr, vr);
        const uint32_t p0 = tile * kTile;
        /* does any of this wave's rows see only part of the tile, or
           none of it? (then every score is checked) */
        bool partial = false;
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
            partial |= !(rlo[rt] <= p0 && rhi[rt] >= p0 + kTile - 1);
        const bool check = __any(partial);

        /* scores: 4 position tiles x 2 row tiles */
        f4 sacc[4][2];
#pragma unroll
        for (int pt = 0; pt < 4; pt++) {
            sacc[pt][0] = f4{0, 0, 0, 0};
            sacc[pt][1] = f4{0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < S::KS; s++)
#pragma unroll
            for (int pt = 0; pt < 4; pt++) {
                const h8 ka = *(const h8 *)&sK[b][16 * pt + l16][32 * s + 8 * g16];
                sacc[pt][0] = mfma(ka, qb[0][s], sacc[pt][0]);
                sacc[pt][1] = mfma(ka, qb[1][s], sacc[pt][1]);
            }

        /* online softmax per row; lane l: row l16 of each row tile at
           positions 16 pt + 4 g16 + i */
        h8 pa[2][2];
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
            float sv[16];
            float mt = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                float x = sacc[e / 4][rt][e % 4];
                if (check) {
                    const uint32_t p = p0 + 16 * (e / 4) + 4 * g16 + e % 4;
                    if (p < rlo[rt] || p > rhi[rt])
                        x = -INFINITY;
                }
                sv[e] = x;
                mt = fmaxf(mt, x);
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float mn = fmaxf(m[rt], mt);
            /* a row that has seen nothing yet keeps its zeros */
            const float ms = mn == -INFINITY ? 0.0f : mn;
            const float alpha = exp2f(m[rt] - ms);
            float ls = 0.0f;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float pw = exp2f(sv[e] - ms);
                ls += pw;
                pa[rt][e / 8][e % 8] = (_Float16)pw;
            }
            l[rt] = l[rt] * alpha + ls;
            m[rt] = mn;
            /* rescale the sums: rows 4 g16 + i of the row tile */
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float ai = __shfl(alpha, 4 * g16 + i, 64);
#pragma unroll
                for (int t = 0; t < S::NT; t++)
                    o[rt][t][i] *= ai;
            }
        }

        /* values: k-slot j of k-step kk is position 32 kk + 4 g16 + j
           (j < 4) or 32 kk + 16 + 4 g16 + j - 4 */
#pragma unroll
        for (int t = 0; t < S::NT; t++) {
            const uint32_t tr = 4 * g16 + (l16 >> 2), tc = 16 * t + 4 * (l16 & 3);
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const h4 x = lds_read_tr(&sV[b][32 * kk + tr][tc]);
                const h4 y = lds_read_tr(&sV[b][32 * kk + 16 + tr][tc]);
                const h8 vb = h8{x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
                o[0][t] = mfma(pa[0][kk], vb, o[0][t]);
                o[1][t] = mfma(pa[1][kk], vb, o[1][t]);
            }
        }
        if (tile < tlast) {
            __syncthreads(); /* every wave is done with the other buffer */
            store(b ^ 1, kr, vr);
            __syncthreads();
        }
    }

    /* ---- out = sums / weights, gated; lane l holds rows 4 g16 + i ---- */
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
        float lt = l[rt];
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float li = __shfl(lt, 4 * g16 + i, 64);
            const uint32_t r = r0 + kPRows * w + 16 * rt + 4 * g16 + i;
            if (r >= R)
                continue;
            const uint32_t j = r / G, h = kvh * G + r % G;
            const float inv = 1.0f / li;
#pragma unroll
            for (int t = 0; t < S::NT; t++) {
                const uint32_t col = 16 * t + l16;
                if (col >= hd)
                    continue;
                const size_t oi = ((size_t)j * A.n_head + h) * hd + col;
                float x = o[rt][t][i] * inv;
                if (A.gate_mode == kGateElem)
                    x *= 1.0f / (1.0f + expf(-sq.gate[oi]));
                else if (A.gate_mode == kGateHead)
                    x *= 1.0f / (1.0f + expf(-sq.gate[(size_t)j * A.n_head + h]));
                sq.out[oi] = x;
            }
        }
    }
}

template <int D>
hipError_t launch_d(const PrefillArgs &a, hipStream_t s)
{
    hipLaunchKernelGGL((prefill_kernel<D>), dim3(a.n_wg), dim3(512), 0, s, a);
    return hipGetLastError();
}

}  // namespace

int prefill_supported(int kv, uint32_t hd)
{
    return kv == kF16 && hd >= 8 && hd % 8 == 0 && hd <= 128;
}

uint32_t prefill_row_blocks(uint32_t n, uint32_t group)
{
    /* a workgroup takes kPBlock of a KV head's n x group rows */
    return (uint32_t)(((uint64_t)n * group + kPBlock - 1) / kPBlock);
}

hipError_t launch_prefill(int kv, const PrefillArgs &a, hipStream_t s)
{
    if (kv != kF16)
        return hipErrorInvalidValue;
    if (a.hd <= 64)
        return launch_d<64>(a, s);
    if (a.hd <= 128)
        return launch_d<128>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace janas
