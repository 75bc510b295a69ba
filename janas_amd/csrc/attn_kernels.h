/*
 * attn_kernels.h - launch descriptors shared by the host API (attn_api.cpp)
 * and the HIP kernels (attn_split.hip, attn_wide.hip, attn_prefill.hip,
 * attn_cache.hip). Internal: not part
 * of the C ABI (include/janas_attn.h).
 */
#ifndef JANAS_AMD_ATTN_KERNELS_H
#define JANAS_AMD_ATTN_KERNELS_H

#include <stdint.h>

#include <hip/hip_runtime.h>

namespace janas {

/* positions a chunk: partials are kept per chunk at absolute offsets, as
   the reference's ATT_CHUNK (attention.c:25) */
constexpr uint32_t kChunk = 256;
/* query rows a split-path workgroup takes: 8 at head sizes up to 256
   (attn_split.hip), 16 above (attn_wide.hip) */
constexpr uint32_t kTileRows = 8;
constexpr uint32_t kWideRows = 16;
inline uint32_t split_tile_rows(uint32_t hd) { return hd > 256 ? kWideRows : kTileRows; }
/* merge_cols of a merge that also puts its outputs into Q8_K blocks */
constexpr uint32_t kMergeQ8k = 256;
/* sequences one launch takes (by value in its arguments) */
constexpr uint32_t kMaxSeqs = 16;
/* merge workgroups a launch keeps at least when it takes 128 columns a
   workgroup (merge_cols) */
constexpr uint64_t kMergeFill = 256;
/* row tiles of kTileRows a split-kernel workgroup takes at most */
constexpr uint32_t kSplitMaxMt = 2;

enum KvType : int { kI8 = 0, kI16 = 1, kF16 = 2, kF32 = 3 };
enum GateMode : int { kGateNone = 0, kGateElem = 1, kGateHead = 2 };

/* One sequence of a call, as the kernels see it. Pointers are device
   addresses. */
struct SeqDesc {
    const void *k, *v;     /* [n_kv][cap][hd] */
    const float *ks, *vs;  /* [n_kv][cap], int8 / int16 only */
    const float *q;        /* [n][n_head][hd] */
    float *out;            /* [n][n_head][hd] */
    const float *gate;     /* per GateMode, or null */
    const uint32_t *last;  /* [n] or null: token j sees up to pos0 + j */
    uint32_t cap, n, pos0, end; /* end: 1 + the last position any token sees */
    uint32_t c0, span;     /* chunks c0 .. c0 + span - 1 are read */
    uint32_t rtiles;       /* workgroups along the query rows (rows = n x
                              group): of split_tile_rows(hd) x mt rows */
    uint32_t wg0;          /* first workgroup of the split launch */
    uint32_t mg0;          /* first workgroup of the merge launch */
    uint32_t nseg;         /* prefill: key segments a row block is split
                              into (1: none, the output is written directly) */
    uint64_t part0;        /* first partial row (of m, l and hd values) */
    void *q8k;             /* the output also as Q8_K blocks, or null */
};

struct SplitArgs {
    SeqDesc seq[kMaxSeqs];
    float *part_ml;        /* [rows][2]: largest score, sum of weights */
    float *part_acc;       /* [rows][hd]: weighted values */
    uint32_t n_seqs, n_wg;
    uint32_t once;         /* every sequence one row workgroup: K/V read
                              once */
    uint32_t mt;           /* split kernel: row tiles a workgroup (1 or 2;
                              split_mt) */
    uint32_t merge_cols;   /* 32 or 128 columns a merge workgroup, or
                              kMergeQ8k: one Q8_K block of 256 outputs */
    uint32_t n_head, n_kv, group, hd, window;
    float scale;
    int ring;
    int gate_mode;
    int int16;             /* the reference's INT16 scores (int8 caches,
                              hd a multiple of 16) */
    /* JANAS_ATTN_SKIPSTAT (attention.c:841-869, :883-898): counters of
       the chunks a (token, head) merged - n[2], then below[2][3] (more than
       8, 16, 32 below the row's largest score), [0] all rows, [1] rows past
       16384 positions - or null when off */
    unsigned long long *skip;
    /* seq[i].wg0 and seq[i].mg0 again, side by side (seq_index) */
    uint32_t wg0s[kMaxSeqs], mg0s[kMaxSeqs];
};

/* The causal MFMA pass over whole prompts (prefill, chunked prefill). */
struct PrefillArgs {
    SeqDesc seq[kMaxSeqs];
    float *part_ml;        /* split sequences: [partial rows][2] */
    float *part_acc;       /* [partial rows][hd]; a sequence's start at its
                              part0, (token, head) major, segment minor */
    uint32_t n_seqs, n_wg;
    uint32_t n_head, n_kv, group, hd, window;
    float scale;
    int ring;
    int gate_mode;
    int halves;            /* the two-halves kernel (prefill_halves_supported):
                              128 rows a workgroup, two key groups */
    int q8k_fused;         /* the kernel writes a sequence's Q8_K blocks
                              with its output (head size 64, 128 or 256, a
                              block's rows in one wave); the segment merge
                              always does */
    int exact;             /* int8 / int16 at float accuracy
                              (prefill_exact_kernel): the planes of the copy
                              the sequences' k and v point at (1 int8, 2
                              int16; launch_xcopy), scales from ks / vs */
    /* seq[i].wg0 and seq[i].mg0 again, side by side (seq_index) */
    uint32_t wg0s[kMaxSeqs], mg0s[kMaxSeqs];
};

/* An int8 / int16 cache's rows of positions p0 .. p0 + np - 1 as the
   exact kernel's f16 planes (xcopy_kernel): plane by plane, row
   kvh np + (p - p0) of each. */
struct XcopyArgs {
    const void *k, *v;     /* the cache, [n_kv][cap][hd] */
    _Float16 *k16, *v16;   /* the copies, [planes][n_kv][np][hd] */
    uint32_t n_kv, cap, hd, ring;
    uint32_t p0, np;
};

/* Rows of a cache write or of the query preparation (attn_cache.hip). */
struct RowArgs {
    float *k;              /* n x heads x hd: keys, or the queries (in place) */
    const float *v;        /* n x heads x hd values, or null (queries) */
    const float *norm;     /* hd weights of the key (query) norm, or null */
    const float *cs, *sn;  /* n x n_rot / 2 */
    void *kc, *vc;         /* the cache, heads x cap x hd; null: queries */
    float *kz, *vz;        /* heads x cap scales (int8 / int16) */
    float eps;
    uint32_t n, heads, hd, n_rot, pos0, cap;
    int kv, ring, v_norm;
};

/* Rows a context shift moves (attn_cache.hip). The copy holds copy_rows
   rows a KV head: rows copy_first .. of the cache, or all of a ring's. */
struct ShiftArgs {
    void *k, *v;
    float *kz, *vz;
    const void *ck, *cv;   /* the copy */
    const float *ckz, *cvz;
    const float *cs, *sn;  /* the shift's angles, n_rot / 2 */
    uint32_t n_kv, hd, cap, n_rot;
    uint32_t first, count; /* positions first .. first + count - 1 move */
    uint32_t drop, copy_first, copy_rows;
    int kv, ring;
};

/* Q8_K blocks of output rows (struct janas_block_q8k, 628 bytes). */
constexpr uint32_t kQ8kBytes = 628;
struct Q8kArgs {
    const float *x;        /* blocks x 256 */
    uint8_t *y;            /* blocks x 628 bytes */
    uint32_t blocks;
};

/* Launchers (attn_split.hip). Return hipSuccess or the launch's error. */
/* The arguments a workgroup's id is made from (a, b: the workgroup count,
   the KV head count), the sequence count and the sequences' starts in
   scalar registers at a kernel's first instruction: asked for together,
   they come in one round trip (left to the scheduler, the starts went out
   only after the wait for the id's arguments) */
__device__ __forceinline__ void starts_early(uint32_t a, uint32_t b, uint32_t n_seqs,
                                             const uint32_t *starts)
{
    static_assert(kMaxSeqs == 16, "the starts as 15 scalar operands");
    asm volatile("" ::"s"(a), "s"(b), "s"(n_seqs), "s"(starts[1]), "s"(starts[2]),
                 "s"(starts[3]), "s"(starts[4]), "s"(starts[5]), "s"(starts[6]),
                 "s"(starts[7]), "s"(starts[8]), "s"(starts[9]), "s"(starts[10]),
                 "s"(starts[11]), "s"(starts[12]), "s"(starts[13]), "s"(starts[14]),
                 "s"(starts[15]));
}
/* The sequence of a launch that workgroup id belongs to: the last whose
   first workgroup (starts[i]: the launch's wg0s or mg0s, the sequences'
   wg0 or mg0 side by side) is at or below id. Branch-free, so the 64 bytes
   of starts are read with the sequence count, in the arguments' first
   round trip, and the sequence's own descriptor in the second. */
__device__ __forceinline__ uint32_t seq_index(const uint32_t *starts, uint32_t n_seqs,
                                              uint32_t id)
{
    uint32_t si = 0;
#pragma unroll
    for (uint32_t i = 1; i < kMaxSeqs; i++)
        si += i < n_seqs && starts[i] <= id;
    return si;
}

hipError_t launch_split(int kv, const SplitArgs &a, hipStream_t s);
hipError_t launch_merge(const SplitArgs &a, uint32_t n_wg, hipStream_t s);
/* columns a merge workgroup takes for a launch of pairs (token, head). */
uint32_t merge_cols(uint64_t pairs, uint32_t hd);
/* 1 when the split kernel has an instance for this element type and
   padded head size. */
int split_supported(int kv, uint32_t hd);
/* row tiles a split-kernel workgroup takes for a launch whose largest
   sequence has `tiles` row tiles (SplitArgs::mt). */
uint32_t split_mt(int kv, uint32_t hd, uint32_t tiles);
/* attn_wide.hip: the split kernel for head sizes 264 .. 512 (8- and 16-bit
   caches); launch_split hands those to it. */
hipError_t launch_wide(int kv, const SplitArgs &a, hipStream_t s);

/* Rows of imported host caches a janas_attn_run takes (attn_cache.hip):
   for tensor t (keys, values, their scales), rows lo, lo + 1, .. (mod cap)
   of every KV head, count of them, packed [head][row] in pinned host memory
   at src[t], into the device copy dst[t] ([n_kv][cap] rows of words[t]
   4-byte words). */
struct RefreshArgs {
    const uint32_t *src[4];
    uint32_t *dst[4];
    uint32_t words[4];
    uint32_t n_t, n_kv, cap, lo, count;
};

/* attn_cache.hip */
hipError_t launch_refresh(const RefreshArgs &a, hipStream_t s);
hipError_t launch_rows(const RowArgs &a, hipStream_t s);
hipError_t launch_shift(const ShiftArgs &a, hipStream_t s);
hipError_t launch_q8k(const Q8kArgs &a, hipStream_t s);

/* attn_scratch.hip: the device address of the fixed partials array
   (JANAS_ATTN_NOALLOC_BYTES) on device dev - scratch_init looks it up once,
   with dev current; scratch_ptr returns it, or null */
int scratch_init(int dev);
void *scratch_ptr(int dev);

/* attn_prefill.hip */
hipError_t launch_prefill(int kv, const PrefillArgs &a, hipStream_t s);
int prefill_supported(int kv, uint32_t hd);
/* row blocks a KV head of an n-token sequence takes (one workgroup each
   per key segment), and the key positions a tile; halves: the two-halves
   kernel's (PrefillArgs::halves) */
uint32_t prefill_row_blocks(uint32_t n, uint32_t group, uint32_t hd, bool halves,
                            int exact = 0);
uint32_t prefill_tile(uint32_t hd, bool halves, int exact = 0);
/* 1 when the two-halves kernel takes this element type and head size */
int prefill_halves_supported(int kv, uint32_t hd);
/* xcopy_kernel: the exact kernel's copy of an int8 / int16 cache's rows
   p0 .. p0 + np - 1, per KV head from p0, as 1 (int8) or 2 (int16) planes
   of n_kv x np x hd f16 each; k16 and v16 hold the planes one after the
   other */
hipError_t launch_xcopy(int kv, const XcopyArgs &a, hipStream_t s);
/* the ordered merge of split sequences' segment partials: a thread takes 4
   columns of one row (a row is one (token, head)), a workgroup
   kPMergeThreads of them; a sequence of n tokens takes pmerge_groups of
   them */
constexpr uint32_t kPMergeThreads = 256;
/* key segments a prefill row block is split into, at most */
constexpr uint32_t kMaxSegs = 16;
inline uint64_t pmerge_groups(uint32_t n, uint32_t n_head, uint32_t hd)
{
    return ((uint64_t)n * n_head * (hd / 4) + kPMergeThreads - 1) / kPMergeThreads;
}
hipError_t launch_prefill_merge(const PrefillArgs &a, uint32_t n_wg, hipStream_t s);

}  // namespace janas

#endif
