/*
 * attn_kernels.h - launch descriptors shared by the host API (attn_api.cpp)
 * and the HIP kernels (attn_split.hip, attn_prefill.hip). Internal: not part
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
/* sequences one launch takes (by value in its arguments) */
constexpr uint32_t kMaxSeqs = 16;

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
    uint32_t rtiles;       /* query-row tiles of 16 (rows = n x group) */
    uint32_t wg0;          /* first workgroup of the split launch */
    uint32_t mg0;          /* first workgroup of the merge launch */
    uint32_t pad_;
    uint64_t part0;        /* first partial row (of m, l and hd values) */
};

struct SplitArgs {
    SeqDesc seq[kMaxSeqs];
    float *part_ml;        /* [rows][2]: largest score, sum of weights */
    float *part_acc;       /* [rows][hd]: weighted values */
    uint32_t n_seqs, n_wg;
    uint32_t n_head, n_kv, group, hd, window;
    float scale;
    int ring;
    int gate_mode;
};

/* The causal MFMA pass over whole prompts (prefill, chunked prefill). */
struct PrefillArgs {
    SeqDesc seq[kMaxSeqs];
    uint32_t n_seqs, n_wg;
    uint32_t n_head, n_kv, group, hd, window;
    float scale;
    int ring;
    int gate_mode;
};

/* Launchers (attn_split.hip). Return hipSuccess or the launch's error. */
hipError_t launch_split(int kv, const SplitArgs &a, hipStream_t s);
hipError_t launch_merge(const SplitArgs &a, uint32_t n_wg, hipStream_t s);
/* 1 when the split kernel has an instance for this element type and
   padded head size. */
int split_supported(int kv, uint32_t hd);

/* attn_prefill.hip */
hipError_t launch_prefill(int kv, const PrefillArgs &a, hipStream_t s);
int prefill_supported(int kv, uint32_t hd);
/* prefill workgroups a KV head of an n-token sequence takes */
uint32_t prefill_row_blocks(uint32_t n, uint32_t group);

}  // namespace janas

#endif
