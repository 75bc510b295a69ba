/*
 * janas_attn.h - KV-cache attention on an MI355X (gfx950), C ABI.
 *
 * Part 1 is a drop-in for the engine's attention header
 * (/root/reference/src/llm/attention.h): the same twelve entry points with
 * the same meaning, so src/llm/model_attn.c and model_assist.c link against
 * libjanas_attn.so unchanged. The cache contract is the reference's: keys
 * and values n_head_kv x n_ctx x head_dim signed bytes (sixteen-bit with
 * janas_attn_set_kv16), one float scale per (KV head, position), position p
 * in row p (or p mod n_ctx in a ring). Pointers may be device memory (used
 * in place) or host memory: a host cache is staged through the device each
 * call (correct, but bounded by PCIe), unless it was imported
 * (janas_attn_import), when only the rows of the call's positions cross.
 *
 * Part 2 extends it for callers that keep everything on the device: f16
 * and f32 caches besides int8 / int16, any number of tokens a call, several
 * sequences a call (each its own cache), the output gate fused, and an
 * asynchronous stream. It has no counterpart in the reference header.
 *
 * Errors. janas_attn_create returns NULL on a geometry the reference
 * rejects (attention.c:998-1000) or when the device cannot be used.
 * janas_attn_run is void, as the reference's: a call the reference would
 * abort on (a ring too small, attention.c:1281-1286) aborts with a message.
 * A device failure is remembered in the instance (janas_attn_status, sticky
 * until cleared) - the reference's GPU backend likewise marks itself broken
 * and the engine carries on on the CPU (gpu_cuda.c:614-616, model.c:698-
 * 705). By default janas_attn_run then aborts, since the library has no CPU
 * path; after janas_attn_set_abort(a, 0) it returns instead, with a host
 * output filled with NaN, so the engine can check the status and fall back
 * to its own attention. The Part 2 entry points return 0 or a negative
 * JANAS_ATTN_E* code, never abort, and remember device failures too.
 */
#ifndef JANAS_ATTN_HIP_H
#define JANAS_ATTN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===== Part 1: the reference's interface (attention.h:26-112) ======== */

/* attention.h:26 - tokens a janas_attn_run call takes */
#define JANAS_ATTN_MAX_BLOCK 64

/* attention.h:43-47. FLOAT: every score over the float query (the
   reference's exact path). INT16 (int8 caches, head_dim a multiple of 16):
   the reference's integer way - the query quantized to int16 a row, exact
   integer scores, the weights quantized to int16 per (chunk, token, head)
   and exact integer value sums (attention.c:158-193, :820-839,
   attention_scores.h) - whose scores, weights and chunk sums are the
   reference's bit for bit. janas_attn_create resolves the asked way as the
   reference does (attention.c:960-982, the JANAS_ATTN environment variable
   first): AUTO is INT16 past 16384 positions; head_dim not a multiple of
   16, or janas_attn_set_kv16(a, 1), makes it FLOAT. Then, as the
   reference's janas_attn_run does (attention.c:1183-1262), AUTO over an
   int8 cache measures both ways once, on the device, at its first call,
   and each call takes INT16 from the position measured on (per one token
   and per block): janas_attn_scores_mode reports the last call's way. The
   measurement is kept in attn_gpu.txt under the cache directory
   ($XDG_CACHE_HOME/janas, else ~/.cache/janas) by device and geometry, as
   the reference keeps attn.txt there, and a later process takes it from
   there. A Part 2 call of any length and any number of sequences measures
   at its first call outside graph capture (the allocation-free entry point
   never does) and chooses the same way - a call of several sequences INT16
   only when each would; until measured, AUTO computes FLOAT. */
enum janas_attn_scores {
    JANAS_ATTN_AUTO = 0,
    JANAS_ATTN_FLOAT = 1,
    JANAS_ATTN_INT16 = 2
};

struct janas_attn;
/* the engine's thread pool (src/common/pool.h:14): accepted, not used */
struct janas_pool;

/* attention.h:58-59 - device bytes of the partials an instance keeps for
   n_ctx positions (the same count as the reference's host partials). */
size_t janas_attn_part_bytes(uint32_t n_head, uint32_t n_head_kv,
                             uint32_t head_dim, uint32_t n_ctx);

/* attention.h:62-64 - NULL on a bad geometry (n_head_kv 0, n_head not a
   multiple of it, head_dim not a multiple of 8 or above 512, n_threads < 1),
   when the device lacks memory, or when no device is there. */
struct janas_attn *janas_attn_create(uint32_t n_head, uint32_t n_head_kv,
                                     uint32_t head_dim, uint32_t n_ctx,
                                     int n_threads, int scores);
/* attention.h:65 */
void janas_attn_destroy(struct janas_attn *a);

/* attention.h:67-69 - 1 / sqrt(head_dim) until set */
void janas_attn_set_scale(struct janas_attn *a, float scale);
/* attention.h:70-72 - token p sees p - window + 1 .. p; 0: all */
void janas_attn_set_window(struct janas_attn *a, uint32_t window);
/* attention.h:73-76 - int16 keys and values with the same scales */
void janas_attn_set_kv16(struct janas_attn *a, int on);
/* attention.h:77-84 - position p in row p mod n_ctx (n_ctx a multiple of
   256); a call must fit (janas_attn_ring_positions) */
void janas_attn_set_ring(struct janas_attn *a, int on);
/* attention.h:85-87 */
uint32_t janas_attn_ring_positions(uint32_t window, uint32_t n);
/* attention.h:89-97 - for the next call only: token j sees up to last[j]
   (host array, n entries, read during that call) */
void janas_attn_set_last(struct janas_attn *a, const uint32_t *last);
/* attention.h:99-102 */
int janas_attn_scores_mode(const struct janas_attn *a);
int janas_attn_scores_auto(const struct janas_attn *a);

/* attention.h:104-112 - q, out: n x n_head x head_dim floats; k, v: the
   layer's cache, ks, vs its scales. n <= JANAS_ATTN_MAX_BLOCK. Synchronous:
   out is written when it returns. */
void janas_attn_run(struct janas_attn *a, struct janas_pool *pool,
                    const float *q, const int8_t *k, const float *ks,
                    const int8_t *v, const float *vs, uint32_t n,
                    uint32_t pos0, float *out);

/* The instance's first device failure since create or the last clear (a
   negative JANAS_ATTN_E* code; argument errors are not kept), or 0.
   No counterpart in attention.h: the reference marks its GPU backend
   broken (gpu_cuda.c:614-616) and the engine tests that flag. */
int janas_attn_status(const struct janas_attn *a);
void janas_attn_clear_status(struct janas_attn *a);
/* 1 (the default): janas_attn_run aborts on a device failure; 0: it
   returns, the output (host memory) filled with NaN. */
void janas_attn_set_abort(struct janas_attn *a, int on);

/* A host cache's device copy, the reference's registry of host memory on
   its GPU (janas_cuda_import / janas_cuda_sync, gpu_cuda.c:372-427; the
   engine imports each sequence's cache and scales, model_gpu.c:663-666,
   and syncs them, :527-545). No counterpart in attention.h.
   janas_attn_import copies host bytes [p, p + bytes) to device memory the
   instance keeps until janas_attn_forget or destroy. A janas_attn_run whose
   k, v, ks or vs (the layer's whole n_head_kv x n_ctx rows) lies in an
   imported range reads its device copy instead of staging the cache over
   PCIe, after taking from the host the rows of the call's positions, pos0
   up to the last position a token sees: the rows the engine has just
   written (model_attn.c writes a block's rows before its attention). Any
   other change to imported rows on the host - a context shift, a restored
   state - must be copied over with janas_attn_sync(a, p, bytes, 1) before
   the next call; janas_attn_sync(a, p, bytes, 0) copies the device's rows
   back. Both are synchronous. They return 0 or a negative JANAS_ATTN_E*
   code: EINVAL for a null pointer or 0 bytes, a range overlapping another
   import only in part, or a sync outside every import; ENOMEM. A range
   inside one already imported returns 0 and copies nothing.
   janas_attn_forget drops the import holding p (no-op if none). */
int janas_attn_import(struct janas_attn *a, const void *p, size_t bytes);
int janas_attn_sync(struct janas_attn *a, const void *p, size_t bytes,
                    int to_device);
void janas_attn_forget(struct janas_attn *a, const void *p);

/* ===== Part 2: the device extension (no counterpart in the reference) = */

enum janas_attn_kv {
    JANAS_ATTN_KV_I8 = 0,  /* int8, float scale per (KV head, position) */
    JANAS_ATTN_KV_I16 = 1, /* int16, the same scales */
    JANAS_ATTN_KV_F16 = 2, /* IEEE half, no scales */
    JANAS_ATTN_KV_F32 = 3  /* float, no scales */
};

enum janas_attn_gate {
    JANAS_ATTN_GATE_NONE = 0,
    JANAS_ATTN_GATE_ELEM = 1, /* out *= sigmoid(g), g n x n_head x head_dim */
    JANAS_ATTN_GATE_HEAD = 2  /* g n x n_head, one gate a head */
};

enum janas_attn_err {
    JANAS_ATTN_OK = 0,
    JANAS_ATTN_EINVAL = -1,  /* bad arguments */
    JANAS_ATTN_ERANGE = -2,  /* positions past the cache, a ring too small,
                                n x n_head above 2^31 - 1 */
    JANAS_ATTN_ENOMEM = -3,  /* device memory */
    JANAS_ATTN_EDEVICE = -4, /* a HIP call failed */
    JANAS_ATTN_ENOTSUP = -5  /* no kernel for this element type / size */
};

/* One sequence of a call. Every pointer is a device address. */
struct janas_attn_seq {
    const void *k, *v;    /* n_head_kv x cap x head_dim elements */
    const float *ks, *vs; /* n_head_kv x cap, int8 / int16 caches only */
    const float *q;       /* n x n_head x head_dim */
    float *out;           /* n x n_head x head_dim */
    const float *gate;    /* per the call's gate mode, or NULL */
    const uint32_t *last; /* n entries (set_last's meaning), or NULL */
    uint32_t cap;         /* rows a KV head: the cache's n_ctx */
    uint32_t n;           /* tokens */
    uint32_t pos0;        /* position of the first */
    uint32_t last_max;    /* with last: last[n - 1]; ignored otherwise */
    /* or NULL: the output (gated) also as Q8_K blocks for the next product,
       n x (n_head * head_dim / 256) struct janas_attn_q8k, as att_out_tok
       makes them (model_attn.c:159-170); n_head * head_dim a multiple of
       256 */
    void *out_q8k;
};

/* struct janas_block_q8k (src/llm/quant.h:283-300): 256 numbers as int8
   with one scale, their sums of 16, the same numbers in 8 blocks of 32 with
   scales of their own and their sums, and the sums of 32 - 628 bytes. */
#define JANAS_ATTN_QK 256
struct janas_attn_q8k {
    float d;
    int8_t qs[JANAS_ATTN_QK];
    int16_t bsums[JANAS_ATTN_QK / 16];
    float d32[8];
    int8_t qs32[JANAS_ATTN_QK];
    int16_t bsums32[JANAS_ATTN_QK / 16];
    int16_t bsums2[JANAS_ATTN_QK / 32];
};

/*
 * Attention of n_seqs sequences on a stream (a hipStream_t; NULL: the
 * instance's own), asynchronous. The instance's geometry, scale, window,
 * ring and scores way (INT16 for int8 caches) apply to all. Blocks of up to
 * JANAS_ATTN_MAX_BLOCK tokens a sequence take the split-KV path, whose
 * chunking matches janas_attn_run bit for bit token by token; longer
 * prompts take the MFMA prefill path - except int8 caches under INT16, which
 * stay on the split-KV path at any length. Over f16 caches the prefill path
 * computes with an f16 query and weights (within 2e-3 of softmax-normalized
 * outputs); over int8 and int16 caches up to head_dim 256 it is
 * float-accurate like the reference's FLOAT way (the cached integers exact,
 * the query and the weights as two f16 planes each, within 1e-5), over a
 * copy of the rows the call sees that the instance holds (2 x planes x
 * n_head_kv x positions x head_dim x 2 bytes; planes 1 for int8, 2 for
 * int16). A prompt whose row blocks alone would
 * leave compute units idle (a short prompt, a chunk of a long one) has its
 * key range split into segments, merged in order through the partials; the
 * split depends on the sequence and the device alone, so its result is the
 * same in any launch. The instance's partials are grown as needed; one call
 * at a time per instance.
 */
int janas_attn_run_dev(struct janas_attn *a, int kv_type, int gate_mode,
                       const struct janas_attn_seq *seqs, uint32_t n_seqs,
                       void *stream);

/* The same, always through the split-KV path (any n). int8, int16 and f16
   caches take head_dim up to 512, f32 caches up to 128
   (JANAS_ATTN_ENOTSUP above). */
int janas_attn_run_dev_split(struct janas_attn *a, int kv_type, int gate_mode,
                             const struct janas_attn_seq *seqs,
                             uint32_t n_seqs, void *stream);

/* The same, always through the MFMA prefill path: f16, int8 and int16
   caches, head_dim up to 512 (JANAS_ATTN_ENOTSUP for f32 caches;
   janas_attn_run_dev then takes the split-KV path). Its arithmetic is the
   FLOAT way's whatever the instance's scores way: float-accurate over int8
   and int16 caches up to head_dim 256, f16 query and weights over f16
   caches, and rows dequantized into f16 over int8 / int16 caches at
   head_dim 264..512. */
int janas_attn_run_dev_prefill(struct janas_attn *a, int kv_type,
                               int gate_mode,
                               const struct janas_attn_seq *seqs,
                               uint32_t n_seqs, void *stream);

/*
 * janas_attn_run_dev without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops that
 * forbid it). No counterpart in the reference. The partials, and the copy
 * of an int8 / int16 prompt's rows, live in one fixed array of
 * JANAS_ATTN_NOALLOC_BYTES that each GPU holds from the library's first
 * janas_attn_create on it until the process ends, instead of the
 * instance's; a call that needs more returns JANAS_ATTN_ERANGE. Calls
 * that overlap on one GPU (any instance, any stream) share that array and
 * race: the caller keeps them in order (one stream, or events).
 */
#define JANAS_ATTN_NOALLOC_BYTES (64u << 20)
int janas_attn_run_dev_noalloc(struct janas_attn *a, int kv_type, int gate_mode,
                               const struct janas_attn_seq *seqs,
                               uint32_t n_seqs, void *stream);

/* For measurement: the split-KV path's kernels one at a time - kernels 1
   the split kernel alone (partials only), 2 the merge alone (over the
   partials a previous call left), 3 both (janas_attn_run_dev_split). */
int janas_attn_run_dev_kernels(struct janas_attn *a, int kv_type,
                               int gate_mode,
                               const struct janas_attn_seq *seqs,
                               uint32_t n_seqs, void *stream, int kernels);

/* A message for a JANAS_ATTN_E* code. */
const char *janas_attn_strerror(int err);

/*
 * Kernel timing for measurement: while on, every launch of the instance is
 * bracketed by HIP events on its stream; janas_attn_prof_read returns, per
 * kernel (0 split, 1 merge, 2 prefill), the launches and their summed
 * milliseconds (synchronizing the stream), and zeroes them.
 */
void janas_attn_prof_enable(struct janas_attn *a, int on);
int janas_attn_prof_read(struct janas_attn *a, uint32_t counts[3],
                         double ms[3]);

/* ===== Part 3: the cache around the attention ========================
   The rules the engine applies to a layer's cache besides reading it
   (src/llm/model_attn.c, model.c, model_state.c), on the device. No
   counterpart in attention.h: the engine does these on the CPU. All take a
   stream (NULL: the default stream), are asynchronous, and return 0 or a
   negative JANAS_ATTN_E* code. */

/* One layer's cache on the device. */
struct janas_attn_cache {
    void *k, *v;          /* n_kv x cap x head_dim elements of kv_type */
    float *ks, *vs;       /* n_kv x cap scales (int8 / int16 caches) */
    uint32_t n_kv;
    uint32_t head_dim;    /* up to 512 */
    uint32_t cap;         /* rows a KV head */
    int kv_type;          /* enum janas_attn_kv */
    int ring;             /* position p in row p mod cap */
};

/*
 * qkv_item's key and value part (model_attn.c:75-146) for tokens pos0 ..
 * pos0 + n - 1: each key row of k (n x n_kv x head_dim floats, device) is
 * rms-normalized with k_norm (head_dim weights, or NULL: none), turned by
 * the NeoX RoPE of its token (cs, sn: n x n_rot / 2 device floats, the
 * engine's tables), each value row of v optionally normalized without
 * weights (v_norm, Gemma 4), and both written into the cache - int8 or
 * int16 with a scale of their own (the largest magnitude becomes 127 or
 * 32767), f16 or f32 as they are. k and v are not modified. Bit for bit the
 * reference's arithmetic.
 */
int janas_attn_cache_write(const struct janas_attn_cache *c, const float *k,
                           const float *v, const float *k_norm, float eps,
                           const float *cs, const float *sn, uint32_t n_rot,
                           int v_norm, uint32_t pos0, uint32_t n,
                           void *stream);

/* The query side of qkv_item (model_attn.c:86-97): rows of q
   (n x n_head x head_dim, device) normalized with q_norm (or not) and
   turned, in place. */
int janas_attn_q_prep(float *q, const float *q_norm, float eps,
                      const float *cs, const float *sn, uint32_t n_rot,
                      uint32_t n, uint32_t n_head, uint32_t head_dim,
                      void *stream);

/*
 * One layer's part of janas_llm_model_shift (model.c:292-377): of the n_pos
 * positions, keep .. keep + drop - 1 are forgotten and the ones after them
 * move down by drop, their keys turned back by the angles of drop positions
 * (cs, sn: n_rot / 2 device floats, as the engine computes them:
 * model.c:323-329) and quantized anew; a ring moves the positions it still
 * holds. int8 / int16 caches. Allocates a copy of the moved rows for the
 * call (and synchronizes the stream to free it).
 */
int janas_attn_cache_shift(const struct janas_attn_cache *c, uint32_t keep,
                           uint32_t drop, uint32_t n_pos, const float *cs,
                           const float *sn, uint32_t n_rot, void *stream);

/*
 * The rows a saved state holds (copy_kv, model_state.c:175-218): of a state
 * of n_pos positions, `rows` positions of every KV head - 0 .. rows - 1, or
 * for a ring the last rows (n_pos - rows .. n_pos - 1, wherever the ring
 * has them) - packed head after head in position order: k, v rows x n_kv x
 * head_dim elements, ks, vs rows x n_kv floats (int8 / int16; NULL
 * otherwise). out 1: cache to the buffers; 0: buffers to the cache. The
 * buffers may be host or device memory.
 */
int janas_attn_cache_copy(const struct janas_attn_cache *c, uint32_t n_pos,
                          uint32_t rows, void *k, void *v, float *ks,
                          float *vs, int out, void *stream);

#ifdef __cplusplus
}
#endif

#endif
