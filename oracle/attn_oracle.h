/*
 * attn_oracle.h - CPU restatement of Janas-LLM's KV-cache attention.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP library is compared
 * against, and the CPU baseline that bench.py times beside the GPU. Nothing
 * in the product (janas_amd/, include/) includes, links or loads it.
 *
 * It follows the reference's algorithm (/root/reference/src/llm/attention.c)
 * step for step: chunks of 256 positions at absolute offsets
 * (attention.c:25-36), one work item per (KV head, chunk) that leaves a
 * softmax partial (largest score, sum of weights, weighted values) per
 * (token, query head) (attention.c:631-810), and a merge of the partials in
 * chunk order (attention.c:870-910). The arithmetic order is that of the
 * reference's x86 FLOAT path, so that on an AVX2+FMA host the outputs agree
 * with the compiled reference bit for bit:
 *   - a score is eight lane sums of fused multiply-adds, lane i % 8, reduced
 *     as (l0+l4)+(l2+l6) + (l1+l5)+(l3+l7), then times scale, then times the
 *     position's key scale (attention.c:228-251, 255-347);
 *   - the weights are janas_exp_det(s - max) (vmath.h:36-52, a Cephes
 *     polynomial), 0 at or past the visible end or below e^-80, summed in
 *     eight lanes paired as (s0+s4)+(s2+s6) + (s1+s5)+(s3+s7)
 *     (attention.c:574-627);
 *   - a weight is then multiplied by its value scale (attention.c:761-763) and
 *     the values summed position by position with fused multiply-adds
 *     (attention.c:431-466);
 *   - the merge weighs chunk c by exp(m_c - max) computed in double and
 *     rounded to float (jmath.c:118-121), adds w * l_c unfused and w * acc_c
 *     fused (quant.c:2419-2431), then multiplies by 1 / sum
 *     (attention.c:870-910).
 * With int16 set (JANAS_ATTN_INT16 over an int8 cache) the reference's
 * integer way is followed instead, again bit for bit:
 *   - each (token, head) query row becomes int16, lrintf(q * 32767 / max|q|),
 *     with the scale max|q| / 32767 (quant_worker, attention.c:820-839);
 *   - a score is the exact int32 sum of the int16 query times the int8 key,
 *     converted to float and multiplied by the query scale, then scale, then
 *     the key scale (attention_scores.h:22-83);
 *   - the weights times the value scales are quantized per (chunk, token,
 *     head) row to 0 .. 32767 with one scale, lrintf(w * 32767 / max w)
 *     (att_wquant_ref, attention.c:158-176), and the values are the exact
 *     int32 sums of those against the int8 values, times that scale
 *     (att_values_i16_ref, attention.c:178-193; attention_scores.h:85-157);
 *   - the largest score and the sum of weights are those of the float way.
 * The element type of the cache is generic: int8 or int16 with one float
 * scale per (KV head, position) - the reference's own formats
 * (attention.h:7-16, 73-76) - or f16 / f32 without scales, the element types
 * the MI355X library also takes; for those the key and value scales are 1.
 */
#ifndef JANAS_ORACLE_ATTN_H
#define JANAS_ORACLE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum orc_kv { ORC_KV_I8 = 0, ORC_KV_I16 = 1, ORC_KV_F16 = 2, ORC_KV_F32 = 3 };

#define ORC_CHUNK 256

struct orc_attn {
    uint32_t n_head, n_kv, hd;
    uint32_t n_ctx;   /* rows per KV head in the cache (its capacity) */
    float scale;      /* of the scores */
    uint32_t window;  /* token p sees p - window + 1 .. p; 0: all */
    int ring;         /* position p in row p mod n_ctx */
    int kv;           /* enum orc_kv */
    int int16;        /* 1: the reference's INT16 scores (below); taken
                         only for int8 caches with hd a multiple of 16, as
                         attention.c:965-982 and :1061-1066 allow it */
};

/*
 * n tokens at positions pos0 .. pos0 + n - 1 attend the cache; q and out are
 * n x n_head x hd, k and v n_kv x n_ctx x hd elements of a->kv, ks and vs
 * n_kv x n_ctx (ignored for f16 / f32). last: NULL, or token j sees up to
 * last[j] (janas_attn_set_last, attention.h:89-97). Returns 0, or -1 on bad
 * arguments / out of memory. n_threads >= 1 threads split the items.
 */
int orc_attn_run(const struct orc_attn *a, const float *q, const void *k,
                 const float *ks, const void *v, const float *vs, uint32_t n,
                 uint32_t pos0, const uint32_t *last, float *out,
                 int n_threads);

/* out *= sigmoid(g), 1 / (1 + e^-g) with e^-g in double
   (model_attn.c:159-170, model_impl.h:646-649). per_head: g is n x n_head
   (one gate a head, broadcast over hd); else n x n_head x hd. */
void orc_gate(const float *g, int per_head, uint32_t n, uint32_t n_head,
              uint32_t hd, float *out);

/* The closed form, in double: softmax over exactly the positions each token
   sees, as tests/test_attention.c:67-92 and :295-318 compute it. */
int orc_attn_exact(const struct orc_attn *a, const float *q, const void *k,
                   const float *ks, const void *v, const float *vs, uint32_t n,
                   uint32_t pos0, const uint32_t *last, double *out);

/* The reference's deterministic exp (vmath.h:36-52), exposed for tests. */
float orc_exp_det(float x);

/* IEEE half to float, exact. */
float orc_f16_to_f32(uint16_t h);

/* janas_attn_ring_positions (attention.c:1048-1054). */
uint32_t orc_ring_positions(uint32_t window, uint32_t n);

#ifdef __cplusplus
}
#endif

#endif
