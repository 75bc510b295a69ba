/*
 * cache_oracle.h - CPU restatement of the rules around Janas-LLM's KV-cache
 * attention that the device library also implements: the K/V cache write
 * (norm, RoPE, 8 / 16-bit quantization), the context shift's re-rotation of
 * cached keys, and the Q8_K quantization of the attention output.
 *
 * TEST INFRASTRUCTURE ONLY. The checker the HIP library is compared against;
 * nothing in the product (janas_amd/, include/) includes, links or loads it.
 * Built with -ffp-contract=off, as the reference (build.sh:169-175): no
 * multiply-add is fused unless written as fmaf, so float results are the
 * reference's bit for bit where the operations are the same.
 */
#ifndef JANAS_ORACLE_CACHE_H
#define JANAS_ORACLE_CACHE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 256

/* struct janas_block_q8k (src/llm/quant.h:283-300): 628 bytes. */
struct orc_q8k {
    float d;
    int8_t qs[ORC_QK];
    int16_t bsums[ORC_QK / 16];
    float d32[8];
    int8_t qs32[ORC_QK];
    int16_t bsums32[ORC_QK / 16];
    int16_t bsums2[ORC_QK / 32];
};

/* janas_q8k_quantize's portable path (quant.c:174-200, q8_32_ref
   quant.c:150-172): n a multiple of 256. */
void orc_q8k_quantize(const float *x, struct orc_q8k *y, size_t n);

/*
 * qkv_item (model_attn.c:75-146) for rows of one layer: for each token j of
 * n and each of n_kv heads, the key row k[j][h] is rms-normalized with
 * k_norm (if not NULL; model_impl.h:635-644), turned by the NeoX RoPE of its
 * token (cs, sn: n x n_rot / 2; model_attn.c:30-39), the value row
 * optionally normalized without weights (v_norm, Gemma 4: model_attn.c:
 * 106-113), and both quantized with a scale of their own (the largest
 * magnitude becomes 127, or 32767 with wide) into row pos0 + j (mod cap with
 * ring) of kc / vc (n_kv x cap x hd) and kz / vz (n_kv x cap).
 * k and v (n x n_kv x hd) are modified in place, as the reference does.
 */
void orc_cache_write(float *k, float *v, const float *k_norm, float eps,
                     const float *cs, const float *sn, uint32_t n_rot,
                     int v_norm, uint32_t n, uint32_t n_kv, uint32_t hd,
                     uint32_t pos0, uint32_t cap, int ring, int wide,
                     void *kc, void *vc, float *kz, float *vz);

/* The query side of qkv_item (model_attn.c:86-97): rows q[j][h]
   (n x n_head x hd) normalized with q_norm (if not NULL) and turned, in
   place. */
void orc_q_prep(float *q, const float *q_norm, float eps, const float *cs,
                const float *sn, uint32_t n_rot, uint32_t n, uint32_t n_head,
                uint32_t hd);

/* unrotate_row (model.c:263-290): a cached key row turned back by the
   angles cs, sn (n_rot / 2 pairs) and quantized anew; row int8 or int16
   (wide), its scale updated. */
void orc_unrotate_row(void *row, float *scale, uint32_t hd, uint32_t half,
                      const float *cs, const float *sn, int wide);

/* One slot's part of janas_llm_model_shift (model.c:304-377): positions
   keep .. keep + drop - 1 forgotten, the n_pos - keep - drop after them
   moved down by drop and their keys turned back; a ring keeps its last
   positions. k, v: n_kv x cap x hd (elt bytes each), kz, vz: n_kv x cap.
   Returns 0, or -1 on bad arguments / out of memory. */
int orc_cache_shift(void *k, void *v, float *kz, float *vz, uint32_t n_kv,
                    uint32_t hd, uint32_t cap, int ring, int wide,
                    uint32_t keep, uint32_t drop, uint32_t n_pos,
                    const float *cs, const float *sn, uint32_t n_rot);

#ifdef __cplusplus
}
#endif

#endif
