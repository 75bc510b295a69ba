/* SPDX-License-Identifier: GPL-3.0-or-later
 * Restates, nearly line for line where bit-exactness needs it, code of
 * Janas-LLM, Copyright (C) 2026 Maurizio Cammalleri, GPL-3.0-or-later:
 * q8_32_ref, janas_q8k_quantize (src/llm/quant.c), rms_norm,
 * rope_neox and the key / value part of qkv_item (src/llm/model_impl.h,
 * src/llm/model_attn.c) and the shift rules of src/llm/model.c. */
/*
 * cache_oracle.c - CPU restatement of the cache-side rules (see
 * cache_oracle.h). TEST INFRASTRUCTURE ONLY. Each function follows the
 * reference's code step for step, citing it; build with -ffp-contract=off.
 */
#include "cache_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- Q8_K (quant.c:150-200) ------------------------------------------ */

/* the eight blocks of 32 with scales of their own (q8_32_ref, quant.c:
   150-172, its det = 0 form) */
static void q8_32(const float *x, struct orc_q8k *y)
{
    for (int k = 0; k < 8; k++) {
        const float *xk = x + 32 * k;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++)
            amax = fmaxf(amax, fabsf(xk[i]));
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        y->d32[k] = d;
        for (int i = 0; i < 32; i++) {
            float q = nearbyintf(xk[i] * id);
            y->qs32[32 * k + i] =
                (int8_t)(q > 127.0f ? 127 : (q < -127.0f ? -127 : q));
        }
    }
    for (int g = 0; g < ORC_QK / 16; g++) {
        int s = 0;
        for (int i = 0; i < 16; i++)
            s += y->qs32[g * 16 + i];
        y->bsums32[g] = (int16_t)s;
    }
}

void orc_q8k_quantize(const float *x, struct orc_q8k *y, size_t n)
{
    /* q8k_quantize_ref (quant.c:174-200) */
    for (size_t b = 0; b < n / ORC_QK; b++, x += ORC_QK) {
        float amax = 0.0f;
        for (int i = 0; i < ORC_QK; i++)
            if (fabsf(x[i]) > amax)
                amax = fabsf(x[i]);
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        y[b].d = d;
        for (int i = 0; i < ORC_QK; i++) {
            int q = (int)lrintf(x[i] * id);
            y[b].qs[i] = (int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
        }
        for (int g = 0; g < ORC_QK / 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++)
                s += y[b].qs[g * 16 + i];
            y[b].bsums[g] = (int16_t)s;
        }
        for (int k = 0; k < ORC_QK / 32; k++)
            y[b].bsums2[k] =
                (int16_t)(y[b].bsums[2 * k] + y[b].bsums[2 * k + 1]);
        q8_32(x, &y[b]);
    }
}

/* ---- norm and RoPE (model_impl.h:635-644, model_attn.c:30-39) -------- */

static void rms_norm(float *out, const float *x, const float *w, uint32_t n,
                     float eps)
{
    double ss = 0.0;
    for (uint32_t i = 0; i < n; i++)
        ss += (double)x[i] * x[i];
    float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (uint32_t i = 0; i < n; i++)
        out[i] = x[i] * scale * w[i];
}

static void rope_neox(float *v, uint32_t n, const float *cs, const float *sn)
{
    uint32_t half = n / 2;
    for (uint32_t i = 0; i < half; i++) {
        float a = v[i], b = v[i + half];
        v[i] = a * cs[i] - b * sn[i];
        v[i + half] = a * sn[i] + b * cs[i];
    }
}

/* ---- the cache write (model_attn.c:75-146) --------------------------- */

void orc_cache_write(float *k, float *v, const float *k_norm, float eps,
                     const float *cs, const float *sn, uint32_t n_rot,
                     int v_norm, uint32_t n, uint32_t n_kv, uint32_t hd,
                     uint32_t pos0, uint32_t cap, int ring, int wide,
                     void *kc, void *vc, float *kz, float *vz)
{
    uint32_t half = n_rot / 2;
    for (uint32_t j = 0; j < n; j++)
        for (uint32_t h = 0; h < n_kv; h++) {
            float *kv = k + ((size_t)j * n_kv + h) * hd;
            float *vr = v + ((size_t)j * n_kv + h) * hd;
            if (k_norm)
                rms_norm(kv, kv, k_norm, hd, eps);
            rope_neox(kv, n_rot, cs + (size_t)j * half, sn + (size_t)j * half);
            uint32_t p = pos0 + j, row = ring ? p % cap : p;
            size_t at = ((size_t)h * cap + row) * hd;
            size_t as = (size_t)h * cap + row;
            if (v_norm) {
                double ss = 0.0;
                for (uint32_t i = 0; i < hd; i++)
                    ss += (double)vr[i] * vr[i];
                float sc = 1.0f / sqrtf((float)(ss / hd) + eps);
                for (uint32_t i = 0; i < hd; i++)
                    vr[i] *= sc;
            }
            float mk = 0.0f, mv = 0.0f;
            for (uint32_t i = 0; i < hd; i++) {
                float a = fabsf(kv[i]), b = fabsf(vr[i]);
                if (a > mk)
                    mk = a;
                if (b > mv)
                    mv = b;
            }
            float top = wide ? 32767.0f : 127.0f;
            kz[as] = mk / top;
            vz[as] = mv / top;
            float ik = mk > 0 ? top / mk : 0.0f;
            float iv = mv > 0 ? top / mv : 0.0f;
            for (uint32_t i = 0; i < hd; i++) {
                if (wide) {
                    ((int16_t *)kc)[at + i] = (int16_t)lrintf(kv[i] * ik);
                    ((int16_t *)vc)[at + i] = (int16_t)lrintf(vr[i] * iv);
                } else {
                    ((int8_t *)kc)[at + i] = (int8_t)lrintf(kv[i] * ik);
                    ((int8_t *)vc)[at + i] = (int8_t)lrintf(vr[i] * iv);
                }
            }
        }
}

void orc_q_prep(float *q, const float *q_norm, float eps, const float *cs,
                const float *sn, uint32_t n_rot, uint32_t n, uint32_t n_head,
                uint32_t hd)
{
    uint32_t half = n_rot / 2;
    for (uint32_t j = 0; j < n; j++)
        for (uint32_t h = 0; h < n_head; h++) {
            float *r = q + ((size_t)j * n_head + h) * hd;
            if (q_norm)
                rms_norm(r, r, q_norm, hd, eps);
            rope_neox(r, n_rot, cs + (size_t)j * half, sn + (size_t)j * half);
        }
}

/* ---- the context shift (model.c:263-377) ----------------------------- */

void orc_unrotate_row(void *row, float *scale, uint32_t hd, uint32_t half,
                      const float *cs, const float *sn, int wide)
{
    float tmp[512], mx = 0.0f, z = *scale;
    int8_t *r8 = row;
    int16_t *r16 = row;
    for (uint32_t i = 0; i < hd; i++)
        tmp[i] = (wide ? (float)r16[i] : (float)r8[i]) * z;
    for (uint32_t i = 0; i < half; i++) {
        float a = tmp[i], b = tmp[i + half];
        tmp[i] = a * cs[i] + b * sn[i];
        tmp[i + half] = b * cs[i] - a * sn[i];
    }
    for (uint32_t i = 0; i < hd; i++)
        if (fabsf(tmp[i]) > mx)
            mx = fabsf(tmp[i]);
    float top = wide ? 32767.0f : 127.0f, inv = mx > 0 ? top / mx : 0.0f;
    for (uint32_t i = 0; i < hd; i++) {
        if (wide)
            r16[i] = (int16_t)lrintf(tmp[i] * inv);
        else
            r8[i] = (int8_t)lrintf(tmp[i] * inv);
    }
    *scale = mx / top;
}

int orc_cache_shift(void *k, void *v, float *kz, float *vz, uint32_t n_kv,
                    uint32_t hd, uint32_t cap, int ring, int wide,
                    uint32_t keep, uint32_t drop, uint32_t n_pos,
                    const float *cs, const float *sn, uint32_t n_rot)
{
    if (!drop || hd > 512 || keep + drop > n_pos || (!ring && n_pos > cap))
        return -1;
    uint32_t move = n_pos - keep - drop, half = n_rot / 2;
    size_t row = (size_t)hd << (wide ? 1 : 0);
    uint8_t *tmp = NULL;
    for (uint32_t h = 0; h < n_kv; h++) {
        uint8_t *kh = (uint8_t *)k + (size_t)h * cap * row;
        uint8_t *vh = (uint8_t *)v + (size_t)h * cap * row;
        float *kzh = kz + (size_t)h * cap, *vzh = vz + (size_t)h * cap;
        if (!ring) {
            if (move) {
                memmove(kh + keep * row, kh + (keep + drop) * row, move * row);
                memmove(vh + keep * row, vh + (keep + drop) * row, move * row);
                memmove(kzh + keep, kzh + keep + drop, move * sizeof(float));
                memmove(vzh + keep, vzh + keep + drop, move * sizeof(float));
            }
            for (uint32_t p = keep; p < keep + move && half; p++)
                orc_unrotate_row(kh + p * row, kzh + p, hd, half, cs, sn, wide);
            continue;
        }
        if (!tmp && !(tmp = malloc(2 * (size_t)cap * (row + sizeof(float)))))
            return -1;
        uint8_t *tk = tmp, *tv = tk + cap * row;
        float *tkz = (float *)(void *)(tv + cap * row), *tvz = tkz + cap;
        memcpy(tk, kh, cap * row);
        memcpy(tv, vh, cap * row);
        memcpy(tkz, kzh, cap * sizeof(float));
        memcpy(tvz, vzh, cap * sizeof(float));
        uint32_t lo = keep + drop;
        if (n_pos > cap && n_pos - cap > lo)
            lo = n_pos - cap;
        for (uint32_t p = lo; p < n_pos; p++) {
            uint32_t src = p % cap, dst = (p - drop) % cap;
            memcpy(kh + dst * row, tk + src * row, row);
            memcpy(vh + dst * row, tv + src * row, row);
            kzh[dst] = tkz[src];
            vzh[dst] = tvz[src];
            if (half)
                orc_unrotate_row(kh + dst * row, kzh + dst, hd, half, cs, sn,
                                 wide);
        }
    }
    free(tmp);
    return 0;
}
