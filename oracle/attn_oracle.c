/* SPDX-License-Identifier: GPL-3.0-or-later
 * Restates, nearly line for line where bit-exactness needs it, code of
 * Janas-LLM, Copyright (C) 2026 Maurizio Cammalleri, GPL-3.0-or-later:
 * att_weights_ref, janas_exp_det, quant_worker, att_wquant_ref and
 * the item / merge steps of src/llm/attention.c and src/llm/vmath.h. */
/*
 * attn_oracle.c - CPU restatement of Janas-LLM's KV-cache attention.
 *
 * TEST INFRASTRUCTURE ONLY (see attn_oracle.h): the checker for the HIP
 * library and the CPU baseline of bench.py. Build flags matter for the bits:
 * -O3 -mavx2 -mfma -ffp-contract=off -fno-math-errno, so that fmaf() is one
 * fused instruction and no other multiply-add is fused, as in the
 * reference's own build (build.sh:169-175).
 */
#include "attn_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ---- element types ---------------------------------------------------- */

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u,
             m = h & 1023u, u;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in float */
        float f = (float)m * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    if (e == 31)
        u = sign | 0x7F800000u | (m << 13);
    else
        u = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* nt rows of hd elements from row r0 on, as floats */
static void rows_to_f32(int kv, const void *base, size_t r0, uint32_t nt,
                        uint32_t hd, float *dst)
{
    size_t n = (size_t)nt * hd, off = r0 * hd;
    switch (kv) {
    case ORC_KV_I8: {
        const int8_t *s = (const int8_t *)base + off;
        for (size_t i = 0; i < n; i++)
            dst[i] = (float)s[i];
        break;
    }
    case ORC_KV_I16: {
        const int16_t *s = (const int16_t *)base + off;
        for (size_t i = 0; i < n; i++)
            dst[i] = (float)s[i];
        break;
    }
    case ORC_KV_F16: {
        const uint16_t *s = (const uint16_t *)base + off;
        for (size_t i = 0; i < n; i++)
            dst[i] = orc_f16_to_f32(s[i]);
        break;
    }
    default:
        memcpy(dst, (const float *)base + off, n * sizeof(float));
    }
}

/* ---- the reference's deterministic exp (vmath.h:36-52) ---------------- */

float orc_exp_det(float x)
{
    /* x = n ln 2 + r, ln 2 in two parts; e^r by the Cephes expf polynomial;
       2^n put into the exponent */
    x = fminf(fmaxf(x, -88.0f), 88.0f);
    float n = nearbyintf(x * 1.44269504088896341f);
    float r = fmaf(-n, 0.693359375f, x);
    r = fmaf(-n, -2.12194440e-4f, r);
    float y = 1.9875691500e-4f;
    y = fmaf(y, r, 1.3981999507e-3f);
    y = fmaf(y, r, 8.3334519073e-3f);
    y = fmaf(y, r, 4.1665795894e-2f);
    y = fmaf(y, r, 1.6666665459e-1f);
    y = fmaf(y, r, 5.0000001201e-1f);
    y = fmaf(y, r * r, r);
    y = y + 1.0f;
    uint32_t e = (uint32_t)((int32_t)n + 127) << 23;
    float p;
    memcpy(&p, &e, 4);
    return y * p;
}

/* ---- one work item: (KV head, chunk) for every token and group head --- */

struct job {
    const struct orc_attn *A;
    const float *q, *ks, *vs;
    const void *k, *v;
    const uint32_t *last;
    float *out;
    uint32_t n, pos0, n_chunks, c0, group;
    float *part; /* n_kv x span x n x group x (hd + 2) */
    int16_t *qi; /* INT16: the quantized query, n x n_head x hd, or NULL */
    float *qs;   /* and its scales, n x n_head */
    atomic_uint next;
};

static uint32_t last_seen(const struct job *a, uint32_t j)
{
    return a->last ? a->last[j] : a->pos0 + j;
}

static float *partial(const struct job *a, uint32_t kvh, uint32_t c,
                      uint32_t j, uint32_t g)
{
    uint32_t span = a->n_chunks - a->c0;
    return a->part +
           ((((size_t)kvh * span + (c - a->c0)) * a->n + j) * a->group + g) *
               (a->A->hd + 2);
}

/* scores: eight lanes of fused sums, lane i % 8, reduced as the reference's
   f32_reduce8 / f32_body tail (attention.c:228-251, :327-345) */
static float dot8(const float *q, const float *k, uint32_t hd)
{
    float a[8] = {0};
    for (uint32_t i = 0; i < hd; i += 8)
        for (int l = 0; l < 8; l++)
            a[l] = fmaf(q[i + l], k[i + l], a[l]);
    return ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}

/* softmax numerators of a row (att_weights_ref / _avx2,
   attention.c:574-627): largest of the first vis, weights, their sum */
static float weights(float *row, uint32_t nt, uint32_t vis, float *mx)
{
    float m = -INFINITY, s[8] = {0};
    for (uint32_t t = 0; t < vis; t++)
        if (row[t] > m)
            m = row[t];
    for (uint32_t t = 0; t < nt; t++) {
        float d = row[t] - m;
        row[t] = t >= vis || d < -80.0f ? 0.0f : orc_exp_det(d);
        s[t % 8] += row[t];
    }
    *mx = m;
    return ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
}

struct scratch {
    float *kf, *vf, *sc; /* chunk rows as floats; a row of scores a slot */
    int16_t *w16;        /* INT16: a slot's quantized weights */
    float *wsc;          /* and their scale */
};

/* INT16 (quant_worker, attention.c:820-839): a query row to int16 with one
   scale, rounded to nearest as lrintf does */
static void quant_row(const float *src, uint32_t hd, int16_t *dst, float *sc)
{
    float mx = 0.0f;
    for (uint32_t i = 0; i < hd; i++) {
        float v = src[i] < 0.0f ? -src[i] : src[i];
        if (v > mx)
            mx = v;
    }
    *sc = mx / 32767.0f;
    float inv = mx > 0.0f ? 32767.0f / mx : 0.0f;
    for (uint32_t i = 0; i < hd; i++)
        dst[i] = (int16_t)lrintf(src[i] * inv);
}

/* INT16 (att_wquant_ref, attention.c:158-176): a row of weights (value
   scales folded in, none negative) to 0 .. 32767 with one scale */
static void quant_weights(const float *row, uint32_t nt, int16_t *w16,
                          float *sc)
{
    float mx = 0.0f;
    for (uint32_t t = 0; t < nt; t++)
        if (row[t] > mx)
            mx = row[t];
    float inv = mx > 0.0f ? 32767.0f / mx : 0.0f;
    for (uint32_t t = 0; t < nt; t++)
        w16[t] = (int16_t)lrintf(row[t] * inv);
    *sc = mx / 32767.0f;
}

static int int16_way(const struct orc_attn *A)
{
    return A->int16 && A->kv == ORC_KV_I8 && A->hd % 16 == 0;
}

static void item(struct job *a, uint32_t it, struct scratch *w)
{
    const struct orc_attn *A = a->A;
    uint32_t hd = A->hd, G = a->group, span = a->n_chunks - a->c0;
    uint32_t c = a->c0 + it % span, kvh = it / span;
    uint32_t t0 = c * ORC_CHUNK, t1 = t0 + ORC_CHUNK;
    uint32_t end = last_seen(a, a->n - 1) + 1;
    if (t1 > end)
        t1 = end;
    uint32_t nt = t1 - t0;
    /* a ring's chunk is contiguous too: n_ctx is a multiple of a chunk
       (attention.c:653-657) */
    size_t r0 = (size_t)kvh * A->n_ctx + (A->ring ? t0 % A->n_ctx : t0);
    const int scaled = A->kv == ORC_KV_I8 || A->kv == ORC_KV_I16;
    const float *ks = scaled ? a->ks + r0 : NULL;
    const float *vs = scaled ? a->vs + r0 : NULL;
    /* tokens before jlo see nothing of this chunk (attention.c:662-674) */
    uint32_t jlo = t0 > a->pos0 ? t0 - a->pos0 : 0;
    if (a->last)
        for (jlo = 0; jlo < a->n && a->last[jlo] < t0; jlo++)
            ;
    for (uint32_t j = 0; j < jlo && j < a->n; j++)
        for (uint32_t g = 0; g < G; g++) {
            float *pm = partial(a, kvh, c, j, g);
            pm[0] = -INFINITY;
            pm[1] = 0.0f;
            memset(pm + 2, 0, hd * sizeof(float));
        }
    if (jlo >= a->n)
        return;
    rows_to_f32(A->kv, a->k, r0, nt, hd, w->kf);
    rows_to_f32(A->kv, a->v, r0, nt, hd, w->vf);
    uint32_t ns = (a->n - jlo) * G;
    const int i16 = a->qi != NULL;
    /* scores of every slot (token, group head) */
    for (uint32_t sl = 0; sl < ns; sl++) {
        uint32_t j = jlo + sl / G, g = sl % G;
        size_t h = (size_t)j * A->n_head + (size_t)kvh * G + g;
        float *row = w->sc + (size_t)sl * ORC_CHUNK;
        if (i16) {
            /* an exact integer sum, then three multiplies
               (attention_scores.h:73-81) */
            const int16_t *qv = a->qi + h * hd;
            const int8_t *K = (const int8_t *)a->k + r0 * hd;
            for (uint32_t t = 0; t < nt; t++) {
                int32_t acc = 0;
                for (uint32_t i = 0; i < hd; i++)
                    acc += (int32_t)qv[i] * K[(size_t)t * hd + i];
                row[t] = (float)acc * a->qs[h] * A->scale * ks[t];
            }
            continue;
        }
        const float *qv = a->q + h * hd;
        for (uint32_t t = 0; t < nt; t++) {
            float s = dot8(qv, w->kf + (size_t)t * hd, hd) * A->scale;
            row[t] = scaled ? s * ks[t] : s;
        }
    }
    /* weights, window, value scale (attention.c:732-772) */
    for (uint32_t sl = 0; sl < ns; sl++) {
        uint32_t j = jlo + sl / G;
        uint32_t vis = last_seen(a, j) + 1 - t0;
        float *pm = partial(a, kvh, c, j, sl % G);
        float *row = w->sc + (size_t)sl * ORC_CHUNK;
        if (A->window && a->pos0 + j + 1 > A->window) {
            uint32_t lo = a->pos0 + j + 1 - A->window;
            if (lo >= t1) {
                pm[0] = -INFINITY;
                pm[1] = 0.0f;
                memset(row, 0, nt * sizeof(float));
                continue;
            }
            for (uint32_t t = t0; t < lo; t++)
                row[t - t0] = -INFINITY;
        }
        pm[1] = weights(row, nt, vis < nt ? vis : nt, pm);
        if (scaled)
            for (uint32_t t = 0; t < nt; t++)
                row[t] *= vs[t];
        if (i16)
            quant_weights(row, nt, w->w16 + (size_t)sl * ORC_CHUNK,
                          &w->wsc[sl]);
    }
    if (i16) {
        /* exact integer sums of the int16 weights times the int8 values,
           then one multiply (att_values_i16_ref, attention.c:178-193) */
        const int8_t *V = (const int8_t *)a->v + r0 * hd;
        for (uint32_t sl = 0; sl < ns; sl++) {
            uint32_t j = jlo + sl / G;
            float *acc = partial(a, kvh, c, j, sl % G) + 2;
            if (A->window && a->pos0 + j + 1 > A->window &&
                a->pos0 + j + 1 - A->window >= t1) {
                /* a chunk wholly before the token's window: no weights */
                memset(acc, 0, hd * sizeof(float));
                continue;
            }
            const int16_t *wq = w->w16 + (size_t)sl * ORC_CHUNK;
            for (uint32_t i = 0; i < hd; i++) {
                int32_t s32 = 0;
                for (uint32_t t = 0; t < nt; t++)
                    s32 += (int32_t)wq[t] * V[(size_t)t * hd + i];
                acc[i] = (float)s32 * w->wsc[sl];
            }
        }
        return;
    }
    /* values: position by position, fused (attention.c:431-466) */
    for (uint32_t sl = 0; sl < ns; sl++) {
        const float *row = w->sc + (size_t)sl * ORC_CHUNK;
        float *acc = partial(a, kvh, c, jlo + sl / G, sl % G) + 2;
        for (uint32_t i = 0; i < hd; i++)
            acc[i] = 0.0f;
        for (uint32_t t = 0; t < nt; t++) {
            const float wt = row[t], *vr = w->vf + (size_t)t * hd;
            for (uint32_t i = 0; i < hd; i++)
                acc[i] = fmaf(wt, vr[i], acc[i]);
        }
    }
}

/* merge of token j, query head h (merge_one, attention.c:870-910) */
static void merge(struct job *a, uint32_t j, uint32_t h)
{
    const struct orc_attn *A = a->A;
    uint32_t hd = A->hd, kvh = h / a->group, g = h % a->group;
    uint32_t nc = (last_seen(a, j) + ORC_CHUNK) / ORC_CHUNK;
    float mx = -INFINITY, sum = 0.0f;
    for (uint32_t c = a->c0; c < nc; c++) {
        float m = partial(a, kvh, c, j, g)[0];
        if (m > mx)
            mx = m;
    }
    float *out = a->out + ((size_t)j * A->n_head + h) * hd;
    for (uint32_t i = 0; i < hd; i++)
        out[i] = 0.0f;
    for (uint32_t c = a->c0; c < nc; c++) {
        const float *pm = partial(a, kvh, c, j, g);
        float w = (float)exp((double)(pm[0] - mx));
        float wl = w * pm[1]; /* unfused, as the reference's build */
        sum += wl;
        for (uint32_t i = 0; i < hd; i++)
            out[i] = fmaf(w, pm[2 + i], out[i]);
    }
    float inv = 1.0f / sum;
    for (uint32_t i = 0; i < hd; i++)
        out[i] *= inv;
}

/* ---- threads ---------------------------------------------------------- */

struct worker {
    struct job *a;
    int phase; /* 0 items, 1 merges */
    int ok;
};

static void *work(void *arg)
{
    struct worker *wk = arg;
    struct job *a = wk->a;
    const struct orc_attn *A = a->A;
    uint32_t span = a->n_chunks - a->c0;
    if (wk->phase == 0) {
        struct scratch s;
        size_t rows = (size_t)ORC_CHUNK * A->hd;
        s.kf = malloc(rows * sizeof(float));
        s.vf = malloc(rows * sizeof(float));
        s.sc = malloc((size_t)a->n * a->group * ORC_CHUNK * sizeof(float));
        s.w16 = malloc((size_t)a->n * a->group * ORC_CHUNK * sizeof(int16_t));
        s.wsc = malloc((size_t)a->n * a->group * sizeof(float));
        if (!s.kf || !s.vf || !s.sc || !s.w16 || !s.wsc) {
            wk->ok = 0;
        } else {
            uint32_t items = A->n_kv * span;
            for (;;) {
                uint32_t it = atomic_fetch_add(&a->next, 1);
                if (it >= items)
                    break;
                item(a, it, &s);
            }
        }
        free(s.kf);
        free(s.vf);
        free(s.sc);
        free(s.w16);
        free(s.wsc);
    } else {
        uint32_t items = a->n * A->n_head;
        for (;;) {
            uint32_t it = atomic_fetch_add(&a->next, 1);
            if (it >= items)
                break;
            merge(a, it / A->n_head, it % A->n_head);
        }
    }
    return NULL;
}

static int run_phase(struct job *a, int phase, int n_threads)
{
    struct worker wk[256];
    pthread_t th[256];
    int created[256] = {0};
    if (n_threads > 256)
        n_threads = 256;
    atomic_store(&a->next, 0);
    for (int t = 0; t < n_threads; t++) {
        wk[t].a = a;
        wk[t].phase = phase;
        wk[t].ok = 1;
    }
    /* a thread that cannot start leaves its items to the others */
    for (int t = 1; t < n_threads; t++)
        created[t] = pthread_create(&th[t], NULL, work, &wk[t]) == 0;
    work(&wk[0]);
    int ok = wk[0].ok;
    for (int t = 1; t < n_threads; t++)
        if (created[t]) {
            pthread_join(th[t], NULL);
            ok &= wk[t].ok;
        }
    return ok ? 0 : -1;
}

uint32_t orc_ring_positions(uint32_t window, uint32_t n)
{
    uint32_t need = window + n + ORC_CHUNK;
    return (need + ORC_CHUNK - 1) / ORC_CHUNK * ORC_CHUNK;
}

static int geometry_ok(const struct orc_attn *A)
{
    return A->n_kv && A->n_head % A->n_kv == 0 && A->hd % 8 == 0 &&
           A->hd <= 512 && A->kv >= ORC_KV_I8 && A->kv <= ORC_KV_F32;
}

int orc_attn_run(const struct orc_attn *A, const float *q, const void *k,
                 const float *ks, const void *v, const float *vs, uint32_t n,
                 uint32_t pos0, const uint32_t *last, float *out, int n_threads)
{
    if (!geometry_ok(A) || n == 0 || n_threads < 1)
        return -1;
    struct job a;
    memset(&a, 0, sizeof a);
    a.A = A;
    a.q = q;
    a.k = k;
    a.v = v;
    a.ks = ks;
    a.vs = vs;
    a.last = last;
    a.out = out;
    a.n = n;
    a.pos0 = pos0;
    a.group = A->n_head / A->n_kv;
    uint32_t end = last ? last[n - 1] + 1 : pos0 + n;
    a.n_chunks = (end + ORC_CHUNK - 1) / ORC_CHUNK;
    /* chunks wholly before the first token's window are never read
       (attention.c:1277-1281) */
    a.c0 = A->window && pos0 + 1 > A->window
               ? (pos0 + 1 - A->window) / ORC_CHUNK
               : 0;
    uint32_t span = a.n_chunks - a.c0;
    if (A->ring && span > A->n_ctx / ORC_CHUNK)
        return -1; /* the ring is too small for this call */
    if (!A->ring && end > A->n_ctx)
        return -1;
    a.part = malloc((size_t)A->n_kv * span * n * a.group * (A->hd + 2) *
                    sizeof(float));
    if (!a.part)
        return -1;
    if (int16_way(A)) {
        size_t rows = (size_t)n * A->n_head;
        a.qi = malloc(rows * A->hd * sizeof(int16_t));
        a.qs = malloc(rows * sizeof(float));
        if (!a.qi || !a.qs) {
            free(a.qi);
            free(a.qs);
            free(a.part);
            return -1;
        }
        for (size_t r = 0; r < rows; r++)
            quant_row(q + r * A->hd, A->hd, a.qi + r * A->hd, &a.qs[r]);
    }
    int rc = run_phase(&a, 0, n_threads);
    if (rc == 0)
        rc = run_phase(&a, 1, n_threads);
    free(a.part);
    free(a.qi);
    free(a.qs);
    return rc;
}

void orc_gate(const float *g, int per_head, uint32_t n, uint32_t n_head,
              uint32_t hd, float *out)
{
    size_t total = (size_t)n * n_head * hd;
    for (size_t i = 0; i < total; i++) {
        float x = per_head ? g[i / hd] : g[i];
        float e = (float)exp(-(double)x);
        out[i] *= 1.0f / (1.0f + e);
    }
}

/* ---- the closed form -------------------------------------------------- */

static double elem(int kv, const void *base, size_t idx)
{
    switch (kv) {
    case ORC_KV_I8:
        return ((const int8_t *)base)[idx];
    case ORC_KV_I16:
        return ((const int16_t *)base)[idx];
    case ORC_KV_F16:
        return orc_f16_to_f32(((const uint16_t *)base)[idx]);
    default:
        return ((const float *)base)[idx];
    }
}

int orc_attn_exact(const struct orc_attn *A, const float *q, const void *k,
                   const float *ks, const void *v, const float *vs, uint32_t n,
                   uint32_t pos0, const uint32_t *last, double *out)
{
    if (!geometry_ok(A) || n == 0)
        return -1;
    uint32_t hd = A->hd, G = A->n_head / A->n_kv;
    const int scaled = A->kv == ORC_KV_I8 || A->kv == ORC_KV_I16;
    uint32_t maxend = (last ? last[n - 1] : pos0 + n - 1) + 1;
    double *s = malloc((size_t)maxend * sizeof(double));
    if (!s)
        return -1;
    for (uint32_t j = 0; j < n; j++) {
        uint32_t p = pos0 + j, hi = last ? last[j] : p;
        uint32_t lo = A->window && p + 1 > A->window ? p + 1 - A->window : 0;
        for (uint32_t h = 0; h < A->n_head; h++) {
            const float *qv = q + ((size_t)j * A->n_head + h) * hd;
            uint32_t kvh = h / G;
            double mx = -INFINITY, sum = 0.0;
            double *o = out + ((size_t)j * A->n_head + h) * hd;
            for (uint32_t t = lo; t <= hi; t++) {
                size_t row = (size_t)kvh * A->n_ctx +
                             (A->ring ? t % A->n_ctx : t);
                double d = 0.0;
                for (uint32_t i = 0; i < hd; i++)
                    d += (double)qv[i] * elem(A->kv, k, row * hd + i);
                s[t] = d * (double)A->scale * (scaled ? (double)ks[row] : 1.0);
                if (s[t] > mx)
                    mx = s[t];
            }
            for (uint32_t i = 0; i < hd; i++)
                o[i] = 0.0;
            for (uint32_t t = lo; t <= hi; t++) {
                size_t row = (size_t)kvh * A->n_ctx +
                             (A->ring ? t % A->n_ctx : t);
                double w = exp(s[t] - mx);
                double wv = w * (scaled ? (double)vs[row] : 1.0);
                sum += w;
                for (uint32_t i = 0; i < hd; i++)
                    o[i] += wv * elem(A->kv, v, row * hd + i);
            }
            for (uint32_t i = 0; i < hd; i++)
                o[i] /= sum;
        }
    }
    free(s);
    return 0;
}
