/*
 * attn_cache_api.cpp - Part 3 of include/janas_attn.h: the cache around the
 * attention (write, query preparation, shift, state rows) over the kernels
 * of attn_cache.hip and strided copies.
 */
#include <stdio.h>
#include <string.h>

#include <algorithm>

#include <hip/hip_runtime.h>

#include "../../include/janas_attn.h"
#include "attn_kernels.h"

using namespace janas;

namespace {

int hip_rc(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return JANAS_ATTN_OK;
    fprintf(stderr, "janas_attn: %s: %s\n", what, hipGetErrorString(e));
    return JANAS_ATTN_EDEVICE;
}

size_t elem_size(int kv)
{
    return kv == kI8 ? 1 : kv == kF32 ? 4 : 2;
}

bool scaled(int kv)
{
    return kv == kI8 || kv == kI16;
}

int check_cache(const janas_attn_cache *c)
{
    if (!c || !c->k || !c->v || c->n_kv == 0 || c->cap == 0 ||
        c->head_dim == 0 || c->head_dim > 512 || c->kv_type < kI8 ||
        c->kv_type > kF32)
        return JANAS_ATTN_EINVAL;
    if (scaled(c->kv_type) && (!c->ks || !c->vs))
        return JANAS_ATTN_EINVAL;
    return JANAS_ATTN_OK;
}

/* rows r0 .. r0 + nr - 1 of every KV head between the cache (pitch cap
   rows) and a packed buffer (pitch n rows, at row d0) */
int copy_rows(const janas_attn_cache *c, uint32_t r0, uint32_t nr,
              uint32_t n, uint32_t d0, void *k, void *v, float *ks, float *vs,
              int out, hipStream_t st)
{
    if (nr == 0)
        return JANAS_ATTN_OK;
    const size_t rowb = (size_t)c->head_dim * elem_size(c->kv_type);
    struct Part {
        void *cache, *buf;
        size_t rb;
    } parts[4] = {{c->k, k, rowb}, {c->v, v, rowb}, {c->ks, ks, 4}, {c->vs, vs, 4}};
    const int np = scaled(c->kv_type) ? 4 : 2;
    for (int i = 0; i < np; i++) {
        char *cp = (char *)parts[i].cache + (size_t)r0 * parts[i].rb;
        char *bp = (char *)parts[i].buf + (size_t)d0 * parts[i].rb;
        const size_t cpitch = (size_t)c->cap * parts[i].rb;
        const size_t bpitch = (size_t)n * parts[i].rb;
        const size_t width = (size_t)nr * parts[i].rb;
        hipError_t e = out ? hipMemcpy2DAsync(bp, bpitch, cp, cpitch, width, c->n_kv,
                                              hipMemcpyDefault, st)
                           : hipMemcpy2DAsync(cp, cpitch, bp, bpitch, width, c->n_kv,
                                              hipMemcpyDefault, st);
        if (e != hipSuccess)
            return hip_rc(e, "cache rows copy");
    }
    return JANAS_ATTN_OK;
}

}  // namespace

extern "C" int janas_attn_cache_write(const struct janas_attn_cache *c,
                                      const float *k, const float *v,
                                      const float *k_norm, float eps,
                                      const float *cs, const float *sn,
                                      uint32_t n_rot, int v_norm,
                                      uint32_t pos0, uint32_t n, void *stream)
{
    int rc = check_cache(c);
    if (rc)
        return rc;
    if (!k || !v || (n_rot && (!cs || !sn)) || n_rot % 2 || n_rot > c->head_dim)
        return JANAS_ATTN_EINVAL;
    if (n == 0)
        return JANAS_ATTN_OK;
    if (!c->ring && (uint64_t)pos0 + n > c->cap)
        return JANAS_ATTN_ERANGE;
    RowArgs a;
    memset(&a, 0, sizeof a);
    a.k = const_cast<float *>(k); /* read only: the cache is written */
    a.v = v;
    a.norm = k_norm;
    a.cs = cs;
    a.sn = sn;
    a.kc = c->k;
    a.vc = c->v;
    a.kz = c->ks;
    a.vz = c->vs;
    a.eps = eps;
    a.n = n;
    a.heads = c->n_kv;
    a.hd = c->head_dim;
    a.n_rot = n_rot;
    a.pos0 = pos0;
    a.cap = c->cap;
    a.kv = c->kv_type;
    a.ring = c->ring != 0;
    a.v_norm = v_norm != 0;
    return hip_rc(launch_rows(a, (hipStream_t)stream), "cache write launch");
}

extern "C" int janas_attn_q_prep(float *q, const float *q_norm, float eps,
                                 const float *cs, const float *sn,
                                 uint32_t n_rot, uint32_t n, uint32_t n_head,
                                 uint32_t head_dim, void *stream)
{
    if (!q || (n_rot && (!cs || !sn)) || n_head == 0 || head_dim == 0 ||
        head_dim > 512 || n_rot % 2 || n_rot > head_dim)
        return JANAS_ATTN_EINVAL;
    if (n == 0)
        return JANAS_ATTN_OK;
    RowArgs a;
    memset(&a, 0, sizeof a);
    a.k = q;
    a.norm = q_norm;
    a.cs = cs;
    a.sn = sn;
    a.eps = eps;
    a.n = n;
    a.heads = n_head;
    a.hd = head_dim;
    a.n_rot = n_rot;
    return hip_rc(launch_rows(a, (hipStream_t)stream), "query launch");
}

extern "C" int janas_attn_cache_shift(const struct janas_attn_cache *c,
                                      uint32_t keep, uint32_t drop,
                                      uint32_t n_pos, const float *cs,
                                      const float *sn, uint32_t n_rot,
                                      void *stream)
{
    int rc = check_cache(c);
    if (rc)
        return rc;
    if (!scaled(c->kv_type))
        return JANAS_ATTN_ENOTSUP;
    /* model.c:304-305 */
    if (drop == 0 || (uint64_t)keep + drop > n_pos || n_rot % 2 ||
        n_rot > c->head_dim || (n_rot && (!cs || !sn)))
        return JANAS_ATTN_EINVAL;
    if (!c->ring && n_pos > c->cap)
        return JANAS_ATTN_ERANGE;
    hipStream_t st = (hipStream_t)stream;
    ShiftArgs a;
    memset(&a, 0, sizeof a);
    a.k = c->k;
    a.v = c->v;
    a.kz = c->ks;
    a.vz = c->vs;
    a.cs = cs;
    a.sn = sn;
    a.n_kv = c->n_kv;
    a.hd = c->head_dim;
    a.cap = c->cap;
    a.n_rot = n_rot;
    a.drop = drop;
    a.kv = c->kv_type;
    a.ring = c->ring != 0;
    if (!c->ring) {
        /* model.c:345-356: the moved rows, read from a copy of them */
        a.first = a.copy_first = keep + drop;
        a.count = a.copy_rows = n_pos - keep - drop;
    } else {
        /* model.c:358-375: the positions the ring still has, from a copy
           of all of it */
        uint32_t lo = keep + drop;
        if (n_pos > c->cap && n_pos - c->cap > lo)
            lo = n_pos - c->cap;
        a.first = lo;
        a.count = n_pos - lo;
        a.copy_first = 0;
        a.copy_rows = c->cap;
    }
    if (a.count == 0)
        return JANAS_ATTN_OK;
    const size_t rowb = (size_t)c->head_dim * elem_size(c->kv_type);
    const size_t kvb = (size_t)c->n_kv * a.copy_rows * rowb;
    const size_t zb = (size_t)c->n_kv * a.copy_rows * sizeof(float);
    char *tmp = nullptr;
    if (hipMalloc(&tmp, 2 * kvb + 2 * zb) != hipSuccess) {
        (void)hipGetLastError();
        return JANAS_ATTN_ENOMEM;
    }
    a.ck = tmp;
    a.cv = tmp + kvb;
    a.ckz = (const float *)(tmp + 2 * kvb);
    a.cvz = (const float *)(tmp + 2 * kvb + zb);
    rc = copy_rows(c, a.copy_first, a.copy_rows, a.copy_rows, 0, tmp, tmp + kvb,
                   (float *)(tmp + 2 * kvb), (float *)(tmp + 2 * kvb + zb), 1, st);
    if (!rc)
        rc = hip_rc(launch_shift(a, st), "shift launch");
    hipError_t e = hipStreamSynchronize(st);
    (void)hipFree(tmp);
    if (!rc && e != hipSuccess)
        rc = hip_rc(e, "shift");
    return rc;
}

extern "C" int janas_attn_cache_copy(const struct janas_attn_cache *c,
                                     uint32_t n_pos, uint32_t rows, void *k,
                                     void *v, float *ks, float *vs, int out,
                                     void *stream)
{
    int rc = check_cache(c);
    if (rc)
        return rc;
    if (!k || !v || (scaled(c->kv_type) && (!ks || !vs)) || rows > n_pos)
        return JANAS_ATTN_EINVAL;
    if (rows > c->cap || (!c->ring && n_pos > c->cap))
        return JANAS_ATTN_ERANGE;
    if (rows == 0)
        return JANAS_ATTN_OK;
    hipStream_t st = (hipStream_t)stream;
    if (!c->ring)
        return copy_rows(c, 0, rows, rows, 0, k, v, ks, vs, out, st);
    /* model_state.c:184-199: positions n_pos - rows .. n_pos - 1 at rows
       p mod cap - at most two runs */
    const uint32_t start = (n_pos - rows) % c->cap;
    const uint32_t len1 = std::min(rows, c->cap - start);
    rc = copy_rows(c, start, len1, rows, 0, k, v, ks, vs, out, st);
    if (!rc && rows > len1)
        rc = copy_rows(c, 0, rows - len1, rows, len1, k, v, ks, vs, out, st);
    return rc;
}
