/*
 * Device-resident tensors (the reference's core/tensor.c:21-427 data model
 * with storage in HBM).  Elements live in a refcounted device block
 * (pg_data_ref); `data` is a host mirror filled on demand.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <assert.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

size_t pg_shape_numel(size_t ndim, const size_t *shape)
{
    size_t n = 1;
    for (size_t i = 0; i < ndim; i++)
        n *= shape[i];
    return n;
}

bool pg_shape_equal(size_t na, const size_t *sa, size_t nb, const size_t *sb)
{
    if (na != nb)
        return false;
    for (size_t i = 0; i < na; i++)
        if (sa[i] != sb[i])
            return false;
    return true;
}

void pgt_set_contig_strides(pg_tensor *t)
{
    size_t acc = 1;
    for (size_t i = t->ndim; i-- > 0;) {
        t->stride[i] = acc;
        acc *= t->shape[i];
    }
}

bool pgt_is_contiguous(const pg_tensor *t)
{
    size_t acc = 1;
    for (size_t i = t->ndim; i-- > 0;) {
        if (t->shape[i] != 1 && t->stride[i] != acc)
            return false;
        acc *= t->shape[i];
    }
    return true;
}

pg_tensor *pgt_alloc(pg_dtype dtype, size_t ndim, const size_t *shape)
{
    if (ndim > PG_MAX_NDIM || (ndim && !shape) || !pg_dtype_is_float(dtype))
        return NULL;
    pg_tensor *t = calloc(1, sizeof *t);
    pg_data_ref *r = calloc(1, sizeof *r);
    if (!t || !r) {
        free(t);
        free(r);
        return NULL;
    }
    t->ndim = ndim;
    for (size_t i = 0; i < ndim; i++)
        t->shape[i] = shape[i];
    pgt_set_contig_strides(t);
    t->numel = pg_shape_numel(ndim, shape);
    t->dtype = dtype;
    t->elem_size = pg_dtype_size(dtype);
    r->nbytes = t->numel * t->elem_size;
    r->ptr = pgd_malloc(r->nbytes ? r->nbytes : 1);
    if (!r->ptr) {
        free(t);
        free(r);
        return NULL;
    }
    r->refs = 1;
    t->data_ref = r;
    t->dev = r->ptr;
    return t;
}

void pgt_narrow_release(pg_data_ref *r)
{
    pg_narrow_pending *p = r ? r->narrow : NULL;
    if (!p)
        return;
    r->narrow = NULL;
    for (int i = 0; i < 2; i++) {
        if (p->own[i])
            pgd_free(p->own[i], p->own_bytes[i]);
        pgt_ref_release(p->hold[i]);
    }
    free(p);
}

void pgt_ref_release(pg_data_ref *r)
{
    if (r && --r->refs == 0) {
        pgt_narrow_release(r);
        pgd_free(r->ptr, r->nbytes);
        if (r->shadow)
            pgd_free(r->shadow, r->shadow_bytes);
        pgt_ref_release(r->act_src_ref);
        free(r);
    }
}

void pg_tensor_free(pg_tensor *t)
{
    if (!t)
        return;
    pgt_ref_release(t->data_ref);
    free(t->data_raw);
    free(t);
}

static bool fill_value(pg_tensor *t, float v)
{
    if (!t->numel)
        return true;
    if (t->dtype == PG_DTYPE_F32)
        return pgd_check(pgk_fill_f32((float *)t->dev, t->numel, v, pgd_stream()), "fill");
    uint16_t h;
    if (t->dtype == PG_DTYPE_BF16) {
        uint32_t x;
        memcpy(&x, &v, 4);
        h = (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
    } else {
        /* f16 of a fill constant: let the device cast kernel round it */
        float *tmp = pgd_malloc(4);
        uint16_t *th = pgd_malloc(2);
        if (!tmp || !th)
            return false;
        pgk_fill_f32(tmp, 1, v, pgd_stream());
        pgk_cast_to16(PG_DTYPE_F16, tmp, th, 1, pgd_stream());
        pgd_d2h(&h, th, 2);
        pgd_free(tmp, 4);
        pgd_free(th, 2);
    }
    return pgd_check(pgk_fill_u16((uint16_t *)t->dev, t->numel, h, pgd_stream()), "fill");
}

bool pgt_settle(const pg_tensor *t)
{
    pg_data_ref *r = t ? t->data_ref : NULL;
    if (!r)
        return true;
    bool ok = true;
    if (r->narrow) {
        /* the narrow product with the arithmetic of the fused pass */
        const pg_narrow_pending *p = r->narrow;
        r->shadow_stale = true;
        ok = pgd_check(pgk_act_bwd16n(0, p->dn, p->wn, p->kw, p->dtype, NULL, (float *)r->ptr, NULL, p->m, p->n,
                                      NULL, (p->n + 7) & ~(size_t)7, 0, NULL, 0, NULL, NULL, NULL, pgd_stream()),
                       "pending narrow product");
        pgt_narrow_release(r);
    }
    if (r->act_pending) {
        /* the elements act(src), with the GEMM epilogue's arithmetic (the
         * unary kernel's ReLU and GELU are the same expressions); the 16-bit
         * copy the epilogue wrote stays current */
        const int op = r->act_pending == PGK_ACT_RELU ? PGK_RELU : PGK_GELU;
        r->act_pending = 0;
        ok = pgd_check(pgk_unary_f32(op, r->act_src, (float *)r->ptr, r->nbytes / 4, 0.0f, 0.0f, pgd_stream()),
                       "pending activation");
        pgt_ref_release(r->act_src_ref);
        r->act_src_ref = NULL;
        r->act_src = NULL;
    }
    if (!r->clip_pending)
        return ok;
    r->clip_pending = false;
    r->shadow_stale = true;
    const pgk_grad_seg seg = {(float *)r->ptr, r->nbytes / 4};
    return pgd_check(pgk_grad_scale_const(&seg, 1, r->clip_mul, r->clip_inv, pgd_stream()), "clip scale") && ok;
}

void pgt_drop_clip(const pg_tensor *t)
{
    pg_data_ref *r = t ? t->data_ref : NULL;
    if (!r)
        return;
    r->clip_pending = false;
    pgt_narrow_release(r);
    if (r->act_pending) {
        r->act_pending = 0;
        pgt_ref_release(r->act_src_ref);
        r->act_src_ref = NULL;
        r->act_src = NULL;
    }
}

void pgt_overwrite(const pg_tensor *t)
{
    if (!t || !t->data_ref || !(t->data_ref->clip_pending || t->data_ref->act_pending || t->data_ref->narrow))
        return;
    /* every element of t is about to be written: a pending clip scale of
     * the whole storage is dropped, of a larger storage applied first */
    if (t->dev == t->data_ref->ptr && t->numel * t->elem_size == t->data_ref->nbytes)
        pgt_drop_clip(t);
    else
        pgt_settle(t);
}

void pgt_materialize(pg_tensor *t)
{
    pgt_settle(t);
    if (t && (t->pg_flags & PG_TENSOR_ZERO_PENDING)) {
        fill_value(t, 0.0f);
        t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
    }
}

pg_tensor *pg_tensor_new_dtype(pg_dtype dtype, size_t ndim, const size_t *shape)
{
    return pg_tensor_zeros_dtype(dtype, ndim, shape);
}

pg_tensor *pg_tensor_empty_dtype(pg_dtype dtype, size_t ndim, const size_t *shape)
{
    return pgt_alloc(dtype, ndim, shape);
}

pg_tensor *pg_tensor_full_dtype(pg_dtype dtype, size_t ndim, const size_t *shape, float value)
{
    pg_tensor *t = pgt_alloc(dtype, ndim, shape);
    if (t && !fill_value(t, value)) {
        pg_tensor_free(t);
        return NULL;
    }
    return t;
}

pg_tensor *pg_tensor_zeros_dtype(pg_dtype dtype, size_t ndim, const size_t *shape)
{
    return pg_tensor_full_dtype(dtype, ndim, shape, 0.0f);
}

pg_tensor *pg_tensor_ones_dtype(pg_dtype dtype, size_t ndim, const size_t *shape)
{
    return pg_tensor_full_dtype(dtype, ndim, shape, 1.0f);
}

pg_tensor *pg_tensor_from_data_dtype(pg_dtype dtype, size_t ndim, const size_t *shape,
                                     const void *data)
{
    pg_tensor *t = pgt_alloc(dtype, ndim, shape);
    if (!t)
        return NULL;
    if (data && !pgd_h2d(t->dev, data, t->numel * t->elem_size)) {
        pg_tensor_free(t);
        return NULL;
    }
    return t;
}

pg_tensor *pg_tensor_new(size_t ndim, const size_t *shape) { return pg_tensor_zeros(ndim, shape); }
pg_tensor *pg_tensor_empty(size_t ndim, const size_t *shape) { return pgt_alloc(PG_DTYPE_F32, ndim, shape); }
pg_tensor *pg_tensor_zeros(size_t ndim, const size_t *shape) { return pg_tensor_full(ndim, shape, 0.0f); }
pg_tensor *pg_tensor_ones(size_t ndim, const size_t *shape) { return pg_tensor_full(ndim, shape, 1.0f); }

pg_tensor *pg_tensor_full(size_t ndim, const size_t *shape, float value)
{
    return pg_tensor_full_dtype(PG_DTYPE_F32, ndim, shape, value);
}

pg_tensor *pg_tensor_from_data(size_t ndim, const size_t *shape, const float *data)
{
    return pg_tensor_from_data_dtype(PG_DTYPE_F32, ndim, shape, data);
}

/* ---- RNG: the reference's splitmix64 stream (tensor.c:289-339) ---- */

static unsigned long long g_rng = 0x9E3779B97F4A7C15ULL;

void pg_seed(unsigned long long seed) { g_rng = seed ? seed : 0x9E3779B97F4A7C15ULL; }

static unsigned long long rng_next(void)
{
    g_rng += 0x9E3779B97F4A7C15ULL;
    unsigned long long z = g_rng;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static float rng_u01(void) { return (float)(rng_next() >> 40) * (1.0f / 16777216.0f); }

void pg_rng_uniform_host(float *out, size_t n, float low, float high)
{
    for (size_t i = 0; i < n; i++)
        out[i] = low + rng_u01() * (high - low);
}

void pg_rng_normal_host(float *out, size_t n, float mean, float stddev)
{
    for (size_t i = 0; i < n; i++) {
        float u1 = rng_u01(), u2 = rng_u01();
        if (u1 < 1e-12f)
            u1 = 1e-12f;
        /* Box-Muller, cosine branch (tensor.c:325-339).  The product is
         * formed as (stddev * cos) * radius: the order the reference's
         * -ffast-math build evaluates it in, so seeded draws agree bit for
         * bit with the reference for any stddev. */
        float radius = sqrtf(-2.0f * logf(u1));
        float c = cosf(2.0f * 3.14159265358979f * u2);
        out[i] = mean + (stddev * c) * radius;
    }
}

static pg_tensor *from_host_gen(size_t ndim, const size_t *shape, int normal, float p, float q)
{
    size_t n = pg_shape_numel(ndim, shape);
    float *h = malloc((n ? n : 1) * sizeof(float));
    if (!h)
        return NULL;
    if (normal)
        pg_rng_normal_host(h, n, p, q);
    else
        pg_rng_uniform_host(h, n, p, q);
    pg_tensor *t = pg_tensor_from_data(ndim, shape, h);
    free(h);
    return t;
}

pg_tensor *pg_tensor_uniform(size_t ndim, const size_t *shape, float low, float high)
{
    return from_host_gen(ndim, shape, 0, low, high);
}

pg_tensor *pg_tensor_normal(size_t ndim, const size_t *shape, float mean, float stddev)
{
    return from_host_gen(ndim, shape, 1, mean, stddev);
}

void pgt_touch(pg_tensor *t)
{
    if (t && t->data_ref)
        t->data_ref->shadow_stale = true;
}

void pg_amd_tensor_modified(pg_tensor *t) { pgt_touch(t); }

pg_tensor *pg_amd_tensor_to_dtype(const pg_tensor *t, pg_dtype dtype)
{
    if (!t || !pg_dtype_is_float(dtype)) {
        pgd_set_err("pg_amd_tensor_to_dtype: null tensor or unknown dtype");
        return NULL;
    }
    if (t->dtype == dtype)
        return pg_tensor_clone(t);
    pgt_settle(t);
    pg_tensor *own;
    const pg_tensor *src = pgt_contiguous(t, &own);
    if (!src)
        return NULL;
    pg_tensor *y = pgt_alloc(dtype, t->ndim, t->shape);
    bool ok = y != NULL;
    if (ok && (t->pg_flags & PG_TENSOR_ZERO_PENDING)) {
        ok = fill_value(y, 0.0f);
    } else if (ok && t->dtype == PG_DTYPE_F32) {
        ok = pgd_check(pgk_cast_to16((int)dtype, src->dev, y->dev, t->numel, pgd_stream()), "pg_amd_tensor_to_dtype");
    } else if (ok && dtype == PG_DTYPE_F32) {
        ok = pgd_check(pgk_cast_from16((int)t->dtype, src->dev, y->dev, t->numel, pgd_stream()),
                       "pg_amd_tensor_to_dtype");
    } else if (ok) {
        /* f16 <-> bf16 through f32 (the widening is exact) */
        float *tmp = pgd_malloc(t->numel * 4 ? t->numel * 4 : 1);
        ok = tmp && pgd_check(pgk_cast_from16((int)t->dtype, src->dev, tmp, t->numel, pgd_stream()),
                              "pg_amd_tensor_to_dtype") &&
             pgd_check(pgk_cast_to16((int)dtype, tmp, y->dev, t->numel, pgd_stream()), "pg_amd_tensor_to_dtype");
        if (tmp)
            pgd_free(tmp, t->numel * 4);
    }
    pg_tensor_free(own);
    if (!ok) {
        pg_tensor_free(y);
        return NULL;
    }
    return y;
}

bool pg_amd_tensor_refresh16(pg_tensor *t)
{
    if (!t || !t->data_ref)
        return false;
    pg_data_ref *r = t->data_ref;
    if (!r->shadow || !r->shadow_stale)
        return true;
    if (r->shadow_cols)
        return pgt_shadow16_rows(t, (pg_dtype)r->shadow_dtype, r->shadow_cols, r->shadow_ld) != NULL;
    return pgt_shadow16(t, (pg_dtype)r->shadow_dtype) != NULL;
}

static void shadow_drop(pg_data_ref *r)
{
    if (r->shadow)
        pgd_free(r->shadow, r->shadow_bytes);
    r->shadow = NULL;
    r->shadow_bytes = 0;
    r->shadow_cols = r->shadow_ld = 0;
}

const uint16_t *pgt_shadow16(pg_tensor *t, pg_dtype dt)
{
    if (!t || !t->data_ref || t->dtype != PG_DTYPE_F32 || (dt != PG_DTYPE_F16 && dt != PG_DTYPE_BF16)) {
        pgd_set_err("shadow16: needs an f32 tensor and a 16-bit dtype");
        return NULL;
    }
    pg_data_ref *r = t->data_ref;
    size_t n = r->nbytes / 4;
    if (r->shadow && r->shadow_cols)
        shadow_drop(r); /* a pitched copy: remade in storage order */
    if (r->shadow && r->shadow_dtype == (int)dt && !r->shadow_stale)
        return r->shadow;
    if (!r->shadow) {
        const size_t bytes = n ? n * 2 : 1;
        r->shadow = pgd_malloc(bytes);
        if (!r->shadow)
            return NULL;
        r->shadow_bytes = bytes;
    }
    r->shadow_dtype = (int)dt;
    /* elements still pending in a deferred forward run: its fused kernel
     * writes the copy beside them, in place of a pass over them */
    if (t->dev == r->ptr && t->numel == n && pga_lazy_shadow16(t, (int)dt, r->shadow)) {
        r->shadow_stale = false;
        return r->shadow;
    }
    pgt_materialize(t);
    if (!pgd_check(pgk_cast_to16((int)dt, r->ptr, r->shadow, n, pgd_stream()), "shadow16"))
        return NULL;
    r->shadow_stale = false;
    return r->shadow;
}

const uint16_t *pgt_shadow16_fresh(const pg_tensor *t, pg_dtype dt)
{
    const pg_data_ref *r = t ? t->data_ref : NULL;
    if (!r || !r->shadow || r->shadow_stale || r->shadow_dtype != (int)dt || r->shadow_cols || t->dev != r->ptr ||
        t->numel * 4 != r->nbytes || (t->pg_flags & PG_TENSOR_ZERO_PENDING) || r->narrow || r->act_pending ||
        r->clip_pending)
        return NULL;
    return r->shadow;
}

uint16_t *pgt_shadow16_target(pg_tensor *t, pg_dtype dt)
{
    if (!t || !t->data_ref || t->dtype != PG_DTYPE_F32 || (dt != PG_DTYPE_F16 && dt != PG_DTYPE_BF16) ||
        t->dev != t->data_ref->ptr || t->numel * 4 != t->data_ref->nbytes)
        return NULL;
    pg_data_ref *r = t->data_ref;
    if (r->shadow && r->shadow_cols)
        shadow_drop(r);
    if (!r->shadow) {
        const size_t bytes = t->numel ? t->numel * 2 : 1;
        r->shadow = pgd_malloc(bytes);
        if (!r->shadow)
            return NULL;
        r->shadow_bytes = bytes;
    }
    r->shadow_dtype = (int)dt;
    r->shadow_stale = true; /* until the writer's launch is queued */
    return r->shadow;
}

const uint16_t *pgt_shadow16_rows(pg_tensor *t, pg_dtype dt, size_t cols, size_t ld)
{
    if (ld == cols)
        return pgt_shadow16(t, dt);
    if (!t || !t->data_ref || t->dtype != PG_DTYPE_F32 || (dt != PG_DTYPE_F16 && dt != PG_DTYPE_BF16) || !cols ||
        ld < cols || (t->data_ref->nbytes / 4) % cols) {
        pgd_set_err("shadow16: needs an f32 tensor of whole rows and a 16-bit dtype");
        return NULL;
    }
    pg_data_ref *r = t->data_ref;
    if (r->shadow && (r->shadow_cols != cols || r->shadow_ld != ld))
        shadow_drop(r);
    if (r->shadow && r->shadow_dtype == (int)dt && !r->shadow_stale)
        return r->shadow;
    const size_t rows = r->nbytes / 4 / cols;
    if (!r->shadow) {
        const size_t bytes = rows * ld ? rows * ld * 2 : 1;
        r->shadow = pgd_malloc(bytes);
        if (!r->shadow)
            return NULL;
        r->shadow_bytes = bytes;
        r->shadow_cols = cols;
        r->shadow_ld = ld;
    }
    r->shadow_dtype = (int)dt;
    pgt_materialize(t);
    /* the pad columns are written as zeros here and never touched again */
    if (!pgd_check(pgk_copy_to16((int)dt, 0, r->ptr, rows, cols, cols, r->shadow, ld, rows, 1, 0, 0, pgd_stream()),
                   "shadow16"))
        return NULL;
    r->shadow_stale = false;
    return r->shadow;
}

pg_tensor *pg_tensor_clone(const pg_tensor *t)
{
    if (!t)
        return NULL;
    pg_tensor *c = pgt_alloc(t->dtype, t->ndim, t->shape);
    if (!c)
        return NULL;
    if (t->pg_flags & PG_TENSOR_ZERO_PENDING) {
        fill_value(c, 0.0f);
        return c;
    }
    pgt_settle(t);
    if (!pgt_is_contiguous(t)) {
        /* a strided view: its elements in row-major order */
        if (!pgd_check(pgk_gather_strided(t->elem_size, t->dev, c->dev, (int)t->ndim, t->shape, t->stride,
                                          pgd_stream()),
                       "pg_tensor_clone")) {
            pg_tensor_free(c);
            return NULL;
        }
        return c;
    }
    pgd_d2d(c->dev, t->dev, t->numel * t->elem_size);
    return c;
}

const pg_tensor *pgt_contiguous(const pg_tensor *t, pg_tensor **owned)
{
    *owned = NULL;
    if (!t)
        return NULL;
    if (pgt_is_contiguous(t))
        return t;
    *owned = pg_tensor_clone(t);
    return *owned;
}

void pg_tensor_fill(pg_tensor *t, float value)
{
    if (!t)
        return;
    t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
    pgt_overwrite(t);
    pgt_touch(t);
    fill_value(t, value);
}

void pg_tensor_copy_from(pg_tensor *dst, const pg_tensor *src)
{
    if (!dst || !src || dst->numel != src->numel || dst->dtype != src->dtype)
        return;
    if (src->pg_flags & PG_TENSOR_ZERO_PENDING) {
        pg_tensor_fill(dst, 0.0f);
        return;
    }
    pgt_settle(src);
    pgt_overwrite(dst);
    dst->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
    pgt_touch(dst);
    pgd_d2d(dst->dev, src->dev, src->numel * src->elem_size);
}

bool pg_tensor_reshape(pg_tensor *t, size_t ndim, const size_t *shape)
{
    if (!t || ndim > PG_MAX_NDIM || pg_shape_numel(ndim, shape) != t->numel || !pgt_is_contiguous(t))
        return false;
    t->ndim = ndim;
    for (size_t i = 0; i < ndim; i++)
        t->shape[i] = shape[i];
    pgt_set_contig_strides(t);
    return true;
}

pg_tensor *pg_tensor_view(const pg_tensor *src)
{
    if (!src || !src->data_ref)
        return NULL;
    pg_tensor *v = calloc(1, sizeof *v);
    if (!v)
        return NULL;
    v->ndim = src->ndim;
    memcpy(v->shape, src->shape, sizeof v->shape);
    memcpy(v->stride, src->stride, sizeof v->stride);
    v->numel = src->numel;
    v->dtype = src->dtype;
    v->elem_size = src->elem_size;
    v->data_ref = src->data_ref;
    v->data_ref->refs++;
    v->dev = src->dev;
    v->is_view = true;
    v->view_parent = (pg_tensor *)src;
    v->pg_flags = src->pg_flags;
    return v;
}

/* tensor.c:575-595: shape and strides permuted, storage shared */
pg_tensor *pg_tensor_permute_view(const pg_tensor *src, const size_t *order)
{
    if (!src || !order)
        return NULL;
    bool seen[PG_MAX_NDIM] = {0};
    for (size_t i = 0; i < src->ndim; i++) {
        if (order[i] >= src->ndim || seen[order[i]])
            return NULL;
        seen[order[i]] = true;
    }
    pg_tensor *v = pg_tensor_view(src);
    if (!v)
        return NULL;
    for (size_t i = 0; i < src->ndim; i++) {
        v->shape[i] = src->shape[order[i]];
        v->stride[i] = src->stride[order[i]];
    }
    return v;
}

pg_tensor *pg_tensor_reshape_view(const pg_tensor *src, size_t ndim, const size_t *shape)
{
    if (!src || ndim > PG_MAX_NDIM || pg_shape_numel(ndim, shape) != src->numel ||
        !pgt_is_contiguous(src))
        return NULL;
    pg_tensor *v = calloc(1, sizeof *v);
    if (!v)
        return NULL;
    v->ndim = ndim;
    for (size_t i = 0; i < ndim; i++)
        v->shape[i] = shape[i];
    pgt_set_contig_strides(v);
    v->numel = src->numel;
    v->dtype = src->dtype;
    v->elem_size = src->elem_size;
    v->data_ref = src->data_ref;
    v->data_ref->refs++;
    v->dev = src->dev;
    v->is_view = true;
    v->view_parent = (pg_tensor *)src;
    v->pg_flags = src->pg_flags;
    return v;
}

bool pg_tensor_copy_to_host(const pg_tensor *t, void *dst)
{
    if (!t || !dst)
        return false;
    size_t nb = t->numel * t->elem_size;
    if (t->pg_flags & PG_TENSOR_ZERO_PENDING) {
        if (!pgd_sync())
            return false;
        memset(dst, 0, nb);
        return true;
    }
    pgt_settle(t);
    return pgd_d2h(dst, t->dev, nb);
}

bool pg_tensor_copy_from_host(pg_tensor *t, const void *src)
{
    if (!t || !src)
        return false;
    t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
    pgt_overwrite(t);
    pgt_touch(t);
    return pgd_h2d(t->dev, src, t->numel * t->elem_size);
}

bool pg_tensor_sync_host(pg_tensor *t)
{
    if (!t)
        return false;
    size_t nb = t->numel * t->elem_size;
    if (!t->data_raw) {
        t->data_raw = malloc(nb ? nb : 1);
        if (!t->data_raw)
            return false;
    }
    return pg_tensor_copy_to_host(t, t->data_raw);
}

bool pg_tensor_sync_device(pg_tensor *t)
{
    if (!t || !t->data_raw)
        return false;
    return pg_tensor_copy_from_host(t, t->data_raw);
}

/* ---- host-side helpers of the reference's tensor utilities ---- */

/* IEEE round-to-nearest-even f32 -> f16 (the device cast's rounding) */
static uint16_t host_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
    if (ex == 255)
        return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    int32_t e = (int32_t)ex - 112;
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t sh = (uint32_t)(14 - e), keep = man >> sh, rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (keep & 1u)))
            keep++;
        return (uint16_t)(sign | keep);
    }
    uint32_t r = man + 0xFFFu + ((man >> 13) & 1u);
    if (r & 0x800000u) {
        r = 0;
        e++;
    }
    return e >= 31 ? (uint16_t)(sign | 0x7C00u) : (uint16_t)(sign | ((uint32_t)e << 10) | (r >> 13));
}

static float host_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, ex = ((uint32_t)h >> 10) & 0x1Fu, man = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (ex == 0 && man == 0) {
        bits = sign;
    } else if (ex == 0) {
        int32_t e = 1;
        while (!(man & 0x400u)) {
            man <<= 1;
            e--;
        }
        bits = sign | ((uint32_t)(e + 112) << 23) | ((man & 0x3FFu) << 13);
    } else {
        bits = sign | (ex == 31 ? 0x7F800000u : (ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static float host_elem(const pg_tensor *t, const void *p)
{
    if (t->dtype == PG_DTYPE_F32) {
        float f;
        memcpy(&f, p, 4);
        return f;
    }
    uint16_t h;
    memcpy(&h, p, 2);
    if (t->dtype == PG_DTYPE_F16)
        return host_f16_to_f32(h);
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* t's elements in row-major order in a malloc'd host buffer (waits) */
static void *host_copy(const pg_tensor *t)
{
    pg_tensor *own;
    const pg_tensor *c = pgt_contiguous(t, &own);
    if (!c)
        return NULL;
    size_t nb = t->numel * t->elem_size;
    void *h = malloc(nb ? nb : 1);
    if (h && !pg_tensor_copy_to_host(c, h)) {
        free(h);
        h = NULL;
    }
    pg_tensor_free(own);
    return h;
}

static pg_tensor *from_host_f32(size_t n, const float *v)
{
    return pg_tensor_from_data(1, &n, v);
}

/* tensor.c:276-287: n = ceil((stop - start) / step) elements start + step*i */
pg_tensor *pg_tensor_arange(float start, float stop, float step)
{
    if (step <= 0.0f || stop <= start)
        return NULL;
    size_t n = (size_t)ceilf((stop - start) / step);
    float *v = malloc((n ? n : 1) * sizeof *v);
    if (!v)
        return NULL;
    for (size_t i = 0; i < n; i++)
        v[i] = start + step * (float)i;
    pg_tensor *t = from_host_f32(n, v);
    free(v);
    return t;
}

/* tensor.c:341-357: num points, the last exactly stop */
pg_tensor *pg_tensor_linspace(float start, float stop, size_t num)
{
    if (num == 0)
        return NULL;
    float *v = malloc(num * sizeof *v);
    if (!v)
        return NULL;
    if (num == 1) {
        v[0] = start;
    } else {
        float step = (stop - start) / (float)(num - 1);
        for (size_t i = 0; i + 1 < num; i++)
            v[i] = start + step * (float)i;
        v[num - 1] = stop;
    }
    pg_tensor *t = from_host_f32(num, v);
    free(v);
    return t;
}

/* tensor.c:359-371 */
pg_tensor *pg_tensor_eye(size_t n)
{
    if (n == 0)
        return NULL;
    size_t shape[2] = {n, n};
    float *v = calloc(n * n, sizeof *v);
    if (!v)
        return NULL;
    for (size_t i = 0; i < n; i++)
        v[i * n + i] = 1.0f;
    pg_tensor *t = pg_tensor_from_data(2, shape, v);
    free(v);
    return t;
}

static size_t flat_offset(const pg_tensor *t, const size_t *idx)
{
    size_t off = 0;
    for (size_t i = 0; i < t->ndim; i++) {
        assert(idx[i] < t->shape[i]);
        off += idx[i] * t->stride[i];
    }
    return off;
}

/* tensor.c:390-398: one element, waiting for the queued work that writes it */
float pg_tensor_get(const pg_tensor *t, const size_t *idx)
{
    assert(t && idx);
    if (t->pg_flags & PG_TENSOR_ZERO_PENDING)
        return 0.0f;
    pgt_settle(t);
    unsigned char b[4] = {0};
    if (!pgd_d2h(b, (const char *)t->dev + flat_offset(t, idx) * t->elem_size, t->elem_size))
        return 0.0f;
    return host_elem(t, b);
}

/* tensor.c:400-407: one element written (rounded to nearest even for
 * f16/bf16), queued on the stream */
void pg_tensor_set(pg_tensor *t, const size_t *idx, float value)
{
    assert(t && idx);
    pgt_materialize(t);
    pgt_touch(t);
    size_t off = flat_offset(t, idx) * t->elem_size;
    if (t->dtype == PG_DTYPE_F32) {
        pgd_h2d((char *)t->dev + off, &value, 4);
        return;
    }
    uint16_t h;
    if (t->dtype == PG_DTYPE_F16) {
        h = host_f32_to_f16(value);
    } else {
        uint32_t x;
        memcpy(&x, &value, 4);
        h = (x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu) ? (uint16_t)(0x7FC0u | ((x >> 16) & 1u))
                                                                 : (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
    }
    pgd_h2d((char *)t->dev + off, &h, 2);
}

/* tensor.c:473-520: |a - b| <= atol + rtol |b| elementwise in f32, 16-bit
 * elements widened; false for other shapes.  Waits for queued work. */
bool pg_tensor_allclose(const pg_tensor *a, const pg_tensor *b, float rtol, float atol)
{
    if (!a || !b || !pg_shape_equal(a->ndim, a->shape, b->ndim, b->shape))
        return false;
    unsigned char *ha = host_copy(a), *hb = ha ? host_copy(b) : NULL;
    bool ok = ha && hb;
    for (size_t i = 0; ok && i < a->numel; i++) {
        float av = host_elem(a, ha + i * a->elem_size), bv = host_elem(b, hb + i * b->elem_size);
        float diff = fabsf(av - bv);
        if (!(diff <= atol + rtol * fabsf(bv)))
            ok = false;
    }
    free(ha);
    free(hb);
    return ok;
}

/* tensor.c:522-545, :597-602: nested brackets, %g elements, rows after the
 * first indented by their depth */
static void print_rec(const pg_tensor *t, const unsigned char *h, size_t dim, size_t off, FILE *out)
{
    fputc('[', out);
    size_t inner = 1;
    for (size_t d = dim + 1; d < t->ndim; d++)
        inner *= t->shape[d];
    for (size_t i = 0; i < t->shape[dim]; i++) {
        if (dim + 1 == t->ndim) {
            fprintf(out, i ? ", %g" : "%g", host_elem(t, h + (off + i) * t->elem_size));
        } else {
            if (i)
                fprintf(out, ",\n%*s", (int)(dim + 1), "");
            print_rec(t, h, dim + 1, off + i * inner, out);
        }
    }
    fputc(']', out);
}

void pg_tensor_print(const pg_tensor *t, FILE *out)
{
    assert(t && out);
    unsigned char *h = host_copy(t);
    if (!h)
        return;
    if (t->ndim)
        print_rec(t, h, 0, 0, out);
    else
        fprintf(out, "%g", host_elem(t, h));
    fputc('\n', out);
    free(h);
}

/* tensor.c:99-118: the reference pools freed host buffers; here the pool is
 * the device allocator's cache of freed blocks */
void pg_tensor_pool_clear(void) { pg_amd_release_cached(); }
size_t pg_tensor_pool_size(void) { return pgd_cached_blocks(); }
size_t pg_tensor_pool_bytes(void) { return pg_amd_bytes_cached(); }
