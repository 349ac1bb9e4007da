/*
 * Device-resident tensors (the reference's core/tensor.c:21-427 data model
 * with storage in HBM).  Elements live in a refcounted device block
 * (pg_data_ref); `data` is a host mirror filled on demand.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

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

void pgt_ref_release(pg_data_ref *r)
{
    if (r && --r->refs == 0) {
        pgd_free(r->ptr, r->nbytes);
        if (r->shadow)
            pgd_free(r->shadow, r->nbytes / 2);
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

void pgt_materialize(pg_tensor *t)
{
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

bool pg_amd_tensor_refresh16(pg_tensor *t)
{
    if (!t || !t->data_ref)
        return false;
    pg_data_ref *r = t->data_ref;
    if (!r->shadow || !r->shadow_stale)
        return true;
    return pgt_shadow16(t, (pg_dtype)r->shadow_dtype) != NULL;
}

const uint16_t *pgt_shadow16(pg_tensor *t, pg_dtype dt)
{
    if (!t || !t->data_ref || t->dtype != PG_DTYPE_F32 || (dt != PG_DTYPE_F16 && dt != PG_DTYPE_BF16)) {
        pgd_set_err("shadow16: needs an f32 tensor and a 16-bit dtype");
        return NULL;
    }
    pg_data_ref *r = t->data_ref;
    size_t n = r->nbytes / 4;
    if (r->shadow && r->shadow_dtype == (int)dt && !r->shadow_stale)
        return r->shadow;
    if (!r->shadow) {
        r->shadow = pgd_malloc(n ? n * 2 : 1);
        if (!r->shadow)
            return NULL;
    }
    r->shadow_dtype = (int)dt;
    pgt_materialize(t);
    if (!pgd_check(pgk_cast_to16((int)dt, r->ptr, r->shadow, n, pgd_stream()), "shadow16"))
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
    if (!pgt_is_contiguous(t)) {
        pgd_set_err("pg_tensor_clone: strided source not supported");
        pg_tensor_free(c);
        return NULL;
    }
    pgd_d2d(c->dev, t->dev, t->numel * t->elem_size);
    return c;
}

void pg_tensor_fill(pg_tensor *t, float value)
{
    if (!t)
        return;
    t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
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
    if (!src)
        return NULL;
    return pg_tensor_reshape_view(src, src->ndim, src->shape);
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
    return pgd_d2h(dst, t->dev, nb);
}

bool pg_tensor_copy_from_host(pg_tensor *t, const void *src)
{
    if (!t || !src)
        return false;
    t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
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
