/*
 * pg_tensor: the reference's tensor ABI (core/tensor.h:15-96) with the
 * storage moved to MI355X HBM.
 *
 * The leading fields keep the reference layout so existing callers compile
 * unchanged.  What differs:
 *   - the elements live in device memory at `dev`; `data` is a host mirror
 *     that is NULL until pg_tensor_sync_host() fills it, and is stale after
 *     any later device write until the next pg_tensor_sync_host();
 *   - a caller that edits the host mirror pushes it back with
 *     pg_tensor_sync_device();
 *   - every constructor and op enqueues its device work on the library
 *     stream (pg_amd_stream()) and returns without waiting for it.
 */
#ifndef PICOGRAD_TENSOR_H
#define PICOGRAD_TENSOR_H

#include <stdbool.h>
#include <stddef.h>
#include <stdio.h>

#include "dtype.h"

#ifdef __cplusplus
extern "C" {
#endif

#define PG_MAX_NDIM 8

typedef struct pg_data_ref {
    void *ptr;     /* device allocation */
    size_t nbytes;
    int refs;
    /* ---- appended: 16-bit (RNE) copy of f32 elements kept beside the
     * storage for the MFMA GEMMs (pg_amd_ag_matmul16); library-internal */
    void *shadow;
    int shadow_dtype;  /* PG_DTYPE_F16 or PG_DTYPE_BF16 */
    bool shadow_stale; /* an in-place write happened after it was made */
    /* rows of shadow_cols elements at a pitch of shadow_ld (zeros between),
     * for a GEMM operand whose rows are not whole 16-byte pieces; 0: the
     * elements in storage order */
    size_t shadow_cols, shadow_ld;
    size_t shadow_bytes; /* its allocation */
    /* a clip-by-norm scale not yet written to the f32 elements: each
     * element's value is (x * clip_mul) * clip_inv (pg_clip_grad_norm);
     * library-internal */
    bool clip_pending;
    float clip_mul, clip_inv;
    /* elements not yet written: each is act(act_src[i]) (act_pending =
     * PG_ACT_RELU or PG_ACT_GELU; 0: none), act_src's storage held through
     * act_src_ref until they are (pg_amd_ag_linear16's output, whose GEMM
     * wrote the pre-activation and the 16-bit copy); library-internal */
    int act_pending;
    const float *act_src;
    struct pg_data_ref *act_src_ref;
    /* elements not yet written: the product of a narrow next layer's dz and
     * weights (its dgrad), formed by the first reader; library-internal */
    struct pg_narrow_pending *narrow;
} pg_data_ref;

typedef struct pg_tensor {
    size_t ndim;
    size_t shape[PG_MAX_NDIM];
    size_t stride[PG_MAX_NDIM];
    size_t numel;
    union {
        float *data;        /* host mirror, f32 view */
        void *data_raw;
        uint16_t *data_u16; /* host mirror, f16/bf16 view */
    };
    pg_data_ref *data_ref;
    bool is_view;
    struct pg_tensor *view_parent;
    pg_dtype dtype;
    size_t elem_size;
    /* ---- appended: device residency ---- */
    void *dev;          /* device address of element 0 */
    unsigned pg_flags;  /* PG_TENSOR_* bits, library-internal */
} pg_tensor;

/* constructors: tensor.h:38-58 of the reference */
pg_tensor *pg_tensor_new_dtype(pg_dtype dtype, size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_empty_dtype(pg_dtype dtype, size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_from_data_dtype(pg_dtype dtype, size_t ndim, const size_t *shape, const void *data);
pg_tensor *pg_tensor_zeros_dtype(pg_dtype dtype, size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_ones_dtype(pg_dtype dtype, size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_full_dtype(pg_dtype dtype, size_t ndim, const size_t *shape, float value);

pg_tensor *pg_tensor_new(size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_empty(size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_zeros(size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_ones(size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_full(size_t ndim, const size_t *shape, float value);
pg_tensor *pg_tensor_from_data(size_t ndim, const size_t *shape, const float *data);
pg_tensor *pg_tensor_arange(float start, float stop, float step);
pg_tensor *pg_tensor_uniform(size_t ndim, const size_t *shape, float low, float high);
pg_tensor *pg_tensor_normal(size_t ndim, const size_t *shape, float mean, float stddev);
pg_tensor *pg_tensor_linspace(float start, float stop, size_t num);
pg_tensor *pg_tensor_eye(size_t n);

pg_tensor *pg_tensor_clone(const pg_tensor *t);
void pg_tensor_free(pg_tensor *t);

static inline float *pg_tensor_f32(const pg_tensor *t) { return (float *)t->data_raw; }
static inline uint16_t *pg_tensor_f16(const pg_tensor *t) { return (uint16_t *)t->data_raw; }
static inline uint16_t *pg_tensor_bf16(const pg_tensor *t) { return (uint16_t *)t->data_raw; }
static inline size_t pg_tensor_nbytes(const pg_tensor *t) { return t->numel * t->elem_size; }

/* splitmix64 stream shared by pg_tensor_uniform/normal (tensor.c:289-339) */
void pg_seed(unsigned long long seed);

/* tensor.h:68-69: one element at a multi-index (strides honoured).  get
 * waits for the queued work and reads the element from device memory; set
 * queues the write (rounded to nearest even for f16/bf16). */
float pg_tensor_get(const pg_tensor *t, const size_t *idx);
void pg_tensor_set(pg_tensor *t, const size_t *idx, float value);

void pg_tensor_fill(pg_tensor *t, float value);
void pg_tensor_copy_from(pg_tensor *dst, const pg_tensor *src);
bool pg_tensor_reshape(pg_tensor *t, size_t ndim, const size_t *shape);

size_t pg_shape_numel(size_t ndim, const size_t *shape);
bool pg_shape_equal(size_t ndim_a, const size_t *shape_a, size_t ndim_b, const size_t *shape_b);

/* tensor.h:78-79: both wait for the queued work.  allclose compares
 * |a - b| <= atol + rtol |b| elementwise in f32 (f16/bf16 widened), false
 * for different shapes; print writes the reference's nested-bracket text. */
bool pg_tensor_allclose(const pg_tensor *a, const pg_tensor *b, float rtol, float atol);
void pg_tensor_print(const pg_tensor *t, FILE *out);

/* views share the storage (reference counted); tensor.h:82-84 */
pg_tensor *pg_tensor_view(const pg_tensor *src);
pg_tensor *pg_tensor_reshape_view(const pg_tensor *src, size_t ndim, const size_t *shape);
pg_tensor *pg_tensor_permute_view(const pg_tensor *src, const size_t *order);

/* serialization, tensor.h:86-91 of the reference: the PGT1 format ("PGT1",
 * u32 version 1, u32 dtype, u32 ndim, u64 shape[ndim], u64 numel, u64
 * elem_size, then the elements row-major).  Saves read the elements from
 * device memory after all queued work; loads return a device tensor.  The
 * files are byte-identical to the reference's, and each reads the other's.
 * Loads reject what the reference rejects (bad magic or version, dtype out
 * of range, ndim 0 or above 8, a dimension of 0 or above 10,000,000, numel
 * or element size disagreeing with the header). */
bool pg_tensor_save(const pg_tensor *t, const char *path);
pg_tensor *pg_tensor_load(const char *path);
bool pg_tensor_save_fp(const pg_tensor *t, FILE *fp);
pg_tensor *pg_tensor_load_fp(FILE *fp);

/* tensor.h:93-95: the reference pools freed host buffers; here the pool
 * is the device allocator's cache of freed blocks (count and bytes held;
 * clear returns them to the driver after the queued work). */
void pg_tensor_pool_clear(void);
size_t pg_tensor_pool_size(void);
size_t pg_tensor_pool_bytes(void);

/* ---- appended: host/device synchronisation ---- */
/* Waits for queued device work, then copies the elements into the host
 * mirror t->data (allocated on first use).  Returns false on failure. */
bool pg_tensor_sync_host(pg_tensor *t);
/* Copies the host mirror back to device memory (after a caller edited it). */
bool pg_tensor_sync_device(pg_tensor *t);
/* Copies numel*elem_size bytes of device data into dst (waits first). */
bool pg_tensor_copy_to_host(const pg_tensor *t, void *dst);
/* Copies numel*elem_size bytes from src into device data (enqueued). */
bool pg_tensor_copy_from_host(pg_tensor *t, const void *src);

#ifdef __cplusplus
}
#endif

#endif
