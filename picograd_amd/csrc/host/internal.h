/*
 * Internal interfaces of the picograd-amd host library (C11).
 */
#ifndef PG_INTERNAL_H
#define PG_INTERNAL_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "picograd/amd.h"
#include "picograd/autograd.h"
#include "picograd/backend.h"
#include "picograd/jit.h"
#include "picograd/sgd.h"
#include "picograd/tensor.h"
#include "../kernels/launch.h"

/* pg_tensor.pg_flags */
#define PG_TENSOR_ZERO_PENDING 1u /* logically zero; device bytes not written */
/* Values pending on a storage: a clip-by-norm scale (pg_data_ref.clip_pending),
 * elements not yet written as act(pre-activation) (act_pending, a
 * linear16 output) or as a narrow product (narrow: a linear16 grad that is
 * the dgrad of a next layer of at most 16 outputs, formed by this layer's
 * backward in its activation pass).  pgt_settle writes them to the elements (before any
 * read of them other than by the optimiser kernels, which apply a pending
 * clip scale as they read), pgt_overwrite drops them when all of the
 * storage is about to be written (else settles), pgt_drop_clip drops them
 * (the storage's value is being discarded). */
bool pgt_settle(const pg_tensor *t);
void pgt_overwrite(const pg_tensor *t);
void pgt_drop_clip(const pg_tensor *t);
/* g = dn . wn^T over an [m, n] f32 storage, dn [m, kw] and wn [n, kw]
 * 16-bit (pgk_act_bwd16n's operands); the pending state owns up to two
 * device buffers (freed with pgd_free) and holds up to two storages */
typedef struct pg_narrow_pending {
    const uint16_t *dn, *wn;
    size_t m, n;
    int kw, dtype;
    void *own[2];
    size_t own_bytes[2];
    pg_data_ref *hold[2];
} pg_narrow_pending;
/* releases r's pending narrow product without writing it */
void pgt_narrow_release(pg_data_ref *r);

/* ---- device layer (device.c) ---- */
bool pgd_ok(void);                 /* init on first use; false if no device */
bool pgd_initialised(void);        /* pg_amd_init has succeeded (never inits) */
/* uploads or deferred forward ops are waiting to be queued: the next
 * pgd_stream()/pgd_sync() queues them (which may compile, allocate or wait) */
bool pgd_work_pending(void);
size_t pgd_cached_blocks(void);    /* freed blocks held by the allocator's cache */
pgk_stream pgd_stream(void);
/* side stream: work launched on pgd_fork()'s stream runs after everything
 * queued before the fork and before everything queued after pgd_join();
 * NULL / false on a device error */
pgk_stream pgd_fork(void);
bool pgd_join(void);
void *pgd_malloc(size_t nbytes);   /* cached, stream-ordered reuse */
void pgd_free(void *p, size_t nbytes);
bool pgd_h2d(void *dst, const void *src, size_t nbytes);  /* enqueued */
bool pgd_d2h(void *dst, const void *src, size_t nbytes);  /* waits */
bool pgd_d2d(void *dst, const void *src, size_t nbytes);  /* enqueued */
bool pgd_sync(void);
/* hands the pending batch of small uploads (see pgd_h2d) to a caller whose
 * kernel performs them: up to max entries are moved to out and no longer
 * pending; 0 when nothing is pending, -1 (nothing moved) when more than max
 * are.  The caller launches on pgd_stream() before queueing anything else. */
int pgd_upload_take(pgk_upload *out, int max);
/* puts a taken entry back at the end of the batch (call in the order taken,
 * before anything else is uploaded) */
void pgd_upload_requeue(const pgk_upload *e);
void pgd_set_err(const char *fmt, ...);
/* records a launcher status; false (and last error set) when non-zero */
bool pgd_check(int status, const char *what);
/* a scratch device buffer of at least nbytes, reused across calls on the
 * stream (grows, never shrinks) */
void *pgd_scratch(int slot, size_t nbytes);
#define PGD_SCRATCH_SLOTS 7 /* slot 5: a GEMM on the side stream; 3 and 6: linear16 bias-grad partials */
/* kernel timer (pg_amd_timer_*): kinds and bracket calls */
enum {
    PGD_T_JIT_MAIN = 0, PGD_T_JIT_FIN = 1, PGD_T_GEMM16 = 2, PGD_T_SGD = 3, PGD_T_STAGE = 4,
    PGD_T_ADAM = 5, PGD_T_CLIP = 6
};
int pgd_tbegin(int kind);
void pgd_tend(int slot);

/* ---- tensors (tensor.c) ---- */
pg_tensor *pgt_alloc(pg_dtype dtype, size_t ndim, const size_t *shape);
void pgt_set_contig_strides(pg_tensor *t);
bool pgt_is_contiguous(const pg_tensor *t);
/* drops one reference to a storage block, freeing it (and its 16-bit
 * copy) with the last */
void pgt_ref_release(pg_data_ref *r);
/* materialise a pending zero (grad tensors) */
void pgt_materialize(pg_tensor *t);
/* 16-bit (RNE) copy of an f32 tensor's elements, kept with its storage:
 * made on first use, remade after an in-place write marked it stale
 * (pgt_touch), rewritten by pg_sgd_step in the pass that updates the
 * elements.  NULL (device error set) on failure. */
const uint16_t *pgt_shadow16(pg_tensor *t, pg_dtype dt);
/* t's 16-bit copy when it is current (t the whole of its storage, nothing
 * pending on it), else NULL; never launches anything */
const uint16_t *pgt_shadow16_fresh(const pg_tensor *t, pg_dtype dt);
/* the buffer of t's 16-bit copy (allocated if missing, marked stale) for a
 * kernel that writes the copy beside t's elements; the writer marks it
 * current (shadow_stale = false) once its launch is queued.  NULL when t is
 * not the whole of its storage or the allocation fails */
uint16_t *pgt_shadow16_target(pg_tensor *t, pg_dtype dt);
/* the same copy held as rows of `cols` elements at a pitch of `ld`
 * (ld % 8 == 0: rows of whole 16-byte pieces) with zeros between, for a
 * GEMM operand whose rows are not; the storage is whole rows of cols */
const uint16_t *pgt_shadow16_rows(pg_tensor *t, pg_dtype dt, size_t cols, size_t ld);
/* records an in-place write of t's elements: its shadow is stale */
void pgt_touch(pg_tensor *t);
/* t itself when contiguous, else a new contiguous tensor holding t's
 * elements in row-major order (*owned set to it; free with
 * pg_tensor_free).  NULL on failure. */
const pg_tensor *pgt_contiguous(const pg_tensor *t, pg_tensor **owned);

/* ---- checkpoint I/O (checkpoint.c) ---- */
#include <stdio.h>
/* nbytes of device memory to / from a file through pinned double buffers
 * on the library stream (the save is ordered after queued work; the load
 * has finished when it returns).  false on a short read / write or a
 * device error. */
bool pgc_dev_to_file(const void *dev, size_t nbytes, FILE *fp);
bool pgc_file_to_dev(void *dev, size_t nbytes, FILE *fp);
/* reads one PGT1 record into dst's storage if dtype and shape match;
 * dst is left unchanged otherwise */
bool pgc_load_into(pg_tensor *dst, FILE *fp);

/* ---- deferred forward ops (autograd.c) ----
 * elementwise forward ops recorded while the JIT is on and run as one fused
 * kernel by pga_lazy_flush(), which the device layer calls before anything
 * else is queued or waited on */
bool pga_lazy_pending(void);
void pga_lazy_flush(void);
/* the pending small run and the fused backward region bwd in one launch
 * (true), or nothing launched (false) */
bool pga_lazy_flush_with_backward(const pg_jit_graph *bwd, size_t lnd, const size_t *ls, const void *const *bin,
                                  size_t bnin, void *const *bout, size_t bnout);
/* t is the output of a pending op: the run is flushed with t's 16-bit copy
 * (dt) also written into dst by its fused kernel.  True when that kernel
 * wrote it; false (the run flushed or left pending, dst not written) else */
bool pga_lazy_shadow16(const pg_tensor *t, int dt, uint16_t *dst);
/* the fused kernels write 16-bit operand copies (pg_amd_jit_copies16) */
bool pga_copies16(void);

/* ---- JIT internals (jit.c) ---- */
/* the graph's kernel is compiled without contracting a product and a sum
 * into one FMA, so it computes what separate kernels per op compute */
void pgj_graph_set_exact(pg_jit_graph *g);

/* ---- RNG (tensor.c) ---- */
void pg_rng_uniform_host(float *out, size_t n, float low, float high);
void pg_rng_normal_host(float *out, size_t n, float mean, float stddev);

/* ---- autograd shared (autograd.c / walker.c) ---- */
void pga_set_err(const char *fmt, ...);
bool pga_op_fusible(pg_ag_op_t op);
/* grad storage: returns the grad tensor ready for a write; *beta is 0 if
 * the writer must overwrite (grad fresh or logically zero), 1 to add */
pg_tensor *pga_grad_for_write(pg_node *n, int *beta);
void pga_backward_node(pg_node *n); /* eager device backward of one node */
/* a new op node over `parents` (retained); takes ownership of value and of
 * ctx (freed with free()); without grad mode or a grad-requiring parent the
 * node is a plain constant and ctx is freed at once */
pg_node *pga_attach(pg_tensor *value, size_t np, pg_node **parents, void (*bwd)(pg_node *), void *ctx,
                    pg_ag_op_t op);

/* forward of an elementwise op on f32 tensors (PGK_* codes), broadcast for
 * binary ops; recorded as a deferred op while the JIT is on, else launched.
 * NULL (autograd error set) on bad input. */
pg_tensor *pga_binary_fwd(int op, const pg_tensor *a, const pg_tensor *b);
pg_tensor *pga_unary_fwd(int op, const pg_tensor *a, float p0, float p1);

typedef struct { size_t axis; bool keepdim; } pga_red_ctx;
typedef struct { float p0, p1; } pga_param_ctx;

/* ---- matmul helpers (gemm.c) ---- */
pg_tensor *pgm_matmul_forward(const pg_tensor *a, const pg_tensor *b);
/* the 16-bit dtype in which a matmul16 node's backward reads its grad whole
 * (its grad [M, N] with N % 8 == 0: a current copy kept with the grad's
 * storage replaces its staging pass), else 0 */
int pgm_mm16_grad16(const pg_node *n);
void pgm_matmul_backward(pg_node *n);
/* a linear16 bias grad whose last step (the sum of its row-block partials)
 * the next activation pass was to run: run it now (the walk's end), or now
 * if it writes into t's storage (t is about to be written) */
void pgm_colsum_flush(void);
void pgm_colsum_flush_for(const pg_tensor *t);
/* pg_amd_ag_linear16's backward and the destructor of its node context
 * (the kept pre-activation), called by pg_node_free */
void pgm_linear16_backward(pg_node *n);
void pgm_linear16_free_ctx(void *ctx);

/* ---- JIT internals used by the walker (jit.c) ---- */
typedef struct pgj_region pgj_region;

/* Extended graph features for fused backward regions. */
int pgj_add_input_ex(pg_jit_graph *g, size_t ndim, const size_t *shape);
/* marks node `id` as an output reduced (summed) onto `ndim/shape`, a shape
 * broadcast-compatible with the loop shape, combining with beta */
void pgj_mark_output_ex(pg_jit_graph *g, int id, size_t ndim, const size_t *shape, int beta);
/* one more output: node id's values rounded to 16 bits (dt16 PG_DTYPE_F16 or
 * PG_DTYPE_BF16, as k_cast_to16 rounds) into a uint16_t buffer of the node's
 * shape, which the launch takes among the outputs; the node must have the
 * loop's full shape */
void pgj_mark_output16(pg_jit_graph *g, int id, int dt16);
/* the graph's stored values pass one asm copy each, read by their stores and
 * column sums (implied by a 16-bit output): set on a graph that stores a
 * 16-bit copy in one mode of its caller and not in another, so both modes
 * compute the same bits */
void pgj_graph_set_launder(pg_jit_graph *g);
int pgj_op_internal(pg_jit_graph *g, int op, int a, int b);
/* dst gains src's nodes (src input i -> dst node in_map[i]) and, after its
 * own, src's outputs, each of which must have the loop shape (lnd, ls) */
bool pgj_graph_append(pg_jit_graph *dst, const pg_jit_graph *src, const int *in_map, size_t lnd, const size_t *ls);
bool pgj_input_shape(const pg_jit_graph *g, size_t i, size_t *ndim, const size_t **shape);
enum { PGJ_OP_GELU_GRAD = 100, PGJ_OP_SIGN = 101, PGJ_OP_ERF_GRAD = 102 };
/* compile (cached) and launch with device pointers; loop shape given
 * explicitly.  Returns false and sets the JIT error on failure. */
bool pgj_launch(pg_jit_graph *g, size_t loop_ndim, const size_t *loop_shape,
                const void *const *inputs, size_t ninputs, void *const *outputs,
                size_t noutputs);
/* A small run as one block (PGJ_SMALL_MAX loop elements at most): the block
 * first performs the given uploads (at most PGJ_SMALL_UPLOAD_BYTES, every
 * address and size a multiple of 16; pgj_small_fits), then the run, then,
 * for red_out >= 0, reduce_all's two stages over output red_out of a 2-D
 * loop shape (pgj_small_reduce_fits): r1[cols] its column sums and
 * r2[0] = scale * sum(r1), the additions of pgk_sum_all2_f32 in its order. */
#define PGJ_SMALL_MAX 16384
#define PGJ_SMALL_UPLOAD_BYTES ((size_t)256 << 10)
bool pgj_small_fits(size_t numel, size_t nup, const pgk_upload *up);
bool pgj_small_reduce_fits(size_t loop_ndim, const size_t *loop_shape);
bool pgj_launch_small(pg_jit_graph *g, size_t loop_ndim, const size_t *loop_shape,
                      const void *const *inputs, size_t ninputs, void *const *outputs,
                      size_t noutputs, const pgk_upload *up, size_t nup, int red_out, float *r1,
                      float *r2, float scale);
extern size_t pgj_stat_compiles, pgj_stat_hits;

#endif
