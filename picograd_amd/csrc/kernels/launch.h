/*
 * C-ABI launchers of the hand-written gfx950 kernels (kernels, .hip files).
 * The C11 host code calls only these; each enqueues on the given stream and
 * returns 0, or a hipError_t value when the launch was rejected.
 */
#ifndef PGK_LAUNCH_H
#define PGK_LAUNCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *pgk_stream; /* hipStream_t */

#define PGK_MAX_NDIM 8

/* unary forward / backward op codes (shared with the JIT codegen) */
enum {
    PGK_NEG = 0, PGK_EXP, PGK_LOG, PGK_SQRT, PGK_SIN, PGK_COS, PGK_RELU,
    PGK_SIGMOID, PGK_TANH, PGK_GELU, PGK_ERF, PGK_ABS, PGK_LEAKY, PGK_CLAMP,
    PGK_UNARY_COUNT
};
/* binary op codes */
enum { PGK_ADD = 0, PGK_SUB, PGK_MUL, PGK_DIV, PGK_BINARY_COUNT };

/* An output of `ndim` dims and two (broadcast) operand stride sets, in
 * elements; a zero stride repeats the operand along that dim. */
typedef struct {
    int ndim;
    int64_t shape[PGK_MAX_NDIM];
    int64_t sa[PGK_MAX_NDIM];
    int64_t sb[PGK_MAX_NDIM];
} pgk_bcast;

/* The no-alloc workspace (scratch.hip): a fixed device array per device.
 * _init records the current device's address of it (once per device) and
 * returns a hipError_t value; pgk_noalloc_scratch returns that address
 * (initialising first for a device not seen yet), NULL on failure. */
size_t pgk_noalloc_scratch_bytes(void);
int pgk_noalloc_scratch_init(void);
void *pgk_noalloc_scratch(void);

int pgk_fill_f32(float *dst, size_t n, float v, pgk_stream s);

/* A batch of small uploads written by one kernel: dst[0..n) = src[0..n)
 * for each entry, src in pinned host memory the device reads directly (a
 * device address of it).  At most PGK_UPLOAD_MAX entries per call; the
 * destinations must not overlap. */
#define PGK_UPLOAD_MAX 32
typedef struct {
    void *dst;
    const void *src;
    size_t n;
} pgk_upload;
int pgk_upload_scatter(const pgk_upload *ents, int n, pgk_stream s);
int pgk_fill_u16(uint16_t *dst, size_t n, uint16_t v, pgk_stream s);

/* y = op(x) */
int pgk_unary_f32(int op, const float *x, float *y, size_t n, float p0, float p1, pgk_stream s);
/* dx = (beta ? dx : 0) + scale * g * op'(x) */
int pgk_unary_bwd_f32(int op, const float *g, const float *x, float *dx, size_t n, float p0,
                      float p1, float scale, int beta, pgk_stream s);
/* y[i] = a[off_a(i)] op b[off_b(i)] over bc->shape */
int pgk_binary_f32(int op, const float *a, const float *b, float *y, const pgk_bcast *bc,
                   pgk_stream s);

/*
 * dst (dst_numel elements) (beta ? += : =) scale * sum of src over the
 * source elements that map onto each dst element.  src is contiguous with
 * shape bc->shape; bc->sa holds dst strides per src dim (0 on reduced dims).
 * Deterministic: each dst element sums its sources in row-major order.
 */
int pgk_reduce_into_f32(float *dst, size_t dst_numel, const float *src, const pgk_bcast *bc,
                        float scale, int beta, pgk_stream s);
/* dst[i] (beta ? += : =) scale * src[off(i)], broadcasting src over bc->shape
 * with strides bc->sa (dst contiguous). */
int pgk_expand_into_f32(float *dst, const float *src, const pgk_bcast *bc, float scale, int beta,
                        pgk_stream s);

/* forward reductions: y[o, i] = scale * sum_l x[o, l, i], summed in
 * fixed slices of l and then across slices (deterministic).  ws holds
 * pgk_sum_axis_workspace() bytes (none needed when that is 0). */
size_t pgk_sum_axis_workspace(size_t outer, size_t len, size_t inner);
int pgk_sum_axis_f32(const float *x, float *y, size_t outer, size_t len, size_t inner,
                     float scale, void *ws, pgk_stream s);
/* Both stages of reduce_all over a contiguous [rows, cols] in one launch:
 * y1[cols] = column sums, y2[0] = scale * sum(y1), with the additions of
 * two pgk_sum_axis_f32 calls in their order.  Only where each stage is a
 * single run (pgk_sum_all2_fits: short axes, cols <= 256); otherwise
 * hipErrorInvalidValue. */
int pgk_sum_all2_fits(size_t rows, size_t cols);
int pgk_sum_all2_f32(const float *x, float *y1, float *y2, size_t rows, size_t cols, float scale,
                     pgk_stream s);
/* The same, in one launch, where the column sums are cut into slices of
 * rows (the slices pgk_sum_axis_f32 takes, each added in row order, then
 * the slices in order) and the sum over the columns is a single run
 * (pgk_sum_all2s_fits: slices x cols <= 1024, cols < 128). */
int pgk_sum_all2s_fits(size_t rows, size_t cols);
int pgk_sum_all2s_f32(const float *x, float *y1, float *y2, size_t rows, size_t cols, float scale,
                      pgk_stream s);

/* dtype casts with the reference's RNE bit rules; dtype 1 = f16, 2 = bf16 */
int pgk_cast_to16(int dtype, const float *src, uint16_t *dst, size_t n, pgk_stream s);
int pgk_cast_from16(int dtype, const uint16_t *src, float *dst, size_t n, pgk_stream s);
/* dst (contiguous) = the ndim-dim strided view at src in row-major order;
 * elem_size 2 or 4 bytes, strides in elements */
int pgk_gather_strided(size_t elem_size, const void *src, void *dst, int ndim, const size_t *shape,
                       const size_t *stride, pgk_stream s);

/*
 * Operand staging for the MFMA GEMM (only where a dimension needs padding
 * to a multiple of 8, and for the f32 -> 16-bit cast of an upstream grad):
 * dst[r * ldd + c] = cvt(src[r * lds + c]) for r < rows, c < cols, zeros
 * for rows [rows, rows_pad) and columns [cols, ldd).  src_dtype 0 = f32
 * (rounded to dtype), else 16-bit of the same dtype; batch copies use the
 * given strides.
 */
int pgk_copy_to16(int dtype, int src_dtype, const void *src, size_t rows, size_t cols, size_t lds,
                  uint16_t *dst, size_t ldd, size_t rows_pad, size_t batch, size_t sstride, size_t dstride,
                  pgk_stream s);

/*
 * C[b][i, j] (beta ? += : =) sum_p A(i, p) B(p, j), f16 (dtype 1) or bf16
 * (dtype 2) operands, f32 accumulate and output.
 *   ta = 0: A(i, p) = a[i * lda + p]    ta = 1: A(i, p) = a[p * lda + i]
 *   tb = 0: B(p, j) = b[j * ldb + p]    tb = 1: B(p, j) = b[p * ldb + j]
 * Requirements: a, b 16-byte aligned; lda, ldb, batch strides multiples of
 * 8.  a_extent / b_extent bound the loads along each operand's i (j) dim:
 * at least m (n), and for an operand with that dim contiguous (ta / tb) a
 * multiple of 8 whose columns [m, a_extent) may be read (zero-padding or
 * real data; never used in the result).  When k % 64 != 0, `ws` must hold
 * pgk_gemm16_workspace(...) bytes (it stages the last k-slab).
 */
size_t pgk_gemm16_workspace(int ta, int tb, size_t m, size_t n, size_t k, size_t batch);

/* Optional epilogue of pgk_gemm16 (one matrix, beta = 0): with
 * v = sum_p A(i, p) B(p, j) + bias[j], it writes C[i, j] = act(v),
 * z[i, j] = v and c16[i, j] = RNE-16-bit(act(v)) (z, c16 at C's leading
 * dim; each NULL to skip).  act codes follow the reference's
 * backend/cpu/gemm.h:37-39. */
enum { PGK_ACT_NONE = 0, PGK_ACT_RELU = 1, PGK_ACT_GELU = 2 };
typedef struct {
    const float *bias; /* [n] or NULL */
    int act;
    float *z;
    uint16_t *c16;
    int dtype16; /* 1 = f16, 2 = bf16 */
    /* C itself is not written (z and c16 are): the caller materialises
     * act(z) when C is first read.  Only where the epilogue rides on the
     * GEMM or the split-K sum (no k-tail, k > 0). */
    int skip_out;
} pgk_epi;
int pgk_gemm16(int dtype, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda,
               size_t stride_a, size_t a_extent, const uint16_t *b, size_t ldb, size_t stride_b, size_t b_extent,
               float *c, size_t ldc, size_t stride_c, size_t batch, int beta, const pgk_epi *epi, void *ws,
               pgk_stream s);
/* The same GEMM planned for `cu_budget` CUs (0: the whole chip), for a
 * launch that runs beside another on the rest of the chip; its workspace
 * size, and the planner's estimate of its time in seconds. */
int pgk_gemm16_cu(int dtype, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda,
                  size_t stride_a, size_t a_extent, const uint16_t *b, size_t ldb, size_t stride_b, size_t b_extent,
                  float *c, size_t ldc, size_t stride_c, size_t batch, int beta, const pgk_epi *epi, void *ws,
                  int cu_budget, pgk_stream s);
size_t pgk_gemm16_workspace_cu(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget);
double pgk_gemm16_time(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget);
/* the tile (1: 128 x 128, 2: 256 x 256, 3: 128 x 256) and split-K factor
 * (*splits) pgk_gemm16_cu's main launch takes for these sizes */
int pgk_gemm16_plan(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget, int *splits);
/* One GEMM problem of pgk_gemm16's parameters */
typedef struct {
    size_t m, n, k;
    const uint16_t *a;
    size_t lda, stride_a, a_extent;
    const uint16_t *b;
    size_t ldb, stride_b, b_extent;
    float *c;
    size_t ldc, stride_c, batch;
    int beta;
} pgk_gemm_desc;
/* A matmul's dgrad d (both operands K-contiguous: ta = tb = 0) and wgrad w
 * (both MN-contiguous: ta = tb = 1) in ONE launch, d planned for cu_d CUs
 * and w for the rest, each split along k as its plan says (one more launch
 * then adds both problems' slices): the two run side by side with no second
 * stream.  cu_d = 0 plans both for the whole chip: d's blocks, then w's,
 * in one grid of several rounds.
 * PGK_GEMM_NOT_PAIRED (nothing launched) when one launch cannot hold the
 * pair: a k that needs a zero-padded tail launch, or the plans choose
 * different tile sizes.  ws: pgk_gemm16_pair_dw_workspace bytes. */
#define PGK_GEMM_NOT_PAIRED (-1)
size_t pgk_gemm16_pair_dw_workspace(const pgk_gemm_desc *d, const pgk_gemm_desc *w, int cu_d, size_t *off_w);
int pgk_gemm16_pair_dw(int dtype, const pgk_gemm_desc *d, const pgk_gemm_desc *w, int cu_d, void *ws,
                       pgk_stream s);

/* MFMA rate probe: `blocks` x 512 threads, each wave 8 x iters bf16
 * 32x32x16 MFMAs, operands from registers (lds 0) or LDS (lds 1); sink
 * receives blocks * 512 floats.  FLOP = blocks * 8 * iters * 8 * 32768. */
int pgk_mfma_probe(int lds, float *sink, size_t sink_floats, int blocks, int iters, pgk_stream s);

/* f32 GEMM, C (beta ? += : =) op(A) op(B); ta/tb select A^T / B^T
 * (A(i,p) = ta ? a[p*lda+i] : a[i*lda+p], same for B(p,j)). */
int pgk_gemm_f32(int ta, int tb, size_t m, size_t n, size_t k, const float *a, size_t lda,
                 size_t stride_a, const float *b, size_t ldb, size_t stride_b, float *c,
                 size_t ldc, size_t stride_c, size_t batch, int beta, pgk_stream s);

/* The last step of a bias grad: out[c] (beta ? += : =) the sum over the
 * nblk row-block partials part[b * n + c], b in order. */
typedef struct {
    const float *part;
    size_t nblk, n;
    float *out;
    int beta;
} pgk_colsum_job;
int pgk_colsum_run(const pgk_colsum_job *job, pgk_stream s);

/* Backward of an activation feeding a 16-bit GEMM: dz = g * act'(z) over
 * a [m, n] f32 grad (act PGK_ACT_*; z the pre-activation, unused for
 * PGK_ACT_NONE), written RNE to d16 rows of ldd (ldd % 8 == 0, zero columns
 * past n); when db is given, db[j] (beta ? += : =) sum_i dz[i, j] in a
 * fixed order (ws holds pgk_act_bwd16_workspace bytes): the pass writes the
 * row-block partials to ws and a second launch adds them, unless defer is
 * given, which then receives that last step as a job (ws must stay as it is
 * until the job runs).  A job given as fold (an earlier pass's deferred
 * one, its partials not in ws) runs in this pass's launch, in a row of extra
 * blocks. */
size_t pgk_act_bwd16_workspace(size_t m, size_t n);
int pgk_act_bwd16(int act, const float *g, const float *z, size_t m, size_t n, uint16_t *d16, size_t ldd,
                  int dtype, float *db, int db_beta, void *ws, const pgk_colsum_job *fold, pgk_colsum_job *defer,
                  pgk_stream s);
/* The same pass with g formed in it as the dgrad of a narrow next layer:
 * g = dn . wn^T, dn [m, kw] and wn [n, kw] 16-bit of ndtype (kw 8 or 16,
 * zero columns past the layer's width), with the MFMA sequence of
 * pgk_gemm16's dgrad of those operands (the same bits), used for dz and,
 * when g is given, written to g [m, n] (every element).  With wsnap, wn is
 * copied there (n x kw).  ws, fold and defer as for pgk_act_bwd16.  With
 * d16 and db NULL only g is written (the narrow dgrad itself); g and d16
 * are not both NULL. */
int pgk_act_bwd16n(int act, const uint16_t *dn, const uint16_t *wn, int kw, int ndtype, uint16_t *wsnap, float *g,
                   const float *z, size_t m, size_t n, uint16_t *d16, size_t ldd, int dtype, float *db, int db_beta,
                   void *ws, const pgk_colsum_job *fold, pgk_colsum_job *defer, pgk_stream s);

/* multi-tensor SGD */
typedef struct {
    float *p;
    const float *g;
    float *buf;       /* NULL when momentum == 0 */
    uint16_t *shadow; /* optional 16-bit copy of p written after the update */
    int shadow_dtype; /* 1 = f16, 2 = bf16 (RNE) */
    size_t n;
    /* shadow_cols != 0: element j's copy at (j / shadow_cols) * shadow_ld +
     * j % shadow_cols (rows padded to a pitch); 0: at j */
    size_t shadow_cols, shadow_ld;
    /* gclip: g is read as (g * gmul) * ginv (a pending clip-by-norm scale) */
    int gclip;
    float gmul, ginv;
} pgk_sgd_seg;
int pgk_sgd_multi(const pgk_sgd_seg *segs, int nseg, float lr, float momentum, float dampening,
                  float weight_decay, int nesterov, pgk_stream s);

/* multi-tensor Adam / AdamW (optim.hip) */
typedef struct {
    float *p;
    const float *g;
    float *m, *v;
    float *vmax;      /* amsgrad only, else NULL */
    uint16_t *shadow; /* optional 16-bit copy of p written after the update */
    int shadow_dtype; /* 1 = f16, 2 = bf16 (RNE) */
    float lr, wd;     /* this tensor's learning rate and weight decay */
    size_t n;
    size_t shadow_cols, shadow_ld; /* as pgk_sgd_seg's */
    int gclip;                     /* as pgk_sgd_seg's */
    float gmul, ginv;
} pgk_adam_seg;
typedef struct {
    float beta1, beta2, eps;
    float bc1;     /* 1 - beta1^t, floored at 1e-12 */
    float inv_bc2; /* 1 / (1 - beta2^t), the floor applied before the division */
    int amsgrad, decoupled;
} pgk_adam_hyper;
int pgk_adam_multi(const pgk_adam_seg *segs, int nseg, const pgk_adam_hyper *h, pgk_stream s);

/* gradient clipping over a list of f32 grads (optim.hip) */
typedef struct {
    float *g;
    size_t n;
} pgk_grad_seg;
/* bytes of workspace pgk_grad_norm needs for these grads */
size_t pgk_grad_norm_workspace(const pgk_grad_seg *segs, int nseg);
/* res[0] = (float)sqrt(sum of squares in f64), the grads added in list
 * order and each in a fixed block order.  With clip set, also
 * res[1] = 1 / (res[0] + eps), res[2] = 1 unless res[0] <= max_norm (else 0)
 * and res[3] = max_norm.  res is 4 floats of device memory. */
int pgk_grad_norm(const pgk_grad_seg *segs, int nseg, int clip, float max_norm, float eps, float *res,
                  void *ws, pgk_stream s);
/* g = (g * res[3]) * res[1] for every grad when res[2] is 1 (the
 * device-side decision pgk_grad_norm took); a tensor must not appear twice
 * in one call */
int pgk_grad_scale(const pgk_grad_seg *segs, int nseg, const float *res, pgk_stream s);
/* g = (g * mul) * inv for every grad (a scale decided on the host) */
int pgk_grad_scale_const(const pgk_grad_seg *segs, int nseg, float mul, float inv, pgk_stream s);
/* g = min(max(g, -c), c) elementwise (NaN kept); a tensor must not
 * appear twice in one call */
int pgk_clip_value(const pgk_grad_seg *segs, int nseg, float c, pgk_stream s);

#ifdef __cplusplus
}
#endif

#endif
