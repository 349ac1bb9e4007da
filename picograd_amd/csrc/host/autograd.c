/*
 * Autograd nodes, forward ops and the eager (non-fused) device backward of
 * each op.  Node ownership and graph construction follow the reference's
 * autograd/autograd.c:64-260 (attach retains parents, requires_grad
 * propagates, no-grad mode builds detached nodes); every value and grad is
 * a device tensor and every op enqueues kernels on the library stream.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- state */

static char g_err[512];
static bool g_grad_enabled = true;
static int g_no_grad_depth;

void pga_set_err(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

const char *pg_autograd_last_error(void) { return g_err; }
bool pg_autograd_is_grad_enabled(void) { return g_grad_enabled && g_no_grad_depth == 0; }
void pg_autograd_set_grad_enabled(bool enabled) { g_grad_enabled = enabled; }
void pg_no_grad_push(void) { g_no_grad_depth++; }
void pg_no_grad_pop(void)
{
    if (g_no_grad_depth > 0)
        g_no_grad_depth--;
}

/* ---------------------------------------------------------------- nodes */

static pg_node *node_wrap(pg_tensor *t, bool requires_grad)
{
    if (!t)
        return NULL;
    pg_node *n = calloc(1, sizeof *n);
    if (!n) {
        pg_tensor_free(t);
        return NULL;
    }
    n->value = t;
    n->requires_grad = requires_grad;
    n->refs = 1;
    return n;
}

static pg_node *attach(pg_tensor *value, size_t np, pg_node **parents, void (*bwd)(pg_node *), void *ctx,
                       pg_ag_op_t op)
{
    if (!value) {
        free(ctx);
        return NULL;
    }
    if (!pg_autograd_is_grad_enabled()) {
        free(ctx);
        return node_wrap(value, false);
    }
    pg_node *n = calloc(1, sizeof *n);
    if (!n) {
        pg_tensor_free(value);
        free(ctx);
        return NULL;
    }
    n->value = value;
    n->backward = bwd;
    n->ctx = ctx;
    n->ag_op = op;
    n->refs = 1;
    if (np) {
        n->parents = malloc(np * sizeof *n->parents);
        if (!n->parents) {
            free(n);
            pg_tensor_free(value);
            free(ctx);
            return NULL;
        }
        for (size_t i = 0; i < np; i++) {
            n->parents[i] = pg_node_retain(parents[i]);
            n->requires_grad |= parents[i]->requires_grad;
        }
        n->nparents = np;
        if (!n->requires_grad) {
            n->backward = NULL;
            free(ctx);
            n->ctx = NULL;
        }
    }
    return n;
}

pg_node *pga_attach(pg_tensor *value, size_t np, pg_node **parents, void (*bwd)(pg_node *), void *ctx,
                    pg_ag_op_t op)
{
    return attach(value, np, parents, bwd, ctx, op);
}

pg_node *pg_var_from_data(size_t ndim, const size_t *shape, const float *data, bool rg)
{
    return node_wrap(pg_tensor_from_data(ndim, shape, data), rg);
}

pg_node *pg_var_from_tensor(const pg_tensor *t, bool rg)
{
    if (!t)
        return NULL;
    pg_tensor *c = pgt_alloc(t->dtype, t->ndim, t->shape);
    if (!c)
        return NULL;
    if (t->pg_flags & PG_TENSOR_ZERO_PENDING)
        pg_tensor_fill(c, 0.0f);
    else
        pgd_d2d(c->dev, t->dev, t->numel * t->elem_size);
    return node_wrap(c, rg);
}

pg_node *pg_var_zeros(size_t ndim, const size_t *shape, bool rg) { return node_wrap(pg_tensor_zeros(ndim, shape), rg); }
pg_node *pg_var_ones(size_t ndim, const size_t *shape, bool rg) { return node_wrap(pg_tensor_ones(ndim, shape), rg); }
pg_node *pg_var_full(size_t ndim, const size_t *shape, float v, bool rg)
{
    return node_wrap(pg_tensor_full(ndim, shape, v), rg);
}
pg_node *pg_var_uniform(size_t ndim, const size_t *shape, float lo, float hi, bool rg)
{
    return node_wrap(pg_tensor_uniform(ndim, shape, lo, hi), rg);
}
pg_node *pg_var_normal(size_t ndim, const size_t *shape, float mean, float sd, bool rg)
{
    return node_wrap(pg_tensor_normal(ndim, shape, mean, sd), rg);
}
pg_node *pg_var_scalar(float v, bool rg) { return pg_var_full(1, (size_t[]){1}, v, rg); }

pg_node *pg_node_retain(pg_node *n)
{
    if (n)
        n->refs++;
    return n;
}

void pg_node_free(pg_node *n)
{
    if (!n)
        return;
    size_t cap = 16, sp = 0;
    pg_node **stk = malloc(cap * sizeof *stk);
    if (!stk)
        return;
    stk[sp++] = n;
    while (sp) {
        pg_node *t = stk[--sp];
        if (--t->refs)
            continue;
        pg_tensor_free(t->value);
        pg_tensor_free(t->grad);
        if (t->backward == pgm_linear16_backward)
            pgm_linear16_free_ctx(t->ctx);
        else
            free(t->ctx);
        if (sp + t->nparents > cap) {
            while (sp + t->nparents > cap)
                cap *= 2;
            pg_node **ns = realloc(stk, cap * sizeof *ns);
            if (!ns)
                break;
            stk = ns;
        }
        for (size_t i = 0; i < t->nparents; i++)
            stk[sp++] = t->parents[i];
        free(t->parents);
        free(t);
    }
    free(stk);
}

pg_node *pg_node_detach(pg_node *n)
{
    if (!n || !n->value)
        return NULL;
    return node_wrap(pg_tensor_clone(n->value), false);
}

/* ---------------------------------------------------------------- grads */

pg_tensor *pga_grad_for_write(pg_node *n, int *beta)
{
    if (!n->grad) {
        n->grad = pgt_alloc(PG_DTYPE_F32, n->value->ndim, n->value->shape);
        *beta = 0;
        return n->grad;
    }
    /* a 16-bit copy kept with the grad no longer matches it (a writer that
     * also writes the copy marks it current after its launch) */
    if (n->grad->data_ref)
        n->grad->data_ref->shadow_stale = true;
    pgm_colsum_flush_for(n->grad); /* its deferred sums land first */
    if (n->grad->pg_flags & PG_TENSOR_ZERO_PENDING) {
        n->grad->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
        pgt_overwrite(n->grad);
        *beta = 0;
    } else {
        pgt_settle(n->grad); /* accumulating reads the current values */
        *beta = 1;
    }
    return n->grad;
}

/* dst grad (+)= scale * (g summed onto dst's shape) */
static void accum(pg_node *dst, const pg_tensor *g, float scale)
{
    if (!dst->requires_grad || !g)
        return;
    int beta;
    pg_tensor *dg = pga_grad_for_write(dst, &beta);
    if (!dg)
        return;
    pgk_bcast bc;
    memset(&bc, 0, sizeof bc);
    bc.ndim = (int)g->ndim;
    size_t off = g->ndim - dg->ndim;
    for (size_t d = 0; d < g->ndim; d++) {
        bc.shape[d] = (int64_t)g->shape[d];
        if (d < off)
            bc.sa[d] = 0;
        else
            bc.sa[d] = dg->shape[d - off] == 1 ? 0 : (int64_t)dg->stride[d - off];
    }
    pgd_check(pgk_reduce_into_f32((float *)dg->dev, dg->numel, (const float *)g->dev, &bc, scale, beta, pgd_stream()),
              "accum");
}

/* ---------------------------------------------------------------- elementwise forward */

static bool need_f32(const pg_tensor *t, const char *what)
{
    if (!t || !t->dev) {
        pga_set_err("%s: null tensor", what);
        return false;
    }
    if (t->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(t)) {
        pga_set_err("%s: needs a contiguous f32 tensor", what);
        return false;
    }
    pgt_materialize((pg_tensor *)t);
    return true;
}

/* broadcast (common.h:6-54 rules); strides of a and b over the out shape */
static bool bcast_desc(const pg_tensor *a, const pg_tensor *b, size_t *ond, size_t *oshape, pgk_bcast *bc)
{
    size_t nd = a->ndim > b->ndim ? a->ndim : b->ndim;
    for (size_t d = 0; d < nd; d++) {
        size_t da = d < nd - a->ndim ? 1 : a->shape[d - (nd - a->ndim)];
        size_t db = d < nd - b->ndim ? 1 : b->shape[d - (nd - b->ndim)];
        if (da != db && da != 1 && db != 1)
            return false;
        oshape[d] = da > db ? da : db;
    }
    *ond = nd;
    memset(bc, 0, sizeof *bc);
    bc->ndim = (int)nd;
    for (size_t d = 0; d < nd; d++) {
        bc->shape[d] = (int64_t)oshape[d];
        size_t ia = d - (nd - a->ndim), ib = d - (nd - b->ndim);
        bc->sa[d] = (d < nd - a->ndim || a->shape[ia] == 1) ? 0 : (int64_t)a->stride[ia];
        bc->sb[d] = (d < nd - b->ndim || b->shape[ib] == 1) ? 0 : (int64_t)b->stride[ib];
    }
    return true;
}

/* ---------------------------------------------------------------- deferred forward ops
 * With the JIT on, elementwise forward ops on f32 tensors are recorded
 * rather than launched.  Each gets its output allocated at once (the node's
 * value has its address and shape from the start), and the run of recorded
 * ops executes as ONE fused kernel that writes every op's output, when
 * anything else is about to be queued on the stream or waited on (the
 * device layer calls pga_lazy_flush at each such point: every launch,
 * copy, sync and upload).  The values are the eager kernels' bit for bit:
 * each op calls the same device function, and the fused body is compiled
 * without contracting one op's product into another's sum.  A run keeps one
 * output shape and at most 16 ops and 16 distinct inputs; a recorded op
 * holds a reference on its operands' and output's storage until it runs,
 * so freeing a node in between recycles nothing the run still touches. */
#define LZ_MAX 16

typedef struct {
    pg_data_ref *ref; /* one reference held while pending */
    void *dev;
    size_t ndim, shape[PG_MAX_NDIM];
} lz_tensor;

typedef struct {
    int code;  /* PG_JIT_* */
    int nin;
    int in[2]; /* >= 0: run input; < 0: -(k + 1) = output of op k */
    lz_tensor out;
    uint16_t *out16; /* with dt16: the output's 16-bit copy is written here too */
    int dt16;
} lz_op;

/* reduce_all over a run's output, recorded with the run when it is small
 * (pgj_small_reduce_fits): both reduction nodes' values come from the run's
 * one-block kernel */
typedef struct {
    bool on;
    int src; /* op index whose output is reduced */
    lz_tensor r1, r2;
    float scale;
} lz_red;

static struct {
    int nops, nin;
    lz_op op[LZ_MAX];
    lz_tensor in[LZ_MAX];
    size_t ndim, shape[PG_MAX_NDIM];
    lz_red red;
    bool flushing;
} g_lz;

bool pga_lazy_pending(void) { return g_lz.nops > 0; }

static int lz_unary_code(int pgk)
{
    switch (pgk) {
    case PGK_NEG: return PG_JIT_NEG;
    case PGK_EXP: return PG_JIT_EXP;
    case PGK_LOG: return PG_JIT_LOG;
    case PGK_SQRT: return PG_JIT_SQRT;
    case PGK_SIN: return PG_JIT_SIN;
    case PGK_COS: return PG_JIT_COS;
    case PGK_RELU: return PG_JIT_RELU;
    case PGK_SIGMOID: return PG_JIT_SIGMOID;
    case PGK_TANH: return PG_JIT_TANH;
    case PGK_GELU: return PG_JIT_GELU;
    case PGK_ERF: return PG_JIT_ERF;
    case PGK_ABS: return PG_JIT_ABS;
    default: return -1; /* parameterised ops run eagerly */
    }
}

static int lz_binary_code(int pgk)
{
    switch (pgk) {
    case PGK_ADD: return PG_JIT_ADD;
    case PGK_SUB: return PG_JIT_SUB;
    case PGK_MUL: return PG_JIT_MUL;
    case PGK_DIV: return PG_JIT_DIV;
    default: return -1;
    }
}

static void lz_hold(lz_tensor *d, pg_data_ref *ref, void *dev, size_t ndim, const size_t *shape)
{
    d->ref = ref;
    ref->refs++;
    d->dev = dev;
    d->ndim = ndim;
    memcpy(d->shape, shape, ndim * sizeof(size_t));
}

/* a stand-in tensor over a pending run's storage, for the launchers */
static void lz_view(pg_tensor *t, const lz_tensor *x)
{
    memset(t, 0, sizeof *t);
    t->ndim = x->ndim;
    memcpy(t->shape, x->shape, x->ndim * sizeof(size_t));
    pgt_set_contig_strides(t);
    t->numel = pg_shape_numel(x->ndim, x->shape);
    t->dtype = PG_DTYPE_F32;
    t->elem_size = 4;
    t->dev = x->dev;
    t->data_ref = x->ref;
}

static bool lz_same(const lz_tensor *x, const pg_tensor *t)
{
    return x->dev == t->dev && pg_shape_equal(x->ndim, x->shape, t->ndim, t->shape);
}

static bool lz_overlaps(const lz_tensor *x, const pg_tensor *t)
{
    const char *a = x->dev, *b = t->dev;
    const size_t na = pg_shape_numel(x->ndim, x->shape) * 4, nb = t->numel * t->elem_size;
    return a < b + nb && b < a + na;
}

/* where operand t comes from in the current run: op output (-(k+1)), run
 * input (>= 0), new input (LZ_MAX), or -LZ_MAX - 1 when it overlaps a
 * pending output without being one (the run must go first) */
static int lz_find(const pg_tensor *t)
{
    for (int k = 0; k < g_lz.nops; k++) {
        if (lz_same(&g_lz.op[k].out, t))
            return -(k + 1);
        if (lz_overlaps(&g_lz.op[k].out, t))
            return -LZ_MAX - 1;
    }
    for (int j = 0; j < g_lz.nin; j++)
        if (lz_same(&g_lz.in[j], t))
            return j;
    return LZ_MAX;
}

/* eager launch of recorded op k (when the fused kernel is unavailable) */
static bool lz_run_eager(int k)
{
    const lz_op *o = &g_lz.op[k];
    pg_tensor x[2], y;
    for (int i = 0; i < o->nin; i++)
        lz_view(&x[i], o->in[i] >= 0 ? &g_lz.in[o->in[i]] : &g_lz.op[-o->in[i] - 1].out);
    lz_view(&y, &o->out);
    if (o->nin == 1) {
        int code = -1;
        for (int c = 0; c < PGK_UNARY_COUNT && code < 0; c++)
            if (lz_unary_code(c) == o->code)
                code = c;
        return pgd_check(pgk_unary_f32(code, x[0].dev, y.dev, y.numel, 0.0f, 0.0f, pgd_stream()), "unary");
    }
    size_t nd, shp[PG_MAX_NDIM];
    pgk_bcast bc;
    if (!bcast_desc(&x[0], &x[1], &nd, shp, &bc))
        return false;
    return pgd_check(pgk_binary_f32(o->code - PG_JIT_ADD + PGK_ADD, x[0].dev, x[1].dev, y.dev, &bc, pgd_stream()),
                     "binary");
}

/* the run as one block with the pending uploads (and the recorded
 * reduction) folded in; g's inputs and outputs are the run's followed by
 * `nx_in` / `nx_out` more (x_in, x_out: a backward region merged into the
 * run).  False when it does not fit or fails to build, with nothing
 * launched and the uploads still pending */
static bool lz_run_small(pg_jit_graph *g, const void *const *x_in, size_t nx_in, void *const *x_out, size_t nx_out)
{
    size_t numel = pg_shape_numel(g_lz.ndim, g_lz.shape);
    if (numel > PGJ_SMALL_MAX)
        return false;
    if (g_lz.red.on && !pgj_small_reduce_fits(g_lz.ndim, g_lz.shape))
        return false;
    /* the pending uploads ride in the block when they fit it; otherwise
     * they stay in the batch, which the launch queues (one k_upload) ahead
     * of the block */
    pgk_upload up[PGK_UPLOAD_MAX];
    int nup = pgd_upload_take(up, PGK_UPLOAD_MAX);
    if (nup > 0 && !pgj_small_fits(numel, (size_t)nup, up)) {
        for (int i = 0; i < nup; i++) /* back to the batch, in order */
            pgd_upload_requeue(&up[i]);
        nup = 0;
    }
    if (nup < 0)
        nup = 0;
    const void *ip[2 * LZ_MAX + 32];
    void *op[2 * LZ_MAX + 32];
    size_t ni = 0, no = 0;
    for (int j = 0; j < g_lz.nin; j++)
        ip[ni++] = g_lz.in[j].dev;
    for (size_t j = 0; j < nx_in; j++)
        ip[ni++] = x_in[j];
    for (int k = 0; k < g_lz.nops; k++)
        op[no++] = g_lz.op[k].out.dev;
    for (size_t k = 0; k < nx_out; k++)
        op[no++] = x_out[k];
    bool ok = pgj_launch_small(g, g_lz.ndim, g_lz.shape, ip, ni, op, no, up, (size_t)nup,
                               g_lz.red.on ? g_lz.red.src : -1, g_lz.red.on ? g_lz.red.r1.dev : NULL,
                               g_lz.red.on ? g_lz.red.r2.dev : NULL, g_lz.red.scale);
    if (!ok)
        for (int i = 0; i < nup; i++)
            pgd_upload_requeue(&up[i]);
    return ok;
}

/* the run's graph: inputs idi[], one op per recorded op (ido[]), every op
 * an output; NULL on failure */
static pg_jit_graph *lz_graph(int *idi, int *ido)
{
    pg_jit_graph *g = pg_jit_graph_new();
    if (!g)
        return NULL;
    pgj_graph_set_exact(g);
    bool built = true;
    for (int j = 0; j < g_lz.nin && built; j++)
        built = (idi[j] = pg_jit_add_input(g, g_lz.in[j].ndim, g_lz.in[j].shape)) >= 0;
    for (int k = 0; k < g_lz.nops && built; k++) {
        int args[2];
        for (int i = 0; i < g_lz.op[k].nin; i++)
            args[i] = g_lz.op[k].in[i] >= 0 ? idi[g_lz.op[k].in[i]] : ido[-g_lz.op[k].in[i] - 1];
        built = (ido[k] = pg_jit_add_op(g, (pg_jit_op_t)g_lz.op[k].code, args, (size_t)g_lz.op[k].nin)) >= 0;
    }
    for (int k = 0; k < g_lz.nops && built; k++)
        pg_jit_mark_output(g, ido[k]);
    if (!built) {
        pg_jit_graph_free(g);
        return NULL;
    }
    return g;
}

/* the run has executed (or failed with its device error recorded): the
 * recorded reduction falls back to its own launch if the run's kernel did
 * not compute it, and every held reference is released */
static void lz_finish(bool ran, bool red_done)
{
    if (g_lz.red.on) {
        if (!red_done && ran)
            pgd_check(pgk_sum_all2_f32(g_lz.op[g_lz.red.src].out.dev, g_lz.red.r1.dev, g_lz.red.r2.dev,
                                       g_lz.shape[0], g_lz.shape[1], g_lz.red.scale, pgd_stream()),
                      "reduce");
        pgt_ref_release(g_lz.red.r1.ref);
        pgt_ref_release(g_lz.red.r2.ref);
        g_lz.red.on = false;
    }
    for (int j = 0; j < g_lz.nin; j++)
        pgt_ref_release(g_lz.in[j].ref);
    for (int k = 0; k < g_lz.nops; k++) {
        pgt_ref_release(g_lz.op[k].out.ref);
        g_lz.op[k].out16 = NULL;
        g_lz.op[k].dt16 = 0;
    }
    g_lz.nops = g_lz.nin = 0;
    g_lz.flushing = false;
}

/* set by pga_lazy_flush: the last run's fused kernel wrote the requested
 * 16-bit copies */
static bool g_lz_wrote16;

void pga_lazy_flush(void)
{
    if (!g_lz.nops || g_lz.flushing)
        return;
    g_lz.flushing = true;
    g_lz_wrote16 = false;
    bool ok = false, red_done = false;
    int idi[LZ_MAX], ido[LZ_MAX];
    pg_jit_graph *g = lz_graph(idi, ido);
    /* requested 16-bit copies: more outputs after the run's own */
    void *x16[LZ_MAX];
    size_t n16 = 0;
    for (int k = 0; k < g_lz.nops && g; k++)
        if (g_lz.op[k].out16) {
            pgj_mark_output16(g, ido[k], g_lz.op[k].dt16);
            x16[n16++] = g_lz.op[k].out16;
        }
    if (g && n16) {
        if (lz_run_small(g, NULL, 0, x16, n16)) {
            ok = red_done = true;
        } else {
            const void *ip[LZ_MAX];
            void *op[2 * LZ_MAX];
            size_t no = 0;
            for (int j = 0; j < g_lz.nin; j++)
                ip[j] = g_lz.in[j].dev;
            for (int k = 0; k < g_lz.nops; k++)
                op[no++] = g_lz.op[k].out.dev;
            for (size_t k = 0; k < n16; k++)
                op[no++] = x16[k];
            ok = pgj_launch(g, g_lz.ndim, g_lz.shape, ip, (size_t)g_lz.nin, op, no);
        }
        g_lz_wrote16 = ok;
        pg_jit_graph_free(g);
        g = NULL;
    }
    if (g) {
        if (lz_run_small(g, NULL, 0, NULL, 0))
            ok = red_done = true;
        pg_jit_exe *exe = !ok ? pg_jit_compile(g) : NULL;
        if (exe) {
            pg_tensor tin[LZ_MAX], tout[LZ_MAX];
            const pg_tensor *pin[LZ_MAX];
            pg_tensor *pout[LZ_MAX];
            for (int j = 0; j < g_lz.nin; j++) {
                lz_view(&tin[j], &g_lz.in[j]);
                pin[j] = &tin[j];
            }
            for (int k = 0; k < g_lz.nops; k++) {
                lz_view(&tout[k], &g_lz.op[k].out);
                pout[k] = &tout[k];
            }
            ok = pg_jit_run(exe, pin, (size_t)g_lz.nin, pout, (size_t)g_lz.nops);
            pg_jit_exe_free(exe);
        }
        pg_jit_graph_free(g);
    }
    bool eager_ok = true;
    for (int k = 0; k < g_lz.nops && !ok; k++)
        if (!(eager_ok = lz_run_eager(k))) /* the device error is recorded; the rest are not run */
            break;
    lz_finish(eager_ok, red_done);
}

static bool g_copies16 = true;
void pg_amd_jit_copies16(bool on) { g_copies16 = on; }
bool pga_copies16(void) { return g_copies16; }

bool pga_lazy_shadow16(const pg_tensor *t, int dt, uint16_t *dst)
{
    if (!g_copies16 || !g_lz.nops || g_lz.flushing || !t || !dst)
        return false;
    int k = lz_find(t);
    if (k >= 0 || k == -LZ_MAX - 1)
        return false; /* not an op's output */
    k = -k - 1;
    g_lz.op[k].out16 = dst;
    g_lz.op[k].dt16 = dt;
    pga_lazy_flush();
    return g_lz_wrote16;
}

static bool lz_overlaps_ptr(const lz_tensor *x, const void *p, size_t nbytes)
{
    const char *a = x->dev, *b = p;
    const size_t na = pg_shape_numel(x->ndim, x->shape) * 4;
    return a < b + nbytes && b < a + na;
}

/* A fused backward region (graph bwd over the loop shape (lnd, ls),
 * inputs bin[], full-shape outputs bout[]) executed in the same one-block
 * kernel as the pending small run, after the run's values in each element
 * (one launch instead of two: config 1's leaves, forward, reduction and
 * backward).  bwd's inputs that are run inputs or outputs read those
 * values; its outputs (the grads) must not overlap the run's tensors.  The
 * merged body is compiled without FMA contraction, as the run is.  True
 * when the merged kernel was launched (the run is then done); false with
 * nothing launched and the run still pending otherwise. */
bool pga_lazy_flush_with_backward(const pg_jit_graph *bwd, size_t lnd, const size_t *ls, const void *const *bin,
                                  size_t bnin, void *const *bout, size_t bnout)
{
    if (!g_lz.nops || g_lz.flushing || !pg_shape_equal(lnd, ls, g_lz.ndim, g_lz.shape) ||
        pg_shape_numel(lnd, ls) > PGJ_SMALL_MAX || bnin > 32 || bnout > 32)
        return false;
    const size_t obytes = pg_shape_numel(lnd, ls) * 4;
    for (size_t o = 0; o < bnout; o++) {
        for (int j = 0; j < g_lz.nin; j++)
            if (lz_overlaps_ptr(&g_lz.in[j], bout[o], obytes))
                return false;
        for (int k = 0; k < g_lz.nops; k++)
            if (lz_overlaps_ptr(&g_lz.op[k].out, bout[o], obytes))
                return false;
        if (g_lz.red.on && (lz_overlaps_ptr(&g_lz.red.r1, bout[o], obytes) ||
                            lz_overlaps_ptr(&g_lz.red.r2, bout[o], obytes)))
            return false;
    }
    int idi[LZ_MAX], ido[LZ_MAX];
    pg_jit_graph *g = lz_graph(idi, ido);
    if (!g)
        return false;
    /* bwd's inputs: a run output or input with the same address and shape,
     * else a new input of the merged kernel (one overlapping a run tensor
     * otherwise cannot be read in the same pass) */
    int in_map[32];
    const void *x_in[32];
    size_t nx = 0;
    bool ok = true;
    for (size_t i = 0; i < bnin && ok; i++) {
        size_t nd;
        const size_t *sh;
        ok = pgj_input_shape(bwd, i, &nd, &sh);
        if (!ok)
            break;
        const size_t nb = pg_shape_numel(nd, sh) * 4;
        in_map[i] = -1;
        for (int k = 0; k < g_lz.nops && in_map[i] < 0 && ok; k++) {
            const lz_tensor *x = &g_lz.op[k].out;
            if (x->dev == bin[i] && pg_shape_equal(x->ndim, x->shape, nd, sh))
                in_map[i] = ido[k];
            else if (lz_overlaps_ptr(x, bin[i], nb))
                ok = false;
        }
        for (int j = 0; j < g_lz.nin && in_map[i] < 0 && ok; j++) {
            const lz_tensor *x = &g_lz.in[j];
            if (x->dev == bin[i] && pg_shape_equal(x->ndim, x->shape, nd, sh))
                in_map[i] = idi[j];
        }
        if (ok && in_map[i] < 0) {
            if (g_lz.nin + nx >= 2 * LZ_MAX) {
                ok = false;
                break;
            }
            ok = (in_map[i] = pg_jit_add_input(g, nd, sh)) >= 0;
            x_in[nx++] = bin[i];
        }
    }
    ok = ok && pgj_graph_append(g, bwd, in_map, lnd, ls);
    if (ok) {
        g_lz.flushing = true;
        ok = lz_run_small(g, x_in, nx, bout, bnout);
        g_lz.flushing = false;
        if (ok)
            lz_finish(true, true);
    }
    pg_jit_graph_free(g);
    return ok;
}

/* reduce_all's two values from the pending run when t is one of its
 * outputs and the run is small: the reduction is recorded and computed by
 * the run's kernel.  False (nothing recorded) otherwise. */
static bool lz_record_reduce_all(const pg_tensor *t, bool mean, pg_tensor **v1, pg_tensor **v2)
{
    if (!g_lz.nops || g_lz.red.on || g_lz.flushing || !pg_autograd_is_jit_enabled() || t->ndim != 2 ||
        !pg_shape_equal(t->ndim, t->shape, g_lz.ndim, g_lz.shape) || !pgj_small_reduce_fits(t->ndim, t->shape) ||
        pg_shape_numel(t->ndim, t->shape) > PGJ_SMALL_MAX)
        return false;
    int src = lz_find(t);
    if (src >= 0 || src <= -LZ_MAX - 1)
        return false;
    const size_t cols = t->shape[1];
    *v1 = pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){cols});
    *v2 = *v1 ? pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){1}) : NULL;
    if (!*v2) {
        pg_tensor_free(*v1);
        *v1 = NULL;
        return false;
    }
    g_lz.red.src = -src - 1;
    g_lz.red.scale = mean ? 1.0f / (float)cols : 1.0f;
    lz_hold(&g_lz.red.r1, (*v1)->data_ref, (*v1)->dev, 1, (*v1)->shape);
    lz_hold(&g_lz.red.r2, (*v2)->data_ref, (*v2)->dev, 1, (*v2)->shape);
    g_lz.red.on = true;
    return true;
}

/* records y = op(x...) into the run; NULL when the op must run eagerly
 * (nothing recorded then) */
static pg_tensor *lz_record(int code, int nin, const pg_tensor *const *x, size_t nd, const size_t *shape)
{
    if (code < 0 || !pg_autograd_is_jit_enabled() || g_lz.flushing)
        return NULL;
    if (g_lz.nops && (g_lz.nops == LZ_MAX || g_lz.red.on || !pg_shape_equal(nd, shape, g_lz.ndim, g_lz.shape)))
        pga_lazy_flush();
    int src[2], fresh = 0;
    for (int i = 0; i < nin; i++) {
        src[i] = lz_find(x[i]);
        if (src[i] == -LZ_MAX - 1) {
            pga_lazy_flush();
            return lz_record(code, nin, x, nd, shape);
        }
        fresh += src[i] == LZ_MAX && !(i == 1 && x[1] == x[0]) ? 1 : 0;
    }
    if (g_lz.nin + fresh > LZ_MAX) {
        pga_lazy_flush();
        return lz_record(code, nin, x, nd, shape);
    }
    pg_tensor *y = pgt_alloc(PG_DTYPE_F32, nd, shape);
    if (!y)
        return NULL;
    if (!g_lz.nops) {
        g_lz.ndim = nd;
        memcpy(g_lz.shape, shape, nd * sizeof(size_t));
    }
    lz_op *o = &g_lz.op[g_lz.nops];
    o->code = code;
    o->nin = nin;
    for (int i = 0; i < nin; i++) {
        if (src[i] == LZ_MAX) {
            if (i == 1 && x[1] == x[0]) {
                src[1] = src[0];
            } else {
                lz_hold(&g_lz.in[g_lz.nin], x[i]->data_ref, x[i]->dev, x[i]->ndim, x[i]->shape);
                src[i] = g_lz.nin++;
            }
        }
        o->in[i] = src[i];
    }
    lz_hold(&o->out, y->data_ref, y->dev, nd, shape);
    g_lz.nops++;
    return y;
}

pg_tensor *pga_binary_fwd(int op, const pg_tensor *a, const pg_tensor *b)
{
    if (!need_f32(a, "binary op") || !need_f32(b, "binary op"))
        return NULL;
    size_t nd, shp[PG_MAX_NDIM];
    pgk_bcast bc;
    if (!bcast_desc(a, b, &nd, shp, &bc)) {
        pga_set_err("binary op: incompatible broadcast shapes");
        return NULL;
    }
    pg_tensor *y = lz_record(lz_binary_code(op), 2, (const pg_tensor *[]){a, b}, nd, shp);
    if (y)
        return y;
    y = pgt_alloc(PG_DTYPE_F32, nd, shp);
    if (!y)
        return NULL;
    if (!pgd_check(pgk_binary_f32(op, (const float *)a->dev, (const float *)b->dev, (float *)y->dev, &bc,
                                  pgd_stream()),
                   "binary")) {
        pg_tensor_free(y);
        return NULL;
    }
    return y;
}

pg_tensor *pga_unary_fwd(int op, const pg_tensor *a, float p0, float p1)
{
    if (!need_f32(a, "unary op"))
        return NULL;
    pg_tensor *y = lz_record(lz_unary_code(op), 1, (const pg_tensor *[]){a}, a->ndim, a->shape);
    if (y)
        return y;
    y = pgt_alloc(PG_DTYPE_F32, a->ndim, a->shape);
    if (!y)
        return NULL;
    if (!pgd_check(pgk_unary_f32(op, (const float *)a->dev, (float *)y->dev, a->numel, p0, p1, pgd_stream()),
                   "unary")) {
        pg_tensor_free(y);
        return NULL;
    }
    return y;
}

/* ---------------------------------------------------------------- eager backward */

/* dst (+)= scale * reduce_to_dst( g OP other ) via a temp of g's shape */
static void accum_binary(pg_node *dst, const pg_tensor *g, int op, const pg_tensor *other, float scale)
{
    if (!dst->requires_grad)
        return;
    size_t nd, shp[PG_MAX_NDIM];
    pgk_bcast bc;
    if (!bcast_desc(g, other, &nd, shp, &bc))
        return;
    pg_tensor *t = pgt_alloc(PG_DTYPE_F32, nd, shp);
    if (!t)
        return;
    pgk_binary_f32(op, (const float *)g->dev, (const float *)other->dev, (float *)t->dev, &bc, pgd_stream());
    accum(dst, t, scale);
    pg_tensor_free(t);
}

static void bwd_add(pg_node *n)
{
    accum(n->parents[0], n->grad, 1.0f);
    accum(n->parents[1], n->grad, 1.0f);
}

static void bwd_sub(pg_node *n)
{
    accum(n->parents[0], n->grad, 1.0f);
    accum(n->parents[1], n->grad, -1.0f);
}

static void bwd_mul(pg_node *n)
{
    accum_binary(n->parents[0], n->grad, PGK_MUL, n->parents[1]->value, 1.0f);
    accum_binary(n->parents[1], n->grad, PGK_MUL, n->parents[0]->value, 1.0f);
}

static void bwd_div(pg_node *n)
{
    pg_node *pa = n->parents[0], *pb = n->parents[1];
    const pg_tensor *g = n->grad;
    accum_binary(pa, g, PGK_DIV, pb->value, 1.0f);
    if (pb->requires_grad) {
        /* -(g * a) / (b * b)  (autograd.c:497-509) */
        pg_tensor *d = pga_binary_fwd(PGK_MUL, pb->value, pb->value);
        pg_tensor *num = d ? pga_binary_fwd(PGK_MUL, g, pa->value) : NULL;
        pg_tensor *t = num ? pga_binary_fwd(PGK_DIV, num, d) : NULL;
        if (t)
            accum(pb, t, -1.0f);
        pg_tensor_free(d);
        pg_tensor_free(num);
        pg_tensor_free(t);
    }
}

static void bwd_neg(pg_node *n) { accum(n->parents[0], n->grad, -1.0f); }

static int unary_code(pg_ag_op_t op)
{
    switch (op) {
    case PG_AG_OP_EXP: return PGK_EXP;
    case PG_AG_OP_LOG: return PGK_LOG;
    case PG_AG_OP_SQRT: return PGK_SQRT;
    case PG_AG_OP_SIN: return PGK_SIN;
    case PG_AG_OP_COS: return PGK_COS;
    case PG_AG_OP_RELU: return PGK_RELU;
    case PG_AG_OP_SIGMOID: return PGK_SIGMOID;
    case PG_AG_OP_TANH: return PGK_TANH;
    case PG_AG_OP_GELU: return PGK_GELU;
    case PG_AG_OP_ERF: return PGK_ERF;
    case PG_AG_OP_ABS: return PGK_ABS;
    case PG_AG_OP_LEAKY_RELU: return PGK_LEAKY;
    case PG_AG_OP_CLAMP: return PGK_CLAMP;
    default: return -1;
    }
}

static void bwd_unary(pg_node *n)
{
    pg_node *p = n->parents[0];
    if (!p->requires_grad)
        return;
    int beta;
    pg_tensor *dg = pga_grad_for_write(p, &beta);
    if (!dg)
        return;
    float p0 = 0, p1 = 0;
    if (n->ctx) {
        p0 = ((pga_param_ctx *)n->ctx)->p0;
        p1 = ((pga_param_ctx *)n->ctx)->p1;
    }
    pgd_check(pgk_unary_bwd_f32(unary_code(n->ag_op), (const float *)n->grad->dev, (const float *)p->value->dev,
                                (float *)dg->dev, dg->numel, p0, p1, 1.0f, beta, pgd_stream()),
              "unary backward");
}

static void bwd_reduce(pg_node *n)
{
    pg_node *p = n->parents[0];
    if (!p->requires_grad)
        return;
    pga_red_ctx *cx = n->ctx;
    const pg_tensor *like = p->value, *g = n->grad;
    float scale = n->ag_op == PG_AG_OP_MEAN ? 1.0f / (float)like->shape[cx->axis] : 1.0f;
    pgk_bcast bc;
    memset(&bc, 0, sizeof bc);
    bc.ndim = (int)like->ndim;
    for (size_t d = 0; d < like->ndim; d++) {
        bc.shape[d] = (int64_t)like->shape[d];
        if (d == cx->axis) {
            bc.sa[d] = 0;
            continue;
        }
        size_t gd = cx->keepdim ? d : (d < cx->axis ? d : d - 1);
        bc.sa[d] = (int64_t)g->stride[gd];
    }
    int beta;
    pg_tensor *dg = pga_grad_for_write(p, &beta);
    if (!dg)
        return;
    pgd_check(pgk_expand_into_f32((float *)dg->dev, (const float *)g->dev, &bc, scale, beta, pgd_stream()),
              "reduce backward");
}

void pga_backward_node(pg_node *n)
{
    if (n->backward && n->grad)
        n->backward(n);
}

/* ---------------------------------------------------------------- op wrappers */

#define BINARY_AG(name, code, bwd, agop)                                                                          \
    pg_node *name(pg_node *a, pg_node *b)                                                                         \
    {                                                                                                             \
        if (!a || !b || !a->value || !b->value) {                                                                 \
            pga_set_err(#name ": null operand");                                                                  \
            return NULL;                                                                                          \
        }                                                                                                         \
        pg_tensor *v = pga_binary_fwd(code, a->value, b->value);                                                  \
        return v ? attach(v, 2, (pg_node *[]){a, b}, bwd, NULL, agop) : NULL;                                     \
    }

BINARY_AG(pg_ag_add, PGK_ADD, bwd_add, PG_AG_OP_ADD)
BINARY_AG(pg_ag_sub, PGK_SUB, bwd_sub, PG_AG_OP_SUB)
BINARY_AG(pg_ag_mul, PGK_MUL, bwd_mul, PG_AG_OP_MUL)
BINARY_AG(pg_ag_div, PGK_DIV, bwd_div, PG_AG_OP_DIV)

static pg_node *unary_ag(pg_node *a, int code, pg_ag_op_t op, void (*bwd)(pg_node *), float p0, float p1,
                         bool with_ctx)
{
    if (!a || !a->value) {
        pga_set_err("unary op: null operand");
        return NULL;
    }
    pg_tensor *v = pga_unary_fwd(code, a->value, p0, p1);
    if (!v)
        return NULL;
    pga_param_ctx *cx = NULL;
    if (with_ctx) {
        cx = malloc(sizeof *cx);
        if (!cx) {
            pg_tensor_free(v);
            return NULL;
        }
        cx->p0 = p0;
        cx->p1 = p1;
    }
    return attach(v, 1, &a, bwd, cx, op);
}

pg_node *pg_ag_neg(pg_node *a) { return unary_ag(a, PGK_NEG, PG_AG_OP_NEG, bwd_neg, 0, 0, false); }
pg_node *pg_ag_exp(pg_node *a) { return unary_ag(a, PGK_EXP, PG_AG_OP_EXP, bwd_unary, 0, 0, false); }
pg_node *pg_ag_log(pg_node *a) { return unary_ag(a, PGK_LOG, PG_AG_OP_LOG, bwd_unary, 0, 0, false); }
pg_node *pg_ag_sqrt(pg_node *a) { return unary_ag(a, PGK_SQRT, PG_AG_OP_SQRT, bwd_unary, 0, 0, false); }
pg_node *pg_ag_sin(pg_node *a) { return unary_ag(a, PGK_SIN, PG_AG_OP_SIN, bwd_unary, 0, 0, false); }
pg_node *pg_ag_cos(pg_node *a) { return unary_ag(a, PGK_COS, PG_AG_OP_COS, bwd_unary, 0, 0, false); }
pg_node *pg_ag_relu(pg_node *a) { return unary_ag(a, PGK_RELU, PG_AG_OP_RELU, bwd_unary, 0, 0, false); }
pg_node *pg_ag_sigmoid(pg_node *a) { return unary_ag(a, PGK_SIGMOID, PG_AG_OP_SIGMOID, bwd_unary, 0, 0, false); }
pg_node *pg_ag_tanh(pg_node *a) { return unary_ag(a, PGK_TANH, PG_AG_OP_TANH, bwd_unary, 0, 0, false); }
pg_node *pg_ag_gelu(pg_node *a) { return unary_ag(a, PGK_GELU, PG_AG_OP_GELU, bwd_unary, 0, 0, false); }
pg_node *pg_ag_erf(pg_node *a) { return unary_ag(a, PGK_ERF, PG_AG_OP_ERF, bwd_unary, 0, 0, false); }
pg_node *pg_ag_abs(pg_node *a) { return unary_ag(a, PGK_ABS, PG_AG_OP_ABS, bwd_unary, 0, 0, false); }
pg_node *pg_ag_leaky_relu(pg_node *a, float alpha)
{
    return unary_ag(a, PGK_LEAKY, PG_AG_OP_LEAKY_RELU, bwd_unary, alpha, 0, true);
}
pg_node *pg_ag_clamp(pg_node *a, float lo, float hi)
{
    if (lo > hi) {
        pga_set_err("clamp: lo > hi");
        return NULL;
    }
    return unary_ag(a, PGK_CLAMP, PG_AG_OP_CLAMP, bwd_unary, lo, hi, true);
}

pg_node *pg_ag_matmul(pg_node *a, pg_node *b)
{
    if (!a || !b || !a->value || !b->value) {
        pga_set_err("matmul: null operand");
        return NULL;
    }
    pg_tensor *v = pgm_matmul_forward(a->value, b->value);
    return v ? attach(v, 2, (pg_node *[]){a, b}, pgm_matmul_backward, NULL, PG_AG_OP_MATMUL) : NULL;
}

/* the reduce node over a computed value v (v is the node's or freed) */
static pg_node *reduce_attach(pg_node *a, size_t axis, bool keepdim, bool mean, pg_tensor *v)
{
    pga_red_ctx *cx = malloc(sizeof *cx);
    if (!cx) {
        pg_tensor_free(v);
        return NULL;
    }
    cx->axis = axis;
    cx->keepdim = keepdim;
    return attach(v, 1, &a, bwd_reduce, cx, mean ? PG_AG_OP_MEAN : PG_AG_OP_SUM);
}

/* reduce.c:90-110 output shape: axis kept as 1 or removed; never 0-d */
static pg_node *ag_reduce(pg_node *a, size_t axis, bool keepdim, bool mean)
{
    if (!a || !a->value || a->value->ndim < 1 || axis >= a->value->ndim) {
        pga_set_err("reduce: bad axis");
        return NULL;
    }
    const pg_tensor *t = a->value;
    if (!need_f32(t, "reduce"))
        return NULL;
    size_t shp[PG_MAX_NDIM], nd = 0;
    for (size_t d = 0; d < t->ndim; d++) {
        if (d == axis) {
            if (keepdim)
                shp[nd++] = 1;
        } else {
            shp[nd++] = t->shape[d];
        }
    }
    if (nd == 0)
        shp[nd++] = 1;
    size_t outer = 1, inner = 1, len = t->shape[axis];
    for (size_t d = 0; d < axis; d++)
        outer *= t->shape[d];
    for (size_t d = axis + 1; d < t->ndim; d++)
        inner *= t->shape[d];
    pg_tensor *v = pgt_alloc(PG_DTYPE_F32, nd, shp);
    if (!v)
        return NULL;
    float scale = mean ? 1.0f / (float)len : 1.0f;
    size_t wsz = pgk_sum_axis_workspace(outer, len, inner);
    void *ws = wsz ? pgd_scratch(2, wsz) : NULL;
    if ((wsz && !ws) ||
        !pgd_check(pgk_sum_axis_f32((const float *)t->dev, (float *)v->dev, outer, len, inner, scale, ws,
                                    pgd_stream()),
                   "reduce")) {
        pg_tensor_free(v);
        return NULL;
    }
    return reduce_attach(a, axis, keepdim, mean, v);
}

pg_node *pg_ag_sum(pg_node *a, size_t axis, bool keepdim) { return ag_reduce(a, axis, keepdim, false); }
pg_node *pg_ag_mean(pg_node *a, size_t axis, bool keepdim) { return ag_reduce(a, axis, keepdim, true); }

/* reduce_all (autograd.c:1018-1043): sum axis 0 until one axis is left, then
 * sum or mean over it -- so mean_all divides by the last axis only */
static pg_node *reduce_all(pg_node *a, bool mean)
{
    if (!a || !a->value || a->value->ndim < 1) {
        pga_set_err("reduce_all: bad operand");
        return NULL;
    }
    const pg_tensor *t = a->value;
    if (t->ndim == 2 && pgk_sum_all2_fits(t->shape[0], t->shape[1])) {
        /* both nodes' values from one launch, the same sums in the same
         * order: the pending run's kernel when t is its output, else
         * pgk_sum_all2_f32 */
        if (!t->dev || t->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(t)) {
            pga_set_err("reduce: needs a contiguous f32 tensor");
            return NULL;
        }
        const size_t cols = t->shape[1];
        pg_tensor *v1 = NULL, *v2 = NULL;
        if (!lz_record_reduce_all(t, mean, &v1, &v2)) {
            if (!need_f32(t, "reduce"))
                return NULL;
            v1 = pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){cols});
            v2 = v1 ? pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){1}) : NULL;
            if (!v2 || !pgd_check(pgk_sum_all2_f32((const float *)t->dev, (float *)v1->dev, (float *)v2->dev,
                                                   t->shape[0], cols, mean ? 1.0f / (float)cols : 1.0f,
                                                   pgd_stream()),
                                  "reduce")) {
                pg_tensor_free(v1);
                pg_tensor_free(v2);
                return NULL;
            }
        }
        pg_node *n1 = reduce_attach(a, 0, false, false, v1);
        if (!n1) {
            pg_tensor_free(v2);
            return NULL;
        }
        pg_node *out = reduce_attach(n1, 0, false, mean, v2);
        pg_node_free(n1);
        return out;
    }
    if (t->ndim == 2 && pgk_sum_all2s_fits(t->shape[0], t->shape[1])) {
        /* sliced column sums: the same sums in the same order as the
         * pg_ag_sum / pg_ag_mean chain below, from one launch */
        if (!need_f32(t, "reduce"))
            return NULL;
        const size_t cols = t->shape[1];
        pg_tensor *v1 = pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){cols});
        pg_tensor *v2 = v1 ? pgt_alloc(PG_DTYPE_F32, 1, (size_t[]){1}) : NULL;
        if (!v2 || !pgd_check(pgk_sum_all2s_f32((const float *)t->dev, (float *)v1->dev, (float *)v2->dev,
                                                t->shape[0], cols, mean ? 1.0f / (float)cols : 1.0f,
                                                pgd_stream()),
                              "reduce")) {
            pg_tensor_free(v1);
            pg_tensor_free(v2);
            return NULL;
        }
        pg_node *n1 = reduce_attach(a, 0, false, false, v1);
        if (!n1) {
            pg_tensor_free(v2);
            return NULL;
        }
        pg_node *out = reduce_attach(n1, 0, false, mean, v2);
        pg_node_free(n1);
        return out;
    }
    pg_node *cur = pg_node_retain(a);
    for (size_t d = a->value->ndim; d > 1; d--) {
        pg_node *nx = pg_ag_sum(cur, 0, false);
        pg_node_free(cur);
        if (!nx)
            return NULL;
        cur = nx;
    }
    pg_node *out = mean ? pg_ag_mean(cur, 0, false) : pg_ag_sum(cur, 0, false);
    pg_node_free(cur);
    return out;
}

pg_node *pg_ag_sum_all(pg_node *a) { return reduce_all(a, false); }
pg_node *pg_ag_mean_all(pg_node *a) { return reduce_all(a, true); }

/* autograd.c:1758-1771 */
pg_node *pg_ag_mse(pg_node *pred, pg_node *target, bool mean)
{
    if (!pred || !target) {
        pga_set_err("mse: null operand");
        return NULL;
    }
    pg_node *d = pg_ag_sub(pred, target);
    if (!d)
        return NULL;
    pg_node *sq = pg_ag_mul(d, d);
    pg_node_free(d);
    if (!sq)
        return NULL;
    pg_node *loss = mean ? pg_ag_mean_all(sq) : pg_ag_sum_all(sq);
    pg_node_free(sq);
    return loss;
}

/* ---------------------------------------------------------------- not in this build */

static pg_node *unsupported(const char *what)
{
    pga_set_err("%s is not part of the MI355X build", what);
    return NULL;
}

pg_node *pg_ag_pow(pg_node *a, pg_node *b) { (void)a; (void)b; return unsupported("pg_ag_pow"); }
pg_node *pg_ag_softmax(pg_node *a, size_t axis) { (void)a; (void)axis; return unsupported("pg_ag_softmax"); }
pg_node *pg_ag_transpose(pg_node *a, size_t x, size_t y) { (void)a; (void)x; (void)y; return unsupported("pg_ag_transpose"); }
pg_node *pg_ag_layernorm(pg_node *x, pg_node *w, pg_node *b, float e) { (void)x; (void)w; (void)b; (void)e; return unsupported("pg_ag_layernorm"); }
pg_node *pg_ag_rmsnorm(pg_node *x, pg_node *w, float e) { (void)x; (void)w; (void)e; return unsupported("pg_ag_rmsnorm"); }
pg_node *pg_ag_batchnorm(pg_node *x, pg_node *w, pg_node *b, float e) { (void)x; (void)w; (void)b; (void)e; return unsupported("pg_ag_batchnorm"); }
pg_node *pg_ag_batchnorm2d(pg_node *x, pg_node *w, pg_node *b, pg_tensor *rm, pg_tensor *rv, float e, float m, bool t)
{
    (void)x; (void)w; (void)b; (void)rm; (void)rv; (void)e; (void)m; (void)t;
    return unsupported("pg_ag_batchnorm2d");
}
pg_node *pg_ag_conv2d(pg_node *x, pg_node *w, pg_node *b, size_t kh, size_t kw, int s, int p)
{
    (void)x; (void)w; (void)b; (void)kh; (void)kw; (void)s; (void)p;
    return unsupported("pg_ag_conv2d");
}
pg_node *pg_ag_embedding(pg_node *w, const pg_tensor *i) { (void)w; (void)i; return unsupported("pg_ag_embedding"); }
pg_node *pg_ag_dropout(pg_node *x, float p, bool t) { (void)x; (void)p; (void)t; return unsupported("pg_ag_dropout"); }
pg_node *pg_ag_cross_entropy(pg_node *l, const size_t *t, size_t n, bool m) { (void)l; (void)t; (void)n; (void)m; return unsupported("pg_ag_cross_entropy"); }
pg_node *pg_ag_bce_with_logits(pg_node *l, const float *t, size_t n, bool m) { (void)l; (void)t; (void)n; (void)m; return unsupported("pg_ag_bce_with_logits"); }
