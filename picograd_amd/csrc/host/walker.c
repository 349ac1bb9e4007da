/*
 * pg_backward: the graph walk (reference autograd/autograd.c:1854-2533).
 *
 * Kept from the reference: the iterative DFS topological order
 * (topo_sort, :1854-1913), grads zeroed at the start of every backward
 * (:2490-2492), the SUM/MEAN chain above the loss folded into one scalar
 * (:1971-2010), the fused-kernel chain rule of :2166-2297, eager per-node
 * backward for the rest, and the jit hit/fallback counters (:2514-2519).
 *
 * MI355X design:
 *  - every grad is a device tensor.  "Zeroed" is a flag (PG_TENSOR_ZERO_PENDING):
 *    the first kernel that writes a grad overwrites it (beta 0), later
 *    contributions accumulate in place (beta 1), and a grad nobody wrote
 *    is filled with zeros once at the end;
 *  - fusion covers every maximal region of elementwise f32 nodes of one
 *    loop shape, not only the chain under the loss: a region is grown from
 *    a root towards its inputs, taking a parent only when all of that
 *    parent's consumers are already in the region, so its grad is complete
 *    inside the kernel.  (The reference takes suffix nodes regardless and
 *    loses the grad a suffix node receives from a consumer outside the
 *    suffix.)  GELU, ERF and ABS are fusible too;
 *  - forward values a region needs are recomputed from the region's
 *    inputs rather than loaded, so a region reads each input tensor once;
 *  - grads of region inputs broadcast over rows (biases) are reduced in the
 *    same kernel; the upstream scalar of the loss is a kernel constant.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <stdlib.h>
#include <string.h>

static bool g_jit_enabled = true;
static bool g_last_was_jit;
static size_t g_jit_hits, g_jit_fallbacks;

void pg_autograd_set_jit(bool enabled) { g_jit_enabled = enabled; }
bool pg_autograd_is_jit_enabled(void) { return g_jit_enabled; }
bool pg_autograd_last_was_jit(void) { return g_last_was_jit; }
size_t pg_autograd_jit_hits(void) { return g_jit_hits; }
size_t pg_autograd_jit_fallbacks(void) { return g_jit_fallbacks; }

/* ---------------------------------------------------------------- order */

typedef struct {
    pg_node **v;
    size_t n, cap;
} nvec;

static bool nv_push(nvec *a, pg_node *x)
{
    if (a->n == a->cap) {
        size_t nc = a->cap ? a->cap * 2 : 32;
        pg_node **p = realloc(a->v, nc * sizeof *p);
        if (!p)
            return false;
        a->v = p;
        a->cap = nc;
    }
    a->v[a->n++] = x;
    return true;
}

/* post-order DFS over parents that require grad (autograd.c:1854-1913);
 * `mark` holds 1 + the node's index in the order while the walk runs */
static bool topo(pg_node *root, nvec *order)
{
    typedef struct {
        pg_node *n;
        size_t i;
    } frame;
    size_t cap = 32, sp = 0;
    frame *stk = malloc(cap * sizeof *stk);
    if (!stk)
        return false;
    root->mark = 1;
    stk[sp++] = (frame){root, 0};
    while (sp) {
        frame *f = &stk[sp - 1];
        if (f->i < f->n->nparents) {
            pg_node *c = f->n->parents[f->i++];
            if (c->requires_grad && !c->mark) {
                c->mark = 1;
                if (sp == cap) {
                    cap *= 2;
                    frame *ns = realloc(stk, cap * sizeof *ns);
                    if (!ns) {
                        free(stk);
                        return false;
                    }
                    stk = ns;
                }
                stk[sp++] = (frame){c, 0};
            }
        } else {
            nv_push(order, f->n);
            sp--;
        }
    }
    free(stk);
    return true;
}

/* index lookup: nodes of the order carry a side table via a small hash */
typedef struct {
    pg_node **keys;
    int *vals;
    size_t cap;
} nmap;

static size_t nm_slot(const nmap *m, const pg_node *k)
{
    size_t h = ((uintptr_t)k >> 4) * 11400714819323198485ull;
    return h & (m->cap - 1);
}

static bool nm_init(nmap *m, size_t n)
{
    m->cap = 16;
    while (m->cap < 2 * n + 2)
        m->cap <<= 1;
    m->keys = calloc(m->cap, sizeof *m->keys);
    m->vals = calloc(m->cap, sizeof *m->vals);
    return m->keys && m->vals;
}

static void nm_put(nmap *m, pg_node *k, int v)
{
    size_t s = nm_slot(m, k);
    while (m->keys[s] && m->keys[s] != k)
        s = (s + 1) & (m->cap - 1);
    m->keys[s] = k;
    m->vals[s] = v;
}

static int nm_get(const nmap *m, const pg_node *k)
{
    size_t s = nm_slot(m, k);
    while (m->keys[s]) {
        if (m->keys[s] == k)
            return m->vals[s];
        s = (s + 1) & (m->cap - 1);
    }
    return -1;
}

static void nm_free(nmap *m)
{
    free(m->keys);
    free(m->vals);
}

/* ---------------------------------------------------------------- fusion */

bool pga_op_fusible(pg_ag_op_t op)
{
    switch (op) {
    case PG_AG_OP_ADD: case PG_AG_OP_SUB: case PG_AG_OP_MUL: case PG_AG_OP_DIV:
    case PG_AG_OP_NEG: case PG_AG_OP_EXP: case PG_AG_OP_LOG: case PG_AG_OP_SQRT:
    case PG_AG_OP_SIN: case PG_AG_OP_COS: case PG_AG_OP_RELU: case PG_AG_OP_SIGMOID:
    case PG_AG_OP_TANH: case PG_AG_OP_GELU: case PG_AG_OP_ERF: case PG_AG_OP_ABS:
        return true;
    default:
        return false;
    }
}

static bool f32c(const pg_tensor *t) { return t && t->dtype == PG_DTYPE_F32 && pgt_is_contiguous(t); }

static bool node_fusible(const pg_node *n)
{
    if (!pga_op_fusible(n->ag_op) || !f32c(n->value))
        return false;
    for (size_t i = 0; i < n->nparents; i++)
        if (!f32c(n->parents[i]->value))
            return false;
    return true;
}

typedef struct {
    nvec *order;
    nmap *idx;
    int *nchild;      /* consumers in the order (with multiplicity) */
    int *inreg_child; /* consumers inside the current region */
    unsigned char *inreg;
    unsigned char *done;
} wctx;

/* build the jit graph of a region and launch it */
typedef struct {
    pg_jit_graph *g;
    wctx *w;
    int *val;  /* jit id of each order node's value, -1 = not yet */
    int *grad; /* jit id of each order node's grad contribution */
    const void *in_ptr[32];
    size_t nin;
    pg_tensor *keep_alive[32];
    /* values of nodes outside the order (no grad) */
    pg_node *ext_node[32];
    int ext_id[32];
    size_t next;
    bool fail;
} rbuild;

static int add_in(rbuild *b, const pg_tensor *t)
{
    if (b->nin >= 32) {
        b->fail = true;
        return -1;
    }
    int id = pgj_add_input_ex(b->g, t->ndim, t->shape);
    if (id < 0) {
        b->fail = true;
        return -1;
    }
    pgt_materialize((pg_tensor *)t);
    b->in_ptr[b->nin++] = t->dev;
    return id;
}

static int jop(rbuild *b, int op, int x, int y)
{
    if (b->fail || x < 0 || (y < -1))
        return (b->fail = true), -1;
    int id = pgj_op_internal(b->g, op, x, y);
    if (id < 0)
        b->fail = true;
    return id;
}

static int jconst(rbuild *b, float v)
{
    int id = pg_jit_add_const(b->g, v);
    if (id < 0)
        b->fail = true;
    return id;
}

static int fwd_code(pg_ag_op_t op)
{
    switch (op) {
    case PG_AG_OP_ADD: return PG_JIT_ADD;
    case PG_AG_OP_SUB: return PG_JIT_SUB;
    case PG_AG_OP_MUL: return PG_JIT_MUL;
    case PG_AG_OP_DIV: return PG_JIT_DIV;
    case PG_AG_OP_NEG: return PG_JIT_NEG;
    case PG_AG_OP_EXP: return PG_JIT_EXP;
    case PG_AG_OP_LOG: return PG_JIT_LOG;
    case PG_AG_OP_SQRT: return PG_JIT_SQRT;
    case PG_AG_OP_SIN: return PG_JIT_SIN;
    case PG_AG_OP_COS: return PG_JIT_COS;
    case PG_AG_OP_RELU: return PG_JIT_RELU;
    case PG_AG_OP_SIGMOID: return PG_JIT_SIGMOID;
    case PG_AG_OP_TANH: return PG_JIT_TANH;
    case PG_AG_OP_GELU: return PG_JIT_GELU;
    case PG_AG_OP_ERF: return PG_JIT_ERF;
    case PG_AG_OP_ABS: return PG_JIT_ABS;
    default: return -1;
    }
}

/* value of node p inside the kernel: recomputed for region nodes, loaded
 * otherwise */
static int value_of(rbuild *b, pg_node *p)
{
    int k = nm_get(b->w->idx, p);
    if (k >= 0 && b->val[k] >= 0)
        return b->val[k];
    if (k < 0) {
        for (size_t i = 0; i < b->next; i++)
            if (b->ext_node[i] == p)
                return b->ext_id[i];
    }
    int id;
    if (k >= 0 && b->w->inreg[k]) {
        int x = value_of(b, p->parents[0]);
        int y = p->nparents > 1 ? value_of(b, p->parents[1]) : -1;
        id = jop(b, fwd_code(p->ag_op), x, y);
    } else {
        id = add_in(b, p->value);
    }
    if (k >= 0)
        b->val[k] = id;
    else if (b->next < 32) {
        b->ext_node[b->next] = p;
        b->ext_id[b->next++] = id;
    } else {
        b->fail = true;
    }
    return id;
}

/* chain rule of one region node for parent pi (autograd.c:2166-2297) */
static int local_contrib(rbuild *b, pg_node *n, size_t pi, int g)
{
    pg_node *x = n->parents[0];
    switch (n->ag_op) {
    case PG_AG_OP_ADD: return g;
    case PG_AG_OP_SUB: return pi == 0 ? g : jop(b, PG_JIT_NEG, g, -1);
    case PG_AG_OP_MUL: return jop(b, PG_JIT_MUL, g, value_of(b, n->parents[pi == 0 ? 1 : 0]));
    case PG_AG_OP_DIV: {
        int vb = value_of(b, n->parents[1]);
        if (pi == 0)
            return jop(b, PG_JIT_DIV, g, vb);
        int va = value_of(b, n->parents[0]);
        int vb2 = jop(b, PG_JIT_MUL, vb, vb);
        int num = jop(b, PG_JIT_MUL, g, va);
        return jop(b, PG_JIT_NEG, jop(b, PG_JIT_DIV, num, vb2), -1);
    }
    case PG_AG_OP_NEG: return jop(b, PG_JIT_NEG, g, -1);
    case PG_AG_OP_EXP: return jop(b, PG_JIT_MUL, g, jop(b, PG_JIT_EXP, value_of(b, x), -1));
    case PG_AG_OP_LOG: return jop(b, PG_JIT_DIV, g, value_of(b, x));
    case PG_AG_OP_SQRT: {
        int s = jop(b, PG_JIT_SQRT, value_of(b, x), -1);
        return jop(b, PG_JIT_MUL, g, jop(b, PG_JIT_DIV, jconst(b, 0.5f), s));
    }
    case PG_AG_OP_SIN: return jop(b, PG_JIT_MUL, g, jop(b, PG_JIT_COS, value_of(b, x), -1));
    case PG_AG_OP_COS:
        return jop(b, PG_JIT_MUL, g, jop(b, PG_JIT_NEG, jop(b, PG_JIT_SIN, value_of(b, x), -1), -1));
    case PG_AG_OP_RELU: return jop(b, PG_JIT_MUL, g, jop(b, PG_JIT_STEP, value_of(b, x), -1));
    case PG_AG_OP_SIGMOID: {
        int s = jop(b, PG_JIT_SIGMOID, value_of(b, x), -1);
        int local = jop(b, PG_JIT_MUL, s, jop(b, PG_JIT_SUB, jconst(b, 1.0f), s));
        return jop(b, PG_JIT_MUL, g, local);
    }
    case PG_AG_OP_TANH: {
        int t = jop(b, PG_JIT_TANH, value_of(b, x), -1);
        int local = jop(b, PG_JIT_SUB, jconst(b, 1.0f), jop(b, PG_JIT_MUL, t, t));
        return jop(b, PG_JIT_MUL, g, local);
    }
    case PG_AG_OP_GELU: return jop(b, PG_JIT_MUL, g, jop(b, PGJ_OP_GELU_GRAD, value_of(b, x), -1));
    case PG_AG_OP_ERF: return jop(b, PG_JIT_MUL, g, jop(b, PGJ_OP_ERF_GRAD, value_of(b, x), -1));
    case PG_AG_OP_ABS: return jop(b, PG_JIT_MUL, g, jop(b, PGJ_OP_SIGN, value_of(b, x), -1));
    default: b->fail = true; return -1;
    }
}

static bool bcast_compat(const pg_tensor *t, size_t lnd, const size_t *ls)
{
    if (t->ndim > lnd)
        return false;
    size_t off = lnd - t->ndim;
    for (size_t d = 0; d < t->ndim; d++)
        if (t->shape[d] != ls[off + d] && t->shape[d] != 1)
            return false;
    return true;
}

/*
 * Grows the region rooted at order index r, builds its kernel and launches
 * it.  root_grad: the root's upstream grad tensor, or NULL to use the
 * constant `scale`.  force_beta0: outputs overwrite (pg_backward_jit).
 * Marks region nodes done on success.
 */
static bool run_region(wctx *w, int r, const pg_tensor *root_grad, float scale, bool force_beta0)
{
    nvec *ord = w->order;
    size_t N = ord->n;
    pg_node *root = ord->v[r];
    const pg_tensor *L = root->value;
    memset(w->inreg, 0, N);
    memset(w->inreg_child, 0, N * sizeof(int));
    w->inreg[r] = 1;
    /* grow to a fixed point */
    bool grew = true;
    while (grew) {
        grew = false;
        for (size_t k = 0; k < N; k++) {
            if (!w->inreg[k])
                continue;
            pg_node *x = ord->v[k];
            for (size_t pi = 0; pi < x->nparents; pi++) {
                pg_node *p = x->parents[pi];
                int pk = nm_get(w->idx, p);
                if (pk < 0 || w->inreg[pk] || w->done[pk])
                    continue;
                if (!node_fusible(p) || !pg_shape_equal(p->value->ndim, p->value->shape, L->ndim, L->shape))
                    continue;
                /* all consumers of p inside the region? count edges */
                int inside = 0;
                for (size_t q = 0; q < N; q++) {
                    if (!w->inreg[q])
                        continue;
                    pg_node *y = ord->v[q];
                    for (size_t j = 0; j < y->nparents; j++)
                        if (y->parents[j] == p)
                            inside++;
                }
                if (inside == w->nchild[pk]) {
                    w->inreg[pk] = 1;
                    grew = true;
                }
            }
        }
    }
    rbuild b;
    memset(&b, 0, sizeof b);
    b.g = pg_jit_graph_new();
    b.w = w;
    b.val = malloc(N * sizeof(int));
    b.grad = malloc(N * sizeof(int));
    if (!b.g || !b.val || !b.grad) {
        pg_jit_graph_free(b.g);
        free(b.val);
        free(b.grad);
        return false;
    }
    for (size_t k = 0; k < N; k++)
        b.val[k] = b.grad[k] = -1;
    b.grad[r] = root_grad ? add_in(&b, root_grad) : jconst(&b, scale);
    /* reverse topological order within the region */
    for (size_t kk = N; kk-- > 0 && !b.fail;) {
        if (!w->inreg[kk] || b.grad[kk] < 0)
            continue;
        pg_node *x = ord->v[kk];
        for (size_t pi = 0; pi < x->nparents && !b.fail; pi++) {
            pg_node *p = x->parents[pi];
            if (!p->requires_grad)
                continue;
            int pk = nm_get(w->idx, p);
            if (pk < 0)
                continue;
            int c = local_contrib(&b, x, pi, b.grad[kk]);
            b.grad[pk] = b.grad[pk] < 0 ? c : jop(&b, PG_JIT_ADD, b.grad[pk], c);
        }
    }
    /* outputs: grads of parents outside the region */
    pg_node *outn[32];
    size_t nout = 0;
    for (size_t k = 0; k < N && !b.fail; k++) {
        if (w->inreg[k] || b.grad[k] < 0)
            continue;
        pg_node *p = ord->v[k];
        if (nout >= 32 || !bcast_compat(p->value, L->ndim, L->shape)) {
            b.fail = true;
            break;
        }
        outn[nout++] = p;
    }
    bool ok = !b.fail && nout > 0;
    void *optr[64];
    int betas[32];
    /* a grad written whole (beta 0, the loop's shape) that a matmul16 node's
     * backward reads as 16 bits gets its copy from the region too, beside
     * the f32 elements (kept with the grad's storage, current from here
     * until the grad is next written) */
    pg_data_ref *ref16[32];
    size_t n16 = 0;
    if (ok) {
        for (size_t i = 0; i < nout; i++) {
            pg_node *p = outn[i];
            int beta;
            pg_tensor *dg = pga_grad_for_write(p, &beta);
            if (!dg) {
                ok = false;
                break;
            }
            betas[i] = force_beta0 ? 0 : beta;
            optr[i] = dg->dev;
            pgj_mark_output_ex(b.g, b.grad[nm_get(w->idx, p)], p->value->ndim, p->value->shape, betas[i]);
        }
        for (size_t i = 0; ok && i < nout; i++) {
            pg_node *p = outn[i];
            const int dt16 = pgm_mm16_grad16(p);
            if (!dt16 || betas[i] || !pg_shape_equal(p->value->ndim, p->value->shape, L->ndim, L->shape))
                continue;
            /* the same arithmetic with the copies on or off */
            pgj_graph_set_launder(b.g);
            if (!pga_copies16())
                continue;
            uint16_t *sh = pgt_shadow16_target(p->grad, (pg_dtype)dt16);
            if (!sh)
                continue;
            pgj_mark_output16(b.g, b.grad[nm_get(w->idx, p)], dt16);
            optr[nout + n16] = sh;
            ref16[n16++] = p->grad->data_ref;
        }
    }
    if (ok) {
        /* a small forward run still pending (config 1: leaves, forward and
         * sum in one block) takes the region into its own launch */
        ok = pga_lazy_flush_with_backward(b.g, L->ndim, L->shape, b.in_ptr, b.nin, optr, nout + n16) ||
             pgj_launch(b.g, L->ndim, L->shape, b.in_ptr, b.nin, optr, nout + n16);
        for (size_t i = 0; ok && i < n16; i++)
            ref16[i]->shadow_stale = false;
        if (!ok) {
            pga_set_err("fused backward failed: %s", pg_jit_last_error());
            /* restore the zero flag of grads the kernel did not write */
            for (size_t i = 0; i < nout; i++)
                if (!betas[i])
                    outn[i]->grad->pg_flags |= PG_TENSOR_ZERO_PENDING;
        }
    }
    if (ok)
        for (size_t k = 0; k < N; k++)
            if (w->inreg[k])
                w->done[k] = 1;
    pg_jit_graph_free(b.g);
    free(b.val);
    free(b.grad);
    return ok;
}

/* ---------------------------------------------------------------- walker */

static void ensure_pending_grad(pg_node *p)
{
    if (!p->requires_grad || p->grad)
        return;
    p->grad = pgt_alloc(PG_DTYPE_F32, p->value->ndim, p->value->shape);
    if (p->grad)
        p->grad->pg_flags |= PG_TENSOR_ZERO_PENDING;
}

typedef enum { MODE_FULL, MODE_SUFFIX_ONLY, MODE_SEEDED } wmode;

static bool walk(pg_node *loss, const pg_tensor *seed, wmode mode)
{
    nvec order = {0};
    if (!topo(loss, &order)) {
        free(order.v);
        return false;
    }
    size_t N = order.n;
    nmap idx;
    wctx w = {0};
    w.order = &order;
    w.idx = &idx;
    bool ok = nm_init(&idx, N);
    w.nchild = calloc(N, sizeof(int));
    w.inreg_child = calloc(N, sizeof(int));
    w.inreg = calloc(N, 1);
    w.done = calloc(N, 1);
    ok = ok && w.nchild && w.inreg_child && w.inreg && w.done;
    bool did_jit = false;
    if (ok) {
        for (size_t k = 0; k < N; k++)
            nm_put(&idx, order.v[k], (int)k);
        for (size_t k = 0; k < N; k++) {
            pg_node *x = order.v[k];
            for (size_t j = 0; j < x->nparents; j++) {
                int pk = nm_get(&idx, x->parents[j]);
                if (pk >= 0)
                    w.nchild[pk]++;
            }
        }
        if (mode != MODE_SUFFIX_ONLY)
            for (size_t k = 0; k < N; k++)
                if (order.v[k]->grad) {
                    order.v[k]->grad->pg_flags |= PG_TENSOR_ZERO_PENDING;
                    pgt_overwrite(order.v[k]->grad); /* its values are discarded */
                }

        if (mode != MODE_SEEDED && g_jit_enabled) {
            /* fold the SUM/MEAN chain above the loss into a scalar */
            pg_node *eff = loss;
            float scale = 1.0f;
            int steps = 0;
            while (eff && (eff->ag_op == PG_AG_OP_SUM || eff->ag_op == PG_AG_OP_MEAN) && eff->nparents &&
                   steps < 32) {
                if (eff->ag_op == PG_AG_OP_MEAN) {
                    pga_red_ctx *rc = eff->ctx;
                    scale *= 1.0f / (float)eff->parents[0]->value->shape[rc->axis];
                }
                eff = eff->parents[0];
                steps++;
            }
            int ek = eff ? nm_get(&idx, eff) : -1;
            if (ek >= 0 && node_fusible(eff)) {
                if (run_region(&w, ek, NULL, scale, mode == MODE_SUFFIX_ONLY)) {
                    did_jit = true;
                    /* the folded prefix is done too */
                    pg_node *q = loss;
                    while (q != eff) {
                        w.done[nm_get(&idx, q)] = 1;
                        q = q->parents[0];
                    }
                }
            } else {
                pga_set_err("loss is not above a fusible elementwise node");
            }
            g_last_was_jit = did_jit;
            if (did_jit)
                g_jit_hits++;
            else
                g_jit_fallbacks++;
        }
        if (mode == MODE_SUFFIX_ONLY)
            goto out;
        if (mode == MODE_SEEDED) {
            loss->grad = pg_tensor_view(seed);
        } else if (!did_jit) {
            int beta;
            pg_tensor *lg = pga_grad_for_write(loss, &beta);
            if (lg)
                pg_tensor_fill(lg, 1.0f);
        }
        for (size_t kk = N; kk-- > 0;) {
            pg_node *x = order.v[kk];
            if (w.done[kk] || !x->backward || !x->grad)
                continue;
            if (x->grad->pg_flags & PG_TENSOR_ZERO_PENDING) {
                /* a zero upstream grad contributes nothing, but the parents'
                 * grads still come into existence (as zeros) */
                for (size_t j = 0; j < x->nparents; j++)
                    ensure_pending_grad(x->parents[j]);
                continue;
            }
            if (g_jit_enabled && node_fusible(x) && run_region(&w, (int)kk, x->grad, 1.0f, false))
                continue;
            x->backward(x);
        }
        if (mode == MODE_SEEDED) {
            pg_tensor_free(loss->grad);
            loss->grad = NULL;
        }
        /* a grad pending as a narrow product over the copy of the weights
         * its consumer's pass made stays so: its first reader writes it (a
         * training step never reads it).  One still over the layer's own
         * 16-bit weights (its consumer did not run) is written now: an
         * optimiser step may rewrite those */
        for (size_t k = 0; k < N; k++) {
            pg_tensor *g = order.v[k]->grad;
            const pg_narrow_pending *np = g && g->data_ref ? g->data_ref->narrow : NULL;
            if (!np || np->hold[1])
                pgt_materialize(g);
        }
    }
out:
    pgm_colsum_flush(); /* a bias grad's sums still deferred to a next pass */
    for (size_t k = 0; k < N; k++)
        order.v[k]->mark = 0;
    free(order.v);
    nm_free(&idx);
    free(w.nchild);
    free(w.inreg_child);
    free(w.inreg);
    free(w.done);
    return mode == MODE_SUFFIX_ONLY ? did_jit : ok;
}

void pg_backward(pg_node *loss)
{
    if (!loss || !loss->requires_grad || !pgd_ok())
        return;
    walk(loss, NULL, MODE_FULL);
}

bool pg_backward_jit(pg_node *loss)
{
    if (!loss || !loss->requires_grad || !pgd_ok())
        return false;
    bool saved = g_jit_enabled;
    g_jit_enabled = true;
    bool ok = walk(loss, NULL, MODE_SUFFIX_ONLY);
    g_jit_enabled = saved;
    return ok;
}

void pg_amd_backward_from(pg_node *root, const pg_tensor *seed)
{
    if (!root || !seed || !root->requires_grad || !pgd_ok())
        return;
    if (seed->dtype != PG_DTYPE_F32 ||
        !pg_shape_equal(seed->ndim, seed->shape, root->value->ndim, root->value->shape)) {
        pga_set_err("pg_amd_backward_from: seed must be f32 with the root's shape");
        return;
    }
    pg_tensor_free(root->grad);
    root->grad = NULL;
    walk(root, seed, MODE_SEEDED);
}
