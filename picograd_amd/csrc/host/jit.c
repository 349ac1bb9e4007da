/*
 * Elementwise fusion JIT for gfx950.
 *
 * Same graph API as the reference's jit/jit.c (node kinds, broadcasting
 * rules of pg_jit_add_op, FNV-1a graph hash, hash + structural-equality
 * cache).  Code generation is new: a graph becomes one HIP kernel compiled
 * in-process by hiprtc for gfx950 and loaded with hipModuleLoadData.
 *
 * Kernel shapes:
 *  - no reduced output: a grid-stride loop over the (dim-collapsed) loop
 *    shape, four consecutive elements per lane with 16-byte loads/stores
 *    whenever the innermost dim allows it;
 *  - with outputs reduced onto a trailing-dims shape (the grad of a bias
 *    broadcast over rows): a [R x C] tiling, 256 threads = 64 column
 *    groups x 4 row lanes, each block walking a band of rows.  Column
 *    partial sums stay in registers, are combined across the 4 row lanes
 *    through LDS in a fixed order and written once per block; a second
 *    kernel of the same module sums the per-block partials in block order.
 *    The result is deterministic (no float atomics).
 * Compiled code objects are cached in memory (graph hash + structural
 * equality) and on disk (hash of the generated source) so a process or a
 * later process pays the hiprtc compile once per distinct graph.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define MAXIO 16
#ifndef PGJ_RED_ROWS
#define PGJ_RED_ROWS 4
#endif

typedef enum { JN_INPUT, JN_CONST, JN_OP } jkind;

typedef struct {
    jkind kind;
    int op; /* pg_jit_op_t or PGJ_OP_* */
    int in[2];
    int nin;
    float cval;
    size_t ndim;
    size_t shape[PG_MAX_NDIM];
    size_t numel;
} jnode;

typedef struct {
    int node;
    size_t ndim;            /* target shape: equals the node's for a plain output */
    size_t shape[PG_MAX_NDIM];
    int beta;
    int dt16; /* 0: f32; PG_DTYPE_F16 / PG_DTYPE_BF16: the node's 16-bit copy (pgj_mark_output16) */
} jout;

struct pg_jit_graph {
    jnode *nodes;
    size_t nn, cap;
    int inputs[MAXIO * 2];
    size_t nin;
    jout outs[MAXIO * 2];
    size_t nout;
    bool exact; /* no FMA contraction between the graph's ops (pgj_graph_set_exact) */
    bool launder; /* stored values through one asm copy (pgj_graph_set_launder) */
};

/* one compiled kernel for one (graph, loop shape) */
typedef struct centry {
    uint64_t hash;
    pg_jit_graph *g; /* structural copy */
    size_t loop_ndim;
    size_t loop_shape[PG_MAX_NDIM];
    hipModule_t mod;
    hipFunction_t fmain, ffin;
    int variant;     /* PGJ_VAR_MAIN, PGJ_VAR_SMALL or PGJ_VAR_SMALL + 1 + reduced output */
    size_t nin, nout; /* the kernel argument block holds max(1, n) pointers of each */
    /* launch plan */
    unsigned grid_x, grid_y, fin_grid;
    int has_red;
    size_t part_floats[MAXIO * 2]; /* per output, partial buffer size (0 = none) */
    size_t part_off[MAXIO * 2];
    size_t part_total;
    struct centry *next;
} centry;

/* kernel variants of one graph: the grid-stride (or [R x C] tiled) kernel,
 * and the one-block kernel of a small run that also performs the pending
 * uploads and, optionally, the two-stage column/total reduction of one of
 * its outputs (PGJ_VAR_SMALL + 1 + that output's index) */
enum { PGJ_VAR_MAIN = 0, PGJ_VAR_SMALL = 1 };
#define PGJ_SMALL_THREADS 1024
#define PGJ_SMALL_UPLOADS 4

/* the small kernel's argument block after its in[NI] and out[NO] pointers
 * (the generated struct asserts the same layout) */
typedef struct {
    pgk_upload up[PGJ_SMALL_UPLOADS];
    unsigned nup, up_pieces;
    float *r1, *r2;
    float scale;
} small_tail;

struct pg_jit_exe {
    centry *e;
    bool owned; /* not in the cache: freed with the exe */
    size_t nin, nout;
    size_t in_ndim[MAXIO], in_shape[MAXIO][PG_MAX_NDIM];
    size_t out_ndim[MAXIO], out_shape[MAXIO][PG_MAX_NDIM];
};

static centry *g_cache;
static size_t g_cache_n;
static bool g_cache_on = true;
static char g_jerr[1024];
size_t pgj_stat_compiles, pgj_stat_hits;

static void jset_err(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_jerr, sizeof g_jerr, fmt, ap);
    va_end(ap);
}

const char *pg_jit_last_error(void) { return g_jerr; }
size_t pg_jit_cache_size(void) { return g_cache_n; }
void pg_jit_set_cache_enabled(bool e) { g_cache_on = e; }
bool pg_jit_is_cache_enabled(void) { return g_cache_on; }
size_t pg_amd_jit_compiles(void) { return pgj_stat_compiles; }
size_t pg_amd_jit_cache_hits(void) { return pgj_stat_hits; }

/* ---------------------------------------------------------------- graph */

pg_jit_graph *pg_jit_graph_new(void) { return calloc(1, sizeof(pg_jit_graph)); }

void pgj_graph_set_launder(pg_jit_graph *g)
{
    if (g)
        g->launder = true;
}

void pgj_graph_set_exact(pg_jit_graph *g)
{
    if (g)
        g->exact = true;
}

void pg_jit_graph_free(pg_jit_graph *g)
{
    if (!g)
        return;
    free(g->nodes);
    free(g);
}

size_t pg_jit_num_inputs(const pg_jit_graph *g) { return g ? g->nin : 0; }
size_t pg_jit_num_outputs(const pg_jit_graph *g) { return g ? g->nout : 0; }
size_t pg_jit_num_nodes(const pg_jit_graph *g) { return g ? g->nn : 0; }

static jnode *new_node(pg_jit_graph *g)
{
    if (g->nn == g->cap) {
        size_t nc = g->cap ? g->cap * 2 : 16;
        jnode *p = realloc(g->nodes, nc * sizeof *p);
        if (!p)
            return NULL;
        g->nodes = p;
        g->cap = nc;
    }
    jnode *n = &g->nodes[g->nn];
    memset(n, 0, sizeof *n);
    return n;
}

static bool shape_ok(size_t ndim, const size_t *shape)
{
    if (ndim == 0 || ndim > PG_MAX_NDIM || !shape)
        return false;
    for (size_t i = 0; i < ndim; i++)
        if (!shape[i])
            return false;
    return true;
}

int pgj_add_input_ex(pg_jit_graph *g, size_t ndim, const size_t *shape)
{
    if (!g || !shape_ok(ndim, shape)) {
        jset_err("invalid input shape");
        return -1;
    }
    if (g->nin >= MAXIO * 2) {
        jset_err("too many inputs");
        return -1;
    }
    jnode *n = new_node(g);
    if (!n) {
        jset_err("oom");
        return -1;
    }
    n->kind = JN_INPUT;
    n->ndim = ndim;
    memcpy(n->shape, shape, ndim * sizeof(size_t));
    n->numel = pg_shape_numel(ndim, shape);
    int id = (int)g->nn++;
    g->inputs[g->nin++] = id;
    return id;
}

int pg_jit_add_input(pg_jit_graph *g, size_t ndim, const size_t *shape)
{
    return pgj_add_input_ex(g, ndim, shape);
}

int pg_jit_add_const(pg_jit_graph *g, float value)
{
    if (!g) {
        jset_err("null graph");
        return -1;
    }
    jnode *n = new_node(g);
    if (!n) {
        jset_err("oom");
        return -1;
    }
    n->kind = JN_CONST;
    n->cval = value;
    n->ndim = 1;
    n->shape[0] = 1;
    n->numel = 1;
    return (int)g->nn++;
}

static bool is_binary(int op)
{
    return op == PG_JIT_ADD || op == PG_JIT_SUB || op == PG_JIT_MUL || op == PG_JIT_DIV;
}

/* numpy broadcast of two shapes (jit.c:113-125 rules) */
static bool bcast2(size_t na, const size_t *sa, size_t nb, const size_t *sb, size_t *nd, size_t *out)
{
    size_t n = na > nb ? na : nb;
    if (n > PG_MAX_NDIM)
        return false;
    for (size_t d = 0; d < n; d++) {
        size_t da = d < n - na ? 1 : sa[d - (n - na)];
        size_t db = d < n - nb ? 1 : sb[d - (n - nb)];
        if (da != db && da != 1 && db != 1)
            return false;
        out[d] = da > db ? da : db;
    }
    *nd = n;
    return true;
}

int pgj_op_internal(pg_jit_graph *g, int op, int a, int b)
{
    if (!g) {
        jset_err("null args");
        return -1;
    }
    int nin = is_binary(op) ? 2 : 1;
    int ins[2] = {a, b};
    for (int i = 0; i < nin; i++)
        if (ins[i] < 0 || (size_t)ins[i] >= g->nn) {
            jset_err("invalid input id %d", ins[i]);
            return -1;
        }
    size_t nd = 0, shp[PG_MAX_NDIM];
    if (nin == 2) {
        jnode *x = &g->nodes[a], *y = &g->nodes[b];
        if (!bcast2(x->ndim, x->shape, y->ndim, y->shape, &nd, shp)) {
            jset_err("incompatible broadcast shapes");
            return -1;
        }
    } else {
        nd = g->nodes[a].ndim;
        memcpy(shp, g->nodes[a].shape, nd * sizeof(size_t));
    }
    jnode *n = new_node(g);
    if (!n) {
        jset_err("oom");
        return -1;
    }
    n->kind = JN_OP;
    n->op = op;
    n->nin = nin;
    n->in[0] = a;
    n->in[1] = nin == 2 ? b : -1;
    n->ndim = nd;
    memcpy(n->shape, shp, nd * sizeof(size_t));
    n->numel = pg_shape_numel(nd, shp);
    return (int)g->nn++;
}

int pg_jit_add_op(pg_jit_graph *g, pg_jit_op_t op, const int *inputs, size_t ninputs)
{
    if (!g || !inputs) {
        jset_err("null args");
        return -1;
    }
    if ((int)op < PG_JIT_ADD || op > PG_JIT_STEP) {
        jset_err("unknown op %d", (int)op);
        return -1;
    }
    if (is_binary(op) && ninputs != 2) {
        jset_err("binary op requires 2 inputs");
        return -1;
    }
    if (!is_binary(op) && ninputs != 1) {
        jset_err("unary op requires 1 input");
        return -1;
    }
    return pgj_op_internal(g, op, inputs[0], ninputs == 2 ? inputs[1] : -1);
}

int pg_jit_add(pg_jit_graph *g, int a, int b) { return pgj_op_internal(g, PG_JIT_ADD, a, b); }
int pg_jit_sub(pg_jit_graph *g, int a, int b) { return pgj_op_internal(g, PG_JIT_SUB, a, b); }
int pg_jit_mul(pg_jit_graph *g, int a, int b) { return pgj_op_internal(g, PG_JIT_MUL, a, b); }
int pg_jit_div(pg_jit_graph *g, int a, int b) { return pgj_op_internal(g, PG_JIT_DIV, a, b); }
int pg_jit_neg(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_NEG, a, -1); }
int pg_jit_exp(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_EXP, a, -1); }
int pg_jit_log(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_LOG, a, -1); }
int pg_jit_sqrt(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_SQRT, a, -1); }
int pg_jit_sin(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_SIN, a, -1); }
int pg_jit_cos(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_COS, a, -1); }
int pg_jit_abs(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_ABS, a, -1); }
int pg_jit_relu(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_RELU, a, -1); }
int pg_jit_sigmoid(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_SIGMOID, a, -1); }
int pg_jit_tanh(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_TANH, a, -1); }
int pg_jit_gelu(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_GELU, a, -1); }
int pg_jit_erf(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_ERF, a, -1); }
int pg_jit_step(pg_jit_graph *g, int a) { return pgj_op_internal(g, PG_JIT_STEP, a, -1); }

void pgj_mark_output_ex(pg_jit_graph *g, int id, size_t ndim, const size_t *shape, int beta)
{
    if (!g || id < 0 || (size_t)id >= g->nn) {
        jset_err("invalid output id");
        return;
    }
    if (g->nout >= MAXIO * 2) {
        jset_err("too many outputs");
        return;
    }
    jout *o = &g->outs[g->nout++];
    o->node = id;
    o->ndim = ndim;
    memcpy(o->shape, shape, ndim * sizeof(size_t));
    o->beta = beta;
    o->dt16 = 0;
}

void pgj_mark_output16(pg_jit_graph *g, int id, int dt16)
{
    if (!g || id < 0 || (size_t)id >= g->nn || (dt16 != PG_DTYPE_F16 && dt16 != PG_DTYPE_BF16)) {
        jset_err("invalid 16-bit output");
        return;
    }
    pgj_mark_output_ex(g, id, g->nodes[id].ndim, g->nodes[id].shape, 0);
    if (g->nout && g->outs[g->nout - 1].node == id)
        g->outs[g->nout - 1].dt16 = dt16;
}

/* Appends src's nodes to dst: src's input i becomes dst's node in_map[i],
 * constants and ops are copied in order, and src's outputs are marked on
 * dst after dst's own (same shapes and betas).  Every output of src must be
 * a full loop-shape output (lnd, ls): the caller's one-block run stores
 * them element by element.  False when that fails (dst may hold unused
 * extra nodes then, and no extra outputs). */
bool pgj_graph_append(pg_jit_graph *dst, const pg_jit_graph *src, const int *in_map, size_t lnd, const size_t *ls)
{
    if (!dst || !src || dst->nout + src->nout > MAXIO * 2)
        return false;
    for (size_t o = 0; o < src->nout; o++)
        if (!pg_shape_equal(src->outs[o].ndim, src->outs[o].shape, lnd, ls))
            return false;
    int *map = malloc((src->nn ? src->nn : 1) * sizeof(int));
    if (!map)
        return false;
    bool ok = true;
    for (size_t id = 0; id < src->nn && ok; id++) {
        const jnode *n = &src->nodes[id];
        if (n->kind == JN_INPUT) {
            map[id] = -1;
            for (size_t i = 0; i < src->nin; i++)
                if (src->inputs[i] == (int)id)
                    map[id] = in_map[i];
            ok = map[id] >= 0 && (size_t)map[id] < dst->nn &&
                 pg_shape_equal(dst->nodes[map[id]].ndim, dst->nodes[map[id]].shape, n->ndim, n->shape);
        } else if (n->kind == JN_CONST) {
            ok = (map[id] = pg_jit_add_const(dst, n->cval)) >= 0;
        } else {
            ok = (map[id] = pgj_op_internal(dst, n->op, map[n->in[0]], n->nin == 2 ? map[n->in[1]] : -1)) >= 0;
        }
    }
    dst->launder = dst->launder || src->launder;
    for (size_t o = 0; o < src->nout && ok; o++) {
        pgj_mark_output_ex(dst, map[src->outs[o].node], src->outs[o].ndim, src->outs[o].shape, src->outs[o].beta);
        if (dst->nout)
            dst->outs[dst->nout - 1].dt16 = src->outs[o].dt16;
    }
    free(map);
    return ok;
}

/* input i's shape */
bool pgj_input_shape(const pg_jit_graph *g, size_t i, size_t *ndim, const size_t **shape)
{
    if (!g || i >= g->nin)
        return false;
    const jnode *n = &g->nodes[g->inputs[i]];
    *ndim = n->ndim;
    *shape = n->shape;
    return true;
}

void pg_jit_mark_output(pg_jit_graph *g, int id)
{
    if (!g || id < 0 || (size_t)id >= g->nn) {
        jset_err("invalid output id");
        return;
    }
    pgj_mark_output_ex(g, id, g->nodes[id].ndim, g->nodes[id].shape, 0);
}

void pg_jit_clear_outputs(pg_jit_graph *g)
{
    if (g)
        g->nout = 0;
}

/* ---------------------------------------------------------------- hash */

static uint64_t fnv(const void *p, size_t n, uint64_t h)
{
    const unsigned char *b = p;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 1099511628211ULL;
    }
    return h;
}

uint64_t pg_jit_graph_hash(const pg_jit_graph *g)
{
    uint64_t h = 14695981039346656037ULL;
    if (!g)
        return h;
    h = fnv(&g->nn, sizeof g->nn, h);
    h = fnv(&g->nin, sizeof g->nin, h);
    h = fnv(&g->nout, sizeof g->nout, h);
    if (g->exact)
        h = fnv("exact", 5, h);
    if (g->launder)
        h = fnv("launder", 7, h);
    for (size_t i = 0; i < g->nout; i++)
        if (g->outs[i].dt16) {
            h = fnv(&i, sizeof i, h);
            h = fnv(&g->outs[i].dt16, sizeof g->outs[i].dt16, h);
        }
    for (size_t i = 0; i < g->nn; i++) {
        const jnode *n = &g->nodes[i];
        h = fnv(&n->kind, sizeof n->kind, h);
        if (n->kind == JN_OP) {
            h = fnv(&n->op, sizeof n->op, h);
            h = fnv(n->in, (size_t)n->nin * sizeof(int), h);
        } else if (n->kind == JN_CONST) {
            h = fnv(&n->cval, sizeof n->cval, h);
        }
        h = fnv(&n->ndim, sizeof n->ndim, h);
        h = fnv(n->shape, n->ndim * sizeof(size_t), h);
    }
    h = fnv(g->inputs, g->nin * sizeof(int), h);
    for (size_t i = 0; i < g->nout; i++) {
        h = fnv(&g->outs[i].node, sizeof(int), h);
        h = fnv(&g->outs[i].ndim, sizeof(size_t), h);
        h = fnv(g->outs[i].shape, g->outs[i].ndim * sizeof(size_t), h);
        h = fnv(&g->outs[i].beta, sizeof(int), h);
    }
    return h;
}

static bool graph_equal(const pg_jit_graph *a, const pg_jit_graph *b)
{
    if (a->nn != b->nn || a->nin != b->nin || a->nout != b->nout || a->exact != b->exact || a->launder != b->launder)
        return false;
    for (size_t i = 0; i < a->nn; i++) {
        const jnode *x = &a->nodes[i], *y = &b->nodes[i];
        if (x->kind != y->kind || x->ndim != y->ndim || memcmp(x->shape, y->shape, x->ndim * sizeof(size_t)))
            return false;
        if (x->kind == JN_OP &&
            (x->op != y->op || x->nin != y->nin || x->in[0] != y->in[0] || (x->nin == 2 && x->in[1] != y->in[1])))
            return false;
        if (x->kind == JN_CONST && memcmp(&x->cval, &y->cval, sizeof(float)))
            return false;
    }
    if (memcmp(a->inputs, b->inputs, a->nin * sizeof(int)))
        return false;
    for (size_t i = 0; i < a->nout; i++) {
        const jout *x = &a->outs[i], *y = &b->outs[i];
        if (x->node != y->node || x->ndim != y->ndim || x->beta != y->beta || x->dt16 != y->dt16 ||
            memcmp(x->shape, y->shape, x->ndim * sizeof(size_t)))
            return false;
    }
    return true;
}

static pg_jit_graph *graph_clone(const pg_jit_graph *g)
{
    pg_jit_graph *c = calloc(1, sizeof *c);
    if (!c)
        return NULL;
    *c = *g;
    c->nodes = malloc((g->nn ? g->nn : 1) * sizeof(jnode));
    if (!c->nodes) {
        free(c);
        return NULL;
    }
    memcpy(c->nodes, g->nodes, g->nn * sizeof(jnode));
    c->cap = g->nn;
    return c;
}

/* ---------------------------------------------------------------- planning */

typedef struct {
    int ndim;
    int64_t dims[PG_MAX_NDIM];
    int64_t numel;
    int nin;
    int in_node[MAXIO * 2];
    bool in_used[MAXIO * 2];
    bool in_direct[MAXIO * 2];
    int64_t istr[MAXIO * 2][PG_MAX_NDIM];
    int nout;
    int out_node[MAXIO * 2];
    int out_red[MAXIO * 2]; /* 1: reduced over dims < ksplit */
    int out_beta[MAXIO * 2];
    int out_dt16[MAXIO * 2]; /* a 16-bit copy of the node (full loop shape, beta 0) */
    bool launder;            /* stored values through one asm copy (emit_launder) */
    int ksplit;
    int64_t R, C;
    int vec;
} plan_t;

/* strides (in elements) of a contiguous `shape` broadcast over the loop
 * shape; false if not broadcast-compatible */
static bool bstrides(size_t ndim, const size_t *shape, size_t lnd, const size_t *ls, int64_t *out)
{
    if (ndim > lnd)
        return false;
    int64_t st[PG_MAX_NDIM];
    int64_t acc = 1;
    for (size_t i = ndim; i-- > 0;) {
        st[i] = acc;
        acc *= (int64_t)shape[i];
    }
    size_t off = lnd - ndim;
    for (size_t d = 0; d < lnd; d++) {
        if (d < off) {
            out[d] = 0;
            continue;
        }
        size_t s = shape[d - off];
        if (s == ls[d])
            out[d] = ls[d] == 1 ? 0 : st[d - off];
        else if (s == 1)
            out[d] = 0;
        else
            return false;
    }
    return true;
}

static void mark_reach(const pg_jit_graph *g, bool *reach)
{
    memset(reach, 0, g->nn);
    int *stk = malloc((g->nn + 1) * sizeof(int));
    size_t sp = 0;
    for (size_t i = 0; i < g->nout; i++)
        if (!reach[g->outs[i].node]) {
            reach[g->outs[i].node] = true;
            stk[sp++] = g->outs[i].node;
        }
    while (sp) {
        const jnode *n = &g->nodes[stk[--sp]];
        if (n->kind != JN_OP)
            continue;
        for (int k = 0; k < n->nin; k++)
            if (!reach[n->in[k]]) {
                reach[n->in[k]] = true;
                stk[sp++] = n->in[k];
            }
    }
    free(stk);
}

static bool make_plan(const pg_jit_graph *g, size_t lnd, const size_t *ls, plan_t *P, const bool *reach)
{
    memset(P, 0, sizeof *P);
    P->launder = g->launder;
    int64_t lstr[MAXIO * 4][PG_MAX_NDIM]; /* inputs then outputs */
    int nrow = 0;
    P->nin = (int)g->nin;
    for (size_t i = 0; i < g->nin; i++) {
        const jnode *n = &g->nodes[g->inputs[i]];
        P->in_node[i] = g->inputs[i];
        P->in_used[i] = reach[g->inputs[i]];
        if (!bstrides(n->ndim, n->shape, lnd, ls, lstr[nrow])) {
            jset_err("input %zu not broadcast-compatible with the loop shape", i);
            return false;
        }
        nrow++;
    }
    P->nout = (int)g->nout;
    int red_first = -1;
    for (size_t i = 0; i < g->nout; i++) {
        const jout *o = &g->outs[i];
        P->out_node[i] = o->node;
        P->out_beta[i] = o->beta;
        P->out_dt16[i] = o->dt16;
        P->launder = P->launder || o->dt16;
        if (!bstrides(o->ndim, o->shape, lnd, ls, lstr[nrow])) {
            jset_err("output %zu shape not broadcast-compatible with the loop shape", i);
            return false;
        }
        size_t on = pg_shape_numel(o->ndim, o->shape);
        size_t ln = pg_shape_numel(lnd, ls);
        P->out_red[i] = on != ln;
        if (o->dt16 && (P->out_red[i] || o->beta)) {
            jset_err("16-bit output %zu must be a full-shape write", i);
            return false;
        }
        if (P->out_red[i]) {
            /* must be a trailing-dims pattern: broadcast (zero stride) over
             * every non-1 dim before the first kept dim, kept after it */
            int first_nz = (int)lnd;
            for (size_t d = 0; d < lnd; d++)
                if (ls[d] != 1 && lstr[nrow][d] != 0) {
                    first_nz = (int)d;
                    break;
                }
            for (size_t d = (size_t)first_nz; d < lnd; d++)
                if (ls[d] != 1 && lstr[nrow][d] == 0) {
                    jset_err("reduced output %zu is not a trailing-dims broadcast", i);
                    return false;
                }
            if (red_first >= 0 && red_first != first_nz) {
                jset_err("reduced outputs disagree on the reduced dims");
                return false;
            }
            red_first = first_nz;
        }
        nrow++;
    }
    /* collapse adjacent loop dims whose strides stay linear in every row;
     * never merge across the first kept dim of the reduced outputs */
    int nd = 0, ks = -1;
    int64_t dims[PG_MAX_NDIM];
    int64_t rs[MAXIO * 4][PG_MAX_NDIM];
    for (size_t d = 0; d < lnd; d++) {
        if (ls[d] == 1)
            continue;
        bool barrier = red_first >= 0 && ks < 0 && (int)d >= red_first;
        if (nd > 0 && !barrier) {
            bool ok = true;
            for (int r = 0; r < nrow && ok; r++) {
                int64_t prev = rs[r][nd - 1], cur = lstr[r][d];
                ok = (prev == 0 && cur == 0) || (cur != 0 && prev == cur * (int64_t)ls[d]);
            }
            if (ok) {
                dims[nd - 1] *= (int64_t)ls[d];
                for (int r = 0; r < nrow; r++)
                    rs[r][nd - 1] = lstr[r][d];
                continue;
            }
        }
        if (barrier)
            ks = nd;
        dims[nd] = (int64_t)ls[d];
        for (int r = 0; r < nrow; r++)
            rs[r][nd] = lstr[r][d];
        nd++;
    }
    if (nd == 0) {
        nd = 1;
        dims[0] = 1;
        for (int r = 0; r < nrow; r++)
            rs[r][0] = 0;
    }
    P->ksplit = red_first >= 0 ? (ks < 0 ? nd : ks) : 0;
    P->ndim = nd;
    memcpy(P->dims, dims, sizeof dims);
    P->numel = 1;
    for (int d = 0; d < nd; d++)
        P->numel *= dims[d];
    for (int i = 0; i < P->nin; i++) {
        memcpy(P->istr[i], rs[i], sizeof(int64_t) * PG_MAX_NDIM);
        bool direct = true;
        int64_t acc = 1;
        for (int d = nd - 1; d >= 0; d--) {
            if (rs[i][d] != (dims[d] == 1 ? rs[i][d] : acc))
                direct = false;
            acc *= dims[d];
        }
        P->in_direct[i] = direct;
    }
    bool any_red = red_first >= 0;
    if (any_red) {
        P->R = 1;
        P->C = 1;
        for (int d = 0; d < nd; d++) {
            if (d < P->ksplit)
                P->R *= dims[d];
            else
                P->C *= dims[d];
        }
    }
    /* vector width 4 when the innermost dim and every used input allow it */
    int64_t inner = dims[nd - 1];
    bool v4 = inner % 4 == 0;
    for (int i = 0; i < P->nin && v4; i++)
        if (P->in_used[i] && !(P->istr[i][nd - 1] == 0 || P->istr[i][nd - 1] == 1))
            v4 = false;
    P->vec = v4 ? 4 : 1;
    return true;
}

/* ---------------------------------------------------------------- codegen */

typedef struct {
    char *s;
    size_t n, cap;
} sbuf;

static void sb_add(sbuf *b, const char *fmt, ...)
{
    va_list ap;
    for (;;) {
        size_t room = b->cap - b->n;
        va_start(ap, fmt);
        int w = vsnprintf(b->s ? b->s + b->n : NULL, room, fmt, ap);
        va_end(ap);
        if (w < 0)
            return;
        if ((size_t)w < room) {
            b->n += (size_t)w;
            return;
        }
        size_t nc = (b->cap ? b->cap * 2 : 8192) + (size_t)w;
        char *p = realloc(b->s, nc);
        if (!p)
            return;
        b->s = p;
        b->cap = nc;
    }
}

static void emit_expr(sbuf *b, const jnode *n, const char *a, const char *c)
{
    switch (n->op) {
    case PG_JIT_ADD: sb_add(b, "(%s + %s)", a, c); break;
    case PG_JIT_SUB: sb_add(b, "(%s - %s)", a, c); break;
    case PG_JIT_MUL: sb_add(b, "(%s * %s)", a, c); break;
    case PG_JIT_DIV: sb_add(b, "(%s / %s)", a, c); break;
    case PG_JIT_NEG: sb_add(b, "(-%s)", a); break;
    case PG_JIT_EXP: sb_add(b, "pgm_exp(%s)", a); break;
    case PG_JIT_LOG: sb_add(b, "logf(%s)", a); break;
    case PG_JIT_SQRT: sb_add(b, "sqrtf(%s)", a); break;
    case PG_JIT_SIN: sb_add(b, "sinf(%s)", a); break;
    case PG_JIT_COS: sb_add(b, "cosf(%s)", a); break;
    case PG_JIT_ABS: sb_add(b, "fabsf(%s)", a); break;
    case PG_JIT_RELU: sb_add(b, "(%s > 0.0f ? %s : 0.0f)", a, a); break;
    case PG_JIT_SIGMOID: sb_add(b, "pgm_sigmoid(%s)", a); break;
    case PG_JIT_TANH: sb_add(b, "tanhf(%s)", a); break;
    case PG_JIT_GELU: sb_add(b, "pgm_gelu(%s)", a); break;
    case PG_JIT_ERF: sb_add(b, "erff(%s)", a); break;
    case PG_JIT_STEP: sb_add(b, "(%s > 0.0f ? 1.0f : 0.0f)", a); break;
    case PGJ_OP_GELU_GRAD: sb_add(b, "pgm_gelu_grad(%s)", a); break;
    case PGJ_OP_SIGN: sb_add(b, "(%s > 0.0f ? 1.0f : (%s < 0.0f ? -1.0f : 0.0f))", a, a); break;
    case PGJ_OP_ERF_GRAD: sb_add(b, "(1.12837916709551f * pgm_exp(-%s * %s))", a, a); break;
    default: sb_add(b, "0.0f"); break;
    }
}

/* offset expression of input i at flat loop index `idx` (a C expression) */
static void emit_offset(sbuf *b, const plan_t *P, int i, const char *idx)
{
    if (P->in_direct[i]) {
        sb_add(b, "(%s)", idx);
        return;
    }
    /* unravel over the collapsed dims, innermost first */
    sb_add(b, "({ IDX _r = (%s); IDX _o = 0; ", idx);
    for (int d = P->ndim - 1; d >= 0; d--) {
        if (P->istr[i][d] != 0)
            sb_add(b, "_o += (_r %% (IDX)%lld) * (IDX)%lld; ", (long long)P->dims[d], (long long)P->istr[i][d]);
        if (d > 0)
            sb_add(b, "_r /= (IDX)%lld; ", (long long)P->dims[d]);
    }
    sb_add(b, "_o; })");
}

/* Values are named v<node>_<copy>_<lane>: `copy` is the unrolled position
 * (several rows or strides per loop iteration), `lane` the element of a
 * 4-wide vector. */

/* loads of every used input for one copy at flat index `idx` */
static void emit_loads(sbuf *b, const plan_t *P, int vec, const char *idx, int u)
{
    for (int i = 0; i < P->nin; i++) {
        if (!P->in_used[i])
            continue;
        int nid = P->in_node[i];
        if (vec == 4 && P->istr[i][P->ndim - 1] != 0) {
            /* an input of the full loop shape is read exactly once: stream it
             * past the caches; broadcast inputs are re-read and stay cached */
            if (P->in_direct[i])
                sb_add(b, "    const pgf4 q%d_%d = __builtin_nontemporal_load((const pgf4 *)(in%d + ", nid, u, i);
            else
                sb_add(b, "    const pgf4 q%d_%d = *(const pgf4 *)(in%d + ", nid, u, i);
            emit_offset(b, P, i, idx);
            sb_add(b, P->in_direct[i] ? "));\n" : ");\n");
            sb_add(b, "    float v%d_%d_0 = q%d_%d.x, v%d_%d_1 = q%d_%d.y, v%d_%d_2 = q%d_%d.z, v%d_%d_3 = q%d_%d.w;\n",
                   nid, u, nid, u, nid, u, nid, u, nid, u, nid, u, nid, u, nid, u);
        } else if (P->in_direct[i]) {
            sb_add(b, "    const float s%d_%d = __builtin_nontemporal_load(in%d + ", nid, u, i);
            emit_offset(b, P, i, idx);
            sb_add(b, ");\n");
        } else {
            sb_add(b, "    const float s%d_%d = in%d[", nid, u, i);
            emit_offset(b, P, i, idx);
            sb_add(b, "];\n");
        }
        if (!(vec == 4 && P->istr[i][P->ndim - 1] != 0))
            for (int e = 0; e < vec; e++)
                sb_add(b, "    float v%d_%d_%d = s%d_%d;\n", nid, u, e, nid, u);
    }
}

/* the straight-line forward recompute and chain rule of one copy */
static void emit_compute(sbuf *b, const pg_jit_graph *g, const bool *reach, int vec, int u)
{
    for (size_t id = 0; id < g->nn; id++) {
        if (!reach[id])
            continue;
        const jnode *n = &g->nodes[id];
        if (n->kind == JN_INPUT)
            continue;
        for (int e = 0; e < vec; e++) {
            if (n->kind == JN_CONST) {
                /* exact hex-float literal of the f32 constant */
                float cv = n->cval;
                if (cv != cv)
                    sb_add(b, "    const float v%zu_%d_%d = __builtin_nanf(\"\");\n", id, u, e);
                else if (cv > 3.4028235e38f || cv < -3.4028235e38f)
                    sb_add(b, "    const float v%zu_%d_%d = %s__builtin_inff();\n", id, u, e, cv < 0 ? "-" : "");
                else
                    sb_add(b, "    const float v%zu_%d_%d = (float)%a;\n", id, u, e, (double)cv);
                continue;
            }
            char sa[40], sc[40];
            snprintf(sa, sizeof sa, "v%d_%d_%d", n->in[0], u, e);
            snprintf(sc, sizeof sc, "v%d_%d_%d", n->nin == 2 ? n->in[1] : n->in[0], u, e);
            sb_add(b, "    const float v%zu_%d_%d = ", id, u, e);
            emit_expr(b, n, sa, sc);
            sb_add(b, ";\n");
        }
    }
}

/* node nid has a full-shape (stored) output */
static bool stored_node(const plan_t *P, int nid)
{
    for (int o = 0; o < P->nout; o++)
        if (!(P->R > 0 && P->out_red[o]) && P->out_node[o] == nid)
            return true;
    return false;
}

/* In a laundering graph (one that stores, or in another mode of the same
 * caller would store, a node's 16-bit copy) each stored node's value of one
 * copy goes through an empty asm (w<node> names it), and its stores and
 * column sums read that copy: whatever the compiler would make of the
 * product behind it (contracted into a column sum's add, or not, a choice
 * that shifts with the number of stores), every consumer reads the one
 * rounded value, so a node's f32 results are the same bits whether or not
 * its 16-bit copy is also stored.  Elsewhere w<node> is a plain alias. */
static void emit_launder(sbuf *b, const plan_t *P, int vec, int u)
{
    for (int o = 0; o < P->nout; o++) {
        if (P->R > 0 && P->out_red[o])
            continue;
        int nid = P->out_node[o], seen = 0;
        for (int q = 0; q < o; q++)
            seen |= !(P->R > 0 && P->out_red[q]) && P->out_node[q] == nid;
        if (seen)
            continue;
        for (int e = 0; e < vec; e++) {
            if (P->launder)
                sb_add(b, "    float w%d_%d_%d = v%d_%d_%d; __asm__(\"\" : \"+v\"(w%d_%d_%d));\n", nid, u, e, nid, u, e,
                       nid, u, e);
            else
                sb_add(b, "    const float w%d_%d_%d = v%d_%d_%d;\n", nid, u, e, nid, u, e);
        }
    }
}

/* stores of the full-shape (not reduced) outputs of one copy (after
 * emit_launder of that copy) */
static void emit_stores(sbuf *b, const plan_t *P, int vec, const char *idx, int u)
{
    for (int o = 0; o < P->nout; o++) {
        if (P->R > 0 && P->out_red[o])
            continue;
        int nid = P->out_node[o];
        if (P->out_dt16[o]) {
            /* the node's 16-bit copy, rounded as k_cast_to16 rounds; ordinary
             * stores (a GEMM reads the copy next: non-temporal ones measured
             * 1.6 % slower on config 5's unfused graph) */
            const int dt = P->out_dt16[o];
            if (vec == 4 && dt == PG_DTYPE_BF16)
                sb_add(b, "    *(pgu2 *)(out%d + %s) = (pgu2){f32x2_to_bf16x2(w%d_%d_0, w%d_%d_1), "
                          "f32x2_to_bf16x2(w%d_%d_2, w%d_%d_3)};\n", o, idx,
                       nid, u, nid, u, nid, u, nid, u);
            else if (vec == 4)
                sb_add(b, "    *(pgu2 *)(out%d + %s) = (pgu2){(unsigned)f32_to_f16(w%d_%d_0) | ((unsigned)f32_to_f16(w%d_%d_1) << 16), "
                          "(unsigned)f32_to_f16(w%d_%d_2) | ((unsigned)f32_to_f16(w%d_%d_3) << 16)};\n",
                       o, idx, nid, u, nid, u, nid, u, nid, u);
            else
                sb_add(b, "    out%d[%s] = to16(%d, w%d_%d_0);\n", o, idx, dt, nid, u);
            continue;
        }
        /* each output element is written once per launch: stream the stores
         * (and the read of an accumulating output) past the caches */
        if (vec == 4) {
            if (P->out_beta[o])
                sb_add(b, "    { pgf4 *p = (pgf4 *)(out%d + %s); pgf4 t = __builtin_nontemporal_load(p);"
                          " t.x += w%d_%d_0; t.y += w%d_%d_1; t.z += w%d_%d_2; t.w += w%d_%d_3;"
                          " __builtin_nontemporal_store(t, p); }\n",
                       o, idx, nid, u, nid, u, nid, u, nid, u);
            else
                sb_add(b, "    __builtin_nontemporal_store((pgf4){w%d_%d_0, w%d_%d_1, w%d_%d_2, w%d_%d_3}, (pgf4 *)(out%d + %s));\n",
                       nid, u, nid, u, nid, u, nid, u, o, idx);
        } else {
            if (P->out_beta[o])
                sb_add(b, "    __builtin_nontemporal_store(__builtin_nontemporal_load(out%d + %s) + w%d_%d_0, out%d + %s);\n",
                       o, idx, nid, u, o, idx);
            else
                sb_add(b, "    __builtin_nontemporal_store(w%d_%d_0, out%d + %s);\n", nid, u, o, idx);
        }
    }
}

/* the device math helpers (kernels/pgmath.h), embedded by the build */
extern const char pgk_math_source[];

static void emit_prologue(sbuf *b, const plan_t *P)
{
    for (int i = 0; i < P->nin; i++)
        if (P->in_used[i])
            sb_add(b, "  const float *__restrict__ in%d = a.in[%d];\n", i, i);
    for (int o = 0; o < P->nout; o++)
        if (P->out_dt16[o])
            sb_add(b, "  unsigned short *__restrict__ out%d = (unsigned short *)a.out[%d];\n", o, o);
        else if (!(P->R > 0 && P->out_red[o]))
            sb_add(b, "  float *__restrict__ out%d = a.out[%d];\n", o, o);
}

/* kernels/convert16.h, embedded by the build: the f32 -> 16-bit rounding of
 * the hand-written kernels, for programs that store 16-bit copies */
extern const char pgk_convert_source[];

static void emit_headers(sbuf *b, const plan_t *P)
{
    sb_add(b, "%s\n", pgk_math_source);
    bool any16 = false;
    for (int o = 0; o < P->nout; o++)
        any16 = any16 || P->out_dt16[o];
    if (any16)
        sb_add(b, "%s\ntypedef unsigned int pgu2 __attribute__((ext_vector_type(2)));\n", pgk_convert_source);
}

static char *gen_source(const pg_jit_graph *g, const plan_t *P, const bool *reach)
{
    sbuf b = {0};
    bool red = P->R > 0;
    bool wide = P->numel >= ((int64_t)1 << 31);
    sb_add(&b, "// picograd-amd fused elementwise kernel (generated)\n");
    emit_headers(&b, P);
    sb_add(&b, "typedef %s IDX;\n", wide ? "unsigned long long" : "unsigned int");
    sb_add(&b, "typedef float pgf4 __attribute__((ext_vector_type(4)));\n");
    /* exactly the pointers this kernel takes (the host packs the same) */
    const int ni = P->nin ? P->nin : 1, no = P->nout ? P->nout : 1;
    if (red)
        sb_add(&b, "struct PgArgs { const float *in[%d]; float *out[%d]; float *part[%d]; };\n", ni, no, no);
    else
        sb_add(&b, "struct PgArgs { const float *in[%d]; float *out[%d]; };\n", ni, no);
    if (!red) {
        /* grid-stride over the flat loop: two strides per iteration, both
         * copies' loads issued before either copy's math */
        int vec = P->vec;
        sb_add(&b, "extern \"C\" __global__ void __launch_bounds__(256) pgjit_main(PgArgs a) {\n");
        if (g->exact)
            sb_add(&b, "#pragma clang fp contract(off)\n");
        emit_prologue(&b, P);
        sb_add(&b, "  const IDX N = (IDX)%lldULL;\n", (long long)P->numel);
        sb_add(&b, "  const IDX step = (IDX)gridDim.x * 256u * %du;\n", vec);
        sb_add(&b, "  IDX i = ((IDX)blockIdx.x * 256u + threadIdx.x) * %du;\n", vec);
        sb_add(&b, "  for (; i + step < N; i += 2u * step) {\n");
        sb_add(&b, "    const IDX i0 = i, i1 = i + step;\n");
        emit_loads(&b, P, vec, "i0", 0);
        emit_loads(&b, P, vec, "i1", 1);
        emit_compute(&b, g, reach, vec, 0);
        emit_compute(&b, g, reach, vec, 1);
        emit_launder(&b, P, vec, 0);
        emit_launder(&b, P, vec, 1);
        emit_stores(&b, P, vec, "i0", 0);
        emit_stores(&b, P, vec, "i1", 1);
        sb_add(&b, "  }\n  if (i < N) {\n    const IDX i0 = i;\n");
        emit_loads(&b, P, vec, "i0", 0);
        emit_compute(&b, g, reach, vec, 0);
        emit_launder(&b, P, vec, 0);
        emit_stores(&b, P, vec, "i0", 0);
        sb_add(&b, "  }\n}\n");
        return b.s;
    }
    /* reduced outputs: [R x C] tiling; 64 column groups x 4 row lanes, each
     * lane walking rows r, r+4, ... of its block's band, two per iteration */
    int vec = (P->C % 4 == 0 && P->vec == 4) ? 4 : 1;
    sb_add(&b, "extern \"C\" __global__ void __launch_bounds__(256) pgjit_main(PgArgs a) {\n");
    if (g->exact)
        sb_add(&b, "#pragma clang fp contract(off)\n");
    emit_prologue(&b, P);
    sb_add(&b, "  const IDX R = (IDX)%lldULL, C = (IDX)%lldULL;\n", (long long)P->R, (long long)P->C);
    sb_add(&b, "  const IDX tc = threadIdx.x & 63u, tr = threadIdx.x >> 6;\n");
    sb_add(&b, "  const IDX c = ((IDX)blockIdx.x * 64u + tc) * %du;\n", vec);
    sb_add(&b, "  const IDX rows_per = (R + gridDim.y - 1) / gridDim.y;\n");
    sb_add(&b, "  const IDX r0 = (IDX)blockIdx.y * rows_per;\n");
    sb_add(&b, "  const IDX r1 = r0 + rows_per < R ? r0 + rows_per : R;\n");
    for (int o = 0; o < P->nout; o++)
        if (P->out_red[o])
            for (int e = 0; e < vec; e++)
                sb_add(&b, "  float acc%d_%d = 0.0f;\n", o, e);
    sb_add(&b, "  if (c < C) {\n");
    sb_add(&b, "  IDX r = r0 + tr;\n");
    /* PGJ_RED_ROWS rows per lane per iteration, all their loads issued
     * before the first compute; the column sums still add rows in order */
    const int RU = PGJ_RED_ROWS;
    static const char *const iname[8] = {"i0", "i1", "i2", "i3", "i4", "i5", "i6", "i7"};
    sb_add(&b, "  for (; r + %du < r1; r += %du) {\n", 4 * (RU - 1), 4 * RU);
    sb_add(&b, "    const IDX i0 = r * C + c");
    for (int u = 1; u < RU; u++)
        sb_add(&b, ", i%d = i0 + %du * C", u, 4 * u);
    sb_add(&b, ";\n");
    for (int u = 0; u < RU; u++)
        emit_loads(&b, P, vec, iname[u], u);
    for (int u = 0; u < RU; u++)
        emit_compute(&b, g, reach, vec, u);
    for (int u = 0; u < RU; u++)
        emit_launder(&b, P, vec, u);
    for (int u = 0; u < RU; u++)
        for (int o = 0; o < P->nout; o++)
            if (P->out_red[o])
                for (int e = 0; e < vec; e++)
                    sb_add(&b, "    acc%d_%d += %c%d_%d_%d;\n", o, e, stored_node(P, P->out_node[o]) ? 'w' : 'v',
                           P->out_node[o], u, e);
    for (int u = 0; u < RU; u++)
        emit_stores(&b, P, vec, iname[u], u);
    sb_add(&b, "  }\n  for (; r < r1; r += 4u) {\n    const IDX i0 = r * C + c;\n");
    emit_loads(&b, P, vec, "i0", 0);
    emit_compute(&b, g, reach, vec, 0);
    emit_launder(&b, P, vec, 0);
    for (int o = 0; o < P->nout; o++)
        if (P->out_red[o])
            for (int e = 0; e < vec; e++)
                sb_add(&b, "    acc%d_%d += %c%d_0_%d;\n", o, e, stored_node(P, P->out_node[o]) ? 'w' : 'v',
                       P->out_node[o], e);
    emit_stores(&b, P, vec, "i0", 0);
    sb_add(&b, "  }\n  }\n");
    /* combine the 4 row lanes in LDS, fixed order, one partial row per block */
    sb_add(&b, "  __shared__ float red[4][%d];\n", 64 * vec);
    for (int o = 0; o < P->nout; o++) {
        if (!P->out_red[o])
            continue;
        for (int e = 0; e < vec; e++)
            sb_add(&b, "  red[tr][tc * %d + %d] = acc%d_%d;\n", vec, e, o, e);
        sb_add(&b, "  __syncthreads();\n");
        sb_add(&b, "  if (tr == 0 && c < C) {\n");
        for (int e = 0; e < vec; e++)
            sb_add(&b, "    a.part[%d][(IDX)blockIdx.y * C + c + %d] = ((red[0][tc*%d+%d] + red[1][tc*%d+%d]) + "
                       "red[2][tc*%d+%d]) + red[3][tc*%d+%d];\n",
                   o, e, vec, e, vec, e, vec, e, vec, e);
        sb_add(&b, "  }\n  __syncthreads();\n");
    }
    sb_add(&b, "}\n");
    /* finisher: out[c] (beta ? += : =) sum over blocks of part[blk][c].
     * 8 column lanes x 128 block lanes per workgroup of 1024 (32 columns
     * with four per lane: each partial row is read as whole 128-byte
     * lines, and a [.., 4096] grad takes 128 workgroups with every load in
     * flight at once); block lane q sums partial rows q, q + 128, ... in
     * that order (eight loads in flight, the adds still in row order) and
     * the 128 lanes are combined by a fixed pairwise tree, so the result
     * does not depend on timing.  Four columns per lane when C allows it. */
    sb_add(&b, "extern \"C\" __global__ void __launch_bounds__(1024) pgjit_fin(PgArgs a, unsigned nblk) {\n");
    sb_add(&b, "  const IDX C = (IDX)%lldULL;\n", (long long)P->C);
    sb_add(&b, "  const IDX tc = threadIdx.x & 7u, tr = threadIdx.x >> 3;\n");
    const char *T = vec == 4 ? "pgf4" : "float";
    sb_add(&b, "  const IDX c = ((IDX)blockIdx.x * 8u + tc) * %du;\n", vec);
    sb_add(&b, "  __shared__ %s red[128][9];\n", T);
    for (int o = 0; o < P->nout; o++) {
        if (!P->out_red[o])
            continue;
        sb_add(&b, "  { const float *__restrict__ pp = a.part[%d];\n", o);
        sb_add(&b, "    %s s = (%s)(0.0f);\n", T, T);
        sb_add(&b, "    if (c < C) {\n      unsigned k = tr;\n");
        sb_add(&b, "      for (; k + 896u < nblk; k += 1024u) {\n        %s v[8];\n", T);
        sb_add(&b, "#pragma unroll\n        for (int q = 0; q < 8; q++) v[q] = *(const %s *)(pp + (IDX)(k + 128u * q) * C + c);\n", T);
        sb_add(&b, "#pragma unroll\n        for (int q = 0; q < 8; q++) s += v[q];\n      }\n");
        sb_add(&b, "      for (; k < nblk; k += 128u) s += *(const %s *)(pp + (IDX)k * C + c);\n    }\n", T);
        sb_add(&b, "    red[tr][tc] = s; __syncthreads();\n");
        sb_add(&b, "    for (unsigned h = 64u; h > 0u; h >>= 1) {\n");
        sb_add(&b, "      if (tr < h) red[tr][tc] += red[tr + h][tc];\n      __syncthreads();\n    }\n");
        sb_add(&b, "    if (tr == 0 && c < C) {\n");
        if (P->out_beta[o])
            sb_add(&b, "      *(%s *)(a.out[%d] + c) += red[0][tc]; }\n", T, o);
        else
            sb_add(&b, "      *(%s *)(a.out[%d] + c) = red[0][tc]; }\n", T, o);
        sb_add(&b, "    __syncthreads(); }\n");
    }
    sb_add(&b, "}\n");
    return b.s;
}

bool pgj_small_reduce_fits(size_t lnd, const size_t *ls)
{
    return lnd == 2 && pgk_sum_all2_fits(ls[0], ls[1]);
}

/* The one-block kernel of a small run (PGJ_SMALL_THREADS lanes):
 *  1. the uploads handed over by the device layer: 16-byte pieces of up to
 *     PGJ_SMALL_UPLOADS entries, four pieces per lane in flight (the source
 *     is host memory read over the bus), then a barrier, after which every
 *     lane sees the uploaded inputs;
 *  2. the run itself, the grid-stride body over one block;
 *  3. with red_out >= 0, reduce_all's two stages over that output, as
 *     k_sum_all2: the output staged in LDS, lane j adds column j over the
 *     rows in order, lane 0 adds the column sums in order and scales. */
static char *gen_source_small(const pg_jit_graph *g, const plan_t *P, const bool *reach, int red_out, size_t lnd,
                              const size_t *ls)
{
    sbuf b = {0};
    const int ni = P->nin ? P->nin : 1, no = P->nout ? P->nout : 1;
    const int vec = P->vec, T = PGJ_SMALL_THREADS;
    sb_add(&b, "// picograd-amd fused elementwise kernel, one-block run (generated)\n");
    emit_headers(&b, P);
    sb_add(&b, "typedef unsigned int IDX;\n");
    sb_add(&b, "typedef float pgf4 __attribute__((ext_vector_type(4)));\n");
    sb_add(&b, "typedef unsigned int pgu4 __attribute__((ext_vector_type(4)));\n");
    sb_add(&b, "struct PgUp { unsigned char *dst; const unsigned char *src; unsigned long long n; };\n");
    sb_add(&b, "struct PgArgs { const float *in[%d]; float *out[%d]; PgUp up[%d]; unsigned nup, up_pieces;"
               " float *r1, *r2; float scale; };\n", ni, no, PGJ_SMALL_UPLOADS);
    sb_add(&b, "static_assert(sizeof(PgArgs) == %zu, \"argument block layout\");\n",
           (size_t)(ni + no) * sizeof(void *) + sizeof(small_tail));
    sb_add(&b, "extern \"C\" __global__ void __launch_bounds__(%d) pgjit_small(PgArgs a) {\n", T);
    if (g->exact)
        sb_add(&b, "#pragma clang fp contract(off)\n");
    /* 1. uploads */
    sb_add(&b, "  if (a.up_pieces) {\n");
    sb_add(&b, "    const unsigned P = a.up_pieces;\n");
    sb_add(&b, "    unsigned base[%d]; unsigned acc = 0;\n", PGJ_SMALL_UPLOADS);
    sb_add(&b, "#pragma unroll\n    for (int e = 0; e < %d; ++e) { base[e] = acc; acc += e < (int)a.nup ?"
               " (unsigned)(a.up[e].n / 16u) : 0u; }\n", PGJ_SMALL_UPLOADS);
    sb_add(&b, "    for (unsigned p0 = threadIdx.x; p0 < P; p0 += 4u * %du) {\n", T);
    sb_add(&b, "      pgu4 v[4]; unsigned q[4]; int en[4];\n");
    sb_add(&b, "#pragma unroll\n      for (int k = 0; k < 4; ++k) {\n");
    sb_add(&b, "        const unsigned p = p0 + (unsigned)k * %du; q[k] = p < P ? p : P - 1u;\n", T);
    sb_add(&b, "        int e = 0;\n#pragma unroll\n        for (int j = 1; j < %d; ++j) e += (j < (int)a.nup && q[k] >= base[j]) ? 1 : 0;\n",
           PGJ_SMALL_UPLOADS);
    sb_add(&b, "        en[k] = e; v[k] = ((const pgu4 *)a.up[e].src)[q[k] - base[e]];\n      }\n");
    sb_add(&b, "#pragma unroll\n      for (int k = 0; k < 4; ++k)\n");
    sb_add(&b, "        if (p0 + (unsigned)k * %du < P) ((pgu4 *)a.up[en[k]].dst)[q[k] - base[en[k]]] = v[k];\n", T);
    sb_add(&b, "    }\n    __syncthreads();\n  }\n");
    /* 2. the run */
    emit_prologue(&b, P);
    sb_add(&b, "  {\n  const IDX N = (IDX)%lldu;\n", (long long)P->numel);
    sb_add(&b, "  const IDX step = %du * %du;\n", T, vec);
    sb_add(&b, "  IDX i = (IDX)threadIdx.x * %du;\n", vec);
    sb_add(&b, "  for (; i + step < N; i += 2u * step) {\n");
    sb_add(&b, "    const IDX i0 = i, i1 = i + step;\n");
    emit_loads(&b, P, vec, "i0", 0);
    emit_loads(&b, P, vec, "i1", 1);
    emit_compute(&b, g, reach, vec, 0);
    emit_compute(&b, g, reach, vec, 1);
    emit_launder(&b, P, vec, 0);
    emit_launder(&b, P, vec, 1);
    emit_stores(&b, P, vec, "i0", 0);
    emit_stores(&b, P, vec, "i1", 1);
    sb_add(&b, "  }\n  if (i < N) {\n    const IDX i0 = i;\n");
    emit_loads(&b, P, vec, "i0", 0);
    emit_compute(&b, g, reach, vec, 0);
    emit_launder(&b, P, vec, 0);
    emit_stores(&b, P, vec, "i0", 0);
    sb_add(&b, "  }\n  }\n");
    /* 3. the reduction */
    if (red_out >= 0 && lnd == 2) {
        const long long R = (long long)ls[0], C = (long long)ls[1];
        sb_add(&b, "  __syncthreads();\n");
        sb_add(&b, "  __shared__ float tile[%lld];\n  __shared__ float col[%lld];\n", R * C, C);
        sb_add(&b, "  {\n    const float *__restrict__ y = a.out[%d];\n", red_out);
        sb_add(&b, "    for (int i0 = threadIdx.x; i0 < %lld; i0 += 4 * %d) {\n      float v[4];\n", R * C, T);
        sb_add(&b, "#pragma unroll\n      for (int k = 0; k < 4; ++k) { const int i = i0 + k * %d; v[k] = y[i < %lld ? i : %lld]; }\n",
               T, R * C, R * C - 1);
        sb_add(&b, "#pragma unroll\n      for (int k = 0; k < 4; ++k) { const int i = i0 + k * %d; if (i < %lld) tile[i] = v[k]; }\n    }\n  }\n",
               T, R * C);
        sb_add(&b, "  __syncthreads();\n");
        sb_add(&b, "  if (threadIdx.x < %lldu) {\n    float acc = 0.0f;\n", C);
        sb_add(&b, "#pragma unroll 8\n    for (int l = 0; l < %lld; ++l) acc += tile[l * %lld + (int)threadIdx.x];\n", R, C);
        sb_add(&b, "    col[threadIdx.x] = acc;\n    a.r1[threadIdx.x] = acc;\n  }\n  __syncthreads();\n");
        sb_add(&b, "  if (threadIdx.x == 0) {\n    float acc = 0.0f;\n");
        sb_add(&b, "    for (int l = 0; l < %lld; ++l) acc += col[l];\n    a.r2[0] = acc * a.scale;\n  }\n", C);
    }
    sb_add(&b, "}\n");
    return b.s;
}

/* ---------------------------------------------------------------- compile */

static const char *cache_dir(void)
{
    static char dir[512];
    if (dir[0])
        return dir;
    const char *e = getenv("PG_JIT_CACHE_DIR");
    if (e && *e)
        snprintf(dir, sizeof dir, "%s", e);
    else
        snprintf(dir, sizeof dir, "/tmp/picograd_amd_jit_%d", (int)getuid());
    mkdir(dir, 0700);
    return dir;
}

static void *read_file(const char *path, size_t *n)
{
    FILE *f = fopen(path, "rb");
    if (!f)
        return NULL;
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *p = sz > 0 ? malloc((size_t)sz) : NULL;
    if (p && fread(p, 1, (size_t)sz, f) != (size_t)sz) {
        free(p);
        p = NULL;
    }
    fclose(f);
    *n = p ? (size_t)sz : 0;
    return p;
}

static void write_file_atomic(const char *path, const void *p, size_t n)
{
    char tmp[700];
    snprintf(tmp, sizeof tmp, "%s.%d.tmp", path, (int)getpid());
    FILE *f = fopen(tmp, "wb");
    if (!f)
        return;
    bool ok = fwrite(p, 1, n, f) == n;
    ok = fclose(f) == 0 && ok;
    if (ok)
        rename(tmp, path);
    else
        unlink(tmp);
}

static bool compile_source(const char *src, hipModule_t *mod)
{
    uint64_t h = fnv(src, strlen(src), 14695981039346656037ULL);
    h = fnv("gfx950-v4", 9, h);
    char path[600];
    snprintf(path, sizeof path, "%s/%016llx.hsaco", cache_dir(), (unsigned long long)h);
    const char *force = getenv("PG_JIT_FORCE_COMPILE_ERROR");
    size_t n = 0;
    void *code = force ? NULL : read_file(path, &n);
    if (!code) {
        hiprtcProgram prog;
        const char *body = force ? "this is not HIP" : src;
        if (hiprtcCreateProgram(&prog, body, "pgjit.hip", 0, NULL, NULL) != HIPRTC_SUCCESS) {
            jset_err("hiprtcCreateProgram failed");
            return false;
        }
        const char *opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                              "-packed-fp32-ops"};
        hiprtcResult r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
        if (r != HIPRTC_SUCCESS) {
            size_t ls = 0;
            hiprtcGetProgramLogSize(prog, &ls);
            char *log = malloc(ls + 1);
            if (log) {
                hiprtcGetProgramLog(prog, log);
                log[ls] = 0;
                jset_err("hiprtc compile failed: %.900s", log);
                free(log);
            } else {
                jset_err("hiprtc compile failed");
            }
            hiprtcDestroyProgram(&prog);
            return false;
        }
        hiprtcGetCodeSize(prog, &n);
        code = malloc(n);
        if (!code || hiprtcGetCode(prog, code) != HIPRTC_SUCCESS) {
            free(code);
            hiprtcDestroyProgram(&prog);
            jset_err("hiprtcGetCode failed");
            return false;
        }
        hiprtcDestroyProgram(&prog);
        pgj_stat_compiles++;
        write_file_atomic(path, code, n);
    }
    if (!pgd_ok()) {
        free(code);
        jset_err("no device: %s", pg_amd_last_error());
        return false;
    }
    hipError_t e = hipModuleLoadData(mod, code);
    free(code);
    if (e != hipSuccess) {
        jset_err("hipModuleLoadData: %s", hipGetErrorString(e));
        return false;
    }
    return true;
}

static void entry_free(centry *e)
{
    if (!e)
        return;
    if (e->mod) {
        pgd_sync();
        hipModuleUnload(e->mod);
    }
    pg_jit_graph_free(e->g);
    free(e);
}

/* finds or builds the kernel for (g, loop shape) */
static centry *get_entry(const pg_jit_graph *g, size_t lnd, const size_t *ls, int variant, bool *owned)
{
    uint64_t h = pg_jit_graph_hash(g);
    h = fnv(&lnd, sizeof lnd, h);
    h = fnv(ls, lnd * sizeof(size_t), h);
    h = fnv(&variant, sizeof variant, h);
    *owned = false;
    if (g_cache_on) {
        for (centry *e = g_cache; e; e = e->next)
            if (e->hash == h && e->variant == variant && e->loop_ndim == lnd &&
                !memcmp(e->loop_shape, ls, lnd * sizeof(size_t)) && graph_equal(g, e->g)) {
                pgj_stat_hits++;
                return e;
            }
    }
    if (g->nout == 0) {
        jset_err("graph has no outputs");
        return NULL;
    }
    if (g->nin > MAXIO * 2 || g->nout > MAXIO * 2) {
        jset_err("too many inputs/outputs");
        return NULL;
    }
    bool *reach = calloc(g->nn ? g->nn : 1, 1);
    if (!reach) {
        jset_err("oom");
        return NULL;
    }
    mark_reach(g, reach);
    plan_t P;
    if (!make_plan(g, lnd, ls, &P, reach)) {
        free(reach);
        return NULL;
    }
    bool red = false;
    for (int o = 0; o < P.nout; o++)
        red |= P.out_red[o] != 0;
    if (!red)
        P.R = 0;
    if (variant != PGJ_VAR_MAIN && (red || P.numel > PGJ_SMALL_MAX)) {
        free(reach);
        jset_err("run too large or reduced: no one-block kernel");
        return NULL;
    }
    char *src = variant == PGJ_VAR_MAIN ? gen_source(g, &P, reach)
                                        : gen_source_small(g, &P, reach, variant - PGJ_VAR_SMALL - 1, lnd, ls);
    free(reach);
    if (!src) {
        jset_err("codegen failed");
        return NULL;
    }
    if (getenv("PG_JIT_DUMP"))
        fprintf(stderr, "---- pgjit source ----\n%s\n", src);
    centry *e = calloc(1, sizeof *e);
    if (!e) {
        free(src);
        jset_err("oom");
        return NULL;
    }
    e->hash = h;
    e->variant = variant;
    e->nin = g->nin;
    e->nout = g->nout;
    e->loop_ndim = lnd;
    memcpy(e->loop_shape, ls, lnd * sizeof(size_t));
    bool ok = compile_source(src, &e->mod);
    free(src);
    if (!ok ||
        hipModuleGetFunction(&e->fmain, e->mod, variant == PGJ_VAR_MAIN ? "pgjit_main" : "pgjit_small") !=
            hipSuccess ||
        (red && hipModuleGetFunction(&e->ffin, e->mod, "pgjit_fin") != hipSuccess)) {
        if (ok)
            jset_err("kernel symbol missing");
        entry_free(e);
        return NULL;
    }
    e->has_red = red;
    if (variant != PGJ_VAR_MAIN) {
        e->grid_x = e->grid_y = 1;
    } else if (!red) {
        int64_t items = (P.numel + P.vec - 1) / P.vec;
        int64_t blocks = (items + 255) / 256;
        if (blocks > 256 * 16)
            blocks = 256 * 16;
        e->grid_x = (unsigned)(blocks < 1 ? 1 : blocks);
        e->grid_y = 1;
    } else {
        int vec = (P.C % 4 == 0 && P.vec == 4) ? 4 : 1;
        int64_t cb = (P.C + 64 * vec - 1) / (64 * vec);
        /* ~16K short-lived blocks of >= 16 rows (4 per row lane, one
         * iteration of PGJ_RED_ROWS = 4): measured on the config-2 shape,
         * 16-row bands take 176 us with 2 rows per lane per iteration and
         * 173 us with 4, against 195 us for 32-row bands and 202 us for
         * 64-row ones; the extra partial rows cost the finisher ~1 us */
        int64_t rb = 16384 / (cb ? cb : 1);
        if (rb < 1)
            rb = 1;
        int64_t max_rb = (P.R + 15) / 16;
        if (rb > max_rb)
            rb = max_rb;
        if (rb < 1)
            rb = 1;
        if (rb > 65535)
            rb = 65535;
        e->grid_x = (unsigned)cb;
        e->grid_y = (unsigned)rb;
        e->fin_grid = (unsigned)((P.C + 8 * vec - 1) / (8 * vec));
        size_t off = 0;
        for (int o = 0; o < P.nout; o++) {
            e->part_floats[o] = P.out_red[o] ? (size_t)rb * (size_t)P.C : 0;
            e->part_off[o] = off;
            off += (e->part_floats[o] + 63) / 64 * 64;
        }
        e->part_total = off;
    }
    e->g = graph_clone(g);
    if (!e->g) {
        entry_free(e);
        jset_err("oom");
        return NULL;
    }
    if (g_cache_on) {
        e->next = g_cache;
        g_cache = e;
        g_cache_n++;
    } else {
        *owned = true;
    }
    return e;
}

/* The kernel's argument block: in[max(1, nin)], out[max(1, nout)], then
 * part[max(1, nout)] for a reduced kernel or the small kernel's tail: only
 * the bytes the kernel declares are passed, not a fixed maximum. */
typedef struct {
    void *p[MAXIO * 6];
    small_tail tail; /* follows p[0 .. k) in the small kernel's block (see pack_small) */
} kargs;

static size_t pack_ptrs(void **p, const void *const *inputs, size_t nin, void *const *outputs, size_t nout)
{
    size_t k = 0;
    for (size_t i = 0; i < (nin ? nin : 1); i++)
        p[k++] = i < nin ? (void *)inputs[i] : NULL;
    for (size_t i = 0; i < (nout ? nout : 1); i++)
        p[k++] = i < nout ? outputs[i] : NULL;
    return k;
}

static bool launch_entry(centry *e, const void *const *inputs, size_t nin, void *const *outputs, size_t nout)
{
    kargs a;
    size_t k = pack_ptrs(a.p, inputs, nin, outputs, nout);
    hipStream_t s = (hipStream_t)pgd_stream();
    if (e->has_red) {
        float *part = pgd_scratch(0, e->part_total * sizeof(float));
        if (!part) {
            jset_err("scratch alloc failed");
            return false;
        }
        for (size_t o = 0; o < (nout ? nout : 1); o++)
            a.p[k++] = o < nout && e->part_floats[o] ? part + e->part_off[o] : NULL;
    }
    void *params[] = {a.p};
    int tk = pgd_tbegin(PGD_T_JIT_MAIN);
    hipError_t err = hipModuleLaunchKernel(e->fmain, e->grid_x, e->grid_y, 1, 256, 1, 1, 0, s, params, NULL);
    pgd_tend(tk);
    if (err == hipSuccess && e->has_red) {
        unsigned nblk = e->grid_y;
        void *fparams[] = {a.p, &nblk};
        tk = pgd_tbegin(PGD_T_JIT_FIN);
        err = hipModuleLaunchKernel(e->ffin, e->fin_grid, 1, 1, 1024, 1, 1, 0, s, fparams, NULL);
        pgd_tend(tk);
    }
    if (err != hipSuccess) {
        jset_err("hipModuleLaunchKernel: %s", hipGetErrorString(err));
        return false;
    }
    return true;
}

bool pgj_launch(pg_jit_graph *g, size_t lnd, const size_t *ls, const void *const *inputs, size_t nin,
                void *const *outputs, size_t nout)
{
    if (!g || nin != g->nin || nout != g->nout) {
        jset_err("pgj_launch: argument count mismatch");
        return false;
    }
    bool owned = false;
    centry *e = get_entry(g, lnd, ls, PGJ_VAR_MAIN, &owned);
    if (!e)
        return false;
    bool ok = launch_entry(e, inputs, nin, outputs, nout);
    if (owned)
        entry_free(e);
    return ok;
}

bool pgj_small_fits(size_t numel, size_t nup, const pgk_upload *up)
{
    if (numel > PGJ_SMALL_MAX || nup > PGJ_SMALL_UPLOADS)
        return false;
    size_t bytes = 0;
    for (size_t i = 0; i < nup; i++) {
        if ((((uintptr_t)up[i].dst) | ((uintptr_t)up[i].src) | up[i].n) & 15)
            return false;
        bytes += up[i].n;
    }
    return bytes <= PGJ_SMALL_UPLOAD_BYTES;
}

bool pgj_launch_small(pg_jit_graph *g, size_t lnd, const size_t *ls, const void *const *inputs, size_t nin,
                      void *const *outputs, size_t nout, const pgk_upload *up, size_t nup, int red_out, float *r1,
                      float *r2, float scale)
{
    if (!g || nin != g->nin || nout != g->nout || (red_out >= 0 && (size_t)red_out >= nout)) {
        jset_err("pgj_launch_small: argument mismatch");
        return false;
    }
    size_t numel = pg_shape_numel(lnd, ls);
    if (!pgj_small_fits(numel, nup, up) || (red_out >= 0 && !pgj_small_reduce_fits(lnd, ls))) {
        jset_err("pgj_launch_small: run does not fit one block");
        return false;
    }
    bool owned = false;
    centry *e = get_entry(g, lnd, ls, PGJ_VAR_SMALL + 1 + red_out, &owned);
    if (!e)
        return false;
    kargs a;
    size_t k = pack_ptrs(a.p, inputs, nin, outputs, nout);
    small_tail t;
    memset(&t, 0, sizeof t);
    size_t pieces = 0;
    for (size_t i = 0; i < nup; i++) {
        t.up[i] = up[i];
        pieces += up[i].n / 16;
    }
    t.nup = (unsigned)nup;
    t.up_pieces = (unsigned)pieces;
    t.r1 = r1;
    t.r2 = r2;
    t.scale = scale;
    /* the tail follows the pointers in one block (pointer-aligned) */
    unsigned char blockbuf[sizeof a.p + sizeof t];
    memcpy(blockbuf, a.p, k * sizeof(void *));
    memcpy(blockbuf + k * sizeof(void *), &t, sizeof t);
    void *params[] = {blockbuf};
    hipStream_t s = (hipStream_t)pgd_stream();
    int tk = pgd_tbegin(PGD_T_JIT_MAIN);
    hipError_t err = hipModuleLaunchKernel(e->fmain, 1, 1, 1, PGJ_SMALL_THREADS, 1, 1, 0, s, params, NULL);
    pgd_tend(tk);
    if (owned)
        entry_free(e);
    if (err != hipSuccess) {
        jset_err("hipModuleLaunchKernel: %s", hipGetErrorString(err));
        return false;
    }
    return true;
}

/* ---------------------------------------------------------------- public API */

pg_jit_exe *pg_jit_compile(pg_jit_graph *g)
{
    if (!g) {
        jset_err("null graph");
        return NULL;
    }
    if (g->nout == 0) {
        jset_err("graph has no outputs");
        return NULL;
    }
    if (g->nin > MAXIO || g->nout > MAXIO) {
        jset_err("too many inputs/outputs (max 16)");
        return NULL;
    }
    const jnode *o0 = &g->nodes[g->outs[0].node];
    for (size_t i = 1; i < g->nout; i++) {
        const jnode *o = &g->nodes[g->outs[i].node];
        if (!pg_shape_equal(o->ndim, o->shape, o0->ndim, o0->shape)) {
            jset_err("multi-output with different shape not supported");
            return NULL;
        }
    }
    bool owned = false;
    centry *e = get_entry(g, o0->ndim, o0->shape, PGJ_VAR_MAIN, &owned);
    if (!e)
        return NULL;
    pg_jit_exe *x = calloc(1, sizeof *x);
    if (!x) {
        if (owned)
            entry_free(e);
        jset_err("oom");
        return NULL;
    }
    x->e = e;
    x->owned = owned;
    x->nin = g->nin;
    x->nout = g->nout;
    for (size_t i = 0; i < g->nin; i++) {
        const jnode *n = &g->nodes[g->inputs[i]];
        x->in_ndim[i] = n->ndim;
        memcpy(x->in_shape[i], n->shape, n->ndim * sizeof(size_t));
    }
    for (size_t i = 0; i < g->nout; i++) {
        x->out_ndim[i] = g->outs[i].ndim;
        memcpy(x->out_shape[i], g->outs[i].shape, g->outs[i].ndim * sizeof(size_t));
    }
    return x;
}

void pg_jit_exe_free(pg_jit_exe *exe)
{
    if (!exe)
        return;
    if (exe->owned)
        entry_free(exe->e);
    free(exe);
}

bool pg_jit_run(pg_jit_exe *exe, const pg_tensor **inputs, size_t ninputs, pg_tensor **outputs, size_t noutputs)
{
    if (!exe || !inputs || !outputs) {
        jset_err("null args");
        return false;
    }
    if (ninputs != exe->nin || noutputs != exe->nout) {
        jset_err("mismatched ninputs/noutputs: got %zu/%zu expected %zu/%zu", ninputs, noutputs, exe->nin,
                 exe->nout);
        return false;
    }
    const void *ip[MAXIO];
    void *op[MAXIO];
    for (size_t i = 0; i < ninputs; i++) {
        const pg_tensor *t = inputs[i];
        if (!t || !t->dev) {
            jset_err("null input %zu", i);
            return false;
        }
        if (!pg_shape_equal(t->ndim, t->shape, exe->in_ndim[i], exe->in_shape[i])) {
            jset_err("input %zu shape mismatch", i);
            return false;
        }
        if (t->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(t)) {
            jset_err("input %zu must be contiguous f32", i);
            return false;
        }
        pgt_materialize((pg_tensor *)t);
        ip[i] = t->dev;
    }
    for (size_t i = 0; i < noutputs; i++) {
        pg_tensor *t = outputs[i];
        if (!t || !t->dev) {
            jset_err("null output %zu", i);
            return false;
        }
        if (!pg_shape_equal(t->ndim, t->shape, exe->out_ndim[i], exe->out_shape[i])) {
            jset_err("output %zu shape mismatch", i);
            return false;
        }
        if (t->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(t)) {
            jset_err("output %zu must be contiguous f32", i);
            return false;
        }
        t->pg_flags &= ~PG_TENSOR_ZERO_PENDING;
        pgt_overwrite(t);
        pgt_touch(t); /* its 16-bit copy, if any, is stale */
        op[i] = t->dev;
    }
    return launch_entry(exe->e, ip, ninputs, op, noutputs);
}

pg_tensor *pg_jit_run_single(pg_jit_exe *exe, const pg_tensor **inputs, size_t ninputs)
{
    if (!exe) {
        jset_err("null exe");
        return NULL;
    }
    if (exe->nout != 1) {
        jset_err("run_single expects 1 output, got %zu", exe->nout);
        return NULL;
    }
    pg_tensor *out = pgt_alloc(PG_DTYPE_F32, exe->out_ndim[0], exe->out_shape[0]);
    if (!out) {
        jset_err("alloc output failed");
        return NULL;
    }
    pg_tensor *outs[1] = {out};
    if (!pg_jit_run(exe, inputs, ninputs, outs, 1)) {
        pg_tensor_free(out);
        return NULL;
    }
    return out;
}

void pg_jit_cache_clear(void)
{
    centry *e = g_cache;
    while (e) {
        centry *nx = e->next;
        entry_free(e);
        e = nx;
    }
    g_cache = NULL;
    g_cache_n = 0;
}
