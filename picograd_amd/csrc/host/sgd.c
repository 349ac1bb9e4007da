/*
 * SGD over device-resident parameters (reference opt/sgd.c).
 *
 * Same registration, defaults, config checks, lazily zeroed momentum
 * buffer and zero_grad-frees-grads behaviour as sgd.c:18-109; the update of
 * sgd.c:147-160 runs for all parameters in one multi-tensor kernel launch
 * (up to 32 tensors per launch, blockIdx.y picks the tensor).
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <assert.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    pg_node *param;
    pg_tensor *buf;
} sgd_state;

struct pg_sgd {
    pg_sgd_cfg cfg;
    sgd_state *st;
    size_t n, cap;
};

pg_sgd_cfg pg_sgd_cfg_default(void)
{
    pg_sgd_cfg c = {.lr = 0.01f, .momentum = 0.0f, .dampening = 0.0f, .weight_decay = 0.0f, .nesterov = false};
    return c;
}

pg_sgd *pg_sgd_new(const pg_sgd_cfg *cfg)
{
    pg_sgd_cfg def = pg_sgd_cfg_default();
    if (!cfg)
        cfg = &def;
    /* sgd.c:43-47 */
    assert(cfg->lr >= 0.0f);
    assert(cfg->momentum >= 0.0f);
    assert(cfg->dampening >= 0.0f);
    assert(cfg->weight_decay >= 0.0f);
    assert(!cfg->nesterov || (cfg->momentum > 0.0f && cfg->dampening == 0.0f));
    pg_sgd *o = calloc(1, sizeof *o);
    if (!o)
        return NULL;
    o->cfg = *cfg;
    return o;
}

void pg_sgd_free(pg_sgd *opt)
{
    if (!opt)
        return;
    for (size_t i = 0; i < opt->n; i++) {
        pg_node_free(opt->st[i].param);
        pg_tensor_free(opt->st[i].buf);
    }
    free(opt->st);
    free(opt);
}

int pg_sgd_add_param(pg_sgd *opt, pg_node *param)
{
    assert(opt && param && param->requires_grad);
    if (opt->n == opt->cap) {
        size_t nc = opt->cap ? opt->cap * 2 : 8;
        sgd_state *p = realloc(opt->st, nc * sizeof *p);
        if (!p)
            return -1;
        opt->st = p;
        opt->cap = nc;
    }
    opt->st[opt->n].param = pg_node_retain(param);
    opt->st[opt->n].buf = NULL;
    opt->n++;
    return 0;
}

size_t pg_sgd_num_params(const pg_sgd *opt) { return opt ? opt->n : 0; }

pg_tensor *pg_amd_sgd_buffer(pg_sgd *opt, size_t i)
{
    return opt && i < opt->n ? opt->st[i].buf : NULL;
}

void pg_sgd_zero_grad(pg_sgd *opt)
{
    assert(opt);
    for (size_t i = 0; i < opt->n; i++) {
        pg_node *p = opt->st[i].param;
        if (p->grad) {
            pg_tensor_free(p->grad);
            p->grad = NULL;
        }
    }
}

void pg_sgd_step(pg_sgd *opt)
{
    assert(opt);
    if (!pgd_ok())
        return;
    const pg_sgd_cfg c = opt->cfg;
    pgk_sgd_seg *segs = calloc(opt->n ? opt->n : 1, sizeof *segs);
    if (!segs)
        return;
    int ns = 0;
    for (size_t i = 0; i < opt->n; i++) {
        pg_node *p = opt->st[i].param;
        pg_tensor *g = p->grad;
        if (!g)
            continue;
        assert(g->numel == p->value->numel);
        if (p->value->dtype != PG_DTYPE_F32) {
            pga_set_err("pg_sgd_step: parameter storage must be f32");
            continue;
        }
        /* a pending zero is written; a pending clip scale is applied by
         * the update kernel as it reads the grad (it stays pending on the
         * grad's storage for any other reader) */
        if (g->pg_flags & PG_TENSOR_ZERO_PENDING)
            pgt_materialize(g);
        pgt_settle(p->value); /* the parameter's own elements, if any are pending */
        const pg_data_ref *gr = g->data_ref;
        if (c.momentum != 0.0f && !opt->st[i].buf) {
            opt->st[i].buf = pg_tensor_zeros(p->value->ndim, p->value->shape);
            if (!opt->st[i].buf)
                continue;
        }
        segs[ns].p = p->value->dev;
        segs[ns].g = g->dev;
        segs[ns].gclip = gr && gr->clip_pending;
        segs[ns].gmul = segs[ns].gclip ? gr->clip_mul : 1.0f;
        segs[ns].ginv = segs[ns].gclip ? gr->clip_inv : 1.0f;
        segs[ns].buf = c.momentum != 0.0f ? opt->st[i].buf->dev : NULL;
        /* a 16-bit shadow of the parameter (kept for the MFMA GEMMs) is
         * rewritten from the updated values in the same pass */
        pg_data_ref *r = p->value->data_ref;
        bool shadow = r && r->shadow && p->value->dev == r->ptr && p->value->numel * 4 == r->nbytes;
        segs[ns].shadow = shadow ? r->shadow : NULL;
        segs[ns].shadow_dtype = shadow ? r->shadow_dtype : 0;
        segs[ns].shadow_cols = shadow ? r->shadow_cols : 0;
        segs[ns].shadow_ld = shadow ? r->shadow_ld : 0;
        if (shadow)
            r->shadow_stale = false;
        else
            pgt_touch(p->value);
        segs[ns].n = p->value->numel;
        ns++;
    }
    int tk = ns ? pgd_tbegin(PGD_T_SGD) : -1;
    if (ns)
        pgd_check(pgk_sgd_multi(segs, ns, c.lr, c.momentum, c.dampening, c.weight_decay, c.nesterov ? 1 : 0,
                                pgd_stream()),
                  "pg_sgd_step");
    pgd_tend(tk);
    free(segs);
}

/* ---------------- momentum checkpoint ("PGSG") ---------------- */

bool pg_amd_sgd_save_fp(const pg_sgd *opt, FILE *fp)
{
    if (!opt || !fp)
        return false;
    const uint32_t ver = 1;
    const uint64_t n = (uint64_t)opt->n;
    if (fwrite("PGSG", 1, 4, fp) != 4 || fwrite(&ver, 4, 1, fp) != 1 || fwrite(&n, 8, 1, fp) != 1)
        return false;
    for (size_t i = 0; i < opt->n; i++) {
        const uint32_t has = opt->st[i].buf ? 1u : 0u;
        if (fwrite(&has, 4, 1, fp) != 1)
            return false;
        if (has && !pg_tensor_save_fp(opt->st[i].buf, fp))
            return false;
    }
    return true;
}

bool pg_amd_sgd_save(const pg_sgd *opt, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "wb");
    if (!fp)
        return false;
    bool ok = pg_amd_sgd_save_fp(opt, fp);
    return fclose(fp) == 0 && ok;
}

bool pg_amd_sgd_load_into_fp(pg_sgd *opt, FILE *fp)
{
    if (!opt || !fp)
        return false;
    char magic[4];
    uint32_t ver = 0;
    uint64_t n = 0;
    if (fread(magic, 1, 4, fp) != 4 || memcmp(magic, "PGSG", 4) != 0)
        return false;
    if (fread(&ver, 4, 1, fp) != 1 || ver != 1)
        return false;
    if (fread(&n, 8, 1, fp) != 1 || n != (uint64_t)opt->n)
        return false;
    for (size_t i = 0; i < opt->n; i++) {
        uint32_t has = 0;
        if (fread(&has, 4, 1, fp) != 1 || has > 1)
            return false;
        sgd_state *s = &opt->st[i];
        if (!has) {
            pg_tensor_free(s->buf);
            s->buf = NULL;
            continue;
        }
        const pg_tensor *v = s->param->value;
        if (!s->buf) {
            s->buf = pg_tensor_empty_dtype(PG_DTYPE_F32, v->ndim, v->shape);
            if (!s->buf)
                return false;
        }
        if (!pgc_load_into(s->buf, fp))
            return false;
    }
    return true;
}

bool pg_amd_sgd_load_into(pg_sgd *opt, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "rb");
    if (!fp)
        return false;
    bool ok = pg_amd_sgd_load_into_fp(opt, fp);
    fclose(fp);
    return ok;
}
