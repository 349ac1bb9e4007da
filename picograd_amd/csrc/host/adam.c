/*
 * Adam / AdamW over device-resident parameters (reference opt/adam.c).
 *
 * Registration, defaults, config checks, per-parameter lr / weight-decay
 * overrides, lazily zeroed moments and zero_grad-frees-grads follow
 * adam.c:27-111.  The update of adam.c:113-181 runs for every parameter
 * that has a grad in one multi-tensor kernel launch (k_adam, up to 32
 * tensors per launch); the bias corrections 1 - beta^t are computed here
 * with powf exactly as adam.c:121-125 does and passed to the kernel, which
 * evaluates the update in the order the reference's -ffast-math build does.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"
#include "picograd/adam.h"

#include <assert.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    pg_node *param;
    pg_tensor *m, *v, *vmax;
    float lr; /* > 0 overrides cfg.lr */
    float wd; /* >= 0 overrides cfg.weight_decay */
} adam_state;

struct pg_adam {
    pg_adam_cfg cfg;
    adam_state *st;
    size_t n, cap;
    unsigned long long step;
};

pg_adam_cfg pg_adam_cfg_default(void)
{
    pg_adam_cfg c = {.lr = 1e-3f, .beta1 = 0.9f, .beta2 = 0.999f, .eps = 1e-8f, .weight_decay = 0.0f,
                     .amsgrad = false, .decoupled_wd = true};
    return c;
}

pg_adam *pg_adam_new(const pg_adam_cfg *cfg)
{
    pg_adam_cfg def = pg_adam_cfg_default();
    if (!cfg)
        cfg = &def;
    /* adam.c:40-44 */
    assert(cfg->lr >= 0.0f);
    assert(cfg->beta1 >= 0.0f && cfg->beta1 < 1.0f);
    assert(cfg->beta2 >= 0.0f && cfg->beta2 < 1.0f);
    assert(cfg->eps > 0.0f);
    assert(cfg->weight_decay >= 0.0f);
    pg_adam *o = calloc(1, sizeof *o);
    if (!o)
        return NULL;
    o->cfg = *cfg;
    return o;
}

static void free_moments(adam_state *s)
{
    pg_tensor_free(s->m);
    pg_tensor_free(s->v);
    pg_tensor_free(s->vmax);
    s->m = s->v = s->vmax = NULL;
}

void pg_adam_free(pg_adam *opt)
{
    if (!opt)
        return;
    for (size_t i = 0; i < opt->n; i++) {
        pg_node_free(opt->st[i].param);
        free_moments(&opt->st[i]);
    }
    free(opt->st);
    free(opt);
}

int pg_adam_add_param(pg_adam *opt, pg_node *param)
{
    return pg_adam_add_param_lr(opt, param, 0.0f, -1.0f);
}

int pg_adam_add_param_lr(pg_adam *opt, pg_node *param, float lr, float wd)
{
    assert(opt && param && param->requires_grad);
    if (opt->n == opt->cap) {
        size_t nc = opt->cap ? opt->cap * 2 : 8;
        adam_state *p = realloc(opt->st, nc * sizeof *p);
        if (!p)
            return -1;
        opt->st = p;
        opt->cap = nc;
    }
    if (!pg_node_retain(param))
        return -1;
    adam_state *s = &opt->st[opt->n++];
    s->param = param;
    s->m = s->v = s->vmax = NULL;
    s->lr = lr;
    s->wd = wd;
    return 0;
}

size_t pg_adam_num_params(const pg_adam *opt) { return opt ? opt->n : 0; }

void pg_adam_set_lr(pg_adam *opt, float lr)
{
    if (opt)
        opt->cfg.lr = lr;
}

float pg_adam_get_lr(const pg_adam *opt) { return opt ? opt->cfg.lr : 0.0f; }

void pg_adam_set_param_lr(pg_adam *opt, size_t idx, float lr)
{
    assert(opt && idx < opt->n);
    opt->st[idx].lr = lr;
}

void pg_adam_set_param_wd(pg_adam *opt, size_t idx, float wd)
{
    assert(opt && idx < opt->n);
    opt->st[idx].wd = wd;
}

void pg_adam_zero_grad(pg_adam *opt)
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

void pg_adam_set_step(pg_adam *opt, unsigned long long s)
{
    if (opt)
        opt->step = s;
}

unsigned long long pg_adam_get_step(const pg_adam *opt) { return opt ? opt->step : 0; }

/* adam.c:121-125 */
static float bias_correction(float beta, unsigned long long step)
{
    float bc = 1.0f - powf(beta, (float)step);
    return bc < 1e-12f ? 1e-12f : bc;
}

void pg_adam_step(pg_adam *opt)
{
    assert(opt);
    if (!pgd_ok())
        return;
    const pg_adam_cfg c = opt->cfg;
    opt->step++;
    /* the reference's build divides by bc2 as a multiply by 1/bc2 */
    pgk_adam_hyper h = {.beta1 = c.beta1,
                        .beta2 = c.beta2,
                        .eps = c.eps,
                        .bc1 = bias_correction(c.beta1, opt->step),
                        .inv_bc2 = 1.0f / bias_correction(c.beta2, opt->step),
                        .amsgrad = c.amsgrad ? 1 : 0,
                        .decoupled = c.decoupled_wd ? 1 : 0};
    pgk_adam_seg *segs = calloc(opt->n ? opt->n : 1, sizeof *segs);
    if (!segs)
        return;
    int ns = 0;
    for (size_t i = 0; i < opt->n; i++) {
        adam_state *s = &opt->st[i];
        pg_node *p = s->param;
        pg_tensor *g = p->grad;
        if (!g)
            continue;
        assert(g->numel == p->value->numel);
        if (p->value->dtype != PG_DTYPE_F32 || g->dtype != PG_DTYPE_F32) {
            pga_set_err("pg_adam_step: parameter and grad storage must be f32");
            continue;
        }
        /* a pending zero is written; a pending clip scale is applied by
         * the update kernel as it reads the grad (it stays pending on the
         * grad's storage for any other reader) */
        if (g->pg_flags & PG_TENSOR_ZERO_PENDING)
            pgt_materialize(g);
        pgt_settle(p->value); /* the parameter's own elements, if any are pending */
        const pg_data_ref *gr = g->data_ref;
        if (!s->m) {
            /* adam.c:140-153: moments created at zero on first use */
            s->m = pg_tensor_zeros(p->value->ndim, p->value->shape);
            s->v = pg_tensor_zeros(p->value->ndim, p->value->shape);
            if (c.amsgrad)
                s->vmax = pg_tensor_zeros(p->value->ndim, p->value->shape);
            if (!s->m || !s->v || (c.amsgrad && !s->vmax)) {
                free_moments(s);
                pgd_set_err("pg_adam_step: cannot allocate the moments");
                continue;
            }
        }
        pgk_adam_seg *q = &segs[ns];
        q->p = p->value->dev;
        q->g = g->dev;
        q->gclip = gr && gr->clip_pending;
        q->gmul = q->gclip ? gr->clip_mul : 1.0f;
        q->ginv = q->gclip ? gr->clip_inv : 1.0f;
        q->m = s->m->dev;
        q->v = s->v->dev;
        q->vmax = c.amsgrad ? s->vmax->dev : NULL;
        /* adam.c:136-138 */
        q->lr = s->lr > 0.0f ? s->lr : c.lr;
        q->wd = s->wd >= 0.0f ? s->wd : c.weight_decay;
        /* a 16-bit copy of the parameter kept for the MFMA GEMMs is rewritten
         * from the updated values in the same pass */
        pg_data_ref *r = p->value->data_ref;
        bool shadow = r && r->shadow && p->value->dev == r->ptr && p->value->numel * 4 == r->nbytes;
        q->shadow = shadow ? r->shadow : NULL;
        q->shadow_dtype = shadow ? r->shadow_dtype : 0;
        q->shadow_cols = shadow ? r->shadow_cols : 0;
        q->shadow_ld = shadow ? r->shadow_ld : 0;
        if (shadow)
            r->shadow_stale = false;
        else
            pgt_touch(p->value);
        q->n = p->value->numel;
        ns++;
    }
    int tk = ns ? pgd_tbegin(PGD_T_ADAM) : -1;
    if (ns)
        pgd_check(pgk_adam_multi(segs, ns, &h, pgd_stream()), "pg_adam_step");
    pgd_tend(tk);
    free(segs);
}

/* ---------------- moment checkpoint ("PGAD") ---------------- */

bool pg_amd_adam_save_fp(const pg_adam *opt, FILE *fp)
{
    if (!opt || !fp)
        return false;
    const uint32_t ver = 1;
    const uint64_t step = (uint64_t)opt->step, n = (uint64_t)opt->n;
    if (fwrite("PGAD", 1, 4, fp) != 4 || fwrite(&ver, 4, 1, fp) != 1 || fwrite(&step, 8, 1, fp) != 1 ||
        fwrite(&n, 8, 1, fp) != 1)
        return false;
    for (size_t i = 0; i < opt->n; i++) {
        const adam_state *s = &opt->st[i];
        const uint32_t flags = (s->m ? 1u : 0u) | (s->m && s->vmax ? 2u : 0u);
        if (fwrite(&flags, 4, 1, fp) != 1)
            return false;
        if ((flags & 1u) && (!pg_tensor_save_fp(s->m, fp) || !pg_tensor_save_fp(s->v, fp)))
            return false;
        if ((flags & 2u) && !pg_tensor_save_fp(s->vmax, fp))
            return false;
    }
    return true;
}

bool pg_amd_adam_save(const pg_adam *opt, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "wb");
    if (!fp)
        return false;
    bool ok = pg_amd_adam_save_fp(opt, fp);
    return fclose(fp) == 0 && ok;
}

/* loads one moment record into *slot, creating it shaped like the
 * parameter when absent */
static bool load_moment(pg_tensor **slot, const pg_tensor *like, FILE *fp)
{
    if (!*slot) {
        *slot = pg_tensor_empty_dtype(PG_DTYPE_F32, like->ndim, like->shape);
        if (!*slot)
            return false;
    }
    return pgc_load_into(*slot, fp);
}

bool pg_amd_adam_load_into_fp(pg_adam *opt, FILE *fp)
{
    if (!opt || !fp)
        return false;
    char magic[4];
    uint32_t ver = 0;
    uint64_t step = 0, n = 0;
    if (fread(magic, 1, 4, fp) != 4 || memcmp(magic, "PGAD", 4) != 0)
        return false;
    if (fread(&ver, 4, 1, fp) != 1 || ver != 1)
        return false;
    if (fread(&step, 8, 1, fp) != 1 || fread(&n, 8, 1, fp) != 1 || n != (uint64_t)opt->n)
        return false;
    for (size_t i = 0; i < opt->n; i++) {
        uint32_t flags = 0;
        if (fread(&flags, 4, 1, fp) != 1 || flags > 3u || flags == 2u)
            return false;
        adam_state *s = &opt->st[i];
        const pg_tensor *like = s->param->value;
        if (!(flags & 1u)) {
            free_moments(s);
            continue;
        }
        if (!load_moment(&s->m, like, fp) || !load_moment(&s->v, like, fp))
            return false;
        if (flags & 2u) {
            if (!load_moment(&s->vmax, like, fp))
                return false;
        } else if (opt->cfg.amsgrad) {
            /* state saved without amsgrad: its running maximum starts at zero */
            pg_tensor_free(s->vmax);
            s->vmax = pg_tensor_zeros(like->ndim, like->shape);
            if (!s->vmax)
                return false;
        } else {
            pg_tensor_free(s->vmax);
            s->vmax = NULL;
        }
    }
    opt->step = (unsigned long long)step;
    return true;
}

bool pg_amd_adam_load_into(pg_adam *opt, const char *path)
{
    if (!path)
        return false;
    FILE *fp = fopen(path, "rb");
    if (!fp)
        return false;
    bool ok = pg_amd_adam_load_into_fp(opt, fp);
    fclose(fp);
    return ok;
}
