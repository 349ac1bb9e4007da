/*
 * Gradient clipping over device-resident grads (reference opt/clip.c).
 *
 * pg_grad_norm and pg_clip_grad_norm reduce the squares of every listed
 * grad in f64 (clip.c:5-18) with one multi-tensor launch and a one-block
 * finisher whose summation order is fixed.  pg_clip_grad_norm queues the
 * scaling pass right behind it: the finisher stores the scale and whether
 * to apply it (clip.c:32-33) in device memory, and the scaling kernel reads
 * them, so the only host wait is the final read of the norm that the API
 * returns.  Grads still pending as zero are skipped (they add nothing and
 * stay zero).  A grad listed twice counts twice in the norm and is scaled
 * twice, as in the reference; its second scaling is a separate launch so
 * no two blocks update one element.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"
#include "picograd/clip.h"

#include <stdlib.h>

/* Collects the grads to visit: NULL nodes, nodes without a grad and grads
 * pending as zero are left out.  round[i] counts the earlier entries with
 * the same storage.  Returns the count, or -1 on allocation failure. */
static int collect(pg_node **params, size_t n, pgk_grad_seg **out, int **round, int *rounds)
{
    pgk_grad_seg *segs = malloc((n ? n : 1) * sizeof *segs);
    int *rd = malloc((n ? n : 1) * sizeof *rd);
    if (!segs || !rd) {
        free(segs);
        free(rd);
        pgd_set_err("gradient clipping: out of host memory");
        return -1;
    }
    int ns = 0, nr = 0;
    for (size_t i = 0; i < n; i++) {
        pg_node *p = params[i];
        if (!p || !p->grad)
            continue;
        pg_tensor *g = p->grad;
        if ((g->pg_flags & PG_TENSOR_ZERO_PENDING) || g->numel == 0)
            continue;
        pgt_settle(g); /* an earlier clip's scale, before the squares are read */
        int r = 0;
        for (int q = 0; q < ns; q++)
            r += segs[q].g == (float *)g->dev ? 1 : 0;
        segs[ns].g = g->dev;
        segs[ns].n = g->numel;
        rd[ns] = r;
        if (r + 1 > nr)
            nr = r + 1;
        ns++;
    }
    *out = segs;
    *round = rd;
    *rounds = nr;
    return ns;
}

/* Whether the scale can stay pending on the grads' storages instead of a
 * pass of its own: each listed grad is the whole of a storage no other
 * listed grad shares (a grad listed twice is scaled twice, clip.c:34-39,
 * which one pending factor cannot express). */
static bool lazy_ok(pg_node **params, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        const pg_tensor *g = params[i] && params[i]->grad ? params[i]->grad : NULL;
        if (!g || (g->pg_flags & PG_TENSOR_ZERO_PENDING) || g->numel == 0)
            continue;
        const pg_data_ref *r = g->data_ref;
        if (!r || g->dev != r->ptr || g->numel * 4 != r->nbytes || g->dtype != PG_DTYPE_F32)
            return false;
        for (size_t j = 0; j < i; j++) {
            const pg_tensor *h = params[j] && params[j]->grad ? params[j]->grad : NULL;
            if (h && h->data_ref == r && !(h->pg_flags & PG_TENSOR_ZERO_PENDING) && h->numel)
                return false;
        }
    }
    return true;
}

/* queues the norm (and with clip, the scaling); writes the norm to *norm
 * after one wait.  Returns false on a device error.  With clip, the scale
 * (max_norm and 1 / (norm + eps), as the finisher computed them) is left
 * pending on the grads' storages when lazy_ok: the next optimiser step
 * applies it as it reads the grads, and any other reader first writes it
 * (pgt_settle), so the grads read as scaled everywhere without a pass of
 * their own between the norm and the step. */
static bool norm_pass(pg_node **params, size_t n, int clip, float max_norm, float eps, float *norm)
{
    const bool lazy = clip && lazy_ok(params, n);
    pgk_grad_seg *segs;
    int *rd, rounds;
    int ns = collect(params, n, &segs, &rd, &rounds);
    if (ns < 0)
        return false;
    bool ok = true;
    if (ns == 0) {
        *norm = 0.0f;
        goto done;
    }
    size_t wsz = pgk_grad_norm_workspace(segs, ns);
    size_t res_off = (wsz + 255) & ~(size_t)255;
    char *ws = pgd_scratch(4, res_off + 256);
    if (!ws) {
        ok = false;
        goto done;
    }
    float *res = (float *)(ws + res_off);
    int tk = pgd_tbegin(PGD_T_CLIP);
    ok = pgd_check(pgk_grad_norm(segs, ns, clip, max_norm, eps, res, ws, pgd_stream()), "grad norm");
    if (ok && lazy) {
        float r4[4];
        pgd_tend(tk);
        ok = pgd_d2h(r4, res, sizeof r4);
        *norm = r4[0];
        if (ok && r4[2] != 0.0f) /* clip.c:32-33: scaled only above max_norm */
            for (size_t i = 0; i < n; i++) {
                pg_tensor *g = params[i] && params[i]->grad ? params[i]->grad : NULL;
                if (!g || (g->pg_flags & PG_TENSOR_ZERO_PENDING) || g->numel == 0)
                    continue;
                g->data_ref->clip_pending = true;
                g->data_ref->clip_mul = r4[3];
                g->data_ref->clip_inv = r4[1];
            }
        goto done;
    }
    if (ok && clip) {
        /* round r holds the r-th repeat of each grad: one launch per round */
        pgk_grad_seg *sub = malloc(ns * sizeof *sub);
        if (!sub) {
            pgd_set_err("gradient clipping: out of host memory");
            ok = false;
        }
        for (int r = 0; ok && r < rounds; r++) {
            int k = 0;
            for (int q = 0; q < ns; q++)
                if (rd[q] == r)
                    sub[k++] = segs[q];
            ok = pgd_check(pgk_grad_scale(sub, k, res, pgd_stream()), "grad scale");
        }
        free(sub);
    }
    pgd_tend(tk);
    if (ok)
        ok = pgd_d2h(norm, res, sizeof(float));
done:
    free(segs);
    free(rd);
    return ok;
}

float pg_grad_norm(pg_node **params, size_t n)
{
    /* clip.c:6 */
    if (!params || n == 0)
        return 0.0f;
    if (!pgd_ok())
        return -1.0f;
    float norm;
    return norm_pass(params, n, 0, 0.0f, 0.0f, &norm) ? norm : -1.0f;
}

float pg_clip_grad_norm(pg_node **params, size_t n, float max_norm, float eps)
{
    /* clip.c:28-29 */
    if (!params || max_norm <= 0.0f)
        return -1.0f;
    if (eps < 0.0f)
        eps = 1e-6f;
    if (n == 0)
        return 0.0f;
    if (!pgd_ok())
        return -1.0f;
    float norm;
    return norm_pass(params, n, 1, max_norm, eps, &norm) ? norm : -1.0f;
}

void pg_clip_grad_value(pg_node **params, size_t n, float clip_value)
{
    /* clip.c:50 */
    if (!params || clip_value <= 0.0f)
        return;
    if (!pgd_ok())
        return;
    pgk_grad_seg *segs;
    int *rd, rounds;
    int ns = collect(params, n, &segs, &rd, &rounds);
    if (ns < 0)
        return;
    pgk_grad_seg *sub = malloc((ns ? ns : 1) * sizeof *sub);
    int tk = ns ? pgd_tbegin(PGD_T_CLIP) : -1;
    for (int r = 0; sub && r < rounds; r++) {
        int k = 0;
        for (int q = 0; q < ns; q++)
            if (rd[q] == r)
                sub[k++] = segs[q];
        if (!pgd_check(pgk_clip_value(sub, k, clip_value, pgd_stream()), "pg_clip_grad_value"))
            break;
    }
    pgd_tend(tk);
    if (!sub)
        pgd_set_err("pg_clip_grad_value: out of host memory");
    free(sub);
    free(segs);
    free(rd);
}
