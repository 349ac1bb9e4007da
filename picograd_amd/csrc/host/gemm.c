/*
 * Matmul forward/backward and the pg_gemm* entry points on device.
 *
 * Shape rules follow the reference's pg_matmul (ops/matmul.c:186-284: same
 * dtype on both sides, 1-D operands as vectors, equal or one-sided batch
 * dims, f32 output) and bwd_matmul (autograd/autograd.c:561-706: dA += dC.B^T,
 * dB += A^T.dC per batch, grads in f32, an unbatched operand accumulating
 * over the batch).
 *
 * f16/bf16 matrices run on the MFMA kernel (pgk_gemm16), which reads each
 * operand where it lies, reduction dim contiguous or not:
 *   forward  C  = A . B      : A [M, K] K-contiguous, B [K, N] N-contiguous
 *   dgrad    dA = dC . B^T   : dC [M, N] and B [K, N], both N-contiguous
 *                              along the reduction
 *   wgrad    dB = A^T . dC   : A [M, K] and dC [M, N], reduction over M
 *                              with the output dims contiguous
 * The only copies are zero-padding of a dimension that is not a multiple of
 * 8 (16-byte loads) and the upstream grad rounded once to the operand dtype
 * (RNE), shared by dgrad and wgrad: the grads are f32-accumulated products
 * of 16-bit operands, the contract of the reference's hgemm/bgemm
 * (backend/cpu/gemm.c:575-629).  f32 operands and 1-D (vector) cases use
 * the f32 FMA kernel.
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include <stdlib.h>
#include <string.h>

static size_t up8(size_t x) { return (x + 7) & ~(size_t)7; }

typedef struct {
    bool av, bv;
    size_t am, ak, bn;
    size_t nbatch;
    bool abat, bbat;
} mm_shape;

static bool mm_shapes(const pg_tensor *a, const pg_tensor *b, mm_shape *s, size_t *rnd, size_t *rshape)
{
    size_t ra = a->ndim, rb = b->ndim;
    if (ra < 1 || rb < 1)
        return false;
    s->av = ra == 1;
    s->bv = rb == 1;
    s->am = s->av ? 1 : a->shape[ra - 2];
    s->ak = a->shape[ra - 1];
    s->bn = s->bv ? 1 : b->shape[rb - 1];
    size_t bk = s->bv ? b->shape[0] : b->shape[rb - 2];
    if (bk != s->ak)
        return false;
    size_t abn = s->av ? 0 : ra - 2, bbn = s->bv ? 0 : rb - 2;
    const size_t *bshape = NULL;
    size_t bnd = 0;
    if (abn && bbn) {
        if (abn != bbn || memcmp(a->shape, b->shape, abn * sizeof(size_t)))
            return false;
        bnd = abn;
        bshape = a->shape;
    } else if (abn) {
        bnd = abn;
        bshape = a->shape;
    } else if (bbn) {
        bnd = bbn;
        bshape = b->shape;
    }
    s->abat = abn > 0;
    s->bbat = bbn > 0;
    s->nbatch = 1;
    size_t n = 0;
    for (size_t d = 0; d < bnd; d++) {
        s->nbatch *= bshape[d];
        rshape[n++] = bshape[d];
    }
    if (!s->av)
        rshape[n++] = s->am;
    if (!s->bv)
        rshape[n++] = s->bn;
    if (n == 0)
        rshape[n++] = 1;
    *rnd = n;
    return true;
}

static void *tmp_alloc(size_t nbytes) { return pgd_malloc(nbytes ? nbytes : 1); }

/* Where a GEMM runs: the main stream with the whole chip, or one of two
 * concurrent launches (main or side stream) with a CU budget and its own
 * scratch slot */
typedef struct {
    pgk_stream st; /* NULL: the main stream */
    int slot;      /* scratch slot of its split-K partials / k-tail slabs */
    int cus;       /* CU budget, 0 = all */
    bool timed;    /* bracket it with the kernel timer */
} gemm_place;

static const gemm_place PLACE_MAIN = {NULL, 1, 0, true};

/* one MFMA GEMM (pgk_gemm16 semantics, optional epilogue); the split-K
 * partials and k-tail slabs come from the library scratch (stream-ordered,
 * so consecutive GEMMs on one stream may share a slot) */
static bool gemm16p(const gemm_place *pl, int dt, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a,
                    size_t lda, size_t sa, size_t aext, const uint16_t *b, size_t ldb, size_t sb, size_t bext,
                    float *c, size_t ldc, size_t sc, size_t batch, int beta, const pgk_epi *epi, const char *what)
{
    size_t wsz = pgk_gemm16_workspace_cu(ta, tb, m, n, k, batch, pl->cus);
    void *ws = NULL;
    if (wsz && !(ws = pgd_scratch(pl->slot, wsz))) {
        pgd_set_err("%s: workspace allocation failed", what);
        return false;
    }
    int tk = pl->timed ? pgd_tbegin(PGD_T_GEMM16) : -1;
    int rc = pgk_gemm16_cu(dt, ta, tb, m, n, k, a, lda, sa, aext, b, ldb, sb, bext, c, ldc, sc, batch, beta, epi, ws,
                           pl->cus, pl->st ? pl->st : pgd_stream());
    pgd_tend(tk);
    return pgd_check(rc, what);
}

static bool gemm16x(int dt, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, size_t sa,
                    size_t aext, const uint16_t *b, size_t ldb, size_t sb, size_t bext, float *c, size_t ldc,
                    size_t sc, size_t batch, int beta, const pgk_epi *epi, const char *what)
{
    return gemm16p(&PLACE_MAIN, dt, ta, tb, m, n, k, a, lda, sa, aext, b, ldb, sb, bext, c, ldc, sc, batch, beta, epi,
                   what);
}

static bool gemm16(int dt, int ta, int tb, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, size_t sa,
                   size_t aext, const uint16_t *b, size_t ldb, size_t sb, size_t bext, float *c, size_t ldc,
                   size_t sc, size_t batch, int beta, const char *what)
{
    return gemm16x(dt, ta, tb, m, n, k, a, lda, sa, aext, b, ldb, sb, bext, c, ldc, sc, batch, beta, NULL, what);
}

/* A matmul's dgrad and wgrad as ONE launch on the whole chip (the paired
 * kernel, both halves planned for all 256 CUs) when both plan 256 x 256
 * tiles without split-K: one launch boundary less, and the second problem's
 * first blocks start on the CUs the first leaves free while its last tiles
 * drain.  Measured 434 against 438 us for config 3's pair and 212 against
 * 215 us for a 4096^3 pair.  False (nothing launched) otherwise. */
static bool pair_full(int dt, const pgk_gemm_desc *dd, const pgk_gemm_desc *dw, const char *what)
{
    int sd = 0, sw = 0;
    if (!dd->m || !dd->n || !dd->k || !dd->batch || !dw->m || !dw->n || !dw->k || !dw->batch)
        return false;
    if (pgk_gemm16_plan(0, 0, dd->m, dd->n, dd->k, dd->batch, 0, &sd) != 2 || sd != 1 ||
        pgk_gemm16_plan(1, 1, dw->m, dw->n, dw->k, dw->batch, 0, &sw) != 2 || sw != 1 || dd->k % 8)
        return false;
    int tk = pgd_tbegin(PGD_T_GEMM16);
    int rc = pgk_gemm16_pair_dw(dt, dd, dw, 0, NULL, pgd_stream());
    pgd_tend(tk);
    if (rc == PGK_GEMM_NOT_PAIRED) /* excluded by the checks above */
        return false;
    return pgd_check(rc, what);
}

/* 16-bit copy of `rows x cols` (leading dim lds, `batch` matrices `sstride`
 * apart) padded with zeros to rows_pad x cols_pad; src_dtype 0 casts f32 */
static uint16_t *stage16(int dt, int src_dtype, const void *src, size_t rows, size_t cols, size_t lds,
                         size_t rows_pad, size_t cols_pad, size_t batch, size_t sstride, size_t *bytes)
{
    *bytes = batch * rows_pad * cols_pad * 2;
    uint16_t *p = tmp_alloc(*bytes);
    if (!p)
        return NULL;
    if (src_dtype == 0 && rows == rows_pad && cols == cols_pad && lds == cols &&
        (batch == 1 || sstride == rows * cols)) {
        /* no padding: a flat cast (16-byte loads and stores) */
        if (!pgd_check(pgk_cast_to16(dt, src, p, batch * rows * cols, pgd_stream()), "stage operand")) {
            pgd_free(p, *bytes);
            return NULL;
        }
        return p;
    }
    if (!pgd_check(pgk_copy_to16(dt, src_dtype, src, rows, cols, lds, p, cols_pad, rows_pad, batch, sstride,
                                 rows_pad * cols_pad, pgd_stream()),
                   "stage operand")) {
        pgd_free(p, *bytes);
        return NULL;
    }
    return p;
}

pg_tensor *pgm_matmul_forward(const pg_tensor *a, const pg_tensor *b)
{
    if (!a || !b || !a->dev || !b->dev) {
        pga_set_err("matmul: null operand");
        return NULL;
    }
    if (a->dtype != b->dtype) {
        pga_set_err("matmul: operands must share a dtype");
        return NULL;
    }
    if (!pgt_is_contiguous(a) || !pgt_is_contiguous(b)) {
        pga_set_err("matmul: operands must be contiguous");
        return NULL;
    }
    mm_shape s;
    size_t rnd, rshape[PG_MAX_NDIM];
    if (!mm_shapes(a, b, &s, &rnd, rshape)) {
        pga_set_err("matmul: shape mismatch");
        return NULL;
    }
    pgt_materialize((pg_tensor *)a);
    pgt_materialize((pg_tensor *)b);
    pg_tensor *c = pgt_alloc(PG_DTYPE_F32, rnd, rshape);
    if (!c)
        return NULL;
    size_t M = s.am, N = s.bn, K = s.ak;
    size_t sa = s.abat ? M * K : 0, sb = s.bbat ? K * N : 0, sc = M * N;
    pgk_stream st = pgd_stream();
    if (a->dtype == PG_DTYPE_F32) {
        pgd_check(pgk_gemm_f32(0, 0, M, N, K, a->dev, K, sa, b->dev, N, sb, c->dev, N, sc, s.nbatch, 0, st),
                  "matmul f32");
        return c;
    }
    int dt = (int)a->dtype;
    /* K padded to 8 needs zero columns of A and zero rows of B; N padded
     * to 8 (B's contiguous dim) needs zero columns of B */
    size_t K8 = up8(K), N8 = up8(N) < 8 ? 8 : up8(N);
    size_t ab = s.abat ? s.nbatch : 1, bb = s.bbat ? s.nbatch : 1;
    const uint16_t *ap = a->dev, *bp = b->dev;
    uint16_t *apad = NULL, *bpad = NULL;
    size_t abytes = 0, bbytes = 0;
    bool ok = true;
    if (K8 != K) {
        apad = stage16(dt, dt, a->dev, M, K, K, M, K8, ab, M * K, &abytes);
        ok = apad != NULL;
        ap = apad;
    }
    if (ok && (K8 != K || N8 != N)) {
        bpad = stage16(dt, dt, b->dev, K, N, N, K8, N8, bb, K * N, &bbytes);
        ok = bpad != NULL;
        bp = bpad;
    }
    size_t ldb = (K8 != K || N8 != N) ? N8 : N;
    if (ok)
        ok = gemm16(dt, 0, 1, M, N, K8, ap, K8, s.abat ? M * K8 : 0, M, bp, ldb, s.bbat ? K8 * ldb : 0,
                    bpad ? N8 : N, c->dev, N, sc, s.nbatch, 0, "matmul mfma");
    if (apad)
        pgd_free(apad, abytes);
    if (bpad)
        pgd_free(bpad, bbytes);
    if (!ok) {
        pga_set_err("matmul: %s", pg_amd_last_error());
        pg_tensor_free(c);
        return NULL;
    }
    return c;
}

/* f32 copy of a 16-bit tensor (vector cases of the backward) */
static float *as_f32(const pg_tensor *t, bool *owned)
{
    *owned = false;
    if (t->dtype == PG_DTYPE_F32)
        return t->dev;
    float *p = tmp_alloc(t->numel * 4);
    if (!p)
        return NULL;
    pgk_cast_from16((int)t->dtype, t->dev, p, t->numel, pgd_stream());
    *owned = true;
    return p;
}

void pgm_matmul_backward(pg_node *n)
{
    pg_node *pa = n->parents[0], *pb = n->parents[1];
    const pg_tensor *a = pa->value, *b = pb->value, *g = n->grad;
    if (!pa->requires_grad && !pb->requires_grad)
        return;
    mm_shape s;
    size_t rnd, rshape[PG_MAX_NDIM];
    if (!mm_shapes(a, b, &s, &rnd, rshape))
        return;
    size_t M = s.am, N = s.bn, K = s.ak, B = s.nbatch;
    pgk_stream st = pgd_stream();
    int ba = 0, bbeta = 0;
    pg_tensor *ga = pa->requires_grad ? pga_grad_for_write(pa, &ba) : NULL;
    pg_tensor *gb = pb->requires_grad ? pga_grad_for_write(pb, &bbeta) : NULL;
    bool mfma = a->dtype != PG_DTYPE_F32 && !s.av && !s.bv;

    if (!mfma) {
        /* f32 kernel (f16/bf16 vectors are upcast, as autograd.c:569-590 does) */
        bool oa, ob;
        float *a32 = as_f32(a, &oa), *b32 = as_f32(b, &ob);
        if (!a32 || !b32)
            return;
        for (size_t z = 0; z < B; z++) {
            const float *gp = (const float *)g->dev + z * M * N;
            if (ga) {
                /* dA[i,p] = sum_j g[i,j] B[p,j] */
                int beta_z = (s.abat || z == 0) ? ba : 1;
                float *dst = (float *)ga->dev + (s.abat ? z * M * K : 0);
                const float *bp = b32 + (s.bbat ? z * K * N : 0);
                pgk_gemm_f32(0, 1, M, K, N, gp, N, 0, bp, N, 0, dst, K, 0, 1, beta_z, st);
            }
            if (gb) {
                int beta_z = (s.bbat || z == 0) ? bbeta : 1;
                float *dst = (float *)gb->dev + (s.bbat ? z * K * N : 0);
                const float *ap = a32 + (s.abat ? z * M * K : 0);
                pgk_gemm_f32(1, 0, K, N, M, ap, K, 0, gp, N, 0, dst, N, 0, 1, beta_z, st);
            }
        }
        if (oa)
            pgd_free(a32, a->numel * 4);
        if (ob)
            pgd_free(b32, b->numel * 4);
        return;
    }

    int dt = (int)a->dtype;
    /* dC rounded once to the operand dtype, [B*M, N8] (zero columns past N) */
    size_t N8 = up8(N) < 8 ? 8 : up8(N), K8 = up8(K) < 8 ? 8 : up8(K);
    size_t gbytes;
    uint16_t *g16 = stage16(dt, 0, g->dev, B * M, N, N, B * M, N8, 1, 0, &gbytes);
    if (!g16)
        return;
    /* dgrad operands: dA[M, K] (+)= dC[M, N] . W[K, N]^T, both contiguous
     * along the reduction (N); W padded to N8 zero columns when needed */
    const uint16_t *wp = b->dev;
    uint16_t *wpad = NULL;
    size_t wbytes = 0, wb = s.bbat ? B : 1;
    if (ga && N8 != N)
        wp = wpad = stage16(dt, dt, b->dev, K, N, N, K, N8, wb, K * N, &wbytes);
    /* wgrad operands: dW[K, N] (+)= A[M, K]^T . dC[M, N], reduction over M
     * with K and N contiguous; A padded to K8 zero columns when needed.
     * When only A is batched the batch folds into the reduction (M_eff =
     * B M) */
    bool fold = s.abat && !s.bbat;
    size_t Bw = fold ? 1 : B, Mw = fold ? B * M : M;
    size_t a_rows = s.abat ? B * M : M;
    const uint16_t *ap = a->dev;
    uint16_t *apad = NULL;
    size_t abytes = 0;
    if (gb && K8 != K)
        ap = apad = stage16(dt, dt, a->dev, a_rows, K, K, a_rows, K8, 1, 0, &abytes);
    size_t lda_w = K8 != K ? K8 : K, sa_w = (s.abat && !fold) ? M * K8 : 0;
    bool d_one = ga && wp && (s.abat || B == 1), w_one = gb && ap && (s.bbat || Bw == 1);
    /* x.x (one node on both sides) has ONE grad: dgrad writes it with the
     * beta taken first, wgrad then adds to it (beta 1), so the two run in
     * that order on the main stream -- never side by side in one launch or
     * on two streams, where wgrad's blocks would read what dgrad's write */
    const bool alias = ga && gb && (ga == gb || ga->data_ref == gb->data_ref);

    /* When each GEMM alone would leave CUs idle (the bmm grads of config 4:
     * 128 blocks each), run the two side by side, each planned for its share
     * of the chip: wgrad on the side stream, dgrad on the main one.  The
     * planner's time estimates pick the split; without a clear win the two
     * run one after the other on the whole chip. */
    gemm_place pd = PLACE_MAIN, pw = PLACE_MAIN;
    int tk = -1;
    if (d_one && w_one && !alias) {
        double td = pgk_gemm16_time(0, 0, M, K, N8, B, 0), tw = pgk_gemm16_time(1, 1, K, N, Mw, Bw, 0);
        double best = 0.85 * (td + tw);
        int best_cus = 0;
        for (int cd = 32; cd <= 224; cd += 32) {
            double a1 = pgk_gemm16_time(0, 0, M, K, N8, B, cd), a2 = pgk_gemm16_time(1, 1, K, N, Mw, Bw, 256 - cd);
            double t = a1 > a2 ? a1 : a2;
            if (t < best) {
                best = t;
                best_cus = cd;
            }
        }
        if (best_cus) {
            tk = pgd_tbegin(PGD_T_GEMM16); /* the pair is one interval */
            pd.timed = pw.timed = false;
            /* one launch holding both when it can (no second stream to
             * fork and join), else the two on two streams */
            pgk_gemm_desc dd = {M, K, N8, g16, N8, M * N8, M, wp, N8, s.bbat ? K * N8 : 0, K, ga->dev, K, M * K, B, ba};
            pgk_gemm_desc dw = {K, N, Mw, ap, lda_w, sa_w, lda_w, g16, N8, Mw * N8, N8, gb->dev, N,
                                s.bbat ? K * N : 0, Bw, bbeta};
            size_t offw = 0, wsz = pgk_gemm16_pair_dw_workspace(&dd, &dw, best_cus, &offw);
            void *ws = wsz ? pgd_scratch(1, wsz) : NULL;
            int rc = wsz && !ws ? PGK_GEMM_NOT_PAIRED : pgk_gemm16_pair_dw(dt, &dd, &dw, best_cus, ws, pgd_stream());
            if (rc != PGK_GEMM_NOT_PAIRED) {
                pgd_check(rc, "dgrad + wgrad");
                pgd_tend(tk);
                if (wpad)
                    pgd_free(wpad, wbytes);
                if (apad)
                    pgd_free(apad, abytes);
                pgd_free(g16, gbytes);
                return;
            }
            /* the side stream's scratch (slot 5) is sized before the fork:
             * growing it afterwards would reuse a freed block in main-stream
             * order, which the side stream does not follow */
            size_t w5 = pgk_gemm16_workspace_cu(1, 1, K, N, Mw, Bw, 256 - best_cus);
            pgk_stream side = !w5 || pgd_scratch(5, w5) ? pgd_fork() : NULL;
            if (side) {
                pd.cus = best_cus;
                pw = (gemm_place){side, 5, 256 - best_cus, false};
            }
        } else {
            pgk_gemm_desc dd = {M, K, N8, g16, N8, M * N8, M, wp, N8, s.bbat ? K * N8 : 0, K, ga->dev, K, M * K, B, ba};
            pgk_gemm_desc dw = {K, N, Mw, ap, lda_w, sa_w, lda_w, g16, N8, Mw * N8, N8, gb->dev, N,
                                s.bbat ? K * N : 0, Bw, bbeta};
            if (pair_full(dt, &dd, &dw, "dgrad + wgrad")) {
                if (wpad)
                    pgd_free(wpad, wbytes);
                if (apad)
                    pgd_free(apad, abytes);
                pgd_free(g16, gbytes);
                return;
            }
        }
    }
    /* dgrad first: with one grad for both (x.x) it holds the first beta */
    if (ga && wp) {
        if (d_one) {
            gemm16p(&pd, dt, 0, 0, M, K, N8, g16, N8, M * N8, M, wp, N8, s.bbat ? K * N8 : 0, K, ga->dev, K, M * K, B,
                    ba, NULL, "dgrad");
        } else {
            /* unbatched A, batched B: dA accumulates over the batch */
            for (size_t z = 0; z < B; z++)
                gemm16(dt, 0, 0, M, K, N8, g16 + z * M * N8, N8, 0, M, wp + z * K * N8, N8, 0, K, ga->dev, K, 0, 1,
                       z == 0 ? ba : 1, "dgrad");
        }
    }
    if (gb && ap) {
        if (w_one) {
            gemm16p(&pw, dt, 1, 1, K, N, Mw, ap, lda_w, sa_w, lda_w, g16, N8, Mw * N8, N8, gb->dev, N,
                    s.bbat ? K * N : 0, Bw, bbeta, NULL, "wgrad");
        } else {
            for (size_t z = 0; z < Bw; z++)
                gemm16(dt, 1, 1, K, N, Mw, ap + z * sa_w, lda_w, 0, lda_w, g16 + z * Mw * N8, N8, 0, N8, gb->dev, N,
                       0, 1, z == 0 ? bbeta : 1, "wgrad");
        }
    }
    if (pw.st)
        pgd_join();
    pgd_tend(tk);
    if (wpad)
        pgd_free(wpad, wbytes);
    if (apad)
        pgd_free(apad, abytes);
    pgd_free(g16, gbytes);
}

/* ---------------------------------------------------------------- pg_gemm* */

void pg_gemm(size_t m, size_t n, size_t k, const float *a, size_t lda, const float *b, size_t ldb, float *c,
             size_t ldc)
{
    if (!pgd_ok())
        return;
    pgd_check(pgk_gemm_f32(0, 0, m, n, k, a, lda, 0, b, ldb, 0, c, ldc, 0, 1, 0, pgd_stream()), "pg_gemm");
}

void pg_gemm_ex(pg_dtype dtype, size_t m, size_t n, size_t k, const void *a, size_t lda, const void *b, size_t ldb,
                float *c, size_t ldc)
{
    if (!pgd_ok())
        return;
    if (dtype == PG_DTYPE_F32) {
        pg_gemm(m, n, k, a, lda, b, ldb, c, ldc);
        return;
    }
    if (!m || !n)
        return;
    int dt = (int)dtype;
    /* A [m, k] (lda) K-contiguous, B [k, n] (ldb) n-contiguous: read in
     * place when the leading dims and bases allow 16-byte loads and n is a
     * multiple of 8; otherwise through zero-padded copies */
    bool direct = !(lda & 7) && !(ldb & 7) && !(((uintptr_t)a | (uintptr_t)b) & 15) && !(n & 7);
    if (direct) {
        gemm16(dt, 0, 1, m, n, k, a, lda, 0, m, b, ldb, 0, n, c, ldc, 0, 1, 0, "pg_gemm_ex");
        return;
    }
    size_t K8 = up8(k), N8 = up8(n) < 8 ? 8 : up8(n), ab, bbytes;
    uint16_t *ap = stage16(dt, dt, a, m, k, lda, m, K8, 1, 0, &ab);
    uint16_t *bp = ap ? stage16(dt, dt, b, k, n, ldb, K8, N8, 1, 0, &bbytes) : NULL;
    if (ap && bp)
        gemm16(dt, 0, 1, m, n, K8, ap, K8, 0, m, bp, N8, 0, N8, c, ldc, 0, 1, 0, "pg_gemm_ex");
    if (ap)
        pgd_free(ap, ab);
    if (bp)
        pgd_free(bp, bbytes);
}

int pg_amd_gemm16_plan(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget, int *splits,
                       double *seconds)
{
    if (seconds)
        *seconds = pgk_gemm16_time(ta, tb, m, n, k, batch, cu_budget);
    return pgk_gemm16_plan(ta, tb, m, n, k, batch, cu_budget, splits);
}

/* pg_gemm_ex with every buffer it needs (the zero-padded operand copies,
 * split-K partials, k-tail slabs) carved from the fixed no-alloc workspace
 * instead of the library allocator.  The operands take the same path as in
 * pg_gemm_ex (read in place when the leading dims and bases allow 16-byte
 * loads and n is a multiple of 8, else both padded to [m, K8] and [K8, N8]),
 * so the kernels, the launch plan and the result bits are the same. */
static size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

int pg_amd_gemm_ex_noalloc(pg_dtype dtype, size_t m, size_t n, size_t k, const void *a, size_t lda, const void *b,
                           size_t ldb, float *c, size_t ldc)
{
    if (!pgd_initialised()) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: call pg_amd_init first (initialising may allocate)");
        return -1;
    }
    if (dtype != PG_DTYPE_F32 && dtype != PG_DTYPE_F16 && dtype != PG_DTYPE_BF16) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: dtype %d is not f32, f16 or bf16", (int)dtype);
        return -1;
    }
    if (!m || !n)
        return 0;
    if ((k && (!a || !b)) || !c || lda < k || ldb < n || ldc < n) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: null operand or a leading dim below its row length");
        return -1;
    }
    /* queueing pending uploads or deferred ops may compile, allocate or wait
     * on a staging slot: refused here rather than done behind the caller */
    if (pgd_work_pending()) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: uploads or deferred ops are pending; call pg_amd_sync() first");
        return -1;
    }
    pgk_stream st = pgd_stream();
    if (dtype == PG_DTYPE_F32)
        return pgd_check(pgk_gemm_f32(0, 0, m, n, k, a, lda, 0, b, ldb, 0, c, ldc, 0, 1, 0, st),
                         "pg_amd_gemm_ex_noalloc")
                   ? 0
                   : -1;
    unsigned char *ws = pgk_noalloc_scratch();
    const size_t cap = pgk_noalloc_scratch_bytes();
    if (!ws) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: no workspace on the current device");
        return -1;
    }
    int dt = (int)dtype;
    bool direct = !(lda & 7) && !(ldb & 7) && !(((uintptr_t)a | (uintptr_t)b) & 15) && !(n & 7);
    size_t K8 = direct ? k : up8(k), N8 = up8(n) < 8 ? 8 : up8(n);
    size_t abytes = direct ? 0 : up256(m * K8 * 2), bbytes = direct ? 0 : up256(K8 * N8 * 2);
    size_t wsz = pgk_gemm16_workspace(0, 1, m, n, K8, 1);
    size_t need = abytes + bbytes + wsz;
    if (need > cap) {
        pgd_set_err("pg_amd_gemm_ex_noalloc: %zux%zux%zu needs %zu bytes of workspace, above the no-alloc "
                    "maximum of %zu",
                    m, n, k, need, cap);
        return -1;
    }
    const uint16_t *ap = a, *bp = b;
    size_t lda2 = lda, ldb2 = ldb, bext = n;
    if (!direct) {
        uint16_t *pa = (uint16_t *)ws, *pb = (uint16_t *)(ws + abytes);
        if (!pgd_check(pgk_copy_to16(dt, dt, a, m, k, lda, pa, K8, m, 1, 0, 0, st), "pg_amd_gemm_ex_noalloc") ||
            !pgd_check(pgk_copy_to16(dt, dt, b, k, n, ldb, pb, N8, K8, 1, 0, 0, st), "pg_amd_gemm_ex_noalloc"))
            return -1;
        ap = pa;
        bp = pb;
        lda2 = K8;
        ldb2 = bext = N8;
    }
    int rc = pgk_gemm16(dt, 0, 1, m, n, K8, ap, lda2, 0, m, bp, ldb2, 0, bext, c, ldc, 0, 1, 0, NULL,
                        wsz ? ws + abytes + bbytes : NULL, st);
    return pgd_check(rc, "pg_amd_gemm_ex_noalloc") ? 0 : -1;
}

void pg_hgemm(size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, const uint16_t *b, size_t ldb, float *c,
              size_t ldc)
{
    pg_gemm_ex(PG_DTYPE_F16, m, n, k, a, lda, b, ldb, c, ldc);
}

void pg_bgemm(size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, const uint16_t *b, size_t ldb, float *c,
              size_t ldc)
{
    pg_gemm_ex(PG_DTYPE_BF16, m, n, k, a, lda, b, ldb, c, ldc);
}

/* ---------------------------------------------------------------- matmul16
 *
 * Mixed-precision matmul of f32 operands on the MFMA kernel: C = q(A).q(B)
 * with q = RNE rounding to f16/bf16 and f32 accumulation; backward
 * dA (+)= q(dC).q(B)^T and dB (+)= q(A)^T.q(dC) into f32 grads.  The
 * reference has no cast op and its matmul needs one dtype on both sides
 * (ops/matmul.c:191), so a bf16-weight network over f32 activations has no
 * reference spelling; this is the linear layer such a network needs.
 *
 * q(X) is the 16-bit shadow kept with X's storage (pgt_shadow16): made once
 * per tensor, shared by forward, dgrad and wgrad, and rewritten by
 * pg_sgd_step in the pass that updates a parameter -- the bf16 weight
 * storage of the layer.  Only a dimension that is not a multiple of 8 (the
 * 16-byte loads) takes a zero-padded copy per call instead.
 */

typedef struct {
    int dt;
} mm16_ctx;

static bool mm16_dims(const pg_tensor *a, const pg_tensor *b, size_t *M, size_t *K, size_t *N)
{
    if (a->ndim != 2 || b->ndim != 2 || a->shape[1] != b->shape[0])
        return false;
    *M = a->shape[0];
    *K = a->shape[1];
    *N = b->shape[1];
    return true;
}

/* q(t) as a [rows_pad, cols_pad] matrix whose first rows x cols hold the
 * rounded elements: the shadow when no padding is needed, the pitched
 * shadow when only the rows are padded (cols_pad: whole 16-byte pieces)
 * and t is its whole storage -- kept, and rewritten by the optimisers like
 * the plain one -- else a padded copy returned in *owned (*bytes long) */
static const uint16_t *operand16(pg_tensor *t, int dt, size_t rows, size_t cols, size_t rows_pad, size_t cols_pad,
                                 uint16_t **owned, size_t *bytes)
{
    *owned = NULL;
    *bytes = 0;
    if (rows == rows_pad && cols == cols_pad)
        return pgt_shadow16(t, (pg_dtype)dt);
    const pg_data_ref *r = t->data_ref;
    if (rows == rows_pad && r && t->dev == r->ptr && t->numel == rows * cols && t->numel * 4 == r->nbytes &&
        pgt_is_contiguous(t))
        return pgt_shadow16_rows(t, (pg_dtype)dt, cols, cols_pad);
    pgt_materialize(t); /* the copy reads the f32 elements */
    *owned = stage16(dt, 0, t->dev, rows, cols, cols, rows_pad, cols_pad, 1, 0, bytes);
    return *owned;
}

static void mm16_backward(pg_node *n)
{
    pg_node *pa = n->parents[0], *pb = n->parents[1];
    pg_tensor *a = pa->value, *b = pb->value;
    const pg_tensor *g = n->grad;
    const int dt = ((const mm16_ctx *)n->ctx)->dt;
    size_t M, K, N;
    if ((!pa->requires_grad && !pb->requires_grad) || !mm16_dims(a, b, &M, &K, &N) || !M || !N || !K)
        return;
    size_t K8 = up8(K), N8 = up8(N);
    size_t gbytes = 0;
    /* the grad's 16-bit copy when the fused backward region wrote it beside
     * the grad (kept with the grad's storage), else a staged copy */
    const uint16_t *gk = N == N8 ? pgt_shadow16_fresh(g, (pg_dtype)dt) : NULL;
    uint16_t *g16 = gk ? (uint16_t *)gk : stage16(dt, 0, g->dev, M, N, N, M, N8, 1, 0, &gbytes);
    if (!g16)
        return;
    /* each grad taken for writing once, then both GEMMs as one whole-chip
     * launch when they pair (as linear16's backward does), else one after
     * the other; a and b in one storage (a.a) share one grad and one kept
     * copy, so then each operand is taken right before its GEMM and dgrad
     * runs first (it holds the grad's first beta) */
    int ba = 0, bb = 0;
    pg_tensor *ga = pa->requires_grad ? pga_grad_for_write(pa, &ba) : NULL;
    pg_tensor *gb = pb->requires_grad ? pga_grad_for_write(pb, &bb) : NULL;
    const bool alias = a->data_ref == b->data_ref || (ga && gb && (ga == gb || ga->data_ref == gb->data_ref));
    uint16_t *ownb = NULL, *owna = NULL;
    size_t obb = 0, oba = 0;
    const uint16_t *qb = ga ? operand16(b, dt, K, N, K, N8, &ownb, &obb) : NULL;
    const uint16_t *qa = gb && !alias ? operand16(a, dt, M, K, M, K8, &owna, &oba) : NULL;
    const pgk_gemm_desc dd = {M, K, N8, g16, N8, 0, M, qb, N8, 0, K, ga ? ga->dev : NULL, K, 0, 1, ba};
    const pgk_gemm_desc dw = {K, N, M, qa, K8, 0, K8, g16, N8, 0, N8, gb ? gb->dev : NULL, N, 0, 1, bb};
    if (!(qb && qa && pair_full(dt, &dd, &dw, "matmul16 dgrad + wgrad"))) {
        if (qb)
            gemm16(dt, 0, 0, M, K, N8, g16, N8, 0, M, qb, N8, 0, K, ga->dev, K, 0, 1, ba, "matmul16 dgrad");
        if (gb && alias)
            qa = operand16(a, dt, M, K, M, K8, &owna, &oba);
        if (qa)
            gemm16(dt, 1, 1, K, N, M, qa, K8, 0, K8, g16, N8, 0, N8, gb->dev, N, 0, 1, bb, "matmul16 wgrad");
    }
    if (ownb)
        pgd_free(ownb, obb);
    if (owna)
        pgd_free(owna, oba);
    if (!gk)
        pgd_free(g16, gbytes);
}

int pgm_mm16_grad16(const pg_node *n)
{
    if (!n || n->backward != mm16_backward || !n->ctx || !n->value || n->value->ndim != 2 || n->value->shape[1] % 8)
        return 0;
    return ((const mm16_ctx *)n->ctx)->dt;
}

pg_node *pg_amd_ag_matmul16(pg_node *a, pg_node *b, pg_dtype dtype)
{
    if (!a || !b || !a->value || !b->value) {
        pga_set_err("matmul16: null operand");
        return NULL;
    }
    pg_tensor *av = a->value, *bv = b->value;
    size_t M, K, N;
    if (dtype != PG_DTYPE_F16 && dtype != PG_DTYPE_BF16) {
        pga_set_err("matmul16: dtype must be PG_DTYPE_F16 or PG_DTYPE_BF16");
        return NULL;
    }
    if (av->dtype != PG_DTYPE_F32 || bv->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(av) ||
        !pgt_is_contiguous(bv)) {
        pga_set_err("matmul16: operands must be contiguous f32");
        return NULL;
    }
    if (!mm16_dims(av, bv, &M, &K, &N)) {
        pga_set_err("matmul16: needs A [M, K] and B [K, N]");
        return NULL;
    }
    if (!pgd_ok()) {
        pga_set_err("matmul16: no device");
        return NULL;
    }
    /* the operands' f32 elements are read only to make a 16-bit copy
     * (operand16 settles them then); a current copy is used as it is */
    if (av->pg_flags & PG_TENSOR_ZERO_PENDING)
        pgt_materialize(av);
    if (bv->pg_flags & PG_TENSOR_ZERO_PENDING)
        pgt_materialize(bv);
    pg_tensor *c = pgt_alloc(PG_DTYPE_F32, 2, (size_t[]){M, N});
    if (!c)
        return NULL;
    const int dt = (int)dtype;
    bool ok = true;
    if (!K) {
        ok = pgd_check(pgk_fill_f32(c->dev, M * N, 0.0f, pgd_stream()), "matmul16");
    } else if (M && N) {
        /* K padded to 8 needs zero columns of q(A) and zero rows of q(B);
         * N padded to 8 (B's contiguous dim) zero columns of q(B) */
        size_t K8 = up8(K), N8 = up8(N);
        uint16_t *oa = NULL, *ob = NULL;
        size_t oab = 0, obb = 0;
        const uint16_t *qa = operand16(av, dt, M, K, M, K8, &oa, &oab);
        const uint16_t *qb = qa ? operand16(bv, dt, K, N, K8, N8, &ob, &obb) : NULL;
        ok = qa && qb && gemm16(dt, 0, 1, M, N, K8, qa, K8, 0, M, qb, N8, 0, N8, c->dev, N, 0, 1, 0, "matmul16");
        if (oa)
            pgd_free(oa, oab);
        if (ob)
            pgd_free(ob, obb);
    }
    if (!ok) {
        pga_set_err("matmul16: %s", pg_amd_last_error());
        pg_tensor_free(c);
        return NULL;
    }
    mm16_ctx *cx = malloc(sizeof *cx);
    if (!cx) {
        pg_tensor_free(c);
        return NULL;
    }
    cx->dt = dt;
    return pga_attach(c, 2, (pg_node *[]){a, b}, mm16_backward, cx, PG_AG_OP_MATMUL);
}

/* ---------------------------------------------------------------- linear16
 *
 * out = act(q(x).q(W) + b) as one MFMA GEMM whose epilogue adds the bias,
 * applies the activation and writes out, the pre-activation z (kept for the
 * backward) and out's 16-bit copy (the next layer's GEMM operand): the
 * forward of the reference's pg_cpu_gemm_fused (backend/cpu/gemm.c:685-726,
 * bias + act after f32 accumulation; nn.c:46-90 builds its linear layers on
 * it) with autograd.  Backward: one pass forms dz = dout * act'(z), writes it
 * RNE-16-bit for the GEMMs and sums its columns into db; then
 * dx += q(dz).q(W)^T and dW += q(x)^T.q(dz).
 */

typedef struct {
    int dt, act;
    pg_tensor *z;  /* pre-activation, NULL for act NONE or when no grad is needed */
    pg_tensor *dz; /* the last backward's 16-bit dz, kept when g_keep_dz is set */
} lin16_ctx;

/* pg_amd_linear16_keep_dz: keep each backward's dz on its node (tests) */
static bool g_keep_dz;
/* pg_amd_linear16_narrow: narrow dgrads on the VALU, fused into the
 * producing linear16 node's activation pass when they can be */
static bool g_narrow = true;

/* The bias grad of the last activation pass whose row-block partials are
 * not yet added: the next activation pass adds them in a row of extra
 * blocks of its own launch (one launch less per layer), or
 * pgm_colsum_flush does, at the end of the backward walk and before that
 * grad is taken for writing again.  The partials sit in scratch slot
 * g_fin_slot; the next pass writes its own into the other slot.  The
 * additions are k_colsum_fin's either way (the same bits). */
#define PGM_FIN_SLOT_A 3
#define PGM_FIN_SLOT_B 6
static pgk_colsum_job g_fin;
static int g_fin_slot = PGM_FIN_SLOT_A;

void pgm_colsum_flush(void)
{
    if (!g_fin.part)
        return;
    const pgk_colsum_job j = g_fin;
    g_fin = (pgk_colsum_job){0};
    pgd_check(pgk_colsum_run(&j, pgd_stream()), "linear16 bias grad sums");
}

void pgm_colsum_flush_for(const pg_tensor *t)
{
    const pg_data_ref *r = t ? t->data_ref : NULL;
    if (!g_fin.part || !r || !r->ptr)
        return;
    const char *lo = r->ptr, *p = (const char *)g_fin.out;
    if (p + g_fin.n * sizeof(float) > lo && p < lo + r->nbytes)
        pgm_colsum_flush();
}

void pgm_linear16_free_ctx(void *ctx)
{
    lin16_ctx *cx = ctx;
    if (cx) {
        pg_tensor_free(cx->z);
        pg_tensor_free(cx->dz);
    }
    free(cx);
}

void pg_amd_linear16_keep_dz(bool keep) { g_keep_dz = keep; }
void pg_amd_linear16_narrow(bool on) { g_narrow = on; }

static const lin16_ctx *lin16_of(const pg_node *n)
{
    return n && n->backward == pgm_linear16_backward ? (const lin16_ctx *)n->ctx : NULL;
}

const pg_tensor *pg_amd_linear16_preact(const pg_node *n)
{
    const lin16_ctx *cx = lin16_of(n);
    return cx ? cx->z : NULL;
}

const pg_tensor *pg_amd_linear16_dz(const pg_node *n)
{
    const lin16_ctx *cx = lin16_of(n);
    return cx ? cx->dz : NULL;
}

/* The narrow dgrad of a layer with at most 16 outputs (dz16 [M, ld] and
 * qw [K, ld], ld = 8 or 16), written into a grad taken fresh (beta 0): when
 * x comes from a linear16 node and gx is the whole of its storage, left
 * pending on gx (pgt_narrow_release / pgt_settle) for that node's backward,
 * which forms it in its activation pass; otherwise formed now.  Either way
 * with the GEMM's MFMA sequence (pgk_act_bwd16n), so the bits are the GEMM's.
 * Takes *dz_owned / *w_owned (set to NULL) when it keeps them. */
static void narrow_dgrad(pg_node *px, pg_tensor *gx, pg_tensor *w, const uint16_t *dz16, void **dz_owned,
                         size_t dzb, pg_data_ref *dz_ref, const uint16_t *qw, uint16_t **w_owned, size_t wb,
                         size_t M, size_t K, size_t N, size_t ld, int dt)
{
    pg_data_ref *r = gx->data_ref;
    pg_narrow_pending *p = NULL;
    if (lin16_of(px) && r && !r->narrow && !r->act_pending && !r->clip_pending && gx->dev == r->ptr &&
        gx->numel * 4 == r->nbytes && pgt_is_contiguous(gx))
        p = calloc(1, sizeof *p);
    if (!p) {
        pgd_check(pgk_act_bwd16n(0, dz16, qw, (int)ld, dt, NULL, gx->dev, NULL, M, K, NULL, up8(K), 0, NULL, 0, NULL,
                                 NULL, NULL, pgd_stream()),
                  "linear16 narrow dgrad");
        return;
    }
    *p = (pg_narrow_pending){.dn = dz16, .wn = qw, .m = M, .n = K, .kw = (int)ld, .dtype = dt};
    p->own[0] = *dz_owned;
    p->own_bytes[0] = *dz_owned ? dzb : 0;
    p->hold[0] = *dz_owned ? NULL : dz_ref;
    p->own[1] = *w_owned;
    p->own_bytes[1] = *w_owned ? wb : 0;
    p->hold[1] = *w_owned ? NULL : w->data_ref;
    for (int i = 0; i < 2; i++)
        if (p->hold[i])
            p->hold[i]->refs++;
    *dz_owned = NULL;
    *w_owned = NULL;
    r->narrow = p;
}

void pgm_linear16_backward(pg_node *n)
{
    pg_node *px = n->parents[0], *pw = n->parents[1], *pb = n->nparents > 2 ? n->parents[2] : NULL;
    pg_tensor *x = px->value, *w = pw->value;
    lin16_ctx *cx = n->ctx;
    const int dt = cx->dt;
    size_t M, K, N;
    if (!mm16_dims(x, w, &M, &K, &N) || !M || !N)
        return;
    const size_t K8 = up8(K), N8 = up8(N);
    const size_t dzb = M * N8 * 2;
    /* dz lives in a tensor kept on the node when asked, else in a
     * temporary freed (stream-ordered) after the GEMMs */
    pg_tensor *keep = NULL;
    if (g_keep_dz) {
        pg_tensor_free(cx->dz);
        cx->dz = keep = pgt_alloc((pg_dtype)dt, 2, (size_t[]){M, N8});
    }
    uint16_t *dz16 = keep ? keep->dev : tmp_alloc(dzb);
    if (!dz16)
        return;
    float *db = NULL;
    int dbeta = 0;
    if (pb && pb->requires_grad) {
        pg_tensor *gb = pga_grad_for_write(pb, &dbeta);
        db = gb ? gb->dev : NULL;
    }
    /* the pass adds the previous pass's deferred bias-grad sums in its own
     * launch and defers its own, their partials in the other scratch slot */
    const pgk_colsum_job fold = g_fin;
    const int slot = fold.part && g_fin_slot == PGM_FIN_SLOT_A ? PGM_FIN_SLOT_B : PGM_FIN_SLOT_A;
    pgk_colsum_job next = {0};
    size_t wsz = db ? pgk_act_bwd16_workspace(M, N) : 0;
    void *ws = wsz ? pgd_scratch(slot, wsz) : NULL;
    int tk = pgd_tbegin(PGD_T_STAGE);
    /* the grad left pending as the next layer's narrow dgrad is formed in
     * the activation pass, each element used for dz there; the grad itself
     * stays pending (written by its first reader, dropped by the next write
     * of the whole grad), its product now over a copy of the narrow weights
     * the pass makes (an optimiser step may rewrite the layer's own) */
    pg_data_ref *gr = n->grad->data_ref;
    pg_narrow_pending *np = gr ? gr->narrow : NULL;
    bool ok;
    if (np && np->m == M && np->n == N && n->grad->dev == gr->ptr) {
        const size_t wsb = N * (size_t)np->kw * 2;
        uint16_t *wsnap = pgd_malloc(wsb);
        ok = (!wsz || ws) &&
             pgd_check(pgk_act_bwd16n(cx->act, np->dn, np->wn, np->kw, np->dtype, wsnap, wsnap ? NULL : n->grad->dev,
                                      cx->z ? cx->z->dev : NULL, M, N, dz16, N8, dt, db, dbeta, ws,
                                      fold.part ? &fold : NULL, &next, pgd_stream()),
                       "linear16 act backward (narrow dgrad)");
        if (ok && wsnap) {
            if (np->own[1])
                pgd_free(np->own[1], np->own_bytes[1]);
            pgt_ref_release(np->hold[1]);
            np->hold[1] = NULL;
            np->own[1] = wsnap;
            np->own_bytes[1] = wsb;
            np->wn = wsnap;
        } else {
            if (wsnap)
                pgd_free(wsnap, wsb);
            if (ok) /* written in the pass */
                pgt_narrow_release(gr);
        }
    } else {
        pgt_settle(n->grad);
        ok = (!wsz || ws) &&
             pgd_check(pgk_act_bwd16(cx->act, n->grad->dev, cx->z ? cx->z->dev : NULL, M, N, dz16, N8, dt, db,
                                     dbeta, ws, fold.part ? &fold : NULL, &next, pgd_stream()),
                       "linear16 act backward");
    }
    if (ok) { /* the folded job ran in the pass */
        g_fin = next;
        g_fin_slot = slot;
    }
    pgd_tend(tk);
    /* each grad taken for writing once (that clears a pending zero and
     * fixes beta), then both GEMMs as one whole-chip launch when they pair,
     * else one after the other */
    int bx = 0, bw = 0;
    pg_tensor *gx = ok && K && px->requires_grad ? pga_grad_for_write(px, &bx) : NULL;
    pg_tensor *gw = ok && K && pw->requires_grad ? pga_grad_for_write(pw, &bw) : NULL;
    uint16_t *ow = NULL, *ox = NULL;
    size_t obw = 0, obx = 0;
    /* x and W in one storage (linear16(x, x) with x square) share one kept
     * 16-bit copy and, for one node, one grad: then each operand is taken
     * right before its GEMM (taking the second may remake the copy the
     * first GEMM reads, which stream order makes safe only once that GEMM
     * is queued) and the GEMMs run one after the other, dgrad first (it
     * holds the grad's first beta) */
    const bool alias = x->data_ref == w->data_ref || (gx && gw && (gx == gw || gx->data_ref == gw->data_ref));
    const uint16_t *qw = gx ? operand16(w, dt, K, N, K, N8, &ow, &obw) : NULL;
    const uint16_t *qx = gw && !alias ? operand16(x, dt, M, K, M, K8, &ox, &obx) : NULL;
    const pgk_gemm_desc dd = {M, K, N8, dz16, N8, 0, M, qw, N8, 0, K, gx ? gx->dev : NULL, K, 0, 1, bx};
    const pgk_gemm_desc dw = {K, N, M, qx, K8, 0, K8, dz16, N8, 0, N8, gw ? gw->dev : NULL, N, 0, 1, bw};
    void *dz_owned = keep ? NULL : dz16;
    if (qw && g_narrow && N <= 16 && !bx && !alias) {
        narrow_dgrad(px, gx, w, dz16, &dz_owned, dzb, keep ? keep->data_ref : NULL, qw, &ow, obw, M, K, N, N8, dt);
        qw = NULL; /* formed, or pending on gx */
    }
    if (!(qw && qx && pair_full(dt, &dd, &dw, "linear16 dgrad + wgrad"))) {
        if (qw)
            gemm16(dt, 0, 0, M, K, N8, dz16, N8, 0, M, qw, N8, 0, K, gx->dev, K, 0, 1, bx, "linear16 dgrad");
        if (gw && alias)
            qx = operand16(x, dt, M, K, M, K8, &ox, &obx);
        if (qx)
            gemm16(dt, 1, 1, K, N, M, qx, K8, 0, K8, dz16, N8, 0, N8, gw->dev, N, 0, 1, bw, "linear16 wgrad");
    }
    if (ow)
        pgd_free(ow, obw);
    if (ox)
        pgd_free(ox, obx);
    if (dz_owned)
        pgd_free(dz_owned, dzb);
}

pg_node *pg_amd_ag_linear16(pg_node *x, pg_node *w, pg_node *b, int act, pg_dtype dtype)
{
    if (!x || !w || !x->value || !w->value || (b && !b->value)) {
        pga_set_err("linear16: null operand");
        return NULL;
    }
    if (dtype != PG_DTYPE_F16 && dtype != PG_DTYPE_BF16) {
        pga_set_err("linear16: dtype must be PG_DTYPE_F16 or PG_DTYPE_BF16");
        return NULL;
    }
    if (act < PGK_ACT_NONE || act > PGK_ACT_GELU) {
        pga_set_err("linear16: act must be PG_ACT_NONE, PG_ACT_RELU or PG_ACT_GELU (0, 1, 2)");
        return NULL;
    }
    pg_tensor *xv = x->value, *wv = w->value, *bv = b ? b->value : NULL;
    size_t M, K, N;
    if (xv->dtype != PG_DTYPE_F32 || wv->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(xv) || !pgt_is_contiguous(wv) ||
        (bv && (bv->dtype != PG_DTYPE_F32 || !pgt_is_contiguous(bv)))) {
        pga_set_err("linear16: operands must be contiguous f32");
        return NULL;
    }
    if (!mm16_dims(xv, wv, &M, &K, &N) || (bv && bv->numel != N)) {
        pga_set_err("linear16: needs x [M, K], W [K, N] and b [N]");
        return NULL;
    }
    if (!pgd_ok()) {
        pga_set_err("linear16: no device");
        return NULL;
    }
    /* x's and W's f32 elements are read only to make a 16-bit copy
     * (operand16 settles them then): a previous linear16 output whose
     * elements are still pending is used through its 16-bit copy alone */
    if (xv->pg_flags & PG_TENSOR_ZERO_PENDING)
        pgt_materialize(xv);
    if (wv->pg_flags & PG_TENSOR_ZERO_PENDING)
        pgt_materialize(wv);
    if (bv)
        pgt_materialize(bv);
    const int dt = (int)dtype;
    const bool grad = pg_autograd_is_grad_enabled() &&
                      (x->requires_grad || w->requires_grad || (b && b->requires_grad));
    pg_tensor *out = pgt_alloc(PG_DTYPE_F32, 2, (size_t[]){M, N});
    pg_tensor *z = (grad && act != PGK_ACT_NONE) ? pgt_alloc(PG_DTYPE_F32, 2, (size_t[]){M, N}) : NULL;
    lin16_ctx *cx = malloc(sizeof *cx);
    bool ok = out && cx && (z || !grad || act == PGK_ACT_NONE);
    /* out's 16-bit copy, kept as its shadow (rows of N need N % 8 == 0 to be
     * a GEMM operand in place) */
    if (ok && N % 8 == 0 && M * N != 0) {
        pg_data_ref *r = out->data_ref;
        r->shadow = pgd_malloc(M * N * 2);
        r->shadow_bytes = M * N * 2;
        r->shadow_dtype = dt;
        r->shadow_stale = true;
        ok = r->shadow != NULL;
    }
    /* with the pre-activation kept (a grad-mode layer with an activation),
     * the GEMM writes z and out's 16-bit copy but not out itself: out's
     * elements stay pending as act(z) until something reads them (the
     * next layer reads the copy, the backward reads z), and are then
     * written by one pass with the epilogue's arithmetic */
    const bool lazy_out = z && act != PGK_ACT_NONE && K && M && N && out->data_ref->shadow;
    if (ok && M && N) {
        pgk_epi epi = {bv ? (const float *)bv->dev : NULL, act, z ? (float *)z->dev : NULL,
                       out->data_ref->shadow, dt, lazy_out ? 1 : 0};
        if (!K) {
            ok = gemm16x(dt, 0, 1, M, N, 0, NULL, 8, 0, M, NULL, 8, 0, up8(N), out->dev, N, 0, 1, 0, &epi,
                         "linear16");
        } else {
            size_t K8 = up8(K), N8 = up8(N);
            uint16_t *oa = NULL, *ob = NULL;
            size_t oab = 0, obb = 0;
            const uint16_t *qx = operand16(xv, dt, M, K, M, K8, &oa, &oab);
            const uint16_t *qw = qx ? operand16(wv, dt, K, N, K8, N8, &ob, &obb) : NULL;
            ok = qx && qw &&
                 gemm16x(dt, 0, 1, M, N, K8, qx, K8, 0, M, qw, N8, 0, N8, out->dev, N, 0, 1, 0, &epi, "linear16");
            if (oa)
                pgd_free(oa, oab);
            if (ob)
                pgd_free(ob, obb);
        }
        if (ok && out->data_ref->shadow)
            out->data_ref->shadow_stale = false;
        if (ok && lazy_out) {
            pg_data_ref *r = out->data_ref;
            r->act_pending = act;
            r->act_src = z->dev;
            r->act_src_ref = z->data_ref;
            z->data_ref->refs++;
        }
    }
    if (!ok) {
        pga_set_err("linear16: %s", pg_amd_last_error());
        pg_tensor_free(out);
        pg_tensor_free(z);
        free(cx);
        return NULL;
    }
    cx->dt = dt;
    cx->act = act;
    cx->z = z;
    cx->dz = NULL;
    pg_node *parents[3] = {x, w, b};
    pg_node *n = pga_attach(out, b ? 3 : 2, parents, pgm_linear16_backward, NULL, PG_AG_OP_MATMUL);
    if (n && n->backward) {
        n->ctx = cx;
    } else {
        pgm_linear16_free_ctx(cx);
    }
    return n;
}
