/*
 * Matmul forward/backward and the pg_gemm* entry points on device.
 *
 * Shape rules follow the reference's pg_matmul (ops/matmul.c:186-284: same
 * dtype on both sides, 1-D operands as vectors, equal or one-sided batch
 * dims, f32 output) and bwd_matmul (autograd/autograd.c:561-706: dA += dC.B^T,
 * dB += A^T.dC per batch, grads in f32, an unbatched operand accumulating
 * over the batch).
 *
 * f16/bf16 matrices run on the MFMA kernel, which wants both operands with
 * the reduction dim contiguous ("NT").  So:
 *   forward  C  = A . B      : B is staged transposed ([N, K])
 *   dgrad    dA = dC . B^T   : dC is cast to the operand dtype; B as is
 *   wgrad    dB = A^T . dC   : A and dC are staged transposed ([K, M], [N, M])
 * Staging also pads the reduction dim to a multiple of 8 with zeros.  The
 * upstream grad is rounded to the operand dtype (RNE) before the GEMMs:
 * the grads are f32-accumulated products of 16-bit operands, the contract
 * of the reference's hgemm/bgemm (backend/cpu/gemm.c:575-629).
 * f32 operands and 1-D (vector) cases use the f32 FMA kernel.
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

/* the MFMA GEMM, bracketed by the kernel timer */
static int gemm16(int dt, size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, size_t sa, const uint16_t *b,
                  size_t ldb, size_t sb, float *c, size_t ldc, size_t sc, size_t batch, int beta, pgk_stream st)
{
    int tk = pgd_tbegin(PGD_T_GEMM16);
    int rc = pgk_gemm16_nt(dt, m, n, k, a, lda, sa, b, ldb, sb, c, ldc, sc, batch, beta, st);
    pgd_tend(tk);
    return rc;
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
    size_t K8 = up8(K);
    size_t bb = s.bbat ? s.nbatch : 1;
    /* B^T staged: [N, K8] per batch */
    uint16_t *bt = tmp_alloc(bb * N * K8 * 2);
    const uint16_t *ap = a->dev;
    uint16_t *apad = NULL;
    bool ok = bt != NULL;
    if (ok)
        ok = pgd_check(pgk_transpose_to16(dt, dt, b->dev, K, N, N, bt, K8, bb, K * N, N * K8, st), "stage B^T");
    if (ok && K8 != K) {
        size_t ab = s.abat ? s.nbatch : 1;
        apad = tmp_alloc(ab * M * K8 * 2);
        ok = apad && pgd_check(pgk_copy_to16(dt, dt, a->dev, M, K, K, apad, K8, ab, M * K, M * K8, st), "stage A");
        ap = apad;
    }
    if (ok)
        ok = pgd_check(gemm16(dt, M, N, K8, ap, K8, s.abat ? M * K8 : 0, bt, K8, s.bbat ? N * K8 : 0,
                                     c->dev, N, sc, s.nbatch, 0, st),
                       "matmul mfma");
    pgd_free(bt, bb * N * K8 * 2);
    if (apad)
        pgd_free(apad, (s.abat ? s.nbatch : 1) * M * K8 * 2);
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
    size_t N8 = up8(N);
    /* dgrad operand: dC rounded to the operand dtype, [B*M, N8] */
    if (ga) {
        size_t gbytes = B * M * N8 * 2;
        uint16_t *g16 = tmp_alloc(gbytes);
        const uint16_t *bp = b->dev;
        uint16_t *bpad = NULL;
        size_t bbytes = (s.bbat ? B : 1) * K * N8 * 2;
        bool ok = g16 && pgd_check(pgk_copy_to16(dt, 0, g->dev, B * M, N, N, g16, N8, 1, 0, 0, st), "stage dC");
        if (ok && N8 != N) {
            bpad = tmp_alloc(bbytes);
            ok = bpad && pgd_check(pgk_copy_to16(dt, dt, b->dev, (s.bbat ? B : 1) * K, N, N, bpad, N8, 1, 0, 0, st),
                                   "stage B");
            bp = bpad;
        }
        if (ok) {
            if (s.abat || B == 1) {
                pgd_check(gemm16(dt, M, K, N8, g16, N8, M * N8, bp, N8, s.bbat ? K * N8 : 0, ga->dev, K,
                                        M * K, B, ba, st),
                          "dgrad");
            } else {
                for (size_t z = 0; z < B; z++)
                    pgd_check(gemm16(dt, M, K, N8, g16 + z * M * N8, N8, 0, bp + z * K * N8, N8, 0, ga->dev,
                                            K, 0, 1, z == 0 ? ba : 1, st),
                              "dgrad");
            }
        }
        pgd_free(g16, gbytes);
        if (bpad)
            pgd_free(bpad, bbytes);
    }
    /* wgrad operands: A^T [K, M8] and dC^T [N, M8] per batch; when only A is
     * batched the batch folds into the reduction (M_eff = B*M) */
    if (gb) {
        bool fold = s.abat && !s.bbat;
        size_t Bw = fold ? 1 : B;
        size_t Mw = fold ? B * M : M;
        size_t M8 = up8(Mw);
        size_t atb = Bw * K * M8 * 2, gtb = Bw * N * M8 * 2;
        uint16_t *at = tmp_alloc(atb), *gt = tmp_alloc(gtb);
        bool ok = at && gt;
        size_t a_bat = s.abat && !fold ? B : 1;
        if (ok)
            ok = pgd_check(pgk_transpose_to16(dt, dt, a->dev, Mw, K, K, at, M8, a_bat, M * K, K * M8, st),
                           "stage A^T");
        if (ok && a_bat < Bw) /* A unbatched but B batched: same A^T for every batch */
            for (size_t z = 1; z < Bw && ok; z++)
                ok = pgd_d2d(at + z * K * M8, at, K * M8 * 2);
        if (ok)
            ok = pgd_check(pgk_transpose_to16(dt, 0, g->dev, Mw, N, N, gt, M8, Bw, Mw * N, N * M8, st),
                           "stage dC^T");
        if (ok) {
            if (s.bbat || Bw == 1) {
                pgd_check(gemm16(dt, K, N, M8, at, M8, K * M8, gt, M8, N * M8, gb->dev, N, s.bbat ? K * N : 0,
                                        Bw, bbeta, st),
                          "wgrad");
            } else {
                for (size_t z = 0; z < Bw; z++)
                    pgd_check(gemm16(dt, K, N, M8, at + z * K * M8, M8, 0, gt + z * N * M8, M8, 0, gb->dev,
                                            N, 0, 1, z == 0 ? bbeta : 1, st),
                              "wgrad");
            }
        }
        pgd_free(at, atb);
        pgd_free(gt, gtb);
    }
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
    pgk_stream st = pgd_stream();
    int dt = (int)dtype;
    size_t K8 = up8(k);
    size_t abytes = m * K8 * 2, bbytes = n * K8 * 2;
    uint16_t *ap = tmp_alloc(abytes), *bt = tmp_alloc(bbytes);
    if (ap && bt && pgd_check(pgk_copy_to16(dt, dt, a, m, k, lda, ap, K8, 1, 0, 0, st), "stage A") &&
        pgd_check(pgk_transpose_to16(dt, dt, b, k, n, ldb, bt, K8, 1, 0, 0, st), "stage B^T"))
        pgd_check(gemm16(dt, m, n, K8, ap, K8, 0, bt, K8, 0, c, ldc, 0, 1, 0, st), "pg_gemm_ex");
    pgd_free(ap, abytes);
    pgd_free(bt, bbytes);
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
