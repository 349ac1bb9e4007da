/*
 * Tensor-level forward ops (the reference's ops/elementwise.h,
 * ops/activations.h and ops/matmul.h) over device tensors: each returns a
 * new f32 tensor whose elements are computed on the device, or NULL on bad
 * input (reason in pg_autograd_last_error()).
 *
 * They run the kernels the autograd ops run (with the JIT on, elementwise
 * ops are recorded and executed as one fused kernel, bit for bit the eager
 * kernels' values), so pg_add(a, b) holds exactly the value of
 * pg_ag_add on nodes of a and b.  Strided views (pg_tensor_permute_view)
 * are gathered into row-major order first.  Shape rules are the
 * reference's: NumPy broadcasting for the binary ops (ops/common.h:6-54),
 * pg_matmul as matmul.c:186-284, pg_bmm as matmul.c:340-369 (three-dim
 * operands with one batch size, one dtype, f32 out).
 */
#define _POSIX_C_SOURCE 200809L
#include "internal.h"

#include "picograd/ops.h"

static pg_tensor *binary(int op, const pg_tensor *a, const pg_tensor *b)
{
    if (!a || !b) {
        pga_set_err("binary op: null tensor");
        return NULL;
    }
    pg_tensor *oa, *ob;
    const pg_tensor *ca = pgt_contiguous(a, &oa), *cb = pgt_contiguous(b, &ob);
    pg_tensor *y = ca && cb ? pga_binary_fwd(op, ca, cb) : NULL;
    pg_tensor_free(oa);
    pg_tensor_free(ob);
    return y;
}

static pg_tensor *unary(int op, const pg_tensor *a, float p0, float p1)
{
    if (!a) {
        pga_set_err("unary op: null tensor");
        return NULL;
    }
    pg_tensor *oa;
    const pg_tensor *ca = pgt_contiguous(a, &oa);
    pg_tensor *y = ca ? pga_unary_fwd(op, ca, p0, p1) : NULL;
    pg_tensor_free(oa);
    return y;
}

static pg_tensor *unsupported(const char *what)
{
    pga_set_err("%s is not part of the MI355X build", what);
    return NULL;
}

/* elementwise.c:556-591 */
pg_tensor *pg_add(const pg_tensor *a, const pg_tensor *b) { return binary(PGK_ADD, a, b); }
pg_tensor *pg_sub(const pg_tensor *a, const pg_tensor *b) { return binary(PGK_SUB, a, b); }
pg_tensor *pg_mul(const pg_tensor *a, const pg_tensor *b) { return binary(PGK_MUL, a, b); }
pg_tensor *pg_div(const pg_tensor *a, const pg_tensor *b) { return binary(PGK_DIV, a, b); }
pg_tensor *pg_pow(const pg_tensor *a, const pg_tensor *b)
{
    (void)a;
    (void)b;
    return unsupported("pg_pow");
}

/* elementwise.c:661-735 */
pg_tensor *pg_neg(const pg_tensor *a) { return unary(PGK_NEG, a, 0.0f, 0.0f); }
pg_tensor *pg_abs(const pg_tensor *a) { return unary(PGK_ABS, a, 0.0f, 0.0f); }
pg_tensor *pg_sqrt(const pg_tensor *a) { return unary(PGK_SQRT, a, 0.0f, 0.0f); }
pg_tensor *pg_exp(const pg_tensor *a) { return unary(PGK_EXP, a, 0.0f, 0.0f); }
pg_tensor *pg_log(const pg_tensor *a) { return unary(PGK_LOG, a, 0.0f, 0.0f); }
pg_tensor *pg_sin(const pg_tensor *a) { return unary(PGK_SIN, a, 0.0f, 0.0f); }
pg_tensor *pg_cos(const pg_tensor *a) { return unary(PGK_COS, a, 0.0f, 0.0f); }
pg_tensor *pg_erf(const pg_tensor *a) { return unary(PGK_ERF, a, 0.0f, 0.0f); }
pg_tensor *pg_clamp(const pg_tensor *a, float lo, float hi)
{
    if (lo > hi) {
        pga_set_err("pg_clamp: lo > hi");
        return NULL;
    }
    return unary(PGK_CLAMP, a, lo, hi);
}

/* activations.c:136-191 */
pg_tensor *pg_relu(const pg_tensor *a) { return unary(PGK_RELU, a, 0.0f, 0.0f); }
pg_tensor *pg_leaky_relu(const pg_tensor *a, float alpha) { return unary(PGK_LEAKY, a, alpha, 0.0f); }
pg_tensor *pg_sigmoid(const pg_tensor *a) { return unary(PGK_SIGMOID, a, 0.0f, 0.0f); }
pg_tensor *pg_tanh(const pg_tensor *a) { return unary(PGK_TANH, a, 0.0f, 0.0f); }
pg_tensor *pg_gelu(const pg_tensor *a) { return unary(PGK_GELU, a, 0.0f, 0.0f); }
pg_tensor *pg_softmax(const pg_tensor *t, size_t axis)
{
    (void)t;
    (void)axis;
    return unsupported("pg_softmax");
}
pg_tensor *pg_log_softmax(const pg_tensor *t, size_t axis)
{
    (void)t;
    (void)axis;
    return unsupported("pg_log_softmax");
}

/* matmul.c:186-284 */
pg_tensor *pg_matmul(const pg_tensor *a, const pg_tensor *b)
{
    if (!a || !b) {
        pga_set_err("pg_matmul: null tensor");
        return NULL;
    }
    pg_tensor *oa, *ob;
    const pg_tensor *ca = pgt_contiguous(a, &oa), *cb = pgt_contiguous(b, &ob);
    pg_tensor *y = ca && cb ? pgm_matmul_forward(ca, cb) : NULL;
    pg_tensor_free(oa);
    pg_tensor_free(ob);
    return y;
}

/* matmul.c:340-369 */
pg_tensor *pg_bmm(const pg_tensor *a, const pg_tensor *b)
{
    if (!a || !b || a->ndim != 3 || b->ndim != 3 || a->shape[0] != b->shape[0] || a->shape[2] != b->shape[1] ||
        a->dtype != b->dtype) {
        pga_set_err("pg_bmm: needs [B, M, K] and [B, K, N] operands of one dtype");
        return NULL;
    }
    return pg_matmul(a, b);
}

pg_tensor *pg_addmm(const pg_tensor *input, const pg_tensor *m1, const pg_tensor *m2, float alpha, float beta)
{
    (void)input;
    (void)m1;
    (void)m2;
    (void)alpha;
    (void)beta;
    return unsupported("pg_addmm");
}

pg_tensor *pg_tensordot(const pg_tensor *a, const pg_tensor *b, size_t ndims, const size_t *axes_a,
                        const size_t *axes_b)
{
    (void)a;
    (void)b;
    (void)ndims;
    (void)axes_a;
    (void)axes_b;
    return unsupported("pg_tensordot");
}
