/*
 * A C caller of the device library, written against include/picograd the
 * way the reference's own callers are written: the fused add + relu and
 * 3-D broadcast graphs of tests/test_jit.c:43-96 checked against the eager
 * tensor ops, the XOR training loop and eager-vs-JIT inference of
 * examples/train_xor_jit.c:24-150, and the tensor utilities of
 * core/tensor.h (arange, linspace, eye, get/set, allclose, permute_view,
 * print, the pool).  Host reads go through pg_tensor_sync_host or
 * pg_tensor_get, the one change a reference caller needs.
 *
 * Exit status 0 when every check passes; each failure prints a line.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "picograd/amd.h"
#include "picograd/autograd.h"
#include "picograd/jit.h"
#include "picograd/ops.h"
#include "picograd/sgd.h"
#include "picograd/tensor.h"

static int g_fail, g_checks;

#define CHECK(c)                                                                                                  \
    do {                                                                                                          \
        g_checks++;                                                                                               \
        if (!(c)) {                                                                                               \
            g_fail++;                                                                                             \
            printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);                                                   \
        }                                                                                                         \
    } while (0)

static int closef(float a, float b) { return fabsf(a - b) <= 1e-5f + 1e-5f * fabsf(b); }

/* test_jit.c:43-70: relu(a[2,4] + b[4]) fused, against eager pg_add + pg_relu */
static void add_relu_known_answer(void)
{
    pg_jit_graph *g = pg_jit_graph_new();
    int a = pg_jit_add_input(g, 2, (size_t[]){2, 4});
    int b = pg_jit_add_input(g, 1, (size_t[]){4});
    int r = pg_jit_relu(g, pg_jit_add(g, a, b));
    pg_jit_mark_output(g, r);
    pg_jit_exe *e = pg_jit_compile(g);
    CHECK(e != NULL);
    if (!e) {
        printf("  jit: %s\n", pg_jit_last_error());
        pg_jit_graph_free(g);
        return;
    }
    float a0[8] = {-1, 2, -3, 4, -5, 6, -7, 8};
    float b0[4] = {10, 20, 30, 40};
    pg_tensor *pa = pg_tensor_from_data(2, (size_t[]){2, 4}, a0);
    pg_tensor *pb = pg_tensor_from_data(1, (size_t[]){4}, b0);
    const pg_tensor *ins[2] = {pa, pb};
    pg_tensor *out = pg_jit_run_single(e, ins, 2);
    CHECK(out != NULL);
    float want[8] = {9, 22, 27, 44, 5, 26, 23, 48};
    CHECK(out && pg_tensor_sync_host(out));
    for (size_t i = 0; out && i < 8; i++)
        CHECK(closef(out->data[i], want[i]));
    pg_tensor *eager = pg_add(pa, pb);
    pg_tensor *eager2 = pg_relu(eager);
    CHECK(eager2 && pg_tensor_allclose(out, eager2, 0.0f, 0.0f));
    pg_tensor_free(pa);
    pg_tensor_free(pb);
    pg_tensor_free(out);
    pg_tensor_free(eager);
    pg_tensor_free(eager2);
    pg_jit_exe_free(e);
    pg_jit_graph_free(g);
}

/* test_jit.c:72-96: (a[2,3,4] + b[3,4]) * c[4] */
static void broadcast_3d(void)
{
    pg_jit_graph *g = pg_jit_graph_new();
    int a = pg_jit_add_input(g, 3, (size_t[]){2, 3, 4});
    int b = pg_jit_add_input(g, 2, (size_t[]){3, 4});
    int c = pg_jit_add_input(g, 1, (size_t[]){4});
    pg_jit_mark_output(g, pg_jit_mul(g, pg_jit_add(g, a, b), c));
    pg_jit_exe *e = pg_jit_compile(g);
    CHECK(e != NULL);
    pg_seed(99);
    pg_tensor *ta = pg_tensor_uniform(3, (size_t[]){2, 3, 4}, -2, 2);
    pg_tensor *tb = pg_tensor_uniform(2, (size_t[]){3, 4}, -2, 2);
    pg_tensor *tc = pg_tensor_uniform(1, (size_t[]){4}, -2, 2);
    const pg_tensor *ins[3] = {ta, tb, tc};
    pg_tensor *jout = e ? pg_jit_run_single(e, ins, 3) : NULL;
    pg_tensor *e0 = pg_add(ta, tb);
    pg_tensor *e1 = pg_mul(e0, tc);
    CHECK(jout && e1 && pg_tensor_allclose(jout, e1, 1e-6f, 1e-6f));
    /* the element at [1,2,3] by hand */
    size_t i3[3] = {1, 2, 3}, i2[2] = {2, 3}, i1[1] = {3};
    float v = (pg_tensor_get(ta, i3) + pg_tensor_get(tb, i2)) * pg_tensor_get(tc, i1);
    CHECK(e1 && closef(pg_tensor_get(e1, i3), v));
    pg_tensor_free(ta);
    pg_tensor_free(tb);
    pg_tensor_free(tc);
    pg_tensor_free(jout);
    pg_tensor_free(e0);
    pg_tensor_free(e1);
    pg_jit_exe_free(e);
    pg_jit_graph_free(g);
}

/* test_jit.c:98-140: each unary op fused against its eager tensor op */
static void unary_ops(void)
{
    pg_jit_op_t ops[] = {PG_JIT_NEG, PG_JIT_EXP, PG_JIT_LOG, PG_JIT_SQRT, PG_JIT_SIN, PG_JIT_COS,
                         PG_JIT_ABS, PG_JIT_RELU, PG_JIT_SIGMOID, PG_JIT_TANH, PG_JIT_GELU, PG_JIT_ERF};
    for (size_t oi = 0; oi < sizeof ops / sizeof ops[0]; oi++) {
        pg_jit_graph *g = pg_jit_graph_new();
        int inp = pg_jit_add_input(g, 1, (size_t[]){8});
        pg_jit_mark_output(g, pg_jit_add_op(g, ops[oi], &inp, 1));
        pg_jit_exe *exe = pg_jit_compile(g);
        CHECK(exe != NULL);
        pg_tensor *t = (ops[oi] == PG_JIT_LOG || ops[oi] == PG_JIT_SQRT) ? pg_tensor_uniform(1, (size_t[]){8}, 0.5f, 2.0f)
                                                                         : pg_tensor_uniform(1, (size_t[]){8}, -2.0f, 2.0f);
        const pg_tensor *ins[1] = {t};
        pg_tensor *jout = exe ? pg_jit_run_single(exe, ins, 1) : NULL;
        pg_tensor *eager = NULL;
        switch (ops[oi]) {
        case PG_JIT_NEG: eager = pg_neg(t); break;
        case PG_JIT_EXP: eager = pg_exp(t); break;
        case PG_JIT_LOG: eager = pg_log(t); break;
        case PG_JIT_SQRT: eager = pg_sqrt(t); break;
        case PG_JIT_SIN: eager = pg_sin(t); break;
        case PG_JIT_COS: eager = pg_cos(t); break;
        case PG_JIT_ABS: eager = pg_abs(t); break;
        case PG_JIT_RELU: eager = pg_relu(t); break;
        case PG_JIT_SIGMOID: eager = pg_sigmoid(t); break;
        case PG_JIT_TANH: eager = pg_tanh(t); break;
        case PG_JIT_GELU: eager = pg_gelu(t); break;
        case PG_JIT_ERF: eager = pg_erf(t); break;
        default: break;
        }
        CHECK(jout && eager && pg_tensor_allclose(jout, eager, 1e-4f, 1e-4f));
        pg_tensor_free(t);
        pg_tensor_free(jout);
        pg_tensor_free(eager);
        pg_jit_exe_free(exe);
        pg_jit_graph_free(g);
    }
}

/* train_xor_jit.c:24-150: XOR with pg_ag ops and SGD (JIT backward), then
 * inference through the eager tensor ops and through fused add + tanh */
static pg_node *forward(pg_node *x, pg_node *w1, pg_node *b1, pg_node *w2, pg_node *b2)
{
    pg_node *mm1 = pg_ag_matmul(x, w1);
    pg_node *z1 = pg_ag_add(mm1, b1);
    pg_node_free(mm1);
    pg_node *h = pg_ag_tanh(z1);
    pg_node_free(z1);
    pg_node *mm2 = pg_ag_matmul(h, w2);
    pg_node_free(h);
    pg_node *y = pg_ag_add(mm2, b2);
    pg_node_free(mm2);
    return y;
}

static void xor_train_and_infer(void)
{
    pg_jit_graph *g1 = pg_jit_graph_new();
    int a = pg_jit_add_input(g1, 2, (size_t[]){4, 8});
    int b = pg_jit_add_input(g1, 1, (size_t[]){8});
    pg_jit_mark_output(g1, pg_jit_tanh(g1, pg_jit_add(g1, a, b)));
    pg_jit_exe *add_tanh = pg_jit_compile(g1);
    pg_jit_graph_free(g1);
    CHECK(add_tanh != NULL);

    pg_seed(7);
    float xraw[8] = {0, 0, 0, 1, 1, 0, 1, 1};
    float yraw[4] = {0, 1, 1, 0};
    pg_node *x = pg_var_from_data(2, (size_t[]){4, 2}, xraw, false);
    pg_node *y = pg_var_from_data(2, (size_t[]){4, 1}, yraw, false);
    pg_node *w1 = pg_var_uniform(2, (size_t[]){2, 8}, -1, 1, true);
    pg_node *b1 = pg_var_zeros(1, (size_t[]){8}, true);
    pg_node *w2 = pg_var_uniform(2, (size_t[]){8, 1}, -1, 1, true);
    pg_node *b2 = pg_var_zeros(1, (size_t[]){1}, true);
    pg_sgd_cfg cfg = pg_sgd_cfg_default();
    cfg.lr = 0.1f;
    cfg.momentum = 0.9f;
    pg_sgd *opt = pg_sgd_new(&cfg);
    pg_sgd_add_param(opt, w1);
    pg_sgd_add_param(opt, b1);
    pg_sgd_add_param(opt, w2);
    pg_sgd_add_param(opt, b2);
    pg_autograd_set_jit(true);
    float first = -1.0f, last = -1.0f;
    for (int it = 0; it < 1000; it++) {
        pg_sgd_zero_grad(opt);
        pg_node *out = forward(x, w1, b1, w2, b2);
        pg_node *d = pg_ag_sub(out, y);
        pg_node *sq = pg_ag_mul(d, d);
        pg_node *loss = pg_ag_mean_all(sq);
        pg_node_free(out);
        pg_node_free(d);
        pg_node_free(sq);
        pg_backward(loss);
        if (it == 0 || it == 999) {
            size_t i0[1] = {0};
            float l = pg_tensor_get(pg_node_value(loss), i0);
            if (it == 0)
                first = l;
            else
                last = l;
        }
        pg_sgd_step(opt);
        pg_node_free(loss);
    }
    printf("xor loss %.6f -> %.6f\n", first, last);
    CHECK(last < 0.05f * first);
    CHECK(pg_autograd_last_was_jit());

    /* inference: eager tensor ops against matmul + fused add+tanh */
    pg_tensor *xt = pg_tensor_from_data(2, (size_t[]){4, 2}, xraw);
    pg_tensor *mm1 = pg_matmul(xt, pg_node_value(w1));
    pg_tensor *z1 = pg_add(mm1, pg_node_value(b1));
    pg_tensor *h = pg_tanh(z1);
    const pg_tensor *ins[2] = {mm1, pg_node_value(b1)};
    pg_tensor *hj = add_tanh ? pg_jit_run_single(add_tanh, ins, 2) : NULL;
    CHECK(h && hj && pg_tensor_allclose(hj, h, 1e-5f, 1e-6f));
    pg_tensor *mm2 = pg_matmul(h, pg_node_value(w2));
    pg_tensor *out = pg_add(mm2, pg_node_value(b2));
    CHECK(out && pg_tensor_sync_host(out));
    for (size_t i = 0; out && i < 4; i++)
        CHECK(fabsf(out->data[i] - yraw[i]) < 0.25f);
    pg_tensor *tensors[] = {xt, mm1, z1, h, hj, mm2, out};
    for (size_t i = 0; i < sizeof tensors / sizeof tensors[0]; i++)
        pg_tensor_free(tensors[i]);
    pg_sgd_free(opt);
    pg_node *nodes[] = {x, y, w1, b1, w2, b2};
    for (size_t i = 0; i < 6; i++)
        pg_node_free(nodes[i]);
    pg_jit_exe_free(add_tanh);
}

/* core/tensor.h utilities on device tensors */
static void tensor_utilities(void)
{
    pg_tensor *ar = pg_tensor_arange(0.5f, 3.0f, 0.75f); /* ceil(2.5 / 0.75) = 4 */
    CHECK(ar && ar->numel == 4);
    size_t i[2] = {3, 0};
    CHECK(ar && pg_tensor_get(ar, i) == 0.5f + 0.75f * 3.0f);
    CHECK(pg_tensor_arange(1.0f, 1.0f, 1.0f) == NULL);
    pg_tensor *ls = pg_tensor_linspace(-1.0f, 1.0f, 5);
    float lw[5] = {-1.0f, -0.5f, 0.0f, 0.5f, 1.0f};
    pg_tensor *lsw = pg_tensor_from_data(1, (size_t[]){5}, lw);
    CHECK(ls && pg_tensor_allclose(ls, lsw, 0.0f, 0.0f));
    pg_tensor *ey = pg_tensor_eye(3);
    size_t d[2] = {1, 1}, o[2] = {1, 2};
    CHECK(ey && pg_tensor_get(ey, d) == 1.0f && pg_tensor_get(ey, o) == 0.0f);
    pg_tensor_set(ey, o, 7.0f);
    CHECK(pg_tensor_get(ey, o) == 7.0f);
    /* bf16 set rounds to nearest even */
    pg_tensor *hb = pg_tensor_zeros_dtype(PG_DTYPE_BF16, 1, (size_t[]){2});
    size_t j[1] = {1};
    pg_tensor_set(hb, j, 1.00390625f); /* 1 + 2^-8: halfway, rounds to even 1.0 */
    CHECK(pg_tensor_get(hb, j) == 1.0f);
    pg_tensor_set(hb, j, 1.01171875f); /* 1 + 3 * 2^-8: halfway, rounds up to 1 + 2^-6 */
    CHECK(pg_tensor_get(hb, j) == 1.015625f);

    /* a transposed view: get follows the strides, clone and pg_add read it
     * in row-major order, allclose against an explicit transpose */
    float m[6] = {1, 2, 3, 4, 5, 6};
    pg_tensor *tm = pg_tensor_from_data(2, (size_t[]){2, 3}, m);
    pg_tensor *tt = pg_tensor_permute_view(tm, (size_t[]){1, 0});
    CHECK(tt && tt->shape[0] == 3 && tt->shape[1] == 2 && tt->is_view);
    size_t k[2] = {2, 1};
    CHECK(tt && pg_tensor_get(tt, k) == 6.0f);
    float mt[6] = {1, 4, 2, 5, 3, 6};
    pg_tensor *want = pg_tensor_from_data(2, (size_t[]){3, 2}, mt);
    pg_tensor *cl = pg_tensor_clone(tt);
    CHECK(cl && pg_tensor_allclose(cl, want, 0.0f, 0.0f));
    pg_tensor *zero = pg_tensor_zeros(1, (size_t[]){2});
    pg_tensor *sum = pg_add(tt, zero);
    CHECK(sum && pg_tensor_allclose(sum, want, 0.0f, 0.0f));
    CHECK(pg_tensor_permute_view(tm, (size_t[]){0, 0}) == NULL);

    /* print: the reference's text */
    char buf[256] = {0};
    FILE *f = fmemopen(buf, sizeof buf, "w");
    pg_tensor_print(want, f);
    fclose(f);
    CHECK(strcmp(buf, "[[1, 4],\n [2, 5],\n [3, 6]]\n") == 0);
    if (strcmp(buf, "[[1, 4],\n [2, 5],\n [3, 6]]\n") != 0)
        printf("  print gave: %s", buf);

    /* bmm: [2,2,3] . [2,3,1] */
    float ba[12] = {1, 2, 3, 4, 5, 6, -1, -2, -3, -4, -5, -6};
    float bb[6] = {1, 0, 2, 0, 1, 1};
    pg_tensor *A = pg_tensor_from_data(3, (size_t[]){2, 2, 3}, ba);
    pg_tensor *B = pg_tensor_from_data(3, (size_t[]){2, 3, 1}, bb);
    pg_tensor *C = pg_bmm(A, B);
    float cw[4] = {7, 16, -5, -11};
    pg_tensor *Cw = pg_tensor_from_data(3, (size_t[]){2, 2, 1}, cw);
    CHECK(C && pg_tensor_allclose(C, Cw, 0.0f, 0.0f));
    CHECK(pg_bmm(A, A) == NULL);
    CHECK(pg_softmax(A, 1) == NULL);

    pg_tensor *all[] = {ar, ls, lsw, ey, hb, tt, tm, want, cl, zero, sum, A, B, C, Cw};
    for (size_t q = 0; q < sizeof all / sizeof all[0]; q++)
        pg_tensor_free(all[q]);
    /* the pool: freed blocks are cached, clear hands them back */
    CHECK(pg_tensor_pool_size() > 0 && pg_tensor_pool_bytes() > 0);
    pg_tensor_pool_clear();
    CHECK(pg_tensor_pool_size() == 0 && pg_tensor_pool_bytes() == 0);
}

int main(void)
{
    if (pg_amd_init() != 0) {
        printf("FAIL no device: %s\n", pg_amd_last_error());
        return 2;
    }
    add_relu_known_answer();
    broadcast_3d();
    unary_ops();
    xor_train_and_infer();
    tensor_utilities();
    pg_amd_sync();
    printf("%d checks, %d failed\n", g_checks, g_fail);
    return g_fail ? 1 : 0;
}
