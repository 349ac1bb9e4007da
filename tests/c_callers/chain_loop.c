/*
 * Config 1's timed loop in C, as the reference's own benchmark runs it
 * (examples/train_xor_jit.c:200-214): per iteration three fresh [64, 64]
 * leaves from host data, (a + b) * c -> relu -> tanh -> sum_all, pg_backward,
 * and every node freed.  The library is loaded with dlopen, so the same
 * program times this build (its stream synchronised once at the end) and
 * the reference's CPU build (oracle/_ref), each resolving only its own
 * symbols.  After the loop the last iteration's grads are read back and
 * checked against the chain rule evaluated here in double precision.
 *
 *   chain_loop <library.so> <iterations> [jit 0|1]
 *
 * Prints one JSON line: {"us_per_iter": ..., "iters": ..., "max_err": ...}.
 * Exit status 0 when the grads agree to 1e-5.
 */
#define _POSIX_C_SOURCE 200809L
#include <dlfcn.h>
#include <math.h>
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <time.h>

#include "picograd/autograd.h"

#define R 64
#define C 64

typedef pg_node *(*var_fn)(size_t, const size_t *, const float *, bool);
typedef pg_node *(*bin_fn)(pg_node *, pg_node *);
typedef pg_node *(*un_fn)(pg_node *);
typedef void (*node_fn)(pg_node *);
typedef void (*jit_fn)(bool);
typedef int (*sync_fn)(void);
typedef bool (*copy_fn)(const pg_tensor *, void *);

static void *sym(void *h, const char *name, bool required)
{
    void *p = dlsym(h, name);
    if (!p && required) {
        fprintf(stderr, "chain_loop: %s missing: %s\n", name, dlerror());
        exit(2);
    }
    return p;
}

/* splitmix64 uniform draws in [-1, 1) (any fixed data will do) */
static float draw(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)((double)(z >> 40) / (double)(1ull << 24) * 2.0 - 1.0);
}

int main(int argc, char **argv)
{
    if (argc < 3) {
        fprintf(stderr, "usage: chain_loop <library.so> <iterations> [jit 0|1]\n");
        return 2;
    }
    void *h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!h) {
        fprintf(stderr, "chain_loop: %s\n", dlerror());
        return 2;
    }
    const long iters = atol(argv[2]);
    var_fn var = (var_fn)sym(h, "pg_var_from_data", true);
    bin_fn add = (bin_fn)sym(h, "pg_ag_add", true), mul = (bin_fn)sym(h, "pg_ag_mul", true);
    un_fn relu = (un_fn)sym(h, "pg_ag_relu", true), tanh_ = (un_fn)sym(h, "pg_ag_tanh", true);
    un_fn sum_all = (un_fn)sym(h, "pg_ag_sum_all", true);
    node_fn backward = (node_fn)sym(h, "pg_backward", true), node_free = (node_fn)sym(h, "pg_node_free", true);
    jit_fn set_jit = (jit_fn)sym(h, "pg_autograd_set_jit", true);
    sync_fn sync = (sync_fn)sym(h, "pg_amd_sync", false);       /* device builds only */
    copy_fn to_host = (copy_fn)sym(h, "pg_tensor_copy_to_host", false);
    set_jit(argc < 4 || atoi(argv[3]) != 0);

    static float a[R * C], b[R * C], c[R * C];
    uint64_t s = 42;
    for (int i = 0; i < R * C; i++) {
        a[i] = draw(&s);
        b[i] = draw(&s);
        c[i] = draw(&s);
    }
    const size_t shp[2] = {R, C};
    pg_node *keep[3] = {0};
    struct timespec t0, t1;
    for (long it = -20; it < iters; it++) { /* 20 untimed warm-up iterations */
        if (it == 0) {
            if (sync)
                sync();
            clock_gettime(CLOCK_MONOTONIC, &t0);
        }
        pg_node *na = var(2, shp, a, true), *nb = var(2, shp, b, true), *nc = var(2, shp, c, true);
        pg_node *x0 = add(na, nb), *x1 = mul(x0, nc), *x2 = relu(x1), *x3 = tanh_(x2), *loss = sum_all(x3);
        backward(loss);
        pg_node *order[8] = {loss, x3, x2, x1, x0, na, nb, nc};
        for (int k = 0; k < 8; k++) {
            if (it == iters - 1 && k >= 5) {
                keep[k - 5] = order[k]; /* the leaves of the last iteration, read below */
                continue;
            }
            node_free(order[k]);
        }
    }
    if (sync)
        sync();
    clock_gettime(CLOCK_MONOTONIC, &t1);
    const double us = ((double)(t1.tv_sec - t0.tv_sec) * 1e6 + (double)(t1.tv_nsec - t0.tv_nsec) / 1e3) / (double)iters;

    /* d/da = d/db = tanh'(relu(u)) relu'(u) c, d/dc = tanh'(relu(u)) relu'(u) (a + b), u = (a + b) c */
    double max_err = 0.0;
    static float g[3][R * C];
    for (int k = 0; k < 3; k++) {
        const pg_tensor *gt = keep[k]->grad;
        if (!gt) {
            fprintf(stderr, "chain_loop: no grad\n");
            return 1;
        }
        if (to_host)
            to_host(gt, g[k]);
        else
            for (int i = 0; i < R * C; i++)
                g[k][i] = ((const float *)gt->data)[i];
    }
    for (int i = 0; i < R * C; i++) {
        const double sum = (double)a[i] + (double)b[i], u = sum * (double)c[i];
        const double r = u > 0.0 ? u : 0.0, th = tanh(r);
        const double d = (1.0 - th * th) * (u > 0.0 ? 1.0 : 0.0);
        const double want[3] = {d * c[i], d * c[i], d * sum};
        for (int k = 0; k < 3; k++) {
            const double e = fabs((double)g[k][i] - want[k]);
            max_err = e > max_err ? e : max_err;
        }
    }
    for (int k = 0; k < 3; k++)
        node_free(keep[k]);
    printf("{\"us_per_iter\": %.4f, \"iters\": %ld, \"max_err\": %.3e}\n", us, iters, max_err);
    return max_err <= 1e-5 ? 0 : 1;
}
