/*
 * CPU oracle for the picograd backward path -- TEST INFRASTRUCTURE ONLY.
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the checker.  The product library never uses it.
 * Each function restates the reference algorithm at the cited file:line.
 */
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------- RNG (tensor.c:289-339) ---------------- */

static unsigned long long g_state = 0x9E3779B97F4A7C15ULL;

void orc_seed(unsigned long long seed)
{
    /* tensor.c:292-297: a zero seed selects the default state */
    g_state = seed != 0 ? seed : 0x9E3779B97F4A7C15ULL;
}

static unsigned long long orc_next(void)
{
    /* splitmix64 finaliser, tensor.c:299-309 */
    g_state += 0x9E3779B97F4A7C15ULL;
    unsigned long long z = g_state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static float orc_u01(void)
{
    /* top 24 bits scaled to [0,1), tensor.c:311-314 */
    return (float)(orc_next() >> 40) * (1.0f / 16777216.0f);
}

void orc_uniform(float *out, size_t n, float low, float high)
{
    /* tensor.c:316-323 */
    for (size_t i = 0; i < n; i++) {
        out[i] = low + orc_u01() * (high - low);
    }
}

void orc_normal(float *out, size_t n, float mean, float stddev)
{
    /* Box-Muller, cosine branch only, one pair of draws per element
     * (tensor.c:325-339) */
    for (size_t i = 0; i < n; i++) {
        float u1 = orc_u01();
        float u2 = orc_u01();
        if (u1 < 1e-12f)
            u1 = 1e-12f;
        /* stddev * radius * cos, formed as (stddev * cos) * radius: the
         * order the reference's -ffast-math build (clang) evaluates it in,
         * which the golden streams pin bit for bit for stddev != 1 */
        float radius = sqrtf(-2.0f * logf(u1));
        float c = cosf(2.0f * 3.14159265358979f * u2);
        out[i] = mean + (stddev * c) * radius;
    }
}

/* ---------------- conversions (convert.h:15-104) ---------------- */

uint16_t orc_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 255) {
        /* Inf stays Inf; NaN keeps the top payload bits and is quieted
         * (convert.h:22-28) */
        if (man == 0)
            return (uint16_t)(sign | 0x7C00u);
        uint16_t q = (uint16_t)(sign | 0x7C00u | (man >> 13));
        if ((q & 0x3FFu) == 0)
            q |= 1u;
        return (uint16_t)(q | 0x200u);
    }
    int32_t e = (int32_t)ex - 112; /* rebias 127 -> 15 */
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        /* subnormal result; below 2^-25 it flushes to signed zero
         * (convert.h:31-43) */
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t sh = (uint32_t)(1 - e) + 13u;
        uint32_t keep = man >> sh;
        uint32_t rem = man & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (keep & 1u)))
            keep++;
        return (uint16_t)(sign | keep);
    }
    /* normal: round the 13 dropped bits to nearest even; a carry out of the
     * mantissa bumps the exponent (convert.h:45-51) */
    uint32_t r = man + 0xFFFu + ((man >> 13) & 1u);
    if (r & 0x800000u) {
        r = 0;
        e++;
    }
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (r >> 13));
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* renormalise a subnormal (convert.h:60-69) */
            int32_t e = 1;
            while ((man & 0x400u) == 0) {
                man <<= 1;
                e--;
            }
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(e + 112) << 23) | (man << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    /* a NaN becomes a positive quiet NaN keeping only bit 16 of the input
     * (the sign is dropped: convert.h:89-92) */
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu) != 0)
        return (uint16_t)(0x7FC0u | ((x >> 16) & 1u));
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

float orc_bf16_to_f32(uint16_t h)
{
    uint32_t bits = (uint32_t)h << 16;
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

void orc_cast_f32(int dtype, const float *src, uint16_t *dst, size_t n)
{
    for (size_t i = 0; i < n; i++)
        dst[i] = dtype == ORC_F16 ? orc_f32_to_f16(src[i]) : orc_f32_to_bf16(src[i]);
}

void orc_round_f32(int dtype, float *x, size_t n)
{
    if (dtype == ORC_F32)
        return;
    for (size_t i = 0; i < n; i++)
        x[i] = dtype == ORC_F16 ? orc_f16_to_f32(orc_f32_to_f16(x[i]))
                                : orc_bf16_to_f32(orc_f32_to_bf16(x[i]));
}

/* ---------------- SGD (sgd.c:111-162) ---------------- */

void orc_sgd_step(float *p, const float *g, float *buf, size_t n, float lr,
                  float momentum, float dampening, float weight_decay,
                  bool nesterov)
{
    for (size_t j = 0; j < n; j++) {
        float gj = g[j];
        if (weight_decay != 0.0f)
            gj += weight_decay * p[j]; /* decay joins the grad first */
        float u = gj;
        if (momentum != 0.0f) {
            /* buffer starts at zero, so step 1 gives (1-d)*g (sgd.c:134-156) */
            buf[j] = buf[j] * momentum + gj * (1.0f - dampening);
            u = nesterov ? gj + momentum * buf[j] : buf[j];
        }
        p[j] -= lr * u;
    }
}

/* ---------------- Adam / AdamW and gradient clipping ---------------- */

float orc_adam_bias_correction(float beta, unsigned long long step)
{
    /* adam.c:121-125: 1 - beta^t in f32 through powf, floored at 1e-12 */
    float bc = 1.0f - powf(beta, (float)step);
    return bc < 1e-12f ? 1e-12f : bc;
}

void orc_adam_step(float *p, const float *g, float *m, float *v, float *vmax,
                   size_t n, float lr, float beta1, float beta2, float eps,
                   float weight_decay, bool amsgrad, bool decoupled,
                   unsigned long long step)
{
    /* adam.c:157-177 in the order the reference's -O3 -ffast-math build
     * evaluates it (its scalar remainder loop, with IEEE sqrt and divide):
     * the moments reassociated to g + b1*(m - g) and g^2 + b2*(v - g^2),
     * v_hat = v * (1/bc2), and lr*m_hat/(sqrt(v_hat) + eps) folded to
     * (m*lr) / ((sqrt(v_hat) + eps) * bc1).  Its 8-wide loop replaces the
     * square root and the quotient by x86 reciprocal estimates plus one
     * Newton step, which this restatement does not follow. */
    const float bc1 = orc_adam_bias_correction(beta1, step);
    const float bc2 = orc_adam_bias_correction(beta2, step);
    const float inv_bc2 = 1.0f / bc2;
    for (size_t j = 0; j < n; j++) {
        float pj = p[j];
        float gj = g[j];
        if (weight_decay != 0.0f) {
            if (decoupled)
                pj -= lr * weight_decay * pj; /* AdamW shrink first (:157-160) */
            else
                gj += weight_decay * pj; /* L2 joins the grad (:164-166) */
        }
        m[j] = gj + beta1 * (m[j] - gj);
        float g2 = gj * gj;
        v[j] = g2 + beta2 * (v[j] - g2);
        float vh = v[j];
        if (amsgrad) {
            if (v[j] > vmax[j])
                vmax[j] = v[j];
            vh = vmax[j];
        }
        float denom = (sqrtf(vh * inv_bc2) + eps) * bc1;
        p[j] = pj - (m[j] * lr) / denom;
    }
}

float orc_grad_norm(float *const *g, const size_t *n, size_t count)
{
    /* clip.c:5-18: squares summed in f64, tensor by tensor in element
     * order; NULL grads skipped */
    double sum = 0.0;
    for (size_t i = 0; i < count; i++) {
        if (!g[i])
            continue;
        for (size_t j = 0; j < n[i]; j++) {
            double x = (double)g[i][j];
            sum += x * x;
        }
    }
    return (float)sqrt(sum);
}

float orc_clip_grad_norm(float *const *g, const size_t *n, size_t count,
                         float max_norm, float eps)
{
    /* clip.c:27-40 */
    if (!g || max_norm <= 0.0f)
        return -1.0f;
    if (eps < 0.0f)
        eps = 1e-6f;
    float total = orc_grad_norm(g, n, count);
    if (total <= max_norm)
        return total;
    /* clip.c:33-39 as the reference's build evaluates it: g*max_norm
     * times the reciprocal of (total + eps) */
    float inv = 1.0f / (total + eps);
    for (size_t i = 0; i < count; i++) {
        if (!g[i])
            continue;
        for (size_t j = 0; j < n[i]; j++)
            g[i][j] = (g[i][j] * max_norm) * inv;
    }
    return total;
}

void orc_clip_grad_value(float *const *g, const size_t *n, size_t count,
                         float clip_value)
{
    /* clip.c:49-61 */
    if (!g || clip_value <= 0.0f)
        return;
    for (size_t i = 0; i < count; i++) {
        if (!g[i])
            continue;
        for (size_t j = 0; j < n[i]; j++) {
            float x = g[i][j];
            if (x > clip_value)
                g[i][j] = clip_value;
            else if (x < -clip_value)
                g[i][j] = -clip_value;
        }
    }
}

/* ---------------- PGT1 / PGMD checkpoint bytes ---------------- */

static size_t orc_put(unsigned char *out, size_t pos, size_t cap, const void *p, size_t n)
{
    if (out && pos + n <= cap)
        memcpy(out + pos, p, n);
    return pos + n;
}

size_t orc_pgt1_write(int dtype, size_t ndim, const size_t *shape, const void *data,
                      unsigned char *out, size_t cap)
{
    /* tensor.c:607-650 for a contiguous tensor: "PGT1", u32 version 1, u32
     * dtype, u32 ndim, u64 shape[ndim], u64 numel, u64 elem_size, then the
     * elements; little-endian (x86) */
    const uint32_t ver = 1, dt = (uint32_t)dtype, nd = (uint32_t)ndim;
    uint64_t numel = 1;
    for (size_t i = 0; i < ndim; i++)
        numel *= (uint64_t)shape[i];
    const uint64_t elem = dtype == ORC_F32 ? 4 : 2;
    size_t pos = orc_put(out, 0, cap, "PGT1", 4);
    pos = orc_put(out, pos, cap, &ver, 4);
    pos = orc_put(out, pos, cap, &dt, 4);
    pos = orc_put(out, pos, cap, &nd, 4);
    for (size_t i = 0; i < ndim; i++) {
        const uint64_t d = (uint64_t)shape[i];
        pos = orc_put(out, pos, cap, &d, 8);
    }
    pos = orc_put(out, pos, cap, &numel, 8);
    pos = orc_put(out, pos, cap, &elem, 8);
    return orc_put(out, pos, cap, data, (size_t)(numel * elem));
}

size_t orc_pgt1_check(const unsigned char *buf, size_t len)
{
    /* the checks of tensor.c:655-702 in their order; returns the record's
     * length when a load would succeed, 0 when it would return NULL */
    size_t pos = 0;
    uint32_t ver, dt, nd;
    uint64_t d, numel, elem, want = 1;
    if (len < 16 || memcmp(buf, "PGT1", 4) != 0)
        return 0;
    memcpy(&ver, buf + 4, 4);
    if (ver != 1)
        return 0;
    memcpy(&dt, buf + 8, 4);
    memcpy(&nd, buf + 12, 4);
    pos = 16;
    if (nd == 0 || nd > 8)
        return 0;
    if (dt >= 3)
        return 0;
    for (uint32_t i = 0; i < nd; i++) {
        if (pos + 8 > len)
            return 0;
        memcpy(&d, buf + pos, 8);
        pos += 8;
        if (d == 0 || d > 10000000)
            return 0;
        want *= d;
    }
    if (pos + 16 > len)
        return 0;
    memcpy(&numel, buf + pos, 8);
    memcpy(&elem, buf + pos + 8, 8);
    pos += 16;
    if (numel != want)
        return 0;
    if (elem != (dt == (uint32_t)ORC_F32 ? 4u : 2u))
        return 0;
    if (len - pos < numel * elem)
        return 0;
    return pos + (size_t)(numel * elem);
}

/* ---------------- GEMM with f32 accumulation ---------------- */

typedef struct {
    int dtype, ta, tb, beta, f64;
    size_t m, n, k, lda, ldb, ldc;
    const void *a, *b;
    void *c;
    size_t r0, r1;
    const float *panels; /* f32 path: B upcast into [n/16][k][16] */
} gemm_job;

static inline float ld_elem(int dtype, const void *p, size_t idx)
{
    if (dtype == ORC_F32)
        return ((const float *)p)[idx];
    uint16_t h = ((const uint16_t *)p)[idx];
    return dtype == ORC_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

/* f32 accumulation, four rows x 16 columns at a time.  Every output is still
 * acc = 0; acc = acc + a[p]*b[p] for p = 0..k-1 in order, each product and
 * sum rounded on its own (the file is built with -ffp-contract=off and AVX2
 * has no FMA without -mfma), so the result is the serial dot product bit for
 * bit; the vectors only run 64 of those chains side by side.  B is upcast
 * once into 16-column panels [n/16][k][16] shared by all threads. */
typedef float orc_v8 __attribute__((vector_size(32)));

__attribute__((target("avx2"))) static void gemm_worker_f32(gemm_job *j, const float *panels)
{
    size_t k = j->k, npan = (j->n + 15) / 16;
    float *arows = malloc((k ? k : 1) * sizeof(float) * 4);
    for (size_t i0 = j->r0; i0 < j->r1; i0 += 4) {
        size_t ni = j->r1 - i0 < 4 ? j->r1 - i0 : 4;
        for (size_t r = 0; r < 4; r++)
            for (size_t p = 0; p < k; p++) {
                size_t i = i0 + (r < ni ? r : 0);
                size_t idx = j->ta ? p * j->lda + i : i * j->lda + p;
                arows[r * k + p] = ld_elem(j->dtype, j->a, idx);
            }
        for (size_t pj = 0; pj < npan; pj++) {
            const float *bp = panels + pj * k * 16;
            orc_v8 acc[4][2];
            memset(acc, 0, sizeof acc);
            for (size_t p = 0; p < k; p++) {
                orc_v8 b0, b1;
                memcpy(&b0, bp + p * 16, 32);
                memcpy(&b1, bp + p * 16 + 8, 32);
                for (size_t r = 0; r < 4; r++) {
                    float av = arows[r * k + p];
                    orc_v8 a8 = {av, av, av, av, av, av, av, av};
                    orc_v8 p0 = a8 * b0, p1 = a8 * b1;
                    acc[r][0] = acc[r][0] + p0;
                    acc[r][1] = acc[r][1] + p1;
                }
            }
            size_t jb = pj * 16, nj = j->n - jb < 16 ? j->n - jb : 16;
            for (size_t r = 0; r < ni; r++) {
                float out[16];
                memcpy(out, acc[r], sizeof out);
                float *cp = (float *)j->c + (i0 + r) * j->ldc + jb;
                for (size_t q = 0; q < nj; q++)
                    cp[q] = j->beta ? cp[q] + out[q] : out[q];
            }
        }
    }
    free(arows);
}

static void *gemm_worker(void *arg)
{
    gemm_job *j = arg;
    if (!j->f64) {
        gemm_worker_f32(j, j->panels);
        return NULL;
    }
    float *arow = malloc(j->k * sizeof(float));
    float *bcol = malloc(j->k * sizeof(float) * 16);
    for (size_t jb = 0; jb < j->n; jb += 16) {
        size_t nj = j->n - jb < 16 ? j->n - jb : 16;
        /* gather 16 columns of B, upcast once */
        for (size_t q = 0; q < nj; q++)
            for (size_t p = 0; p < j->k; p++) {
                size_t idx = j->tb ? (jb + q) * j->ldb + p : p * j->ldb + jb + q;
                bcol[q * j->k + p] = ld_elem(j->dtype, j->b, idx);
            }
        for (size_t i = j->r0; i < j->r1; i++) {
            for (size_t p = 0; p < j->k; p++) {
                size_t idx = j->ta ? p * j->lda + i : i * j->lda + p;
                arow[p] = ld_elem(j->dtype, j->a, idx);
            }
            for (size_t q = 0; q < nj; q++) {
                const float *bc = bcol + q * j->k;
                if (j->f64) {
                    double acc = 0.0;
                    for (size_t p = 0; p < j->k; p++)
                        acc += (double)arow[p] * (double)bc[p];
                    ((double *)j->c)[i * j->ldc + jb + q] = acc;
                } else {
                    float acc = 0.0f;
                    for (size_t p = 0; p < j->k; p++)
                        acc += arow[p] * bc[p];
                    float *cp = (float *)j->c + i * j->ldc + jb + q;
                    *cp = j->beta ? *cp + acc : acc;
                }
            }
        }
    }
    free(arow);
    free(bcol);
    return NULL;
}

static void gemm_run(int dtype, int ta, int tb, size_t m, size_t n, size_t k,
                     const void *a, size_t lda, const void *b, size_t ldb,
                     void *c, size_t ldc, int beta, int f64, int nthreads)
{
    if (nthreads < 1)
        nthreads = 1;
    if ((size_t)nthreads > m)
        nthreads = m ? (int)m : 1;
    gemm_job *jobs = calloc((size_t)nthreads, sizeof(gemm_job));
    pthread_t *th = calloc((size_t)nthreads, sizeof(pthread_t));
    size_t per = (m + (size_t)nthreads - 1) / (size_t)nthreads;
    float *panels = NULL;
    if (!f64) {
        size_t npan = (n + 15) / 16;
        size_t nf = npan * k * 16;
        panels = malloc((nf ? nf : 1) * sizeof(float));
        for (size_t pj = 0; pj < npan; pj++)
            for (size_t p = 0; p < k; p++)
                for (size_t q = 0; q < 16; q++) {
                    size_t col = pj * 16 + q;
                    size_t idx = tb ? col * ldb + p : p * ldb + col;
                    panels[(pj * k + p) * 16 + q] = col < n ? ld_elem(dtype, b, idx) : 0.0f;
                }
    }
    for (int t = 0; t < nthreads; t++) {
        gemm_job *j = &jobs[t];
        j->dtype = dtype; j->ta = ta; j->tb = tb; j->beta = beta; j->f64 = f64;
        j->m = m; j->n = n; j->k = k; j->lda = lda; j->ldb = ldb; j->ldc = ldc;
        j->a = a; j->b = b; j->c = c; j->panels = panels;
        j->r0 = (size_t)t * per < m ? (size_t)t * per : m;
        j->r1 = j->r0 + per < m ? j->r0 + per : m;
    }
    for (int t = 1; t < nthreads; t++)
        pthread_create(&th[t], NULL, gemm_worker, &jobs[t]);
    gemm_worker(&jobs[0]);
    for (int t = 1; t < nthreads; t++)
        pthread_join(th[t], NULL);
    free(panels);
    free(jobs);
    free(th);
}

void orc_gemm_acc32(int dtype, int ta, int tb, size_t m, size_t n, size_t k,
                    const void *a, size_t lda, const void *b, size_t ldb,
                    float *c, size_t ldc, int beta, int nthreads)
{
    gemm_run(dtype, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, beta, 0, nthreads);
}

void orc_gemm_acc64(int dtype, int ta, int tb, size_t m, size_t n, size_t k,
                    const void *a, size_t lda, const void *b, size_t ldb,
                    double *c, size_t ldc, int nthreads)
{
    gemm_run(dtype, ta, tb, m, n, k, a, lda, b, ldb, c, ldc, 0, 1, nthreads);
}

/* ---------------- elementwise chains ---------------- */

float orc_sigmoid(float x)
{
    /* activations.c:149-160 / jit.c:334 */
    return 1.0f / (1.0f + expf(-x));
}

float orc_gelu(float x)
{
    /* exact erf form, activations.c:166-173 */
    return 0.5f * x * (1.0f + erff(x * 0.70710678118f));
}

static float gelu_grad(float x)
{
    /* grad_gelu, autograd.c:794-801 */
    const float sqrt_2pi = 2.50662827463f;
    const float inv_sqrt2 = 0.70710678118f;
    float erf_term = erff(x * inv_sqrt2);
    float phi = expf(-0.5f * x * x) / sqrt_2pi;
    return 0.5f * (1.0f + erf_term) + x * phi;
}

void orc_gelu_backward(const float *z, const float *g, float *out, size_t n)
{
    /* bwd_unary_elemwise with grad_gelu (autograd.c:519-559, :794-801):
     * out = g * gelu'(z) */
    for (size_t i = 0; i < n; i++)
        out[i] = g[i] * gelu_grad(z[i]);
}

void orc_chain1_backward(const float *a, const float *b, const float *c,
                         size_t n, float *da, float *db, float *dc)
{
    /* forward: t0 = a+b, t1 = t0*c, t2 = relu(t1), t3 = tanh(t2);
     * upstream of t3 is the sum_all scale 1.  Local grads as the JIT suffix
     * emits them: tanh' = 1 - tanh(x)^2 recomputed from the input
     * (autograd.c:2260-2267), relu' = step(x) (:2244-2249), mul' = other
     * operand (:2189-2194), add' = 1 (:2176). */
    for (size_t i = 0; i < n; i++) {
        float t0 = a[i] + b[i];
        float t1 = t0 * c[i];
        float t2 = t1 > 0.0f ? t1 : 0.0f;
        float th = tanhf(t2);
        float g2 = 1.0f * (1.0f - th * th);
        float g1 = g2 * (t1 > 0.0f ? 1.0f : 0.0f);
        float g0 = g1 * c[i];
        dc[i] = g1 * t0;
        da[i] = g0;
        db[i] = g0;
    }
}

void orc_chain2_backward(const float *x, const float *bias, const float *g,
                         size_t R, size_t C, float *dx, float *dg,
                         float *dbias, double *dbias64)
{
    /* forward: t0 = x+bias, t1 = gelu(t0), t2 = sigmoid(g), y = t1*t2.
     * dL/dt1 = t2, dL/dt2 = t1, dg = dt2 * s(1-s), dt0 = dt1 * gelu'(t0),
     * dx = dt0, dbias[c] = sum over rows of dt0 (row order, f32). */
    for (size_t c = 0; c < C; c++) {
        dbias[c] = 0.0f;
        if (dbias64)
            dbias64[c] = 0.0;
    }
    for (size_t r = 0; r < R; r++) {
        for (size_t c = 0; c < C; c++) {
            size_t i = r * C + c;
            float t0 = x[i] + bias[c];
            float t1 = orc_gelu(t0);
            float s = orc_sigmoid(g[i]);
            float dt1 = 1.0f * s;
            float dt2 = 1.0f * t1;
            dg[i] = dt2 * (s * (1.0f - s));
            float dt0 = dt1 * gelu_grad(t0);
            dx[i] = dt0;
            dbias[c] += dt0;
            if (dbias64)
                dbias64[c] += (double)dt0;
        }
    }
}

float orc_mse_grad_scale(size_t ndim, const size_t *shape, bool mean)
{
    if (!mean || ndim == 0)
        return 2.0f;
    return 2.0f * (1.0f / (float)shape[ndim - 1]);
}

/* ---------------- config-5 MLP training step ---------------- */

void orc_mlp_step(int dtype, size_t L, const size_t *dims, size_t batch,
                  const float *x, const float *target, float *const *W,
                  float *const *b, float *const *Wbuf, float *const *bbuf,
                  float *const *dW, float *const *db, float lr,
                  float momentum, float dampening, float weight_decay,
                  bool nesterov, float *loss, int nthreads)
{
    /* forward (nn.c:117-125 per layer: matmul then broadcast bias add;
     * gelu activations.c:166-173 between layers):
     *   z_l = q(h_{l-1}) . q(W_l) + b_l,  h_l = gelu(z_l),  out = z_L
     * q rounds to dtype (identity for ORC_F32); products accumulate in f32. */
    size_t B = batch, maxd = 0;
    for (size_t l = 0; l <= L; l++)
        if (dims[l] > maxd)
            maxd = dims[l];
    float **z = calloc(L + 1, sizeof *z), **h = calloc(L + 1, sizeof *h);
    float *qw = malloc(maxd * maxd * sizeof(float));
    float *qh = malloc(B * maxd * sizeof(float));
    float *g = malloc(B * maxd * sizeof(float));
    float *gprev = malloc(B * maxd * sizeof(float));
    for (size_t l = 1; l <= L; l++) {
        z[l] = malloc(B * dims[l] * sizeof(float));
        h[l] = malloc(B * dims[l] * sizeof(float));
    }
    h[0] = (float *)x;
    for (size_t l = 1; l <= L; l++) {
        size_t K = dims[l - 1], N = dims[l];
        memcpy(qh, h[l - 1], B * K * sizeof(float));
        orc_round_f32(dtype, qh, B * K);
        memcpy(qw, W[l - 1], K * N * sizeof(float));
        orc_round_f32(dtype, qw, K * N);
        orc_gemm_acc32(ORC_F32, 0, 0, B, N, K, qh, K, qw, N, z[l], N, 0, nthreads);
        for (size_t i = 0; i < B; i++)
            for (size_t j = 0; j < N; j++) {
                z[l][i * N + j] += b[l - 1][j];
                h[l][i * N + j] = orc_gelu(z[l][i * N + j]);
            }
    }
    /* loss = mean_all((out - t)^2): sum over rows, then the mean over the
     * last axis (autograd.c:1018-1043, :1758-1771) */
    size_t NL = dims[L];
    double acc = 0.0;
    for (size_t i = 0; i < B * NL; i++) {
        double d = (double)z[L][i] - (double)target[i];
        acc += d * d;
    }
    *loss = (float)(acc / (double)NL);
    /* d(loss)/d(out): the fused suffix hands g = 1/NL to mul(d, d), whose
     * two operand grads g*d add up (autograd.c:2166-2297, :2289-2295) */
    const float scale = 1.0f / (float)NL;
    for (size_t i = 0; i < B * NL; i++) {
        float d = z[L][i] - target[i];
        g[i] = scale * d + scale * d;
    }
    for (size_t l = L; l >= 1; l--) {
        size_t K = dims[l - 1], N = dims[l];
        /* g = dL/dz_l.  Bias grad: rows summed in order (autograd.c:364-387) */
        for (size_t j = 0; j < N; j++)
            db[l - 1][j] = 0.0f;
        for (size_t i = 0; i < B; i++)
            for (size_t j = 0; j < N; j++)
                db[l - 1][j] += g[i * N + j];
        /* GEMM grads of the matmul (autograd.c:561-706) on rounded operands:
         * dW = q(h_{l-1})^T . q(g),  dh_{l-1} = q(g) . q(W_l)^T */
        float *qg = malloc(B * N * sizeof(float));
        memcpy(qg, g, B * N * sizeof(float));
        orc_round_f32(dtype, qg, B * N);
        memcpy(qh, h[l - 1], B * K * sizeof(float));
        orc_round_f32(dtype, qh, B * K);
        orc_gemm_acc32(ORC_F32, 1, 0, K, N, B, qh, K, qg, N, dW[l - 1], N, 0, nthreads);
        if (l > 1) {
            memcpy(qw, W[l - 1], K * N * sizeof(float));
            orc_round_f32(dtype, qw, K * N);
            orc_gemm_acc32(ORC_F32, 0, 1, B, K, N, qg, N, qw, N, gprev, K, 0, nthreads);
            /* through gelu (grad_gelu, autograd.c:794-801) */
            for (size_t i = 0; i < B * K; i++)
                g[i] = gprev[i] * gelu_grad(z[l - 1][i]);
        }
        free(qg);
    }
    /* one SGD step per parameter, W_l then b_l (sgd.c:111-162) */
    for (size_t l = 1; l <= L; l++) {
        size_t K = dims[l - 1], N = dims[l];
        orc_sgd_step(W[l - 1], dW[l - 1], Wbuf[l - 1], K * N, lr, momentum,
                     dampening, weight_decay, nesterov);
        orc_sgd_step(b[l - 1], db[l - 1], bbuf[l - 1], N, lr, momentum,
                     dampening, weight_decay, nesterov);
    }
    for (size_t l = 1; l <= L; l++) {
        free(z[l]);
        free(h[l]);
    }
    free(z);
    free(h);
    free(qw);
    free(qh);
    free(g);
    free(gprev);
}
