/*
 * CPU oracle for the picograd backward path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C11 restatement of the reference CPU algorithms this build
 * replaces on the GPU.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker: the product library
 * (picograd_amd/) never links, calls or falls back to anything here.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the reference checkout).  How each one is pinned:
 *   orc_seed/orc_uniform/orc_normal   golden RNG streams from the compiled
 *                                     reference (tests/golden) -- bit-exact
 *   orc_f32_to_bf16 ... orc_f16_to_f32 exhaustive 2^16 decode + special
 *                                     values + random sample vs the
 *                                     reference's convert.h built as a shim
 *   orc_sgd_step                      test_opt.c:48-138 known answers and
 *                                     golden multi-step trajectories
 *   orc_gemm_acc32                    f64 brute force, ragged shapes, and the
 *                                     reference pg_gemm_ex (bgemm/hgemm)
 *   orc_chain1_backward               golden C1 grads (JIT on and off)
 *   orc_chain2_backward               golden C2 grads at a reduced shape
 *   orc_mse_grad_scale                golden mse/mean_all graphs
 *   orc_adam_step                     golden six-step trajectories of the
 *                                     reference (five configurations): bit
 *                                     for bit on the elements its build
 *                                     computes with IEEE sqrt/divide, within
 *                                     2^-21 of the update elsewhere (its x86
 *                                     reciprocal estimates); closed forms
 *                                     (test_training.c:237-268)
 *   orc_grad_norm, orc_clip_*         golden clip fixtures bit for bit;
 *                                     closed forms
 *   orc_pgt1_write, orc_pgt1_check    files written by the reference's
 *                                     pg_tensor_save / pg_module_save byte
 *                                     for byte; its loader's verdict on 14
 *                                     crafted headers
 *   orc_mlp_step                      golden two-step f32 MLP training run
 *                                     of the reference (ORC_F32); the 16-bit
 *                                     modes differ only by orc_round_f32 on
 *                                     the GEMM operands, pinned above
 * No function here is "parity unpinned".
 */
#ifndef PG_ORACLE_H
#define PG_ORACLE_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2 };

/* RNG: splitmix64 stream (tensor.c:289-339). */
void orc_seed(unsigned long long seed);
void orc_uniform(float *out, size_t n, float low, float high);
void orc_normal(float *out, size_t n, float mean, float stddev);

/* RNE conversions (convert.h:15-104). */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_cast_f32(int dtype, const float *src, uint16_t *dst, size_t n);
void orc_round_f32(int dtype, float *x, size_t n); /* x = f32(dtype(x)) */

/* SGD (sgd.c:111-162): one step over one parameter tensor. */
void orc_sgd_step(float *p, const float *g, float *buf, size_t n, float lr,
                  float momentum, float dampening, float weight_decay,
                  bool nesterov);

/*
 * Adam / AdamW (adam.c:113-181): one step over one parameter tensor.  `step`
 * is the optimiser's counter after its increment (1 on the first step); m, v
 * (and vmax when amsgrad) start at zero.  lr and weight_decay are the values
 * in force for this tensor (the per-parameter overrides of :136-138 already
 * resolved by the caller).  Evaluated in the order the reference's
 * -ffast-math build uses: m = g + b1*(m - g), v = g^2 + b2*(v - g^2),
 * p -= (m*lr) / ((sqrt(v * (1/bc2)) + eps) * bc1), IEEE sqrt and divide.
 */
float orc_adam_bias_correction(float beta, unsigned long long step);
void orc_adam_step(float *p, const float *g, float *m, float *v, float *vmax,
                   size_t n, float lr, float beta1, float beta2, float eps,
                   float weight_decay, bool amsgrad, bool decoupled,
                   unsigned long long step);

/* Gradient clipping over `count` grads g[i] of n[i] elements (NULL skipped):
 * global L2 norm (clip.c:5-18), clip by norm (:27-40, returns the norm
 * before clipping, -1 on bad arguments; scaled as (g*max_norm) *
 * (1/(norm + eps)), the reference build's order), clip by value (:49-61). */
float orc_grad_norm(float *const *g, const size_t *n, size_t count);
float orc_clip_grad_norm(float *const *g, const size_t *n, size_t count,
                         float max_norm, float eps);
void orc_clip_grad_value(float *const *g, const size_t *n, size_t count,
                         float clip_value);

/*
 * Checkpoint bytes.  orc_pgt1_write lays out one tensor as the reference's
 * pg_tensor_save_fp does (tensor.c:607-650) into out (when cap allows) and
 * returns the record's size.  orc_pgt1_check applies pg_tensor_load_fp's
 * checks (tensor.c:655-702) and returns the record's size if a load would
 * succeed, else 0.  dtype: ORC_F32 / ORC_F16 / ORC_BF16 (the reference's
 * pg_dtype values 0 / 1 / 2).
 */
size_t orc_pgt1_write(int dtype, size_t ndim, const size_t *shape, const void *data,
                      unsigned char *out, size_t cap);
size_t orc_pgt1_check(const unsigned char *buf, size_t len);

/*
 * C[i,j] (+)= sum_p A(i,p) * B(p,j), every product formed from f32 values
 * (16-bit operands upcast first) and accumulated in f32 in p order.
 * A(i,p) = ta ? a[p*lda+i] : a[i*lda+p];  B(p,j) = tb ? b[j*ldb+p] : b[p*ldb+j].
 * dtype selects how a and b are read (ORC_F32: float*, else uint16_t*).
 * beta 0 overwrites C, 1 adds into it.  Threads over rows of C.
 * Restates the f32-accumulate contract of pg_cpu_gemm_ex (gemm.c:575-629)
 * and the dgrad/wgrad products of bwd_matmul (autograd.c:655-692).
 */
void orc_gemm_acc32(int dtype, int ta, int tb, size_t m, size_t n, size_t k,
                    const void *a, size_t lda, const void *b, size_t ldb,
                    float *c, size_t ldc, int beta, int nthreads);
/* Same product accumulated in f64 (the error yardstick). */
void orc_gemm_acc64(int dtype, int ta, int tb, size_t m, size_t n, size_t k,
                    const void *a, size_t lda, const void *b, size_t ldb,
                    double *c, size_t ldc, int nthreads);

/* out = g * gelu'(z), the eager GELU backward (autograd.c:519-559, :794-801) */
void orc_gelu_backward(const float *z, const float *g, float *out, size_t n);

/*
 * Config-1 chain: loss = sum_all(tanh(relu((a+b)*c))), flat n elements.
 * Writes dL/da, dL/db, dL/dc (autograd.c:2166-2297 chain rule as the JIT
 * suffix applies it; autograd.c:519-559 for the eager local grads).
 */
void orc_chain1_backward(const float *a, const float *b, const float *c,
                         size_t n, float *da, float *db, float *dc);

/*
 * Config-2 chain: loss = sum_all(gelu(x + bias) * sigmoid(g)), x,g [R,C],
 * bias [C].  dx, dg [R,C]; dbias [C] summed over rows in row order in f32
 * (autograd.c:364-387), dbias64 (optional) the same sum in f64.
 * GELU' follows grad_gelu (autograd.c:794-801), sigmoid' the JIT form
 * s*(1-s) (autograd.c:2251-2258).
 */
void orc_chain2_backward(const float *x, const float *bias, const float *g,
                         size_t R, size_t C, float *dx, float *dg,
                         float *dbias, double *dbias64);

/* Forward values used by the chains (activations.c:113-173). */
float orc_gelu(float x);
float orc_sigmoid(float x);

/*
 * Config-5 training step of an L-layer MLP, in place.  dims[0..L] are the
 * layer widths, W[l] [dims[l], dims[l+1]] and b[l] [dims[l+1]] the f32
 * master parameters, Wbuf/bbuf their momentum buffers (zeros before the
 * first step), x [batch, dims[0]], target [batch, dims[L]].
 *   forward   z_l = q(h_{l-1}).q(W_l) + b_l, h_l = gelu(z_l), out = z_L
 *             (nn.c:117-125 linear, activations.c:166-173 gelu)
 *   loss      mse(out, target, mean) (autograd.c:1758-1771, mean over the
 *             last axis only)
 *   backward  bias grads row-ordered sums (autograd.c:364-387); dW =
 *             q(h)^T.q(g), dh = q(g).q(W)^T (autograd.c:561-706); gelu'
 *             (autograd.c:794-801); no grad for x
 *   update    orc_sgd_step per parameter, W_l then b_l (sgd.c:111-162)
 * q rounds to dtype (RNE), the identity for ORC_F32 -- where this is the
 * reference's own f32 step, pinned by a golden run of the reference.
 * dW/db receive the grads; *loss the forward loss before the update.
 */
void orc_mlp_step(int dtype, size_t L, const size_t *dims, size_t batch,
                  const float *x, const float *target, float *const *W,
                  float *const *b, float *const *Wbuf, float *const *bbuf,
                  float *const *dW, float *const *db, float lr,
                  float momentum, float dampening, float weight_decay,
                  bool nesterov, float *loss, int nthreads);

/*
 * Upstream-grad scale that pg_ag_mse(pred, tgt, mean) hands to d = pred-tgt:
 * 2 * (mean ? 1/shape[ndim-1] : 1)   (autograd.c:1018-1043, :1758-1771;
 * reduce_all only divides by the last remaining axis).
 */
float orc_mse_grad_scale(size_t ndim, const size_t *shape, bool mean);

#ifdef __cplusplus
}
#endif

#endif
