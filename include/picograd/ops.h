/*
 * Tensor-level forward ops: the reference's ops/elementwise.h:6-19,
 * ops/activations.h:6-12 and ops/matmul.h:6-10, same names and signatures,
 * over device tensors.  Each returns a new f32 tensor (caller frees it with
 * pg_tensor_free) computed on the device and queued on the library stream,
 * or NULL on bad input, with the reason in pg_autograd_last_error().
 *
 * Values equal the corresponding pg_ag_* op's bit for bit (the same
 * kernels).  Binary ops broadcast as the reference does (ops/common.h:6-54);
 * pg_matmul follows matmul.c:186-284 (one dtype on both sides, 1-D
 * operands as vectors, batch dims, f32 out; f16/bf16 on the MFMA units with
 * f32 accumulation), pg_bmm matmul.c:340-369.  Strided views are read in
 * row-major order.  pg_pow, pg_softmax, pg_log_softmax, pg_addmm and
 * pg_tensordot are outside the backward path this library rebuilds: they
 * return NULL with that reason.
 */
#ifndef PICOGRAD_OPS_H
#define PICOGRAD_OPS_H

#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ops/elementwise.h:6-19 */
pg_tensor *pg_add(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_sub(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_mul(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_div(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_pow(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_neg(const pg_tensor *a);
pg_tensor *pg_abs(const pg_tensor *a);
pg_tensor *pg_sqrt(const pg_tensor *a);
pg_tensor *pg_clamp(const pg_tensor *a, float lo, float hi);
pg_tensor *pg_exp(const pg_tensor *a);
pg_tensor *pg_log(const pg_tensor *a);
pg_tensor *pg_sin(const pg_tensor *a);
pg_tensor *pg_cos(const pg_tensor *a);
pg_tensor *pg_erf(const pg_tensor *a);

/* ops/activations.h:6-12 */
pg_tensor *pg_relu(const pg_tensor *a);
pg_tensor *pg_leaky_relu(const pg_tensor *a, float alpha);
pg_tensor *pg_sigmoid(const pg_tensor *a);
pg_tensor *pg_tanh(const pg_tensor *a);
pg_tensor *pg_gelu(const pg_tensor *a);
pg_tensor *pg_softmax(const pg_tensor *t, size_t axis);
pg_tensor *pg_log_softmax(const pg_tensor *t, size_t axis);

/* ops/matmul.h:6-10 */
pg_tensor *pg_matmul(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_bmm(const pg_tensor *a, const pg_tensor *b);
pg_tensor *pg_addmm(const pg_tensor *input, const pg_tensor *m1, const pg_tensor *m2,
                    float alpha, float beta);
pg_tensor *pg_tensordot(const pg_tensor *a, const pg_tensor *b,
                        size_t ndims, const size_t *axes_a, const size_t *axes_b);

#ifdef __cplusplus
}
#endif

#endif
