/*
 * GEMM entry points of the reference's backend/backend.h:118-136, with
 * device pointers.  Contract kept: row-major, leading dimensions in
 * elements, C overwritten (beta = 0), A and B as uint16_t for F16/BF16, C
 * f32 accumulated in f32.  a, b and c are device addresses (for example
 * pg_tensor.dev); the call is enqueued on the library stream.
 * pg_gemm (f32 x f32) is also device-side.
 */
#ifndef PICOGRAD_BACKEND_H
#define PICOGRAD_BACKEND_H

#include <stddef.h>
#include <stdint.h>

#include "dtype.h"

#ifdef __cplusplus
extern "C" {
#endif

void pg_gemm(size_t m, size_t n, size_t k, const float *a, size_t lda, const float *b, size_t ldb,
             float *c, size_t ldc);
void pg_gemm_ex(pg_dtype dtype, size_t m, size_t n, size_t k, const void *a, size_t lda,
                const void *b, size_t ldb, float *c, size_t ldc);
void pg_hgemm(size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, const uint16_t *b,
              size_t ldb, float *c, size_t ldc);
void pg_bgemm(size_t m, size_t n, size_t k, const uint16_t *a, size_t lda, const uint16_t *b,
              size_t ldb, float *c, size_t ldc);

/* pg_gemm_ex that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * contract, kernels and result bits as pg_gemm_ex; the buffers those need
 * (zero-padded operand copies, split-K partials, k-tail slabs) come from a
 * fixed 32 MiB workspace that each device holds for the life of the
 * process, instead of the library allocator.  A call whose buffers exceed
 * it is rejected.  Calls share the workspace: they are ordered on the
 * library stream, and calls overlapping on one device from two host
 * threads would race.  Work other calls left waiting to be queued (batched
 * uploads, deferred elementwise ops: queueing them may compile, allocate or
 * wait) makes the call fail instead; pg_amd_sync() queues it.  Returns 0,
 * or -1 with pg_amd_last_error() set (library not initialised by
 * pg_amd_init, such work pending, bad arguments, workspace too small,
 * launch failure). */
int pg_amd_gemm_ex_noalloc(pg_dtype dtype, size_t m, size_t n, size_t k, const void *a, size_t lda,
                           const void *b, size_t ldb, float *c, size_t ldc);

#ifdef __cplusplus
}
#endif

#endif
