/*
 * MI355X-specific entry points of picograd-amd.  None has a counterpart in
 * the reference; they expose what a device-resident backend adds: the
 * stream all work is queued on, explicit synchronisation, allocator state
 * and backward seeded with an explicit upstream gradient.
 */
#ifndef PICOGRAD_AMD_H
#define PICOGRAD_AMD_H

#include <stdbool.h>
#include <stddef.h>
#include <stdio.h>

#include "adam.h"
#include "autograd.h"
#include "sgd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Selects the device and creates the library stream.  Idempotent; every
 * other entry point calls it.  Returns 0 on success. */
int pg_amd_init(void);
/* The hipStream_t (as void*) every kernel of the library is launched on. */
void *pg_amd_stream(void);
/* Waits for all queued work.  Returns 0 on success. */
int pg_amd_sync(void);
/* Last device-layer error message ("" if none). */
const char *pg_amd_last_error(void);
/* Bytes held by live tensors / kept in the allocator's free lists. */
size_t pg_amd_bytes_in_use(void);
size_t pg_amd_bytes_cached(void);
/* Returns cached device blocks to the driver (waits for the stream). */
void pg_amd_release_cached(void);

/* pg_backward() with the root's upstream gradient given explicitly instead
 * of 1 (like torch's backward(gradient)).  seed must have the root value's
 * shape, f32; it is read, not kept, and must stay valid until the stream has
 * run the backward.  The fused loss-suffix JIT does not apply here. */
void pg_amd_backward_from(pg_node *root, const pg_tensor *seed);

/* Mixed-precision matmul of f32 nodes, A [M, K] . B [K, N] -> f32 [M, N],
 * computed on the MFMA units: both operands are rounded to `dtype`
 * (PG_DTYPE_BF16 or PG_DTYPE_F16, round to nearest even) and the products
 * accumulated in f32.  Backward rounds the upstream grad the same way and
 * accumulates f32 grads into both operands: dA += q(dC).q(B)^T,
 * dB += q(A)^T.q(dC).  The rounded copy of each operand is kept with its
 * storage and reused until the tensor is written again; pg_sgd_step
 * rewrites it for a parameter in the same pass as the update, so the GEMMs
 * of a bf16-weight layer read bf16 weights without a cast per step.
 * Returns NULL (pg_autograd_last_error) for other dtypes or shapes.
 * The reference's matmul requires one dtype on both sides
 * (ops/matmul.c:191) and has no cast op, so it has no counterpart. */
pg_node *pg_amd_ag_matmul16(pg_node *a, pg_node *b, pg_dtype dtype);

/* Tells the library that t's device elements were written behind its back
 * (through t->dev by pg_gemm/pg_gemm_ex or the caller's own kernels), so a
 * kept 16-bit copy is remade before its next use.  Writes through the
 * library's own calls (ops, pg_tensor_fill/copy_from/copy_from_host/
 * sync_device, pg_jit_run outputs, pg_sgd_step) are tracked already. */
void pg_amd_tensor_modified(pg_tensor *t);

/* A new tensor of t's elements converted to `dtype` on the device: f32 to
 * f16/bf16 rounds to nearest even with the bit rules of the reference's
 * core/convert.h:15-104 (f16 subnormals IEEE-correct), 16-bit to f32 is
 * exact, equal dtypes copy.  The device form of convert.h:106-152's batch
 * converters, which the reference exposes only as inline host functions.
 * NULL (pg_amd_last_error) on failure. */
pg_tensor *pg_amd_tensor_to_dtype(const pg_tensor *t, pg_dtype dtype);

/* Remakes t's kept 16-bit copy now if it has one that a write made stale
 * (the next GEMM would otherwise remake it on first use).  Enqueued on the
 * library stream; false on a device error.  No counterpart in the
 * reference, which keeps no such copies. */
bool pg_amd_tensor_refresh16(pg_tensor *t);

/* Activation codes of pg_amd_ag_linear16: the reference's PG_ACT_* values
 * (backend/cpu/gemm.h:37-39). */
#ifndef PG_ACT_NONE
#define PG_ACT_NONE 0
#define PG_ACT_RELU 1
#define PG_ACT_GELU 2
#endif

/* Linear layer out = act(q(x).q(W) + b) with x [M, K], W [K, N], b [N]
 * (or NULL), all f32 nodes, q and the f32 accumulation as in
 * pg_amd_ag_matmul16, act one of PG_ACT_*.  One MFMA GEMM computes it: its
 * epilogue adds the bias, applies the activation, keeps the pre-activation
 * for the backward and writes out's 16-bit copy for the next layer.
 * Backward: dz = dout * act'(pre-activation) (GELU' and ReLU' as
 * pg_ag_gelu / pg_ag_relu), db += column sums of dz, dx += q(dz).q(W)^T,
 * dW += q(x)^T.q(dz) -- the grads of matmul16 + add + act, in fewer passes.
 * The reference computes this forward in pg_cpu_gemm_fused
 * (backend/cpu/gemm.c:685-726, the fused path of nn.c:46-90) without an
 * autograd form; it has no counterpart in the autograd ABI.
 * Returns NULL (pg_autograd_last_error) for bad shapes, dtype or act. */
pg_node *pg_amd_ag_linear16(pg_node *x, pg_node *w, pg_node *b, int act, pg_dtype dtype);

/* Read access to what a linear16 node's backward works from, for checking
 * the fused activation backward against a CPU model (no counterpart in the
 * reference, whose fused GEMM has no backward):
 *  - pg_amd_linear16_preact: the kept pre-activation z = q(x).q(W) + b
 *    (f32 [M, N]), or NULL for act PG_ACT_NONE or a node built without
 *    grads.  Borrowed: valid while the node lives.
 *  - pg_amd_linear16_keep_dz(true): from then on each linear16 backward
 *    keeps the 16-bit dz it computed, q(dout * act'(z)) as [M, N8] with
 *    N8 = N rounded up to 8 (zero columns past N), on its node, replacing
 *    the previous one, instead of freeing it (costs M * N8 * 2 bytes per
 *    node until the node is freed).  pg_amd_linear16_dz returns it
 *    (borrowed; PG_DTYPE_BF16 or F16 bits), or NULL. */
const pg_tensor *pg_amd_linear16_preact(const pg_node *n);
void pg_amd_linear16_keep_dz(bool keep);
const pg_tensor *pg_amd_linear16_dz(const pg_node *n);

/* Narrow dgrads of linear16 layers (no counterpart in the reference).  The
 * dgrad dx = q(dz).q(W)^T of a layer with at most 16 outputs, written into a
 * grad with no earlier contribution, is formed by a pass that runs the
 * GEMM's own MFMA sequence per 32 x 32 tile (so dx has the GEMM's bits)
 * and writes dx once.  When x comes from another linear16 node, that
 * node's backward forms it in its own activation pass (reading z and the
 * narrow operands, writing dx and its dz) instead of reading back a
 * written dx; any other reader of dx before then forms it first.
 * pg_amd_linear16_narrow(false) turns both off (the GEMM launch, then
 * the activation pass reading dx); on by default. */
void pg_amd_linear16_narrow(bool on);

/* The 16-bit operand copies of matmul16 (pg_amd_ag_matmul16) written by the
 * fused elementwise kernels beside their f32 outputs, in place of a cast
 * pass over them: a deferred forward run whose output a matmul16 takes as
 * its operand (b = gelu(x + bias); matmul16(b, W)), and a fused backward
 * region that writes a matmul16 node's grad whole.  Each copy is rounded as
 * the cast kernel rounds, so every result is the same bit for bit either
 * way.  pg_amd_jit_copies16(false) turns both off (the cast pass runs);
 * on by default. */
void pg_amd_jit_copies16(bool on);

/* JIT compile statistics: programs compiled by hiprtc, and cache lookups
 * that found a loaded kernel. */
size_t pg_amd_jit_compiles(void);
size_t pg_amd_jit_cache_hits(void);

/* The launch plan of a 16-bit MFMA GEMM C[m, n] over a reduction of k
 * (batch entries of it), as the library's GEMM paths choose it (a
 * measurement and test aid): returns the tile (1: 128 x 128, four waves;
 * 2: 256 x 256, eight waves; 3: 128 x 256, eight waves; 4: the skinny
 * kernel for n <= 16 with B MN-contiguous and at least 1009 rows, 16 rows
 * of C per block, one launch with no split), stores the
 * split-K factor (1 = none) in *splits and the planner's time estimate in
 * seconds in *seconds (either may be NULL).  cu_budget: the CUs the launch
 * may occupy when it shares the chip with another (a matmul's dgrad and
 * wgrad run side by side when each alone leaves CUs idle), 0 for all.
 * ta = 1: A is MN-contiguous (A^T stored), tb = 1: B is MN-contiguous; only
 * a k that is not a multiple of 8 with a K-contiguous operand changes the
 * plan. */
int pg_amd_gemm16_plan(int ta, int tb, size_t m, size_t n, size_t k, size_t batch, int cu_budget, int *splits,
                       double *seconds);

/* Attainable bf16 MFMA rate of this device in TFLOP/s (a measurement aid
 * for rooflines): one block of eight waves per CU issues back-to-back
 * v_mfma_f32_32x32x16_bf16 on pseudo-random bf16 operands, from registers
 * (lds = 0) or read from LDS one k-step ahead like the GEMM (lds = 1).
 * Waits for the stream.  Returns a negative value on failure. */
double pg_amd_mfma_probe(int lds);

/* ---- checkpoints of device parameters and optimiser state ----
 * Parameter lists in the reference's module checkpoint format (PGMD,
 * nn/module.c:88-185: "PGMD", u32 version 1, u64 count, then one PGT1
 * record per parameter value), so a file saved here loads with the
 * reference's pg_module_load / pg_module_load_into and the reverse: the
 * reference's pg_module has no device counterpart here, so the list is
 * passed as nodes (pg_module_params order).  load_into copies each record
 * into the matching node's value on the device; a count, dtype or shape
 * mismatch returns false (records before it are already loaded, as in the
 * reference). */
bool pg_amd_params_save(pg_node *const *params, size_t n, const char *path);
bool pg_amd_params_save_fp(pg_node *const *params, size_t n, FILE *fp);
bool pg_amd_params_load_into(pg_node *const *params, size_t n, const char *path);
bool pg_amd_params_load_into_fp(pg_node *const *params, size_t n, FILE *fp);

/* The momentum buffer of the optimiser's i-th parameter (registration
 * order), owned by the optimiser; NULL before the first pg_sgd_step that
 * updated it, without momentum, or for i out of range.  The reference keeps
 * the buffers private (opt/sgd.c:6-16); callers that save, restore or reset
 * optimiser state on the device read them here. */
pg_tensor *pg_amd_sgd_buffer(pg_sgd *opt, size_t i);

/* Optimiser state, which the reference cannot checkpoint (its SGD momentum
 * and Adam moments live only in memory; adam.h:42-44 lets a caller restore
 * the step counter alone).  Formats, built from PGT1 records:
 *   SGD   "PGSG", u32 version 1, u64 nparams, per parameter u32 has_buf (0
 *         or 1) then the momentum buffer's PGT1 record when has_buf;
 *   Adam  "PGAD", u32 version 1, u64 step, u64 nparams, per parameter u32
 *         flags (bit 0: m and v follow, bit 1: the amsgrad maximum follows)
 *         then those PGT1 records.
 * load_into restores the state of an optimiser built with the same
 * parameters (count and shapes checked, false on a mismatch); a parameter
 * saved without state gets none, so its next step starts from zero as a
 * fresh optimiser's does.  The hyper-parameters stay the caller's. */
bool pg_amd_sgd_save(const pg_sgd *opt, const char *path);
bool pg_amd_sgd_save_fp(const pg_sgd *opt, FILE *fp);
bool pg_amd_sgd_load_into(pg_sgd *opt, const char *path);
bool pg_amd_sgd_load_into_fp(pg_sgd *opt, FILE *fp);
bool pg_amd_adam_save(const pg_adam *opt, const char *path);
bool pg_amd_adam_save_fp(const pg_adam *opt, FILE *fp);
bool pg_amd_adam_load_into(pg_adam *opt, const char *path);
bool pg_amd_adam_load_into_fp(pg_adam *opt, FILE *fp);

/* Kernel timer: while enabled, the fused backward kernel (kind 0), its
 * reduction finisher (1), the MFMA GEMMs (2), the SGD kernel (3), the
 * GEMM operand staging (4), the Adam kernel (5) and the gradient-clipping
 * passes (6) are bracketed by HIP events on the library stream.
 * pg_amd_timer_read waits for the stream and returns the summed
 * milliseconds of one kind (and the number of launches). */
void pg_amd_timer_enable(int on);
double pg_amd_timer_read(int kind, size_t *count);
void pg_amd_timer_reset(void);

#ifdef __cplusplus
}
#endif

#endif
