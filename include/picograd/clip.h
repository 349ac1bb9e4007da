/*
 * Gradient clipping over device-resident grads: the reference's
 * opt/clip.h:12-29 entry points that take a list of parameter nodes.
 *
 * The global norm is summed in f64 as clip.c:5-18 does, by a multi-tensor
 * reduction with a fixed summation order (so repeated calls agree bit for
 * bit); pg_clip_grad_norm queues the scaling pass behind the reduction with
 * the decision taken on the device, then waits for the stream once to
 * return the norm.  NULL nodes and nodes without a grad are skipped.
 *
 * The pg_module conveniences (clip.h:21, :25, :29) are not provided: the
 * reference's nn modules are not part of this library.
 *
 * A device failure returns -1 from the two functions returning a norm,
 * with the message in pg_amd_last_error().
 */
#ifndef PICOGRAD_CLIP_H
#define PICOGRAD_CLIP_H

#include "autograd.h"

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* clip.h:12-18: returns the norm before clipping, -1 on bad arguments
 * (params NULL or max_norm <= 0); eps < 0 means 1e-6 */
float pg_clip_grad_norm(pg_node **params, size_t n, float max_norm, float eps);

/* clip.h:23-24: each grad value clamped into [-clip_value, clip_value];
 * clip_value <= 0 does nothing */
void pg_clip_grad_value(pg_node **params, size_t n, float clip_value);

/* clip.h:27-28: the global L2 norm of the grads, without clipping */
float pg_grad_norm(pg_node **params, size_t n);

#ifdef __cplusplus
}
#endif

#endif
