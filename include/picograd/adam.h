/*
 * Adam / AdamW: same ABI, defaults, per-parameter overrides and update rule
 * as the reference's opt/adam.h:12-44 and adam.c:27-181.  pg_adam_step()
 * updates every registered parameter that has a grad in one fused device
 * kernel launch (up to 32 tensors per launch) and returns without waiting;
 * the first and second moments (and the amsgrad running maximum) live in
 * device memory beside the parameters.
 */
#ifndef PICOGRAD_ADAM_H
#define PICOGRAD_ADAM_H

#include "autograd.h"

#include <stdbool.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* adam.h:12-20 */
typedef struct {
    float lr;
    float beta1;
    float beta2;
    float eps;
    float weight_decay;
    bool amsgrad;
    bool decoupled_wd; /* true = AdamW (decay applied to the weights), false = L2 */
} pg_adam_cfg;

/* adam.h:22, adam.c:27-37: lr 1e-3, betas 0.9/0.999, eps 1e-8, AdamW */
pg_adam_cfg pg_adam_cfg_default(void);

typedef struct pg_adam pg_adam;

/* adam.h:26-27; a NULL cfg takes the defaults; invalid values assert
 * (adam.c:40-44) */
pg_adam *pg_adam_new(const pg_adam_cfg *cfg);
void pg_adam_free(pg_adam *opt);

/* adam.h:29-32: registration retains the node; lr <= 0 or wd < 0 keeps the
 * optimiser-wide value */
int pg_adam_add_param(pg_adam *opt, pg_node *param);
int pg_adam_add_param_lr(pg_adam *opt, pg_node *param, float lr, float wd);
size_t pg_adam_num_params(const pg_adam *opt);

/* adam.h:34-37 */
void pg_adam_set_lr(pg_adam *opt, float lr);
float pg_adam_get_lr(const pg_adam *opt);
void pg_adam_set_param_lr(pg_adam *opt, size_t idx, float lr);
void pg_adam_set_param_wd(pg_adam *opt, size_t idx, float wd);

/* adam.h:39-40: zero_grad frees the grads (adam.c:102-108) */
void pg_adam_zero_grad(pg_adam *opt);
void pg_adam_step(pg_adam *opt);

/* adam.h:42-44: the step counter the bias corrections use */
void pg_adam_set_step(pg_adam *opt, unsigned long long step);
unsigned long long pg_adam_get_step(const pg_adam *opt);

#ifdef __cplusplus
}
#endif

#endif
