/* tnpa_internal.h -- entry points of libtnpa.so that are not part of its public ABI (include/tnpa.h).
 *
 * They expose how tnpa_backward splits its work into kernel launches, for the benchmark (which times each launch on
 * its own) and the tests (which check that the launches run one by one equal the whole call, and that the optional
 * row-scaled dO workspace changes nothing beyond rounding). The split may change with any build; callers of the
 * public ABI never depend on it. None of these has a counterpart in the reference.
 */
#ifndef TNPA_INTERNAL_H
#define TNPA_INTERNAL_H

#include <stdint.h>

#include "../../include/tnpa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Options of the backward plan. 0 is what tnpa_backward runs. */
#define TNPA_X_PRESCALE_ON 1  /* write row_scale * dO into the workspace first and stream it (where the plan would not) */
#define TNPA_X_PRESCALE_OFF 2 /* never write it: the dK/dV kernels apply the row scale themselves */
#define TNPA_X_DS_OFF 4       /* dQ recomputes S and dP (no dS tiles in the workspace) where the plan would read dS */

/* Workspace bytes of the backward plan with these options (-1 for an invalid problem or options). */
int64_t tnpa_x_workspace_bytes(const tnpa_problem_t* problem, int32_t opts);

/* Number of kernel launches of the plan (-1 for an invalid problem or options). */
int32_t tnpa_x_launches(const tnpa_problem_t* problem, int32_t opts);

/* Short name of launch i of the plan ("scale", "kv", "dv", "dk", "q", "qds", "dpar"), or "" when i is out of range. */
const char* tnpa_x_launch_name(const tnpa_problem_t* problem, int32_t opts, int32_t i);

/* Runs the plan's launches (only = -1) or launch `only` alone; a launch run alone reads what the launches before it
 * wrote into the workspace by an earlier call. tnpa_backward(p, g, s) == tnpa_x_backward(p, g, 0, -1, s). */
int tnpa_x_backward(const tnpa_problem_t* problem, const tnpa_grads_t* grads, int32_t opts, int32_t only,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TNPA_INTERNAL_H */
