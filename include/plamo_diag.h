/* Measurement entry point of the MI355X backend.
 *
 * No counterpart in the reference (which reads GPU time from Metal command
 * buffer timestamps, runtime/metal.m:235): the benchmark uses it to time one
 * decode kernel in isolation with HIP events on the backend's own stream, for
 * the roofline of the dominant kernel.
 */
#ifndef PLAMO_DIAG_H
#define PLAMO_DIAG_H
#include "plamo_backend.h"

#ifdef __cplusplus
extern "C" {
#endif

enum plamo_hip_kernel {
    PLAMO_HIP_QKV = 0,      /* pre-norm + QKV projection GEMV */
    PLAMO_HIP_O = 1,        /* attention output projection GEMV */
    PLAMO_HIP_GATE_UP = 2,  /* residual + pre-MLP norm + gate/up GEMV + SwiGLU */
    PLAMO_HIP_DOWN = 3,     /* down projection GEMV */
    PLAMO_HIP_HEAD = 4,     /* final norm + vocabulary head GEMV */
    PLAMO_HIP_ATTENTION = 5 /* decode attention over the layer's current rows */
};
/* Launches kernel `which` of `layer` `reps` times on the live decode
 * workspace of a prepared model (after at least one decode step) and reports
 * the mean milliseconds per launch and the algorithmic HBM bytes one launch
 * must move (weights for projections; K and V rows for attention). The
 * workspace contents are scratch afterwards: the next decode step rewrites
 * them. Returns 0 when the model is not prepared or an argument is invalid. */
int plamo_hip_time_kernel(struct plamo_metal *, struct model *, uint64_t layer, int which,
                          int reps, double *ms_per_launch, double *bytes_per_launch);

/* Test hook of the failure contract (runtime/metal.h:63-67): from the next
 * call on, the decode attention's output-projection blocks wait for `extra`
 * more finished KV heads than exist and give up after `polls` polls
 * (0: the default bound), so the call must return -1 with one counted error
 * while every kernel still exits normally. plamo_hip_debug_waits(m, 0, 0)
 * restores the normal waits. No counterpart in the reference. */
void plamo_hip_debug_waits(struct plamo_metal *, uint32_t extra, uint32_t polls);

#ifdef __cplusplus
}
#endif
#endif
