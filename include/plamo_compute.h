/* Compute dispatch ABI (hooks) of the token loop.
 *
 * The reference keeps one function pointer per hot operation plus an opaque
 * backend context; the CPU layer calls through them when set and runs its own
 * kernels otherwise (runtime/compute.h:8-14, storage in src/prefetch.s:37-52).
 * This library defines that storage and installs its HIP implementations when
 * a backend is opened (the reference does the same at runtime/metal.m:900-910
 * and removes them at runtime/metal.m:938-948).
 *
 * Hook return conventions (src/forward.s:19-25, src/prefill.s:19-24,
 * src/model.s:71-79):
 *   forward / prefill:  1 = done, 0 = declined with model state untouched,
 *                      -1 = failed after partial writes, never retried;
 *   mlp:                1 = done, 0 = declined with states untouched;
 *   matvec / matmul:    void; the backend is responsible for the result.
 */
#ifndef PLAMO_COMPUTE_H
#define PLAMO_COMPUTE_H
#include "plamo_model.h"
#include "plamo_parallel.h"

#ifdef __cplusplus
extern "C" {
#endif

/* runtime/compute.h:8-14 */
extern void *plamo_compute_context;
extern void (*plamo_matvec_kernel)(const uint16_t *, const float *, float *, uint64_t, uint64_t,
                                   void *);
extern void (*plamo_matmul_kernel)(const struct plamo_matmul *, void *);
extern int (*plamo_mlp_kernel)(const struct mlp *, float *, uint64_t, void *);
extern int (*plamo_forward_kernel)(struct model *, uint64_t, void *);
extern int (*plamo_prefill_kernel)(struct model *, const uint32_t *, uint64_t, float *, void *);

/* The optional weight provider (plamo_weight_provider, plamo_weight_context,
 * plamo_weight_chunk_bytes) is declared with the model globals in
 * plamo_model.h. The GPU backend installs the identity provider with chunk
 * bytes 0. */

/* The platform CPU path behind the trampolines. On the reference platform this
 * is the AArch64 assembly (src/forward.s:33-81, src/prefill.s:31-178); this
 * library has no CPU implementation of its own, so a host program that wants
 * the decline-then-CPU behaviour registers one here. With none registered a
 * declined hook makes plamo_forward/plamo_prefill return 0. */
struct plamo_cpu_path {
    int (*forward)(struct model *, uint64_t);
    int (*prefill)(struct model *, const uint32_t *, uint64_t, float *);
};
void plamo_register_cpu_path(const struct plamo_cpu_path *);

#ifdef __cplusplus
}
#endif
#endif
