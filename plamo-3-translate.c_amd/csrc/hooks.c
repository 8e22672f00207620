/* Compute dispatch layer of the token loop: hook storage and trampolines.
 *
 * Restates in C what the reference keeps in assembly so the engine links on
 * Linux: the hook and weight-provider globals (src/prefetch.s:27-52), the
 * tri-state trampolines of the decode and prompt entries (src/forward.s:9-31,
 * src/prefill.s:7-30) and the host argmax (src/token.s:37-63). The
 * trampolines never retry a hook that returned -1; a hook that declines (0)
 * hands the call to the registered platform CPU path, and without one the
 * call fails. This file computes nothing on the model.
 */
#include "../../include/plamo_compute.h"
#include <math.h>
#include <string.h>

void *plamo_compute_context;
void (*plamo_matvec_kernel)(const uint16_t *, const float *, float *, uint64_t, uint64_t, void *);
void (*plamo_matmul_kernel)(const struct plamo_matmul *, void *);
int (*plamo_mlp_kernel)(const struct mlp *, float *, uint64_t, void *);
int (*plamo_forward_kernel)(struct model *, uint64_t, void *);
int (*plamo_prefill_kernel)(struct model *, const uint32_t *, uint64_t, float *, void *);
const void *(*plamo_weight_provider)(const void *, uint64_t, void *);
void *plamo_weight_context;
uint64_t plamo_weight_chunk_bytes;

static struct plamo_cpu_path cpu_path;

void plamo_register_cpu_path(const struct plamo_cpu_path *path) {
    if (path)
        cpu_path = *path;
    else
        memset(&cpu_path, 0, sizeof cpu_path);
}

int plamo_forward(struct model *model, uint64_t token) {
    if (plamo_forward_kernel) {
        int result = plamo_forward_kernel(model, token, plamo_compute_context);
        if (result)
            return result == 1;
    }
    return cpu_path.forward ? cpu_path.forward(model, token) : 0;
}

int plamo_prefill(struct model *model, const uint32_t *ids, uint64_t tokens, float *states) {
    if (!tokens)
        return 0;
    if (plamo_prefill_kernel) {
        int result = plamo_prefill_kernel(model, ids, tokens, states, plamo_compute_context);
        if (result)
            return result == 1;
    }
    return cpu_path.prefill ? cpu_path.prefill(model, ids, tokens, states) : 0;
}

uint64_t plamo_argmax(const float *x, uint64_t n) {
    if (!n || isnan(x[0]))
        return UINT64_MAX;
    uint64_t best = 0;
    float value = x[0];
    for (uint64_t i = 1; i < n; ++i) {
        if (isnan(x[i]))
            return UINT64_MAX;
        if (x[i] > value) {
            value = x[i];
            best = i;
        }
    }
    return best;
}
