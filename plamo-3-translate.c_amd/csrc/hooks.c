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
#include <emmintrin.h>
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

/* src/token.s:37-63: index of the first maximal element (strict >), any NaN
 * gives UINT64_MAX. Two SSE2 passes: the maximum with a NaN check, then the
 * first element equal to it (equivalent to the strict sequential scan: equal
 * values never replace the first one). */
uint64_t plamo_argmax(const float *x, uint64_t n) {
    if (!n)
        return UINT64_MAX;
    __m128 m0 = _mm_set1_ps(x[0]), m1 = m0, m2 = m0, m3 = m0;
    __m128 unordered = _mm_setzero_ps();
    uint64_t i = 0;
    for (; i + 16 <= n; i += 16) {
        const __m128 a = _mm_loadu_ps(x + i), b = _mm_loadu_ps(x + i + 4);
        const __m128 c = _mm_loadu_ps(x + i + 8), d = _mm_loadu_ps(x + i + 12);
        unordered = _mm_or_ps(unordered, _mm_or_ps(_mm_cmpunord_ps(a, b), _mm_cmpunord_ps(c, d)));
        m0 = _mm_max_ps(m0, a);
        m1 = _mm_max_ps(m1, b);
        m2 = _mm_max_ps(m2, c);
        m3 = _mm_max_ps(m3, d);
    }
    if (_mm_movemask_ps(unordered))
        return UINT64_MAX;
    __m128 m = _mm_max_ps(_mm_max_ps(m0, m1), _mm_max_ps(m2, m3));
    m = _mm_max_ps(m, _mm_shuffle_ps(m, m, _MM_SHUFFLE(1, 0, 3, 2)));
    m = _mm_max_ps(m, _mm_shuffle_ps(m, m, _MM_SHUFFLE(2, 3, 0, 1)));
    float value = _mm_cvtss_f32(m);
    for (; i < n; ++i) {
        if (isnan(x[i]))
            return UINT64_MAX;
        if (x[i] > value)
            value = x[i];
    }
    const __m128 v = _mm_set1_ps(value);
    for (i = 0; i + 16 <= n; i += 16) {
        const int hit = _mm_movemask_ps(_mm_cmpeq_ps(_mm_loadu_ps(x + i), v)) |
                        _mm_movemask_ps(_mm_cmpeq_ps(_mm_loadu_ps(x + i + 4), v)) << 4 |
                        _mm_movemask_ps(_mm_cmpeq_ps(_mm_loadu_ps(x + i + 8), v)) << 8 |
                        _mm_movemask_ps(_mm_cmpeq_ps(_mm_loadu_ps(x + i + 12), v)) << 12;
        if (hit)
            return i + (uint64_t)__builtin_ctz((unsigned)hit);
    }
    for (; i < n; ++i)
        if (x[i] == value)
            return i;
    return UINT64_MAX; /* unreachable: the maximum is one of the elements */
}
