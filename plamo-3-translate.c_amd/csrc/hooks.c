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
#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
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
 * gives UINT64_MAX. Two passes: the maximum with a NaN check, then the first
 * element equal to it (equivalent to the strict sequential scan: equal values
 * never replace the first one). The logits a decode step writes to pinned
 * host memory are cold in the CPU's caches; over 100000 of them the first
 * pass reads DRAM, and wider vectors issue its loads sooner (SSE2 11.7 us,
 * AVX2 9.9, AVX-512 9.1 on the MI355X host). The widest the CPU has is chosen
 * at the first call; PLAMO_ARGMAX_ISA=sse2 or avx2 caps it (every form gives
 * the same index). */
__attribute__((target("avx512f"))) static uint64_t argmax_avx512(const float *x, uint64_t n) {
    __m512 m0 = _mm512_set1_ps(x[0]), m1 = m0, m2 = m0, m3 = m0;
    __mmask16 unordered = 0;
    uint64_t i = 0;
    for (; i + 64 <= n; i += 64) {
        const __m512 a = _mm512_loadu_ps(x + i), b = _mm512_loadu_ps(x + i + 16);
        const __m512 c = _mm512_loadu_ps(x + i + 32), d = _mm512_loadu_ps(x + i + 48);
        unordered |= (__mmask16)(_mm512_cmp_ps_mask(a, b, _CMP_UNORD_Q) |
                                 _mm512_cmp_ps_mask(c, d, _CMP_UNORD_Q));
        m0 = _mm512_max_ps(m0, a);
        m1 = _mm512_max_ps(m1, b);
        m2 = _mm512_max_ps(m2, c);
        m3 = _mm512_max_ps(m3, d);
    }
    if (unordered)
        return UINT64_MAX;
    float value = _mm512_reduce_max_ps(_mm512_max_ps(_mm512_max_ps(m0, m1), _mm512_max_ps(m2, m3)));
    for (; i < n; ++i) {
        if (isnan(x[i]))
            return UINT64_MAX;
        if (x[i] > value)
            value = x[i];
    }
    const __m512 v = _mm512_set1_ps(value);
    for (i = 0; i + 64 <= n; i += 64) {
        const uint64_t hit =
            (uint64_t)_mm512_cmp_ps_mask(_mm512_loadu_ps(x + i), v, _CMP_EQ_OQ) |
            (uint64_t)_mm512_cmp_ps_mask(_mm512_loadu_ps(x + i + 16), v, _CMP_EQ_OQ) << 16 |
            (uint64_t)_mm512_cmp_ps_mask(_mm512_loadu_ps(x + i + 32), v, _CMP_EQ_OQ) << 32 |
            (uint64_t)_mm512_cmp_ps_mask(_mm512_loadu_ps(x + i + 48), v, _CMP_EQ_OQ) << 48;
        if (hit)
            return i + (uint64_t)__builtin_ctzll(hit);
    }
    for (; i < n; ++i)
        if (x[i] == value)
            return i;
    return UINT64_MAX; /* unreachable: the maximum is one of the elements */
}

__attribute__((target("avx2"))) static uint64_t argmax_avx2(const float *x, uint64_t n) {
    __m256 m0 = _mm256_set1_ps(x[0]), m1 = m0, m2 = m0, m3 = m0;
    __m256 unordered = _mm256_setzero_ps();
    uint64_t i = 0;
    for (; i + 32 <= n; i += 32) {
        const __m256 a = _mm256_loadu_ps(x + i), b = _mm256_loadu_ps(x + i + 8);
        const __m256 c = _mm256_loadu_ps(x + i + 16), d = _mm256_loadu_ps(x + i + 24);
        unordered = _mm256_or_ps(unordered, _mm256_or_ps(_mm256_cmp_ps(a, b, _CMP_UNORD_Q),
                                                         _mm256_cmp_ps(c, d, _CMP_UNORD_Q)));
        m0 = _mm256_max_ps(m0, a);
        m1 = _mm256_max_ps(m1, b);
        m2 = _mm256_max_ps(m2, c);
        m3 = _mm256_max_ps(m3, d);
    }
    if (_mm256_movemask_ps(unordered))
        return UINT64_MAX;
    float lanes[8];
    _mm256_storeu_ps(lanes, _mm256_max_ps(_mm256_max_ps(m0, m1), _mm256_max_ps(m2, m3)));
    float value = lanes[0];
    for (int k = 1; k < 8; ++k)
        if (lanes[k] > value)
            value = lanes[k];
    for (; i < n; ++i) {
        if (isnan(x[i]))
            return UINT64_MAX;
        if (x[i] > value)
            value = x[i];
    }
    const __m256 v = _mm256_set1_ps(value);
    for (i = 0; i + 32 <= n; i += 32) {
        const unsigned hit =
            (unsigned)_mm256_movemask_ps(_mm256_cmp_ps(_mm256_loadu_ps(x + i), v, _CMP_EQ_OQ)) |
            (unsigned)_mm256_movemask_ps(_mm256_cmp_ps(_mm256_loadu_ps(x + i + 8), v, _CMP_EQ_OQ)) << 8 |
            (unsigned)_mm256_movemask_ps(_mm256_cmp_ps(_mm256_loadu_ps(x + i + 16), v, _CMP_EQ_OQ)) << 16 |
            (unsigned)_mm256_movemask_ps(_mm256_cmp_ps(_mm256_loadu_ps(x + i + 24), v, _CMP_EQ_OQ)) << 24;
        if (hit)
            return i + (uint64_t)__builtin_ctz(hit);
    }
    for (; i < n; ++i)
        if (x[i] == value)
            return i;
    return UINT64_MAX; /* unreachable: the maximum is one of the elements */
}

static uint64_t argmax_sse2(const float *x, uint64_t n);

uint64_t plamo_argmax(const float *x, uint64_t n) {
    static uint64_t (*impl)(const float *, uint64_t);
    if (!n)
        return UINT64_MAX;
    if (!impl) {
        const char *cap = getenv("PLAMO_ARGMAX_ISA");
        const int max_level = !cap ? 2 : !strcmp(cap, "sse2") ? 0 : !strcmp(cap, "avx2") ? 1 : 2;
        __builtin_cpu_init();
        impl = max_level >= 2 && __builtin_cpu_supports("avx512f") ? argmax_avx512
               : max_level >= 1 && __builtin_cpu_supports("avx2")  ? argmax_avx2
                                                                   : argmax_sse2;
    }
    return impl(x, n);
}

static uint64_t argmax_sse2(const float *x, uint64_t n) {
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
