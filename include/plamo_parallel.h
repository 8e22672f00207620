/* The projection descriptor the hooks and plamo_metal_linear take
 * (runtime/parallel.h:5-11).
 *
 * runtime/parallel.h also declares the engine's CPU thread pool
 * (plamo_parallel_open/threads/close, runtime/parallel.c), which stays with
 * the engine. A translation unit that includes that header first keeps its
 * definition of the struct; this one then adds nothing, so the engine's
 * sources compile unchanged against these headers.
 */
#ifndef PLAMO_HIP_PARALLEL_H
#define PLAMO_HIP_PARALLEL_H
#include <stdint.h>

#ifndef PLAMO_PARALLEL_H
/* Strides are in FP32 elements. */
struct plamo_matmul {
    const uint16_t *weights;
    const float *input;
    float *output;
    uint64_t rows, columns, tokens, input_stride, output_stride;
};
#endif

#ifdef __cplusplus
static_assert(sizeof(struct plamo_matmul) == 64, "descriptor ABI: matmul");
#else
_Static_assert(sizeof(struct plamo_matmul) == 64, "descriptor ABI: matmul");
#endif
#endif
