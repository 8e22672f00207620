/* Descriptor graph of a PLaMo-3 model over borrowed BF16 weights, the layout
 * of tools/model_layout.py:71-199: one workspace shared by all layers, per-layer
 * raw-K / V / rotated-K rows, sliding layers holding window + 1 rows, every
 * pattern-th layer global with its own frequencies and concentration. The
 * synthetic builder and the checkpoint loader both instantiate it. Internal to
 * the library. */
#ifndef PLAMO_LAYOUT_H
#define PLAMO_LAYOUT_H
#include "../../include/plamo_synthetic.h"

#ifdef __cplusplus
extern "C" {
#endif

struct plamo_layout_layer {
    const uint16_t *pre, *post, *qkv, *qn, *kn, *o, *mlp_pre, *mlp_post, *gu, *down;
};

struct plamo_layout {
    uint64_t hidden, layers, qh, kh, dim, intermediate, vocab;
    uint64_t window;          /* sliding layers hold window + 1 rows */
    uint64_t global_capacity; /* rows of a global layer */
    uint64_t pattern;         /* layer i is global when (i + 1) % pattern == 0; 0: none */
    const uint16_t *embedding, *head, *norm;
    const struct plamo_layout_layer *layer; /* [layers] */
    const float *local_freq, *global_freq;  /* [dim / 2] */
    float local_scale, global_scale;
};

/* FP32 RoPE inverse frequencies (tools/rope_constants.py:21-52): the default
 * table of `theta`, or with yarn != 0 its YaRN blend. `out` holds half floats. */
void plamo_layout_frequencies(double theta, uint64_t half, int yarn, double factor,
                              double original, double beta_fast, double beta_slow, float *out);

/* Host arrays and descriptors of one instance; the weights stay borrowed. */
struct plamo_synthetic_instance *plamo_layout_instantiate(const struct plamo_layout *, int pinned,
                                                          char *error, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
