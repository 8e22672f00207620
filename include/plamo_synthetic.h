/* Synthetic PLaMo-3 model descriptors for the BASELINE configurations.
 *
 * No reference counterpart as an API: it builds the same descriptor graph the
 * reference's generator emits for a real checkpoint (tools/model_layout.py:71-199:
 * shared per-model workspace, per-layer KV/rotated buffers, sliding capacity
 * window+1, every pattern-th layer global with the YaRN table and
 * concentration, tools/rope_constants.py:21-70), but from a config instead of
 * a safetensors file, with seeded random BF16 weights. The reference's own
 * GPU tests build such graphs by hand (tests/metal_decode.c:95-175).
 *
 * Weights live in one host arena returned as a plamo_mapping, so it can be
 * handed to plamo_metal_open() like the mmapped weight files of the engine.
 */
#ifndef PLAMO_SYNTHETIC_H
#define PLAMO_SYNTHETIC_H
#include "plamo_model.h"

#ifdef __cplusplus
extern "C" {
#endif

struct plamo_synthetic_config {
    uint64_t hidden, layers, qh, kh, dim, intermediate, vocab;
    uint64_t window;          /* sliding layers hold window + 1 rows */
    uint64_t global_capacity; /* rows of a global (full-attention) layer */
    uint64_t pattern;         /* layer i is global when (i+1) % pattern == 0; 0: none */
    uint64_t seed;
    double weight_std;        /* projections, norms and head ~ N(0, weight_std) */
    double embedding_std;     /* embedding table ~ N(0, embedding_std) */
    int tied;                 /* head is the embedding table */
    double local_theta;       /* default RoPE base of sliding layers */
    double global_theta;      /* YaRN base of global layers */
    double yarn_factor, yarn_original, yarn_beta_fast, yarn_beta_slow;
};

struct plamo_synthetic;
struct plamo_synthetic_instance;

/* Fills the BASELINE defaults (RoPE/YaRN constants of docs/config.json,
 * window 2048, pattern 8, std 0.02) around the given shape. */
void plamo_synthetic_defaults(struct plamo_synthetic_config *, uint64_t hidden, uint64_t layers,
                              uint64_t qh, uint64_t kh, uint64_t dim, uint64_t intermediate,
                              uint64_t vocab);
/* Generates the weights (threads > 1 splits the work; results do not depend on
 * the thread count). NULL with a message on failure. */
struct plamo_synthetic *plamo_synthetic_build(const struct plamo_synthetic_config *,
                                              unsigned threads, char *error, size_t cap);
void plamo_synthetic_free(struct plamo_synthetic *);
const struct plamo_mapping *plamo_synthetic_weights(const struct plamo_synthetic *);
/* FP32 RoPE inverse frequencies of a layer (dim/2 floats). */
const float *plamo_synthetic_frequencies(const struct plamo_synthetic *, uint64_t layer);

/* A model instance: descriptors, workspace, KV caches and outputs over the
 * shared weights. pinned != 0 allocates host arrays as page-locked memory
 * (faster device copies); otherwise anonymous mappings. */
struct plamo_synthetic_instance *plamo_synthetic_instantiate(const struct plamo_synthetic *,
                                                             int pinned, char *error, size_t cap);
void plamo_synthetic_release(struct plamo_synthetic_instance *);
struct model *plamo_synthetic_model(struct plamo_synthetic_instance *);
/* Sets every cache to `rows` rows of raw K and V ~ N(0,1) (seeded), marks the
 * rotated keys stale (processed_count 0) so the first step rebuilds them. */
int plamo_synthetic_fill_kv(struct plamo_synthetic_instance *, uint64_t rows, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
