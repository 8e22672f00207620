/* Model descriptor ABI of the PLaMo-3-Translate token loop.
 *
 * These layouts are the contract between the engine (runtime/engine.c), the
 * CPU layer and a compute backend. They are byte-for-byte the reference's
 * descriptor ABI so that a binary built against the reference headers can
 * hand its descriptors to this backend unchanged:
 *   - struct qkv/cache/rotation/gqa/mixer/mlp/layer/model:
 *       runtime/model.h:7-60 (sizes asserted at runtime/model.h:76-86)
 *   - struct plamo_mapping / plamo_weight_spec: runtime/model.h:61-70
 *   - struct plamo_matmul: runtime/parallel.h:5-10, declared in plamo_parallel.h
 *
 * Conventions (all from the reference):
 *   - weights are BF16 bit patterns (uint16_t), row-major [rows, columns];
 *   - activations, KV rows and logits are FP32;
 *   - KV caches are token-major [capacity, kv_heads * head_dim];
 *   - rotation->out holds RoPE-rotated keys at local row positions
 *     0..count-1; processed_count/scale_bits tell which rows are current
 *     (src/cache_rope.s:11-33).
 */
#ifndef PLAMO_MODEL_H
#define PLAMO_MODEL_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct qkv {
    const float *input;
    const uint16_t *weight, *qn, *kn;
    float *out;
    uint64_t hidden, qh, kh, dim;
};
struct cache {
    float *k, *v;
    uint64_t capacity, count, width, sliding;
};
struct rotation {
    struct cache *cache;
    float *out;
    const float *freq;
    float *cos, *sin;
    uint64_t heads, dim, processed_count, scale_bits;
};
struct gqa {
    float *q, *k, *v, *out, *scores;
    uint64_t tokens, dim, qh, kh;
};
struct mixer {
    struct qkv *qkv;
    struct cache *cache;
    struct rotation *rotation;
    struct gqa *gqa;
    const uint16_t *weight;
    float *out;
    uint64_t hidden;
};
struct mlp {
    float *state;
    const uint16_t *pre, *post, *gu, *down;
    float *normalized, *branch, *scratch;
    uint64_t hidden, intermediate;
};
struct layer {
    float *state;
    const uint16_t *pre, *post;
    float *normalized, *branch;
    struct mixer *mixer;
    struct mlp *mlp;
    uint64_t hidden;
};
struct model {
    const uint16_t *embedding;
    uint64_t vocab, hidden;
    float *state;
    struct layer **layers;
    uint64_t count;
    float *scales;
    const uint16_t *norm;
    float *normalized;
    const uint16_t *head;
    float *logits;
};
struct plamo_mapping {
    void *base;
    uint64_t bytes;
};
struct plamo_weight_spec {
    const char *name;
    uint64_t rank;
    const uint64_t *shape;
    void **slot;
};

#ifdef __cplusplus
#define PLAMO_STATIC_ASSERT static_assert
#else
#define PLAMO_STATIC_ASSERT _Static_assert
#endif
PLAMO_STATIC_ASSERT(sizeof(struct model) == 88, "descriptor ABI: model");
PLAMO_STATIC_ASSERT(sizeof(struct qkv) == 72, "descriptor ABI: qkv");
PLAMO_STATIC_ASSERT(sizeof(struct cache) == 48, "descriptor ABI: cache");
PLAMO_STATIC_ASSERT(sizeof(struct rotation) == 72, "descriptor ABI: rotation");
PLAMO_STATIC_ASSERT(sizeof(struct gqa) == 72, "descriptor ABI: gqa");
PLAMO_STATIC_ASSERT(sizeof(struct mixer) == 56, "descriptor ABI: mixer");
PLAMO_STATIC_ASSERT(sizeof(struct mlp) == 80, "descriptor ABI: mlp");
PLAMO_STATIC_ASSERT(sizeof(struct layer) == 64, "descriptor ABI: layer");
PLAMO_STATIC_ASSERT(offsetof(struct layer, mixer) == 40, "descriptor ABI: layer");
PLAMO_STATIC_ASSERT(offsetof(struct cache, count) == 24, "descriptor ABI: cache");
PLAMO_STATIC_ASSERT(offsetof(struct rotation, processed_count) == 56, "descriptor ABI: rotation");

/* The engine's model globals (runtime/model.h:88-101). The reference
 * generates them into assembly from a model profile at build time
 * (tools/generate_model.py:20-41, src/model_layout.s, src/prefetch.s); this
 * library fills them at run time from a checkpoint directory
 * (plamo_model_set_directory() in plamo_checkpoint.h, or $PLAMO_MODEL_DIR read
 * when the library loads), so the four strings are writable arrays here:
 *   plamo_vocab_path        <directory>/tokenizer.jsonl;
 *   plamo_model_name        "plamo-3-translate-<size>" when config.json has the
 *                           shape of a published profile (tools/profiles/<size>),
 *                           else "plamo-3-translate-custom";
 *   plamo_model_repository, plamo_model_revision  the profile's manifest values,
 *                           else empty. */
enum { PLAMO_MAX_WEIGHT_FILES = 64 };
extern struct model plamo_model;
extern struct plamo_mapping plamo_weight_mappings[PLAMO_MAX_WEIGHT_FILES];
extern int64_t plamo_weight_fds[PLAMO_MAX_WEIGHT_FILES];
extern uint64_t plamo_weight_mapping_count, plamo_weight_file_count;
extern char plamo_vocab_path[], plamo_model_name[], plamo_model_repository[],
    plamo_model_revision[];
extern struct plamo_weight_spec plamo_weight_schema[];
/* plamo_model_patches: {descriptor field address, schema slot address} pairs,
 * terminated by a zero pair, filled by plamo_model_open(). plamo_io_policy and
 * plamo_io_stats[4] ({bytes staged, read calls, ...}, src/prefetch.s:28-66)
 * are kept for the engine: the GPU path reads no weight file during a token,
 * so the statistics stay zero. */
extern uint64_t plamo_model_patches[], plamo_io_policy, plamo_io_stats[4];
/* runtime/model.h:97-100 (storage src/prefetch.s:31-36). */
extern const void *(*plamo_weight_provider)(const void *, uint64_t, void *);
extern void *plamo_weight_context;
extern uint64_t plamo_weight_chunk_bytes;
/* src/model_open.s:6-60: opens the model directory once per process.
 * 1 = ready (repeat calls succeed at once), 0 = failure (message on stderr). */
int plamo_model_open(void);
/* src/model_init.s:1-25: for a patch table as above, 1 after storing every
 * slot's pointer into its descriptor field, or 0 with nothing stored when a
 * slot holds NULL. The engine calls it after moving the weights
 * (runtime/engine.c:69-74). */
int plamo_model_patch(void *patches);

/* Token-loop entry points of the compute dispatch layer (runtime/model.h:103-105,
 * src/forward.s:9-31, src/prefill.s:7-30, src/token.s:37-63). The trampolines
 * call the installed backend hook; a declined hook (0) falls through to the
 * platform CPU path registered with plamo_register_cpu_path(), and a failed
 * hook (-1) is never retried. Both return 1 on success and 0 on failure. */
int plamo_prefill(struct model *, const uint32_t *, uint64_t, float *);
int plamo_forward(struct model *, uint64_t);
/* First maximal index (strict >); empty or any NaN gives UINT64_MAX. */
uint64_t plamo_argmax(const float *, uint64_t);
/* Defined by the engine (runtime/engine.c:46-55), not by this library: counts
 * and rotation bookkeeping back to zero without touching weights or KV rows. */
void plamo_reset_request(struct model *);

#ifdef __cplusplus
}
#endif
#endif
