/* GPU backend API of the token loop, implemented for MI355X (gfx950).
 *
 * This is the plain-C interface the reference engine binds for its GPU
 * backend (runtime/metal.h:5-88). The function names, argument meanings,
 * struct layouts and tri-state results are kept identical so runtime/engine.c
 * links against this library instead of runtime/metal*.m without a change;
 * "metal" in the names is the reference's spelling of "the GPU backend".
 *
 * MI355X design (what differs from the reference behind the same contract):
 *   - every weight range named by the config mappings or by preload() is
 *     copied once into HBM and stays resident (288 GB per GPU);
 *   - KV caches, rotated keys and activations live in HBM; the model's host
 *     arrays (state, normalized, logits, K, V, rotated K) are refreshed before
 *     each successful call returns, and host-side edits (prefix restore, draft
 *     restore, request reset, a CPU fallback step) are detected at the next
 *     call and uploaded;
 *   - one decode step is one hipGraph launch.
 */
#ifndef PLAMO_BACKEND_H
#define PLAMO_BACKEND_H
#include "plamo_model.h"
#include "plamo_parallel.h"

#ifdef __cplusplus
extern "C" {
#endif

/* runtime/weight_cache.h:7-11. A translation unit that includes the engine's
 * runtime/weight_cache.h first (as runtime/metal.h:3-4 does) keeps its
 * definition. */
#ifndef PLAMO_WEIGHT_CACHE_H
struct plamo_weight_cache_info {
    uint64_t budget_bytes, max_budget_bytes, cached_bytes, staging_bytes;
    uint64_t hits, hit_bytes, misses, resizes;
    uint64_t storage_bytes;
};
#endif

/* runtime/metal.h:6-13 */
enum plamo_metal_memory { PLAMO_METAL_AUTO, PLAMO_METAL_RESIDENT, PLAMO_METAL_STREAM };
enum plamo_metal_precision { PLAMO_METAL_FP32 };
enum plamo_metal_packing {
    PLAMO_PACK_AUTO,
    PLAMO_PACK_RAW,
    PLAMO_PACK_LOSSLESS,
    PLAMO_PACK_DRAFT_Q4
};
/* runtime/metal.h:14-28. maps/count name the weight files: with memory AUTO or
 * RESIDENT each mapping is copied to HBM at open. reserve, available,
 * disk_cache_path, revision, packing and prefer_texture_weights are accepted
 * and ignored (they steer Apple unified-memory policies). */
struct plamo_metal_config {
    enum plamo_metal_memory memory;
    enum plamo_metal_precision precision;
    enum plamo_metal_packing packing;
    uint64_t working_weight_bytes;
    const struct plamo_mapping *maps;
    const int64_t *fds;
    size_t count;
    const struct plamo_weight_spec *schema;
    uint64_t reserve;
    uint64_t (*available)(void);
    const char *disk_cache_path, *revision;
    unsigned prefer_texture_weights;
};
/* runtime/metal.h:29-44 */
struct plamo_metal_info {
    char device[128], precision[16], weight_storage[24], note[256];
    struct plamo_weight_cache_info cache;
    uint64_t dispatches, command_buffers, fused_mlps, fused_decodes, fused_prefills, cpu_fallbacks,
        errors;
    uint64_t allocated_bytes, recommended_working_set_bytes;
    uint64_t packed_weight_bytes;
    uint64_t weight_heap_bytes;
    uint64_t private_weight_bytes;
    uint64_t disk_cache_hits, disk_cache_weight_bytes, disk_cache_storage_bytes;
    uint64_t disk_cache_mapped_bytes;
    uint64_t disk_cache_mapping_bytes;
    uint64_t verification_batches, verified_tokens, committed_tokens;
    unsigned residency_sets;
    double gpu_seconds;
};
struct plamo_metal;

/* runtime/metal.h:48-49. Opens device 0 (HIP_VISIBLE_DEVICES selects it),
 * uploads the mapped weights and installs the hooks when no other backend
 * owns them. NULL with a message in error[cap] on failure. */
struct plamo_metal *plamo_metal_open(const struct plamo_metal_config *, char *error, size_t cap);
/* runtime/metal.h:50. Frees device memory and removes the hooks it installed. */
void plamo_metal_close(struct plamo_metal *);
/* runtime/metal.h:51. Nothing to rebalance: HBM is not shared with the host. */
void plamo_metal_maintain(struct plamo_metal *);
/* runtime/metal.h:52 */
void plamo_metal_get_info(const struct plamo_metal *, struct plamo_metal_info *);
/* runtime/metal.h:53-56. Copies [ptr, ptr+bytes) to HBM unless already
 * resident. 0 on allocation or copy failure. */
int plamo_metal_preload(struct plamo_metal *, const void *, uint64_t bytes);
/* runtime/metal.h:57-59. Waits for outstanding uploads. */
int plamo_metal_warm_cache(struct plamo_metal *);
/* runtime/metal.h:60-62. Validates descriptors, allocates device KV, RoPE
 * tables and workspace, and builds the decode graph. 0 on a rejected model. */
int plamo_metal_prepare_model(struct plamo_metal *, struct model *);
/* runtime/metal.h:63-67. One complete FP32 decode step. 1 = done (host state,
 * normalized, logits, KV rows and counts updated), 0 = declined with nothing
 * changed (a projection is not resident, or STREAM memory), -1 = failure. */
int plamo_metal_forward(struct plamo_metal *, struct model *, uint64_t token);
/* runtime/metal.h:68-74. Layer-major prompt processing. states (nullable)
 * receives every prompt token's final-layer state [tokens, hidden]. */
int plamo_metal_prefill(struct plamo_metal *, struct model *, const uint32_t *, uint64_t tokens,
                        float *states);
/* runtime/metal.h:75 */
enum { PLAMO_VERIFY_MAX = 16 };
/* runtime/metal.h:76-81. Batched forward of candidate ids without changing
 * canonical state; next[i] = argmax of candidate i's logits. Commit candidates
 * strictly in order from 0; a forward/prefill discards the rest. */
int plamo_metal_verify(struct plamo_metal *, struct model *, const uint32_t *, uint64_t tokens,
                       uint32_t *next);
int plamo_metal_commit(struct plamo_metal *, struct model *, uint64_t index);
/* runtime/metal.h:82-85. Synchronous projection output[t] = W * input[t] for
 * every token t (strides in FP32 elements). 0 = not handled. */
int plamo_metal_linear(struct plamo_metal *, const struct plamo_matmul *);
/* No counterpart in the reference. The projection of plamo_metal_linear for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): input and output are the caller's
 * DEVICE buffers (FP32, strides in elements), the weights a host address made
 * resident by the config mappings or plamo_metal_preload, and the GEMM's
 * scratch (split-K partial tiles, arrival counters, BF16 planes of the input)
 * a static device array of PLAMO_HIP_STATIC_SCRATCH_BYTES held by each GPU
 * until the process ends. Nothing is allocated. Rejected (0, reason in
 * info.note): tokens > 1 with 3 * round_up(tokens, 128) * columns * 2 bytes
 * of planes above PLAMO_HIP_STATIC_PLANE_BYTES, weights not resident, no
 * static scratch on the device, an input or output that is not device memory
 * of the backend's GPU spanning every strided row, or a call that overlaps
 * another on the same GPU (from any backend instance of the process: one
 * call at a time owns the array, the other is refused). Enqueued on the
 * backend's stream; returns after completion with the same bits as
 * plamo_metal_linear. */
#define PLAMO_HIP_STATIC_PLANE_BYTES (32ull << 20)
#define PLAMO_HIP_STATIC_SCRATCH_BYTES ((64ull << 10) + (64ull << 20) + PLAMO_HIP_STATIC_PLANE_BYTES)
int plamo_hip_linear_static(struct plamo_metal *, const struct plamo_matmul *);
/* runtime/metal.h:86-88. Complete MLP branch on states[tokens, hidden]. */
int plamo_metal_mlp(struct plamo_metal *, const struct mlp *, float *states, uint64_t tokens);

#ifdef __cplusplus
}
#endif
#endif
