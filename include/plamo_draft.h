/* In-process speculative proposer for the MI355X backend.
 *
 * The reference engine speculates with a draft model that runs in a separate
 * worker process over a pipe (runtime/draft.c:70-168, the peer loop
 * runtime/worker.c:198-317). This library runs the draft model in the same
 * process, on the same GPU, through a second backend instance, behind the
 * reference's draft interface (runtime/draft.h:7-20): the engine's calls
 * (runtime/engine.c:316, 522-566) are unchanged.
 */
#ifndef PLAMO_DRAFT_H
#define PLAMO_DRAFT_H
#include <stdint.h>

#include "plamo_backend.h"
#include "plamo_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* runtime/draft.h:5. The magic tags the reference's draft-pipe frames; the
 * in-process proposer has no pipe and never sends one. */
enum { PLAMO_DRAFT_MAX = 16, PLAMO_DRAFT_MAGIC = 0x504c4431 };

struct plamo_draft;

/* runtime/draft.h:9. Returns the proposer installed with
 * plamo_hip_draft_install (ownership passes to the caller), or NULL when none
 * is installed or PLAMO_SPECULATIVE=0 (runtime/draft.c:95-98). */
struct plamo_draft *plamo_draft_open(void);
/* runtime/draft.h:10 */
void plamo_draft_close(struct plamo_draft *);
/* runtime/draft.h:11. Prefills the draft with the request's prompt; the text
 * is tokenized by the callback given to plamo_hip_draft_set_tokenizer (the
 * reference's peer tokenizes with its own engine). 1 ok, 0 failed. */
int plamo_draft_reset(struct plamo_draft *, const char *text, unsigned direction);
/* runtime/draft.h:12. ids[0] = first, then up to limit - 1 greedy draft
 * tokens (at most the current horizon; stops after EOS ids 1 or 16 and, when
 * enabled, at a low top-2 margin, runtime/worker.c:246-296). Returns the
 * count, 0 on failure. */
unsigned plamo_draft_propose(struct plamo_draft *, uint32_t first, unsigned limit, uint32_t *ids);
/* runtime/draft.h:13. The target consumed `consumed` of the proposed ids
 * (including ids[0]): the draft keeps exactly those in its cache
 * (runtime/worker.c:298-311) and updates its horizon (runtime/draft.c:196-211).
 * 1 ok, 0 failed. */
int plamo_draft_accept(struct plamo_draft *, unsigned consumed);

/* Host-side rollback of a model's KV rows (runtime/draft.h:15-20, semantics
 * of runtime/draft.c:213-296): a checkpoint saves the rows a bounded suffix of
 * `limit` steps could evict from a full sliding window; restore keeps
 * `accepted` of `processed` steps and marks rotations stale. The in-process
 * proposer uses it only when a sliding window was full; otherwise it rewinds
 * on the device (plamo_hip_rewind). */
struct plamo_draft_checkpoint;
struct plamo_draft_checkpoint *plamo_draft_checkpoint(struct model *, unsigned limit);
int plamo_draft_restore(struct plamo_draft_checkpoint *, unsigned processed, unsigned accepted);
void plamo_draft_checkpoint_free(struct plamo_draft_checkpoint *);

/* ---- no reference counterpart: the in-process proposer's setup ---------- */

/* Opens a proposer over `draft` (descriptors and host arrays borrowed until
 * close) with its own backend instance (config as plamo_metal_open; the
 * draft's weights are made resident). NULL on failure with a message. */
struct plamo_draft *plamo_hip_draft_open(struct model *draft,
                                         const struct plamo_metal_config *config, char *error,
                                         size_t cap);
/* Makes `draft` the proposer plamo_draft_open hands out next (once). */
void plamo_hip_draft_install(struct plamo_draft *draft);
/* Tokenizer for plamo_draft_reset: returns the id count (UINT64_MAX on
 * failure) and points *ids at ids valid until the next call. */
typedef uint64_t (*plamo_hip_tokenize_fn)(void *context, const char *text, unsigned direction,
                                          const uint32_t **ids);
void plamo_hip_draft_set_tokenizer(struct plamo_draft *, plamo_hip_tokenize_fn, void *context);
/* plamo_draft_reset with the prompt already tokenized. 1 ok, 0 failed. */
int plamo_hip_draft_reset_ids(struct plamo_draft *, const uint32_t *ids, uint64_t count);

struct plamo_hip_draft_stats {
    uint64_t proposals;        /* successful plamo_draft_propose calls */
    uint64_t proposed_tokens;  /* draft tokens proposed (ids[1..]) */
    uint64_t accepted_tokens;  /* of those, consumed by the target */
    uint64_t draft_steps;      /* draft forward steps */
    uint64_t device_rewinds;   /* rollbacks done on the device */
    uint64_t host_restores;    /* rollbacks through a host checkpoint */
    unsigned horizon;          /* current proposal horizon */
};
void plamo_hip_draft_get_stats(const struct plamo_draft *, struct plamo_hip_draft_stats *);

/* Horizon after an acceptance (runtime/draft.c:196-211): requested and
 * proposed of the last proposal, consumed by the target. */
unsigned plamo_hip_draft_next_horizon(unsigned horizon, unsigned requested, unsigned proposed,
                                      unsigned consumed);

/* The engine's decode loop (runtime/engine.c:514-566) over a target backend
 * whose prefill has just run (model->logits hold the first token's logits):
 * greedy tokens until max_tokens, EOS (ids 1 and 16) or a cancelling token
 * callback. With *draft set, each round proposes up to `block` tokens
 * (0 = PLAMO_SPECULATIVE_TOKENS or 16, runtime/engine.c:326-333), verifies
 * them in one batched target call and commits the agreeing prefix; the
 * draft is prefilled with `prompt` before its first proposal. A draft that
 * fails, or whose vocabulary differs from the target's, is closed and *draft
 * cleared, and decoding continues without it (runtime/engine.c:422-426).
 * Returns 1, or 0 with a message on a target failure. */
struct plamo_hip_decode_result {
    uint64_t completion_tokens, decode_steps;
    uint64_t speculative_batches, speculative_tokens, proposed_tokens, accepted_tokens;
    double draft_seconds, decode_seconds;
    unsigned finish; /* 0 length, 1 stop (EOS), 2 cancelled */
};
typedef int (*plamo_hip_token_fn)(uint32_t id, void *context); /* 0 cancels */
int plamo_hip_decode(struct plamo_metal *target, struct model *model, struct plamo_draft **draft,
                     const uint32_t *prompt, uint64_t prompt_tokens, unsigned max_tokens,
                     unsigned block, plamo_hip_token_fn token, void *context,
                     struct plamo_hip_decode_result *result, char *error, size_t cap);

/* Undoes the last `steps` decode steps of `model` on `m`: every layer's
 * cache count (and processed count, GQA tokens) drops by `steps` on the host
 * and on the device, without uploading rows. State and logits are left as
 * they are. 0 (nothing changed) when a layer has fewer rows or a sliding
 * window is full (its rows were shifted). */
int plamo_hip_rewind(struct plamo_metal *m, struct model *model, uint64_t steps);

/* The backend keeps the device KV authoritative during a request and finds
 * host edits between calls (prompt-prefix restore, request reset, a draft
 * restore, a CPU step) from the per-layer count, processed_count, scale_bits
 * and the first and last 16 values of the last K and V rows. A prefill that
 * starts on 1..64 cached rows (a restorable prompt prefix,
 * runtime/prompt_cache.h:8) uploads them whatever these show. A caller that
 * rewrites other rows while all of these stay unchanged calls this first:
 * every layer's host rows are then uploaded by the next call. No reference
 * counterpart (the reference shares the host arrays with its GPU,
 * runtime/metal_model.m:57-119). */
void plamo_hip_invalidate(struct plamo_metal *m);

#ifdef __cplusplus
}
#endif
#endif
