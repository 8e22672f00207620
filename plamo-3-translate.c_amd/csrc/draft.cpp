// In-process speculative proposer and the speculative decode loop.
//
// The reference speculates with a 0.8B draft model in a child process reached
// over pipes (runtime/draft.c:70-168), whose peer loop (runtime/worker.c:
// 198-317) prefills the prompt, proposes greedy tokens with a checkpoint of
// the KV rows a proposal could evict, and rolls back what the target did not
// consume. Here the draft model runs in the caller's process on its own
// backend instance (own stream, own HBM copies of the draft weights), so a
// proposal costs draft decode steps and nothing else. A rollback of rows
// still present lowers the counts on host and device (plamo_hip_rewind); only
// when a sliding window has shifted rows out does it fall back to the
// reference's host checkpoint, which the backend then re-uploads.
#include "../../include/plamo_backend.h"
#include "../../include/plamo_draft.h"
#include "../../include/plamo_model.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <new>
#include <vector>

namespace {

// Token ids the reference peer and engine treat as end of text
// (runtime/worker.c:246, runtime/engine.c:397).
bool is_eos(uint32_t id) { return id == 1 || id == 16; }

// Largest vocabulary the reference's draft protocol accepts
// (runtime/draft.c:162-163, 188-190).
constexpr uint32_t kProtocolVocab = 107520;

double now_seconds() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch())
        .count();
}

}  // namespace

// ---------------------------------------------------------------- host checkpoint
// runtime/draft.c:213-296: a checkpoint keeps, per layer, the count and the
// first min(count, limit) K and V rows: the rows a suffix of at most `limit`
// steps can shift out of a full sliding window.
struct plamo_draft_checkpoint {
    unsigned limit = 0;
    struct Saved {
        struct mixer *mixer;
        uint64_t count;
        std::vector<float> k, v;
    };
    std::vector<Saved> layers;
};

extern "C" {

void plamo_draft_checkpoint_free(struct plamo_draft_checkpoint *s) { delete s; }

struct plamo_draft_checkpoint *plamo_draft_checkpoint(struct model *model, unsigned limit) {
    if (!model || !limit || limit > PLAMO_DRAFT_MAX) return nullptr;
    auto *s = new (std::nothrow) struct plamo_draft_checkpoint();
    if (!s) return nullptr;
    s->limit = limit;
    try {
        s->layers.reserve(model->count);
        for (uint64_t i = 0; i < model->count; ++i) {
            struct mixer *mx = model->layers[i]->mixer;
            const struct cache *c = mx->cache;
            if (c->capacity < limit || c->count > c->capacity) {
                delete s;
                return nullptr;
            }
            uint64_t rows = c->count < limit ? c->count : limit;
            s->layers.push_back({mx, c->count, std::vector<float>(c->k, c->k + rows * c->width),
                                 std::vector<float>(c->v, c->v + rows * c->width)});
        }
    } catch (...) {
        delete s;
        return nullptr;
    }
    return s;
}

// Keeps `accepted` of the `processed` steps taken since the checkpoint. A
// layer that shifted rows out gets them back from the checkpoint; rotated keys
// are marked stale (processed_count 0), as runtime/draft.c:288-295 does.
int plamo_draft_restore(struct plamo_draft_checkpoint *s, unsigned processed, unsigned accepted) {
    if (!s || accepted > processed || processed > s->limit) return 0;
    struct Plan {
        uint64_t shifted, keep;  // rows to bring back, rows kept
    };
    std::vector<Plan> plan(s->layers.size());
    for (size_t i = 0; i < s->layers.size(); ++i) {
        const auto &l = s->layers[i];
        const struct cache *c = l.mixer->cache;
        uint64_t all = l.count + processed, want = l.count + accepted;
        uint64_t expect = all < c->capacity ? all : c->capacity;
        if ((!c->sliding && all > c->capacity) || c->count != expect) return 0;
        uint64_t lost = all > c->capacity ? all - c->capacity : 0;     // shifted out
        uint64_t gone = want > c->capacity ? want - c->capacity : 0;   // would be anyway
        uint64_t keep = want - gone, back = lost - gone;
        if (lost > l.k.size() / (c->width ? c->width : 1) || back > keep) return 0;
        plan[i] = {back, keep};
    }
    for (size_t i = 0; i < s->layers.size(); ++i) {
        const auto &l = s->layers[i];
        struct cache *c = l.mixer->cache;
        const uint64_t w = c->width, back = plan[i].shifted, keep = plan[i].keep;
        if (back) {
            // Rows [0, keep - back) of the kept window are the current rows
            // [0, keep - back) moved up by `back`; the first `back` rows come
            // from the checkpoint, starting where the kept window starts.
            uint64_t gone = l.count + accepted > c->capacity ? l.count + accepted - c->capacity : 0;
            memmove(c->k + back * w, c->k, (keep - back) * w * 4);
            memmove(c->v + back * w, c->v, (keep - back) * w * 4);
            memcpy(c->k, l.k.data() + gone * w, back * w * 4);
            memcpy(c->v, l.v.data() + gone * w, back * w * 4);
        }
        c->count = keep;
        l.mixer->rotation->processed_count = 0;
        l.mixer->rotation->scale_bits = 0;
        l.mixer->gqa->tokens = keep;
    }
    return 1;
}

}  // extern "C"

// ---------------------------------------------------------------- proposer
struct plamo_draft {
    struct model *model = nullptr;
    struct plamo_metal *backend = nullptr;
    // runtime/worker.c:199-212: optional confidence stop.
    float min_margin = 0.0f;
    unsigned min_tokens = 2;
    bool explicit_margin = false, explicit_minimum = false;
    // runtime/draft.c:16-20
    unsigned horizon = 8, requested = 0, proposed = 0;
    // The open proposal (runtime/worker.c:215-217).
    bool pending = false, broken = false;
    unsigned processed = 0;
    uint32_t ids[PLAMO_DRAFT_MAX] = {};
    struct plamo_draft_checkpoint *saved = nullptr;  // only when a sliding window may shift
    plamo_hip_tokenize_fn tokenize = nullptr;
    void *tokenize_context = nullptr;
    plamo_hip_draft_stats stats{};
};

namespace {

plamo_draft *installed = nullptr;

void drop_proposal(plamo_draft *d) {
    plamo_draft_checkpoint_free(d->saved);
    d->saved = nullptr;
    d->pending = false;
}

// One draft decode step; the draft's logits land in its host array.
bool draft_step(plamo_draft *d, uint32_t id) {
    if (plamo_metal_forward(d->backend, d->model, id) != 1) return false;
    ++d->stats.draft_steps;
    return true;
}

bool parse_settings(plamo_draft *d, char *error, size_t cap) {
    // runtime/worker.c:199-210: malformed settings refuse to start the peer.
    if (const char *s = getenv("PLAMO_DRAFT_MIN_MARGIN")) {
        char *end = nullptr;
        float v = strtof(s, &end);
        if (!*s || *end || !isfinite(v) || v < 0) {
            if (error && cap) snprintf(error, cap, "invalid PLAMO_DRAFT_MIN_MARGIN");
            return false;
        }
        d->min_margin = v;
        d->explicit_margin = true;
    }
    if (const char *s = getenv("PLAMO_DRAFT_MIN_TOKENS")) {
        char *end = nullptr;
        unsigned long v = strtoul(s, &end, 10);
        if (!*s || *end || v < 1 || v > PLAMO_DRAFT_MAX) {
            if (error && cap) snprintf(error, cap, "invalid PLAMO_DRAFT_MIN_TOKENS");
            return false;
        }
        d->min_tokens = (unsigned)v;
        d->explicit_minimum = true;
    }
    return true;
}

}  // namespace

extern "C" {

unsigned plamo_hip_draft_next_horizon(unsigned horizon, unsigned requested, unsigned proposed,
                                      unsigned consumed) {
    // runtime/draft.c:199-210: a first-token rejection drops to two-token
    // blocks; any shortfall returns to eight; full acceptance doubles up to
    // eight, then jumps to the maximum.
    if (consumed == 1 && proposed > 1) return 2;
    if (consumed < proposed || proposed < requested) return 8;
    if (horizon < 8) return horizon * 2;
    return PLAMO_DRAFT_MAX;
}

struct plamo_draft *plamo_hip_draft_open(struct model *draft,
                                         const struct plamo_metal_config *config, char *error,
                                         size_t cap) {
    if (!draft || !draft->count || !draft->vocab) {
        if (error && cap) snprintf(error, cap, "no draft model");
        return nullptr;
    }
    auto *d = new (std::nothrow) plamo_draft();
    if (!d) {
        if (error && cap) snprintf(error, cap, "out of memory");
        return nullptr;
    }
    d->model = draft;
    if (!parse_settings(d, error, cap)) {
        delete d;
        return nullptr;
    }
    d->backend = plamo_metal_open(config, error, cap);
    if (!d->backend) {
        delete d;
        return nullptr;
    }
    // runtime/draft.c:148-150: the peer keeps every projection resident.
    if (!plamo_metal_prepare_model(d->backend, draft) || !plamo_metal_warm_cache(d->backend)) {
        if (error && cap) {
            struct plamo_metal_info info;
            plamo_metal_get_info(d->backend, &info);
            snprintf(error, cap, "draft model rejected: %s", info.note);
        }
        plamo_metal_close(d->backend);
        delete d;
        return nullptr;
    }
    d->stats.horizon = d->horizon;
    return d;
}

void plamo_hip_draft_install(struct plamo_draft *draft) {
    if (installed && installed != draft) plamo_draft_close(installed);
    installed = draft;
}

struct plamo_draft *plamo_draft_open(void) {
    // runtime/draft.c:95-98
    const char *enabled = getenv("PLAMO_SPECULATIVE");
    if (enabled && !strcmp(enabled, "0")) return nullptr;
    plamo_draft *d = installed;
    installed = nullptr;
    return d;
}

void plamo_draft_close(struct plamo_draft *d) {
    if (!d) return;
    if (installed == d) installed = nullptr;
    drop_proposal(d);
    plamo_metal_close(d->backend);
    delete d;
}

void plamo_hip_draft_set_tokenizer(struct plamo_draft *d, plamo_hip_tokenize_fn fn,
                                   void *context) {
    if (!d) return;
    d->tokenize = fn;
    d->tokenize_context = context;
}

int plamo_hip_draft_reset_ids(struct plamo_draft *d, const uint32_t *ids, uint64_t count) {
    if (!d || d->broken || !ids || !count) return 0;
    for (uint64_t i = 0; i < count; ++i)
        if (ids[i] >= d->model->vocab) return 0;
    drop_proposal(d);
    // runtime/engine.c:46-55, then the prompt's prefill (runtime/worker.c:
    // 229-236 translates with max_tokens 1: prefill only).
    struct model *m = d->model;
    for (uint64_t i = 0; i < m->count; ++i) {
        struct layer *l = m->layers[i];
        l->state = m->state;
        l->mixer->cache->count = 0;
        l->mixer->rotation->processed_count = 0;
        l->mixer->rotation->scale_bits = 0;
        l->mixer->gqa->tokens = 0;
    }
    if (plamo_metal_prefill(d->backend, m, ids, count, nullptr) != 1) {
        d->broken = true;
        return 0;
    }
    // runtime/draft.c:173-176
    d->horizon = 8;
    d->requested = d->proposed = 0;
    d->stats.horizon = d->horizon;
    return 1;
}

int plamo_draft_reset(struct plamo_draft *d, const char *text, unsigned direction) {
    // runtime/worker.c:229: direction 0..2, at most 16384 bytes of text.
    if (!d || !d->tokenize || !text || direction > 2 || strlen(text) > 16384) return 0;
    const uint32_t *ids = nullptr;
    uint64_t n = d->tokenize(d->tokenize_context, text, direction, &ids);
    if (n == UINT64_MAX || !ids) return 0;
    return plamo_hip_draft_reset_ids(d, ids, n);
}

unsigned plamo_draft_propose(struct plamo_draft *d, uint32_t first, unsigned limit,
                             uint32_t *ids) {
    // runtime/draft.c:179-194 and runtime/worker.c:237-296.
    if (!d || d->broken || !ids || !limit || limit > PLAMO_DRAFT_MAX || d->pending) return 0;
    struct model *m = d->model;
    if (first >= m->vocab || first >= kProtocolVocab) return 0;
    if (limit > d->horizon) limit = d->horizon;
    // Longer blocks pay off only while the draft stays confident
    // (runtime/worker.c:239-243).
    float margin = !d->explicit_margin && limit > 8 ? 1.0f : d->min_margin;
    unsigned minimum = !d->explicit_minimum && limit > 8 ? 8 : d->min_tokens;
    // A device rewind needs every row a rollback keeps still in place: true
    // unless a sliding window can shift during this proposal.
    bool may_shift = false;
    for (uint64_t i = 0; i < m->count; ++i) {
        const struct cache *c = m->layers[i]->mixer->cache;
        if (c->sliding && c->count + limit > c->capacity) may_shift = true;
    }
    if (may_shift && !(d->saved = plamo_draft_checkpoint(m, limit))) return 0;
    d->pending = true;
    d->processed = 0;
    unsigned count = 1;
    d->ids[0] = first;
    float confidence = INFINITY;
    while (count < limit && !is_eos(d->ids[count - 1])) {
        if (margin > 0 && count >= minimum && confidence < margin) break;
        if (!draft_step(d, d->ids[count - 1])) {
            d->broken = true;
            return 0;
        }
        ++d->processed;
        uint64_t id = plamo_argmax(m->logits, m->vocab);
        if (id >= m->vocab || id >= kProtocolVocab) {
            d->broken = true;
            return 0;
        }
        if (margin > 0) {
            float best = m->logits[id];
            m->logits[id] = -INFINITY;
            uint64_t second = plamo_argmax(m->logits, m->vocab);
            m->logits[id] = best;
            float gap = second < m->vocab ? best - m->logits[second] : INFINITY;
            if (gap < confidence) confidence = gap;
            if (count >= minimum && confidence < margin) break;
        }
        d->ids[count++] = (uint32_t)id;
    }
    d->requested = limit;
    d->proposed = count;
    memcpy(ids, d->ids, count * sizeof *ids);
    ++d->stats.proposals;
    d->stats.proposed_tokens += count - 1;
    return count;
}

int plamo_draft_accept(struct plamo_draft *d, unsigned consumed) {
    // runtime/worker.c:298-311, then runtime/draft.c:196-211.
    if (!d || d->broken || !d->pending || consumed > d->proposed) return 0;
    bool ok = true;
    if (consumed < d->processed) {
        unsigned undo = d->processed - consumed;
        if (!d->saved && plamo_hip_rewind(d->backend, d->model, undo)) {
            ++d->stats.device_rewinds;
        } else if (d->saved && plamo_draft_restore(d->saved, d->processed, consumed)) {
            ++d->stats.host_restores;
        } else {
            ok = false;
        }
    } else if (consumed == d->processed + 1) {
        ok = draft_step(d, d->ids[d->processed]);
    }
    drop_proposal(d);
    if (!ok) {
        d->broken = true;
        return 0;
    }
    d->horizon = plamo_hip_draft_next_horizon(d->horizon, d->requested, d->proposed, consumed);
    d->stats.horizon = d->horizon;
    d->stats.accepted_tokens += consumed ? consumed - 1 : 0;
    return 1;
}

void plamo_hip_draft_get_stats(const struct plamo_draft *d, struct plamo_hip_draft_stats *out) {
    if (!out) return;
    if (!d) {
        memset(out, 0, sizeof *out);
        return;
    }
    *out = d->stats;
}

// ---------------------------------------------------------------- decode loop
int plamo_hip_decode(struct plamo_metal *target, struct model *model, struct plamo_draft **draft,
                     const uint32_t *prompt, uint64_t prompt_tokens, unsigned max_tokens,
                     unsigned block, plamo_hip_token_fn token, void *context,
                     struct plamo_hip_decode_result *r, char *error, size_t cap) {
    if (!target || !model || !r || !max_tokens) {
        if (error && cap) snprintf(error, cap, "invalid decode request");
        return 0;
    }
    memset(r, 0, sizeof *r);
    if (!block) {
        // runtime/engine.c:326-333
        block = PLAMO_VERIFY_MAX;
        if (const char *s = getenv("PLAMO_SPECULATIVE_TOKENS")) {
            char *end = nullptr;
            unsigned long v = strtoul(s, &end, 10);
            if (!*end && v >= 2 && v <= PLAMO_VERIFY_MAX) block = (unsigned)v;
        }
    }
    if (block > PLAMO_VERIFY_MAX) block = PLAMO_VERIFY_MAX;
    auto disable = [&]() {
        plamo_draft_close(*draft);
        *draft = nullptr;
    };
    // Token ids must mean the same text to both models.
    if (draft && *draft && (*draft)->model->vocab != model->vocab) disable();
    bool speculate = draft && *draft && max_tokens > 1 && block >= 2 && prompt && prompt_tokens;
    bool draft_ready = false;
    // runtime/engine.c:395-420 without the text: EOS stops, the callback
    // may cancel.
    auto emit = [&](uint32_t id) -> int {
        if (is_eos(id)) {
            r->finish = 1;
            return 0;
        }
        if (id >= model->vocab) {
            if (error && cap) snprintf(error, cap, "invalid generated token");
            return -1;
        }
        if (token && !token(id, context)) {
            r->finish = 2;
            return 0;
        }
        ++r->completion_tokens;
        return 1;
    };
    double start = now_seconds();
    while (r->completion_tokens < max_tokens) {
        uint64_t best = plamo_argmax(model->logits, model->vocab);
        uint32_t id = best < model->vocab ? (uint32_t)best : UINT32_MAX;
        int emitted = emit(id);
        if (emitted < 0) return 0;
        if (!emitted || r->completion_tokens == max_tokens) break;
        if (speculate) {
            unsigned limit = max_tokens - (unsigned)r->completion_tokens;
            if (limit > block) limit = block;
            uint32_t proposed[PLAMO_VERIFY_MAX], next[PLAMO_VERIFY_MAX];
            double t0 = now_seconds();
            if (!draft_ready) draft_ready = plamo_hip_draft_reset_ids(*draft, prompt, prompt_tokens);
            unsigned n = draft_ready ? plamo_draft_propose(*draft, id, limit, proposed) : 0;
            r->draft_seconds += now_seconds() - t0;
            if (!n) {
                disable();
                speculate = false;
            } else {
                int verified = plamo_metal_verify(target, model, proposed, n, next);
                if (verified < 0) {
                    if (error && cap) snprintf(error, cap, "candidate verification failed");
                    return 0;
                }
                if (verified) {
                    ++r->speculative_batches;
                    r->proposed_tokens += n - 1;
                    unsigned consumed = 0;
                    bool stop = false;
                    for (unsigned j = 0; j < n; ++j) {
                        if (j) {
                            if (proposed[j] != next[j - 1]) break;
                            emitted = emit(proposed[j]);
                            if (emitted < 0) return 0;
                            if (!emitted) {
                                stop = true;
                                break;
                            }
                        }
                        if (plamo_metal_commit(target, model, j) != 1) {
                            if (error && cap) snprintf(error, cap, "candidate commit failed");
                            return 0;
                        }
                        ++consumed;
                        ++r->decode_steps;
                    }
                    r->speculative_tokens += consumed;
                    r->accepted_tokens += consumed ? consumed - 1 : 0;
                    t0 = now_seconds();
                    if (!plamo_draft_accept(*draft, consumed)) {
                        disable();
                        speculate = false;
                    }
                    r->draft_seconds += now_seconds() - t0;
                    if (stop) break;
                    continue;
                }
                // Verification declined: nothing changed on the target.
                disable();
                speculate = false;
            }
        }
        if (plamo_metal_forward(target, model, id) != 1) {
            if (error && cap) snprintf(error, cap, "decode failed");
            return 0;
        }
        ++r->decode_steps;
    }
    r->decode_seconds = now_seconds() - start;
    return 1;
}

}  // extern "C"
