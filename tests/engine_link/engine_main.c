/* A host program over the reference's engine (runtime/engine.h), linked with
 * runtime/engine.c and runtime/prompt_cache.c compiled from the reference and
 * libplamo_hip.so as its GPU backend. Test infrastructure only.
 *
 *   engine_host tokenize <direction> <text>
 *       tokenizer-only engine (no model, no GPU): prints the prompt ids.
 *   engine_host translate <direction> <max_tokens> <text>
 *       opens the model of $PLAMO_MODEL_DIR with the GPU backend and resident
 *       weights, prepares it (fixed prefixes captured), translates, and prints
 *       one JSON line: prompt ids, generated ids, cached prompt tokens, finish
 *       reason, decode steps and the backend's counters. With
 *       $ENGINE_HOST_DUMP set, it also writes the model's final logits and
 *       state there (raw float32, logits first).
 * Exit status 0 on success; 1 with the engine's error on stderr.
 */
#include "engine.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

struct collected {
    uint32_t ids[4096];
    unsigned count;
};

static int on_token(uint32_t id, const char *bytes, size_t count, void *context) {
    (void)bytes, (void)count;
    struct collected *c = context;
    if (c->count < sizeof c->ids / sizeof c->ids[0])
        c->ids[c->count++] = id;
    return 1;
}

static void print_ids(const char *key, const uint32_t *ids, uint64_t n) {
    printf("\"%s\": [", key);
    for (uint64_t i = 0; i < n; ++i)
        printf(i ? ", %u" : "%u", ids[i]);
    printf("]");
}

int main(int argc, char **argv) {
    char error[512] = {0};
    struct plamo_engine_info info;
    if (argc == 4 && !strcmp(argv[1], "tokenize")) {
        struct plamo_engine *e = plamo_engine_open(PLAMO_MEMORY_AUTO, 1, 0, PLAMO_BACKEND_CPU,
                                                   &info, error, sizeof error);
        if (!e) {
            fprintf(stderr, "%s\n", error);
            return 1;
        }
        const uint32_t *ids;
        uint64_t n = plamo_engine_tokenize(e, argv[3], (unsigned)atoi(argv[2]), &ids, error,
                                           sizeof error);
        if (n == UINT64_MAX) {
            fprintf(stderr, "%s\n", error);
            return 1;
        }
        printf("{\"memory_mode\": \"%s\", ", info.memory_mode);
        print_ids("ids", ids, n);
        printf("}\n");
        return 0;
    }
    if (argc != 5 || strcmp(argv[1], "translate")) {
        fprintf(stderr, "usage: engine_host tokenize <direction> <text>\n"
                        "       engine_host translate <direction> <max_tokens> <text>\n");
        return 2;
    }
    const unsigned direction = (unsigned)atoi(argv[2]), max_tokens = (unsigned)atoi(argv[3]);
    struct plamo_engine *e = plamo_engine_open(PLAMO_MEMORY_RESIDENT, 0, 0, PLAMO_BACKEND_METAL,
                                               &info, error, sizeof error);
    if (!e) {
        fprintf(stderr, "%s\n", error);
        return 1;
    }
    if (!plamo_engine_prepare(e, error, sizeof error)) {
        fprintf(stderr, "%s\n", error);
        return 1;
    }
    const uint32_t *borrowed;
    uint64_t n = plamo_engine_tokenize(e, argv[4], direction, &borrowed, error, sizeof error);
    if (n == UINT64_MAX || n > 4096) {
        fprintf(stderr, "%s\n", error);
        return 1;
    }
    uint32_t *prompt = malloc((size_t)(n ? n : 1) * sizeof *prompt);
    struct collected *out = calloc(1, sizeof *out);
    if (!prompt || !out)
        return 1;
    memcpy(prompt, borrowed, (size_t)n * sizeof *prompt);
    struct plamo_callbacks cb = {NULL, on_token, out};
    struct plamo_result r;
    if (!plamo_engine_translate(e, argv[4], direction, max_tokens, &cb, &r, error,
                                sizeof error)) {
        fprintf(stderr, "%s\n", error);
        return 1;
    }
    const char *dump = getenv("ENGINE_HOST_DUMP");
    if (dump) {
        FILE *f = fopen(dump, "wb");
        if (!f || fwrite(plamo_model.logits, 4, plamo_model.vocab, f) != plamo_model.vocab ||
            fwrite(plamo_model.state, 4, plamo_model.hidden, f) != plamo_model.hidden ||
            fclose(f)) {
            fprintf(stderr, "cannot write %s\n", dump);
            return 1;
        }
    }
    plamo_engine_get_info(e, &info);
    printf("{\"backend\": \"%s\", \"memory_mode\": \"%s\", ", info.backend, info.memory_mode);
    print_ids("prompt", prompt, n);
    printf(", ");
    print_ids("generated", out->ids, out->count);
    printf(", \"prefix_tokens\": [%llu, %llu], \"cached_prompt_tokens\": %llu, "
           "\"finish_reason\": \"%s\", \"decode_steps\": %llu, \"completion_tokens\": %llu, "
           "\"cpu_fallbacks\": %llu, \"errors\": %llu, \"fused_decodes\": %llu, "
           "\"fused_prefills\": %llu, \"device\": \"%s\"}\n",
           (unsigned long long)info.prefix_tokens[0], (unsigned long long)info.prefix_tokens[1],
           (unsigned long long)r.cached_prompt_tokens, r.finish_reason,
           (unsigned long long)r.decode_steps, (unsigned long long)r.completion_tokens,
           (unsigned long long)info.gpu.cpu_fallbacks, (unsigned long long)info.gpu.errors,
           (unsigned long long)info.gpu.fused_decodes, (unsigned long long)info.gpu.fused_prefills,
           info.gpu.device);
    free(prompt);
    free(out);
    return 0;
}
