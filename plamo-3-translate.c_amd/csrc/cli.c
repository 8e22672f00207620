/* plamo-hip: a Linux command-line host for the MI355X backend.
 *
 * The reference's CLI (runtime/cli.c) tokenizes a text, opens its engine
 * (runtime/engine.c:125-333: model globals from plamo_model_open, the Metal
 * backend, an optional draft) and streams greedy tokens. This host does the
 * same through the library's C boundary only: plamo_model_open over a
 * checkpoint directory (src/model_open.s), plamo_metal_open /
 * plamo_metal_prepare_model / plamo_metal_prefill (runtime/metal.h), and the
 * engine's decode loop with optional in-process speculative decoding
 * (plamo_hip_decode, runtime/engine.c:514-566). Prompts are token ids: the
 * engine's tokenizer (runtime/tokenizer.c) is not part of this build.
 *
 * Exit status as the reference's (runtime/cli.c:129-141): 0 done, 1 failure
 * (or a cancelled stream), 2 usage error.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../../include/plamo_backend.h"
#include "../../include/plamo_checkpoint.h"
#include "../../include/plamo_draft.h"
#include "../../include/plamo_model.h"
#include "../../include/plamo_synthetic.h"

enum { MAX_PROMPT = 8192 };

static void usage(FILE *out) {
    fprintf(out,
            "usage: plamo-hip [--model DIR] [--draft DIR] [--max-tokens 1..4096]\n"
            "                 [--speculative-tokens 1..16] [--] IDS...\n"
            "  IDS          prompt token ids, decimal, separated by spaces or commas\n"
            "  --model      checkpoint directory (config.json, *.safetensors);\n"
            "               default $PLAMO_MODEL_DIR\n"
            "  --draft      a second checkpoint that proposes tokens in process\n"
            "               (speculative decoding; output identical to greedy)\n"
            "  Prints the generated token ids. Greedy decoding on an MI355X: FP32\n"
            "  activations and arithmetic, original BF16 weights.\n");
}

/* A decimal count in 1..limit without sign or leading zero. */
static int count(const char *text, unsigned limit, unsigned *out) {
    char *end;
    errno = 0;
    unsigned long v = strtoul(text, &end, 10);
    if (errno || text[0] < '1' || text[0] > '9' || *end || v > limit) return 0;
    *out = (unsigned)v;
    return 1;
}

/* Appends the comma-separated ids of one argument. 0 on a malformed id. */
static int parse_ids(const char *text, uint32_t *ids, uint64_t *n) {
    const char *p = text;
    while (*p) {
        if (*p == ',') {
            ++p;
            continue;
        }
        if (*p < '0' || *p > '9') return 0;
        char *end;
        errno = 0;
        unsigned long long v = strtoull(p, &end, 10);
        if (errno || v > UINT32_MAX || (*end && *end != ',') || *n >= MAX_PROMPT) return 0;
        ids[(*n)++] = (uint32_t)v;
        p = end;
    }
    return 1;
}

static int print_token(uint32_t id, void *context) {
    (void)context;
    return printf("%" PRIu32 " ", id) > 0 && !fflush(stdout);
}

static double now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

int main(int argc, char **argv) {
    const char *model_dir = NULL, *draft_dir = NULL;
    unsigned max_tokens = 256, block = 0;
    static uint32_t ids[MAX_PROMPT];
    uint64_t n = 0;
    int separator = 0;
    for (int i = 1; i < argc; ++i) {
        const char *arg = argv[i];
        if (!separator && (!strcmp(arg, "--help") || !strcmp(arg, "-h"))) {
            usage(stdout);
            return 0;
        }
        if (!separator && !strcmp(arg, "--")) {
            separator = 1;
            continue;
        }
        if (!separator && arg[0] == '-' && arg[1] == '-') {
            if (++i == argc) goto invalid;
            const char *value = argv[i];
            if (!strcmp(arg, "--model"))
                model_dir = value;
            else if (!strcmp(arg, "--draft"))
                draft_dir = value;
            else if (!strcmp(arg, "--max-tokens")) {
                if (!count(value, 4096, &max_tokens)) goto invalid;
            } else if (!strcmp(arg, "--speculative-tokens")) {
                if (!count(value, PLAMO_VERIFY_MAX, &block)) goto invalid;
            } else
                goto invalid;
            continue;
        }
        if (!parse_ids(arg, ids, &n)) goto invalid;
    }
    if (!n) {
        usage(argc == 1 ? stdout : stderr);
        return argc == 1 ? 0 : 2;
    }

    char error[512];
    if (model_dir && !plamo_model_set_directory(model_dir)) {
        fprintf(stderr, "plamo-hip: model directory path too long\n");
        return 1;
    }
    if (!model_dir && !getenv("PLAMO_MODEL_DIR")) {
        fprintf(stderr, "plamo-hip: no model: pass --model DIR or set PLAMO_MODEL_DIR\n");
        return 1;
    }
    double t0 = now();
    if (!plamo_model_open()) return 1; /* the binder reported why */
    for (uint64_t i = 0; i < n; ++i)
        if (ids[i] >= plamo_model.vocab) {
            fprintf(stderr, "plamo-hip: token id %" PRIu32 " is outside the vocabulary (%" PRIu64 ")\n",
                    ids[i], plamo_model.vocab);
            return 2;
        }
    struct plamo_metal_config config;
    memset(&config, 0, sizeof config);
    config.maps = plamo_weight_mappings;
    config.fds = plamo_weight_fds;
    config.count = plamo_weight_mapping_count;
    config.schema = plamo_weight_schema;
    struct plamo_metal *gpu = plamo_metal_open(&config, error, sizeof error);
    if (!gpu) {
        fprintf(stderr, "plamo-hip: %s\n", error);
        return 1;
    }
    int status = 1;
    struct plamo_checkpoint *draft_ck = NULL;
    struct plamo_synthetic_instance *draft_model = NULL;
    struct plamo_draft *draft = NULL;
    if (plamo_metal_prepare_model(gpu, &plamo_model) != 1) {
        fprintf(stderr, "plamo-hip: cannot make the weights resident\n");
        goto done;
    }
    if (draft_dir) {
        draft_ck = plamo_checkpoint_open(draft_dir, 0, error, sizeof error);
        if (draft_ck) draft_model = plamo_checkpoint_instantiate(draft_ck, 1, error, sizeof error);
        if (draft_model) {
            struct plamo_metal_config dc;
            size_t maps = 0;
            memset(&dc, 0, sizeof dc);
            dc.maps = plamo_checkpoint_mappings(draft_ck, &maps);
            dc.count = maps;
            dc.schema = plamo_checkpoint_schema(draft_ck);
            draft = plamo_hip_draft_open(plamo_synthetic_model(draft_model), &dc, error,
                                         sizeof error);
        }
        if (!draft) {
            fprintf(stderr, "plamo-hip: draft: %s\n", error);
            goto done;
        }
    }
    double load = now() - t0;
    t0 = now();
    int r = plamo_metal_prefill(gpu, &plamo_model, ids, n, NULL);
    if (r != 1) {
        fprintf(stderr, "plamo-hip: prefill %s\n", r ? "failed" : "declined");
        goto done;
    }
    double prefill = now() - t0;
    struct plamo_hip_decode_result result;
    if (!plamo_hip_decode(gpu, &plamo_model, &draft, ids, n, max_tokens, block, print_token, NULL,
                          &result, error, sizeof error)) {
        fprintf(stderr, "plamo-hip: %s\n", error);
        goto done;
    }
    if (putchar('\n') == EOF || fflush(stdout)) goto done;
    fprintf(stderr,
            "plamo-hip: %" PRIu64 " prompt tokens, %" PRIu64 " completion tokens (%s); load %.2f s, "
            "prefill %.2f ms, decode %.2f tok/s",
            n, result.completion_tokens,
            result.finish == 1 ? "stop" : result.finish == 2 ? "cancelled" : "length", load,
            prefill * 1e3,
            result.decode_seconds > 0 ? result.completion_tokens / result.decode_seconds : 0.0);
    if (draft_dir)
        fprintf(stderr, "; speculative %" PRIu64 " batches, %" PRIu64 " proposed, %" PRIu64 " accepted",
                result.speculative_batches, result.proposed_tokens, result.accepted_tokens);
    fputc('\n', stderr);
    status = result.finish == 2 || ferror(stdout);
done:
    if (draft) plamo_draft_close(draft);
    if (draft_model) plamo_synthetic_release(draft_model);
    if (draft_ck) plamo_checkpoint_close(draft_ck);
    plamo_metal_close(gpu);
    return status;
invalid:
    usage(stderr);
    return 2;
}
