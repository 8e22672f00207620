/* plamo-hip: a Linux host for the MI355X backend, one-shot or as a worker.
 *
 * The reference's CLI (runtime/cli.c) tokenizes a text, opens its engine
 * (runtime/engine.c:125-333: model globals from plamo_model_open, the Metal
 * backend, an optional draft) and streams greedy tokens; its persistent worker
 * (runtime/worker.c) serves binary request frames with JSONL events. This host
 * does both through the library's C boundary only: plamo_model_open over a
 * checkpoint directory (src/model_open.s), plamo_metal_open /
 * plamo_metal_prepare_model / plamo_metal_prefill (runtime/metal.h), and the
 * engine's decode loop with optional in-process speculative decoding
 * (plamo_hip_decode, runtime/engine.c:514-566). Prompts are token ids: the
 * engine's tokenizer (runtime/tokenizer.c over AArch64 assembly) is not part
 * of this build.
 *
 * One-shot: prints the generated ids. Exit status as the reference's
 * (runtime/cli.c:129-141): 0 done, 1 failure (or a cancelled stream), 2 usage.
 *
 * --worker: the reference worker's protocol (runtime/worker.c:1-4, 427-489).
 * A request is four little-endian u32 {op, direction, max_tokens, text_bytes}
 * followed by exactly text_bytes of UTF-8 (at most 16384): op 1 generates,
 * op 2 tokenizes, op 3 with the other fields zero cancels the running
 * generation (ignored when idle). The text is the prompt's decimal token ids
 * separated by spaces, commas or newlines. Events are JSON lines on stdout:
 * "ready" once the model is resident, then per request "prefill", "token"
 * (token_id; hex is empty without a tokenizer) and "done", or "tokenized", or
 * "error" {code: protocol_error | invalid_input | inference_failed}. End of
 * input ends the worker with status 0; a malformed frame ends it with 1.
 */
#define _POSIX_C_SOURCE 200809L
#include <errno.h>
#include <inttypes.h>
#include <poll.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/resource.h>
#include <time.h>
#include <unistd.h>

#include "../../include/plamo_backend.h"
#include "../../include/plamo_checkpoint.h"
#include "../../include/plamo_draft.h"
#include "../../include/plamo_model.h"
#include "../../include/plamo_synthetic.h"

enum { MAX_PROMPT = 8192, MAX_FRAME_TEXT = 16384 };

static void usage(FILE *out) {
    fprintf(out,
            "usage: plamo-hip [--model DIR] [--draft DIR] [--max-tokens 1..4096]\n"
            "                 [--speculative-tokens 1..16] [--] IDS...\n"
            "       plamo-hip --worker [--model DIR] [--draft DIR] [--speculative-tokens 1..16]\n"
            "  IDS          prompt token ids, decimal, separated by spaces or commas\n"
            "  --model      checkpoint directory (config.json, *.safetensors);\n"
            "               default $PLAMO_MODEL_DIR\n"
            "  --draft      a second checkpoint that proposes tokens in process\n"
            "               (speculative decoding; output identical to greedy)\n"
            "  --worker     serve binary request frames on stdin, JSON events on stdout\n"
            "  Prints the generated token ids. Greedy decoding on an MI355X: FP32\n"
            "  activations and arithmetic, original BF16 weights.\n");
}

/* A whole decimal number 1..limit: digits only, first digit not 0. */
static int parse_count(const char *text, unsigned limit, unsigned *out) {
    uint64_t value = 0;
    if (*text < '1' || *text > '9')
        return 0;
    for (const char *p = text; *p; ++p) {
        if (*p < '0' || *p > '9')
            return 0;
        value = value * 10 + (uint64_t)(*p - '0');
        if (value > limit)
            return 0;
    }
    *out = (unsigned)value;
    return 1;
}

static int is_separator(char c) { return c == ',' || c == ' ' || c == '\t' || c == '\n' || c == '\r'; }

/* Appends the ids of [text, end): decimal ids between separators. 0 on a
 * malformed id or when more than MAX_PROMPT ids are given. */
static int parse_ids(const char *text, const char *end, uint32_t *ids, uint64_t *n) {
    const char *p = text;
    while (p < end) {
        if (is_separator(*p)) {
            ++p;
            continue;
        }
        uint64_t value = 0;
        const char *start = p;
        for (; p < end && !is_separator(*p); ++p) {
            if (*p < '0' || *p > '9' || p - start > 10)
                return 0;
            value = value * 10 + (uint64_t)(*p - '0');
        }
        if (value > UINT32_MAX || *n >= MAX_PROMPT)
            return 0;
        ids[(*n)++] = (uint32_t)value;
    }
    return 1;
}

static double now(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

/* ---- the model, the backend and the optional draft ---- */

struct host {
    struct plamo_metal *gpu;
    struct plamo_checkpoint *draft_ck;
    struct plamo_synthetic_instance *draft_model;
    struct plamo_draft *draft;
    unsigned block;
    double load_seconds, preload_seconds;
};

static void host_close(struct host *h) {
    if (h->draft)
        plamo_draft_close(h->draft);
    if (h->draft_model)
        plamo_synthetic_release(h->draft_model);
    if (h->draft_ck)
        plamo_checkpoint_close(h->draft_ck);
    if (h->gpu)
        plamo_metal_close(h->gpu);
    memset(h, 0, sizeof *h);
}

/* 1 with the model resident on the GPU; 0 with a message. */
static int host_open(struct host *h, const char *draft_dir, char *error, size_t cap) {
    double t0 = now();
    if (!plamo_model_open()) {
        snprintf(error, cap, "cannot open the model (see the message above)");
        return 0;
    }
    struct plamo_metal_config config;
    memset(&config, 0, sizeof config);
    config.memory = PLAMO_METAL_RESIDENT;
    config.maps = plamo_weight_mappings;
    config.fds = plamo_weight_fds;
    config.count = plamo_weight_mapping_count;
    config.schema = plamo_weight_schema;
    h->gpu = plamo_metal_open(&config, error, cap);
    if (!h->gpu)
        return 0;
    h->load_seconds = now() - t0;
    t0 = now();
    if (plamo_metal_prepare_model(h->gpu, &plamo_model) != 1) {
        snprintf(error, cap, "cannot make the weights resident");
        return 0;
    }
    if (draft_dir) {
        char why[512] = "cannot open the draft";
        h->draft_ck = plamo_checkpoint_open(draft_dir, 0, why, sizeof why);
        if (h->draft_ck)
            h->draft_model = plamo_checkpoint_instantiate(h->draft_ck, 1, why, sizeof why);
        if (h->draft_model) {
            struct plamo_metal_config dc;
            size_t maps = 0;
            memset(&dc, 0, sizeof dc);
            dc.maps = plamo_checkpoint_mappings(h->draft_ck, &maps);
            dc.count = maps;
            dc.schema = plamo_checkpoint_schema(h->draft_ck);
            h->draft =
                plamo_hip_draft_open(plamo_synthetic_model(h->draft_model), &dc, why, sizeof why);
        }
        if (!h->draft) {
            snprintf(error, cap, "draft: %s", why);
            return 0;
        }
    }
    h->preload_seconds = now() - t0;
    h->load_seconds += h->preload_seconds;
    return 1;
}

/* Counts and rotation bookkeeping back to zero, as the engine does before
 * every request (runtime/engine.c:46-55); the backend sees the host edit. */
static void reset_request(struct model *m) {
    for (uint64_t i = 0; i < m->count; ++i) {
        struct layer *l = m->layers[i];
        l->state = m->state;
        l->mixer->cache->count = 0;
        l->mixer->rotation->processed_count = 0;
        l->mixer->rotation->scale_bits = 0;
        l->mixer->gqa->tokens = 0;
    }
}

static const char *finish_name(unsigned finish) {
    return finish == 1 ? "stop" : finish == 2 ? "cancelled" : "length";
}

/* ---- one-shot ---- */

static int print_token(uint32_t id, void *context) {
    (void)context;
    return printf("%" PRIu32 " ", id) > 0 && !fflush(stdout);
}

static int one_shot(struct host *h, const uint32_t *ids, uint64_t n, unsigned max_tokens,
                    int speculative) {
    char error[512];
    double t0 = now();
    int r = plamo_metal_prefill(h->gpu, &plamo_model, ids, n, NULL);
    if (r != 1) {
        fprintf(stderr, "plamo-hip: prefill %s\n", r ? "failed" : "declined");
        return 1;
    }
    double prefill = now() - t0;
    struct plamo_hip_decode_result result;
    if (!plamo_hip_decode(h->gpu, &plamo_model, &h->draft, ids, n, max_tokens, h->block,
                          print_token, NULL, &result, error, sizeof error)) {
        fprintf(stderr, "plamo-hip: %s\n", error);
        return 1;
    }
    if (putchar('\n') == EOF || fflush(stdout))
        return 1;
    fprintf(stderr,
            "plamo-hip: %" PRIu64 " prompt tokens, %" PRIu64 " completion tokens (%s); load %.2f s, "
            "prefill %.2f ms, decode %.2f tok/s",
            n, result.completion_tokens, finish_name(result.finish), h->load_seconds,
            prefill * 1e3,
            result.decode_seconds > 0 ? (double)result.completion_tokens / result.decode_seconds
                                      : 0.0);
    if (speculative)
        fprintf(stderr, "; speculative %" PRIu64 " batches, %" PRIu64 " proposed, %" PRIu64 " accepted",
                result.speculative_batches, result.proposed_tokens, result.accepted_tokens);
    fputc('\n', stderr);
    return result.finish == 2 || ferror(stdout);
}

/* ---- worker (runtime/worker.c:1-4, 427-489) ---- */

static int channel_failed;

/* 1 read, 0 end of input before any byte, -1 error or a partial read. */
static int read_exact(void *data, size_t bytes) {
    size_t done = 0;
    while (done < bytes) {
        ssize_t n = read(STDIN_FILENO, (char *)data + done, bytes - done);
        if (n < 0 && errno == EINTR)
            continue;
        if (n <= 0)
            return done == 0 && n == 0 ? 0 : -1;
        done += (size_t)n;
    }
    return 1;
}

static void json_text(const char *s) {
    putchar('"');
    for (; *s; ++s) {
        const unsigned char c = (unsigned char)*s;
        if (c == '"' || c == '\\')
            printf("\\%c", c);
        else if (c < 0x20)
            printf("\\u%04x", c);
        else
            putchar(c);
    }
    putchar('"');
}

static void error_event(const char *code, const char *message) {
    printf("{\"event\":\"error\",\"code\":");
    json_text(code);
    printf(",\"message\":");
    json_text(message);
    printf("}\n");
    fflush(stdout);
}

static uint64_t weight_bytes(void) {
    uint64_t total = 0;
    for (uint64_t i = 0; i < plamo_weight_mapping_count; ++i)
        total += plamo_weight_mappings[i].bytes;
    return total;
}

static void memory_object(const struct plamo_metal_info *info) {
    printf("{\"mode\":\"resident\",\"weight_bytes\":%" PRIu64 ",\"preloaded_weight_bytes\":%" PRIu64
           ",\"allocated_bytes\":%" PRIu64 "}",
           weight_bytes(), info->cache.cached_bytes, info->allocated_bytes);
}

static void compute_object(const struct plamo_metal_info *info) {
    printf("{\"backend\":\"hip\",\"device\":");
    json_text(info->device);
    printf(",\"precision\":");
    json_text(info->precision);
    printf(",\"weight_storage\":");
    json_text(info->weight_storage);
    printf(",\"verification_batches\":%" PRIu64 ",\"verified_tokens\":%" PRIu64
           ",\"committed_tokens\":%" PRIu64 ",\"gpu_dispatches\":%" PRIu64
           ",\"command_buffers\":%" PRIu64 ",\"fused_decodes\":%" PRIu64
           ",\"fused_prefills\":%" PRIu64 ",\"cpu_fallbacks\":%" PRIu64 ",\"errors\":%" PRIu64
           ",\"gpu_seconds\":%.9f,\"allocated_bytes\":%" PRIu64 ",\"note\":",
           info->verification_batches, info->verified_tokens, info->committed_tokens,
           info->dispatches, info->command_buffers, info->fused_decodes, info->fused_prefills,
           info->cpu_fallbacks, info->errors, info->gpu_seconds, info->allocated_bytes);
    json_text(info->note);
    putchar('}');
}

struct stream {
    double start, first_token;
    uint64_t emitted;
};

/* Streams one token; between tokens a pending frame must be a cancel
 * (runtime/worker.c:115-132). Returning 0 ends the generation. */
static int token_event(uint32_t id, void *context) {
    struct stream *s = context;
    struct pollfd fd = {STDIN_FILENO, POLLIN, 0};
    if (poll(&fd, 1, 0) > 0) {
        if (fd.revents & POLLHUP)
            return 0;
        if (fd.revents & POLLIN) {
            uint32_t frame[4];
            if (read_exact(frame, sizeof frame) != 1 || frame[0] != 3 || frame[1] || frame[2] ||
                frame[3])
                channel_failed = 1;
            return 0;
        }
    }
    if (!s->emitted++)
        s->first_token = now() - s->start;
    printf("{\"event\":\"token\",\"token_id\":%" PRIu32 ",\"hex\":\"\"}\n", id);
    return fflush(stdout) == 0;
}

static void generate(struct host *h, const uint32_t *ids, uint64_t n, unsigned max_tokens) {
    char error[512];
    struct plamo_metal_info info;
    struct stream s = {now(), 0, 0};
    reset_request(&plamo_model);
    plamo_metal_get_info(h->gpu, &info);
    printf("{\"event\":\"prefill\",\"prompt_tokens\":%" PRIu64 ",\"memory\":", n);
    memory_object(&info);
    puts("}");
    fflush(stdout);
    const double gpu_before = info.gpu_seconds;
    int r = plamo_metal_prefill(h->gpu, &plamo_model, ids, n, NULL);
    if (r != 1) {
        error_event("inference_failed", r ? "prefill failed" : "prefill declined");
        return;
    }
    const double prefill_seconds = now() - s.start;
    plamo_metal_get_info(h->gpu, &info);
    const double prefill_gpu = info.gpu_seconds - gpu_before;
    const int speculative = h->draft != NULL;
    struct plamo_hip_decode_result result;
    if (!plamo_hip_decode(h->gpu, &plamo_model, &h->draft, ids, n, max_tokens, h->block,
                          token_event, &s, &result, error, sizeof error)) {
        error_event("inference_failed", error);
        return;
    }
    struct rusage usage;
    getrusage(RUSAGE_SELF, &usage);
    plamo_metal_get_info(h->gpu, &info);
    printf("{\"event\":\"done\",\"finish_reason\":\"%s\",\"usage\":{\"prompt_tokens\":%" PRIu64
           ",\"completion_tokens\":%" PRIu64 ",\"total_tokens\":%" PRIu64
           ",\"cached_prompt_tokens\":0},\"timings\":{\"prefill_seconds\":%.9f,"
           "\"decode_seconds\":%.9f,\"first_token_seconds\":%.9f,\"total_seconds\":%.9f,"
           "\"decode_steps\":%" PRIu64 ",\"prefill_gpu_seconds\":%.9f},"
           "\"process_peak_rss_bytes\":%ld,\"memory\":",
           finish_name(result.finish), n, result.completion_tokens, n + result.completion_tokens,
           prefill_seconds, result.decode_seconds, s.first_token, now() - s.start,
           result.decode_steps, prefill_gpu, usage.ru_maxrss * 1024L);
    memory_object(&info);
    printf(",\"speculative\":{\"enabled\":%s,\"block_tokens\":%u,\"batches\":%" PRIu64
           ",\"consumed_tokens\":%" PRIu64 ",\"proposed_tokens\":%" PRIu64
           ",\"accepted_tokens\":%" PRIu64 ",\"draft_seconds\":%.9f},\"compute\":",
           speculative ? "true" : "false", speculative ? (h->block ? h->block : PLAMO_VERIFY_MAX) : 0,
           result.speculative_batches, result.speculative_tokens, result.proposed_tokens,
           result.accepted_tokens, result.draft_seconds);
    compute_object(&info);
    puts("}");
    fflush(stdout);
}

static int worker(struct host *h) {
    static uint32_t ids[MAX_PROMPT];
    static char text[MAX_FRAME_TEXT + 1];
    struct plamo_metal_info info;
    plamo_metal_get_info(h->gpu, &info);
    printf("{\"event\":\"ready\",\"protocol\":1,\"model\":");
    json_text(plamo_model_name);
    printf(",\"repository\":");
    json_text(plamo_model_repository);
    printf(",\"revision\":");
    json_text(plamo_model_revision);
    printf(",\"worker_pid\":%ld,\"load_seconds\":%.9f,\"preload_seconds\":%.9f,\"threads\":1,"
           "\"memory\":",
           (long)getpid(), h->load_seconds, h->preload_seconds);
    memory_object(&info);
    printf(",\"prompt_cache\":{\"en_ja_tokens\":0,\"ja_en_tokens\":0,\"bytes\":0,"
           "\"prepare_seconds\":0},\"speculative\":{\"enabled\":%s,\"block_tokens\":%u},"
           "\"compute\":",
           h->draft ? "true" : "false", h->draft ? (h->block ? h->block : PLAMO_VERIFY_MAX) : 0);
    compute_object(&info);
    puts("}");
    fflush(stdout);
    for (;;) {
        uint32_t frame[4];
        const int got = read_exact(frame, sizeof frame);
        if (got == 0)
            return 0;
        if (got < 0) {
            error_event("protocol_error", "incomplete request header");
            return 1;
        }
        const unsigned op = frame[0], direction = frame[1], max_tokens = frame[2],
                       bytes = frame[3];
        if (op == 3 && !direction && !max_tokens && !bytes)
            continue; /* a cancel that arrived after its generation ended */
        if ((op != 1 && op != 2) || bytes > MAX_FRAME_TEXT) {
            error_event("protocol_error", "invalid request frame");
            return 1;
        }
        if (read_exact(text, bytes) != 1) {
            error_event("protocol_error", "incomplete text");
            return 1;
        }
        text[bytes] = 0;
        uint64_t n = 0;
        if (memchr(text, 0, bytes)) {
            error_event("invalid_input", "NUL characters are not supported");
            continue;
        }
        if (direction > 2) {
            error_event("invalid_input", "direction must be 0, 1 or 2");
            continue;
        }
        if (!parse_ids(text, text + bytes, ids, &n)) {
            error_event("invalid_input", "the prompt must be decimal token ids");
            continue;
        }
        uint64_t bad = n;
        for (uint64_t i = 0; i < n && bad == n; ++i)
            if (ids[i] >= plamo_model.vocab)
                bad = i;
        if (bad != n) {
            error_event("invalid_input", "a token id is outside the vocabulary");
            continue;
        }
        if (op == 2) {
            printf("{\"event\":\"tokenized\",\"prompt_tokens\":%" PRIu64 ",\"token_ids\":[", n);
            for (uint64_t i = 0; i < n; ++i)
                printf("%s%" PRIu32, i ? "," : "", ids[i]);
            printf("]}\n");
            fflush(stdout);
            continue;
        }
        if (!n || n > 4096 || !max_tokens || max_tokens > 4096) {
            error_event("invalid_input", "generation needs 1..4096 prompt ids and max_tokens in 1..4096");
            continue;
        }
        generate(h, ids, n, max_tokens);
        if (channel_failed) {
            error_event("protocol_error", "a frame other than cancel arrived during generation");
            return 1;
        }
    }
}

int main(int argc, char **argv) {
    const char *model_dir = NULL, *draft_dir = NULL;
    unsigned max_tokens = 256, block = 0;
    int separator = 0, serve = 0;
    static uint32_t ids[MAX_PROMPT];
    uint64_t n = 0;
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
        if (!separator && !strcmp(arg, "--worker")) {
            serve = 1;
            continue;
        }
        if (!separator && arg[0] == '-' && arg[1] == '-') {
            if (++i == argc)
                goto invalid;
            const char *value = argv[i];
            if (!strcmp(arg, "--model"))
                model_dir = value;
            else if (!strcmp(arg, "--draft"))
                draft_dir = value;
            else if (!strcmp(arg, "--max-tokens")) {
                if (!parse_count(value, 4096, &max_tokens))
                    goto invalid;
            } else if (!strcmp(arg, "--speculative-tokens")) {
                if (!parse_count(value, PLAMO_VERIFY_MAX, &block))
                    goto invalid;
            } else
                goto invalid;
            continue;
        }
        if (!parse_ids(arg, arg + strlen(arg), ids, &n))
            goto invalid;
    }
    if (serve ? n != 0 : !n) {
        if (!serve && argc == 1) {
            usage(stdout);
            return 0;
        }
        goto invalid;
    }
    if (model_dir && !plamo_model_set_directory(model_dir)) {
        fprintf(stderr, "plamo-hip: model directory path too long\n");
        return 1;
    }
    if (!model_dir && !getenv("PLAMO_MODEL_DIR")) {
        const char *message = "no model: pass --model DIR or set PLAMO_MODEL_DIR";
        if (serve)
            error_event("startup_failed", message);
        else
            fprintf(stderr, "plamo-hip: %s\n", message);
        return 1;
    }
    if (!serve) {
        if (!plamo_model_open())
            return 1; /* the binder reported why */
        for (uint64_t i = 0; i < n; ++i)
            if (ids[i] >= plamo_model.vocab) {
                fprintf(stderr,
                        "plamo-hip: token id %" PRIu32 " is outside the vocabulary (%" PRIu64 ")\n",
                        ids[i], plamo_model.vocab);
                return 2;
            }
    }
    char error[512];
    struct host h;
    memset(&h, 0, sizeof h);
    h.block = block;
    if (!host_open(&h, draft_dir, error, sizeof error)) {
        if (serve)
            error_event("startup_failed", error);
        else
            fprintf(stderr, "plamo-hip: %s\n", error);
        host_close(&h);
        return 1;
    }
    const int status = serve ? worker(&h) : one_shot(&h, ids, n, max_tokens, draft_dir != NULL);
    host_close(&h);
    return status;
invalid:
    usage(stderr);
    return 2;
}
