/* Linux stand-ins for the engine's host modules that cannot be built on Linux,
 * so that the reference's runtime/engine.c and runtime/prompt_cache.c link and
 * run against libplamo_hip.so. Test infrastructure only.
 *
 *   - runtime/tokenizer.c calls the reference's AArch64 tokenizer assembly
 *     (plamo_vocab_load, plamo_encode_marked, ...). A toy byte tokenizer with
 *     the same interface (runtime/tokenizer.h:9-17) takes its place: the
 *     vocabulary file holds the vocabulary size; direction 0 encodes the bytes
 *     alone, direction 1/2 wraps them in fixed translation prefix 0/1 and an
 *     end marker; ids decode to "<id>". The two prefixes have the shape of
 *     the reference's template prefixes (see toy_prefix).
 *   - runtime/resident.c (mach/mach.h), runtime/parallel.c (sys/qos.h,
 *     sysctl) and runtime/weight_cache.c (F_NOCACHE) are Darwin-only. With the
 *     GPU backend open the engine calls only the memory probes among them
 *     (runtime/engine.c:122-123, 161); the rest report that the CPU memory
 *     modes are unavailable here.
 * Declarations come from the reference's own headers.
 */
#include "parallel.h"
#include "resident.h"
#include "tokenizer.h"
#include "weight_cache.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---- tokenizer ---- */

enum { TOY_FIRST_BYTE_ID = 32, TOY_END_ID = 17, TOY_MAX_IDS = 4096 + 64, TOY_PREFIX_IDS = 12 };
/* The shape of the reference's translation prefixes (src/prompt.s:64-66 through
 * runtime/tokenizer.c:178-184): bos, tag, "dataset", msg, "translation", tag,
 * "input", key, "lang", val, the language, msg. Twelve ids that differ only in
 * the language id at index 10 and end in the same id. */
static const uint32_t toy_prefix[2][TOY_PREFIX_IDS] = {
    {20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 29, 23},
    {20, 21, 22, 23, 24, 21, 25, 26, 27, 28, 30, 23}};

struct plamo_tokenizer {
    uint64_t vocab;
    uint32_t ids[TOY_MAX_IDS];
    char text[32];
};

struct plamo_tokenizer *plamo_tokenizer_open(const char *path, char *error, size_t cap) {
    FILE *f = fopen(path, "r");
    unsigned long long vocab = 0;
    if (!f || fscanf(f, "%llu", &vocab) != 1 || vocab <= TOY_FIRST_BYTE_ID + 1) {
        if (f)
            fclose(f);
        snprintf(error, cap, "cannot read vocabulary %s", path);
        return NULL;
    }
    fclose(f);
    struct plamo_tokenizer *t = calloc(1, sizeof *t);
    if (!t) {
        snprintf(error, cap, "cannot allocate tokenizer");
        return NULL;
    }
    t->vocab = vocab;
    return t;
}

void plamo_tokenizer_close(struct plamo_tokenizer *t) { free(t); }

uint64_t plamo_tokenizer_prefix(struct plamo_tokenizer *t, unsigned direction, const uint32_t **ids,
                                char *error, size_t cap) {
    if (direction > 1) {
        snprintf(error, cap, "no prefix for direction %u", direction);
        return UINT64_MAX;
    }
    memcpy(t->ids, toy_prefix[direction], sizeof toy_prefix[direction]);
    *ids = t->ids;
    return sizeof toy_prefix[direction] / sizeof toy_prefix[direction][0];
}

uint64_t plamo_tokenizer_encode(struct plamo_tokenizer *t, const char *text, unsigned direction,
                                const uint32_t **ids, char *error, size_t cap) {
    if (direction > 2) {
        snprintf(error, cap, "direction must be 0, 1 or 2");
        return UINT64_MAX;
    }
    uint64_t n = 0;
    if (direction) {
        memcpy(t->ids, toy_prefix[direction - 1], sizeof toy_prefix[0]);
        n = sizeof toy_prefix[0] / sizeof toy_prefix[0][0];
    }
    for (const unsigned char *p = (const unsigned char *)text; *p; ++p) {
        if (n + 2 > TOY_MAX_IDS) {
            snprintf(error, cap, "text too long");
            return UINT64_MAX;
        }
        t->ids[n++] = TOY_FIRST_BYTE_ID + (uint32_t)(*p % (t->vocab - TOY_FIRST_BYTE_ID));
    }
    if (direction)
        t->ids[n++] = TOY_END_ID;
    *ids = t->ids;
    return n;
}

uint64_t plamo_tokenizer_decode(struct plamo_tokenizer *t, uint32_t id, const char **bytes) {
    int n = snprintf(t->text, sizeof t->text, "<%u>", id);
    *bytes = t->text;
    return (uint64_t)n;
}

/* ---- memory probes and the Darwin-only memory modes ---- */

uint64_t plamo_physical_memory(void) {
    long pages = sysconf(_SC_PHYS_PAGES), size = sysconf(_SC_PAGESIZE);
    return pages > 0 && size > 0 ? (uint64_t)pages * (uint64_t)size : 0;
}

uint64_t plamo_reclaimable_memory(void) {
    long pages = sysconf(_SC_AVPHYS_PAGES), size = sysconf(_SC_PAGESIZE);
    return pages > 0 && size > 0 ? (uint64_t)pages * (uint64_t)size : 0;
}

int plamo_resident_copy(const struct plamo_mapping *in, const int64_t *fds, size_t count,
                        uint64_t reserve, struct plamo_mapping *out, char *error, size_t cap) {
    (void)in, (void)fds, (void)reserve;
    memset(out, 0, count * sizeof *out);
    snprintf(error, cap, "CPU-resident weights are not available in this host");
    return 0;
}

void plamo_resident_release(struct plamo_mapping *maps, size_t count) { (void)maps, (void)count; }

int plamo_rebase_weights(struct plamo_weight_spec *schema, const struct plamo_mapping *from,
                         const struct plamo_mapping *to, size_t count) {
    (void)schema, (void)from, (void)to, (void)count;
    return 0;
}

struct plamo_weight_cache *plamo_weight_cache_open(const struct plamo_mapping *maps,
                                                   const int64_t *fds, size_t count,
                                                   uint64_t reserve, uint64_t (*available)(void),
                                                   char *error, size_t cap) {
    (void)maps, (void)fds, (void)count, (void)reserve, (void)available;
    snprintf(error, cap, "the adaptive weight cache is not available in this host");
    return NULL;
}

void plamo_weight_cache_close(struct plamo_weight_cache *c) { (void)c; }
void plamo_weight_cache_rebalance(struct plamo_weight_cache *c) { (void)c; }
void plamo_weight_cache_get_info(const struct plamo_weight_cache *c,
                                 struct plamo_weight_cache_info *info) {
    (void)c;
    memset(info, 0, sizeof *info);
}
int plamo_weight_cache_preload(struct plamo_weight_cache *c, const void *p, uint64_t bytes) {
    (void)c, (void)p, (void)bytes;
    return 0;
}
const void *plamo_weight_cache_acquire(const void *p, uint64_t bytes, void *context) {
    (void)bytes, (void)context;
    return p;
}

/* A null scheduler is the documented single-threaded fallback
 * (runtime/parallel.h:13-15). */
struct plamo_parallel *plamo_parallel_open(unsigned threads) {
    (void)threads;
    return NULL;
}
unsigned plamo_parallel_threads(const struct plamo_parallel *p) { return p ? 0 : 1; }
void plamo_parallel_close(struct plamo_parallel *p) { (void)p; }
