// The host side of the bench's prefill flow under AddressSanitizer and UBSan:
// synthetic build, page-locked instances (heap allocations here), the
// prompt-prefix capture and restore copies (runtime/prompt_cache.c:15-82, as
// bench.py's capture/restore make them after the engine's request reset,
// runtime/engine.c:46-55), and the rows the backend's prefill copies from
// the device into the host arrays per layer (K, V and rotated K rows
// [count, min(count + T, capacity)); the whole window when a sliding layer
// overflows), then release and free, cycle after cycle. Prints
// "done N cycles".
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <sanitizer/asan_interface.h>

#include "plamo_model.h"
#include "plamo_synthetic.h"

// The instance's host arrays are whole 4 KiB pages; the tail past a cache's
// capacity rows is poisoned while the rows are written, so a row written one
// past the capacity is reported, not absorbed by the rounding.
static void poison_tail(const float *a, uint64_t capacity, uint64_t width, int on) {
    const size_t used = capacity * width * sizeof(float), whole = (used + 4095) / 4096 * 4096;
    if (whole > used) {
        if (on)
            ASAN_POISON_MEMORY_REGION((const char *)a + used, whole - used);
        else
            ASAN_UNPOISON_MEMORY_REGION((const char *)a + used, whole - used);
    }
}

static void poison_caches(struct model *m, int on) {
    for (uint64_t i = 0; i < m->count; ++i) {
        const struct cache *c = m->layers[i]->mixer->cache;
        poison_tail(c->k, c->capacity, c->width, on);
        poison_tail(c->v, c->capacity, c->width, on);
        poison_tail(m->layers[i]->mixer->rotation->out, c->capacity, c->width, on);
    }
}

static void mirror_rows(float *dst, uint64_t first, uint64_t end, uint64_t width, float tag) {
    for (uint64_t r = first; r < end; ++r)
        for (uint64_t c = 0; c < width; ++c) dst[r * width + c] = tag + (float)r;
}

int main(int argc, char **argv) {
    const int cycles = argc > 1 ? atoi(argv[1]) : 4;
    const uint64_t prefix = 12, bodies[] = {69, 116, 443};
    struct plamo_synthetic_config cfg;
    plamo_synthetic_defaults(&cfg, 256, 4, 2, 1, 128, 512, 300);
    cfg.window = 64;
    cfg.global_capacity = 512;
    cfg.pattern = 2;
    cfg.seed = 5;
    char err[256];
    struct plamo_synthetic *s = plamo_synthetic_build(&cfg, 2, err, sizeof err);
    if (!s) {
        fprintf(stderr, "build: %s\n", err);
        return 1;
    }
    for (int cycle = 0; cycle < cycles; ++cycle) {
        struct plamo_synthetic_instance *in = plamo_synthetic_instantiate(s, 1, err, sizeof err);
        if (!in) {
            fprintf(stderr, "instantiate: %s\n", err);
            return 1;
        }
        struct model *m = plamo_synthetic_model(in);
        poison_caches(m, 1);
        if (!plamo_synthetic_fill_kv(in, prefix, 100 + cycle)) return 1;
        float *snap[64][3];
        for (uint64_t i = 0; i < m->count; ++i) {
            const struct cache *c = m->layers[i]->mixer->cache;
            const struct rotation *r = m->layers[i]->mixer->rotation;
            const size_t bytes = prefix * c->width * sizeof(float);
            const float *src[3] = {c->k, c->v, r->out};
            for (int a = 0; a < 3; ++a) {
                snap[i][a] = malloc(bytes);
                memcpy(snap[i][a], src[a], bytes);
            }
        }
        for (size_t b = 0; b < sizeof bodies / sizeof bodies[0]; ++b) {
            const uint64_t T = bodies[b];
            for (uint64_t i = 0; i < m->count; ++i) {
                struct cache *c = m->layers[i]->mixer->cache;
                struct rotation *r = m->layers[i]->mixer->rotation;
                c->count = 0;
                r->processed_count = 0;
                const size_t bytes = prefix * c->width * sizeof(float);
                memcpy(c->k, snap[i][0], bytes);
                memcpy(c->v, snap[i][1], bytes);
                memcpy(r->out, snap[i][2], bytes);
                c->count = prefix;
                r->processed_count = prefix;
                const int overflow = prefix + T > c->capacity;
                const uint64_t first = overflow ? 0 : c->count;
                const uint64_t end = prefix + T < c->capacity ? prefix + T : c->capacity;
                mirror_rows(c->k, first, end, c->width, 1.0f);
                mirror_rows(c->v, first, end, c->width, 2.0f);
                mirror_rows(r->out, first, end, c->width, 3.0f);
                c->count = end;
                r->processed_count = end;
            }
        }
        for (uint64_t i = 0; i < m->count; ++i)
            for (int a = 0; a < 3; ++a) free(snap[i][a]);
        poison_caches(m, 0);
        plamo_synthetic_release(in);
    }
    plamo_synthetic_free(s);
    printf("done %d cycles\n", cycles);
    return 0;
}
