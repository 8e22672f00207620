// Mutation fuzz of config.json parsing and plamo_checkpoint_open() over a
// checkpoint directory written by tests/checkpoint_writer.py: byte
// substitutions, deletions and truncations of config.json, each opened with
// a random global capacity (AddressSanitizer + UBSan host build, driven by
// tests/test_parser_fuzz.py). The original config.json is written back at the end.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "plamo_checkpoint.h"

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }

int main(int argc, char **argv) {
    const char *dir = argv[1];
    long iters = argc > 2 ? atol(argv[2]) : 20000;
    char path[512];
    snprintf(path, sizeof path, "%s/config.json", dir);
    FILE *f = fopen(path, "rb");
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    char *base = malloc(n);
    if (fread(base, 1, n, f) != (size_t)n) return 1;
    fclose(f);
    char err[256];
    struct plamo_checkpoint *ck = plamo_checkpoint_open(dir, 64, err, sizeof err);
    if (!ck) { printf("seed rejected: %s\n", err); return 1; }
    plamo_checkpoint_close(ck);
    const char special[] = "{}[]:,\"0123456789 \\-.eEtrufalsn";
    long opened = 0;
    char *buf = malloc(n + 64);
    for (long it = 0; it < iters; ++it) {
        long sz = n;
        memcpy(buf, base, n);
        int muts = 1 + (int)(rnd() % 6);
        for (int m = 0; m < muts; ++m) {
            long at = (long)(rnd() % (uint64_t)sz);
            switch (rnd() % 4) {
            case 0: buf[at] = special[rnd() % (sizeof special - 1)]; break;
            case 1: buf[at] = (char)rnd(); break;
            case 2: if (buf[at] >= '0' && buf[at] <= '9') buf[at] = '0' + (char)(rnd() % 10); break;
            default: memmove(buf + at, buf + at + 1, sz - at - 1); --sz; break;
            }
        }
        if (rnd() % 10 == 0) sz = (long)(rnd() % (uint64_t)(sz + 1));
        f = fopen(path, "wb");
        fwrite(buf, 1, sz, f);
        fclose(f);
        ck = plamo_checkpoint_open(dir, rnd() % 3 == 0 ? 0 : 1 + rnd() % 100, err, sizeof err);
        if (ck) {
            ++opened;
            size_t count = 0;
            (void)plamo_checkpoint_mappings(ck, &count);
            (void)plamo_checkpoint_schema(ck);
            plamo_checkpoint_close(ck);
        }
    }
    f = fopen(path, "wb");
    fwrite(base, 1, n, f);
    fclose(f);
    printf("done %ld iterations, %ld opened\n", iters, opened);
    free(buf);
    free(base);
    return 0;
}
