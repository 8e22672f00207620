// Mutation fuzz of the safetensors primitives (include/plamo_checkpoint.h),
// built for the host with AddressSanitizer and UBSan by
// tests/test_parser_fuzz.py. Every mutated file is its own exact-size heap
// block, so any read past the mapped bytes is reported. Exit status 0 with a
// summary line; the sanitizers abort on the first finding.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "plamo_checkpoint.h"

static uint64_t rs = 88172645463325252ull;
static uint64_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }

int main(int argc, char **argv) {
    long iters = argc > 1 ? atol(argv[1]) : 200000;
    const char *hdr = "{\"__metadata__\":{\"format\":\"pt\",\"x\":\"y\"},"
                      "\"a\":{\"dtype\":\"BF16\",\"shape\":[2,3],\"data_offsets\":[0,12]},"
                      "\"b\":{\"shape\":[4],\"dtype\":\"BF16\",\"data_offsets\":[12,20]},"
                      "\"c\":{\"dtype\":\"BF16\",\"shape\":[],\"data_offsets\":[20,22]}}   ";
    uint64_t n = strlen(hdr);
    size_t size = 8 + n + 22;
    unsigned char *base = malloc(size);
    for (int i = 0; i < 8; ++i) base[i] = (unsigned char)(n >> (8 * i));
    memcpy(base + 8, hdr, n);
    for (size_t i = 8 + n; i < size; ++i) base[i] = (unsigned char)i;
    struct plamo_safetensors_view v;
    struct plamo_tensor t;
    if (!plamo_safetensors_view(base, size, &v) || !plamo_find_tensor(base, size, "b", &t) ||
        t.rank != 1 || t.dims[0] != 4) {
        printf("seed file rejected\n");
        return 1;
    }
    const char special[] = "{}[]:,\"0123456789 \\-.eE";
    long found = 0;
    for (long it = 0; it < iters; ++it) {
        size_t sz = size;
        if (rnd() % 4 == 0) sz = rnd() % (size + 1);
        unsigned char *f = malloc(sz ? sz : 1);
        memcpy(f, base, sz);
        int muts = 1 + (int)(rnd() % 4);
        for (int m = 0; m < muts && sz; ++m) {
            size_t at = rnd() % sz;
            if (at < 8 && rnd() % 2) continue;
            f[at] = rnd() % 2 ? (unsigned char)special[rnd() % (sizeof special - 1)] : (unsigned char)rnd();
        }
        if (sz >= 8 && rnd() % 8 == 0) {  // header length near the edges
            uint64_t len = rnd() % 3 == 0 ? sz - 8 : (rnd() % 2 ? n : rnd() % (sz + 16));
            for (int i = 0; i < 8; ++i) f[i] = (unsigned char)(len >> (8 * i));
        }
        const char *names[] = {"a", "b", "c", "zz", "__metadata__", ""};
        for (int k = 0; k < 6; ++k) found += plamo_find_tensor(f, sz, names[k], &t);
        if (plamo_safetensors_view(f, sz, &v)) {
            const char *p = v.header, *end = v.header + v.header_size;
            struct plamo_json_token tok;
            for (int guard = 0; guard < 10000 && p < end; ++guard) {
                int k = plamo_json_next(p, end, &tok);
                if (k == PLAMO_JSON_END || k == PLAMO_JSON_BAD) break;
                p = tok.next;
            }
            struct plamo_tensor_field tf;
            for (int k = 0; k < 4; ++k) {
                uint64_t a = rnd() % (v.header_size + 1), b = a + rnd() % (v.header_size + 1 - a);
                plamo_tensor_descriptor(v.header + a, v.header + b, v.data_size, &tf);
                struct plamo_number num;
                plamo_parse_u64(v.header + a, v.header + b, &num);
            }
        }
        free(f);
    }
    free(base);
    printf("done %ld iterations, %ld finds\n", iters, found);
    return 0;
}
