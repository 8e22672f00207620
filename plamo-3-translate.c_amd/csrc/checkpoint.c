/* Real checkpoints on Linux: the reference's safetensors binder in C
 * (src/load.s, src/json.s, src/tensor.s, src/find.s, src/resolve.s,
 * src/bind.s, src/model_open.s), and the schema / descriptor layout the
 * reference generates at build time (tools/weight_schema.py,
 * tools/model_layout.py, tools/rope_constants.py) evaluated from config.json.
 */
#define _GNU_SOURCE
#include "../../include/plamo_checkpoint.h"

#include <ctype.h>
#include <dirent.h>
#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "layout.h"

/* ---------------------------------------------------------------- envelope */

int plamo_safetensors_view(const void *file, uint64_t size, struct plamo_safetensors_view *out) {
    memset(out, 0, sizeof *out);
    if (!file || size < 10)
        return 0;
    uint64_t n;
    memcpy(&n, file, 8);
    if (n > size - 8 || n < 2 || n > 100000000) /* safetensors caps headers at 100 MB */
        return 0;
    const char *h = (const char *)file + 8;
    if (h[0] != '{')
        return 0;
    uint64_t last = n - 1;
    while (last > 0 && h[last] == ' ')
        --last;
    if (last == 0 || h[last] != '}')
        return 0;
    out->header = h;
    out->header_size = n;
    out->data = h + n;
    out->data_size = size - 8 - n;
    return 1;
}

int plamo_parse_u64(const char *p, const char *end, struct plamo_number *out) {
    out->next = NULL;
    out->value = 0;
    if (!p || p >= end)
        return 0;
    const char *q = p;
    uint64_t value = 0;
    while (q < end && (unsigned)(*q - '0') <= 9) {
        const uint64_t digit = (uint64_t)(*q - '0');
        if (value > (UINT64_MAX - digit) / 10)
            return 0;
        value = value * 10 + digit;
        ++q;
        /* A zero is a whole number: "01" is not JSON. */
        if (value == 0 && q < end && (unsigned)(*q - '0') <= 9)
            return 0;
    }
    if (q == p)
        return 0;
    out->next = q;
    out->value = value;
    return 1;
}

/* ---------------------------------------------------------------- lexer */

static int is_space(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r'; }

int plamo_json_next(const char *p, const char *end, struct plamo_json_token *t) {
    memset(t, 0, sizeof *t);
    while (p < end && is_space(*p))
        ++p;
    if (p >= end) {
        t->next = p;
        return PLAMO_JSON_END;
    }
    const char c = *p;
    if (c == '{' || c == '}' || c == '[' || c == ']' || c == ':' || c == ',') {
        t->next = p + 1;
        t->start = p;
        t->length = 1;
        return (unsigned char)c;
    }
    if (c == '"') {
        const char *q = p + 1;
        for (;;) {
            if (q >= end)
                return PLAMO_JSON_BAD;
            const unsigned char ch = (unsigned char)*q++;
            if (ch == '"')
                break;
            if (ch < 32)
                return PLAMO_JSON_BAD;
            if (ch != '\\')
                continue;
            if (q >= end)
                return PLAMO_JSON_BAD;
            const char e = *q++;
            if (strchr("\"\\/bfnrt", e) && e)
                continue;
            if (e != 'u')
                return PLAMO_JSON_BAD;
            for (int i = 0; i < 4; ++i) {
                if (q >= end)
                    return PLAMO_JSON_BAD;
                const char x = (char)(*q++ | 32);
                if (!((x >= '0' && x <= '9') || (x >= 'a' && x <= 'f')))
                    return PLAMO_JSON_BAD;
            }
        }
        t->next = q;
        t->start = p + 1;
        t->length = (uint64_t)(q - (p + 1) - 1);
        return PLAMO_JSON_STRING;
    }
    struct plamo_number num;
    if (!plamo_parse_u64(p, end, &num))
        return PLAMO_JSON_BAD;
    if (num.next < end) {
        const char f = *num.next;
        if (!is_space(f) && f != ',' && f != ']' && f != '}')
            return PLAMO_JSON_BAD;
    }
    t->next = num.next;
    t->start = p;
    t->length = (uint64_t)(num.next - p);
    t->value = num.value;
    return PLAMO_JSON_UINT;
}

/* A key token equal to the NUL-terminated ASCII `s` (raw bytes: an escaped
 * key never matches). */
static int key_is(const struct plamo_json_token *t, const char *s) {
    const size_t n = strlen(s);
    return t->length == n && memcmp(t->start, s, n) == 0;
}

/* ---------------------------------------------------------------- tensors */

int plamo_tensor_descriptor(const char *p, const char *end, uint64_t data_bytes,
                            struct plamo_tensor_field *out) {
    memset(out, 0, sizeof *out);
    struct plamo_tensor_field r;
    memset(&r, 0, sizeof r);
    struct plamo_json_token t;
    unsigned seen = 0;
    uint64_t elements = 1;
#define EXPECT(code)                                                                               \
    do {                                                                                           \
        if (plamo_json_next(p, end, &t) != (code))                                                 \
            return 0;                                                                              \
        p = t.next;                                                                                \
    } while (0)
    EXPECT('{');
    for (;;) {
        EXPECT(PLAMO_JSON_STRING);
        if (key_is(&t, "dtype")) {
            if (seen & 1)
                return 0;
            seen |= 1;
            EXPECT(':');
            EXPECT(PLAMO_JSON_STRING);
            if (!key_is(&t, "BF16"))
                return 0;
        } else if (key_is(&t, "shape")) {
            if (seen & 2)
                return 0;
            seen |= 2;
            EXPECT(':');
            EXPECT('[');
            int code = plamo_json_next(p, end, &t);
            p = t.next;
            if (code != ']') {
                for (;;) {
                    if (code != PLAMO_JSON_UINT || r.rank >= 4)
                        return 0;
                    if (t.value && elements > UINT64_MAX / t.value)
                        return 0;
                    elements *= t.value;
                    r.dims[r.rank++] = t.value;
                    code = plamo_json_next(p, end, &t);
                    p = t.next;
                    if (code == ']')
                        break;
                    if (code != ',')
                        return 0;
                    code = plamo_json_next(p, end, &t);
                    p = t.next;
                }
            }
        } else if (key_is(&t, "data_offsets")) {
            if (seen & 4)
                return 0;
            seen |= 4;
            EXPECT(':');
            EXPECT('[');
            EXPECT(PLAMO_JSON_UINT);
            const uint64_t begin = t.value;
            EXPECT(',');
            EXPECT(PLAMO_JSON_UINT);
            const uint64_t stop = t.value;
            if (stop < begin || stop > data_bytes)
                return 0;
            r.offset = begin;
            r.bytes = stop - begin;
            EXPECT(']');
        } else {
            return 0;
        }
        const int code = plamo_json_next(p, end, &t);
        p = t.next;
        if (code == ',')
            continue;
        if (code != '}' || seen != 7)
            return 0;
        break;
    }
#undef EXPECT
    if (elements >> 63 || elements * 2 != r.bytes)
        return 0;
    r.next = p;
    *out = r;
    return 1;
}

int plamo_find_tensor(const void *file, uint64_t size, const char *name, struct plamo_tensor *out) {
    memset(out, 0, sizeof *out);
    struct plamo_safetensors_view v;
    if (!plamo_safetensors_view(file, size, &v))
        return 0;
    const char *p = v.header, *end = v.header + v.header_size;
    struct plamo_json_token t;
#define STEP() (code = plamo_json_next(p, end, &t), p = t.next, code)
    int code;
    if (STEP() != '{')
        return 0;
    if (STEP() == '}')
        return 0;
    for (;;) {
        if (code != PLAMO_JSON_STRING)
            return 0;
        const size_t n = strlen(name);
        const int match = t.length == n && memcmp(t.start, name, n) == 0;
        if (key_is(&t, "__metadata__")) {
            /* A string-to-string object. */
            if (STEP() != ':' || STEP() != '{')
                return 0;
            if (STEP() != '}') {
                for (;;) {
                    if (code != PLAMO_JSON_STRING || STEP() != ':' || STEP() != PLAMO_JSON_STRING)
                        return 0;
                    if (STEP() == '}')
                        break;
                    if (code != ',')
                        return 0;
                    (void)STEP();
                }
            }
        } else {
            if (STEP() != ':')
                return 0;
            struct plamo_tensor_field f;
            if (!plamo_tensor_descriptor(p, end, v.data_size, &f))
                return 0;
            p = f.next;
            if (match) {
                out->data = (const uint16_t *)((const char *)v.data + f.offset);
                out->bytes = f.bytes;
                out->rank = f.rank;
                memcpy(out->dims, f.dims, sizeof f.dims);
                return 1;
            }
        }
        if (STEP() != ',')
            return 0;
        (void)STEP();
    }
#undef STEP
}

const uint16_t *plamo_resolve_weight(const struct plamo_mapping *shards, uint64_t count,
                                     const char *name, uint64_t rank, const uint64_t *dims) {
    if (rank > 4)
        return NULL;
    for (uint64_t i = 0; i < count; ++i) {
        struct plamo_tensor t;
        if (!plamo_find_tensor(shards[i].base, shards[i].bytes, name, &t))
            continue;
        if (t.rank != rank)
            return NULL;
        for (uint64_t d = 0; d < rank; ++d)
            if (t.dims[d] != dims[d])
                return NULL;
        return t.data;
    }
    return NULL;
}

int plamo_bind_weights(const struct plamo_mapping *shards, uint64_t count,
                       struct plamo_weight_spec *schema) {
    for (struct plamo_weight_spec *s = schema; s->name; ++s) {
        const uint16_t *data = plamo_resolve_weight(shards, count, s->name, s->rank, s->shape);
        if (!data) {
            for (struct plamo_weight_spec *c = schema; c->name; ++c)
                *c->slot = NULL;
            return 0;
        }
        *s->slot = (void *)data;
    }
    return 1;
}

/* ---------------------------------------------------------------- config.json */

/* A small reader for the values config.json holds (objects, arrays, strings,
 * numbers, true/false/null): it finds one member by a path of keys. */
struct cfg {
    const char *p, *end;
};

static void cfg_space(struct cfg *c) {
    while (c->p < c->end && is_space(*c->p))
        ++c->p;
}

static int cfg_skip(struct cfg *c, int depth);

static int cfg_string(struct cfg *c, const char **s, size_t *n) {
    cfg_space(c);
    if (c->p >= c->end || *c->p != '"')
        return 0;
    const char *q = ++c->p;
    while (c->p < c->end && *c->p != '"') {
        if (*c->p == '\\')
            ++c->p;
        ++c->p;
    }
    if (c->p >= c->end)
        return 0;
    if (s) {
        *s = q;
        *n = (size_t)(c->p - q);
    }
    ++c->p;
    return 1;
}

static int cfg_skip(struct cfg *c, int depth) {
    cfg_space(c);
    if (c->p >= c->end || depth > 32)
        return 0;
    const char ch = *c->p;
    if (ch == '"')
        return cfg_string(c, NULL, NULL);
    if (ch == '{' || ch == '[') {
        const char close = ch == '{' ? '}' : ']';
        ++c->p;
        cfg_space(c);
        if (c->p < c->end && *c->p == close) {
            ++c->p;
            return 1;
        }
        for (;;) {
            if (ch == '{') {
                if (!cfg_string(c, NULL, NULL))
                    return 0;
                cfg_space(c);
                if (c->p >= c->end || *c->p++ != ':')
                    return 0;
            }
            if (!cfg_skip(c, depth + 1))
                return 0;
            cfg_space(c);
            if (c->p >= c->end)
                return 0;
            if (*c->p == ',') {
                ++c->p;
                continue;
            }
            if (*c->p++ != close)
                return 0;
            return 1;
        }
    }
    /* number, true, false, null */
    const char *q = c->p;
    while (c->p < c->end && (isalnum((unsigned char)*c->p) || strchr("+-.", *c->p)))
        ++c->p;
    return c->p > q;
}

/* Positions c at the value of `key` in the object c points at. */
static int cfg_member(struct cfg *c, const char *key) {
    cfg_space(c);
    if (c->p >= c->end || *c->p != '{')
        return 0;
    ++c->p;
    cfg_space(c);
    if (c->p < c->end && *c->p == '}')
        return 0;
    for (;;) {
        const char *s;
        size_t n;
        if (!cfg_string(c, &s, &n))
            return 0;
        cfg_space(c);
        if (c->p >= c->end || *c->p++ != ':')
            return 0;
        if (n == strlen(key) && memcmp(s, key, n) == 0)
            return 1;
        if (!cfg_skip(c, 0))
            return 0;
        cfg_space(c);
        if (c->p >= c->end || *c->p != ',')
            return 0;
        ++c->p;
    }
}

/* The value at a path of up to three keys: 1 found, 0 absent. */
static int cfg_find(const char *text, size_t size, const char *k1, const char *k2, const char *k3,
                    struct cfg *out) {
    struct cfg c = {text, text + size};
    if (!cfg_member(&c, k1) || (k2 && !cfg_member(&c, k2)) || (k3 && !cfg_member(&c, k3)))
        return 0;
    cfg_space(&c);
    *out = c;
    return 1;
}

static int cfg_number(const char *text, size_t size, const char *k1, const char *k2,
                      const char *k3, double *value) {
    struct cfg c;
    if (!cfg_find(text, size, k1, k2, k3, &c))
        return 0;
    char buf[64];
    size_t n = 0;
    while (c.p < c.end && n < sizeof buf - 1 && (isalnum((unsigned char)*c.p) || strchr("+-.", *c.p)))
        buf[n++] = *c.p++;
    buf[n] = 0;
    char *stop;
    *value = strtod(buf, &stop);
    return n && *stop == 0;
}

static int cfg_bool(const char *text, size_t size, const char *key, int *value) {
    struct cfg c;
    if (!cfg_find(text, size, key, NULL, NULL, &c))
        return 0;
    if ((size_t)(c.end - c.p) >= 4 && !memcmp(c.p, "true", 4)) {
        *value = 1;
        return 1;
    }
    if ((size_t)(c.end - c.p) >= 5 && !memcmp(c.p, "false", 5)) {
        *value = 0;
        return 1;
    }
    return 0;
}

static int cfg_is_string(const char *text, size_t size, const char *k1, const char *k2,
                         const char *k3, const char *want) {
    struct cfg c;
    const char *s;
    size_t n;
    return cfg_find(text, size, k1, k2, k3, &c) && cfg_string(&c, &s, &n) && n == strlen(want) &&
           memcmp(s, want, n) == 0;
}

static int read_config(const char *text, size_t size, struct plamo_checkpoint_config *c,
                       char *error, size_t cap) {
    memset(c, 0, sizeof *c);
    static const char *const shape_keys[] = {"hidden_size",       "num_hidden_layers",
                                             "num_attention_heads", "num_key_value_heads",
                                             "head_dim",          "intermediate_size",
                                             "vocab_size",        "window_size",
                                             "sliding_window_pattern", "max_position_embeddings"};
    uint64_t *fields[] = {&c->hidden, &c->layers, &c->qh, &c->kh, &c->dim, &c->intermediate,
                          &c->vocab, &c->window, &c->pattern, &c->max_positions};
    for (size_t i = 0; i < sizeof fields / sizeof *fields; ++i) {
        double v;
        if (!cfg_number(text, size, shape_keys[i], NULL, NULL, &v) || v < 0 || v != floor(v) ||
            v > 1e12) {
            snprintf(error, cap, "config.json: %s missing or not a whole number", shape_keys[i]);
            return 0;
        }
        *fields[i] = (uint64_t)v;
    }
    if (!cfg_bool(text, size, "tie_word_embeddings", &c->tied)) {
        snprintf(error, cap, "config.json: tie_word_embeddings missing");
        return 0;
    }
    /* tools/rope_constants.py:55-76: sliding layers use sliding_attention,
     * global layers full_attention (YaRN when its rope_type says so). */
    if (!cfg_number(text, size, "rope_parameters", "sliding_attention", "rope_theta",
                    &c->local_theta) ||
        !cfg_number(text, size, "rope_parameters", "full_attention", "rope_theta",
                    &c->global_theta)) {
        snprintf(error, cap, "config.json: rope_parameters.{sliding,full}_attention.rope_theta missing");
        return 0;
    }
    c->global_yarn = cfg_is_string(text, size, "rope_parameters", "full_attention", "rope_type",
                                   "yarn");
    c->factor = 1;
    if (!cfg_number(text, size, "rope_parameters", "full_attention", "factor", &c->factor) &&
        c->global_yarn) {
        snprintf(error, cap, "config.json: full_attention.factor missing");
        return 0;
    }
    if (c->global_yarn &&
        (!cfg_number(text, size, "rope_parameters", "full_attention",
                     "original_max_position_embeddings", &c->original) ||
         !cfg_number(text, size, "rope_parameters", "full_attention", "beta_fast", &c->beta_fast) ||
         !cfg_number(text, size, "rope_parameters", "full_attention", "beta_slow", &c->beta_slow))) {
        snprintf(error, cap, "config.json: YaRN parameters of full_attention missing");
        return 0;
    }
    if (!c->hidden || !c->layers || c->layers > 128 || !c->qh || !c->kh || c->qh % c->kh ||
        !c->dim || c->dim % 2 || !c->intermediate || !c->vocab || !c->window) {
        snprintf(error, cap, "config.json: unsupported model shape");
        return 0;
    }
    return 1;
}

/* ---------------------------------------------------------------- checkpoint */

struct plamo_checkpoint {
    struct plamo_checkpoint_config config;
    uint64_t global_capacity;
    struct plamo_mapping maps[PLAMO_MAX_WEIGHT_FILES];
    int fds[PLAMO_MAX_WEIGHT_FILES];
    size_t count;
    /* tools/weight_schema.py:15-44 order, with names, shapes and slots. */
    struct plamo_weight_spec *schema;
    char *names;
    uint64_t *shapes;
    const uint16_t **slots;
    const uint16_t *embedding, *head, *norm;
    struct plamo_layout_layer *layers;
    float *local_freq, *global_freq;
    float local_scale, global_scale;
};

static int by_name(const void *a, const void *b) {
    return strcmp(*(char *const *)a, *(char *const *)b);
}

static char *read_text(const char *path, size_t *size) {
    FILE *f = fopen(path, "rb");
    if (!f)
        return NULL;
    char *buf = NULL;
    if (fseek(f, 0, SEEK_END) == 0) {
        long n = ftell(f);
        if (n >= 0 && n < (1 << 24) && fseek(f, 0, SEEK_SET) == 0 && (buf = malloc((size_t)n + 1))) {
            if (fread(buf, 1, (size_t)n, f) != (size_t)n) {
                free(buf);
                buf = NULL;
            } else {
                buf[n] = 0;
                *size = (size_t)n;
            }
        }
    }
    fclose(f);
    return buf;
}

/* Appends one schema entry whose slot feeds `target` once bound. */
struct schema_builder {
    struct plamo_checkpoint *ck;
    size_t n;
    const uint16_t ***targets;
};

static void add_entry(struct schema_builder *b, const char *name, uint64_t rank, uint64_t d0,
                      uint64_t d1, const uint16_t **target) {
    struct plamo_checkpoint *ck = b->ck;
    const size_t n = b->n++;
    char *slot_name = ck->names + n * 64;
    snprintf(slot_name, 64, "%s", name);
    ck->shapes[2 * n] = d0;
    ck->shapes[2 * n + 1] = d1;
    ck->schema[n] = (struct plamo_weight_spec){slot_name, rank, ck->shapes + 2 * n,
                                               (void **)&ck->slots[n]};
    b->targets[n] = target;
}

/* tools/weight_schema.py:15-44: embedding, final norm, the head unless tied,
 * then ten tensors per layer in this order. 1 bound, -1 not bound, 0 no memory. */
static int build_schema(struct plamo_checkpoint *ck) {
    const struct plamo_checkpoint_config *c = &ck->config;
    const uint64_t h = c->hidden, d = c->dim, q = c->qh * d, kv = c->kh * d;
    const size_t entries = 3 + 10 * c->layers;
    ck->schema = calloc(entries + 1, sizeof *ck->schema);
    ck->names = calloc(entries, 64);
    ck->shapes = calloc(entries * 2, sizeof *ck->shapes);
    ck->slots = calloc(entries, sizeof *ck->slots);
    ck->layers = calloc(c->layers, sizeof *ck->layers);
    const uint16_t ***targets = calloc(entries, sizeof *targets);
    if (!ck->schema || !ck->names || !ck->shapes || !ck->slots || !ck->layers || !targets) {
        free(targets);
        return 0;
    }
    struct schema_builder b = {ck, 0, targets};
    add_entry(&b, "model.embed_tokens.weight", 2, c->vocab, h, &ck->embedding);
    add_entry(&b, "model.norm.weight", 1, h, 0, &ck->norm);
    if (!c->tied)
        add_entry(&b, "lm_head.weight", 2, c->vocab, h, &ck->head);
    for (uint64_t i = 0; i < c->layers; ++i) {
        struct plamo_layout_layer *l = &ck->layers[i];
        char name[64];
#define LAYER(suffix, rank, d0, d1, field)                                                          \
    snprintf(name, sizeof name, "model.layers.layers.%llu." suffix, (unsigned long long)i);      \
    add_entry(&b, name, rank, d0, d1, &l->field)
        LAYER("mixer.qkv_proj.weight", 2, q + 2 * kv, h, qkv);
        LAYER("mixer.o_proj.weight", 2, h, q, o);
        LAYER("mixer.q_norm.weight", 1, d, 0, qn);
        LAYER("mixer.k_norm.weight", 1, d, 0, kn);
        LAYER("mlp.gate_up_proj.weight", 2, 2 * c->intermediate, h, gu);
        LAYER("mlp.down_proj.weight", 2, h, c->intermediate, down);
        LAYER("pre_mixer_norm.weight", 1, h, 0, pre);
        LAYER("post_mixer_norm.weight", 1, h, 0, post);
        LAYER("pre_mlp_norm.weight", 1, h, 0, mlp_pre);
        LAYER("post_mlp_norm.weight", 1, h, 0, mlp_post);
#undef LAYER
    }
    const int bound = plamo_bind_weights(ck->maps, ck->count, ck->schema);
    if (bound) {
        for (size_t i = 0; i < b.n; ++i)
            *targets[i] = ck->slots[i];
        if (c->tied)
            ck->head = ck->embedding;
    }
    free(targets);
    return bound ? 1 : -1;
}

/* The schema entry that did not resolve (for the error message). */
static const char *unresolved(const struct plamo_checkpoint *ck) {
    for (const struct plamo_weight_spec *s = ck->schema; s->name; ++s)
        if (!plamo_resolve_weight(ck->maps, ck->count, s->name, s->rank, s->shape))
            return s->name;
    return "?";
}

struct plamo_checkpoint *plamo_checkpoint_open(const char *directory, uint64_t global_capacity,
                                               char *error, size_t cap) {
    struct plamo_checkpoint *ck = calloc(1, sizeof *ck);
    char path[4096];
    if (!ck) {
        snprintf(error, cap, "cannot allocate checkpoint");
        return NULL;
    }
    for (size_t i = 0; i < PLAMO_MAX_WEIGHT_FILES; ++i)
        ck->fds[i] = -1;
    size_t size = 0;
    snprintf(path, sizeof path, "%s/config.json", directory);
    char *text = read_text(path, &size);
    if (!text) {
        snprintf(error, cap, "cannot read %s", path);
        goto fail;
    }
    if (!read_config(text, size, &ck->config, error, cap)) {
        free(text);
        goto fail;
    }
    free(text);
    const struct plamo_checkpoint_config *c = &ck->config;
    ck->global_capacity = global_capacity ? global_capacity : 8192;
    if (ck->global_capacity > c->max_positions)
        ck->global_capacity = c->max_positions;
    if (!ck->global_capacity)
        ck->global_capacity = 1;

    /* Shards: every *.safetensors file, in name order. */
    DIR *dir = opendir(directory);
    if (!dir) {
        snprintf(error, cap, "cannot open directory %s", directory);
        goto fail;
    }
    char *names[PLAMO_MAX_WEIGHT_FILES];
    size_t found = 0;
    struct dirent *e;
    int too_many = 0;
    while ((e = readdir(dir))) {
        const size_t len = strlen(e->d_name);
        if (len <= 12 || strcmp(e->d_name + len - 12, ".safetensors"))
            continue;
        if (found == PLAMO_MAX_WEIGHT_FILES) {
            too_many = 1;
            break;
        }
        names[found++] = strdup(e->d_name);
    }
    closedir(dir);
    qsort(names, found, sizeof *names, by_name);
    int mapped = !too_many && found > 0;
    for (size_t i = 0; i < found; ++i) {
        if (mapped) {
            snprintf(path, sizeof path, "%s/%s", directory, names[i]);
            const int fd = open(path, O_RDONLY | O_CLOEXEC);
            struct stat st;
            void *base = MAP_FAILED;
            if (fd >= 0 && fstat(fd, &st) == 0 && st.st_size > 0)
                base = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
            if (base == MAP_FAILED) {
                if (fd >= 0)
                    close(fd);
                snprintf(error, cap, "cannot map %s", path);
                mapped = 0;
            } else {
                ck->maps[ck->count] = (struct plamo_mapping){base, (uint64_t)st.st_size};
                ck->fds[ck->count++] = fd;
            }
        }
        free(names[i]);
    }
    if (too_many) {
        snprintf(error, cap, "more than %d safetensors files in %s", PLAMO_MAX_WEIGHT_FILES,
                 directory);
        goto fail;
    }
    if (!found) {
        snprintf(error, cap, "no .safetensors files in %s", directory);
        goto fail;
    }
    if (!mapped)
        goto fail;

    const int bound = build_schema(ck);
    if (bound <= 0) {
        if (bound < 0)
            snprintf(error, cap, "tensor %s is missing, not BF16, or of another shape",
                     unresolved(ck));
        else
            snprintf(error, cap, "cannot allocate the weight schema");
        goto fail;
    }
    const uint64_t half = c->dim / 2;
    ck->local_freq = calloc(half, sizeof(float));
    ck->global_freq = calloc(half, sizeof(float));
    if (!ck->local_freq || !ck->global_freq) {
        snprintf(error, cap, "cannot allocate RoPE tables");
        goto fail;
    }
    plamo_layout_frequencies(c->local_theta, half, 0, 0, 0, 0, 0, ck->local_freq);
    plamo_layout_frequencies(c->global_theta, half, c->global_yarn, c->factor, c->original,
                             c->beta_fast, c->beta_slow, ck->global_freq);
    /* Concentration 1 for a default table, 1 + 0.1 ln(factor) for YaRN
     * (tools/rope_constants.py:68-70, tools/model_layout.py:184-188). */
    ck->local_scale = 1.0f;
    ck->global_scale = c->global_yarn ? (float)(1.0 + 0.1 * log(c->factor)) : 1.0f;
    return ck;
fail:
    plamo_checkpoint_close(ck);
    return NULL;
}

void plamo_checkpoint_close(struct plamo_checkpoint *ck) {
    if (!ck)
        return;
    for (size_t i = 0; i < ck->count; ++i) {
        munmap(ck->maps[i].base, ck->maps[i].bytes);
        if (ck->fds[i] >= 0)
            close(ck->fds[i]);
    }
    free(ck->schema);
    free(ck->names);
    free(ck->shapes);
    free(ck->slots);
    free(ck->layers);
    free(ck->local_freq);
    free(ck->global_freq);
    free(ck);
}

const struct plamo_checkpoint_config *plamo_checkpoint_config(const struct plamo_checkpoint *ck) {
    return &ck->config;
}

const struct plamo_mapping *plamo_checkpoint_mappings(const struct plamo_checkpoint *ck,
                                                      size_t *count) {
    if (count)
        *count = ck->count;
    return ck->maps;
}

const struct plamo_weight_spec *plamo_checkpoint_schema(const struct plamo_checkpoint *ck) {
    return ck->schema;
}

struct plamo_synthetic_instance *plamo_checkpoint_instantiate(const struct plamo_checkpoint *ck,
                                                              int pinned, char *error, size_t cap) {
    const struct plamo_checkpoint_config *c = &ck->config;
    const struct plamo_layout lay = {c->hidden,       c->layers,        c->qh,
                                     c->kh,           c->dim,           c->intermediate,
                                     c->vocab,        c->window,        ck->global_capacity,
                                     c->pattern,      ck->embedding,    ck->head,
                                     ck->norm,        ck->layers,       ck->local_freq,
                                     ck->global_freq, ck->local_scale,  ck->global_scale};
    return plamo_layout_instantiate(&lay, pinned, error, cap);
}

/* ---------------------------------------------------------------- engine globals */

struct model plamo_model;
struct plamo_mapping plamo_weight_mappings[PLAMO_MAX_WEIGHT_FILES];
int64_t plamo_weight_fds[PLAMO_MAX_WEIGHT_FILES];
uint64_t plamo_weight_mapping_count, plamo_weight_file_count;
struct plamo_weight_spec plamo_weight_schema[PLAMO_MAX_SCHEMA];
char plamo_vocab_path[4096 + 32], plamo_model_name[64] = "plamo-3-translate-custom",
                                  plamo_model_repository[80], plamo_model_revision[64];
/* Pairs plus the zero terminator: one descriptor field per schema entry (the
 * tied head reuses the embedding's slot in place of its own entry). */
uint64_t plamo_model_patches[2 * PLAMO_MAX_SCHEMA];
uint64_t plamo_io_policy, plamo_io_stats[4];

static char model_directory[4096];
static struct plamo_checkpoint *opened;
static struct plamo_synthetic_instance *opened_instance;

/* The published profiles (tools/profiles/{0.8b,2b,8b,31b}/config.json shapes
 * and manifest.json repository revisions): the engine keys behaviour on the
 * name (runtime/engine.c:146-149, 322-324). */
static const struct {
    uint64_t hidden, layers, qh, kh, intermediate;
    int tied;
    const char *size, *revision;
} profiles[] = {
    {1536, 16, 16, 1, 6144, 0, "0.8b", "573eb1be9fd8c44402650810c680104e5aec81e8"},
    {2560, 24, 24, 4, 10240, 0, "2b", "78355e2f59605d1c2c7c46e915333ffded24c8ff"},
    {4096, 32, 32, 4, 16384, 0, "8b", "19ecab3fb31424ee937b7503730318b50e55771c"},
    {5120, 64, 64, 8, 25600, 1, "31b", "d6743d65c2cc61a07ff0fb2c3ff3cf7fd8ca36eb"},
};

static void set_profile_strings(const char *directory) {
    snprintf(plamo_vocab_path, sizeof plamo_vocab_path, "%s/tokenizer.jsonl", directory);
    snprintf(plamo_model_name, sizeof plamo_model_name, "plamo-3-translate-custom");
    plamo_model_repository[0] = plamo_model_revision[0] = 0;
    char path[4096 + 16], error[256];
    snprintf(path, sizeof path, "%s/config.json", directory);
    size_t size = 0;
    char *text = read_text(path, &size);
    struct plamo_checkpoint_config c;
    if (!text)
        return;
    const int ok = read_config(text, size, &c, error, sizeof error);
    free(text);
    for (size_t i = 0; ok && i < sizeof profiles / sizeof *profiles; ++i)
        if (profiles[i].hidden == c.hidden && profiles[i].layers == c.layers &&
            profiles[i].qh == c.qh && profiles[i].kh == c.kh &&
            profiles[i].intermediate == c.intermediate && profiles[i].tied == c.tied) {
            snprintf(plamo_model_name, sizeof plamo_model_name, "plamo-3-translate-%s",
                     profiles[i].size);
            snprintf(plamo_model_repository, sizeof plamo_model_repository, "pfnet/%s",
                     plamo_model_name);
            snprintf(plamo_model_revision, sizeof plamo_model_revision, "%s", profiles[i].revision);
        }
}

int plamo_model_set_directory(const char *directory) {
    if (!directory || strlen(directory) >= sizeof model_directory || opened)
        return 0;
    strcpy(model_directory, directory);
    set_profile_strings(directory);
    return 1;
}

/* The generated profile is part of the reference binary, so its strings exist
 * before main(); here $PLAMO_MODEL_DIR plays that part when the library loads. */
__attribute__((constructor)) static void model_directory_from_environment(void) {
    const char *dir = getenv("PLAMO_MODEL_DIR");
    if (dir && *dir)
        (void)plamo_model_set_directory(dir);
}

/* src/model_init.s:1-25: check every slot, then store. */
int plamo_model_patch(void *patches) {
    const uint64_t *p = patches;
    for (const uint64_t *q = p; q[0]; q += 2)
        if (!*(void *const *)(uintptr_t)q[1])
            return 0;
    for (; p[0]; p += 2)
        *(void **)(uintptr_t)p[0] = *(void *const *)(uintptr_t)p[1];
    return 1;
}

/* The descriptor fields each schema entry feeds, in build_schema's order. */
static void build_patches(const struct plamo_checkpoint *ck, struct model *m) {
    const struct plamo_checkpoint_config *c = &ck->config;
    size_t n = 0;
#define PATCH(field, entry)                                                                        \
    do {                                                                                           \
        plamo_model_patches[2 * n] = (uint64_t)(uintptr_t) & (field);                              \
        plamo_model_patches[2 * n + 1] = (uint64_t)(uintptr_t)ck->schema[entry].slot;              \
        ++n;                                                                                       \
    } while (0)
    PATCH(m->embedding, 0);
    PATCH(m->norm, 1);
    PATCH(m->head, c->tied ? 0 : 2);
    const size_t base = c->tied ? 2 : 3;
    for (uint64_t i = 0; i < c->layers; ++i) {
        struct layer *l = m->layers[i];
        const size_t e = base + 10 * i;
        PATCH(l->mixer->qkv->weight, e + 0);
        PATCH(l->mixer->weight, e + 1);
        PATCH(l->mixer->qkv->qn, e + 2);
        PATCH(l->mixer->qkv->kn, e + 3);
        PATCH(l->mlp->gu, e + 4);
        PATCH(l->mlp->down, e + 5);
        PATCH(l->pre, e + 6);
        PATCH(l->post, e + 7);
        PATCH(l->mlp->pre, e + 8);
        PATCH(l->mlp->post, e + 9);
    }
#undef PATCH
    plamo_model_patches[2 * n] = plamo_model_patches[2 * n + 1] = 0;
}

int plamo_model_open(void) {
    if (opened)
        return 1;
    const char *dir = model_directory[0] ? model_directory : getenv("PLAMO_MODEL_DIR");
    if (!dir) {
        fprintf(stderr, "plamo_model_open: no model directory (plamo_model_set_directory or "
                        "PLAMO_MODEL_DIR)\n");
        return 0;
    }
    char error[512];
    struct plamo_checkpoint *ck = plamo_checkpoint_open(dir, 0, error, sizeof error);
    if (!ck) {
        fprintf(stderr, "plamo_model_open: %s\n", error);
        return 0;
    }
    if (ck->config.layers > (PLAMO_MAX_SCHEMA - 4) / 10) {
        fprintf(stderr, "plamo_model_open: %llu layers exceed the engine tables\n",
                (unsigned long long)ck->config.layers);
        plamo_checkpoint_close(ck);
        return 0;
    }
    /* Page-locked host arrays when the runtime grants them (the backend then
     * writes them in place), ordinary mappings otherwise. */
    struct plamo_synthetic_instance *in = plamo_checkpoint_instantiate(ck, 1, error, sizeof error);
    if (!in)
        in = plamo_checkpoint_instantiate(ck, 0, error, sizeof error);
    if (!in) {
        fprintf(stderr, "plamo_model_open: %s\n", error);
        plamo_checkpoint_close(ck);
        return 0;
    }
    if (!model_directory[0])
        set_profile_strings(dir);
    plamo_model = *plamo_synthetic_model(in);
    for (size_t i = 0; i < ck->count; ++i) {
        plamo_weight_mappings[i] = ck->maps[i];
        plamo_weight_fds[i] = ck->fds[i];
    }
    plamo_weight_mapping_count = plamo_weight_file_count = ck->count;
    size_t n = 0;
    for (const struct plamo_weight_spec *s = ck->schema; s->name; ++s)
        plamo_weight_schema[n++] = *s;
    plamo_weight_schema[n] = (struct plamo_weight_spec){0};
    build_patches(ck, &plamo_model);
    opened = ck;
    opened_instance = in;
    return 1;
}
