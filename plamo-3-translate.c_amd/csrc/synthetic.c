/* Synthetic PLaMo-3 descriptor graphs with seeded BF16 weights.
 *
 * Layout rules follow the reference generator (tools/model_layout.py:71-199):
 * one workspace shared by all layers (state, normalized, branch, QKV output,
 * attention output, MLP scratch, scores, cos/sin scratch, logits), per-layer
 * raw-K / V / rotated-K buffers, sliding layers with window+1 rows, every
 * pattern-th layer global with the YaRN frequencies and concentration
 * (tools/rope_constants.py:21-70). Weight values come from a 65536-entry
 * normal quantile table indexed by splitmix64 output, so generation is cheap
 * and independent of the thread count.
 */
#define _GNU_SOURCE
#include "layout.h"
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

enum { TABLE = 65536, CHUNK = 1 << 20 };

struct tensor {
    uint64_t offset, count; /* in BF16 elements */
    uint64_t seed;
    int embedding;          /* uses embedding_std */
};

struct layer_weights {
    uint64_t pre, post, qkv, qn, kn, o, mlp_pre, mlp_post, gu, down;
};

struct plamo_synthetic {
    struct plamo_synthetic_config config;
    struct plamo_mapping mapping;
    uint16_t *arena;
    uint64_t embedding, head, norm;
    struct layer_weights *layers;
    float *local_freq, *global_freq;
    float local_scale, global_scale;
    uint16_t weight_table[TABLE], embedding_table[TABLE];
};

struct allocation {
    void *base;
    size_t bytes;
    int pinned;
};

struct plamo_synthetic_instance {
    struct model model;
    struct layer *layer;
    struct layer **layers;
    struct mixer *mixer;
    struct qkv *qkv;
    struct cache *cache;
    struct rotation *rotation;
    struct gqa *gqa;
    struct mlp *mlp;
    float *scales;
    struct allocation *allocations;
    size_t count, capacity;
};

static uint64_t splitmix64(uint64_t *state) {
    uint64_t z = (*state += UINT64_C(0x9e3779b97f4a7c15));
    z = (z ^ (z >> 30)) * UINT64_C(0xbf58476d1ce4e5b9);
    z = (z ^ (z >> 27)) * UINT64_C(0x94d049bb133111eb);
    return z ^ (z >> 31);
}

static uint16_t to_bf16(float value) {
    uint32_t u;
    memcpy(&u, &value, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Standard normal quantile of p by bisection on the CDF 0.5*erfc(-x/sqrt 2). */
static double normal_quantile(double p) {
    double lo = -12, hi = 12;
    for (int i = 0; i < 80; ++i) {
        double mid = 0.5 * (lo + hi);
        if (0.5 * erfc(-mid / M_SQRT2) < p)
            lo = mid;
        else
            hi = mid;
    }
    return 0.5 * (lo + hi);
}

static void quantile_table(double *out) {
    static double cached[TABLE];
    static int ready;
    static pthread_mutex_t mutex = PTHREAD_MUTEX_INITIALIZER;
    pthread_mutex_lock(&mutex);
    if (!ready) {
        for (int i = 0; i < TABLE / 2; ++i) {
            double q = normal_quantile((i + 0.5) / TABLE);
            cached[i] = q;
            cached[TABLE - 1 - i] = -q;
        }
        ready = 1;
    }
    pthread_mutex_unlock(&mutex);
    memcpy(out, cached, sizeof cached);
}

/* tools/rope_constants.py:21-52, each fp() a float rounding. */
void plamo_layout_frequencies(double theta, uint64_t half, int yarn, double factor,
                              double original, double beta_fast, double beta_slow, float *out) {
    double low = 0, high = 0;
    if (yarn) {
        low = (double)half * log(original / (beta_fast * 2 * M_PI)) / log(theta);
        high = (double)half * log(original / (beta_slow * 2 * M_PI)) / log(theta);
    }
    for (uint64_t i = 0; i < half; ++i) {
        float frequency = (float)pow(theta, (double)i / (double)half);
        float value = (float)(1.0 / (double)frequency);
        if (yarn) {
            float low_f = (float)low;
            float numerator = (float)((double)i - (double)low_f);
            float denominator = (float)(high - low);
            float ramp = (float)((double)numerator / (double)denominator);
            double clamped = ramp < 0 ? 0 : ramp > 1 ? 1 : ramp;
            float mask = (float)(1.0 - clamped);
            float interpolated = (float)(1.0 / (double)(float)(factor * (double)frequency));
            float keep = (float)(1.0 - (double)mask);
            float a = (float)((double)interpolated * (double)keep);
            float b = (float)((double)value * (double)mask);
            value = (float)((double)a + (double)b);
        }
        out[i] = value;
    }
}

void plamo_synthetic_defaults(struct plamo_synthetic_config *c, uint64_t hidden, uint64_t layers,
                              uint64_t qh, uint64_t kh, uint64_t dim, uint64_t intermediate,
                              uint64_t vocab) {
    memset(c, 0, sizeof *c);
    c->hidden = hidden;
    c->layers = layers;
    c->qh = qh;
    c->kh = kh;
    c->dim = dim;
    c->intermediate = intermediate;
    c->vocab = vocab;
    /* docs/config.json: window 2048, pattern 8; the engine caps a request at
     * 4096 prompt + 4096 output tokens (runtime/engine.c:432-448), so global
     * layers get 8192 rows instead of the 262144-row virtual capacity. */
    c->window = 2048;
    c->global_capacity = 8192;
    c->pattern = 8;
    c->seed = 1;
    c->weight_std = 0.02;
    c->embedding_std = 0.02;
    c->local_theta = 10000;
    c->global_theta = 1000000;
    c->yarn_factor = 256;
    c->yarn_original = 4096;
    c->yarn_beta_fast = 32;
    c->yarn_beta_slow = 1;
}

struct fill_job {
    const struct plamo_synthetic *s;
    const struct tensor *tensors;
    size_t tensor_count;
    uint64_t next_chunk, total_chunks;
    uint64_t *chunk_starts; /* prefix sums of chunks per tensor */
    pthread_mutex_t mutex;
};

static void fill_chunk(const struct plamo_synthetic *s, const struct tensor *t, uint64_t chunk) {
    uint64_t first = chunk * CHUNK, end = first + CHUNK;
    if (end > t->count)
        end = t->count;
    uint64_t state = t->seed ^ (chunk * UINT64_C(0xd1b54a32d192ed03));
    const uint16_t *table = t->embedding ? s->embedding_table : s->weight_table;
    uint16_t *out = s->arena + t->offset;
    uint64_t i = first;
    for (; i + 4 <= end; i += 4) {
        uint64_t r = splitmix64(&state);
        out[i] = table[r & 0xffff];
        out[i + 1] = table[(r >> 16) & 0xffff];
        out[i + 2] = table[(r >> 32) & 0xffff];
        out[i + 3] = table[r >> 48];
    }
    uint64_t r = splitmix64(&state);
    for (; i < end; ++i, r >>= 16)
        out[i] = table[r & 0xffff];
}

static void *fill_worker(void *arg) {
    struct fill_job *job = arg;
    for (;;) {
        pthread_mutex_lock(&job->mutex);
        uint64_t global = job->next_chunk++;
        pthread_mutex_unlock(&job->mutex);
        if (global >= job->total_chunks)
            return NULL;
        size_t t = 0;
        while (global >= job->chunk_starts[t + 1])
            ++t;
        fill_chunk(job->s, &job->tensors[t], global - job->chunk_starts[t]);
    }
}

struct plamo_synthetic *plamo_synthetic_build(const struct plamo_synthetic_config *config,
                                              unsigned threads, char *error, size_t cap) {
    const struct plamo_synthetic_config *c = config;
    if (!c->hidden || !c->layers || !c->qh || !c->kh || c->qh % c->kh || !c->dim || c->dim % 2 ||
        !c->intermediate || !c->vocab || c->layers > 128) {
        snprintf(error, cap, "invalid synthetic model shape");
        return NULL;
    }
    struct plamo_synthetic *s = calloc(1, sizeof *s);
    if (!s) {
        snprintf(error, cap, "cannot allocate synthetic model");
        return NULL;
    }
    s->config = *c;
    s->layers = calloc(c->layers, sizeof *s->layers);
    s->local_freq = calloc(c->dim / 2, 4);
    s->global_freq = calloc(c->dim / 2, 4);
    size_t tensor_cap = 3 + 10 * c->layers;
    struct tensor *tensors = calloc(tensor_cap, sizeof *tensors);
    if (!s->layers || !s->local_freq || !s->global_freq || !tensors) {
        free(tensors);
        plamo_synthetic_free(s);
        snprintf(error, cap, "cannot allocate synthetic model");
        return NULL;
    }
    double quantiles[TABLE];
    quantile_table(quantiles);
    for (int i = 0; i < TABLE; ++i) {
        s->weight_table[i] = to_bf16((float)(quantiles[i] * c->weight_std));
        s->embedding_table[i] = to_bf16((float)(quantiles[i] * c->embedding_std));
    }
    plamo_layout_frequencies(c->local_theta, c->dim / 2, 0, 0, 0, 0, 0, s->local_freq);
    plamo_layout_frequencies(c->global_theta, c->dim / 2, 1, c->yarn_factor, c->yarn_original,
                             c->yarn_beta_fast, c->yarn_beta_slow, s->global_freq);
    s->local_scale = 1.0f;
    s->global_scale = (float)(1.0 + 0.1 * log(c->yarn_factor));

    /* Arena layout, every tensor 256-byte aligned. */
    uint64_t h = c->hidden, d = c->dim, qkv_rows = (c->qh + 2 * c->kh) * d;
    uint64_t offset = 0;
    size_t n = 0;
    uint64_t seed = c->seed;
#define PLACE(field, elements, emb)                                                                \
    do {                                                                                           \
        field = offset;                                                                            \
        tensors[n++] = (struct tensor){offset, (elements), splitmix64(&seed), (emb)};              \
        offset += ((elements) + 127) / 128 * 128;                                                  \
    } while (0)
    PLACE(s->embedding, c->vocab * h, 1);
    if (c->tied)
        s->head = s->embedding;
    else
        PLACE(s->head, c->vocab * h, 0);
    PLACE(s->norm, h, 0);
    for (uint64_t i = 0; i < c->layers; ++i) {
        struct layer_weights *w = &s->layers[i];
        PLACE(w->pre, h, 0);
        PLACE(w->post, h, 0);
        PLACE(w->qkv, qkv_rows * h, 0);
        PLACE(w->qn, d, 0);
        PLACE(w->kn, d, 0);
        PLACE(w->o, h * c->qh * d, 0);
        PLACE(w->mlp_pre, h, 0);
        PLACE(w->mlp_post, h, 0);
        PLACE(w->gu, 2 * c->intermediate * h, 0);
        PLACE(w->down, h * c->intermediate, 0);
    }
#undef PLACE
    uint64_t bytes = offset * 2;
    void *arena = mmap(NULL, bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (arena == MAP_FAILED) {
        free(tensors);
        plamo_synthetic_free(s);
        snprintf(error, cap, "cannot map %llu bytes of synthetic weights",
                 (unsigned long long)bytes);
        return NULL;
    }
    /* 2 MiB pages: a 17 GB arena otherwise costs millions of page faults. */
    (void)madvise(arena, bytes, MADV_HUGEPAGE);
    s->arena = arena;
    s->mapping.base = arena;
    s->mapping.bytes = bytes;

    struct fill_job job = {s, tensors, n, 0, 0, NULL, PTHREAD_MUTEX_INITIALIZER};
    job.chunk_starts = calloc(n + 1, sizeof *job.chunk_starts);
    if (!job.chunk_starts) {
        free(tensors);
        plamo_synthetic_free(s);
        snprintf(error, cap, "cannot allocate synthetic model");
        return NULL;
    }
    for (size_t i = 0; i < n; ++i)
        job.chunk_starts[i + 1] = job.chunk_starts[i] + (tensors[i].count + CHUNK - 1) / CHUNK;
    job.total_chunks = job.chunk_starts[n];
    if (threads < 1)
        threads = 1;
    if (threads > 64)
        threads = 64;
    pthread_t workers[64];
    unsigned started = 0;
    for (unsigned i = 1; i < threads; ++i)
        if (!pthread_create(&workers[started], NULL, fill_worker, &job))
            ++started;
    fill_worker(&job);
    for (unsigned i = 0; i < started; ++i)
        pthread_join(workers[i], NULL);
    free(job.chunk_starts);
    free(tensors);
    return s;
}

void plamo_synthetic_free(struct plamo_synthetic *s) {
    if (!s)
        return;
    if (s->arena)
        munmap(s->arena, s->mapping.bytes);
    free(s->layers);
    free(s->local_freq);
    free(s->global_freq);
    free(s);
}

const struct plamo_mapping *plamo_synthetic_weights(const struct plamo_synthetic *s) {
    return &s->mapping;
}

static int is_global(const struct plamo_synthetic_config *c, uint64_t layer) {
    return c->pattern && (layer + 1) % c->pattern == 0;
}

const float *plamo_synthetic_frequencies(const struct plamo_synthetic *s, uint64_t layer) {
    return is_global(&s->config, layer) ? s->global_freq : s->local_freq;
}

static void *allocate(struct plamo_synthetic_instance *in, uint64_t floats, int pinned) {
    if (in->count == in->capacity)
        return NULL;
    size_t bytes = (size_t)((floats * 4 + 4095) / 4096 * 4096);
    if (!bytes)
        bytes = 4096;
    void *base = NULL;
    if (pinned) {
        if (hipHostMalloc(&base, bytes, hipHostMallocDefault) != hipSuccess)
            return NULL;
        memset(base, 0, bytes);
    } else {
        base = mmap(NULL, bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
        if (base == MAP_FAILED)
            return NULL;
    }
    in->allocations[in->count++] = (struct allocation){base, bytes, pinned};
    return base;
}

static int layout_global(const struct plamo_layout *c, uint64_t layer) {
    return c->pattern && (layer + 1) % c->pattern == 0;
}

struct plamo_synthetic_instance *plamo_layout_instantiate(const struct plamo_layout *c, int pinned,
                                                          char *error, size_t cap) {
    uint64_t L = c->layers, h = c->hidden, d = c->dim;
    struct plamo_synthetic_instance *in = calloc(1, sizeof *in);
    if (!in) {
        snprintf(error, cap, "cannot allocate model instance");
        return NULL;
    }
    in->capacity = 16 + 3 * L;
    in->allocations = calloc(in->capacity, sizeof *in->allocations);
    in->layer = calloc(L, sizeof *in->layer);
    in->layers = calloc(L, sizeof *in->layers);
    in->mixer = calloc(L, sizeof *in->mixer);
    in->qkv = calloc(L, sizeof *in->qkv);
    in->cache = calloc(L, sizeof *in->cache);
    in->rotation = calloc(L, sizeof *in->rotation);
    in->gqa = calloc(L, sizeof *in->gqa);
    in->mlp = calloc(L, sizeof *in->mlp);
    in->scales = calloc(L, sizeof *in->scales);
    if (!in->allocations || !in->layer || !in->layers || !in->mixer || !in->qkv || !in->cache ||
        !in->rotation || !in->gqa || !in->mlp || !in->scales)
        goto fail;
    uint64_t max_capacity = c->window + 1;
    for (uint64_t i = 0; i < L; ++i)
        if (layout_global(c, i) && c->global_capacity > max_capacity)
            max_capacity = c->global_capacity;
    /* Shared workspace (tools/model_layout.py:183-196). */
    float *state = allocate(in, h, pinned), *normalized = allocate(in, h, pinned);
    float *branch = allocate(in, h, pinned);
    float *qkvout = allocate(in, (c->qh + 2 * c->kh) * d, pinned);
    float *attention = allocate(in, c->qh * d, pinned);
    float *mlpscratch = allocate(in, 2 * c->intermediate, pinned);
    float *scores = allocate(in, max_capacity, pinned);
    float *cos = allocate(in, d / 2, pinned), *sin = allocate(in, d / 2, pinned);
    float *logits = allocate(in, c->vocab, pinned);
    if (!state || !normalized || !branch || !qkvout || !attention || !mlpscratch || !scores ||
        !cos || !sin || !logits)
        goto fail;
    struct model *m = &in->model;
    m->embedding = c->embedding;
    m->vocab = c->vocab;
    m->hidden = h;
    m->state = state;
    m->layers = in->layers;
    m->count = L;
    m->scales = in->scales;
    m->norm = c->norm;
    m->normalized = normalized;
    m->head = c->head;
    m->logits = logits;
    for (uint64_t i = 0; i < L; ++i) {
        const struct plamo_layout_layer *lw = &c->layer[i];
        int global = layout_global(c, i);
        uint64_t capacity = global ? c->global_capacity : c->window + 1;
        struct cache *cache = &in->cache[i];
        cache->capacity = capacity;
        cache->width = c->kh * d;
        cache->sliding = !global;
        cache->k = allocate(in, capacity * cache->width, pinned);
        cache->v = allocate(in, capacity * cache->width, pinned);
        float *rotated = allocate(in, capacity * cache->width, pinned);
        if (!cache->k || !cache->v || !rotated)
            goto fail;
        struct rotation *r = &in->rotation[i];
        *r = (struct rotation){cache, rotated, global ? c->global_freq : c->local_freq, cos, sin,
                               c->kh, d, 0, 0};
        struct qkv *q = &in->qkv[i];
        *q = (struct qkv){normalized, lw->qkv, lw->qn, lw->kn, qkvout, h, c->qh, c->kh, d};
        struct gqa *g = &in->gqa[i];
        *g = (struct gqa){qkvout, rotated, cache->v, attention, scores, 0, d, c->qh, c->kh};
        struct mixer *mx = &in->mixer[i];
        *mx = (struct mixer){q, cache, r, g, lw->o, branch, h};
        struct mlp *p = &in->mlp[i];
        *p = (struct mlp){state, lw->mlp_pre, lw->mlp_post, lw->gu, lw->down, normalized, branch,
                          mlpscratch, h, c->intermediate};
        struct layer *l = &in->layer[i];
        *l = (struct layer){state, lw->pre, lw->post, normalized, branch, mx, p, h};
        in->layers[i] = l;
        in->scales[i] = global ? c->global_scale : c->local_scale;
    }
    return in;
fail:
    snprintf(error, cap, "cannot allocate model instance buffers");
    plamo_synthetic_release(in);
    return NULL;
}

struct plamo_synthetic_instance *plamo_synthetic_instantiate(const struct plamo_synthetic *s,
                                                             int pinned, char *error, size_t cap) {
    const struct plamo_synthetic_config *c = &s->config;
    struct plamo_layout_layer *layers = calloc(c->layers, sizeof *layers);
    if (!layers) {
        snprintf(error, cap, "cannot allocate model instance");
        return NULL;
    }
    const uint16_t *w = s->arena;
    for (uint64_t i = 0; i < c->layers; ++i) {
        const struct layer_weights *lw = &s->layers[i];
        layers[i] = (struct plamo_layout_layer){w + lw->pre,     w + lw->post,     w + lw->qkv,
                                                w + lw->qn,      w + lw->kn,       w + lw->o,
                                                w + lw->mlp_pre, w + lw->mlp_post, w + lw->gu,
                                                w + lw->down};
    }
    struct plamo_layout lay = {c->hidden,    c->layers,         c->qh,
                               c->kh,        c->dim,            c->intermediate,
                               c->vocab,     c->window,         c->global_capacity,
                               c->pattern,   w + s->embedding,  w + s->head,
                               w + s->norm,  layers,            s->local_freq,
                               s->global_freq, s->local_scale,  s->global_scale};
    struct plamo_synthetic_instance *in = plamo_layout_instantiate(&lay, pinned, error, cap);
    free(layers);
    return in;
}

void plamo_synthetic_release(struct plamo_synthetic_instance *in) {
    if (!in)
        return;
    for (size_t i = 0; i < in->count; ++i) {
        if (in->allocations[i].pinned)
            (void)hipHostFree(in->allocations[i].base);
        else
            munmap(in->allocations[i].base, in->allocations[i].bytes);
    }
    free(in->allocations);
    free(in->layer);
    free(in->layers);
    free(in->mixer);
    free(in->qkv);
    free(in->cache);
    free(in->rotation);
    free(in->gqa);
    free(in->mlp);
    free(in->scales);
    free(in);
}

struct model *plamo_synthetic_model(struct plamo_synthetic_instance *in) {
    return &in->model;
}

/* Raw K and V ~ N(0,1) via Box-Muller on splitmix64 doubles. */
int plamo_synthetic_fill_kv(struct plamo_synthetic_instance *in, uint64_t rows, uint64_t seed) {
    struct model *m = &in->model;
    for (uint64_t i = 0; i < m->count; ++i) {
        struct cache *c = m->layers[i]->mixer->cache;
        if (rows > c->capacity)
            return 0;
    }
    for (uint64_t i = 0; i < m->count; ++i) {
        struct mixer *mx = m->layers[i]->mixer;
        struct cache *c = mx->cache;
        uint64_t state = seed ^ (i * UINT64_C(0x9e3779b97f4a7c15));
        float *targets[2] = {c->k, c->v};
        for (int t = 0; t < 2; ++t)
            for (uint64_t j = 0; j < rows * c->width; j += 2) {
                double u1 = ((splitmix64(&state) >> 11) + 0.5) * 0x1.0p-53;
                double u2 = (splitmix64(&state) >> 11) * 0x1.0p-53;
                double radius = sqrt(-2.0 * log(u1));
                targets[t][j] = (float)(radius * cos(2 * M_PI * u2));
                if (j + 1 < rows * c->width)
                    targets[t][j + 1] = (float)(radius * sin(2 * M_PI * u2));
            }
        c->count = rows;
        mx->rotation->processed_count = 0;
        mx->rotation->scale_bits = 0;
    }
    return 1;
}
