/* CPU oracle of the PLaMo-3-Translate token loop — TEST INFRASTRUCTURE ONLY.
 * Used by tests/ and by bench.py's cpu_baseline leg; never by the product.
 *
 * Parity status of every function is listed in the header comment of the
 * test that pins it (tests/test_oracle_*.py). Op order follows the reference
 * line by line; "fmaf" marks the places the reference fuses (fmla/fmadd/fmsub).
 */
#define _GNU_SOURCE
#include "plamo_oracle.h"
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

float oracle_bf16(uint16_t bits) {
    /* src/token.s:16-25: widening is a 16-bit shift. */
    uint32_t u = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t oracle_to_bf16(float value) {
    /* Round to nearest even (used only to build synthetic fixtures). */
    uint32_t u;
    memcpy(&u, &value, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* tests/activation_reference.s:6-48 (constants :129-132). */
float oracle_exp(float x) {
    if (!(x >= -87.0f)) /* b.lt is taken for NaN too */
        return 0.0f;
    if (x > 88.0f)
        return INFINITY;
    float n = rintf(x * 1.4426950408889634f);
    int32_t i = (int32_t)n;
    float r = fmaf(-n, 0.6931471805599453f, x);
    float p = fmaf(0.0001984126984126984f, r, 0.001388888888888889f);
    p = fmaf(p, r, 0.008333333333333333f);
    p = fmaf(p, r, 0.041666666666666664f);
    p = fmaf(p, r, 0.16666666666666666f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    uint32_t bits = (uint32_t)(i + 127) << 23;
    float scale;
    memcpy(&scale, &bits, 4);
    return p * scale;
}

/* tests/activation_reference.s:51-95: sequential max, exp, sequential sum, divide. */
void oracle_softmax(float *x, uint64_t n) {
    if (!n)
        return;
    float m = x[0];
    for (uint64_t i = 1; i < n; ++i)
        m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        float e = oracle_exp(x[i] - m);
        x[i] = e;
        sum = sum + e;
    }
    for (uint64_t i = 0; i < n; ++i)
        x[i] = x[i] / sum;
}

/* tests/activation_reference.s:99-126: out = g / (exp(-g) + 1) * u. */
void oracle_swiglu(const float *gate_up, float *out, uint64_t n) {
    const float *up = gate_up + n;
    for (uint64_t i = 0; i < n; ++i) {
        float g = gate_up[i];
        float d = oracle_exp(-g) + 1.0f;
        out[i] = (g / d) * up[i];
    }
}

/* tests/matvec_reference.s:6-32: four FMA lanes over k mod 4, the pairwise
 * (a0+a1)+(a2+a3) reduction, then a sequential FMA tail. */
static void matvec_rows(const uint16_t *w, const float *x, float *y, uint64_t rows,
                        uint64_t cols) {
    uint64_t body = cols / 4 * 4;
    for (uint64_t r = 0; r < rows; ++r) {
        const uint16_t *row = w + r * cols;
        float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        for (uint64_t k = 0; k < body; k += 4) {
            a0 = fmaf(oracle_bf16(row[k]), x[k], a0);
            a1 = fmaf(oracle_bf16(row[k + 1]), x[k + 1], a1);
            a2 = fmaf(oracle_bf16(row[k + 2]), x[k + 2], a2);
            a3 = fmaf(oracle_bf16(row[k + 3]), x[k + 3], a3);
        }
        float s = (a0 + a1) + (a2 + a3);
        for (uint64_t k = body; k < cols; ++k)
            s = fmaf(oracle_bf16(row[k]), x[k], s);
        y[r] = s;
    }
}

/* The same products for a block of tokens (src/matmul.s:1-4: a matmul is,
 * bit for bit, one matvec per token). Each weight row is widened once per
 * block of TOKEN_BLOCK tokens; the block's inputs are interleaved in pairs of
 * tokens ([x_a(k..k+3) | x_b(k..k+3)] for every k step of 4), so one 8-wide
 * fused multiply-add serves two tokens. Per token the arithmetic is
 * matvec_rows' own: lane l accumulates k = l mod 4, then (a0 + a1) +
 * (a2 + a3), then the sequential tail; the tokens only share the weight loads. */
enum { TOKEN_BLOCK = 64 };

static __thread float *widened, *pairs;
static __thread uint64_t widened_cols;

/* BF16 -> FP32 of a row, eight at a time (the 16-bit shift of oracle_bf16). */
static void widen_row(const uint16_t *src, float *dst, uint64_t cols) {
    uint64_t k = 0;
    for (; k + 8 <= cols; k += 8) {
        __m256i v = _mm256_cvtepu16_epi32(_mm_loadu_si128((const __m128i *)(src + k)));
        _mm256_storeu_si256((__m256i *)(dst + k), _mm256_slli_epi32(v, 16));
    }
    for (; k < cols; ++k)
        dst[k] = oracle_bf16(src[k]);
}

static void lanes_to_sums(__m256 acc, const float *w, const float *xa, const float *xb,
                          uint64_t cols, float *ya, float *yb) {
    uint64_t body = cols / 4 * 4;
    float l[8];
    _mm256_storeu_ps(l, acc);
    float sa = (l[0] + l[1]) + (l[2] + l[3]), sb = (l[4] + l[5]) + (l[6] + l[7]);
    for (uint64_t k = body; k < cols; ++k) {
        sa = fmaf(w[k], xa[k], sa);
        sb = fmaf(w[k], xb[k], sb);
    }
    *ya = sa;
    if (yb)
        *yb = sb;
}

static void matmul_rows(const uint16_t *w, const float *x, uint64_t x_stride, float *y,
                        uint64_t y_stride, uint64_t rows, uint64_t cols, uint64_t tokens) {
    enum { RB = 4 };  /* weight rows per register block (times two token pairs) */
    const uint64_t body = cols / 4 * 4;
    if (widened_cols < cols) {
        free(widened);
        free(pairs);
        widened = malloc(RB * cols * sizeof(float));
        pairs = malloc((uint64_t)TOKEN_BLOCK * (body + 4) * sizeof(float));
        widened_cols = widened && pairs ? cols : 0;
        if (!widened_cols)
            abort();
    }
    for (uint64_t t0 = 0; t0 < tokens; t0 += TOKEN_BLOCK) {
        const uint64_t t1 = t0 + TOKEN_BLOCK < tokens ? t0 + TOKEN_BLOCK : tokens;
        const uint64_t np = (t1 - t0 + 1) / 2;  /* token pairs (the last may be single) */
        for (uint64_t p = 0; p < np; ++p) {
            const float *xa = x + (t0 + 2 * p) * x_stride;
            const float *xb = t0 + 2 * p + 1 < t1 ? xa + x_stride : xa;
            float *dst = pairs + p * 2 * body;
            for (uint64_t k = 0; k < body; k += 4) {
                memcpy(dst + 2 * k, xa + k, 16);
                memcpy(dst + 2 * k + 4, xb + k, 16);
            }
        }
        for (uint64_t r0 = 0; r0 < rows; r0 += RB) {
            const uint64_t nr = rows - r0 < RB ? rows - r0 : RB;
            for (uint64_t i = 0; i < RB; ++i)
                widen_row(w + (r0 + (i < nr ? i : 0)) * cols, widened + i * cols, cols);
            const float *w0 = widened, *w1 = w0 + cols, *w2 = w1 + cols, *w3 = w2 + cols;
            for (uint64_t p = 0; p < np; p += 2) {
                const uint64_t q = np - p < 2 ? np - p : 2;
                const float *x0 = pairs + p * 2 * body, *x1 = pairs + (p + q - 1) * 2 * body;
                __m256 a00 = _mm256_setzero_ps(), a01 = a00, a10 = a00, a11 = a00, a20 = a00,
                       a21 = a00, a30 = a00, a31 = a00;
                for (uint64_t k = 0; k < body; k += 4) {
                    const __m256 v0 = _mm256_loadu_ps(x0 + 2 * k), v1 = _mm256_loadu_ps(x1 + 2 * k);
                    __m256 b = _mm256_broadcast_ps((const __m128 *)(w0 + k));
                    a00 = _mm256_fmadd_ps(b, v0, a00);
                    a01 = _mm256_fmadd_ps(b, v1, a01);
                    b = _mm256_broadcast_ps((const __m128 *)(w1 + k));
                    a10 = _mm256_fmadd_ps(b, v0, a10);
                    a11 = _mm256_fmadd_ps(b, v1, a11);
                    b = _mm256_broadcast_ps((const __m128 *)(w2 + k));
                    a20 = _mm256_fmadd_ps(b, v0, a20);
                    a21 = _mm256_fmadd_ps(b, v1, a21);
                    b = _mm256_broadcast_ps((const __m128 *)(w3 + k));
                    a30 = _mm256_fmadd_ps(b, v0, a30);
                    a31 = _mm256_fmadd_ps(b, v1, a31);
                }
                const __m256 acc[RB][2] = {{a00, a01}, {a10, a11}, {a20, a21}, {a30, a31}};
                for (uint64_t i = 0; i < nr; ++i)
                    for (uint64_t j = 0; j < q; ++j) {
                        const uint64_t ta = t0 + 2 * (p + j), tb = ta + 1;
                        const float *xa = x + ta * x_stride;
                        const int two = tb < t1;
                        lanes_to_sums(acc[i][j], widened + i * cols, xa,
                                      two ? xa + x_stride : xa, cols, y + ta * y_stride + r0 + i,
                                      two ? y + tb * y_stride + r0 + i : NULL);
                    }
            }
        }
    }
}

/* Row-split thread pool for the CPU baseline: rows are cut in groups of 24
 * and handed out in contiguous slices, as runtime/parallel.c:35-48 does.
 * Splitting rows does not change any row's arithmetic. A job is one matvec
 * (tokens == 1) or the token-blocked products of a prompt. */
enum { ROW_GROUP = 24, MAX_THREADS = 64 };
static struct {
    pthread_mutex_t mutex;
    pthread_cond_t start, done;
    pthread_t threads[MAX_THREADS];
    unsigned count, created, pending;  /* active threads, worker threads made + 1 */
    uint64_t generation;
    const uint16_t *w;
    const float *x;
    float *y;
    uint64_t rows, cols, tokens, x_stride, y_stride;
} pool = {.mutex = PTHREAD_MUTEX_INITIALIZER, .start = PTHREAD_COND_INITIALIZER,
          .done = PTHREAD_COND_INITIALIZER};

static void pool_slice(unsigned index) {
    uint64_t groups = (pool.rows + ROW_GROUP - 1) / ROW_GROUP;
    uint64_t first = groups * index / pool.count * ROW_GROUP;
    uint64_t end = groups * (index + 1) / pool.count * ROW_GROUP;
    if (end > pool.rows)
        end = pool.rows;
    if (first >= end)
        return;
    if (pool.tokens == 1)
        matvec_rows(pool.w + first * pool.cols, pool.x, pool.y + first, end - first, pool.cols);
    else
        matmul_rows(pool.w + first * pool.cols, pool.x, pool.x_stride, pool.y + first,
                    pool.y_stride, end - first, pool.cols, pool.tokens);
}

static void *pool_main(void *arg) {
    unsigned index = (unsigned)(uintptr_t)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&pool.mutex);
    for (;;) {
        while (seen == pool.generation)
            pthread_cond_wait(&pool.start, &pool.mutex);
        seen = pool.generation;
        if (index >= pool.count)
            continue; /* idle at the current thread count */
        pthread_mutex_unlock(&pool.mutex);
        pool_slice(index);
        pthread_mutex_lock(&pool.mutex);
        if (!--pool.pending)
            pthread_cond_signal(&pool.done);
    }
    return NULL;
}

void oracle_set_threads(unsigned threads) {
    if (threads < 1)
        threads = 1;
    if (threads > MAX_THREADS)
        threads = MAX_THREADS;
    pthread_mutex_lock(&pool.mutex);
    /* Index 0 is the calling thread. Workers are made once and stay; those at
     * or past the active count sit out each job. */
    for (unsigned i = pool.created ? pool.created : 1; i < threads; ++i)
        pthread_create(&pool.threads[i], NULL, pool_main, (void *)(uintptr_t)i);
    if (threads > pool.created)
        pool.created = threads;
    pool.count = threads;
    pthread_mutex_unlock(&pool.mutex);
}

unsigned oracle_threads(void) {
    return pool.count ? pool.count : 1;
}

static void run_pool(const uint16_t *w, const float *x, uint64_t x_stride, float *y,
                     uint64_t y_stride, uint64_t rows, uint64_t cols, uint64_t tokens) {
    unsigned threads = oracle_threads();
    if (threads <= 1 || rows < (uint64_t)threads * ROW_GROUP || rows * cols < 256 * 1024) {
        if (tokens == 1)
            matvec_rows(w, x, y, rows, cols);
        else
            matmul_rows(w, x, x_stride, y, y_stride, rows, cols, tokens);
        return;
    }
    pthread_mutex_lock(&pool.mutex);
    pool.w = w;
    pool.x = x;
    pool.y = y;
    pool.rows = rows;
    pool.cols = cols;
    pool.tokens = tokens;
    pool.x_stride = x_stride;
    pool.y_stride = y_stride;
    pool.pending = threads - 1;
    ++pool.generation;
    pthread_cond_broadcast(&pool.start);
    pthread_mutex_unlock(&pool.mutex);
    pool_slice(0);
    pthread_mutex_lock(&pool.mutex);
    while (pool.pending)
        pthread_cond_wait(&pool.done, &pool.mutex);
    pthread_mutex_unlock(&pool.mutex);
}

void oracle_matvec(const uint16_t *w, const float *x, float *y, uint64_t rows, uint64_t cols) {
    run_pool(w, x, 0, y, 0, rows, cols, 1);
}

/* src/matmul.s:1-4: a matmul is, bit for bit, one matvec per token. */
void oracle_matmul(const struct plamo_matmul *m) {
    for (uint64_t t = 0; t < m->tokens; ++t)
        oracle_matvec(m->weights, m->input + t * m->input_stride, m->output + t * m->output_stride,
                      m->rows, m->columns);
}

/* The token-blocked form of oracle_matmul (the same bits; the prefill's
 * projections use it, as the reference's prompt path runs GEMM tiles,
 * src/matmul8x3.s). */
void oracle_matmul_blocked(const struct plamo_matmul *m) {
    if (!m->tokens)
        return;
    if (m->tokens == 1) {
        oracle_matvec(m->weights, m->input, m->output, m->rows, m->columns);
        return;
    }
    run_pool(m->weights, m->input, m->input_stride, m->output, m->output_stride, m->rows,
             m->columns, m->tokens);
}

/* tests/rmsnorm_reference.s:8-34. */
void oracle_rmsnorm(const float *x, const uint16_t *w, float *y, uint64_t n, float eps,
                    float offset) {
    if (!n)
        return;
    float ss = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        float t = x[i] * x[i];
        ss = ss + t;
    }
    float ms = ss / (float)n;
    ms = ms + eps;
    float r = sqrtf(ms);
    float inv = 1.0f / r;
    for (uint64_t i = 0; i < n; ++i) {
        float scale = oracle_bf16(w[i]) + offset;
        y[i] = (x[i] * inv) * scale;
    }
}

/* src/model.s:41-62 */
void oracle_residual(float *state, const float *branch, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i)
        state[i] = state[i] + branch[i];
}

/* tests/attention_reference.s:9-71. */
void oracle_attention_head(const float *q, const float *k, const float *v, float *out,
                           float *scores, uint64_t n, uint64_t d, uint64_t stride) {
    float scale = 1.0f / sqrtf((float)d);
    for (uint64_t t = 0; t < n; ++t) {
        float s = 0.0f;
        for (uint64_t j = 0; j < d; ++j)
            s = fmaf(q[j], k[t * stride + j], s);
        scores[t] = s * scale;
    }
    oracle_softmax(scores, n);
    for (uint64_t j = 0; j < d; ++j) {
        float s = 0.0f;
        for (uint64_t t = 0; t < n; ++t)
            s = fmaf(scores[t], v[t * stride + j], s);
        out[j] = s;
    }
}

/* tests/attention_reference.s:78-112: q head h reads kv head h / (qh / kh). */
void oracle_gqa(const struct gqa *g) {
    uint64_t group = g->qh / g->kh, stride = g->kh * g->dim;
    for (uint64_t h = 0; h < g->qh; ++h) {
        uint64_t kv = h / group;
        oracle_attention_head(g->q + h * g->dim, g->k + kv * g->dim, g->v + kv * g->dim,
                              g->out + h * g->dim, g->scores, g->tokens, g->dim, stride);
    }
}

/* tests/rope_reference.s:14-30 / src/rope.s:15-58: separate mul/sub/add, no FMA. */
void oracle_rope_copy(const float *src, float *dst, const float *cos, const float *sin,
                      uint64_t heads, uint64_t half) {
    for (uint64_t h = 0; h < heads; ++h) {
        const float *a = src + h * 2 * half;
        float *o = dst + h * 2 * half;
        for (uint64_t j = 0; j < half; ++j) {
            float x0 = a[j], x1 = a[j + half], c = cos[j], s = sin[j];
            float p0 = x0 * c, p1 = x1 * s;
            float r0 = p0 - p1;
            float p2 = x1 * c, p3 = x0 * s;
            float r1 = p2 + p3;
            o[j] = r0;
            o[j + half] = r1;
        }
    }
}

/* src/trig.s:5-44: double range reduction by 2*pi, Taylor polynomials in r^2. */
void oracle_sincos(double angle, float out[2]) {
    static const double two_pi = 6.283185307179586;
    static const double sin_c[8] = {2.8114572543455206e-15, -7.647163731819816e-13,
                                    1.6059043836821613e-10, -2.505210838544172e-08,
                                    2.7557319223985893e-06, -0.0001984126984126984,
                                    0.008333333333333333,   -0.16666666666666666};
    static const double cos_c[8] = {4.779477332387385e-14,  -1.1470745597729725e-11,
                                    2.08767569878681e-09,   -2.755731922398589e-07,
                                    2.48015873015873e-05,   -0.001388888888888889,
                                    0.041666666666666664,   -0.5};
    double n = rint(angle / two_pi);
    double r = fma(-n, two_pi, angle);
    double r2 = r * r;
    double p = sin_c[0];
    for (int i = 1; i < 8; ++i)
        p = fma(p, r2, sin_c[i]);
    p = fma(p, r2, 1.0);
    out[0] = (float)(p * r);
    p = cos_c[0];
    for (int i = 1; i < 8; ++i)
        p = fma(p, r2, cos_c[i]);
    p = fma(p, r2, 1.0);
    out[1] = (float)p;
}

/* src/rope_table.s:5-30: FP32 angle, double sincos, FP32 concentration. */
void oracle_rope_table(const float *freq, uint64_t position, uint64_t half, float *cos,
                       float *sin, float scale) {
    float p = (float)position;
    for (uint64_t j = 0; j < half; ++j) {
        float angle = freq[j] * p;
        float sc[2];
        oracle_sincos((double)angle, sc);
        sin[j] = sc[0] * scale;
        cos[j] = sc[1] * scale;
    }
}

/* tools/rope_constants.py:21-52: every fp() is a float rounding. */
void oracle_rope_frequencies(double theta, uint64_t half, int yarn, double factor,
                             double original_max_positions, double beta_fast, double beta_slow,
                             float *out) {
    double low = 0, high = 0;
    if (yarn) {
        low = (double)half * log(original_max_positions / (beta_fast * 2 * M_PI)) / log(theta);
        high = (double)half * log(original_max_positions / (beta_slow * 2 * M_PI)) / log(theta);
    }
    for (uint64_t i = 0; i < half; ++i) {
        float frequency = (float)pow(theta, (double)i / (double)half);
        float extrapolated = (float)(1.0 / (double)frequency);
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
            float b = (float)((double)extrapolated * (double)mask);
            extrapolated = (float)((double)a + (double)b);
        }
        out[i] = extrapolated;
    }
}

/* tools/rope_constants.py:68-70 */
float oracle_rope_concentration(int yarn, double factor) {
    return yarn ? (float)(1.0 + 0.1 * log(factor)) : 1.0f;
}

/* tests/cache_reference.s:8-56: append unrotated K and V at row count; a full
 * sliding cache drops its oldest row first; a full global cache refuses. */
int oracle_cache_append(struct cache *c, const float *k, const float *v) {
    if (!c->capacity || !c->width || c->count > c->capacity)
        return 0;
    uint64_t count = c->count;
    if (count == c->capacity) {
        if (!c->sliding)
            return 0;
        uint64_t words = (c->capacity - 1) * c->width;
        for (uint64_t i = 0; i < words; ++i) {
            c->k[i] = c->k[i + c->width];
            c->v[i] = c->v[i + c->width];
        }
        --count;
    }
    memcpy(c->k + count * c->width, k, c->width * 4);
    memcpy(c->v + count * c->width, v, c->width * 4);
    c->count = count + 1;
    return 1;
}

/* src/cache_rope.s:11-75: reuse rotated rows when exactly one row was added at
 * the same concentration, otherwise rotate every row at its local position.
 * The cos/sin scratch is left holding the table of row count-1. */
void oracle_cache_rope_cached(struct rotation *r, float scale) {
    uint32_t bits;
    memcpy(&bits, &scale, 4);
    uint64_t count = r->cache->count, start = 0;
    if (count) {
        if (r->scale_bits == (uint64_t)bits && r->processed_count + 1 == count)
            start = r->processed_count;
        uint64_t width = r->cache->width, half = r->dim / 2;
        for (uint64_t row = start; row < count; ++row) {
            oracle_rope_table(r->freq, row, half, r->cos, r->sin, scale);
            oracle_rope_copy(r->cache->k + row * width, r->out + row * width, r->cos, r->sin,
                             r->heads, half);
        }
    }
    r->processed_count = count;
    r->scale_bits = bits;
}

/* src/qkv.s:36-67: offset-1 RMSNorm on every Q and K head; V untouched. */
void oracle_qk_norm(float *qkv, const uint16_t *qn, const uint16_t *kn, uint64_t qh, uint64_t kh,
                    uint64_t dim) {
    for (uint64_t h = 0; h < qh + kh; ++h)
        oracle_rmsnorm(qkv + h * dim, h < qh ? qn : kn, qkv + h * dim, dim, 0.000001f, 1.0f);
}

/* src/qkv.s:7-32 */
void oracle_qkv(const struct qkv *q) {
    oracle_matvec(q->weight, q->input, q->out, (q->qh + 2 * q->kh) * q->dim, q->hidden);
    oracle_qk_norm(q->out, q->qn, q->kn, q->qh, q->kh, q->dim);
}

/* src/mixer.s:33-80: append, refresh rotated keys, rotate Q at row count-1,
 * attend over every cached row. */
int oracle_mixer_attention(struct mixer *m, float *qkv_out, float *attention_out, float scale) {
    struct cache *c = m->cache;
    const struct qkv *q = m->qkv;
    struct rotation *r = m->rotation;
    float *k = qkv_out + q->qh * q->dim, *v = k + c->width;
    if (!oracle_cache_append(c, k, v))
        return 0;
    oracle_cache_rope_cached(r, scale);
    oracle_rope_copy(qkv_out, qkv_out, r->cos, r->sin, q->qh, q->dim / 2);
    struct gqa g = {qkv_out,       r->out,      c->v,        attention_out, m->gqa->scores,
                    c->count,      m->gqa->dim, m->gqa->qh,  m->gqa->kh};
    oracle_gqa(&g);
    return 1;
}

/* src/mixer.s:4-29 */
int oracle_mixer(struct mixer *m, float scale) {
    oracle_qkv(m->qkv);
    if (!oracle_mixer_attention(m, m->qkv->out, m->gqa->out, scale))
        return 0;
    oracle_matvec(m->weight, m->gqa->out, m->out, m->hidden, m->gqa->dim * m->gqa->qh);
    return 1;
}

/* src/model.s:8-40 */
void oracle_mlp(const uint16_t *gu, const uint16_t *down, const float *input, float *output,
                float *scratch, uint64_t hidden, uint64_t intermediate) {
    oracle_matvec(gu, input, scratch, 2 * intermediate, hidden);
    oracle_swiglu(scratch, scratch, intermediate);
    oracle_matvec(down, scratch, output, hidden, intermediate);
}

/* src/model.s:67-110 (CPU branch) */
void oracle_mlp_branch(const struct mlp *m) {
    oracle_rmsnorm(m->state, m->pre, m->normalized, m->hidden, 0.000001f, 1.0f);
    oracle_mlp(m->gu, m->down, m->normalized, m->branch, m->scratch, m->hidden, m->intermediate);
    oracle_rmsnorm(m->branch, m->post, m->branch, m->hidden, 0.000001f, 0.08944271909999159f);
    oracle_residual(m->state, m->branch, m->hidden);
}

/* src/layer.s:8-48 */
int oracle_layer(struct layer *l, float scale) {
    oracle_rmsnorm(l->state, l->pre, l->normalized, l->hidden, 0.000001f, 1.0f);
    l->mixer->qkv->input = l->normalized;
    l->mixer->out = l->branch;
    if (!oracle_mixer(l->mixer, scale))
        return 0;
    oracle_rmsnorm(l->branch, l->post, l->branch, l->hidden, 0.000001f, 0.2f);
    oracle_residual(l->state, l->branch, l->hidden);
    l->mlp->state = l->state;
    oracle_mlp_branch(l->mlp);
    return 1;
}

/* src/token.s:6-33: out-of-range ids leave the output untouched. */
int oracle_embedding(const uint16_t *embedding, uint64_t token, uint64_t vocab, uint64_t hidden,
                     float *out) {
    if (token >= vocab)
        return 0;
    for (uint64_t i = 0; i < hidden; ++i)
        out[i] = oracle_bf16(embedding[token * hidden + i]);
    return 1;
}

static void final_head(struct model *m) {
    oracle_rmsnorm(m->state, m->norm, m->normalized, m->hidden, 0.000001f, 1.0f);
    oracle_matvec(m->head, m->normalized, m->logits, m->vocab, m->hidden);
}

static int forward_common(struct model *m, uint64_t token, int logits) {
    if (!oracle_embedding(m->embedding, token, m->vocab, m->hidden, m->state))
        return 0;
    for (uint64_t i = 0; i < m->count; ++i) {
        m->layers[i]->state = m->state;
        if (!oracle_layer(m->layers[i], m->scales[i]))
            return 0;
    }
    if (logits)
        final_head(m);
    return 1;
}

/* src/forward.s:36-81 (CPU branch of _plamo_forward). */
int oracle_forward(struct model *m, uint64_t token) {
    return forward_common(m, token, 1);
}

/* src/forward.s:33-35: caches and state advance; normalized/logits untouched. */
int oracle_forward_hidden(struct model *m, uint64_t token) {
    return forward_common(m, token, 0);
}

static void project(const uint16_t *w, const float *x, uint64_t x_stride, float *y,
                    uint64_t y_stride, uint64_t rows, uint64_t cols, uint64_t tokens) {
    struct plamo_matmul mm = {w, x, y, rows, cols, tokens, x_stride, y_stride};
    oracle_matmul_blocked(&mm);
}

/* Workspace of one prompt: per token the normalized input, projection
 * outputs, attention output, residual branch and SwiGLU activation. */
struct prompt_rows {
    float *norm, *qkv, *attn, *branch, *gu, *act;
};

/* src/batch.s:61-223 (_plamo_layer_batch): one layer over every prompt
 * token. The projections run as token-blocked products (bit for bit one
 * matvec per token); the Q/K norm, cache append, key rotation and attention
 * run token by token in prompt order, since each token attends over the rows
 * the earlier ones appended. Per token the operations are oracle_layer's. */
static int layer_batch(struct layer *l, float scale, float *states, uint64_t n,
                       const struct prompt_rows *b) {
    struct mixer *mx = l->mixer;
    const struct qkv *q = mx->qkv;
    const struct mlp *p = l->mlp;
    const uint64_t h = l->hidden, qw = (q->qh + 2 * q->kh) * q->dim;
    const uint64_t aw = mx->gqa->qh * mx->gqa->dim, inter = p->intermediate;
    for (uint64_t t = 0; t < n; ++t)
        oracle_rmsnorm(states + t * h, l->pre, b->norm + t * h, h, 0.000001f, 1.0f);
    project(q->weight, b->norm, h, b->qkv, qw, qw, h, n);
    for (uint64_t t = 0; t < n; ++t) {
        oracle_qk_norm(b->qkv + t * qw, q->qn, q->kn, q->qh, q->kh, q->dim);
        if (!oracle_mixer_attention(mx, b->qkv + t * qw, b->attn + t * aw, scale))
            return 0;
    }
    project(mx->weight, b->attn, aw, b->branch, h, h, aw, n);
    for (uint64_t t = 0; t < n; ++t) {
        float *br = b->branch + t * h, *st = states + t * h;
        oracle_rmsnorm(br, l->post, br, h, 0.000001f, 0.2f);
        oracle_residual(st, br, h);
        oracle_rmsnorm(st, p->pre, b->norm + t * h, h, 0.000001f, 1.0f);
    }
    project(p->gu, b->norm, h, b->gu, 2 * inter, 2 * inter, h, n);
    for (uint64_t t = 0; t < n; ++t)
        oracle_swiglu(b->gu + t * 2 * inter, b->act + t * inter, inter);
    project(p->down, b->act, inter, b->branch, h, h, inter, n);
    for (uint64_t t = 0; t < n; ++t) {
        float *br = b->branch + t * h;
        oracle_rmsnorm(br, p->post, br, h, 0.000001f, 0.08944271909999159f);
        oracle_residual(states + t * h, br, h);
    }
    return 1;
}

/* tests/prefill_reference.s:7-88: embeddings first, then layer-major over all
 * tokens; the final token's state, final norm and head give the logits. The
 * per-layer state pointer is restored to model->state afterwards, as the
 * engine's request reset would (runtime/engine.c:49). */
int oracle_prefill(struct model *m, const uint32_t *ids, uint64_t n, float *states) {
    if (!n)
        return 0;
    uint64_t h = m->hidden, qw = 0, aw = 0, inter = 0;
    for (uint64_t i = 0; i < m->count; ++i) {
        const struct mixer *mx = m->layers[i]->mixer;
        uint64_t w = (mx->qkv->qh + 2 * mx->qkv->kh) * mx->qkv->dim;
        qw = w > qw ? w : qw;
        w = mx->gqa->qh * mx->gqa->dim;
        aw = w > aw ? w : aw;
        inter = m->layers[i]->mlp->intermediate > inter ? m->layers[i]->mlp->intermediate : inter;
    }
    float *owned = states ? NULL : malloc(n * h * 4);
    struct prompt_rows b = {malloc(n * h * 4), malloc(n * qw * 4), malloc(n * aw * 4),
                            malloc(n * h * 4), malloc(n * 2 * inter * 4), malloc(n * inter * 4)};
    if (!states)
        states = owned;
    int ok = states && b.norm && b.qkv && b.attn && b.branch && b.gu && b.act;
    for (uint64_t t = 0; t < n && ok; ++t)
        ok = oracle_embedding(m->embedding, ids[t], m->vocab, h, states + t * h);
    for (uint64_t i = 0; i < m->count && ok; ++i)
        ok = layer_batch(m->layers[i], m->scales[i], states, n, &b);
    for (uint64_t i = 0; i < m->count; ++i)
        m->layers[i]->state = m->state;
    if (ok) {
        memcpy(m->state, states + (n - 1) * h, h * 4);
        final_head(m);
    }
    free(b.norm);
    free(b.qkv);
    free(b.attn);
    free(b.branch);
    free(b.gu);
    free(b.act);
    free(owned);
    return ok;
}

/* src/token.s:37-63 */
uint64_t oracle_argmax(const float *x, uint64_t n) {
    if (!n || isnan(x[0]))
        return UINT64_MAX;
    uint64_t best = 0;
    float value = x[0];
    for (uint64_t i = 1; i < n; ++i) {
        if (isnan(x[i]))
            return UINT64_MAX;
        if (x[i] > value) {
            value = x[i];
            best = i;
        }
    }
    return best;
}

/* runtime/engine.c:30-38: FNV-1a 64 over raw bytes. */
uint64_t oracle_fnv1a(const void *data, uint64_t bytes, uint64_t hash) {
    const unsigned char *p = data;
    for (uint64_t i = 0; i < bytes; ++i)
        hash = (hash ^ p[i]) * UINT64_C(0x100000001b3);
    return hash;
}
