/* CPU oracle of the PLaMo-3-Translate token loop — TEST INFRASTRUCTURE ONLY.
 *
 * A scalar C restatement of the reference's FP32 CPU path, in the exact
 * operation order of its bit-exact specification (the tests/..._reference.s files) and
 * of the production assembly that is bit-identical to it (the src/ assembly). It is the
 * checker for the HIP backend and the CPU baseline of bench.py; nothing in the
 * product links or calls it. Every function names the reference file:line it
 * follows in plamo_oracle.c.
 *
 * Build: gcc -O2 -ffp-contract=off (no contraction: fused multiply-adds appear
 * only where the reference fuses, written as fmaf/fma).
 */
#ifndef PLAMO_ORACLE_H
#define PLAMO_ORACLE_H
#include "../include/plamo_model.h"
#include "../include/plamo_parallel.h"

#ifdef __cplusplus
extern "C" {
#endif

float oracle_bf16(uint16_t bits);
uint16_t oracle_to_bf16(float value);
float oracle_exp(float x);
void oracle_softmax(float *x, uint64_t n);
void oracle_swiglu(const float *gate_up, float *out, uint64_t n);
void oracle_matvec(const uint16_t *w, const float *x, float *y, uint64_t rows, uint64_t cols);
void oracle_matmul(const struct plamo_matmul *m);
void oracle_matmul_blocked(const struct plamo_matmul *m);
void oracle_set_threads(unsigned threads);
unsigned oracle_threads(void);
void oracle_rmsnorm(const float *x, const uint16_t *w, float *y, uint64_t n, float eps,
                    float offset);
void oracle_residual(float *state, const float *branch, uint64_t n);
void oracle_attention_head(const float *q, const float *k, const float *v, float *out,
                           float *scores, uint64_t n, uint64_t d, uint64_t stride);
void oracle_gqa(const struct gqa *g);
void oracle_rope_copy(const float *src, float *dst, const float *cos, const float *sin,
                      uint64_t heads, uint64_t half);
void oracle_sincos(double angle, float out[2]);
void oracle_rope_table(const float *freq, uint64_t position, uint64_t half, float *cos,
                       float *sin, float scale);
void oracle_rope_frequencies(double theta, uint64_t half, int yarn, double factor,
                             double original_max_positions, double beta_fast, double beta_slow,
                             float *out);
float oracle_rope_concentration(int yarn, double factor);
int oracle_cache_append(struct cache *c, const float *k, const float *v);
void oracle_cache_rope_cached(struct rotation *r, float scale);
void oracle_qk_norm(float *qkv, const uint16_t *qn, const uint16_t *kn, uint64_t qh, uint64_t kh,
                    uint64_t dim);
void oracle_qkv(const struct qkv *q);
int oracle_mixer_attention(struct mixer *m, float *qkv_out, float *attention_out, float scale);
int oracle_mixer(struct mixer *m, float scale);
void oracle_mlp(const uint16_t *gu, const uint16_t *down, const float *input, float *output,
                float *scratch, uint64_t hidden, uint64_t intermediate);
void oracle_mlp_branch(const struct mlp *m);
int oracle_layer(struct layer *l, float scale);
int oracle_embedding(const uint16_t *embedding, uint64_t token, uint64_t vocab, uint64_t hidden,
                     float *out);
int oracle_forward(struct model *m, uint64_t token);
int oracle_forward_hidden(struct model *m, uint64_t token);
int oracle_prefill(struct model *m, const uint32_t *ids, uint64_t n, float *states);
uint64_t oracle_argmax(const float *x, uint64_t n);
uint64_t oracle_fnv1a(const void *data, uint64_t bytes, uint64_t hash);

#ifdef __cplusplus
}
#endif
#endif
