// Launchers of the gfx950 token-loop kernels (implemented in kernels.hip).
//
// Every launcher enqueues on the given stream and returns the launch status.
// Shapes are checked by the caller (backend.cpp) before any launch: a kernel
// trusts its sizes, so a wrong size would fault instead of failing.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace plamo {

// Per-call values the kernels read from device memory, so a captured decode
// graph stays valid from one step to the next (the host rewrites this block
// before every launch).
enum { kMaxLayers = 128, kMaxVerify = 16 };
struct StepParams {
    uint32_t token;             // decode token id
    uint32_t tokens;            // prompt / candidate rows of this call
    uint32_t count[kMaxLayers]; // cache rows of each layer before this call
    uint32_t done[kMaxLayers];  // fused attention: finished KV heads (zero at launch)
    uint32_t error;             // fused attention: a wait gave up (zero at launch)
    // Bounded wait of the fused attention's O blocks: the target is the KV
    // heads plus wait_extra, polled at most wait_limit times (0: 2^22).
    // Both are zero outside tests, which raise them from the host so that a
    // wait gives up and the failure path runs with every kernel exiting.
    uint32_t wait_extra, wait_limit;
    // Nonzero tag of this decode step, new for every step of a backend: the
    // fused attention's blocks publish it in their completion flags.
    uint32_t step;
};

// Norm applied in a GEMV prologue: x = rms(src) * (bf16(w) + offset).
// With residual, the prologue first forms src' = src + rms(branch) *
// (bf16(rw) + roffset) and block 0 stores src' to state_out.
struct Prologue {
    const float *src;        // vector to normalize (or raw input when w == nullptr)
    const uint16_t *w;       // norm weights; nullptr: use src as is
    float offset;
    const float *branch;     // residual branch; nullptr: no residual
    const uint16_t *rw;
    float roffset;
    float *state_out;        // written by block 0 when branch != nullptr
    float *norm_out;         // written by block 0 when non-null (normalized x)
    // Block 0 copies *status to *status_out when non-null (the decode head
    // hands the step's error word to a pinned host word this way).
    const uint32_t *status;
    uint32_t *status_out;
};

hipError_t launch_rope_table(hipStream_t, const float *freq, float scale, uint32_t half,
                             uint64_t first_row, uint64_t rows, float *table);
// Row gather widened from BF16: token t reads ids[t], or params->token when
// ids is null. With `publish`, block 0 also copies *params (a pinned host
// block, read over the bus) to *publish for the later kernels of the step.
hipError_t launch_embed(hipStream_t, const uint16_t *embedding, const uint32_t *ids,
                        const StepParams *params, uint32_t tokens, uint32_t hidden, float *out,
                        StepParams *publish = nullptr);
// y[r] = W[r,:] . x (x from the prologue). swiglu_half > 0: rows r and
// r + swiglu_half are gate/up and y[r] = silu(gate) * up for r < swiglu_half.
hipError_t launch_gemv(hipStream_t, const uint16_t *w, uint64_t rows, uint64_t cols,
                       const Prologue &pro, float *y, uint64_t swiglu_half, int blocks_hint);
// Scratch of the split-BF16 GEMM: the three BF16 planes of X, split-K partial
// tiles and per-tile arrival counters (zero-initialized; every launch leaves
// them zero).
struct GemmWorkspace {
    float *partial;
    uint64_t partial_floats;
    uint32_t *counter_base;
    uint32_t counters;
    uint16_t *planes;
    uint64_t plane_elems;
    uint32_t cus;  // compute units (grid sizing)
};
struct GemmSplit {
    const float *x;
    uint64_t ldx;
    const uint16_t *w;
    uint32_t n, k, t, tp, splits;
    float *y;
    uint64_t ldy;
    float *partial;
    uint32_t *counters;
    uint16_t *planes;
    uint32_t xcd_group;  // nonzero: the M tiles of a weight tile share an XCD (see the kernel)
    // Nonzero (the intermediate size I): the rows are a gate/up pair [2I]
    // and each tile takes gate and up rows of the same intermediate columns;
    // the epilogue writes silu(gate) * up as the BF16 planes `act` (rows
    // padded to act_tp) instead of y.
    uint32_t swiglu;
    uint16_t *act;
    uint32_t act_tp;
};
constexpr uint64_t kGemmPartialFloats = 16ull << 20;  // 64 MiB
constexpr uint32_t kGemmCounters = 8192;
// BF16 elements of the planes a GEMM of `tokens` rows and `cols` columns needs.
uint64_t gemm_plane_elems(uint64_t tokens, uint64_t cols);
// C[t, r] = sum_k X[t, k] * W[r, k]. With a workspace, at most 5 tokens and
// K a multiple of 512: FP32 FMAs on the vector ALUs, weights streamed as in
// the decode GEMV. Otherwise, with a workspace, more than one token and K a
// multiple of 64: BF16 matrix cores on the exact three-term split of X; else
// FP32 MFMA with BF16 weights widened in LDS.
// planes_ready: the BF16 planes of X for the matrix-core path are already in
// ws->planes (written by launch_norm_rows / launch_residual_norm_rows /
// launch_swiglu_rows / launch_prompt_attention with gemm_planes_rows(tokens,
// cols, ws) rows), and x is not read; other paths read x as usual.
hipError_t launch_gemm(hipStream_t, const float *x, uint64_t x_stride, const uint16_t *w,
                       uint64_t rows, uint64_t cols, uint64_t tokens, float *y,
                       uint64_t y_stride, const GemmWorkspace *ws, bool planes_ready = false);
// The padded rows of the BF16 planes launch_gemm's matrix-core path reads for
// `tokens` rows of `cols` columns, or 0 when another path takes the call.
uint32_t gemm_planes_rows(uint64_t tokens, uint64_t cols, const GemmWorkspace *ws);
// Multi-row RMSNorm; with branch: state += rms(branch) * (bf16(w) + offset).
// With planes, the normalized rows also go into the BF16 planes of
// launch_gemm's matrix-core path, `padded` rows (gemm_planes_rows of the
// consuming projection; rows past `rows` zero), so that projection can take
// planes_ready.
hipError_t launch_norm_rows(hipStream_t, const float *x, uint64_t x_stride, const uint16_t *w,
                            float offset, float *y, uint64_t y_stride, uint64_t width,
                            uint64_t rows, uint16_t *planes = nullptr, uint32_t padded = 0);
// launch_residual_rows followed by launch_norm_rows of the updated rows into
// norm, in one launch (width <= 8192; hipErrorInvalidValue otherwise), planes
// as launch_norm_rows (16-byte-aligned rows only; hipErrorInvalidValue else).
hipError_t launch_residual_norm_rows(hipStream_t, float *state, const float *branch,
                                     const uint16_t *wr, float off_r, const uint16_t *wn,
                                     float off_n, float *norm, uint64_t norm_stride,
                                     uint64_t width, uint64_t rows, uint16_t *planes = nullptr,
                                     uint32_t padded = 0);
hipError_t launch_residual_rows(hipStream_t, float *state, const float *branch,
                                const uint16_t *w, float offset, uint64_t width, uint64_t rows);
// With planes, writes the activation as the BF16 planes of a following
// launch_gemm over `padded` rows (gemm_planes_rows of the activation) instead
// of `out`.
hipError_t launch_swiglu_rows(hipStream_t, const float *gate_up, float *out,
                              uint64_t intermediate, uint64_t rows, uint16_t *planes = nullptr,
                              uint32_t padded = 0);
// act[t, i] = silu(g) * u of the gate/up projection (rows i and
// intermediate + i of w): the token GEMV writes act directly; other shapes
// go through launch_gemm into gate_up ([tokens][2 * intermediate]) and
// launch_swiglu_rows. act_planes (gemm_planes_rows(tokens, intermediate, ws),
// nonzero) writes the activation only as BF16 planes, for a launch_gemm of
// act with planes_ready over `ws` with its planes at *act_at: when the
// workspace holds the input's planes and the activation's side by side, the
// gate/up GEMM forms them in its epilogue (*act_at past the input's);
// otherwise a separate SwiGLU launch writes them at ws->planes. Shapes
// without either route fail.
hipError_t launch_gemm_swiglu(hipStream_t, const float *x, uint64_t x_stride, const uint16_t *w,
                              uint64_t intermediate, uint64_t cols, uint64_t tokens, float *act,
                              float *gate_up, const GemmWorkspace *ws, bool planes_ready = false,
                              uint32_t act_planes = 0, uint16_t **act_at = nullptr);
// The workspace columns a launch_gemm_swiglu over `cols` input columns needs
// for its epilogue to write the activation planes (input and activation
// planes side by side).
inline uint64_t gemm_swiglu_cols(uint64_t cols, uint64_t intermediate) {
    return cols + intermediate;
}

// Q/K head RMSNorm + RoPE + cache append for `tokens` rows of one layer.
struct QkvPost {
    float *qkv;              // [tokens, (qh+2kh)*dim] projection output (read)
    float *q_out;            // [tokens, qh*dim] normalized, rotated Q
    const uint16_t *qn, *kn;
    const float *table;      // RoPE rows [position][dim]: cos | sin
    const StepParams *params;
    uint32_t layer, qh, kh, dim, tokens, capacity;
    // K/V destination rows: row t goes to dst_*[(row0 + t) * width], where
    // row0 = params->count[layer] when rows_from_count, else 0.
    float *k_raw, *v, *k_rot;
    int rows_from_count;
    int rotate_k;            // 0: leave k_rot alone (sliding overflow)
    float *stage;            // optional [3][width] copy of the last row (decode mirror)
};
hipError_t launch_qkv_post(hipStream_t, const QkvPost &);

// Decode attention for one token, fused with the decode form of QkvPost: each
// block normalizes and rotates the query heads of its KV head, the block that
// owns row `count` also normalizes/rotates the new key and appends K, V and
// rotated K (plus the mirror stage), and every block runs an online softmax
// over its share of rows [0, count]; the last block of a KV head merges the
// partials. Requires decode_attention_supported(dim, qh / kh), splits <= 8 and
// count < capacity (a full sliding window takes the general path). Up to 256
// rows run in one block per KV head; longer contexts use up to `splits` blocks.
struct DecodeAttention {
    const float *qkv;        // [(qh+2kh)*dim] projection output
    const uint16_t *qn, *kn;
    const float *freq;       // RoPE frequencies [dim / 2] of the layer's table
    float rope_scale;        // and its concentration (rope_cos_sin)
    float *k_raw, *v, *k_rot;  // cache rows [rows, kh*dim]
    uint32_t rows;           // allocated cache rows (every tile row is clamped below it)
    float *stage;            // optional [3][kh*dim] copy of the appended row
    float *host_k, *host_v, *host_rot;  // optional device views of the host cache rows
    float *out;              // [qh*dim]
    float *partial;          // scratch [kh][splits][qh/kh][dim + 2]
    uint32_t *counters;      // [kh] zero-initialized; reset by the kernel
    const StepParams *params;
    uint32_t layer, qh, kh, dim, splits;
};
hipError_t launch_decode_attention(hipStream_t, const DecodeAttention &);
bool decode_attention_supported(uint32_t dim, uint32_t group);
// Decode attention fused with the output projection y = W_o . attention
// (rows = hidden, cols = qh * dim). `done` must be zero at launch and counts
// the finished KV heads; x is the attention output (a.out).
struct AttentionO {
    DecodeAttention a;
    const uint16_t *w;
    const float *x;
    float *y;
    uint32_t rows, cols, heads;
    uint32_t *done;
    uint32_t *error;
    // Per attention block of this layer, the step tag of its last completed
    // partial (kAttentionFlags words, zero when allocated): up to
    // kDecodeShortRows allocated rows the O blocks wait on these instead of
    // `done`.
    uint32_t *flags;
};
constexpr uint32_t kAttentionFlags = 64;
hipError_t launch_attention_o(hipStream_t, const AttentionO &);
bool attention_o_supported(uint32_t dim, uint32_t group, uint64_t cols);
// Blocks per KV head that cover `rows` cache rows (DecodeAttention::splits
// must be at least this for the largest row count of the launch).
// Allocated rows up to which the decode attention uses its short-context
// blocks (32 rows each; 64 in the fused attention + O launch, whose O blocks
// merge the partials); a decode step whose rows all stay below it may cap
// the attention's view of the allocation here.
constexpr uint32_t kDecodeShortRows = 256;
uint32_t decode_attention_splits(uint64_t rows);

// General causal attention for `tokens` query rows. Key j of query t is the
// virtual row j of [cache rows 0..prefix) ++ [new rows 0..tokens). With
// window > 0 query t sees only the last `window` virtual rows ending at its
// own row and keys are rotated on the fly at their window-local position.
struct PromptAttention {
    const float *q;          // [tokens, qh*dim] rotated Q
    const float *k_cache, *v_cache;  // rotated (or raw when window) cache rows
    const float *k_new, *v_new;      // rotated (or raw when window) new rows
    const float *table;
    float *out;              // [tokens, qh*dim]
    uint32_t prefix, tokens, qh, kh, dim, window;
    // Optional scratch for key splits (prompt_attention_scratch floats): few
    // query tiles then spread their keys over several blocks and a merge.
    float *partial;
    // Optional: the output rows as launch_gemm's BF16 planes (rows padded to
    // `padded`) instead of FP32 rows in `out`, so the O projection's GEMM
    // reads them with planes_ready. Rows past `tokens` are not written (each
    // GEMM output row depends on its own input row only, and rows past the
    // token count are never stored). Only where
    // prompt_attention_writes_planes holds.
    uint16_t *planes;
    uint32_t padded;
};
hipError_t launch_prompt_attention(hipStream_t, const PromptAttention &);
bool prompt_attention_writes_planes(uint32_t dim, uint32_t qh, uint32_t kh, uint32_t window);
// Floats of split scratch launch_prompt_attention uses for this shape (0: none).
uint64_t prompt_attention_scratch(uint32_t prefix, uint32_t tokens, uint32_t qh, uint32_t kh,
                                  uint32_t dim, uint32_t window);

// Rotates cache rows [0, rows) of raw K into rotated K at their row position.
hipError_t launch_rerotate(hipStream_t, const float *k_raw, float *k_rot, const float *table,
                           uint64_t rows, uint32_t kh, uint32_t dim);
// Sliding-window commit: the final `keep` rows of [cache 0..prefix) ++
// [new 0..tokens) become cache rows 0..keep, rotated at their new positions.
hipError_t launch_window_store(hipStream_t, float *k_raw, float *v, float *k_rot,
                               const float *new_k, const float *new_v, uint64_t new_stride,
                               const float *table, float *scratch, uint64_t prefix,
                               uint64_t tokens, uint64_t keep, uint32_t kh, uint32_t dim);
// Batched row copies (one launch for every layer of a commit).
struct CopyRow {
    const float *src;
    float *dst;
    uint64_t floats;
};
hipError_t launch_copy_rows(hipStream_t, const CopyRow *table, uint32_t entries);
// p[0, words) = value (a kernel, so that it is also safe inside captured graphs).
hipError_t launch_fill(hipStream_t, uint32_t *p, uint64_t words, uint32_t value);
// Raises the dynamic LDS limit of the GEMV variants to hold `cols` floats.
hipError_t configure_gemv(uint64_t max_cols);
// First maximal index per row (strict >); any NaN gives 0xffffffff. scratch:
// argmax_scratch_bytes(rows) of device memory.
hipError_t launch_argmax_rows(hipStream_t, const float *x, uint64_t width, uint64_t rows,
                              uint32_t *out, void *scratch);
uint64_t argmax_scratch_bytes(uint64_t rows);

}  // namespace plamo
