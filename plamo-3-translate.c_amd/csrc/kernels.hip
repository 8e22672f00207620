// gfx950 kernels of the PLaMo-3-Translate token loop.
//
// Numerics follow the reference's FP32 path (tests/*_reference.s): BF16
// weights are widened by a 16-bit shift, every product and sum is FP32, the
// exponential is the reference's degree-7 polynomial, and RoPE uses separate
// multiplies and adds. This file is compiled with -ffp-contract=off, so a
// fused multiply-add appears only where written (__builtin_fmaf). Reduction
// orders are fixed (wave butterflies, then waves in index order), so results
// are run-to-run deterministic; they differ from the CPU's sequential order
// only by FP32 rounding.
#include "kernels.h"

namespace plamo {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;

__device__ __forceinline__ float bf16f(uint32_t bits) { return __uint_as_float(bits << 16); }

// tests/activation_reference.s:6-48.
// Branch-free: the polynomial runs on x clamped to [-87, 88] (identical to x
// inside that range) and the out-of-range results are selected afterwards.
__device__ __forceinline__ float plamo_exp(float x) {
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -87.0f), 88.0f);
    float n = __builtin_rintf(xc * 1.4426950408889634f);
    int i = (int)n;
    float r = __builtin_fmaf(-n, 0.6931471805599453f, xc);
    float p = __builtin_fmaf(0.0001984126984126984f, r, 0.001388888888888889f);
    p = __builtin_fmaf(p, r, 0.008333333333333333f);
    p = __builtin_fmaf(p, r, 0.041666666666666664f);
    p = __builtin_fmaf(p, r, 0.16666666666666666f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float v = p * __int_as_float((i + 127) << 23);
    v = x > 88.0f ? __builtin_inff() : v;
    return x >= -87.0f ? v : 0.0f;
}

// Cross-lane reductions on DPP (row-local moves, a few cycles each) and
// readlane, not LDS permutes. Every lane ends with the same bits: each stage
// adds a value and its partner's, and a + b == b + a.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppSwap1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppSwap2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within 16

// Sum over each 16-lane row, in every lane of the row.
__device__ __forceinline__ float row_sum16(float v) {
    v = v + dpp<kDppSwap1>(v);
    v = v + dpp<kDppSwap2>(v);
    v = v + dpp<kDppHalfMirror>(v);
    v = v + dpp<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<kDppSwap1>(v));
    v = fmaxf(v, dpp<kDppSwap2>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppMirror>(v));
    return v;
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// Combine the four rows' (row-uniform) values: (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float rows_sum(float v) {
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float rows_max(float v) {
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
                 fmaxf(lane_value(v, 32), lane_value(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) { return rows_sum(row_sum16(v)); }
// wave_sum's value in lane 63 alone, without scalar registers: after the row
// sums, row 1 adds row 0's and row 3 row 2's (row_bcast:15), then row 3 adds
// lane 31's (row_bcast:31), so lane 63 holds (r2 + r3) + (r0 + r1).
__device__ __forceinline__ float wave_total(float v) {
    v = row_sum16(v);
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    v = v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}
__device__ __forceinline__ float wave_max(float v) { return rows_max(row_max16(v)); }

// Cross-block hand-off without a device-scope fence (which writes back and
// invalidates the whole L2): partials are written through to the coherence
// point (agent-scope atomic stores), the writer waits for its stores to
// complete before it counts itself in, and the last block reads the partials
// from the coherence point (agent-scope atomic loads), past any stale L2 copy.
__device__ __forceinline__ void store_through(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_through(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Returns true in the block that completes a group of `expected` blocks
// (counter left at zero for the next launch); call from all threads.
__device__ __forceinline__ bool arrive_last(uint32_t *counter, uint32_t expected, int *flag) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t done =
            __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = done + 1 == expected;
        if (*flag) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *flag;
}

// Counts the calling block in *counter after every store of the block has
// completed; the result is not needed, so the add does not wait for its
// return. Call from all threads.
__device__ __forceinline__ void signal_done(uint32_t *counter) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        (void)__hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait until *counter reaches target, for a whole block: wave 0
// polls (one request per poll) while the other waves wait at the barrier, so
// a launch's waiting blocks keep the counter's memory channel free for the
// arrivals. Returns false when the wait gave up after `limit` polls; call
// from every thread of the block.
__device__ __forceinline__ bool block_wait(const uint32_t *counter, uint32_t target,
                                           uint32_t limit, int *flag) {
    if (threadIdx.x < 64) {
        bool ok = true;
        for (uint32_t spins = 0;
             __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target;) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= limit) {
                ok = false;
                break;
            }
        }
        if (threadIdx.x == 0) *flag = ok;
    }
    __syncthreads();
    return *flag;
}

// Bounded wait until flags[0, n) all hold `tag`, for a whole block: wave 0
// polls (one load per lane and poll) while the other waves wait at the
// barrier. Each flag has one writer, so no arrival contends for an address.
// Returns false when the wait gave up after `limit` polls; call from every
// thread of the block.
__device__ __forceinline__ bool flags_wait(const uint32_t *flags, uint32_t n, uint32_t tag,
                                           uint32_t limit, int *flag) {
    if (threadIdx.x < 64) {
        bool ok = true;
        for (uint32_t spins = 0;;) {
            bool mine = true;
            for (uint32_t b = threadIdx.x; b < n; b += 64)
                mine = mine && __hip_atomic_load(const_cast<uint32_t *>(flags + b),
                                                 __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) == tag;
            if (__builtin_amdgcn_ballot_w64(!mine) == 0) break;
            __builtin_amdgcn_s_sleep(2);
            if (++spins >= limit) {
                ok = false;
                break;
            }
        }
        if (threadIdx.x == 0) *flag = ok;
    }
    __syncthreads();
    return *flag;
}

// The device's own status for the host: block 0 of a launch that carries a
// Prologue with `status_out` copies the step's error word there (the decode
// head, a pinned host word), so a step whose bounded wait gave up is reported
// by the call instead of leaving NaN logits behind a success.
__device__ __forceinline__ void publish_status(const Prologue &pro, uint32_t bid) {
    if (bid == 0 && threadIdx.x == 0 && pro.status_out)
        *pro.status_out = __hip_atomic_load(pro.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// 1 / sqrt(mean(x^2) + 1e-6) for a 256-thread block (tests/rmsnorm_reference.s:8-21
// arithmetic per element; the sum is a fixed tree).
__device__ float block_rms_inverse(const float *x, uint32_t n, float *red) {
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
        float t = x[i] * x[i];
        s = s + t;
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float total = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    float ms = total / (float)n;
    ms = ms + 0.000001f;
    float r = __builtin_sqrtf(ms);
    return 1.0f / r;
}

// Same as block_rms_inverse when each thread already holds its partial sum.
__device__ float block_inverse_from_partial(float s, uint32_t n, float *red) {
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float total = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    float ms = total / (float)n;
    ms = ms + 0.000001f;
    float r = __builtin_sqrtf(ms);
    return 1.0f / r;
}


// ---------------------------------------------------------------- RoPE table
// src/rope_table.s:5-30 with src/trig.s:5-44, evaluated per (row, j) in FP64:
// the cosine and sine of frequency j at `position`, times `scale`. The table
// kernel and the decode attention (which rotates at the step's position
// without a table lookup) share it, so both give the same bits.
__device__ __forceinline__ void rope_cos_sin(float freq, float scale, float position, float &cs,
                                             float &sn) {
    float angle = freq * position;
    double a = (double)angle;
    const double two_pi = 6.283185307179586;
    double n = __builtin_rint(a / two_pi);
    double r = __builtin_fma(-n, two_pi, a);
    double r2 = r * r;
    double p = 2.8114572543455206e-15;
    p = __builtin_fma(p, r2, -7.647163731819816e-13);
    p = __builtin_fma(p, r2, 1.6059043836821613e-10);
    p = __builtin_fma(p, r2, -2.505210838544172e-08);
    p = __builtin_fma(p, r2, 2.7557319223985893e-06);
    p = __builtin_fma(p, r2, -0.0001984126984126984);
    p = __builtin_fma(p, r2, 0.008333333333333333);
    p = __builtin_fma(p, r2, -0.16666666666666666);
    p = __builtin_fma(p, r2, 1.0);
    float s = (float)(p * r);
    p = 4.779477332387385e-14;
    p = __builtin_fma(p, r2, -1.1470745597729725e-11);
    p = __builtin_fma(p, r2, 2.08767569878681e-09);
    p = __builtin_fma(p, r2, -2.755731922398589e-07);
    p = __builtin_fma(p, r2, 2.48015873015873e-05);
    p = __builtin_fma(p, r2, -0.001388888888888889);
    p = __builtin_fma(p, r2, 0.041666666666666664);
    p = __builtin_fma(p, r2, -0.5);
    p = __builtin_fma(p, r2, 1.0);
    float c = (float)p;
    cs = c * scale;
    sn = s * scale;
}

__global__ __launch_bounds__(kThreads) void rope_table_kernel(const float *freq, float scale,
                                                              uint32_t half, uint64_t first_row,
                                                              uint64_t rows, float *table) {
    uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= rows * half) return;
    uint64_t row = first_row + e / half;
    uint32_t j = (uint32_t)(e % half);
    float *out = table + row * 2 * half;
    rope_cos_sin(freq[j], scale, (float)row, out[j], out[half + j]);
}

hipError_t launch_rope_table(hipStream_t stream, const float *freq, float scale, uint32_t half,
                             uint64_t first_row, uint64_t rows, float *table) {
    uint64_t n = rows * half;
    if (!n) return hipSuccess;
    rope_table_kernel<<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
        freq, scale, half, first_row, rows, table);
    return hipGetLastError();
}

// ---------------------------------------------------------------- embedding
// src/token.s:6-33: row gather widened from BF16.
// A decode step's embedding also publishes the step's parameters: `publish`
// (when non-null) is the device copy every later kernel of the step reads,
// and `params` the host's pinned block, read here over the bus; block 0
// copies it whole (zeroing done counts, the error word and nothing else the
// host did not write). The step then needs no separate upload.
__global__ __launch_bounds__(kThreads) void embed_kernel(const uint16_t *embedding,
                                                         const uint32_t *ids,
                                                         const StepParams *params,
                                                         StepParams *publish,
                                                         uint32_t hidden, float *out) {
    uint32_t t = blockIdx.y;
    if (publish && blockIdx.x == 0 && t == 0) {
        const uint32_t *src = (const uint32_t *)params;
        uint32_t *dst = (uint32_t *)publish;
        for (uint32_t i = threadIdx.x; i < sizeof(StepParams) / 4; i += kThreads) dst[i] = src[i];
    }
    uint32_t id = ids ? ids[t] : params->token;
    const uint16_t *row = embedding + (uint64_t)id * hidden;
    float *o = out + (uint64_t)t * hidden;
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < hidden; i += gridDim.x * kThreads)
        o[i] = bf16f(row[i]);
}

hipError_t launch_embed(hipStream_t stream, const uint16_t *embedding, const uint32_t *ids,
                        const StepParams *params, uint32_t tokens, uint32_t hidden, float *out,
                        StepParams *publish) {
    unsigned bx = (hidden + kThreads - 1) / kThreads;
    if (bx > 16) bx = 16;
    embed_kernel<<<dim3(bx, tokens), kThreads, 0, stream>>>(embedding, ids, params, publish, hidden,
                                                            out);
    return hipGetLastError();
}

// ---------------------------------------------------------------- GEMV
// Decode projections. The prologue normalizes the input vector into LDS
// (every block computes the same bits); then each wave streams pairs of BF16
// rows with 16-byte non-temporal loads, FMA-accumulates against the LDS copy,
// and butterfly-reduces. With SWIGLU the pair is (gate row r, up row r+half)
// and the output is silu(gate) * up (tests/activation_reference.s:99-126).
// Loads one batch of a wave's stream: 4 chunks (of 8 BF16 each) per lane from
// chunk c of the row pair.
template <bool SWIGLU>
__device__ __forceinline__ void gemv_load(const uint16_t *w, uint64_t rows, uint64_t cols,
                                          uint64_t half, uint64_t pairs, uint64_t pair,
                                          uint64_t c, u32x4 (&qa)[4], u32x4 (&qb)[4]) {
    const uint64_t chunks = cols / 8;
    const uint64_t ra = SWIGLU ? pair : 2 * pair;
    const uint64_t rb0 = SWIGLU ? pair + half : 2 * pair + 1;
    const uint64_t rb = rb0 < rows ? rb0 : ra;
    const u32x4 *va = (const u32x4 *)(w + ra * cols), *vb = (const u32x4 *)(w + rb * cols);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (c + 64 * j < chunks) {
            qa[j] = __builtin_nontemporal_load(va + c + 64 * j);
            qb[j] = __builtin_nontemporal_load(vb + c + 64 * j);
        }
}

__device__ __forceinline__ void gemv_accumulate(const float *xs, uint64_t chunks, uint64_t c,
                                                const u32x4 (&qa)[4], const u32x4 (&qb)[4],
                                                float &acc_a, float &acc_b) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (c + 64 * j < chunks) {
            const f32x4 *xp = (const f32x4 *)(xs + (c + 64 * j) * 8);
            f32x4 x0 = xp[0], x1 = xp[1];
            float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            uint32_t ua[4] = {qa[j].x, qa[j].y, qa[j].z, qa[j].w};
            uint32_t ub[4] = {qb[j].x, qb[j].y, qb[j].z, qb[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc_a = __builtin_fmaf(bf16f(ua[e] & 0xffffu), xv[2 * e], acc_a);
                acc_a = __builtin_fmaf(__uint_as_float(ua[e] & 0xffff0000u), xv[2 * e + 1], acc_a);
                acc_b = __builtin_fmaf(bf16f(ub[e] & 0xffffu), xv[2 * e], acc_b);
                acc_b = __builtin_fmaf(__uint_as_float(ub[e] & 0xffff0000u), xv[2 * e + 1], acc_b);
            }
        }
    }
}

template <bool SWIGLU>
__device__ __forceinline__ void gemv_store(float *y, uint64_t rows, uint64_t pair, float acc_a,
                                           float acc_b, uint32_t lane) {
    acc_a = wave_sum(acc_a);
    acc_b = wave_sum(acc_b);
    if (lane == 0) {
        if (SWIGLU) {
            float d = plamo_exp(-acc_a) + 1.0f;
            y[pair] = (acc_a / d) * acc_b;
        } else {
            y[2 * pair] = acc_a;
            if (2 * pair + 1 < rows) y[2 * pair + 1] = acc_b;
        }
    }
}

// Norm prologue (src/forward.s layer entry: offset-1 RMSNorm, with the
// previous branch's residual folded in). The one-round-trip form gives each
// thread a contiguous slice of E elements (16 up to 4096 columns, 24 for
// 6144): its loads go out in one batch, then two block reductions.
// prologue_load issues the loads, prologue_finish writes the normalized vector
// to LDS (and block 0 the optional state/norm copies).
template <int E>
struct ProloguePart {
    float sv[E], bv[E], wv[E], rv[E];
    uint32_t i0;
    bool fast, mine;
};
template <int E>
__device__ __forceinline__ void prologue_begin(const Prologue &pro, uint32_t n,
                                               ProloguePart<E> &pp) {
    pp.fast = pro.w && n % E == 0 && n <= E * kThreads &&
              !(((uintptr_t)pro.src | (uintptr_t)pro.w |
                 (pro.branch ? ((uintptr_t)pro.branch | (uintptr_t)pro.rw) : 0)) & 15);
    pp.i0 = threadIdx.x * E;
    pp.mine = pp.fast && pp.i0 < n;
}
template <int E>
__device__ __forceinline__ void prologue_load(const Prologue &pro, ProloguePart<E> &pp) {
    static_assert(E % 8 == 0, "whole 16-byte loads");
    if (pp.mine) {
#pragma unroll
        for (int q = 0; q < E / 4; ++q) {
            f32x4 a = *(const f32x4 *)(pro.src + pp.i0 + 4 * q);
            pp.sv[4 * q] = a.x; pp.sv[4 * q + 1] = a.y; pp.sv[4 * q + 2] = a.z; pp.sv[4 * q + 3] = a.w;
        }
#pragma unroll
        for (int q = 0; q < E / 8; ++q) {
            u32x4 u = *(const u32x4 *)(pro.w + pp.i0 + 8 * q);
            uint32_t uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                pp.wv[8 * q + 2 * e] = bf16f(uu[e] & 0xffffu);
                pp.wv[8 * q + 2 * e + 1] = __uint_as_float(uu[e] & 0xffff0000u);
            }
        }
        if (pro.branch) {
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
                f32x4 a = *(const f32x4 *)(pro.branch + pp.i0 + 4 * q);
                pp.bv[4 * q] = a.x; pp.bv[4 * q + 1] = a.y; pp.bv[4 * q + 2] = a.z; pp.bv[4 * q + 3] = a.w;
            }
#pragma unroll
            for (int q = 0; q < E / 8; ++q) {
                u32x4 u = *(const u32x4 *)(pro.rw + pp.i0 + 8 * q);
                uint32_t uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pp.rv[8 * q + 2 * e] = bf16f(uu[e] & 0xffffu);
                    pp.rv[8 * q + 2 * e + 1] = __uint_as_float(uu[e] & 0xffff0000u);
                }
            }
        }
    }
}
template <int E>
__device__ __forceinline__ void prologue_finish(const Prologue &pro, uint32_t n,
                                                ProloguePart<E> &pp, float *xs, float *red,
                                                uint32_t bid) {
    if (pp.fast) {
        float ss = 0.0f;
        if (pro.branch) {
            if (pp.mine)
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    float t = pp.bv[k] * pp.bv[k];
                    ss = ss + t;
                }
            const float ib = block_inverse_from_partial(ss, n, red);
            if (pp.mine)
#pragma unroll
                for (int k = 0; k < E; ++k) {
                    float b = pp.bv[k] * ib;
                    float scale = pp.rv[k] + pro.roffset;
                    pp.sv[k] = pp.sv[k] + b * scale;
                }
            if (bid == 0 && pro.state_out && pp.mine)
#pragma unroll
                for (int q = 0; q < E / 4; ++q)
                    *(f32x4 *)(pro.state_out + pp.i0 + 4 * q) =
                        f32x4{pp.sv[4 * q], pp.sv[4 * q + 1], pp.sv[4 * q + 2], pp.sv[4 * q + 3]};
            ss = 0.0f;
        }
        if (pp.mine)
#pragma unroll
            for (int k = 0; k < E; ++k) {
                float t = pp.sv[k] * pp.sv[k];
                ss = ss + t;
            }
        const float is = block_inverse_from_partial(ss, n, red);
        if (pp.mine)
#pragma unroll
            for (int q = 0; q < E / 4; ++q) {
                f32x4 x;
                x.x = (pp.sv[4 * q] * is) * (pp.wv[4 * q] + pro.offset);
                x.y = (pp.sv[4 * q + 1] * is) * (pp.wv[4 * q + 1] + pro.offset);
                x.z = (pp.sv[4 * q + 2] * is) * (pp.wv[4 * q + 2] + pro.offset);
                x.w = (pp.sv[4 * q + 3] * is) * (pp.wv[4 * q + 3] + pro.offset);
                *(f32x4 *)(xs + pp.i0 + 4 * q) = x;
                if (bid == 0 && pro.norm_out) *(f32x4 *)(pro.norm_out + pp.i0 + 4 * q) = x;
            }
        __syncthreads();
    } else if (!pro.w) {
        for (uint32_t i = threadIdx.x; i < n; i += kThreads) xs[i] = pro.src[i];
        __syncthreads();
    } else {
        float ib = 1.0f;
        if (pro.branch) ib = block_rms_inverse(pro.branch, n, red);
        for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
            float v = pro.src[i];
            if (pro.branch) {
                float b = pro.branch[i] * ib;
                float scale = bf16f(pro.rw[i]) + pro.roffset;
                v = v + b * scale;
            }
            xs[i] = v;
        }
        __syncthreads();
        if (pro.branch && bid == 0 && pro.state_out)
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) pro.state_out[i] = xs[i];
        float is = block_rms_inverse(xs, n, red);
        for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
            float scale = bf16f(pro.w[i]) + pro.offset;
            xs[i] = (xs[i] * is) * scale;
        }
        __syncthreads();
        if (bid == 0 && pro.norm_out)
            for (uint32_t i = threadIdx.x; i < n; i += kThreads) pro.norm_out[i] = xs[i];
    }
}

// Decode projections with a norm prologue (or a raw input the register GEMV
// does not cover). Vector-memory loads complete in order on CDNA, so the
// prologue's own loads are issued first, then the first three weight batches,
// so the norm's reductions overlap the weights in flight. The weight stream
// keeps three batches in flight: batch i+3 is requested as batch i is consumed.
// With SWIGLU the pair is (gate row r, up row r+half) and the output is
// silu(gate) * up (tests/activation_reference.s:99-126).
template <bool VEC, bool SWIGLU>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const uint16_t *__restrict__ w,
                                                        uint64_t rows, uint64_t cols,
                                                        Prologue pro, float *__restrict__ y,
                                                        uint64_t half) {
    extern __shared__ __attribute__((aligned(16))) float xs[];
    __shared__ float red[4];
    const uint32_t bid = blockIdx.x, nblocks = gridDim.x;
    const uint32_t n = (uint32_t)cols;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t pairs = SWIGLU ? half : (rows + 1) / 2;
    const uint64_t chunks = cols / 8, nb = (chunks + 255) / 256;
    const uint64_t step = (uint64_t)nblocks * 4;
    const uint64_t p0 = (uint64_t)bid * 4 + wave;
    // Batches of this wave: nb per row pair, pairs p0, p0 + step, ...
    const uint64_t total = p0 < pairs ? ((pairs - 1 - p0) / step + 1) * nb : 0;
    ProloguePart<16> pp;
    prologue_begin(pro, n, pp);
    prologue_load(pro, pp);
    __builtin_amdgcn_sched_barrier(0);
    // Three batches in flight: the first three go out before the prologue.
    u32x4 qa0[4], qb0[4], qa1[4], qb1[4], qa2[4], qb2[4];
    auto issue = [&](uint64_t it, u32x4(&qa)[4], u32x4(&qb)[4]) {
        gemv_load<SWIGLU>(w, rows, cols, half, pairs, p0 + (it / nb) * step,
                          lane + (it % nb) * 256, qa, qb);
    };
    if (VEC) {
        if (total > 0) issue(0, qa0, qb0);
        if (total > 1) issue(1, qa1, qb1);
        if (total > 2) issue(2, qa2, qb2);
    }
    __builtin_amdgcn_sched_barrier(0);
    prologue_finish(pro, n, pp, xs, red, bid);
    publish_status(pro, bid);

    if (VEC) {
        float acc_a = 0.0f, acc_b = 0.0f;
        auto consume = [&](uint64_t it, const u32x4(&qa)[4], const u32x4(&qb)[4]) {
            gemv_accumulate(xs, chunks, lane + (it % nb) * 256, qa, qb, acc_a, acc_b);
            if (it % nb == nb - 1) {
                gemv_store<SWIGLU>(y, rows, p0 + (it / nb) * step, acc_a, acc_b, lane);
                acc_a = acc_b = 0.0f;
            }
        };
        // Steady state: every refill is a real batch, issued unconditionally
        // (so the compiler keeps exact wait counts); the tail has no refills
        // past the stream.
        uint64_t it = 0;
        for (; it + 5 < total; it += 3) {
            consume(it, qa0, qb0);
            issue(it + 3, qa0, qb0);
            consume(it + 1, qa1, qb1);
            issue(it + 4, qa1, qb1);
            consume(it + 2, qa2, qb2);
            issue(it + 5, qa2, qb2);
        }
        if (it < total) {
            consume(it, qa0, qb0);
            if (it + 3 < total) issue(it + 3, qa0, qb0);
        }
        if (it + 1 < total) {
            consume(it + 1, qa1, qb1);
            if (it + 4 < total) issue(it + 4, qa1, qb1);
        }
        if (it + 2 < total) consume(it + 2, qa2, qb2);
        if (it + 3 < total) consume(it + 3, qa0, qb0);
        if (it + 4 < total) consume(it + 4, qa1, qb1);
    } else {
        for (uint64_t p = p0; p < pairs; p += step) {
            const uint64_t ra = SWIGLU ? p : 2 * p;
            const uint64_t rb = SWIGLU ? p + half : 2 * p + 1;
            const uint16_t *wa = w + ra * cols;
            const uint16_t *wb = w + (rb < rows ? rb : ra) * cols;
            float acc_a = 0.0f, acc_b = 0.0f;
            for (uint64_t k = lane; k < cols; k += 64) {
                acc_a = __builtin_fmaf(bf16f(wa[k]), xs[k], acc_a);
                acc_b = __builtin_fmaf(bf16f(wb[k]), xs[k], acc_b);
            }
            gemv_store<SWIGLU>(y, rows, p, acc_a, acc_b, lane);
        }
    }
}

// Raw-input projections (attention output, MLP down): each lane keeps its
// slice of x in registers (KC chunks of 8 columns), WPR waves split a row's
// columns, and a wave streams U rows at a time. No LDS staging of x, so the
// 16K-column down projection is not occupancy-limited by LDS.
template <int KC, int WPR, int U>
__global__ __launch_bounds__(kThreads) void gemv_reg_kernel(const uint16_t *__restrict__ w,
                                                            uint64_t rows, uint64_t cols,
                                                            const float *__restrict__ src,
                                                            float *__restrict__ y) {
    constexpr int GROUPS = 4 / WPR;
    __shared__ float part[4][U];
    const uint32_t bid = blockIdx.x, nblocks = gridDim.x;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t pidx = wave % WPR, grp = wave / WPR;
    const uint64_t col0 = (uint64_t)pidx * KC * 512 + lane * 8;
    const uint64_t units = (rows + U - 1) / U;
    const uint64_t step = (uint64_t)nblocks * GROUPS;
    u32x4 wv[U][KC];
    auto load = [&](uint64_t unit) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint64_t r = unit * U + u;
            if (r >= rows) r = rows - 1;
            const u32x4 *p = (const u32x4 *)(w + r * cols + col0);
#pragma unroll
            for (int c = 0; c < KC; ++c) wv[u][c] = __builtin_nontemporal_load(p + c * 64);
        }
    };
    const uint64_t ubase = (uint64_t)bid * GROUPS;
    if (ubase + grp < units) load(ubase + grp);
    float x[KC][8];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const f32x4 *xp = (const f32x4 *)(src + col0 + c * 512);
        f32x4 a = xp[0], b = xp[1];
        x[c][0] = a.x; x[c][1] = a.y; x[c][2] = a.z; x[c][3] = a.w;
        x[c][4] = b.x; x[c][5] = b.y; x[c][6] = b.z; x[c][7] = b.w;
    }
    for (uint64_t ub = ubase; ub < units; ub += step) {
        const uint64_t unit = ub + grp;
        const bool valid = unit < units;
        if (ub != ubase && valid) load(unit);
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const uint32_t q[4] = {wv[u][c].x, wv[u][c].y, wv[u][c].z, wv[u][c].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a = __builtin_fmaf(bf16f(q[e] & 0xffffu), x[c][2 * e], a);
                    a = __builtin_fmaf(__uint_as_float(q[e] & 0xffff0000u), x[c][2 * e + 1], a);
                }
            }
            acc[u] = wave_sum(a);
        }
        if (WPR == 1) {
            if (lane == 0 && valid)
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (unit * U + u < rows) y[unit * U + u] = acc[u];
        } else {
            if (lane == 0)
#pragma unroll
                for (int u = 0; u < U; ++u) part[wave][u] = acc[u];
            __syncthreads();
            if (pidx == 0 && lane == 0 && valid)
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    float t = part[wave][u];
#pragma unroll
                    for (int q = 1; q < WPR; ++q) t += part[wave + q][u];
                    if (unit * U + u < rows) y[unit * U + u] = t;
                }
            __syncthreads();
        }
    }
}

// Decode projections with a norm prologue, x held in registers: the block
// normalizes x into LDS, then every wave copies the whole vector into its
// registers (lane l holds columns 512c + 8l .. 512c + 8l + 7) and streams U
// rows per step; with SWIGLU the step is the pair (gate row p, up row
// p + half) and the output silu(gate) * up (tests/activation_reference.s:99-126).
// The first rows' weights are requested before the prologue's reductions.
// With PF each wave requests its next step's weights before computing the
// current one (two register sets), so a wave never waits on a load it could
// have issued a step earlier; it pays where the second set does not lower
// the waves a SIMD holds.
template <int KC, int U, bool SWIGLU, int WPR = 1, bool PF = false>
__global__ __launch_bounds__(kThreads) void gemv_regp_kernel(const uint16_t *__restrict__ w,
                                                             uint64_t rows, uint64_t cols,
                                                             Prologue pro, float *__restrict__ y,
                                                             uint64_t half) {
    static_assert(!SWIGLU || U == 2, "a SwiGLU step is one gate/up row pair");
    // WPR waves share a step, each holding KC of the row's KC * WPR chunks;
    // their sums meet in LDS.
    constexpr int GROUPS = 4 / WPR;
    extern __shared__ __attribute__((aligned(16))) float xs[];
    __shared__ float red[4];
    __shared__ float part[4][U];
    const uint32_t bid = blockIdx.x, nblocks = gridDim.x;
    const uint32_t n = (uint32_t)cols;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t pidx = wave % WPR, grp = wave / WPR;
    // Unit (row or row pair) indices fit 32 bits (the launcher checks rows);
    // 64-bit arithmetic only forms addresses.
    const uint32_t col0 = pidx * KC * 512 + lane * 8;
    const uint32_t units = (uint32_t)(SWIGLU ? half : (rows + U - 1) / U);
    const uint32_t step = nblocks * GROUPS;
    const uint32_t ubase = bid * GROUPS;
    const uint32_t u0 = ubase + grp;
    // cols = 512 * KC * WPR: 16 elements per thread up to 4096, 24 for 6144.
    ProloguePart<(KC * WPR * 512 > 16 * kThreads ? 24 : 16)> pp;
    prologue_begin(pro, n, pp);
    prologue_load(pro, pp);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 wa[U][KC], wb[PF ? U : 1][PF ? KC : 1];
    const uint32_t last = (uint32_t)rows - 1, uhalf = (uint32_t)half;
    auto load = [&](uint32_t unit, auto &wv) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t r = SWIGLU ? unit + u * uhalf : unit * U + u;
            if (r > last) r = last;
            const u32x4 *p = (const u32x4 *)(w + (uint64_t)r * cols + col0);
#pragma unroll
            for (int c = 0; c < KC; ++c) wv[u][c] = __builtin_nontemporal_load(p + c * 64);
        }
    };
    if (u0 < units) load(u0, wa);
    __builtin_amdgcn_sched_barrier(0);
    prologue_finish(pro, n, pp, xs, red, bid);
    publish_status(pro, bid);
    float x[KC][8];
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const f32x4 a = *(const f32x4 *)(xs + col0 + c * 512);
        const f32x4 b = *(const f32x4 *)(xs + col0 + c * 512 + 4);
        x[c][0] = a.x; x[c][1] = a.y; x[c][2] = a.z; x[c][3] = a.w;
        x[c][4] = b.x; x[c][5] = b.y; x[c][6] = b.z; x[c][7] = b.w;
    }
    auto compute = [&](const auto &wv, uint32_t unit) {
        const bool valid = unit < units;
        float acc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                const uint32_t q[4] = {wv[u][c].x, wv[u][c].y, wv[u][c].z, wv[u][c].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    a = __builtin_fmaf(bf16f(q[e] & 0xffffu), x[c][2 * e], a);
                    a = __builtin_fmaf(__uint_as_float(q[e] & 0xffff0000u), x[c][2 * e + 1], a);
                }
            }
            acc[u] = wave_sum(a);
        }
        if (WPR > 1) {
            if (lane == 0)
#pragma unroll
                for (int u = 0; u < U; ++u) part[wave][u] = acc[u];
            __syncthreads();
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float t = part[grp * WPR][u];
#pragma unroll
                for (int q = 1; q < WPR; ++q) t += part[grp * WPR + q][u];
                acc[u] = t;
            }
            __syncthreads();
        }
        if (lane == 0 && pidx == 0 && valid) {
            if (SWIGLU) {
                const float d = plamo_exp(-acc[0]) + 1.0f;
                y[unit] = (acc[0] / d) * acc[1];
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (unit * U + u < rows) y[unit * U + u] = acc[u];
            }
        }
    };
    // With WPR > 1 every wave of the block runs every trip (barriers inside),
    // so the trip condition depends on the block only.
    auto more = [&](uint32_t ub) { return WPR == 1 ? ub + grp < units : ub < units; };
    if constexpr (!PF) {
        for (uint32_t ub = ubase; more(ub); ub += step) {
            const uint32_t unit = ub + grp;
            if (ub != ubase && unit < units) load(unit, wa);
            compute(wa, unit);
        }
    } else {
        // Two trips per iteration, the register sets alternating.
        for (uint32_t ub = ubase; more(ub); ub += 2 * step) {
            const uint32_t ua = ub + grp, ubn = ua + step;
            if (ubn < units) load(ubn, wb);
            compute(wa, ua);
            if (!more(ub + step)) break;
            if (ubn + step < units) load(ubn + step, wa);
            compute(wb, ubn);
        }
    }
}

// Column counts the register GEMV covers: cols = 512 * KC * WPR.
template <int KC, int WPR, int U>
static hipError_t gemv_reg_variant(hipStream_t stream, const uint16_t *w, uint64_t rows,
                                   uint64_t cols, const float *src, float *y, int blocks_hint) {
    constexpr int GROUPS = 4 / WPR;
    uint64_t units = (rows + U - 1) / U;
    uint64_t blocks = (units + GROUPS - 1) / GROUPS;
    if (blocks_hint > 0 && blocks > (uint64_t)blocks_hint) blocks = blocks_hint;
    gemv_reg_kernel<KC, WPR, U><<<(unsigned)blocks, kThreads, 0, stream>>>(w, rows, cols, src, y);
    return hipGetLastError();
}

static bool gemv_reg_launch(hipStream_t stream, const uint16_t *w, uint64_t rows, uint64_t cols,
                            const float *src, float *y, int blocks_hint, hipError_t *status) {
    if (((uintptr_t)w & 15) || ((uintptr_t)src & 15) || cols % 512) return false;
    switch (cols / 512) {
    case 1: *status = gemv_reg_variant<1, 1, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 2: *status = gemv_reg_variant<2, 1, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 4: *status = gemv_reg_variant<4, 1, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 5: *status = gemv_reg_variant<5, 1, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 8: *status = gemv_reg_variant<8, 1, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 12: *status = gemv_reg_variant<6, 2, 2>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 16: *status = gemv_reg_variant<8, 2, 1>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 20: *status = gemv_reg_variant<5, 4, 1>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 32: *status = gemv_reg_variant<8, 4, 1>(stream, w, rows, cols, src, y, blocks_hint); return true;
    case 48: *status = gemv_reg_variant<12, 4, 1>(stream, w, rows, cols, src, y, blocks_hint); return true;
    default: return false;
    }
}

static hipError_t configure_token_gemv();

hipError_t configure_gemv(uint64_t max_cols) {
    hipError_t e = configure_token_gemv();
    if (e != hipSuccess) return e;
    int lds = (int)(max_cols * sizeof(float));
    if (lds <= 65536) return hipSuccess;
    const void *kernels[] = {(const void *)gemv_kernel<true, true>, (const void *)gemv_kernel<true, false>,
                             (const void *)gemv_kernel<false, true>, (const void *)gemv_kernel<false, false>};
    for (const void *k : kernels) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <bool VEC, bool SWIGLU>
static hipError_t gemv_variant(hipStream_t stream, const uint16_t *w, uint64_t rows,
                               uint64_t cols, const Prologue &pro, float *y, uint64_t half,
                               int blocks_hint) {
    size_t lds = cols * sizeof(float);
    uint64_t pairs = SWIGLU ? half : (rows + 1) / 2;
    uint64_t blocks = (pairs + 3) / 4;
    if (blocks_hint > 0 && blocks > (uint64_t)blocks_hint) blocks = blocks_hint;
    if (!blocks) blocks = 1;
    gemv_kernel<VEC, SWIGLU><<<(unsigned)blocks, kThreads, lds, stream>>>(w, rows, cols, pro, y,
                                                                          half);
    return hipGetLastError();
}

// Register-x prologue GEMV for widths of whole 512-column chunks (KC chunks
// per wave, WPR waves per step). Grid: one step (U rows or a gate/up pair) per
// wave group at most, capped at the blocks the GPU holds at once.
template <int KC, int WPR = 1, bool PF = false>
static hipError_t regp_variant(hipStream_t stream, const uint16_t *w, uint64_t rows,
                               uint64_t cols, const Prologue &pro, float *y, uint64_t half,
                               int blocks_hint) {
    constexpr int GROUPS = 4 / WPR;
    const uint64_t units = half ? half : (rows + 1) / 2;
    uint64_t blocks = (units + GROUPS - 1) / GROUPS;
    // blocks_hint is two blocks per CU. SwiGLU grids take more: the split-row
    // variant exactly the three per CU it holds at once (a second, partial
    // generation would add a tail), the others four (measured best).
    const uint64_t cap = blocks_hint > 0
                             ? (uint64_t)blocks_hint * (half ? (WPR > 1 ? 3 : 4) : 2) / 2
                             : blocks;
    if (blocks > cap) blocks = cap;
    const size_t lds = cols * sizeof(float);
    if (half)
        gemv_regp_kernel<KC, 2, true, WPR, PF><<<(unsigned)blocks, kThreads, lds, stream>>>(w, rows, cols, pro, y, half);
    else
        gemv_regp_kernel<KC, 2, false, WPR, PF><<<(unsigned)blocks, kThreads, lds, stream>>>(w, rows, cols, pro, y, 0);
    return hipGetLastError();
}

static bool regp_launch(hipStream_t stream, const uint16_t *w, uint64_t rows, uint64_t cols,
                        const Prologue &pro, float *y, uint64_t half, int blocks_hint,
                        hipError_t *status) {
    if (!pro.w || cols % 512 || ((uintptr_t)w & 15) || rows >= (1ull << 31)) return false;
    switch (cols / 512) {
    case 4: *status = regp_variant<4>(stream, w, rows, cols, pro, y, half, blocks_hint); return true;
    case 5: *status = regp_variant<5>(stream, w, rows, cols, pro, y, half, blocks_hint); return true;
    case 8: *status = regp_variant<8>(stream, w, rows, cols, pro, y, half, blocks_hint); return true;
    case 12: *status = regp_variant<6, 2, true>(stream, w, rows, cols, pro, y, half, blocks_hint); return true;
    default: return false;
    }
}

hipError_t launch_gemv(hipStream_t stream, const uint16_t *w, uint64_t rows, uint64_t cols,
                       const Prologue &pro, float *y, uint64_t swiglu_half, int blocks_hint) {
    hipError_t status;
    if (!pro.w && !swiglu_half && gemv_reg_launch(stream, w, rows, cols, pro.src, y, blocks_hint, &status))
        return status;
    if (regp_launch(stream, w, rows, cols, pro, y, swiglu_half, blocks_hint, &status)) return status;
    bool vec = cols % 8 == 0 && ((uintptr_t)w & 15) == 0;
    if (swiglu_half)
        return vec ? gemv_variant<true, true>(stream, w, rows, cols, pro, y, swiglu_half, blocks_hint)
                   : gemv_variant<false, true>(stream, w, rows, cols, pro, y, swiglu_half, blocks_hint);
    return vec ? gemv_variant<true, false>(stream, w, rows, cols, pro, y, 0, blocks_hint)
               : gemv_variant<false, false>(stream, w, rows, cols, pro, y, 0, blocks_hint);
}

// ---------------------------------------------------------------- GEMM
// Prompt / candidate projections on FP32 MFMA (v_mfma_f32_16x16x4_f32).
// Block tile BM tokens x BN weight rows, K step 32; the BF16 weight panel is
// widened to FP32 while it is staged into LDS. Operand layout of the 16x16x4
// instruction: lane l supplies A[l%16][l/16] and B[l/16][l%16] and receives
// D[4*(l/16)+v][l%16], v = 0..3.
constexpr int kBK = 32;
template <int BM, int BN, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_kernel(const float *__restrict__ x,
                                                        uint64_t x_stride,
                                                        const uint16_t *__restrict__ w,
                                                        uint64_t rows, uint64_t cols,
                                                        uint64_t tokens, float *__restrict__ y,
                                                        uint64_t y_stride) {
    constexpr int WM = BM >= 32 ? 2 : 1;  // waves along tokens
    constexpr int WN = 4 / WM;            // waves along rows
    constexpr int MT = BM / (16 * WM);
    constexpr int NT = BN / (16 * WN);
    __shared__ float as[BM][kBK + 1];
    __shared__ float bs[BN][kBK + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const uint64_t m0 = (uint64_t)blockIdx.y * BM, n0 = (uint64_t)blockIdx.x * BN;
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint64_t k0 = 0; k0 < cols; k0 += kBK) {
        const bool full_k = k0 + kBK <= cols;
        for (int i = threadIdx.x; i < BM * (kBK / 4); i += kThreads) {
            int r = i / (kBK / 4), c = (i % (kBK / 4)) * 4;
            uint64_t t = m0 + r, k = k0 + c;
            float v0 = 0, v1 = 0, v2 = 0, v3 = 0;
            if (t < tokens) {
                const float *src = x + t * x_stride + k;
                if (VEC && full_k) {
                    f32x4 v = *(const f32x4 *)src;
                    v0 = v.x; v1 = v.y; v2 = v.z; v3 = v.w;
                } else {
                    if (k < cols) v0 = src[0];
                    if (k + 1 < cols) v1 = src[1];
                    if (k + 2 < cols) v2 = src[2];
                    if (k + 3 < cols) v3 = src[3];
                }
            }
            as[r][c] = v0; as[r][c + 1] = v1; as[r][c + 2] = v2; as[r][c + 3] = v3;
        }
        for (int i = threadIdx.x; i < BN * (kBK / 8); i += kThreads) {
            int r = i / (kBK / 8), c = (i % (kBK / 8)) * 8;
            uint64_t row = n0 + r, k = k0 + c;
            float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (row < rows) {
                const uint16_t *src = w + row * cols + k;
                if (VEC && full_k) {
                    u32x4 q = __builtin_nontemporal_load((const u32x4 *)src);
                    uint32_t u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[2 * e] = bf16f(u[e] & 0xffffu);
                        v[2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (k + e < cols) v[e] = bf16f(src[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) bs[r][c + e] = v[e];
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 4) {
            float a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; ++i) a[i] = as[wm * (BM / WM) + i * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int j = 0; j < NT; ++j) b[j] = bs[wn * (BN / WN) + j * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            uint64_t col = n0 + wn * (BN / WN) + j * 16 + (lane & 15);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                uint64_t t = m0 + wm * (BM / WM) + i * 16 + 4 * (lane >> 4) + v;
                if (t < tokens && col < rows) y[t * y_stride + col] = acc[i][j][v];
            }
        }
}

template <int BM, int BN>
static hipError_t gemm_variant(hipStream_t stream, const float *x, uint64_t x_stride,
                               const uint16_t *w, uint64_t rows, uint64_t cols, uint64_t tokens,
                               float *y, uint64_t y_stride) {
    dim3 grid((unsigned)((rows + BN - 1) / BN), (unsigned)((tokens + BM - 1) / BM));
    bool vec = cols % 8 == 0 && x_stride % 4 == 0 && ((uintptr_t)w & 15) == 0 &&
               ((uintptr_t)x & 15) == 0;
    if (vec)
        gemm_kernel<BM, BN, true><<<grid, kThreads, 0, stream>>>(x, x_stride, w, rows, cols,
                                                                 tokens, y, y_stride);
    else
        gemm_kernel<BM, BN, false><<<grid, kThreads, 0, stream>>>(x, x_stride, w, rows, cols,
                                                                  tokens, y, y_stride);
    return hipGetLastError();
}

// ---------------------------------------------------------------- split-BF16 MFMA GEMM
// C[t, r] = sum_k X[t, k] * W[r, k] with FP32 X and BF16 W on the BF16 matrix
// cores, exactly: each FP32 x is split into three BF16 terms
// x = hi + mid + lo (hi = x truncated to 8 significant bits, mid = the next 8
// of the remainder, lo = the rest, which has at most 8 significant bits), so
// the split loses nothing, every product W * term is exact in FP32, and the
// three products accumulate in FP32 (v_mfma_f32_32x32x16_bf16). Weights are
// used as stored, with no widening.
//
// split_planes_kernel writes the three terms as BF16 planes once per GEMM,
// stage-major: [K / 32][3][Tp][32] (Tp = T rounded up to the block's row tile,
// padding rows zero), so one stage of a row tile is contiguous.
// The GEMM block is 4 waves as 2 x 2, each wave WM x WN tiles of 32 x 32, so
// a block covers BM = 64 WM token rows by BN = 64 WN weight rows; K advances
// 32 per stage through three LDS buffers (two blocks per CU for WN = 2), with
// PD stages in flight in registers. Each block starts its K loop at its
// own stage (rotating): weight rows are a multiple of 4 KB apart, so blocks in
// lockstep would all read one memory channel. LDS rows are 64 bytes with their four
// 16-byte granules XOR-swizzled by row, which keeps the fragment reads and the
// staging writes free of bank conflicts. Grid: (N tiles, M tiles, K splits);
// with several K splits each block writes its partial tile and the last block
// of a tile sums the partials in split order (deterministic).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kSplitBK = 32;  // K per stage: four 16-byte granules of BF16 per row
constexpr uint32_t kSplitBM = 64;  // tokens per block of every routed tiling (two waves of 32)

__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
    return (b & 0xffff0000u) | (a >> 16);
}
// Physical granule of logical granule q in LDS row r.
__device__ __forceinline__ uint32_t swizzle(uint32_t r, uint32_t q) {
    return q ^ ((r ^ (r >> 2)) & 3);
}
// Columns c .. c + 3 of row `row` into the BF16 planes of launch_gemm's
// matrix-core path (the layout split_planes_kernel writes: [c / 32][plane]
// [padded row][c % 32], the exact three-term split).
__device__ __forceinline__ void write_planes4(uint16_t *planes, uint32_t padded, uint32_t row,
                                              uint32_t c, f32x4 v) {
    uint32_t h[4], md[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = __float_as_uint(v[e]) & 0xffff0000u;
        const float r = v[e] - __uint_as_float(h[e]);
        md[e] = __float_as_uint(r) & 0xffff0000u;
        lo[e] = __float_as_uint(r - __uint_as_float(md[e]));
    }
    const uint64_t at = ((uint64_t)(c / kSplitBK) * 3 * padded + row) * kSplitBK + c % kSplitBK;
    const uint64_t pl = (uint64_t)padded * kSplitBK;
    *(u32x2 *)(planes + at) = u32x2{pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3])};
    *(u32x2 *)(planes + at + pl) = u32x2{pack_hi16(md[0], md[1]), pack_hi16(md[2], md[3])};
    *(u32x2 *)(planes + at + 2 * pl) = u32x2{pack_hi16(lo[0], lo[1]), pack_hi16(lo[2], lo[3])};
}
// One column's value: the same three terms as write_planes4.
__device__ __forceinline__ void write_planes1(uint16_t *planes, uint32_t padded, uint32_t row,
                                              uint32_t c, float v) {
    const uint32_t h = __float_as_uint(v) & 0xffff0000u;
    const float r = v - __uint_as_float(h);
    const uint32_t md = __float_as_uint(r) & 0xffff0000u;
    const uint32_t lo = __float_as_uint(r - __uint_as_float(md));
    const uint64_t at = ((uint64_t)(c / kSplitBK) * 3 * padded + row) * kSplitBK + c % kSplitBK;
    const uint64_t pl = (uint64_t)padded * kSplitBK;
    planes[at] = (uint16_t)(h >> 16);
    planes[at + pl] = (uint16_t)(md >> 16);
    planes[at + 2 * pl] = (uint16_t)(lo >> 16);
}

__global__ __launch_bounds__(256) void split_planes_kernel(const float *x, uint64_t ldx,
                                                           uint32_t rows, uint32_t padded,
                                                           uint32_t k, uint16_t *planes) {
    const uint64_t e = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    const uint64_t total = (uint64_t)padded * k;
    if (e >= total) return;
    const uint32_t row = (uint32_t)(e / k), col = (uint32_t)(e % k);
    // Stage-major destination: [col / 32][plane][row][col % 32].
    const uint64_t at = ((uint64_t)(col / kSplitBK) * 3 * padded + row) * kSplitBK + col % kSplitBK;
    const uint64_t pl = (uint64_t)padded * kSplitBK;
    f32x4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
    if (row < rows) {
        a = *(const f32x4 *)(x + row * ldx + col);
        b = *(const f32x4 *)(x + row * ldx + col + 4);
    }
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[8], md[8], lo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h[i] = __float_as_uint(v[i]) & 0xffff0000u;
        const float r = v[i] - __uint_as_float(h[i]);
        md[i] = __float_as_uint(r) & 0xffff0000u;
        lo[i] = __float_as_uint(r - __uint_as_float(md[i]));
    }
    *(u32x4 *)(planes + at) = u32x4{pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]),
                                    pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7])};
    *(u32x4 *)(planes + at + pl) = u32x4{pack_hi16(md[0], md[1]), pack_hi16(md[2], md[3]),
                                         pack_hi16(md[4], md[5]), pack_hi16(md[6], md[7])};
    *(u32x4 *)(planes + at + 2 * pl) = u32x4{pack_hi16(lo[0], lo[1]), pack_hi16(lo[2], lo[3]),
                                             pack_hi16(lo[4], lo[5]), pack_hi16(lo[6], lo[7])};
}

template <int WM, int WN, int GM = 2, int GN = 2, int PD = 3>
__global__ __launch_bounds__(64 * GM * GN, (WN > 2 || GM * GN > 4) ? 1 : 2) void gemm_split_kernel(
    GemmSplit g) {
    constexpr int NT = 64 * GM * GN;                             // threads: GM x GN waves
    constexpr int BM = 32 * WM * GM, BN = 32 * WN * GN;
    constexpr int AG = 3 * BM * 4, WG = BN * 4, SG = AG + WG;  // granules per stage
    constexpr int APT = AG / NT, WPT = WG / NT;                 // granules per thread
    static_assert(AG % NT == 0 && WG % NT == 0, "whole granules per thread");
    extern __shared__ u32x4 lds[];                               // [3][SG]
    __shared__ int is_last;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wm = wave / GN, wn = wave % GN;
    // Tile of this block. The dispatcher hands blocks to the 8 XCDs in turn
    // (linear block id modulo 8), each with its own L2. With xcd_group, the
    // M tiles of one (weight tile, K split) get consecutive turns on one XCD,
    // so the weight tile crosses HBM once and the other M tiles read it from
    // that XCD's L2 (without it, every M tile re-streams the whole matrix).
    uint32_t bn = blockIdx.x, bm = blockIdx.y, bz = blockIdx.z;
    if (g.xcd_group) {
        const uint32_t lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
        const uint32_t slot = lin / 8, group = slot / gridDim.y * 8 + lin % 8;
        bm = slot % gridDim.y;
        bn = group % gridDim.x;
        bz = group / gridDim.x;
    }
    const uint32_t m0 = bm * BM, n0 = bn * BN;
    const uint32_t kper = g.k / g.splits;
    const uint32_t kbeg = bz * kper, nst = kper / kSplitBK;
    const uint32_t first = bn % nst;  // rotation of this block's stages
    const uint64_t stage_elems = 3ull * g.tp * kSplitBK;  // planes of one stage

    // Staging: granule G = threadIdx + 256 i of the stage; A granules first.
    const uint16_t *asrc[APT];
    uint32_t adst[APT];
#pragma unroll
    for (int i = 0; i < APT; ++i) {
        const uint32_t G = threadIdx.x + NT * i, R = G / 4, q = G % 4;
        const uint32_t p = R / BM, r = R % BM;
        asrc[i] = g.planes + ((uint64_t)p * g.tp + m0 + r) * kSplitBK + 8 * q;
        adst[i] = R * 4 + swizzle(R, q);
    }
    // With swiglu, tile row r of wave column wn and 32-row group j takes the
    // gate (j even) or up (j odd) row of intermediate column
    // bn BN/2 + wn 16 WN + (j / 2) 32 + r % 32: a lane's accumulators j and
    // j + 1 then hold the gate and up sums of one column.
    const uint16_t *wsrc[WPT];
    uint32_t wdst[WPT];
#pragma unroll
    for (int i = 0; i < WPT; ++i) {
        const uint32_t G = threadIdx.x + NT * i, r = G / 4, q = G % 4;
        uint32_t row = min(n0 + r, g.n - 1);
        if (g.swiglu) {
            const uint32_t j = r / 32 % WN;
            const uint32_t col = bn * (BN / 2) + r / (32 * WN) * (16 * WN) + j / 2 * 32 + r % 32;
            row = (j & 1) ? g.swiglu + col : col;
        }
        wsrc[i] = g.w + (uint64_t)row * g.k + 8 * q;
        wdst[i] = AG + r * 4 + swizzle(r, q);
    }
    u32x4 av[PD][APT], wv[PD][WPT];
    auto load = [&](int slot, uint32_t stage) {
        uint32_t s = first + min(stage, nst - 1);
        s = s < nst ? s : s - nst;
        const uint32_t ks = kbeg / kSplitBK + s;
#pragma unroll
        for (int i = 0; i < APT; ++i)
            av[slot][i] = *(const u32x4 *)(asrc[i] + (uint64_t)ks * stage_elems);
#pragma unroll
        for (int i = 0; i < WPT; ++i)
            wv[slot][i] = *(const u32x4 *)(wsrc[i] + (uint64_t)ks * kSplitBK);
    };
    auto store = [&](int slot, uint32_t buf) {
        u32x4 *st = lds + buf * SG;
#pragma unroll
        for (int i = 0; i < APT; ++i) st[adst[i]] = av[slot][i];
#pragma unroll
        for (int i = 0; i < WPT; ++i) st[wdst[i]] = wv[slot][i];
    };
    // Fragments of K step ks (16 columns) of the stage in LDS buffer buf.
    auto frag = [&](uint32_t buf, int ks, bf16x8 (&a)[3][WM], bf16x8 (&b)[WN]) {
        const u32x4 *st = lds + buf * SG;
        const uint32_t q = 2 * ks + (lane >> 5);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int p = 0; p < 3; ++p) {
                const uint32_t R = p * BM + wm * 32 * WM + 32 * i + (lane & 31);
                a[p][i] = __builtin_bit_cast(bf16x8, st[R * 4 + swizzle(R, q)]);
            }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const uint32_t r = wn * 32 * WN + 32 * j + (lane & 31);
            b[j] = __builtin_bit_cast(bf16x8, st[AG + r * 4 + swizzle(r, q)]);
        }
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    auto mfma = [&](const bf16x8 (&a)[3][WM], const bf16x8 (&b)[WN]) {
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[p][i], b[j], acc[i][j],
                                                                         0, 0, 0);
    };

    // Three LDS buffers: stage j + 1 is already in LDS (written during step
    // j - 1) while step j computes stage j, so step j reads the fragments of
    // its own second K step and of stage j + 1's first K step under its
    // MFMAs, writes stage j + 2 into the third buffer, and the next step
    // starts on its MFMAs right after the one barrier per step. Stage s
    // lives in register slot s % PD from its load (step s - 2 - PD) to its
    // LDS write (step s - 2). Loads past the last stage are clamped to it and
    // writes past the last stage land in a buffer no step reads. Every split
    // has at least two stages (K is a multiple of 64).
#pragma unroll
    for (int sl = 0; sl < PD; ++sl) load(sl, sl);
    store(0, 0);
    store(1 % PD, 1);
    load(0, PD);
    load(1 % PD, PD + 1);
    __syncthreads();
    constexpr int NF = 3 * WM + WN, NMF = 3 * WM * WN;  // reads, MFMAs per K step
    bf16x8 a0[3][WM], b0[WN], a1[3][WM], b1[WN];
    frag(0, 0, a0, b0);
    uint32_t cur = 0;  // LDS buffer of stage j
    auto step = [&](int sl, uint32_t j) {
        const int ps = (sl + 2) % PD;  // register slot of stage j + 2
        const uint32_t nxt = cur == 2 ? 0 : cur + 1, nn = nxt == 2 ? 0 : nxt + 1;
        frag(cur, 1, a1, b1);
        mfma(a0, b0);
        store(ps, nn);
        load(ps, j + 2 + PD);
        frag(nxt, 0, a0, b0);
        mfma(a1, b1);
        // Issue order: per MFMA one second-step read, then one LDS write with
        // one global load, then one next-stage read; the matrix cores never
        // wait behind the barrier for LDS (C4 prefill GEMMs 7-12 % faster
        // than reads after the barrier and writes after the MFMAs).
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        }
#pragma unroll
        for (int i = 0; i < APT + WPT; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // LDS write
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load
        }
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        if constexpr (2 * NMF > 2 * NF + APT + WPT)
            __builtin_amdgcn_sched_group_barrier(0x008, 2 * NMF - 2 * NF - APT - WPT, 0);
        // Each step is its own issue-order region, its MFMAs ahead of the
        // barrier.
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        cur = nxt;
    };
    // Whole rounds of PD steps run without a branch, so every path into a
    // step has issued the same loads and the compiler's wait before each LDS
    // write lets the PD - 1 younger stages' loads stay in flight (a skipped
    // step on some path would make it wait for nearly all of them). The last
    // nst % PD steps follow.
    uint32_t j0 = 0;
    for (; j0 + PD <= nst; j0 += PD) {
#pragma unroll
        for (int sl = 0; sl < PD; ++sl) step(sl, j0 + sl);
    }
#pragma unroll
    for (int sl = 0; sl + 1 < PD; ++sl)
        if (j0 + sl < nst) step(sl, j0 + sl);

    // D layout of v_mfma_f32_32x32x16: value v of lane l is row
    // 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32 of the 32 x 32 tile.
    const uint32_t tile = bm * gridDim.x + bn;
    const uint32_t tiles = gridDim.x * gridDim.y;
    if (g.splits > 1) {
        // Partial tile, laid out [split][tile][wave][i][j][v][lane] (coalesced).
        float *part = g.partial + ((uint64_t)bz * tiles + tile) * (BM * BN);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    store_through(part + (((wave * WM + i) * WN + j) * 16 + v) * 64 + lane,
                                  acc[i][j][v]);
        if (!arrive_last(&g.counters[tile], g.splits, &is_last)) return;
        // Sum the partials in split order; each split's 64 values are loaded
        // together.
        const float *base = g.partial + (uint64_t)tile * (BM * BN) + wave * WM * WN * 1024 + lane;
        float sum[WM][WN][16];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    sum[i][j][v] = load_through(base + ((i * WN + j) * 16 + v) * 64);
        for (uint32_t sp = 1; sp < g.splits; ++sp) {
            const float *ps = base + (uint64_t)sp * tiles * (BM * BN);
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
#pragma unroll
                    for (int v = 0; v < 16; ++v)
                        sum[i][j][v] = sum[i][j][v] + load_through(ps + ((i * WN + j) * 16 + v) * 64);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[i][j][v] = sum[i][j][v];
    }
    if (g.swiglu) {
        // silu(gate) * up as in swiglu_planes_kernel (tests/activation_reference.s:99-126),
        // written as the activation's BF16 planes; padding rows are not written.
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; j += 2) {
                const uint32_t col = bn * (BN / 2) + wn * 16 * WN + j / 2 * 32 + (lane & 31);
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t row =
                        m0 + wm * 32 * WM + 32 * i + 8 * (v / 4) + 4 * (lane >> 5) + v % 4;
                    const float gate = acc[i][j][v], up = acc[i][j + 1][v];
                    const float d = plamo_exp(-gate) + 1.0f;
                    if (row < g.t) write_planes1(g.act, g.act_tp, row, col, (gate / d) * up);
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const uint32_t col = n0 + wn * 32 * WN + 32 * j + (lane & 31);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const uint32_t row =
                    m0 + wm * 32 * WM + 32 * i + 8 * (v / 4) + 4 * (lane >> 5) + v % 4;
                if (row < g.t && col < g.n) g.y[(uint64_t)row * g.ldy + col] = acc[i][j][v];
            }
        }
}

template <int WM, int WN, int GM = 2, int GN = 2, int PD = 3>
static hipError_t gemm_split_variant(hipStream_t stream, GemmSplit g, const GemmWorkspace &ws,
                                     bool planes_ready = false) {
    constexpr uint32_t BM = 32 * WM * GM, BN = 32 * WN * GN;
    static_assert(BM == kSplitBM, "gemm_planes_rows pads the planes to kSplitBM rows");
    const uint32_t nt = (g.n + BN - 1) / BN, mt = (g.t + BM - 1) / BM;
    const uint32_t tiles = nt * mt, stages = g.k / kSplitBK;
    g.tp = mt * BM;
    if ((uint64_t)3 * g.tp * g.k > ws.plane_elems) return hipErrorInvalidValue;
    // At most one block per CU (each K split adds a partial tile to write and
    // sum; C4 at 443 tokens, O: 4 splits 61 us, 2 splits 55; QKV: 2 splits
    // 95, 1 split 93; at 116 tokens QKV with 2 splits ties 4), each split at
    // least four stages.
    uint32_t splits = 1;
    while (tiles * splits * 2 <= 256 && stages % (2 * splits) == 0 &&
           stages / (2 * splits) >= 4 && splits < 8)
        splits *= 2;
    // Fewer splits while the partial tiles exceed the workspace (not straight
    // to one: a 96-tile projection would then leave most CUs idle).
    while (splits > 1 && ((uint64_t)splits * tiles * BM * BN > ws.partial_floats ||
                          tiles > ws.counters))
        splits /= 2;
    g.splits = splits;
    g.partial = ws.partial;
    g.counters = ws.counter_base;
    g.planes = ws.planes;
    // Grouping needs whole turns of the 8 XCDs: (weight tiles x splits) % 8 == 0.
    g.xcd_group = mt > 1 && (nt * splits) % 8 == 0;
    const uint64_t elems = (uint64_t)g.tp * g.k;
    if (!planes_ready)
        split_planes_kernel<<<(unsigned)((elems / 8 + 255) / 256), 256, 0, stream>>>(
            g.x, g.ldx, g.t, g.tp, g.k, ws.planes);
    const size_t lds = 3 * (size_t)(3 * BM * 4 + BN * 4) * sizeof(u32x4);
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void *)gemm_split_kernel<WM, WN, GM, GN, PD>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    gemm_split_kernel<WM, WN, GM, GN, PD><<<dim3(nt, mt, splits), 64 * GM * GN, lds, stream>>>(g);
    return hipGetLastError();
}

// ---------------------------------------------------------------- skinny split-BF16 GEMM
// C[t, r] = sum_k X[t, k] * W[r, k] for at most 16 tokens (candidate
// verification, short prompts, granular projections). Weight-streaming: each
// weight byte is read once, as in the decode GEMV. v_mfma_f32_16x16x32_bf16
// takes 16 weight rows as M and the tokens (padded to 16 with zeros) as N;
// each FP32 x is split into its three exact BF16 terms in registers (the split
// of split_planes_kernel), so the products are exact and accumulate in FP32.
//
// Grid (row blocks, K slices). A block stages X[:, slice] in LDS once (rows
// padded by 16 bytes against bank conflicts), then each of its 4 waves streams
// R tiles of 16 weight rows over the slice, two steps of 32 U columns in
// flight (register double buffer). With several K slices, each block writes
// its tiles to the workspace and the last block of a row block adds them in
// slice order (deterministic).
//
// MFMA u of a step takes columns 32 u .. 32 u + 31 and lane quarter q the 8
// starting at 32 u + 8 q, so one load instruction reads 64 contiguous bytes of
// each of its 16 rows. Lane layout of v_mfma_f32_16x16x32: A row and B column
// = lane % 16; D value e of lane l is row 4 (l / 16) + e, column l % 16.
struct SkinnyGemm {
    const float *x;
    uint64_t ldx;
    const uint16_t *w;
    uint32_t n, k, t, kc, slices;
    float *y;
    uint64_t ldy;
    float *partial;
    uint32_t *counters;
};

constexpr uint32_t kSkinnyTokens = 16;
constexpr uint32_t kSkinnyU = 4;
constexpr uint32_t kSkinnyStep = 32 * kSkinnyU;       // columns per step
constexpr uint32_t kSkinnyLdsFloats = 12288;          // X slice budget per block (48 KiB)

template <int R, int U>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(SkinnyGemm g) {
    constexpr uint32_t KS = 32 * U;
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [t][kc + 4]
    __shared__ int is_last;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t col = lane & 15, q = lane >> 4;
    const uint32_t k0 = blockIdx.y * g.kc, stride = g.kc + 4;
    const uint32_t r0 = (blockIdx.x * 4 + wave) * 16 * R;
    // Stage the slice of X.
    const uint32_t g4 = g.kc / 4;
    for (uint32_t e = threadIdx.x; e < g.t * g4; e += 256) {
        const uint32_t tok = e / g4, c = (e - tok * g4) * 4;
        *(f32x4 *)(xs + tok * stride + c) =
            *(const f32x4 *)(g.x + (uint64_t)tok * g.ldx + k0 + c);
    }
    const uint16_t *wr[R];
#pragma unroll
    for (int rt = 0; rt < R; ++rt)
        wr[rt] = g.w + (uint64_t)min(r0 + 16 * rt + col, g.n - 1) * g.k + k0 + 8 * q;
    const bool live = col < g.t;  // B column = token
    const float *xl = xs + (live ? col : 0) * stride + 8 * q;
    const uint32_t steps = g.kc / KS;  // even

    f32x4 acc[R];
#pragma unroll
    for (int rt = 0; rt < R; ++rt) acc[rt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 a0[R][U], a1[R][U];
    auto load = [&](u32x4 (&a)[R][U], uint32_t s) {
#pragma unroll
        for (int rt = 0; rt < R; ++rt)
#pragma unroll
            for (int u = 0; u < U; ++u)
                a[rt][u] = __builtin_nontemporal_load(
                    (const u32x4 *)(wr[rt] + (uint64_t)s * KS + 32 * u));
    };
    auto compute = [&](const u32x4 (&a)[R][U], uint32_t s) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            f32x4 x0 = *(const f32x4 *)(xl + s * KS + 32 * u);
            f32x4 x1 = *(const f32x4 *)(xl + s * KS + 32 * u + 4);
            const float v8[8] = {live ? x0.x : 0.0f, live ? x0.y : 0.0f, live ? x0.z : 0.0f,
                                 live ? x0.w : 0.0f, live ? x1.x : 0.0f, live ? x1.y : 0.0f,
                                 live ? x1.z : 0.0f, live ? x1.w : 0.0f};
            uint32_t h[8], md[8], lo[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                h[e] = __float_as_uint(v8[e]) & 0xffff0000u;
                const float r = v8[e] - __uint_as_float(h[e]);
                md[e] = __float_as_uint(r) & 0xffff0000u;
                lo[e] = __float_as_uint(r - __uint_as_float(md[e]));
            }
            const bf16x8 bh = __builtin_bit_cast(
                bf16x8, u32x4{pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]),
                              pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7])});
            const bf16x8 bm = __builtin_bit_cast(
                bf16x8, u32x4{pack_hi16(md[0], md[1]), pack_hi16(md[2], md[3]),
                              pack_hi16(md[4], md[5]), pack_hi16(md[6], md[7])});
            const bf16x8 bl = __builtin_bit_cast(
                bf16x8, u32x4{pack_hi16(lo[0], lo[1]), pack_hi16(lo[2], lo[3]),
                              pack_hi16(lo[4], lo[5]), pack_hi16(lo[6], lo[7])});
#pragma unroll
            for (int rt = 0; rt < R; ++rt) {
                const bf16x8 av = __builtin_bit_cast(bf16x8, a[rt][u]);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bh, acc[rt], 0, 0, 0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bm, acc[rt], 0, 0, 0);
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bl, acc[rt], 0, 0, 0);
            }
        }
    };
    // Loads are unconditional inside the loop (two steps per trip, the last
    // pair peeled) so the compiler keeps exact wait counts.
    // sched_barrier keeps each group of loads whole and in place, so waiting
    // for one buffer never waits for the other's prefetch.
    load(a0, 0);
    __syncthreads();
    uint32_t s = 0;
    for (; s + 2 < steps; s += 2) {
        load(a1, s + 1);
        __builtin_amdgcn_sched_barrier(0);
        compute(a0, s);
        __builtin_amdgcn_sched_barrier(0);
        load(a0, s + 2);
        __builtin_amdgcn_sched_barrier(0);
        compute(a1, s + 1);
        __builtin_amdgcn_sched_barrier(0);
    }
    load(a1, s + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(a0, s);
    __builtin_amdgcn_sched_barrier(0);
    compute(a1, s + 1);

    if (g.slices > 1) {
        // Tile layout [slice][row block][wave][rt][lane][4] (coalesced).
        float *part = g.partial +
                      (((uint64_t)blockIdx.y * gridDim.x + blockIdx.x) * 4 + wave) * R * 256;
#pragma unroll
        for (int rt = 0; rt < R; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) store_through(part + (rt * 4 + e) * 64 + lane, acc[rt][e]);
        if (!arrive_last(&g.counters[blockIdx.x], g.slices, &is_last)) return;
        const uint64_t slice_floats = (uint64_t)gridDim.x * 4 * R * 256;
        const float *base = g.partial + ((uint64_t)blockIdx.x * 4 + wave) * R * 256 + lane;
#pragma unroll
        for (int rt = 0; rt < R; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[rt][e] = load_through(base + (rt * 4 + e) * 64);
        for (uint32_t sl = 1; sl < g.slices; ++sl)
#pragma unroll
            for (int rt = 0; rt < R; ++rt)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[rt][e] = acc[rt][e] +
                                 load_through(base + sl * slice_floats + (rt * 4 + e) * 64);
    }
    if (!live) return;
    float *yr = g.y + (uint64_t)col * g.ldy;
#pragma unroll
    for (int rt = 0; rt < R; ++rt) {
        const uint32_t row = r0 + 16 * rt + 4 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (row + e < g.n) yr[row + e] = acc[rt][e];
    }
}

// Slices of K: the fewest whose X slice fits the LDS budget, doubled while
// the grid is under two blocks per CU and each slice keeps at least four
// steps. 0 when K does not split into even step counts.
static uint32_t skinny_slices(uint64_t cols, uint64_t tokens, uint32_t row_blocks) {
    const uint64_t unit = 2 * kSkinnyStep;
    if (cols % unit) return 0;
    const uint64_t units = cols / unit;
    uint32_t slices = 0;
    for (uint32_t sl = 1; sl <= units && sl <= 64; ++sl)
        if (units % sl == 0 && tokens * (cols / sl + 4) <= kSkinnyLdsFloats) {
            slices = sl;
            break;
        }
    if (!slices) return 0;
    while ((uint64_t)row_blocks * slices < 512 && units % (2 * slices) == 0 &&
           cols / (2 * slices) >= 2 * unit && slices < 64)
        slices *= 2;
    return slices;
}

template <int R>
static hipError_t skinny_gemm_variant(hipStream_t stream, SkinnyGemm g, const GemmWorkspace *ws) {
    const uint32_t row_blocks = (g.n + 64 * R - 1) / (64 * R);
    uint32_t slices = skinny_slices(g.k, g.t, row_blocks);
    if (!slices) return hipErrorInvalidValue;
    if (slices > 1 && (!ws || !ws->partial || row_blocks > ws->counters ||
                       (uint64_t)slices * row_blocks * 4 * R * 256 > ws->partial_floats))
        return hipErrorInvalidValue;
    g.slices = slices;
    g.kc = g.k / slices;
    g.partial = ws ? ws->partial : nullptr;
    g.counters = ws ? ws->counter_base : nullptr;
    const size_t lds = (size_t)g.t * (g.kc + 4) * 4;
    skinny_gemm_kernel<R, kSkinnyU><<<dim3(row_blocks, slices), 256, lds, stream>>>(g);
    return hipGetLastError();
}

static bool skinny_supported(const float *x, uint64_t x_stride, const uint16_t *w, uint64_t rows,
                             uint64_t cols, uint64_t tokens) {
    return tokens <= kSkinnyTokens && rows < (1u << 31) && cols <= (1u << 30) &&
           x_stride % 4 == 0 && !((uintptr_t)x & 15) && !((uintptr_t)w & 15) &&
           skinny_slices(cols, tokens, 1 << 20) != 0;
}

// ---------------------------------------------------------------- token GEMV
// C[t, r] = sum_k X[t, k] * W[r, k] for 1..5 tokens (candidate verification,
// short prompts) on the vector ALUs, with the decode GEMV's weight stream:
// lane l reads the 16 bytes at column 512 c + 8 l of a row, so one load
// instruction covers 1 KB of one row (the matrix-core operand layout covers
// 16 rows x 64 B per instruction and streams about a third slower).
//
// Grid (row groups, K slices). A block stages X[:, slice] in LDS; each wave
// takes units of U = 8 rows (with SwiGLU: gate rows 4j .. 4j + 3 and up rows
// half + 4j .. half + 4j + 3) and streams a unit over the slice KC = 2 chunks
// (16 KB) per sub-step, two sub-steps in flight. Each x read from LDS feeds
// U rows: fewer rows per unit left the waves waiting on LDS. Every weight is multiplied
// into T accumulators (per lane, row and token one FMA chain in column
// order); the 64 lanes are summed once per unit (wave butterfly) and the sums
// staged in LDS. With one slice they are the results; with several, each
// block writes its sums through to the workspace and the last block of a row
// group adds the slices in order, so results are run-to-run deterministic.
struct TokenGemv {
    const float *x;
    uint64_t ldx;
    const uint16_t *w;
    uint32_t n, k, ks, slices, half, local;
    float *y;
    uint64_t ldy;
    float *partial;
    uint32_t *counters;
};

// Up to five tokens the vector ALUs keep pace with the weight stream; from
// six, the x reads from LDS (2 T / U bytes per weight byte) bound the kernel
// and the matrix-core skinny GEMM is faster.
constexpr uint32_t kTokenMax = 5;
constexpr uint32_t kTokenU = 8;
constexpr uint32_t kTokenKC = 2;
constexpr uint32_t kTokenXBytes = 128 * 1024;    // X slice per block
constexpr uint32_t kTokenLdsBytes = 156 * 1024;  // X slice + staged sums: one block per CU

// EVEN: the slice's chunk count is a multiple of KC (every sub-step is whole):
// the FMAs run without a chunk test, and a row's KC registers are reissued
// together once its last chunk is consumed, so each row's 2 KB goes out as
// one contiguous run (C5 verify(5) 14.84 -> 14.66 ms against reissuing in
// consumption order, chunk by chunk).
template <int T, bool EVEN>
__global__ __launch_bounds__(256, 1) void token_gemv_kernel(TokenGemv g) {
    static_assert(T >= 1 && T <= (int)kTokenMax, "token count the plan admits");
    constexpr uint32_t U = kTokenU, KC = kTokenKC, UT = U * T, H = U / 2;
    extern __shared__ __attribute__((aligned(16))) float tg_lds[];
    // X slice [T][ks], each 512-column chunk as two planes: lane l's columns
    // 8 l .. 8 l + 3 at 4 l, and 8 l + 4 .. 8 l + 7 at 256 + 4 l, so both of a
    // lane's 16-byte reads are 1 KB contiguous across the wave.
    float *xs = tg_lds;
    float *outs = tg_lds + T * g.ks;  // [wave][local][U][T]
    __shared__ int is_last;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t k0 = blockIdx.y * g.ks;
    const uint32_t chunks = g.ks / 512, nsub = (chunks + KC - 1) / KC;
    const bool swiglu = g.half != 0;
    const uint32_t units = swiglu ? g.half / H : (g.n + U - 1) / U;
    const uint32_t first = blockIdx.x * 4 + wave, stride = gridDim.x * 4;
    const uint32_t mine = first < units ? (units - first + stride - 1) / stride : 0;
    const uint16_t *wl = g.w + k0 + lane * 8;
    const uint32_t last = g.n - 1;

    u32x4 a0[U][KC], a1[U][KC];
    // The weight register a[u][c] of sub-step (ul, sub). Past the wave's last
    // unit, or past the slice's last chunk, the lanes read the slice's first
    // chunk of row 0 instead: the number of loads stays fixed, so the
    // compiler's wait counts stay exact, and the (wave-uniform) offset is a
    // select rather than a branch.
    auto load_one = [&](u32x4 &a, uint32_t ul, uint32_t sub, uint32_t u, uint32_t c) {
        const uint32_t unit = first + ul * stride;
        uint32_t r = swiglu ? (u < H ? H * unit + u : g.half + H * unit + (u - H))
                            : unit * U + u;
        r = r > last ? last : r;
        const bool ok = ul < mine && sub * KC + c < chunks;
        const uint64_t off = (uint64_t)r * g.k + (sub * KC + c) * 512;
        a = __builtin_nontemporal_load((const u32x4 *)(wl + (ok ? off : 0)));
    };
    // A whole sub-step's loads: row by row when the reloads go out that way
    // (EVEN), else in the order the FMAs consume them (chunk, then row).
    auto load = [&](u32x4 (&a)[U][KC], uint32_t ul, uint32_t sub) {
        if (EVEN) {
#pragma unroll
            for (uint32_t u = 0; u < U; ++u)
#pragma unroll
                for (uint32_t c = 0; c < KC; ++c) load_one(a[u][c], ul, sub, u, c);
        } else {
#pragma unroll
            for (uint32_t c = 0; c < KC; ++c)
#pragma unroll
                for (uint32_t u = 0; u < U; ++u) load_one(a[u][c], ul, sub, u, c);
        }
    };
    float acc[U][T];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < T; ++t) acc[u][t] = 0.0f;
    // One sub-step's FMAs. The weight registers are reissued for the sub-step
    // two ahead (nl, ns) as soon as they are unpacked, so a load has about two
    // sub-steps of compute to land instead of one.
    auto step = [&](u32x4 (&a)[U][KC], uint32_t ul, uint32_t sub, uint32_t nl, uint32_t ns) {
#pragma unroll
        for (uint32_t c = 0; c < KC; ++c) {
            const uint32_t chunk = sub * KC + c;
            if (!EVEN && chunk >= chunks) {
#pragma unroll
                for (uint32_t u = 0; u < U; ++u) load_one(a[u][c], nl, ns, u, c);
            } else {
                const float *xc = xs + chunk * 512 + lane * 4;
                float xv[T][8];
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const f32x4 p = *(const f32x4 *)(xc + t * g.ks);
                    const f32x4 q = *(const f32x4 *)(xc + t * g.ks + 256);
                    xv[t][0] = p.x; xv[t][1] = p.y; xv[t][2] = p.z; xv[t][3] = p.w;
                    xv[t][4] = q.x; xv[t][5] = q.y; xv[t][6] = q.z; xv[t][7] = q.w;
                }
#pragma unroll
                for (uint32_t u = 0; u < U; ++u) {
                    const uint32_t q[4] = {a[u][c].x, a[u][c].y, a[u][c].z, a[u][c].w};
                    float wv[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        wv[2 * e] = bf16f(q[e] & 0xffffu);
                        wv[2 * e + 1] = __uint_as_float(q[e] & 0xffff0000u);
                    }
                    if (!EVEN) {
                        load_one(a[u][c], nl, ns, u, c);
                    } else if (c + 1 == KC) {
#pragma unroll
                        for (uint32_t cc = 0; cc < KC; ++cc) load_one(a[u][cc], nl, ns, u, cc);
                    }
                    __builtin_amdgcn_sched_barrier(0);  // reloads go out before the FMAs
#pragma unroll
                    for (int t = 0; t < T; ++t)
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            acc[u][t] = __builtin_fmaf(wv[e], xv[t][e], acc[u][t]);
                }
            }
        }
        if (sub + 1 == nsub) {  // the unit's slice is done
            float *o = outs + (wave * g.local + ul) * UT;
#pragma unroll
            for (uint32_t u = 0; u < U; ++u)
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    const float s = wave_total(acc[u][t]);
                    if (lane == 63) o[u * T + t] = s;
                    acc[u][t] = 0.0f;
                }
        }
    };
    auto advance = [&](uint32_t &ul, uint32_t &sub) {
        if (++sub == nsub) {
            sub = 0;
            ++ul;
        }
    };

    uint32_t lu = 0, ls = 0;  // next sub-step to load
    // The prologue issues a0's loads strictly before a1's, as the loop does:
    // the wait counts at the loop head merge both orders.
    load(a0, lu, ls);
    advance(lu, ls);
    __builtin_amdgcn_sched_barrier(0);
    load(a1, lu, ls);
    advance(lu, ls);
    __builtin_amdgcn_sched_barrier(0);
    // Stage X[:, slice]: one direct-to-LDS load per (token, chunk, plane),
    // spread over the waves and all in flight at once. Lane l's 16 bytes land
    // at 16 l of the plane, which is the plane layout above: plane 0 of a
    // chunk holds columns 8 l .. 8 l + 3, plane 1 columns 8 l + 4 .. 8 l + 7.
    {
        const uint32_t planes = T * chunks * 2;
        for (uint32_t i = wave; i < planes; i += 4) {
            const uint32_t t = i / (2 * chunks), r = i - t * 2 * chunks, c = r >> 1, pl = r & 1;
            const float *src = g.x + (uint64_t)t * g.ldx + k0 + c * 512 + pl * 4 + lane * 8;
            __builtin_amdgcn_global_load_lds(
                src, (__attribute__((address_space(3))) void *)(xs + t * g.ks + c * 512 + pl * 256),
                16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    const uint32_t items = mine * nsub;
    uint32_t cu = 0, cs = 0;  // next sub-step to compute
    // Whole pairs in the loop, so every path back to its head has the same
    // loads in flight and the waits before each row's FMAs leave the two
    // sub-steps ahead outstanding.
    for (uint32_t i = 0; i + 1 < items; i += 2) {
        step(a0, cu, cs, lu, ls);
        advance(cu, cs);
        advance(lu, ls);
        __builtin_amdgcn_sched_barrier(0);
        step(a1, cu, cs, lu, ls);
        advance(cu, cs);
        advance(lu, ls);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (items & 1) step(a0, cu, cs, lu, ls);
    __syncthreads();

    const uint32_t per = 4 * g.local * UT;  // staged sums of the block
    if (g.slices > 1) {
        float *part = g.partial + ((uint64_t)blockIdx.y * gridDim.x + blockIdx.x) * per;
        for (uint32_t e = threadIdx.x; e < per; e += 256) store_through(part + e, outs[e]);
        if (!arrive_last(&g.counters[blockIdx.x], g.slices, &is_last)) return;
        for (uint32_t e = threadIdx.x; e < per; e += 256) {
            const float *p = g.partial + (uint64_t)blockIdx.x * per + e;
            float s = load_through(p);
            for (uint32_t sl = 1; sl < g.slices; ++sl)
                s += load_through(p + (uint64_t)sl * gridDim.x * per);
            outs[e] = s;
        }
        __syncthreads();
    }
    if (swiglu) {
        // silu(gate) * up (tests/activation_reference.s:99-126).
        for (uint32_t e = threadIdx.x; e < 4 * g.local * H * T; e += 256) {
            const uint32_t t = e % T, u = (e / T) % H, wl_ = e / (H * T);  // wl_ = w * local + ul
            const uint32_t w = wl_ / g.local, ul = wl_ - w * g.local;
            const uint32_t unit = blockIdx.x * 4 + w + ul * stride;
            if (unit >= units) continue;
            const float gt = outs[(wl_ * U + u) * T + t], up = outs[(wl_ * U + u + H) * T + t];
            const float d = plamo_exp(-gt) + 1.0f;
            g.y[(uint64_t)t * g.ldy + H * unit + u] = (gt / d) * up;
        }
    } else {
        for (uint32_t e = threadIdx.x; e < per; e += 256) {
            const uint32_t t = e % T, u = (e / T) % U, wl_ = e / UT;
            const uint32_t w = wl_ / g.local, ul = wl_ - w * g.local;
            const uint32_t unit = blockIdx.x * 4 + w + ul * stride, row = unit * U + u;
            if (unit < units && row < g.n) g.y[(uint64_t)t * g.ldy + row] = outs[e];
        }
    }
}

struct TokenPlan {
    uint32_t slices, ks, blocks, local;
    size_t lds;
};

// Slices: the fewest (dividing the 512-column chunks) whose X slice fits
// kTokenXBytes (a 6144-wide projection of 5 tokens needs none). Row groups:
// one block per CU over all slices, fewer when rows run out, more when the
// staged sums would not fit the LDS budget. (Two blocks per CU with 64 KB
// slices: verify(5) at C5 17.7 against 17.0 ms.)
static bool token_plan(uint64_t rows, uint64_t cols, uint64_t tokens, uint64_t half,
                       uint32_t cus, TokenPlan &p) {
    if (!tokens || tokens > kTokenMax || !rows || cols % 512 || cols > (1u << 30) ||
        rows >= (1u << 30) || (half && (half % (kTokenU / 2) || rows != 2 * half)))
        return false;
    const uint64_t chunks = cols / 512;
    const uint64_t units = half ? half / (kTokenU / 2) : (rows + kTokenU - 1) / kTokenU;
    const uint64_t budget = kTokenLdsBytes / 4 / tokens;  // floats per block per token
    // The grid for `slices` K slices; false when its X slice or staged sums
    // do not fit.
    auto shape = [&](uint64_t slices, TokenPlan &q) {
        const uint64_t ks = cols / slices;
        if (tokens * ks * 4 > kTokenXBytes || budget <= ks) return false;
        uint64_t blocks = std::max<uint64_t>(1, 1ull * std::max<uint32_t>(cus, 1) / slices);
        blocks = std::min<uint64_t>(blocks, (units + 3) / 4);
        const uint64_t max_local = (budget - ks) / (4 * kTokenU);
        if (!max_local) return false;
        uint64_t local = (units + 4 * blocks - 1) / (4 * blocks);
        if (local > max_local) {
            blocks = (units + 4 * max_local - 1) / (4 * max_local);
            local = (units + 4 * blocks - 1) / (4 * blocks);
        }
        if (blocks > 65535) return false;
        q.slices = (uint32_t)slices;
        q.ks = (uint32_t)ks;
        q.blocks = (uint32_t)blocks;
        q.local = (uint32_t)local;
        q.lds = (size_t)tokens * (ks + 4 * kTokenU * local) * 4;
        return true;
    };
    // The fewest slices that fit. When those leave the waves unequal shares
    // of the units, the slicing with the shortest longest-wave stream (units
    // x slice columns) instead, if it is at least a tenth shorter: with 4
    // tokens, a 24576-column down projection in 3 slices leaves its 768 units
    // 3 or 2 per wave (68.8 us), in 4 slices exactly 3.
    bool found = false;
    uint64_t best = 0, first_cost = 0;
    for (uint64_t d = 1; d <= chunks; ++d) {
        TokenPlan q;
        if (chunks % d || !shape(d, q)) continue;
        const uint64_t cost = (uint64_t)q.local * q.ks;
        if (!found) {
            p = q;
            best = first_cost = cost;
            found = true;
            if (units % (4ull * q.blocks) == 0) break;  // equal shares
        } else if (cost < best && cost * 10 <= first_cost * 9) {
            p = q;
            best = cost;
        }
    }
    return found;
}

// The token GEMV stages up to kTokenLdsBytes, above the default 64 KiB.
static hipError_t configure_token_gemv() {
    const void *kernels[] = {
        (const void *)token_gemv_kernel<1, false>, (const void *)token_gemv_kernel<2, false>,
        (const void *)token_gemv_kernel<3, false>, (const void *)token_gemv_kernel<4, false>,
        (const void *)token_gemv_kernel<5, false>, (const void *)token_gemv_kernel<1, true>,
        (const void *)token_gemv_kernel<2, true>,  (const void *)token_gemv_kernel<3, true>,
        (const void *)token_gemv_kernel<4, true>,  (const void *)token_gemv_kernel<5, true>};
    for (const void *k : kernels) {
        hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kTokenLdsBytes);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <int T>
static hipError_t token_gemv_variant(hipStream_t stream, const TokenGemv &g, const TokenPlan &p) {
    if ((p.ks / 512) % kTokenKC == 0)
        token_gemv_kernel<T, true><<<dim3(p.blocks, p.slices), 256, p.lds, stream>>>(g);
    else
        token_gemv_kernel<T, false><<<dim3(p.blocks, p.slices), 256, p.lds, stream>>>(g);
    return hipGetLastError();
}

// hipErrorNotSupported (nothing launched) when the shape or the workspace
// does not fit the token GEMV.
static hipError_t launch_token_gemv(hipStream_t stream, const float *x, uint64_t x_stride,
                                    const uint16_t *w, uint64_t rows, uint64_t cols,
                                    uint64_t tokens, uint64_t half, float *y, uint64_t y_stride,
                                    const GemmWorkspace *ws) {
    TokenPlan p;
    if (!ws || !token_plan(rows, cols, tokens, half, ws->cus, p) || x_stride % 4 ||
        ((uintptr_t)x & 15) || ((uintptr_t)w & 15))
        return hipErrorNotSupported;
    if (p.slices > 1 && (!ws->partial || !ws->counter_base || p.blocks > ws->counters ||
                         (uint64_t)p.slices * p.blocks * 4 * p.local * kTokenU * tokens >
                             ws->partial_floats))
        return hipErrorNotSupported;
    TokenGemv g{};
    g.x = x;
    g.ldx = x_stride;
    g.w = w;
    g.n = (uint32_t)rows;
    g.k = (uint32_t)cols;
    g.ks = p.ks;
    g.slices = p.slices;
    g.half = (uint32_t)half;
    g.local = p.local;
    g.y = y;
    g.ldy = y_stride;
    g.partial = ws->partial;
    g.counters = ws->counter_base;
    switch (tokens) {
    case 1: return token_gemv_variant<1>(stream, g, p);
    case 2: return token_gemv_variant<2>(stream, g, p);
    case 3: return token_gemv_variant<3>(stream, g, p);
    case 4: return token_gemv_variant<4>(stream, g, p);
    default: return token_gemv_variant<5>(stream, g, p);
    }
}

static bool gemm_split_supported(const float *x, uint64_t x_stride, const uint16_t *w,
                                 uint64_t cols) {
    return cols % (2 * kSplitBK) == 0 && x_stride % 4 == 0 && !((uintptr_t)x & 15) &&
           !((uintptr_t)w & 15) && cols <= (1u << 30);
}

uint64_t gemm_plane_elems(uint64_t tokens, uint64_t cols) {
    return 3 * ((tokens + 127) / 128 * 128) * cols;
}

uint32_t gemm_planes_rows(uint64_t tokens, uint64_t cols, const GemmWorkspace *ws) {
    if (tokens <= kSkinnyTokens || tokens >= (1u << 31) || cols % (2 * kSplitBK) ||
        cols > (1u << 30) || !ws || !ws->planes)
        return 0;
    const uint64_t tp = (tokens + kSplitBM - 1) / kSplitBM * kSplitBM;
    return 3 * tp * cols <= ws->plane_elems && gemm_plane_elems(tokens, cols) <= ws->plane_elems
               ? (uint32_t)tp
               : 0;
}

// Wide tiles (256 weight rows per block, each wave 32 tokens x 128 rows)
// except for short prompts' projections with few row tiles and K below 8192,
// which take 128-row tiles (each wave 32 x 64) and get more blocks. Measured
// per C4 projection at 69-1024 tokens against 128-token tiles of 8 waves
// (64 x 64 each): the wide 64-token tiles win from 200 tokens on (443: QKV
// 125.7 -> 101.4 us, O 76.1 -> 64.4, gate/up 433.6 -> 399.9, down 227.6 ->
// 213.1), and down at 116 (76.3 -> 75.2, K 16384).
static bool gemm_split_wide(uint64_t rows, uint64_t cols, uint64_t tokens) {
    return tokens > 128 || cols >= 8192 || (rows + 255) / 256 >= 64;
}
// The matrix-core GEMM's tiling for g.n rows, g.t tokens (both tilings have
// an even number of 32-row groups per wave, as a swiglu launch needs). Three
// K stages in registers ahead of the LDS stages (2 and 4 measured within
// 1-4 % of it, either way, with three LDS buffers).
// The weights are read with ordinary loads: each 64-byte stage of a row is
// half a 128-byte cache line whose other half the next stage reads, and
// non-temporal loads, which let the line go, measured slower in place (C4 at
// 443 tokens: QKV 114.1 -> 97.2 us, O 67.9 -> 60.6, gate/up 381.9 -> 362.5,
// down 200.0 -> 187.5; at 116: QKV 40.6 -> 36.9, gate/up equal within the
// spread between boxes).
// Past 128 tokens, a projection whose 256-row tiles leave CUs idle takes
// 192-row tiles when their count still fits one round of 256 blocks (not for
// SwiGLU, whose gate/up pairing needs an even number of 32-row groups per
// wave): C4 QKV at 443 tokens, 7 x 24 = 168 against 7 x 32 = 224 blocks,
// 87.4-89.3 -> 81.7-85.7 us with planes ready.
static bool gemm_split_192(const GemmSplit &g) {
    if (g.swiglu || g.t <= 128 || g.n % 192) return false;
    const uint64_t mt = (g.t + kSplitBM - 1) / kSplitBM;
    const uint64_t b256 = mt * ((g.n + 255) / 256), b192 = mt * (g.n / 192);
    return b256 < 256 && b192 <= 256 && b192 > b256;
}
static hipError_t gemm_split_route(hipStream_t stream, const GemmSplit &g, const GemmWorkspace &ws,
                                   bool planes_ready) {
    if (gemm_split_192(g)) return gemm_split_variant<1, 3, 2, 2, 3>(stream, g, ws, planes_ready);
    return gemm_split_wide(g.n, g.k, g.t)
               ? gemm_split_variant<1, 4, 2, 2, 3>(stream, g, ws, planes_ready)
               : gemm_split_variant<1, 2, 2, 2, 3>(stream, g, ws, planes_ready);
}
// Rows of one tile of the route above (the swiglu pairing needs the
// intermediate size to be whole half tiles).
static uint32_t gemm_split_tile_rows(uint64_t rows, uint64_t cols, uint64_t tokens) {
    return gemm_split_wide(rows, cols, tokens) ? 256 : 128;
}

hipError_t launch_gemm(hipStream_t stream, const float *x, uint64_t x_stride, const uint16_t *w,
                       uint64_t rows, uint64_t cols, uint64_t tokens, float *y,
                       uint64_t y_stride, const GemmWorkspace *ws, bool planes_ready) {
    if (!tokens || !rows) return hipSuccess;
    // planes_ready callers may not have written x: only the matrix-core route
    // below may take them.
    if (planes_ready && tokens <= kSkinnyTokens) return hipErrorInvalidValue;
    {
        hipError_t e = launch_token_gemv(stream, x, x_stride, w, rows, cols, tokens, 0, y,
                                         y_stride, ws);
        if (e != hipErrorNotSupported) return e;
    }
    if (skinny_supported(x, x_stride, w, rows, cols, tokens)) {
        SkinnyGemm g{};
        g.x = x;
        g.ldx = x_stride;
        g.w = w;
        g.n = (uint32_t)rows;
        g.k = (uint32_t)cols;
        g.t = (uint32_t)tokens;
        g.y = y;
        g.ldy = y_stride;
        hipError_t e = rows >= 16384 ? skinny_gemm_variant<2>(stream, g, ws)
                                     : skinny_gemm_variant<1>(stream, g, ws);
        if (e != hipErrorInvalidValue) return e;
    }
    if (ws && ws->planes && tokens > 1 && rows < (1u << 31) && tokens < (1u << 31) &&
        gemm_split_supported(x, x_stride, w, cols) &&
        gemm_plane_elems(tokens, cols) <= ws->plane_elems) {
        GemmSplit g{};
        g.x = x;
        g.ldx = x_stride;
        g.w = w;
        g.n = (uint32_t)rows;
        g.k = (uint32_t)cols;
        g.t = (uint32_t)tokens;
        g.y = y;
        g.ldy = y_stride;
        return gemm_split_route(stream, g, *ws, planes_ready);
    }
    if (planes_ready) return hipErrorInvalidValue;
    if (tokens <= 16) return gemm_variant<16, 64>(stream, x, x_stride, w, rows, cols, tokens, y, y_stride);
    return gemm_variant<64, 64>(stream, x, x_stride, w, rows, cols, tokens, y, y_stride);
}

hipError_t launch_gemm_swiglu(hipStream_t stream, const float *x, uint64_t x_stride,
                              const uint16_t *w, uint64_t intermediate, uint64_t cols,
                              uint64_t tokens, float *act, float *gate_up,
                              const GemmWorkspace *ws, bool planes_ready, uint32_t act_planes,
                              uint16_t **act_at) {
    if (act_at) *act_at = ws ? ws->planes : nullptr;
    if (!tokens || !intermediate) return hipSuccess;
    // Checked before anything is launched: a failure leaves the stream as it was.
    if (act_planes && (!ws || !ws->planes || 3ull * act_planes * intermediate > ws->plane_elems ||
                       act_planes < tokens || intermediate % (2 * kSplitBK) ||
                       intermediate >= (1u << 30) || ((uintptr_t)gate_up & 15)))
        return hipErrorInvalidValue;
    // The gate/up GEMM writes the activation planes from its epilogue, past
    // the input's planes (which its running blocks still read), when the
    // workspace holds both: one launch less and no FP32 gate/up rows.
    if (act_planes && act_at && tokens > kSkinnyTokens && tokens < (1u << 31) &&
        2 * intermediate < (1u << 31) && gemm_split_supported(x, x_stride, w, cols) &&
        intermediate % (gemm_split_tile_rows(2 * intermediate, cols, tokens) / 2) == 0 &&
        gemm_planes_rows(tokens, cols, ws) == act_planes) {
        const uint64_t in_elems = 3ull * act_planes * cols;
        if (in_elems + 3ull * act_planes * intermediate <= ws->plane_elems) {
            GemmSplit g{};
            g.x = x;
            g.ldx = x_stride;
            g.w = w;
            g.n = (uint32_t)(2 * intermediate);
            g.k = (uint32_t)cols;
            g.t = (uint32_t)tokens;
            g.swiglu = (uint32_t)intermediate;
            g.act = ws->planes + in_elems;
            g.act_tp = act_planes;
            *act_at = g.act;
            return gemm_split_route(stream, g, *ws, planes_ready);
        }
    }
    // The token GEMV reads x and writes act as FP32 only: it takes neither
    // input planes in place of x nor planes for the output.
    if (!planes_ready && !act_planes) {
        hipError_t e = launch_token_gemv(stream, x, x_stride, w, 2 * intermediate, cols, tokens,
                                         intermediate, act, intermediate, ws);
        if (e != hipErrorNotSupported) return e;
    }
    hipError_t e = launch_gemm(stream, x, x_stride, w, 2 * intermediate, cols, tokens, gate_up,
                               2 * intermediate, ws, planes_ready);
    if (e != hipSuccess) return e;
    return launch_swiglu_rows(stream, gate_up, act, intermediate, tokens,
                              act_planes ? ws->planes : nullptr, act_planes);
}

// ---------------------------------------------------------------- row norms
__global__ __launch_bounds__(kThreads) void norm_rows_kernel(const float *x, uint64_t x_stride,
                                                             const uint16_t *w, float offset,
                                                             float *y, uint64_t y_stride,
                                                             uint32_t width) {
    __shared__ float red[4];
    const float *xr = x + blockIdx.x * x_stride;
    float *yr = y + blockIdx.x * y_stride;
    float inv = block_rms_inverse(xr, width, red);
    for (uint32_t i = threadIdx.x; i < width; i += kThreads) {
        float scale = bf16f(w[i]) + offset;
        yr[i] = (xr[i] * inv) * scale;
    }
}


// norm_rows_kernel with the row held in registers, 16-byte accesses (width a
// multiple of 4, at most 8192): every load goes out before the sum, where the
// strided loop above waits on each in turn (C5 verify's first norm 15 us).
// With planes, blocks past `rows` (up to `padded`) write zero planes only.
template <int NV>
__global__ __launch_bounds__(kThreads) void norm_rows4_kernel(const float *x, uint64_t x_stride,
                                                              const uint16_t *w, float offset,
                                                              float *y, uint64_t y_stride,
                                                              uint32_t width, uint16_t *planes,
                                                              uint32_t padded, uint32_t rows) {
    __shared__ float red[4];
    const uint32_t groups = width / 4;
    if (blockIdx.x >= rows) {
        for (uint32_t i = threadIdx.x; i < groups; i += kThreads)
            write_planes4(planes, padded, blockIdx.x, 4 * i, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        return;
    }
    const float *xr = x + blockIdx.x * x_stride;
    float *yr = y + blockIdx.x * y_stride;
    f32x4 v[NV];
    u32x2 g[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = threadIdx.x + kThreads * j;
        const uint32_t c = (i < groups ? i : groups - 1) * 4;
        const f32x4 xv = *(const f32x4 *)(xr + c);
        const u32x2 wv = *(const u32x2 *)(w + c);
        v[j] = i < groups ? xv : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        g[j] = wv;
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float t = v[j][e] * v[j][e];
            ss = ss + t;
        }
    const float inv = block_inverse_from_partial(ss, width, red);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = threadIdx.x + kThreads * j;
        const uint32_t wb[4] = {g[j].x & 0xffffu, g[j].x >> 16, g[j].y & 0xffffu, g[j].y >> 16};
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (v[j][e] * inv) * (bf16f(wb[e]) + offset);
        if (i < groups) {
            *(f32x4 *)(yr + 4 * i) = o;
            if (planes) write_planes4(planes, padded, blockIdx.x, 4 * i, o);
        }
    }
}

hipError_t launch_norm_rows(hipStream_t stream, const float *x, uint64_t x_stride,
                            const uint16_t *w, float offset, float *y, uint64_t y_stride,
                            uint64_t width, uint64_t rows, uint16_t *planes, uint32_t padded) {
    if (!rows) return hipSuccess;
    if (planes && (padded < rows || width % (2 * kSplitBK))) return hipErrorInvalidValue;
    if (width % 4 == 0 && width <= 8192 && x_stride % 4 == 0 && y_stride % 4 == 0 &&
        !((uintptr_t)x & 15) && !((uintptr_t)y & 15) && !((uintptr_t)w & 7)) {
        const uint32_t wd = (uint32_t)width, n = (uint32_t)rows;
        const unsigned grid = planes ? padded : n;
        if (width <= 2048)
            norm_rows4_kernel<2><<<grid, kThreads, 0, stream>>>(x, x_stride, w, offset, y,
                                                                y_stride, wd, planes, padded, n);
        else if (width <= 4096)
            norm_rows4_kernel<4><<<grid, kThreads, 0, stream>>>(x, x_stride, w, offset, y,
                                                                y_stride, wd, planes, padded, n);
        else
            norm_rows4_kernel<8><<<grid, kThreads, 0, stream>>>(x, x_stride, w, offset, y,
                                                                y_stride, wd, planes, padded, n);
        return hipGetLastError();
    }
    norm_rows_kernel<<<(unsigned)rows, kThreads, 0, stream>>>(x, x_stride, w, offset, y, y_stride,
                                                              (uint32_t)width);
    if (planes) {
        const uint64_t elems = (uint64_t)padded * width;
        split_planes_kernel<<<(unsigned)((elems / 8 + 255) / 256), 256, 0, stream>>>(
            y, y_stride, (uint32_t)rows, padded, (uint32_t)width, planes);
    }
    return hipGetLastError();
}

// src/layer.s:33-40 / src/model.s:90-108: state += rms(branch) * (w + offset).
__global__ __launch_bounds__(kThreads) void residual_rows_kernel(float *state, const float *branch,
                                                                 const uint16_t *w, float offset,
                                                                 uint32_t width) {
    __shared__ float red[4];
    const float *b = branch + (uint64_t)blockIdx.x * width;
    float *s = state + (uint64_t)blockIdx.x * width;
    float inv = block_rms_inverse(b, width, red);
    for (uint32_t i = threadIdx.x; i < width; i += kThreads) {
        float scale = bf16f(w[i]) + offset;
        float v = (b[i] * inv) * scale;
        s[i] = s[i] + v;
    }
}

// Residual then the next norm of the same rows, with the row in registers:
// state += rms(branch) * (bf16(wr) + off_r); norm = rms(state) * (bf16(wn) +
// off_n). One block per row; element i of the row lives in thread i % 256.
template <int NE>
__global__ __launch_bounds__(kThreads) void residual_norm_rows_kernel(
    float *state, const float *branch, const uint16_t *wr, float off_r, const uint16_t *wn,
    float off_n, float *norm, uint64_t norm_stride, uint32_t width) {
    __shared__ float red[4];
    const uint64_t row = blockIdx.x;
    float b[NE], st[NE];
    uint16_t gr[NE], gn[NE];
    // Unconditional loads at a clamped index (a guarded load would become a
    // branch with a full wait per element), then a select.
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const uint32_t i = threadIdx.x + kThreads * j;
        const uint32_t c = i < width ? i : width - 1;
        const bool in = i < width;
        const float bv = branch[row * width + c], sv = state[row * width + c];
        const uint16_t rv = wr[c], nv = wn[c];
        b[j] = in ? bv : 0.0f;
        st[j] = in ? sv : 0.0f;
        gr[j] = in ? rv : 0;
        gn[j] = in ? nv : 0;
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const float t = b[j] * b[j];
        ss = ss + t;
    }
    const float inv = block_inverse_from_partial(ss, width, red);
    float ss2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const uint32_t i = threadIdx.x + kThreads * j;
        const float v = (b[j] * inv) * (bf16f(gr[j]) + off_r);
        st[j] = st[j] + v;
        if (i < width) state[row * width + i] = st[j];
        const float t = st[j] * st[j];
        ss2 = ss2 + t;
    }
    const float inv2 = block_inverse_from_partial(ss2, width, red);
#pragma unroll
    for (int j = 0; j < NE; ++j) {
        const uint32_t i = threadIdx.x + kThreads * j;
        if (i < width) norm[row * norm_stride + i] = (st[j] * inv2) * (bf16f(gn[j]) + off_n);
    }
}

// residual_norm_rows_kernel with 16-byte accesses (width a multiple of 4):
// thread i holds elements 4 (i + kThreads j) .. + 3.
template <int NV>
__global__ __launch_bounds__(kThreads) void residual_norm_rows4_kernel(
    float *state, const float *branch, const uint16_t *wr, float off_r, const uint16_t *wn,
    float off_n, float *norm, uint64_t norm_stride, uint32_t width, uint16_t *planes,
    uint32_t padded, uint32_t rows) {
    __shared__ float red[4];
    const uint64_t row = blockIdx.x;
    const uint32_t groups = width / 4;
    if (blockIdx.x >= rows) {  // padding rows of the planes
        for (uint32_t i = threadIdx.x; i < groups; i += kThreads)
            write_planes4(planes, padded, blockIdx.x, 4 * i, f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        return;
    }
    f32x4 b[NV], st[NV];
    u32x2 gr[NV], gn[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t g = threadIdx.x + kThreads * j;
        const uint32_t c = (g < groups ? g : groups - 1) * 4;
        const bool in = g < groups;
        const f32x4 bv = *(const f32x4 *)(branch + row * width + c);
        const f32x4 sv = *(const f32x4 *)(state + row * width + c);
        const u32x2 rv = *(const u32x2 *)(wr + c), nv = *(const u32x2 *)(wn + c);
        const f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        b[j] = in ? bv : z;
        st[j] = in ? sv : z;
        gr[j] = in ? rv : u32x2{0u, 0u};
        gn[j] = in ? nv : u32x2{0u, 0u};
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float t = b[j][e] * b[j][e];
            ss = ss + t;
        }
    const float inv = block_inverse_from_partial(ss, width, red);
    float ss2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t g = threadIdx.x + kThreads * j;
        const uint32_t w[4] = {gr[j].x & 0xffffu, gr[j].x >> 16, gr[j].y & 0xffffu, gr[j].y >> 16};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = (b[j][e] * inv) * (bf16f(w[e]) + off_r);
            st[j][e] = st[j][e] + v;
            const float t = st[j][e] * st[j][e];
            ss2 = ss2 + t;
        }
        if (g < groups) *(f32x4 *)(state + row * width + 4 * g) = st[j];
    }
    const float inv2 = block_inverse_from_partial(ss2, width, red);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t g = threadIdx.x + kThreads * j;
        const uint32_t w[4] = {gn[j].x & 0xffffu, gn[j].x >> 16, gn[j].y & 0xffffu, gn[j].y >> 16};
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (st[j][e] * inv2) * (bf16f(w[e]) + off_n);
        if (g < groups) {
            *(f32x4 *)(norm + row * norm_stride + 4 * g) = o;
            if (planes) write_planes4(planes, padded, blockIdx.x, 4 * g, o);
        }
    }
}

hipError_t launch_residual_norm_rows(hipStream_t stream, float *state, const float *branch,
                                     const uint16_t *wr, float off_r, const uint16_t *wn,
                                     float off_n, float *norm, uint64_t norm_stride,
                                     uint64_t width, uint64_t rows, uint16_t *planes,
                                     uint32_t padded) {
    if (!rows) return hipSuccess;
    if (planes && (padded < rows || width % (2 * kSplitBK))) return hipErrorInvalidValue;
    const uint32_t w = (uint32_t)width;
    if (width % 4 == 0 && norm_stride % 4 == 0 && !((uintptr_t)state & 15) &&
        !((uintptr_t)branch & 15) && !((uintptr_t)norm & 15) && !((uintptr_t)wr & 7) &&
        !((uintptr_t)wn & 7) && width <= 8192) {
        const uint32_t n = (uint32_t)rows;
        const unsigned grid = planes ? padded : n;
        if (width <= 2048)
            residual_norm_rows4_kernel<2><<<grid, kThreads, 0, stream>>>(
                state, branch, wr, off_r, wn, off_n, norm, norm_stride, w, planes, padded, n);
        else if (width <= 4096)
            residual_norm_rows4_kernel<4><<<grid, kThreads, 0, stream>>>(
                state, branch, wr, off_r, wn, off_n, norm, norm_stride, w, planes, padded, n);
        else
            residual_norm_rows4_kernel<8><<<grid, kThreads, 0, stream>>>(
                state, branch, wr, off_r, wn, off_n, norm, norm_stride, w, planes, padded, n);
        return hipGetLastError();
    }
    if (planes) return hipErrorInvalidValue;
    if (width <= 2048)
        residual_norm_rows_kernel<8><<<(unsigned)rows, kThreads, 0, stream>>>(
            state, branch, wr, off_r, wn, off_n, norm, norm_stride, w);
    else if (width <= 4096)
        residual_norm_rows_kernel<16><<<(unsigned)rows, kThreads, 0, stream>>>(
            state, branch, wr, off_r, wn, off_n, norm, norm_stride, w);
    else if (width <= 8192)
        residual_norm_rows_kernel<32><<<(unsigned)rows, kThreads, 0, stream>>>(
            state, branch, wr, off_r, wn, off_n, norm, norm_stride, w);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_residual_rows(hipStream_t stream, float *state, const float *branch,
                                const uint16_t *w, float offset, uint64_t width, uint64_t rows) {
    if (!rows) return hipSuccess;
    residual_rows_kernel<<<(unsigned)rows, kThreads, 0, stream>>>(state, branch, w, offset,
                                                                  (uint32_t)width);
    return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void swiglu_rows_kernel(const float *gate_up, float *out,
                                                               uint64_t intermediate,
                                                               uint64_t total) {
    uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= total) return;
    uint64_t t = e / intermediate, i = e % intermediate;
    const float *row = gate_up + t * 2 * intermediate;
    float g = row[i], u = row[intermediate + i];
    float d = plamo_exp(-g) + 1.0f;
    out[e] = (g / d) * u;
}

// swiglu_rows_kernel straight into the BF16 planes of the down projection's
// matrix-core GEMM (the layout and three-term split of split_planes_kernel),
// four columns per thread; rows past `rows` (up to `padded`) get zero planes.
// The FP32 activation is not written: the GEMM reads the planes only.
__global__ __launch_bounds__(kThreads) void swiglu_planes_kernel(const float *gate_up,
                                                                 uint32_t intermediate,
                                                                 uint32_t rows, uint32_t padded,
                                                                 uint16_t *planes) {
    const uint32_t quads = intermediate / 4;
    const uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= (uint64_t)quads * padded) return;
    const uint32_t t = (uint32_t)(e / quads), c = (uint32_t)(e % quads) * 4;
    f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (t < rows) {
        const float *row = gate_up + (uint64_t)t * 2 * intermediate;
        const f32x4 g = *(const f32x4 *)(row + c), u = *(const f32x4 *)(row + intermediate + c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float d = plamo_exp(-g[i]) + 1.0f;
            v[i] = (g[i] / d) * u[i];
        }
    }
    write_planes4(planes, padded, t, c, v);
}

hipError_t launch_swiglu_rows(hipStream_t stream, const float *gate_up, float *out,
                              uint64_t intermediate, uint64_t rows, uint16_t *planes,
                              uint32_t padded) {
    if (planes) {
        if (intermediate % (2 * kSplitBK) || intermediate >= (1u << 30) || padded < rows ||
            ((uintptr_t)gate_up & 15))
            return hipErrorInvalidValue;
        const uint64_t threads = intermediate / 4 * padded;
        if (!threads) return hipSuccess;
        swiglu_planes_kernel<<<(unsigned)((threads + kThreads - 1) / kThreads), kThreads, 0,
                               stream>>>(gate_up, (uint32_t)intermediate, (uint32_t)rows, padded,
                                         planes);
        return hipGetLastError();
    }
    uint64_t total = intermediate * rows;
    if (!total) return hipSuccess;
    swiglu_rows_kernel<<<(unsigned)((total + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
        gate_up, out, intermediate, total);
    return hipGetLastError();
}

// ---------------------------------------------------------------- QKV post
// src/qkv.s:36-67 (offset-1 head RMSNorm), src/cache.s:8 (append raw K, V),
// src/cache_rope.s:44-75 + tests/rope_reference.s:14-30 (rotate).
__global__ __launch_bounds__(64) void qkv_post_kernel(QkvPost a) {
    const uint32_t h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const uint32_t dim = a.dim, half = dim / 2, width = a.kh * dim;
    const uint32_t stride = (a.qh + 2 * a.kh) * dim;
    const float *x = a.qkv + (uint64_t)t * stride + (uint64_t)h * dim;
    const uint32_t count0 = a.params ? a.params->count[a.layer] : 0;
    uint32_t position = count0 + t;
    if (position > a.capacity - 1) position = a.capacity - 1;
    float s = 0.0f;
    for (uint32_t i = lane; i < dim; i += 64) {
        float v = x[i] * x[i];
        s = s + v;
    }
    s = wave_sum(s);
    float ms = s / (float)dim;
    ms = ms + 0.000001f;
    float inv = 1.0f / __builtin_sqrtf(ms);
    const uint16_t *nw = h < a.qh ? a.qn : a.kn;
    const float *cs = a.table + (uint64_t)position * dim;
    const bool last = t + 1 == a.tokens;
    for (uint32_t j = lane; j < half; j += 64) {
        float sa = bf16f(nw[j]) + 1.0f, sb = bf16f(nw[j + half]) + 1.0f;
        float va = (x[j] * inv) * sa;
        float vb = (x[j + half] * inv) * sb;
        float c = cs[j], sn = cs[half + j];
        float p0 = va * c, p1 = vb * sn;
        float ra = p0 - p1;
        float p2 = vb * c, p3 = va * sn;
        float rb = p2 + p3;
        if (h < a.qh) {
            float *q = a.q_out + (uint64_t)t * a.qh * dim + (uint64_t)h * dim;
            q[j] = ra;
            q[j + half] = rb;
        } else {
            const uint32_t kv = h - a.qh;
            const uint64_t row = (a.rows_from_count ? count0 : 0) + t;
            const uint64_t o = row * width + (uint64_t)kv * dim;
            const float *vsrc = a.qkv + (uint64_t)t * stride + (uint64_t)(a.qh + a.kh + kv) * dim;
            float v0 = vsrc[j], v1 = vsrc[j + half];
            a.k_raw[o + j] = va;
            a.k_raw[o + j + half] = vb;
            a.v[o + j] = v0;
            a.v[o + j + half] = v1;
            if (a.rotate_k) {
                a.k_rot[o + j] = ra;
                a.k_rot[o + j + half] = rb;
            }
            if (a.stage && last) {
                float *st = a.stage + (uint64_t)kv * dim;
                st[j] = va;
                st[j + half] = vb;
                st[width + j] = v0;
                st[width + j + half] = v1;
                st[2 * width + j] = ra;
                st[2 * width + j + half] = rb;
            }
        }
    }
}

hipError_t launch_qkv_post(hipStream_t stream, const QkvPost &a) {
    if (!a.tokens) return hipSuccess;
    qkv_post_kernel<<<dim3(a.qh + a.kh, a.tokens), 64, 0, stream>>>(a);
    return hipGetLastError();
}

// ---------------------------------------------------------------- decode attention
// Decode attention for one KV head group per block, with the reference's
// softmax (tests/attention_reference.s:8-112: scores as FMA chains times
// 1/sqrt(d), the maximum over all rows, exp, sum, weighted value sum).
// Blocks of 8 waves take up to ROWS rows; longer contexts are split across
// blocks whose partials (max, sum, weighted values) the last block of the KV
// head merges.
//
// Phase 0: every load goes out at once, none waiting for the row count: the
// query heads, the new key/value and their norm weights, and the block's
// fixed tile of ROWS cached K and V rows (rows [ROWS * split, ROWS * split + ROWS),
// clamped to the allocation; rows at or past the count are masked once it
// has arrived). The rotation of the step's position is evaluated in FP64 as
// the table's rows are (no table lookup after the count). The query heads are
// normalized and rotated into LDS while the rows are in flight; the last wave
// normalizes, rotates and appends the new row.
// Phase 1: scores. For each pass a wave takes RW rows, 16 lanes per row (each
// lane DIM/16 dims), reduced with DPP; scores go to LDS [row][head].
// Phase 2: per head (one wave each) the maximum, exp in place, and the sum.
// Phase 3: values. Lanes own DIM/64 adjacent columns; each wave accumulates
// its rows' weighted values, the waves are summed in LDS.
constexpr uint32_t kAttnWaves = 8, kAttnThreads = 64 * kAttnWaves;
// Rows per block, one pass per wave: a block loads at most ROWS K and V rows,
// so a context is spread over many CUs (one CU's load path is the limit
// otherwise). Up to kShortAlloc allocated rows, kShortRows per block (more
// blocks in flight for a short context); beyond, kRowsPerBlock (fewer partials
// to merge for a long one).
constexpr uint32_t kRowsPerBlock = 64, kShortRows = 32, kShortAlloc = kDecodeShortRows;

__host__ __device__ constexpr uint32_t attention_rows(uint64_t rows) {
    return rows <= kShortAlloc ? kShortRows : kRowsPerBlock;
}

// One attention block (KV head kvh, row split `split`). With `done`, the block
// that completes a KV head's output writes it through to the coherence point
// and counts the head in *done (the fused O projection waits on it).
template <int DIM, int G, int W, int ROWS, bool OM = false>
__device__ __forceinline__ void attention_block(const DecodeAttention &a, uint32_t kvh,
                                                uint32_t split, uint32_t *done) {
    constexpr uint32_t RW = ROWS / W;  // rows per wave
    constexpr uint32_t P = W * RW;              // rows per pass (one block)
    constexpr int HPW = (G + W - 1) / W;        // query heads per wave
    constexpr int PL = DIM / 64;             // value columns per lane
    constexpr int KD = DIM / 16;             // key dims per lane
    constexpr int KR = RW / 4;               // key rows per lane
    constexpr uint32_t HALF = DIM / 2;
    constexpr uint32_t rec = DIM + 2;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    __shared__ int is_last;
    __shared__ float stats[G][2];  // per head: maximum, sum of exp
    const uint32_t width = a.kh * DIM;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *qs = smem;                            // [G][DIM]
    float *knew = qs + G * DIM;                  // [DIM] rotated new key
    float *vnew = knew + DIM;                    // [DIM]
    float *sc = vnew + DIM;                      // [ROWS + 1][G]
    float *wpart = sc + (ROWS + 1) * G;          // [W][G][DIM]

    // The step's query/key/value heads: wave w normalizes query heads w,
    // w + W, ..., the last wave the new key; lane j < DIM/2 holds elements j
    // and j + DIM/2. Loaded unconditionally (lanes and waves with no use read
    // valid data they ignore) and kept as raw bits until used. They go out
    // first: they do not depend on the row count.
    const bool kwave = wave == W - 1;
    const bool hl = lane < HALF;
    const uint32_t hj = lane % HALF;
    float qx[HPW][2], kx[2], vx[2];
    uint32_t qwb[2], kwb[2];
    auto load_inputs = [&]() {
#pragma unroll
        for (int h = 0; h < HPW; ++h) {
            const uint32_t g = wave + h * W;
            const float *qsrc = a.qkv + (uint64_t)(kvh * G + (g < (uint32_t)G ? g : 0)) * DIM;
            qx[h][0] = qsrc[hj];
            qx[h][1] = qsrc[hj + HALF];
        }
        const float *ksrc = a.qkv + (uint64_t)(a.qh + kvh) * DIM;
        const float *vsrc = a.qkv + (uint64_t)(a.qh + a.kh + kvh) * DIM;
        qwb[0] = a.qn[hj];
        qwb[1] = a.qn[hj + HALF];
        kx[0] = ksrc[hj];
        kx[1] = ksrc[hj + HALF];
        kwb[0] = a.kn[hj];
        kwb[1] = a.kn[hj + HALF];
        vx[0] = vsrc[hj];
        vx[1] = vsrc[hj + HALF];
    };
    load_inputs();
    const float freq = a.freq[hj];

    const uint32_t count = a.params->count[a.layer];
    const uint32_t lo = split * ROWS;
    const uint32_t last_row = a.rows - 1;
    const float *kbase = a.k_rot + (uint64_t)kvh * DIM;
    const float *vbase = a.v + (uint64_t)kvh * DIM;
    const uint32_t kd0 = (lane & 15) * KD, rg = lane >> 4;
    // Tile rows past the allocation read its last row (every address stays in
    // bounds); whatever such rows hold is masked below.
    auto tile_row = [&](uint32_t row) -> uint32_t { return row < last_row ? row : last_row; };
    const uint32_t voff = lane * PL * 4;
    auto load_k = [&](uint32_t base, float (&kr)[KR][KD]) {
#pragma unroll
        for (int j = 0; j < KR; ++j) {
            const uint32_t row = tile_row(base + rg + 4 * j);
            const char *k = (const char *)(kbase + (uint64_t)row * width + kd0);
#pragma unroll
            for (int i = 0; i < KD; i += 4) {
                f32x4 x = *(const f32x4 *)(k + 4 * i);
                kr[j][i] = x.x;
                kr[j][i + 1] = x.y;
                kr[j][i + 2] = x.z;
                kr[j][i + 3] = x.w;
            }
        }
    };
    auto load_v = [&](uint32_t base, float (&vr)[RW][PL]) {
#pragma unroll
        for (int r = 0; r < (int)RW; ++r) {
            const char *vp = (const char *)(vbase + (uint64_t)tile_row(base + r) * width) + voff;
            if (PL == 2) {
                f32x2 x = *(const f32x2 *)vp;
                vr[r][0] = x.x;
                vr[r][PL - 1] = x.y;
            } else {
#pragma unroll
                for (int e = 0; e < PL; ++e) vr[r][e] = ((const float *)vp)[e];
            }
        }
    };
    const uint32_t base0 = lo + wave * RW;
    float kc0[KR][KD], vc0[RW][PL];
    // K before V: the scores need K first and loads return in order.
    __builtin_amdgcn_sched_barrier(0);
    load_k(base0, kc0);
    __builtin_amdgcn_sched_barrier(0);
    load_v(base0, vc0);
    __builtin_amdgcn_sched_barrier(0);

    // The tile's share of rows [0, count] (the appended row, index count, is
    // scored from LDS); tiles past them have nothing to do.
    const uint32_t n = count + 1;
    if (lo >= n) return;
    const uint32_t splits = (n + ROWS - 1) / ROWS;
    const uint32_t hi = lo + ROWS < n ? lo + ROWS : n;
    const bool owner = count >= lo && count < hi;
    const uint32_t hr = hi < count ? hi : count;  // cached rows of this block
    float rc, rs;
    rope_cos_sin(freq, a.rope_scale, (float)count, rc, rs);

    // Offset-1 head RMSNorm then split-half rotation (src/qkv.s:36-67,
    // tests/rope_reference.s:14-30).
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
        const uint32_t g = wave + h * W;
        if (g >= (uint32_t)G) break;
        float ss = hl ? qx[h][0] * qx[h][0] : 0.0f;
        float t = hl ? qx[h][1] * qx[h][1] : 0.0f;
        ss = wave_sum(ss + t);
        float ms = ss / (float)DIM;
        ms = ms + 0.000001f;
        const float inv = 1.0f / __builtin_sqrtf(ms);
        if (hl) {
            float va = (qx[h][0] * inv) * (bf16f(qwb[0]) + 1.0f);
            float vb = (qx[h][1] * inv) * (bf16f(qwb[1]) + 1.0f);
            float p0 = va * rc, p1 = vb * rs, p2 = vb * rc, p3 = va * rs;
            qs[g * DIM + lane] = p0 - p1;
            qs[g * DIM + lane + HALF] = p2 + p3;
        }
    }
    if (kwave && owner) {
        float ss = hl ? kx[0] * kx[0] : 0.0f;
        float t = hl ? kx[1] * kx[1] : 0.0f;
        ss = wave_sum(ss + t);
        float ms = ss / (float)DIM;
        ms = ms + 0.000001f;
        const float inv = 1.0f / __builtin_sqrtf(ms);
        if (hl) {
            const uint64_t o = (uint64_t)count * width + (uint64_t)kvh * DIM;
            float va = (kx[0] * inv) * (bf16f(kwb[0]) + 1.0f);
            float vb = (kx[1] * inv) * (bf16f(kwb[1]) + 1.0f);
            float p0 = va * rc, p1 = vb * rs, p2 = vb * rc, p3 = va * rs;
            float ra = p0 - p1, rb = p2 + p3;
            knew[lane] = ra;
            knew[lane + HALF] = rb;
            vnew[lane] = vx[0];
            vnew[lane + HALF] = vx[1];
            a.k_raw[o + lane] = va;
            a.k_raw[o + lane + HALF] = vb;
            a.k_rot[o + lane] = ra;
            a.k_rot[o + lane + HALF] = rb;
            a.v[o + lane] = vx[0];
            a.v[o + lane + HALF] = vx[1];
            if (a.stage) {
                float *st = a.stage + (uint64_t)kvh * DIM;
                st[lane] = va;
                st[lane + HALF] = vb;
                st[width + lane] = vx[0];
                st[width + lane + HALF] = vx[1];
                st[2 * width + lane] = ra;
                st[2 * width + lane + HALF] = rb;
            }
            if (a.host_k) {
                a.host_k[o + lane] = va;
                a.host_k[o + lane + HALF] = vb;
                a.host_v[o + lane] = vx[0];
                a.host_v[o + lane + HALF] = vx[1];
                a.host_rot[o + lane] = ra;
                a.host_rot[o + lane + HALF] = rb;
            }
        }
    }
    __syncthreads();

    // Phase 1: scores of the cached rows, then of the appended row.
    const float scale = 1.0f / __builtin_sqrtf((float)DIM);
    // All G x KR dot products and their reductions are formed before any is
    // stored: the chains are independent, and a masked store between them
    // would split the code into blocks the scheduler cannot interleave.
    auto score = [&](uint32_t base, const float (&kc)[KR][KD]) {
        float s[G][KR];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float q[KD];
#pragma unroll
            for (int i = 0; i < KD; i += 4) {
                f32x4 x = *(const f32x4 *)(qs + g * DIM + kd0 + i);
                q[i] = x.x;
                q[i + 1] = x.y;
                q[i + 2] = x.z;
                q[i + 3] = x.w;
            }
#pragma unroll
            for (int j = 0; j < KR; ++j) {
                float t = 0.0f;
#pragma unroll
                for (int i = 0; i < KD; ++i) t = __builtin_fmaf(q[i], kc[j][i], t);
                s[g][j] = t;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < KR; ++j) s[g][j] = row_sum16(s[g][j]);
        if ((lane & 15) == 0) {
#pragma unroll
            for (int j = 0; j < KR; ++j) {
                const uint32_t row = base + rg + 4 * j;
                if (row < hr)
#pragma unroll
                    for (int g = 0; g < G; ++g) sc[(row - lo) * G + g] = s[g][j] * scale;
            }
        }
    };
    // The pass runs straight-line and unconditionally (rows past the range are
    // masked): a loop here would merge two load histories and the compiler
    // would then wait for every load in flight. (Blocks never hold more rows
    // than one pass; the loop covers a caller that under-sizes the splits.)
    score(base0, kc0);
    for (uint32_t b = base0 + P; b < hr; b += P) {
        load_k(b, kc0);
        score(b, kc0);
    }
    if (kwave && owner) {
        for (int g = 0; g < G; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < PL; ++e)
                s = __builtin_fmaf(qs[g * DIM + lane * PL + e], knew[lane * PL + e], s);
            s = wave_sum(s);
            if (lane == 0) sc[(count - lo) * G + g] = s * scale;
        }
    }
    __syncthreads();

    // Phase 2: per head, the maximum over the block's rows, exp in place, sum.
    const uint32_t rows = (owner ? count + 1 : hr) - lo;
    for (uint32_t g = wave; g < (uint32_t)G; g += W) {
        float mx = -__builtin_inff();
        for (uint32_t r = lane; r < rows; r += 64) mx = fmaxf(mx, sc[r * G + g]);
        mx = wave_max(mx);
        float sum = 0.0f;
        for (uint32_t r = lane; r < rows; r += 64) {
            const float p = plamo_exp(sc[r * G + g] - mx);
            sc[r * G + g] = p;
            sum += p;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            stats[g][0] = mx;
            stats[g][1] = sum;
        }
    }
    __syncthreads();

    // Phase 3: weighted values.
    float acc[G][PL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < PL; ++e) acc[g][e] = 0.0f;
    auto accumulate = [&](uint32_t base, const float (&vc)[RW][PL]) {
#pragma unroll
        for (int r = 0; r < (int)RW; ++r) {
            const uint32_t row = base + r;
            float pr[G];
            if (G % 4 == 0) {
#pragma unroll
                for (int g = 0; g < G; g += 4) {
                    f32x4 x = *(const f32x4 *)(sc + (row - lo) * G + g);
                    pr[g] = x.x;
                    pr[g + 1] = x.y;
                    pr[g + 2] = x.z;
                    pr[g + 3] = x.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g) pr[g] = sc[(row - lo) * G + g];
            }
            // Rows past the count are selected away (their memory may hold
            // any bits, and 0 * NaN is NaN).
            const bool live = row < hr;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = live ? pr[g] : 0.0f;
#pragma unroll
                for (int e = 0; e < PL; ++e)
                    acc[g][e] = __builtin_fmaf(p, live ? vc[r][e] : 0.0f, acc[g][e]);
            }
        }
    };
    accumulate(base0, vc0);
    for (uint32_t b = base0 + P; b < hr; b += P) {
        load_v(b, vc0);
        accumulate(b, vc0);
    }
    if (kwave && owner) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float p = sc[(count - lo) * G + g];
#pragma unroll
            for (int e = 0; e < PL; ++e)
                acc[g][e] = __builtin_fmaf(p, vnew[lane * PL + e], acc[g][e]);
        }
    }
    // Sum the waves in LDS.
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < PL; ++e) wpart[(wave * G + g) * DIM + lane * PL + e] = acc[g][e];
    __syncthreads();
    if (OM) {
        // Unnormalized partial of this split for the O blocks to merge:
        // values [split][qh][DIM], then (maximum, sum) [split][qh][2].
        float *stats_out = a.partial + (uint64_t)a.splits * a.qh * DIM;
        for (uint32_t i = threadIdx.x; i < G * DIM; i += W * 64) {
            const uint32_t g = i / DIM, d = i % DIM;
            float o = 0.0f;
#pragma unroll
            for (uint32_t w = 0; w < (uint32_t)W; ++w) o = o + wpart[(w * G + g) * DIM + d];
            const uint64_t head = (uint64_t)split * a.qh + kvh * G + g;
            store_through(a.partial + head * DIM + d, o);
            if (d < 2) store_through(stats_out + head * 2 + d, stats[g][d]);
        }
        // `done` is this block's flag here: the step's tag once every store
        // of the partial has completed.
        wait_stores();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_store(done, a.params->step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    for (uint32_t i = threadIdx.x; i < G * DIM; i += W * 64) {
        const uint32_t g = i / DIM, d = i % DIM;
        float o = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < (uint32_t)W; ++w) o = o + wpart[(w * G + g) * DIM + d];
        if (splits == 1) {
            const float r = o / stats[g][1];
            if (done)
                store_through(a.out + (uint64_t)(kvh * G + g) * DIM + d, r);
            else
                a.out[(uint64_t)(kvh * G + g) * DIM + d] = r;
        } else {
            float *bp = a.partial + ((uint64_t)(kvh * a.splits + split) * G + g) * rec;
            if (d == 0) {
                store_through(bp, stats[g][0]);
                store_through(bp + 1, stats[g][1]);
            }
            store_through(bp + 2 + d, o);
        }
    }
    if (splits == 1) {
        if (done) signal_done(done);
        return;
    }
    // The last block of this KV head merges the partials. They were written
    // through by the other blocks before they counted themselves, and no
    // block of this launch has read them before, so plain loads see them (the
    // launch started with invalidated caches); up to kMergeBatch splits are
    // loaded in one round trip.
    if (!arrive_last(&a.counters[kvh], splits, &is_last)) return;
    constexpr uint32_t kMergeBatch = 8;
    for (uint32_t i = threadIdx.x; i < G * DIM; i += W * 64) {
        const uint32_t g = i / DIM, d = i % DIM;
        const float *bp = a.partial + ((uint64_t)kvh * a.splits * G + g) * rec;
        float mx = -__builtin_inff(), sum = 0.0f, o = 0.0f;
        if (splits <= kMergeBatch) {
            float m[kMergeBatch], l[kMergeBatch], v[kMergeBatch];
#pragma unroll
            for (uint32_t sI = 0; sI < kMergeBatch; ++sI) {
                const float *q = bp + (uint64_t)(sI < splits ? sI : 0) * G * rec;
                m[sI] = q[0];
                l[sI] = q[1];
                v[sI] = q[2 + d];
            }
#pragma unroll
            for (uint32_t sI = 0; sI < kMergeBatch; ++sI)
                if (sI < splits) mx = fmaxf(mx, m[sI]);
#pragma unroll
            for (uint32_t sI = 0; sI < kMergeBatch; ++sI) {
                if (sI >= splits) break;
                const float f = plamo_exp(m[sI] - mx);
                sum = __builtin_fmaf(l[sI], f, sum);
                o = __builtin_fmaf(v[sI], f, o);
            }
        } else {
            for (uint32_t sI = 0; sI < splits; ++sI) mx = fmaxf(mx, bp[(uint64_t)sI * G * rec]);
            for (uint32_t sI = 0; sI < splits; ++sI) {
                const float *q = bp + (uint64_t)sI * G * rec;
                const float f = plamo_exp(q[0] - mx);
                sum = __builtin_fmaf(q[1], f, sum);
                o = __builtin_fmaf(q[2 + d], f, o);
            }
        }
        if (done)
            store_through(a.out + (uint64_t)(kvh * G + g) * DIM + d, o / sum);
        else
            a.out[(uint64_t)(kvh * G + g) * DIM + d] = o / sum;
    }
    if (done) signal_done(done);
}

template <int DIM, int G, int ROWS>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(DecodeAttention a) {
    attention_block<DIM, G, kAttnWaves, ROWS>(a, blockIdx.x, blockIdx.y, nullptr);
}

// Attention fused with the output projection (src/mixer.s:60-80: O = W_o .
// attention). Blocks [0, kh * splits) run attention (block b: KV head
// b % kh, split b / kh); the rest compute O rows. An O block streams its
// weight rows into registers first, then waits until every KV head's output
// is counted in `done` (the attention blocks have lower indices, so they are
// dispatched first and never wait), reads the attention output and finishes
// its dot products: the O weights cross HBM while attention runs. The wait is
// bounded; a block that gives up writes NaN rows (they surface as a failed
// argmax) and sets *error.
// O rows per wave of the fused kernel, and the LDS every block of it claims:
// more than half of a CU's 160 KiB, so a CU holds one block. With the KV
// rows allocated in small steps the launch (64 attention blocks at C4 below
// 256 rows plus 128 O blocks) then fits the 256 CUs at once: every O block
// requests its weights at the start, and no O block's 256 KB of weight loads
// shares a CU's load path with an attention block's latency-bound loads.
// (Rows per wave, C4 ms per step: 2: 3.114, 3: 3.089, 4: 3.053, 5: 3.060,
// 6: 3.114.)
// 8192-wide rows (16 chunks) take 2 rows per wave: 4 would hold 256 VGPRs
// of weights per lane.
constexpr int kORows = 4;
constexpr size_t kAttentionOLds = 96 * 1024;
__host__ __device__ constexpr int o_rows_per_wave(int kc) { return kc > 12 ? 2 : kORows; }

// Rows per attention block when the O blocks merge the partials (OM): at
// most kDecodeShortRows / kMergeRows splits per KV head.
constexpr uint32_t kMergeRows = 64, kOMergeSplits = kDecodeShortRows / kMergeRows;

// The attention output for the O blocks of an OM launch: every thread of the
// block merges 8-column segments of the split partials (the merge of
// attention_block: maximum, exp rescale, FMA sums in split order, divide) into
// LDS. Partials were written through and counted before the wait ended, and
// no block of this launch read them earlier, so plain loads see them.
template <int DIM>
__device__ __forceinline__ void merge_partials(const AttentionO &f, uint32_t live, float *xs) {
    const float *vals = f.a.partial;
    const float *stats = f.a.partial + (uint64_t)f.a.splits * f.a.qh * DIM;
    for (uint32_t seg = threadIdx.x; seg < f.cols / 8; seg += kAttnThreads) {
        const uint32_t col = seg * 8, hq = col / DIM, d0 = col % DIM;
        float m[kOMergeSplits], l[kOMergeSplits], v[kOMergeSplits][8];
#pragma unroll
        for (uint32_t sI = 0; sI < kOMergeSplits; ++sI) {
            if (sI >= f.a.splits) break;
            const uint64_t head = (uint64_t)sI * f.a.qh + hq;
            const f32x2 ml = *(const f32x2 *)(stats + head * 2);
            const f32x4 a = *(const f32x4 *)(vals + head * DIM + d0);
            const f32x4 b = *(const f32x4 *)(vals + head * DIM + d0 + 4);
            m[sI] = ml.x;
            l[sI] = ml.y;
            v[sI][0] = a.x; v[sI][1] = a.y; v[sI][2] = a.z; v[sI][3] = a.w;
            v[sI][4] = b.x; v[sI][5] = b.y; v[sI][6] = b.z; v[sI][7] = b.w;
        }
        float out[8];
        if (live == 1) {
#pragma unroll
            for (int e = 0; e < 8; ++e) out[e] = v[0][e] / l[0];
        } else {
            float mx = -__builtin_inff(), sum = 0.0f, o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
            for (uint32_t sI = 0; sI < kOMergeSplits; ++sI)
                if (sI < live) mx = fmaxf(mx, m[sI]);
#pragma unroll
            for (uint32_t sI = 0; sI < kOMergeSplits; ++sI) {
                if (sI >= live) break;
                const float fs = plamo_exp(m[sI] - mx);
                sum = __builtin_fmaf(l[sI], fs, sum);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(v[sI][e], fs, o[e]);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) out[e] = o[e] / sum;
        }
        *(f32x4 *)(xs + col) = f32x4{out[0], out[1], out[2], out[3]};
        *(f32x4 *)(xs + col + 4) = f32x4{out[4], out[5], out[6], out[7]};
    }
    __syncthreads();
}

template <int KC, int DIM = 128, bool OM = false>
__device__ __forceinline__ void oproj_block(const AttentionO &f, uint32_t ob) {
    constexpr int U = o_rows_per_wave(KC);
    __shared__ int waited;
    extern __shared__ __attribute__((aligned(16))) float xs[];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t r0 = (ob * kAttnWaves + wave) * U;
    if (ob * kAttnWaves * U >= f.rows) return;  // block-uniform: the wait below is block-wide
    u32x4 wv[U][KC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t r = min(r0 + u, f.rows - 1);
        const u32x4 *p = (const u32x4 *)(f.w + (uint64_t)r * f.cols + lane * 8);
#pragma unroll
        for (int c = 0; c < KC; ++c) wv[u][c] = __builtin_nontemporal_load(p + c * 64);
    }
    // Zero in the step's parameters means: wait for every KV head, up to
    // 2^22 polls. Other values exist for tests, which raise the target past
    // the heads so that the wait gives up while every block still exits.
    // Every wave holds its weight rows before it reads the step's parameters
    // and joins the wait. Reading them while the weights are in flight (as
    // scalar loads, or as agent-scope vector loads) measured 0.6-0.9 us per
    // C4 layer slower.
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t wait_limit = f.a.params->wait_limit;
    const uint32_t wait_extra = f.a.params->wait_extra;
    const uint32_t step = OM ? f.a.params->step : 0;
    const uint32_t count = OM ? f.a.params->count[f.a.layer] : 0;
    const uint32_t limit = wait_limit ? wait_limit : (1u << 22);
    bool ok;
    if (OM) {
        // The live splits' blocks (the first kh * live of the launch) have
        // published this step's tag; a nonzero wait_extra asks for a tag no
        // block writes.
        const uint32_t live = (count + kMergeRows) / kMergeRows;
        ok = flags_wait(f.flags, f.a.kh * live, step + wait_extra, limit, &waited);
        merge_partials<DIM>(f, live, xs);
    } else {
        ok = block_wait(f.done, f.heads + wait_extra, limit, &waited);
    }
    float acc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) acc[u] = 0.0f;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
        const f32x4 *xp = (const f32x4 *)((OM ? xs : f.x) + c * 512 + lane * 8);
        const f32x4 x0 = xp[0], x1 = xp[1];
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t q[4] = {wv[u][c].x, wv[u][c].y, wv[u][c].z, wv[u][c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[u] = __builtin_fmaf(bf16f(q[e] & 0xffffu), x[2 * e], acc[u]);
                acc[u] = __builtin_fmaf(__uint_as_float(q[e] & 0xffff0000u), x[2 * e + 1], acc[u]);
            }
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const float v = wave_sum(acc[u]);
        if (lane == 0 && r0 + u < f.rows) f.y[r0 + u] = ok ? v : __builtin_nanf("");
    }
    if (!ok && threadIdx.x == 0) atomicOr(f.error, 1u);
}

template <int DIM, int G, int KC, int ROWS, bool OM = false>
__global__ __launch_bounds__(kAttnThreads) void attention_o_kernel(AttentionO f) {
    const uint32_t attention_blocks = f.a.kh * f.a.splits;
    if (blockIdx.x < attention_blocks)
        attention_block<DIM, G, kAttnWaves, ROWS, OM>(f.a, blockIdx.x % f.a.kh,
                                                      blockIdx.x / f.a.kh,
                                                      OM ? f.flags + blockIdx.x : f.done);
    else
        oproj_block<KC, DIM, OM>(f, blockIdx.x - attention_blocks);
}

bool decode_attention_supported(uint32_t dim, uint32_t group) {
    return (dim == 64 || dim == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 6 || group == 8 || group == 16);
}

uint32_t decode_attention_splits(uint64_t rows) {
    const uint32_t per = attention_rows(rows);
    return (uint32_t)((rows + per - 1) / per);
}

static size_t decode_attention_lds(uint32_t dim, uint32_t group, uint32_t rows,
                                   uint32_t waves = kAttnWaves) {
    return (group * dim + 2 * dim + (rows + 1) * group + waves * group * dim) *
           sizeof(float);
}

// Rows per block follow the allocated rows (attention_rows); a.splits is
// decode_attention_splits of the same count.
template <int DIM, int G, int ROWS>
static hipError_t decode_attention_rows(hipStream_t stream, const DecodeAttention &a) {
    size_t lds = decode_attention_lds(DIM, G, ROWS);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)decode_attention_kernel<DIM, G, ROWS>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    decode_attention_kernel<DIM, G, ROWS><<<dim3(a.kh, a.splits), kAttnThreads, lds, stream>>>(a);
    return hipGetLastError();
}

template <int DIM, int G>
static hipError_t decode_attention_variant(hipStream_t stream, const DecodeAttention &a) {
    return attention_rows(a.rows) == kShortRows
               ? decode_attention_rows<DIM, G, kShortRows>(stream, a)
               : decode_attention_rows<DIM, G, kRowsPerBlock>(stream, a);
}

template <int DIM>
static hipError_t decode_attention_dim(hipStream_t stream, const DecodeAttention &a) {
    switch (a.qh / a.kh) {
    case 1: return decode_attention_variant<DIM, 1>(stream, a);
    case 2: return decode_attention_variant<DIM, 2>(stream, a);
    case 4: return decode_attention_variant<DIM, 4>(stream, a);
    case 6: return decode_attention_variant<DIM, 6>(stream, a);
    case 8: return decode_attention_variant<DIM, 8>(stream, a);
    default: return decode_attention_variant<DIM, 16>(stream, a);
    }
}

template <int DIM, int G, int KC, int ROWS, bool OM = false>
static hipError_t attention_o_variant(hipStream_t stream, const AttentionO &f) {
    const size_t lds = std::max(decode_attention_lds(DIM, G, ROWS), kAttentionOLds);
    hipError_t e = hipFuncSetAttribute((const void *)attention_o_kernel<DIM, G, KC, ROWS, OM>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    const uint32_t per_block = o_rows_per_wave(KC) * kAttnWaves;
    const uint32_t oblocks = (f.rows + per_block - 1) / per_block;
    attention_o_kernel<DIM, G, KC, ROWS, OM>
        <<<f.a.kh * f.a.splits + oblocks, kAttnThreads, lds, stream>>>(f);
    return hipGetLastError();
}

// Up to kDecodeShortRows allocated rows the O blocks merge the partials of
// kMergeRows-row attention blocks (no merging attention block, no second
// hand-off); beyond, the last attention block of each KV head merges them.
template <int DIM, int G, int KC>
static hipError_t attention_o_rows(hipStream_t stream, const AttentionO &f) {
    if (f.a.rows <= kDecodeShortRows && f.flags &&
        f.a.kh * ((f.a.rows + kMergeRows - 1) / kMergeRows) <= kAttentionFlags) {
        AttentionO m = f;
        m.a.splits = (f.a.rows + kMergeRows - 1) / kMergeRows;
        return attention_o_variant<DIM, G, KC, kMergeRows, true>(stream, m);
    }
    return attention_o_variant<DIM, G, KC, kRowsPerBlock>(stream, f);
}

template <int DIM, int G>
static hipError_t attention_o_cols(hipStream_t stream, const AttentionO &f) {
    switch (f.cols / 512) {
    case 4: return attention_o_rows<DIM, G, 4>(stream, f);
    case 6: return attention_o_rows<DIM, G, 6>(stream, f);
    case 8: return attention_o_rows<DIM, G, 8>(stream, f);
    case 12: return attention_o_rows<DIM, G, 12>(stream, f);
    default: return attention_o_rows<DIM, G, 16>(stream, f);
    }
}

template <int DIM>
static hipError_t attention_o_dim(hipStream_t stream, const AttentionO &f) {
    switch (f.a.qh / f.a.kh) {
    case 1: return attention_o_cols<DIM, 1>(stream, f);
    case 2: return attention_o_cols<DIM, 2>(stream, f);
    case 4: return attention_o_cols<DIM, 4>(stream, f);
    case 6: return attention_o_cols<DIM, 6>(stream, f);
    case 8: return attention_o_cols<DIM, 8>(stream, f);
    default: return attention_o_cols<DIM, 16>(stream, f);
    }
}

bool attention_o_supported(uint32_t dim, uint32_t group, uint64_t cols) {
    return decode_attention_supported(dim, group) &&
           (cols == 2048 || cols == 3072 || cols == 4096 || cols == 6144 || cols == 8192);
}

hipError_t launch_attention_o(hipStream_t stream, const AttentionO &f) {
    if (!attention_o_supported(f.a.dim, f.a.qh / f.a.kh, f.cols) || f.cols != f.a.qh * f.a.dim ||
        f.a.splits < 1 || f.a.splits > 65535 || !f.done || !f.error || f.heads != f.a.kh ||
        ((uintptr_t)f.w & 15) || ((uintptr_t)f.x & 15))
        return hipErrorInvalidValue;
    return f.a.dim == 64 ? attention_o_dim<64>(stream, f) : attention_o_dim<128>(stream, f);
}

hipError_t launch_decode_attention(hipStream_t stream, const DecodeAttention &a) {
    if (!decode_attention_supported(a.dim, a.qh / a.kh) || a.splits < 1 || a.splits > 65535)
        return hipErrorInvalidValue;
    return a.dim == 64 ? decode_attention_dim<64>(stream, a) : decode_attention_dim<128>(stream, a);
}

// ---------------------------------------------------------------- prompt attention
// Causal attention for a block of up to 16 queries of one head, online softmax
// over key tiles of 32 rows. Without a window the keys are the materialized
// rotated rows; with a window (sliding cache overflow) each key is rotated at
// its position inside the query's window, as the CPU path does after every
// shift (src/cache_rope.s:15-27 rotates all rows at local positions).
constexpr int kQT = 16, kKT = 32;
__global__ __launch_bounds__(kThreads) void prompt_attention_kernel(PromptAttention a,
                                                                    uint32_t split_rows) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const uint32_t dim = a.dim, half = dim / 2, width = a.kh * dim;
    float *qs = smem;                    // [kQT][dim]
    float *ks = qs + kQT * dim;          // [kKT][dim + 1]
    float *vs = ks + kKT * (dim + 1);    // [kKT][dim]
    float *ps = vs + kKT * dim;          // [kQT][kKT]
    float *corr = ps + kQT * kKT;        // [kQT]
    float *mrow = corr + kQT;            // [kQT]
    float *lrow = mrow + kQT;            // [kQT]
    const uint32_t h = blockIdx.x, kvh = h / (a.qh / a.kh);
    const uint32_t t0 = blockIdx.y * kQT;
    const uint32_t nq = a.tokens - t0 < (uint32_t)kQT ? a.tokens - t0 : kQT;
    // Staging loads are unconditional at clamped indices, eight per thread in
    // flight, then selected: a guarded load would wait for each element.
    for (uint32_t base = threadIdx.x; base < kQT * dim; base += 8 * kThreads) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t i = min(base + j * kThreads, kQT * dim - 1);
            const uint32_t q = min(i / dim, nq - 1), d = i % dim;
            v[j] = a.q[(uint64_t)(t0 + q) * a.qh * dim + (uint64_t)h * dim + d];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t i = base + j * kThreads;
            if (i < kQT * dim) qs[i] = i / dim < nq ? v[j] : 0.0f;
        }
    }
    if (threadIdx.x < kQT) {
        mrow[threadIdx.x] = -__builtin_inff();
        lrow[threadIdx.x] = 0.0f;
    }
    // Key range of the block: virtual rows [lo_min, hi_max), cut to its split
    // [z * split_rows, (z + 1) * split_rows) when keys are split.
    uint32_t hi_max = a.prefix + t0 + nq;
    uint32_t lo_min = 0;
    if (a.window && a.prefix + t0 + 1 > a.window) lo_min = a.prefix + t0 + 1 - a.window;
    if (split_rows) {
        lo_min = max(lo_min, blockIdx.z * split_rows);
        hi_max = min(hi_max, (blockIdx.z + 1) * split_rows);
    }
    const float scale = 1.0f / __builtin_sqrtf((float)dim);
    // Output ownership: thread -> query tid/16, dims (tid%16) + 16*i.
    const uint32_t oq = threadIdx.x / 16, od = threadIdx.x % 16;
    float o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = 0.0f;
    __syncthreads();
    for (uint32_t k0 = lo_min; k0 < hi_max; k0 += kKT) {
        const uint32_t nk = hi_max - k0 < (uint32_t)kKT ? hi_max - k0 : kKT;
        for (uint32_t base = threadIdx.x; base < kKT * dim; base += 8 * kThreads) {
            float kv8[8], vv8[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = min(base + j * kThreads, kKT * dim - 1);
                const uint32_t r = min(i / dim, nk - 1), d = i % dim;
                const uint32_t vrow = k0 + r;
                const float *kp = vrow < a.prefix ? a.k_cache + (uint64_t)vrow * width
                                                  : a.k_new + (uint64_t)(vrow - a.prefix) * width;
                const float *vp = vrow < a.prefix ? a.v_cache + (uint64_t)vrow * width
                                                  : a.v_new + (uint64_t)(vrow - a.prefix) * width;
                kv8[j] = kp[(uint64_t)kvh * dim + d];
                vv8[j] = vp[(uint64_t)kvh * dim + d];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t i = base + j * kThreads;
                if (i >= kKT * dim) continue;
                const uint32_t r = i / dim, d = i % dim;
                ks[r * (dim + 1) + d] = r < nk ? kv8[j] : 0.0f;
                vs[r * dim + d] = r < nk ? vv8[j] : 0.0f;
            }
        }
        __syncthreads();
        // Scores: thread -> query tid/16, keys tid%16 and tid%16 + 16.
        {
            const uint32_t q = threadIdx.x / 16;
            const uint32_t t = t0 + q;
            const uint32_t hi = a.prefix + t + 1;
            uint32_t lo = 0;
            if (a.window && hi > a.window) lo = hi - a.window;
            float sv[2];
            float tile_max = -__builtin_inff();
            for (int e = 0; e < 2; ++e) {
                uint32_t kr = threadIdx.x % 16 + 16 * e, vrow = k0 + kr;
                float s = -__builtin_inff();
                if (q < nq && kr < nk && vrow >= lo && vrow < hi) {
                    const float *qv = qs + q * dim;
                    const float *kv = ks + kr * (dim + 1);
                    float acc = 0.0f;
                    if (a.window) {
                        const float *cs = a.table + (uint64_t)(vrow - lo) * dim;
                        for (uint32_t j = 0; j < half; ++j) {
                            float x0 = kv[j], x1 = kv[j + half], c = cs[j], sn = cs[half + j];
                            float p0 = x0 * c, p1 = x1 * sn;
                            float r0 = p0 - p1;
                            acc = __builtin_fmaf(qv[j], r0, acc);
                        }
                        for (uint32_t j = 0; j < half; ++j) {
                            float x0 = kv[j], x1 = kv[j + half], c = cs[j], sn = cs[half + j];
                            float p2 = x1 * c, p3 = x0 * sn;
                            float r1 = p2 + p3;
                            acc = __builtin_fmaf(qv[j + half], r1, acc);
                        }
                    } else {
                        for (uint32_t j = 0; j < dim; ++j) acc = __builtin_fmaf(qv[j], kv[j], acc);
                    }
                    s = acc * scale;
                }
                sv[e] = s;
                tile_max = fmaxf(tile_max, s);
            }
            // Reduce over the 16 lanes of this query.
            for (int off = 8; off > 0; off >>= 1) tile_max = fmaxf(tile_max, __shfl_xor(tile_max, off, 16));
            float m_old = mrow[q];
            float m_new = fmaxf(m_old, tile_max);
            float c = 1.0f, psum = 0.0f;
            for (int e = 0; e < 2; ++e) {
                float p = 0.0f;
                if (m_new != -__builtin_inff() && sv[e] != -__builtin_inff()) p = plamo_exp(sv[e] - m_new);
                ps[q * kKT + threadIdx.x % 16 + 16 * e] = p;
                psum += p;
            }
            for (int off = 8; off > 0; off >>= 1) psum += __shfl_xor(psum, off, 16);
            if (m_new != -__builtin_inff()) c = plamo_exp(m_old - m_new);
            __syncthreads();
            if (threadIdx.x % 16 == 0) {
                corr[q] = c;
                mrow[q] = m_new;
                lrow[q] = lrow[q] * c + psum;
            }
        }
        __syncthreads();
        {
            const float c = corr[oq];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                uint32_t d = i * 16 + od;
                if (d < dim) {
                    float acc = o[i] * c;
                    for (uint32_t kr = 0; kr < nk; ++kr)
                        acc = __builtin_fmaf(ps[oq * kKT + kr], vs[kr * dim + d], acc);
                    o[i] = acc;
                }
            }
        }
        __syncthreads();
    }
    if (oq < nq) {
        if (split_rows) {
            // Record [split][token][head]: unnormalized output, running max, sum.
            float *rec = a.partial +
                         (((uint64_t)blockIdx.z * a.tokens + t0 + oq) * a.qh + h) * (dim + 2);
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (i * 16 + od < dim) rec[i * 16 + od] = o[i];
            if (od == 0) {
                rec[dim] = mrow[oq];
                rec[dim + 1] = lrow[oq];
            }
            return;
        }
        float l = lrow[oq];
        float *out = a.out + (uint64_t)(t0 + oq) * a.qh * dim + (uint64_t)h * dim;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (i * 16 + od < dim) out[i * 16 + od] = o[i] / l;
    }
}

// One wave per (token, head), four per block. Lane z loads split z's maximum
// and sum, and the factors exp(m_z - m) go to the wave's LDS slots; then the
// sum of weights and each output column are accumulated over the splits in
// split order, skipping splits that saw no key (maximum -inf), as a plain
// sequential loop over the records would. With `planes`, each output value
// is written as its three BF16 terms for the O projection's GEMM instead.
constexpr uint32_t kMergeSplits = 64;
__global__ __launch_bounds__(256) void attention_merge_kernel(const float *partial,
                                                              uint32_t splits, uint64_t stride,
                                                              uint32_t dim, float *out,
                                                              uint32_t qh, uint32_t pairs,
                                                              uint16_t *planes, uint32_t padded) {
    __shared__ float fz_s[4][kMergeSplits], lz_s[4][kMergeSplits];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t pair = blockIdx.x * 4 + wave;  // token * qh + head
    if (pair >= pairs) return;  // per wave; the kernel has no block barrier
    float *fz = fz_s[wave], *lz = lz_s[wave];
    const float *p = partial + (uint64_t)pair * (dim + 2);
    const bool in = lane < splits;
    const float mz = in ? p[lane * stride + dim] : -__builtin_inff();
    const float sz = in ? p[lane * stride + dim + 1] : 0.0f;
    const float m = wave_max(mz);
    const bool on = mz != -__builtin_inff();
    const uint64_t live = __ballot(on);
    fz[lane] = on ? plamo_exp(mz - m) : 0.0f;
    lz[lane] = sz;
    // The wave's own LDS writes are seen by its later reads (in order).
    __builtin_amdgcn_wave_barrier();
    float l = 0.0f;
    for (uint32_t z = 0; z < splits; ++z)
        if (live >> z & 1) l += lz[z] * fz[z];
    for (uint32_t d = lane; d < dim; d += 64) {
        float acc = 0.0f;
        uint32_t z = 0;
        for (; z + 8 <= splits; z += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = p[(z + j) * stride + d];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (live >> (z + j) & 1) acc += v[j] * fz[z + j];
        }
        for (; z < splits; ++z)
            if (live >> z & 1) acc += p[z * stride + d] * fz[z];
        const float o = acc / l;
        if (planes)
            write_planes1(planes, padded, pair / qh, pair % qh * dim + d, o);
        else
            out[(uint64_t)pair * dim + d] = o;
    }
}

// Key splits: only when the query tiles alone leave the GPU mostly idle (a
// few candidate or prompt tokens over a long prefix): about four blocks per
// CU of one key tile each, at most 64 splits, within the scratch bound.
constexpr uint64_t kAttentionScratchFloats = 8ull << 20;
static uint32_t prompt_attention_splits(uint32_t prefix, uint32_t tokens, uint32_t qh,
                                        uint32_t dim, uint32_t *split_rows) {
    const uint32_t tiles = (tokens + kQT - 1) / kQT, keys = prefix + tokens;
    const uint32_t blocks = qh * tiles;
    *split_rows = 0;
    if (blocks >= 256 || keys <= 2 * kKT) return 1;
    uint32_t splits = (1024 + blocks - 1) / blocks;
    splits = min(splits, min(64u, (keys + kKT - 1) / kKT));
    while (splits > 1 && (uint64_t)splits * tokens * qh * (dim + 2) > kAttentionScratchFloats)
        --splits;
    if (splits <= 1) return 1;
    uint32_t rows = (keys + splits - 1) / splits;
    rows = (rows + kKT - 1) / kKT * kKT;
    *split_rows = rows;
    return (keys + rows - 1) / rows;
}


// ---------------------------------------------------------------- prompt attention on matrix cores
// The same causal attention without a sliding window, with Q K^T and P V on
// the FP32 matrix cores (v_mfma_f32_16x16x4_f32: FP32 operands, products and
// sums in FP32; only the summation order differs from the scalar form, as
// it already does there). Block: KV head blockIdx.x, query tokens
// [16 * blockIdx.y, + 16), key split blockIdx.z; wave g is query head
// kvh * G + g, so the G heads of a group share every staged key and value
// tile. Per tile of 32 keys a wave forms S = Q K^T for its 16 tokens (Q held
// in registers as the A operand, K read from LDS as B), masks what the token
// may not see, updates its running maximum and sum row by row (a token's
// scores sit in one 16-lane row of the D layout: DPP row reductions), writes
// P to LDS and reads it back in the A layout for O += P V.
// D layout: lane l holds rows 4 * (l / 16) + v (v = 0..3) of column l % 16.
constexpr int kMQ = 16, kMK = 32;
template <int DIM>
constexpr size_t prompt_mfma_lds(int g) {
    return ((size_t)kMK * (DIM + 2) + (size_t)kMK * (DIM + 16) + (size_t)g * kMQ * (kMK + 2)) *
           sizeof(float);
}

template <int DIM, int G>
__global__ __launch_bounds__(64 * G) void prompt_attention_mfma_kernel(PromptAttention a,
                                                                       uint32_t split_rows) {
    constexpr int KS = DIM + 2;   // K row stride: B reads hit 32 distinct banks
    constexpr int VS = DIM + 16;  // V row stride: the two 16-lane halves use opposite banks
    constexpr int PS = kMK + 2;   // P row stride
    constexpr int NT = DIM / 16;  // output column tiles of 16
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *ks = smem;          // [kMK][KS]
    float *vs = ks + kMK * KS; // [kMK][VS]
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float *ps = vs + kMK * VS + wave * kMQ * PS;  // [kMQ][PS] of this wave
    const uint32_t kvh = blockIdx.x, h = kvh * G + wave;
    const uint32_t width = a.kh * DIM;
    const uint32_t t0 = blockIdx.y * kMQ;
    const uint32_t nq = a.tokens - t0 < (uint32_t)kMQ ? a.tokens - t0 : kMQ;
    const uint32_t col = lane & 15, grp = lane >> 4;
    // A operand of Q K^T: q[k4] = Q[token t0 + col][4 * k4 + grp] (token rows
    // past the prompt repeat its last token; their results are dropped).
    float q[DIM / 4];
    {
        const float *qrow = a.q + (uint64_t)(t0 + (col < nq ? col : nq - 1)) * a.qh * DIM +
                            (uint64_t)h * DIM + grp;
#pragma unroll
        for (int k4 = 0; k4 < DIM / 4; ++k4) q[k4] = qrow[4 * k4];
    }
    uint32_t hi_max = a.prefix + t0 + nq, lo_min = 0;
    if (split_rows) {
        lo_min = blockIdx.z * split_rows;
        hi_max = hi_max < lo_min + split_rows ? hi_max : lo_min + split_rows;
    }
    const float scale = 1.0f / __builtin_sqrtf((float)DIM);
    const float ninf = -__builtin_inff();
    f32x4 o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) o[n] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[4], l_run[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        m_run[v] = ninf;
        l_run[v] = 0.0f;
    }
    for (uint32_t k0 = lo_min; k0 < hi_max; k0 += kMK) {
        const uint32_t nk = hi_max - k0 < (uint32_t)kMK ? hi_max - k0 : kMK;
        __syncthreads();  // the previous tile's K, V and P reads are done
        // The tile's K and V rows, up to four 16-byte pieces of each per
        // thread in flight before any is stored (one round trip per round).
        constexpr uint32_t kPieces = kMK * (DIM / 4), kStride = 64 * G;
        constexpr uint32_t kPer = (kPieces + kStride - 1) / kStride, kRound = kPer < 4 ? kPer : 4;
        for (uint32_t base = 0; base < kPer; base += kRound) {
            f32x4 kv[kRound], vv[kRound];
#pragma unroll
            for (uint32_t j = 0; j < kRound; ++j) {
                const uint32_t i = threadIdx.x + (base + j) * kStride;
                const uint32_t r = i / (DIM / 4), c = (i % (DIM / 4)) * 4;
                const uint32_t vrow = k0 + (r < nk ? r : nk - 1);
                const float *kp = vrow < a.prefix ? a.k_cache + (uint64_t)vrow * width
                                                  : a.k_new + (uint64_t)(vrow - a.prefix) * width;
                const float *vp = vrow < a.prefix ? a.v_cache + (uint64_t)vrow * width
                                                  : a.v_new + (uint64_t)(vrow - a.prefix) * width;
                if (i < kPieces) {
                    kv[j] = *(const f32x4 *)(kp + (uint64_t)kvh * DIM + c);
                    vv[j] = *(const f32x4 *)(vp + (uint64_t)kvh * DIM + c);
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < kRound; ++j) {
                const uint32_t i = threadIdx.x + (base + j) * kStride;
                if (i >= kPieces) continue;
                const uint32_t r = i / (DIM / 4), c = (i % (DIM / 4)) * 4;
                f32x4 k = kv[j], v = vv[j];
                if (r >= nk) k = v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                float *kd = ks + r * KS + c;
                kd[0] = k.x; kd[1] = k.y; kd[2] = k.z; kd[3] = k.w;
                *(f32x4 *)(vs + r * VS + c) = v;
            }
        }
        __syncthreads();
        // S for keys k0 + col and k0 + 16 + col.
        f32x4 s0 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
        for (int k4 = 0; k4 < DIM / 4; ++k4) {
            const float b0 = ks[col * KS + 4 * k4 + grp];
            const float b1 = ks[(16 + col) * KS + 4 * k4 + grp];
            s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(q[k4], b0, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(q[k4], b1, s1, 0, 0, 0);
        }
        float corr[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const uint32_t row = 4 * grp + v;
            const uint32_t visible = a.prefix + t0 + row + 1;  // keys of token t0 + row
            const uint32_t r0 = k0 + col, r1 = k0 + 16 + col;
            const bool live = row < nq;
            const float x0 = live && col < nk && r0 < visible ? s0[v] * scale : ninf;
            const float x1 = live && 16 + col < nk && r1 < visible ? s1[v] * scale : ninf;
            const float m_new = fmaxf(m_run[v], row_max16(fmaxf(x0, x1)));
            const float p0 = m_new == ninf || x0 == ninf ? 0.0f : plamo_exp(x0 - m_new);
            const float p1 = m_new == ninf || x1 == ninf ? 0.0f : plamo_exp(x1 - m_new);
            const float c = m_new == ninf ? 1.0f : plamo_exp(m_run[v] - m_new);
            l_run[v] = l_run[v] * c + row_sum16(p0 + p1);
            m_run[v] = m_new;
            corr[v] = c;
            ps[row * PS + col] = p0;
            ps[row * PS + 16 + col] = p1;
        }
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int v = 0; v < 4; ++v) o[n][v] = o[n][v] * corr[v];
        __syncthreads();  // P of every wave is in LDS
        // O += P V: A = P[token col][key 4 k4 + grp], B = V[key 4 k4 + grp][16 n + col].
#pragma unroll
        for (int k4 = 0; k4 < kMK / 4; ++k4) {
            const float pa = ps[col * PS + 4 * k4 + grp];
            const float *vrow = vs + (4 * k4 + grp) * VS + col;
#pragma unroll
            for (int n = 0; n < NT; ++n)
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vrow[16 * n], o[n], 0, 0, 0);
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const uint32_t row = 4 * grp + v;
        if (row >= nq) continue;  // uniform over each 16-lane row of the D layout
        const uint32_t t = t0 + row;
        if (split_rows) {
            // Record [split][token][head]: unnormalized output, running max, sum.
            float *rec = a.partial + (((uint64_t)blockIdx.z * a.tokens + t) * a.qh + h) * (DIM + 2);
#pragma unroll
            for (int n = 0; n < NT; ++n) rec[16 * n + col] = o[n][v];
            if (col == 0) {
                rec[DIM] = m_run[v];
                rec[DIM + 1] = l_run[v];
            }
        } else {
            float *out = a.out + (uint64_t)t * a.qh * DIM + (uint64_t)h * DIM;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const float y = o[n][v] / l_run[v];
                if (!a.planes) {
                    out[16 * n + col] = y;
                } else {
                    // Lanes 4j .. 4j + 3 hold four adjacent columns: the
                    // first writes them as one group of planes.
                    const float y1 = __shfl_down(y, 1, 4), y2 = __shfl_down(y, 2, 4),
                                y3 = __shfl_down(y, 3, 4);
                    if (col % 4 == 0)
                        write_planes4(a.planes, a.padded, t, h * DIM + 16 * n + col,
                                      f32x4{y, y1, y2, y3});
                }
            }
        }
    }
}

static bool prompt_mfma_supported(uint32_t dim, uint32_t qh, uint32_t kh, uint32_t window) {
    if (window || !kh || qh % kh || (dim != 64 && dim != 128)) return false;
    const uint32_t g = qh / kh;
    return g == 1 || g == 2 || g == 4 || g == 6 || g == 8 || g == 16;
}

// Key splits of the matrix-core form, toward about 512 blocks, while its
// blocks (one per KV head and 16 tokens) number fewer: a causal prompt's
// last query tiles see every key, and without splits their blocks alone set
// the launch's length (C4, 443 tokens after a 12-token prefix: 224 blocks,
// 75-80 us per layer; three splits 45.8 us plus a 12 us merge).
static uint32_t prompt_mfma_splits(uint32_t prefix, uint32_t tokens, uint32_t qh, uint32_t kh,
                                   uint32_t dim, uint32_t *split_rows) {
    const uint32_t tiles = (tokens + kMQ - 1) / kMQ, keys = prefix + tokens;
    const uint32_t blocks = kh * tiles;
    *split_rows = 0;
    if (blocks >= 512 || keys <= 2 * kMK) return 1;
    uint32_t splits = (512 + blocks - 1) / blocks;
    splits = min(splits, min(64u, (keys + kMK - 1) / kMK));
    while (splits > 1 && (uint64_t)splits * tokens * qh * (dim + 2) > kAttentionScratchFloats)
        --splits;
    if (splits <= 1) return 1;
    uint32_t rows = (keys + splits - 1) / splits;
    rows = (rows + kMK - 1) / kMK * kMK;
    *split_rows = rows;
    return (keys + rows - 1) / rows;
}

template <int DIM, int G>
static hipError_t prompt_mfma_variant(hipStream_t stream, const PromptAttention &a, uint32_t splits,
                                      uint32_t rows) {
    dim3 grid(a.kh, (a.tokens + kMQ - 1) / kMQ, splits);
    prompt_attention_mfma_kernel<DIM, G>
        <<<grid, 64 * G, prompt_mfma_lds<DIM>(G), stream>>>(a, splits > 1 ? rows : 0);
    return hipGetLastError();
}

template <int DIM>
static hipError_t prompt_mfma_dim(hipStream_t stream, const PromptAttention &a, uint32_t splits,
                                  uint32_t rows) {
    switch (a.qh / a.kh) {
    case 1: return prompt_mfma_variant<DIM, 1>(stream, a, splits, rows);
    case 2: return prompt_mfma_variant<DIM, 2>(stream, a, splits, rows);
    case 4: return prompt_mfma_variant<DIM, 4>(stream, a, splits, rows);
    case 6: return prompt_mfma_variant<DIM, 6>(stream, a, splits, rows);
    case 8: return prompt_mfma_variant<DIM, 8>(stream, a, splits, rows);
    default: return prompt_mfma_variant<DIM, 16>(stream, a, splits, rows);
    }
}

uint64_t prompt_attention_scratch(uint32_t prefix, uint32_t tokens, uint32_t qh, uint32_t kh,
                                  uint32_t dim, uint32_t window) {
    uint32_t rows;
    const uint32_t splits = prompt_mfma_supported(dim, qh, kh, window)
                                ? prompt_mfma_splits(prefix, tokens, qh, kh, dim, &rows)
                                : prompt_attention_splits(prefix, tokens, qh, dim, &rows);
    return splits > 1 ? (uint64_t)splits * tokens * qh * (dim + 2) : 0;
}

bool prompt_attention_writes_planes(uint32_t dim, uint32_t qh, uint32_t kh, uint32_t window) {
    return prompt_mfma_supported(dim, qh, kh, window);
}

hipError_t launch_prompt_attention(hipStream_t stream, const PromptAttention &a) {
    if (!a.tokens) return hipSuccess;
    // Planes come from the matrix-core form only; the scalar form refuses
    // them rather than leave them unwritten.
    if (a.planes && (!prompt_mfma_supported(a.dim, a.qh, a.kh, a.window) || a.padded < a.tokens ||
                     (a.qh * a.dim) % (2 * kSplitBK)))
        return hipErrorInvalidValue;
    uint32_t rows = 0, splits = 1;
    hipError_t e;
    if (prompt_mfma_supported(a.dim, a.qh, a.kh, a.window)) {
        if (a.partial) splits = prompt_mfma_splits(a.prefix, a.tokens, a.qh, a.kh, a.dim, &rows);
        e = a.dim == 64 ? prompt_mfma_dim<64>(stream, a, splits, rows)
                        : prompt_mfma_dim<128>(stream, a, splits, rows);
    } else {
        size_t lds = (kQT * a.dim + kKT * (a.dim + 1) + kKT * a.dim + kQT * kKT + 3 * kQT) * sizeof(float);
        if (a.partial) splits = prompt_attention_splits(a.prefix, a.tokens, a.qh, a.dim, &rows);
        dim3 grid(a.qh, (a.tokens + kQT - 1) / kQT, splits);
        prompt_attention_kernel<<<grid, kThreads, lds, stream>>>(a, splits > 1 ? rows : 0);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    if (splits > 1)
        attention_merge_kernel<<<(a.tokens * a.qh + 3) / 4, 256, 0, stream>>>(
            a.partial, splits, (uint64_t)a.tokens * a.qh * (a.dim + 2), a.dim, a.out, a.qh,
            a.tokens * a.qh, a.planes, a.padded);
    return hipGetLastError();
}

// ---------------------------------------------------------------- rotation maintenance
__global__ __launch_bounds__(kThreads) void rerotate_kernel(const float *k_raw, float *k_rot,
                                                            const float *table, uint64_t rows,
                                                            uint32_t kh, uint32_t dim) {
    const uint32_t half = dim / 2;
    uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    uint64_t per_row = (uint64_t)kh * half;
    if (e >= rows * per_row) return;
    uint64_t row = e / per_row;
    uint32_t head = (uint32_t)((e % per_row) / half), j = (uint32_t)(e % half);
    uint64_t o = row * kh * dim + (uint64_t)head * dim;
    float x0 = k_raw[o + j], x1 = k_raw[o + j + half];
    const float *cs = table + row * dim;
    float c = cs[j], s = cs[half + j];
    float p0 = x0 * c, p1 = x1 * s;
    float p2 = x1 * c, p3 = x0 * s;
    k_rot[o + j] = p0 - p1;
    k_rot[o + j + half] = p2 + p3;
}

hipError_t launch_rerotate(hipStream_t stream, const float *k_raw, float *k_rot,
                           const float *table, uint64_t rows, uint32_t kh, uint32_t dim) {
    uint64_t n = rows * kh * (dim / 2);
    if (!n) return hipSuccess;
    rerotate_kernel<<<(unsigned)((n + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
        k_raw, k_rot, table, rows, kh, dim);
    return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void window_gather_kernel(const float *k_raw, const float *v,
                                                                 const float *new_k,
                                                                 const float *new_v,
                                                                 uint64_t new_stride,
                                                                 float *scratch, uint64_t prefix,
                                                                 uint64_t first, uint64_t keep,
                                                                 uint32_t width) {
    uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (e >= keep * width) return;
    uint64_t i = e / width, c = e % width, vrow = first + i;
    float kv, vv;
    if (vrow < prefix) {
        kv = k_raw[vrow * width + c];
        vv = v[vrow * width + c];
    } else {
        kv = new_k[(vrow - prefix) * new_stride + c];
        vv = new_v[(vrow - prefix) * new_stride + c];
    }
    scratch[e] = kv;
    scratch[keep * width + e] = vv;
}

hipError_t launch_window_store(hipStream_t stream, float *k_raw, float *v, float *k_rot,
                               const float *new_k, const float *new_v, uint64_t new_stride,
                               const float *table, float *scratch, uint64_t prefix,
                               uint64_t tokens, uint64_t keep, uint32_t kh, uint32_t dim) {
    uint32_t width = kh * dim;
    uint64_t n = keep * width;
    if (!n) return hipSuccess;
    uint64_t first = prefix + tokens - keep;
    unsigned blocks = (unsigned)((n + kThreads - 1) / kThreads);
    window_gather_kernel<<<blocks, kThreads, 0, stream>>>(k_raw, v, new_k, new_v, new_stride,
                                                          scratch, prefix, first, keep, width);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(k_raw, scratch, n * 4, hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    e = hipMemcpyAsync(v, scratch + n, n * 4, hipMemcpyDeviceToDevice, stream);
    if (e != hipSuccess) return e;
    return launch_rerotate(stream, k_raw, k_rot, table, keep, kh, dim);
}

// ---------------------------------------------------------------- row copies
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(const CopyRow *table) {
    const CopyRow e = table[blockIdx.y];
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < e.floats;
         i += (uint64_t)gridDim.x * kThreads)
        e.dst[i] = e.src[i];
}

hipError_t launch_copy_rows(hipStream_t stream, const CopyRow *table, uint32_t entries) {
    if (!entries) return hipSuccess;
    copy_rows_kernel<<<dim3(8, entries), kThreads, 0, stream>>>(table);
    return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void fill_kernel(uint32_t *p, uint64_t words,
                                                        uint32_t value) {
    for (uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x; i < words;
         i += (uint64_t)gridDim.x * kThreads)
        p[i] = value;
}

hipError_t launch_fill(hipStream_t stream, uint32_t *p, uint64_t words, uint32_t value) {
    if (!words) return hipSuccess;
    const uint64_t blocks = std::min<uint64_t>((words + kThreads - 1) / kThreads, 1024);
    fill_kernel<<<(unsigned)blocks, kThreads, 0, stream>>>(p, words, value);
    return hipGetLastError();
}

// ---------------------------------------------------------------- argmax
// src/token.s:37-63: first maximal index; NaN anywhere gives 0xffffffff.
// First maximal index of each row (strict >, ties to the lower index); a row
// holding any NaN gives 0xffffffff. Rows are split over kArgmaxChunks blocks:
// each writes (maximum, index, NaN seen) of its chunk, then one wave per row
// combines the chunks in index order.
constexpr uint32_t kArgmaxChunks = 64;
struct ArgmaxPart {
    float best;
    uint32_t index;  // 0xffffffff: the chunk holds no number
    uint32_t nan;
};

__device__ __forceinline__ void argmax_take(float &best, uint32_t &index, float v, uint32_t i) {
    if (i != 0xffffffffu && (index == 0xffffffffu || v > best || (v == best && i < index))) {
        best = v;
        index = i;
    }
}

__global__ __launch_bounds__(kThreads) void argmax_chunk_kernel(const float *x, uint64_t width,
                                                                ArgmaxPart *part) {
    __shared__ float bv[4];
    __shared__ uint32_t bi[4], bn[4];
    const float *row = x + (uint64_t)blockIdx.x * width;
    const uint64_t chunk = (width + kArgmaxChunks - 1) / kArgmaxChunks;
    const uint64_t lo = blockIdx.y * chunk, hi = min(width, lo + chunk);
    float best = -__builtin_inff();
    uint32_t index = 0xffffffffu, nan = 0;
    // Four loads in flight per thread; each thread visits its indices in
    // increasing order, so strict > keeps the first maximum.
    for (uint64_t base = lo + threadIdx.x; base < hi; base += 4 * kThreads) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t i = base + (uint64_t)j * kThreads;
            v[j] = i < hi ? row[i] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t i = base + (uint64_t)j * kThreads;
            if (i >= hi) continue;
            if (v[j] != v[j]) nan = 1;
            else if (index == 0xffffffffu || v[j] > best) {
                best = v[j];
                index = (uint32_t)i;
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(index, o, 64);
        nan |= __shfl_xor(nan, o, 64);
        argmax_take(best, index, ov, oi);
    }
    const uint32_t wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        bv[wave] = best;
        bi[wave] = index;
        bn[wave] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        uint32_t id = bi[0], any = bn[0];
        for (int w = 1; w < 4; ++w) {
            any |= bn[w];
            argmax_take(b, id, bv[w], bi[w]);
        }
        part[(uint64_t)blockIdx.x * kArgmaxChunks + blockIdx.y] = ArgmaxPart{b, id, any};
    }
}

__global__ __launch_bounds__(64) void argmax_merge_kernel(const ArgmaxPart *part, uint32_t *out) {
    const ArgmaxPart p = part[(uint64_t)blockIdx.x * kArgmaxChunks + threadIdx.x];
    float best = p.best;
    uint32_t index = p.index, nan = p.nan;
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(index, o, 64);
        nan |= __shfl_xor(nan, o, 64);
        argmax_take(best, index, ov, oi);
    }
    if (threadIdx.x == 0) out[blockIdx.x] = nan ? 0xffffffffu : index;
}

uint64_t argmax_scratch_bytes(uint64_t rows) { return rows * kArgmaxChunks * sizeof(ArgmaxPart); }

hipError_t launch_argmax_rows(hipStream_t stream, const float *x, uint64_t width, uint64_t rows,
                              uint32_t *out, void *scratch) {
    if (!rows) return hipSuccess;
    ArgmaxPart *part = (ArgmaxPart *)scratch;
    argmax_chunk_kernel<<<dim3((unsigned)rows, kArgmaxChunks), kThreads, 0, stream>>>(x, width,
                                                                                     part);
    argmax_merge_kernel<<<(unsigned)rows, 64, 0, stream>>>(part, out);
    return hipGetLastError();
}

}  // namespace plamo
