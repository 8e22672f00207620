// MI355X backend of the PLaMo-3-Translate token loop.
//
// Implements the reference's GPU backend API (runtime/metal.h:48-88) on HIP:
// it replaces runtime/metal.m, runtime/metal_model.m and runtime/metal_weights.m.
// Weights named by the config mappings or by preload() are copied to HBM once.
// KV caches, rotated keys and workspace live in HBM; the model's host arrays
// are refreshed before each successful call returns (the reference shares
// them zero-copy with the GPU, runtime/metal_model.m:57-119), and host edits
// between calls are detected and uploaded. A decode step is one hipGraph.
#include "../../include/plamo_backend.h"
#include "../../include/plamo_checkpoint.h"
#include "../../include/plamo_compute.h"
#include "../../include/plamo_diag.h"
#include "../../include/plamo_draft.h"
#include "kernels.h"

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <vector>

using namespace plamo;

// CPU kernels of the reference platform (runtime/parallel.h:21-22). Used only
// when a projection hook cannot run on the GPU, as runtime/metal.m:398-409
// does; absent on platforms without the reference CPU layer.
extern "C" void plamo_bf16_matvec_serial(const uint16_t *, const float *, float *, uint64_t,
                                         uint64_t) __attribute__((weak));
extern "C" void plamo_bf16_matmul_core(const struct plamo_matmul *) __attribute__((weak));

namespace {

constexpr float kAttentionOffset = 0.2f;                  // src/layer.s:51
constexpr float kMlpOffset = 0.08944271909999159f;        // src/model.s:111
// Device KV rows allocated per layer at first, doubled on demand. Small on
// purpose: the decode attention launch has one block per KV head per 32
// allocated rows (up to 256 rows; per 64 beyond), and the blocks past the
// current row count still pass through the CU slots ahead of the
// O-projection blocks of the same launch.
constexpr uint64_t kInitialRows = 256;
constexpr uint64_t kMaxPrompt = 4096;                     // runtime/metal_model.m:540

struct Range {
    uintptr_t host;
    uint64_t bytes;
    char *dev;
};

struct RopeTable {
    std::vector<float> freq;  // host copy used as the identity of the table
    uint32_t dim = 0;
    uint32_t scale_bits = 0;
    float *freq_dev = nullptr;
    float *table = nullptr;   // [rows][dim]: cos | sin
    uint64_t rows = 0;
};

struct Layer {
    const uint16_t *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
    uint16_t *norms = nullptr;  // device: pre | post | mlp_pre | mlp_post | qn | kn
    const uint16_t *pre, *post, *mlp_pre, *mlp_post, *qn, *kn;
    uint32_t qh = 0, kh = 0, dim = 0, hidden = 0, inter = 0, width = 0;
    uint64_t capacity = 0;
    bool sliding = false;
    bool fused = false;  // decode attention fused with the Q/K norm and KV append
    uint32_t rope = 0;
    float *k = nullptr, *v = nullptr, *rot = nullptr;
    float *host_k = nullptr, *host_v = nullptr, *host_rot = nullptr;  // device views of pinned host rows
    uint64_t rows = 0;          // device rows allocated
    // Shadow of the host bookkeeping after this backend's last return: the
    // counters and a sample of the last K and V rows ([K sample | V sample]).
    bool synced = false;
    uint64_t count = 0, processed = 0, scale_bits = 0;
    std::vector<float> last_kv;
    uint64_t verify_prefix = 0;
    bool verify_stale = false;  // device rebuilt rotated rows the host still has stale
};

struct Buffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};

}  // namespace

struct plamo_metal {
    plamo_metal_config config{};
    plamo_metal_info info{};
    int device = 0;
    int cus = 256;
    hipStream_t stream = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    // A prompt's cache rows return to the host arrays on copy_stream, layer by
    // layer after layer_events[i] (recorded on `stream` once the layer's rows
    // are final), overlapping the later layers.
    hipStream_t copy_stream = nullptr;
    hipEvent_t layer_events[kMaxLayers] = {};
    // A prompt's restored-prefix upload runs on copy_stream, beside the
    // prompt's first launches; upload_event marks its end, and the first
    // launch that reads cached rows waits for it (upload_pending).
    hipEvent_t upload_event = nullptr;
    bool upload_pending = false;
    std::vector<Range> ranges;
    bool hooks = false;

    struct model *model = nullptr;
    // What the prepared state was built from besides the descriptor address:
    // host arrays, weights and shapes (a new model at a freed one's address
    // must not inherit its graph or pinned-host views).
    std::vector<uintptr_t> fingerprint;
    std::vector<Layer> layers;
    std::vector<RopeTable> ropes;
    const uint16_t *embedding = nullptr, *head = nullptr;
    uint16_t *final_norm = nullptr;
    uint64_t max_width = 0, max_qkv = 0, max_attention = 0, max_inter = 0, max_cols = 0;
    uint64_t max_partial = 0;  // qh * (dim + 2) over layers
    uint32_t max_splits = 1;   // attention blocks per KV head at full capacity

    StepParams *params_host = nullptr, *params_dev = nullptr;
    StepParams *params_view = nullptr;  // device view of params_host (pinned)
    // Decode workspace.
    float *state_a = nullptr, *state_b = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr,
          *branch = nullptr, *act = nullptr, *down_out = nullptr, *partial = nullptr;
    uint32_t *counters = nullptr;
    uint32_t *attention_flags = nullptr;  // [layers][kAttentionFlags] step tags
    uint32_t step_tag = 0;                // last decode step's tag
    float *outbox = nullptr, *outbox_host = nullptr;  // logits | state | normalized | stage
    uint64_t outbox_floats = 0;
    // When every host array a step updates is pinned and device-visible, the
    // graph writes them in place (no host-side mirror copies).
    bool host_direct = false;
    // PLAMO_HIP_EAGER_DECODE=1 at open: every decode step launches its kernels
    // one by one instead of replaying the captured graph (same kernels, same
    // arguments). For profilers that trace kernel launches but not graph
    // replays.
    bool eager_decode = false;
    float *host_state = nullptr, *host_norm = nullptr, *host_logits = nullptr;
    // The device's error word of the last call, copied by the call's last
    // kernel (or a copy) into pinned host memory; status_dev is its device view.
    uint32_t *status_host = nullptr, *status_dev = nullptr;
    // Prompt / candidate workspace (grown on demand).
    uint64_t prompt_rows = 0;
    Buffer p_state, p_norm, p_qkv, p_q, p_attn, p_branch, p_gu, p_act, p_side_k, p_side_v,
        p_ids, p_window, p_logits, p_attn_split;
    uint32_t *ids_host = nullptr;
    // Candidate results kept for commit.
    float *v_state = nullptr, *v_norm = nullptr, *v_logits = nullptr, *v_prop = nullptr;
    float *v_host = nullptr;  // pinned: states | normalized | logits | proposals
    bool prop_on_host = true;  // the last verify copied its proposals into v_host
    uint32_t *v_next = nullptr, *v_next_host = nullptr;
    void *v_argmax = nullptr;  // argmax partials of the candidate logits
    CopyRow *copy_table = nullptr, *copy_table_host = nullptr;
    CopyRow *upload_table = nullptr;  // pinned: host-to-device rows of sync_from_host
    const CopyRow *upload_view = nullptr;  // its device view
    uint64_t verification_tokens = 0, verification_index = 0;

    Buffer lin_in, lin_out, mlp_state, mlp_norm, mlp_gu, mlp_act, mlp_branch, mlp_norms;
    GemmWorkspace gemm{};  // split-K partial tiles and arrival counters

    hipGraphExec_t graph = nullptr;
    uint64_t epoch = 1, graph_epoch = 0;
    // The same step for contexts below kDecodeShortRows rows in every layer,
    // with the attention's view of the allocation capped there.
    hipGraphExec_t graph_short = nullptr;
    uint64_t graph_short_epoch = 0;
    // Kernels and copies each captured graph holds (counted at capture).
    int graph_dispatches = 0, graph_short_dispatches = 0;
    std::vector<void *> allocations;
};

// Scratch of plamo_hip_linear_static: [arrival counters | split-K partial
// tiles | BF16 planes of the input]. The partial region has the size of the
// allocating GEMM workspace, so both entry points choose the same tiling and
// produce the same bits. In host code `scratch` names a host-side stand-in:
// only its device address (static_scratch[device], taken once per device at
// plamo_metal_open) is ever passed to the GPU.
constexpr uint64_t kStaticCounterBytes = 64ull << 10;
constexpr uint64_t kStaticPartialBytes = kGemmPartialFloats * sizeof(float);
static_assert(kStaticCounterBytes >= kGemmCounters * sizeof(uint32_t), "counters fit");
static_assert(kStaticCounterBytes + kStaticPartialBytes + PLAMO_HIP_STATIC_PLANE_BYTES ==
                  PLAMO_HIP_STATIC_SCRATCH_BYTES, "scratch layout");
static __device__ __align__(256) unsigned char scratch[PLAMO_HIP_STATIC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static void *static_scratch[kMaxDevices];
// One call at a time owns a GPU's scratch, whichever backend instance makes
// it: a call that finds it taken is refused instead of sharing it.
static std::atomic<bool> static_scratch_busy[kMaxDevices];

namespace {

int problem(plamo_metal *m, const char *format, ...) {
    va_list args;
    va_start(args, format);
    vsnprintf(m->info.note, sizeof m->info.note, format, args);
    va_end(args);
    ++m->info.errors;
    return 0;
}

// A failure after device work started: the device KV may no longer match the
// host arrays, so every layer is uploaded again at the next call. The
// reference's contract for this case is -1, never retried (runtime/metal.h:63-67).
int fail(plamo_metal *m) {
    for (Layer &l : m->layers) l.synced = false;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->copy_stream) (void)hipStreamSynchronize(m->copy_stream);
    (void)hipGetLastError();
    return -1;
}

#define HIP_FAIL(m, call)                                                                          \
    do {                                                                                           \
        hipError_t e_ = (call);                                                                    \
        if (e_ != hipSuccess) {                                                                    \
            problem(m, "%s: %s", #call, hipGetErrorString(e_));                                    \
            return fail(m);                                                                        \
        }                                                                                          \
    } while (0)

#define HIP_TRY(m, call)                                                                           \
    do {                                                                                           \
        hipError_t e_ = (call);                                                                    \
        if (e_ != hipSuccess)                                                                      \
            return problem(m, "%s: %s", #call, hipGetErrorString(e_));                             \
    } while (0)

template <typename T>
T *dev_alloc(plamo_metal *m, uint64_t count) {
    void *p = nullptr;
    uint64_t bytes = count * sizeof(T);
    if (!bytes) bytes = 16;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        problem(m, "cannot allocate %llu bytes of HBM", (unsigned long long)bytes);
        return nullptr;
    }
    m->allocations.push_back(p);
    m->info.allocated_bytes += bytes;
    return (T *)p;
}

void dev_free(plamo_metal *m, void *p) {
    if (!p) return;
    auto it = std::find(m->allocations.begin(), m->allocations.end(), p);
    if (it != m->allocations.end()) m->allocations.erase(it);
    (void)hipFree(p);
}

bool ensure(plamo_metal *m, Buffer &b, uint64_t bytes) {
    if (b.bytes >= bytes) return true;
    dev_free(m, b.ptr);
    b.ptr = dev_alloc<char>(m, bytes);
    b.bytes = b.ptr ? bytes : 0;
    return b.ptr != nullptr;
}

template <typename T>
T *as(Buffer &b) {
    return (T *)b.ptr;
}

uint32_t float_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// The shadow's sample of a layer's last K and V rows: their first and last
// kProbe values (the whole rows when narrower). A step writes these rows from
// the device, so they are cold in the host's caches: sampling keeps the check
// to a few cache lines per layer instead of whole rows.
constexpr uint64_t kProbe = 16;
uint64_t probe_floats(uint64_t width) { return width < 2 * kProbe ? width : 2 * kProbe; }

void probe_row(const float *row, uint64_t width, float *out) {
    if (width < 2 * kProbe) {
        memcpy(out, row, width * 4);
        return;
    }
    memcpy(out, row, kProbe * 4);
    memcpy(out + kProbe, row + width - kProbe, kProbe * 4);
}

bool probe_equal(const float *row, uint64_t width, const float *saved) {
    if (width < 2 * kProbe) return !memcmp(row, saved, width * 4);
    return !memcmp(row, saved, kProbe * 4) &&
           !memcmp(row + width - kProbe, saved + kProbe, kProbe * 4);
}

// ---------------------------------------------------------------- weights
const void *resolve(const plamo_metal *m, const void *host, uint64_t bytes) {
    // Ranges are sorted by start and may nest (a preloaded window inside a
    // mapping); any range that holds [host, host + bytes) will do.
    uintptr_t a = (uintptr_t)host;
    auto it = std::upper_bound(m->ranges.begin(), m->ranges.end(), a,
                               [](uintptr_t v, const Range &r) { return v < r.host; });
    while (it != m->ranges.begin()) {
        --it;
        if (a + bytes <= it->host + it->bytes) return it->dev + (a - it->host);
    }
    return nullptr;
}

int add_range(plamo_metal *m, const void *host, uint64_t bytes) {
    if (!host || !bytes) return 1;
    if (resolve(m, host, bytes)) return 1;
    // A safetensors shard keeps its tensors at offsets of its data section,
    // which starts 8 + header-length bytes in (8-byte aligned by the format):
    // the copy is placed so that the data section starts on a 256-byte
    // boundary, keeping the 16-byte row alignment the vector kernels take.
    uint64_t shift = 0;
    struct plamo_safetensors_view view;
    if (plamo_safetensors_view(host, bytes, &view))
        shift = (256 - (uint64_t)((const char *)view.data - (const char *)host) % 256) % 256;
    char *base = dev_alloc<char>(m, bytes + shift);
    if (!base) return 0;
    char *dev = base + shift;
    if (hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        dev_free(m, base);
        return problem(m, "cannot copy %llu weight bytes to HBM", (unsigned long long)bytes);
    }
    Range r{(uintptr_t)host, bytes, dev};
    m->ranges.insert(std::upper_bound(m->ranges.begin(), m->ranges.end(), r,
                                      [](const Range &x, const Range &y) { return x.host < y.host; }),
                     r);
    m->info.cache.cached_bytes += bytes;
    m->info.private_weight_bytes += bytes;
    ++m->info.cache.misses;
    return 1;
}

// ---------------------------------------------------------------- model setup
// Candidate buffers of verify/commit. All or nothing: v_state is set only
// when every buffer exists, so a later call never runs on a partial set.
void free_verify(plamo_metal *m) {
    for (float **p : {&m->v_state, &m->v_norm, &m->v_logits, &m->v_prop}) {
        dev_free(m, *p);
        *p = nullptr;
    }
    dev_free(m, m->v_next);
    m->v_next = nullptr;
    dev_free(m, m->v_argmax);
    m->v_argmax = nullptr;
    dev_free(m, m->copy_table);
    m->copy_table = nullptr;
    if (m->v_host) (void)hipHostFree(m->v_host);
    if (m->v_next_host) (void)hipHostFree(m->v_next_host);
    if (m->copy_table_host) (void)hipHostFree(m->copy_table_host);
    m->v_host = nullptr;
    m->v_next_host = nullptr;
    m->copy_table_host = nullptr;
}

bool alloc_verify(plamo_metal *m, uint64_t L, uint64_t h, uint64_t V) {
    const uint64_t prop = L * 3 * kMaxVerify * m->max_width;
    float *state = dev_alloc<float>(m, kMaxVerify * h);
    m->v_norm = dev_alloc<float>(m, kMaxVerify * h);
    m->v_logits = dev_alloc<float>(m, kMaxVerify * V);
    m->v_prop = dev_alloc<float>(m, prop);
    m->v_next = dev_alloc<uint32_t>(m, kMaxVerify);
    m->v_argmax = dev_alloc<char>(m, argmax_scratch_bytes(kMaxVerify));
    m->copy_table = dev_alloc<CopyRow>(m, 6 * kMaxLayers);  // device and host rows per layer
    bool ok = state && m->v_norm && m->v_logits && m->v_prop && m->v_next && m->v_argmax &&
              m->copy_table;
    ok = ok && hipHostMalloc((void **)&m->v_host, (kMaxVerify * (2 * h + V) + prop) * 4,
                             hipHostMallocDefault) == hipSuccess;
    ok = ok && hipHostMalloc((void **)&m->v_next_host, kMaxVerify * 4, hipHostMallocDefault) ==
                   hipSuccess;
    ok = ok && hipHostMalloc((void **)&m->copy_table_host, 6 * kMaxLayers * sizeof(CopyRow),
                             hipHostMallocDefault) == hipSuccess;
    if (!ok) {
        (void)hipGetLastError();
        dev_free(m, state);
        free_verify(m);
        problem(m, "cannot allocate verification buffers");
        return false;
    }
    m->v_state = state;
    return true;
}

void release_model(plamo_metal *m) {
    for (hipGraphExec_t *g : {&m->graph, &m->graph_short})
        if (*g) {
            (void)hipGraphExecDestroy(*g);
            *g = nullptr;
        }
    for (Layer &l : m->layers) {
        dev_free(m, l.norms);
        dev_free(m, l.k);
        dev_free(m, l.v);
        dev_free(m, l.rot);
    }
    for (RopeTable &r : m->ropes) {
        dev_free(m, r.freq_dev);
        dev_free(m, r.table);
    }
    m->layers.clear();
    m->ropes.clear();
    dev_free(m, m->final_norm);
    m->final_norm = nullptr;
    m->model = nullptr;
    m->fingerprint.clear();
    m->head = m->embedding = nullptr;
    m->prompt_rows = 0;
    free_verify(m);
    m->verification_tokens = 0;
    ++m->epoch;
}

int ensure_rope_rows(plamo_metal *m, RopeTable &r, uint64_t rows) {
    if (rows <= r.rows) return 1;
    uint64_t target = r.rows ? r.rows : 128;
    while (target < rows) target *= 2;
    float *table = dev_alloc<float>(m, target * r.dim);
    if (!table) return 0;
    if (r.rows)
        HIP_TRY(m, hipMemcpyAsync(table, r.table, r.rows * r.dim * 4, hipMemcpyDeviceToDevice,
                                  m->stream));
    float scale;
    memcpy(&scale, &r.scale_bits, 4);
    HIP_TRY(m, launch_rope_table(m->stream, r.freq_dev, scale, r.dim / 2, r.rows, target - r.rows,
                                 table));
    HIP_TRY(m, hipStreamSynchronize(m->stream));
    dev_free(m, r.table);
    r.table = table;
    r.rows = target;
    ++m->epoch;
    return 1;
}

int ensure_kv_rows(plamo_metal *m, Layer &l, uint64_t rows) {
    if (rows <= l.rows) return 1;
    uint64_t target = l.rows ? l.rows : kInitialRows;
    while (target < rows) target *= 2;
    if (target > l.capacity) target = l.capacity;
    float *k = dev_alloc<float>(m, target * l.width), *v = dev_alloc<float>(m, target * l.width),
          *rot = dev_alloc<float>(m, target * l.width);
    if (!k || !v || !rot) return 0;
    if (l.rows) {
        // A pending prefix upload may still be writing the old rows.
        if (m->upload_pending) HIP_TRY(m, hipStreamWaitEvent(m->stream, m->upload_event, 0));
        uint64_t bytes = l.rows * l.width * 4;
        HIP_TRY(m, hipMemcpyAsync(k, l.k, bytes, hipMemcpyDeviceToDevice, m->stream));
        HIP_TRY(m, hipMemcpyAsync(v, l.v, bytes, hipMemcpyDeviceToDevice, m->stream));
        HIP_TRY(m, hipMemcpyAsync(rot, l.rot, bytes, hipMemcpyDeviceToDevice, m->stream));
        HIP_TRY(m, hipStreamSynchronize(m->stream));
    }
    dev_free(m, l.k);
    dev_free(m, l.v);
    dev_free(m, l.rot);
    l.k = k;
    l.v = v;
    l.rot = rot;
    l.rows = target;
    ++m->epoch;
    return 1;
}

// Device address of pinned host memory, or nullptr for pageable memory.
float *device_view(void *p) {
    hipPointerAttribute_t attr{};
    if (!p || hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (attr.type != hipMemoryTypeHost || !attr.devicePointer) return nullptr;
    return (float *)attr.devicePointer;
}

void find_host_views(plamo_metal *m, struct model *model) {
    m->host_state = device_view(model->state);
    m->host_norm = device_view(model->normalized);
    m->host_logits = device_view(model->logits);
    bool ok = m->host_state && m->host_norm && m->host_logits;
    for (uint64_t i = 0; i < model->count; ++i) {
        Layer &d = m->layers[i];
        struct mixer *mx = model->layers[i]->mixer;
        d.host_k = device_view(mx->cache->k);
        d.host_v = device_view(mx->cache->v);
        d.host_rot = device_view(mx->rotation->out);
        ok = ok && d.host_k && d.host_v && d.host_rot;
    }
    m->host_direct = ok;
}

std::vector<uintptr_t> model_fingerprint(const struct model *model) {
    std::vector<uintptr_t> f;
    if (!model) return f;
    f = {(uintptr_t)model->count, (uintptr_t)model->hidden, (uintptr_t)model->vocab,
         (uintptr_t)model->state, (uintptr_t)model->normalized, (uintptr_t)model->logits,
         (uintptr_t)model->embedding, (uintptr_t)model->head, (uintptr_t)model->norm};
    if (model->count > kMaxLayers || !model->layers) return f;
    for (uint64_t i = 0; i < model->count; ++i) {
        const struct layer *l = model->layers[i];
        if (!l || !l->mixer || !l->mixer->cache || !l->mixer->rotation || !l->mixer->qkv ||
            !l->mlp) {
            f.push_back(0);
            continue;
        }
        const struct cache *c = l->mixer->cache;
        f.insert(f.end(), {(uintptr_t)c->k, (uintptr_t)c->v, (uintptr_t)l->mixer->rotation->out,
                           (uintptr_t)c->capacity, (uintptr_t)c->width, (uintptr_t)c->sliding,
                           (uintptr_t)l->mixer->qkv->weight, (uintptr_t)l->mixer->weight,
                           (uintptr_t)l->mlp->gu, (uintptr_t)l->mlp->down,
                           (uintptr_t)l->mlp->intermediate, (uintptr_t)l->mixer->rotation->freq});
    }
    return f;
}

int prepare(plamo_metal *m, struct model *model) {
    std::vector<uintptr_t> f = model_fingerprint(model);
    if (m->model == model && f == m->fingerprint) {
        // The fingerprint holds addresses only. A model rebuilt at the same
        // addresses may have host arrays that are no longer pinned (or pinned
        // anew): the direct-write views are checked on the state array (an
        // instance's arrays are allocated alike) before kernels write them.
        if (m->host_direct && device_view(model->state) != m->host_state) {
            find_host_views(m, model);
            for (Layer &l : m->layers) l.synced = false;
            ++m->epoch;  // the captured graphs hold the old views
        }
        return 1;
    }
    release_model(m);
    if (!model || !model->count || model->count > kMaxLayers || !model->hidden ||
        model->hidden > UINT32_MAX || !model->vocab || model->vocab > UINT32_MAX ||
        !model->embedding || !model->head || !model->norm || !model->state ||
        !model->normalized || !model->logits || !model->scales)
        return 0;
    uint64_t h = model->hidden;
    m->layers.resize(model->count);
    m->max_width = m->max_qkv = m->max_attention = m->max_inter = m->max_partial = 0;
    m->max_splits = 1;
    m->max_cols = h;
    for (uint64_t i = 0; i < model->count; ++i) {
        const struct layer *l = model->layers[i];
        const struct qkv *q = l->mixer->qkv;
        const struct cache *c = l->mixer->cache;
        const struct rotation *r = l->mixer->rotation;
        const struct mlp *p = l->mlp;
        // runtime/metal_model.m:223-235, plus this backend's kernel limit
        // head_dim <= 256.
        if (l->hidden != h || q->hidden != h || p->hidden != h || l->mixer->hidden != h ||
            !q->kh || !q->qh || q->qh % q->kh || !q->dim || q->dim % 2 ||
            q->dim > 256 || !c->capacity || c->capacity > UINT32_MAX ||
            c->width != q->kh * q->dim || r->cache != c || r->heads != q->kh ||
            r->dim != q->dim || !p->intermediate || p->intermediate > UINT32_MAX / 2 ||
            !r->freq || !c->k || !c->v || !r->out) {
            release_model(m);
            return 0;
        }
        Layer &d = m->layers[i];
        d.qh = (uint32_t)q->qh;
        d.kh = (uint32_t)q->kh;
        d.dim = (uint32_t)q->dim;
        d.hidden = (uint32_t)h;
        d.inter = (uint32_t)p->intermediate;
        d.width = (uint32_t)c->width;
        d.capacity = c->capacity;
        d.sliding = c->sliding != 0;
        d.fused = decode_attention_supported(d.dim, d.qh / d.kh);
        d.pre = l->pre;
        d.post = l->post;
        d.mlp_pre = p->pre;
        d.mlp_post = p->post;
        d.qn = q->qn;
        d.kn = q->kn;
        // Norm weights are small: always private device copies
        // (runtime/metal_model.m:294-303 copies them as well).
        uint64_t words = 4 * h + 2 * (uint64_t)d.dim;
        d.norms = dev_alloc<uint16_t>(m, words);
        if (!d.norms) {
            release_model(m);
            return 0;
        }
        const uint16_t *src[6] = {l->pre, l->post, p->pre, p->post, q->qn, q->kn};
        uint64_t len[6] = {h, h, h, h, d.dim, d.dim}, off = 0;
        for (int j = 0; j < 6; ++j) {
            if (hipMemcpy(d.norms + off, src[j], len[j] * 2, hipMemcpyHostToDevice) != hipSuccess) {
                (void)hipGetLastError();
                release_model(m);
                return problem(m, "cannot copy norm weights");
            }
            off += len[j];
        }
        uint32_t scale = float_bits(model->scales[i]);
        size_t rope = 0;
        for (; rope < m->ropes.size(); ++rope) {
            RopeTable &t = m->ropes[rope];
            if (t.dim == d.dim && t.scale_bits == scale &&
                !memcmp(t.freq.data(), r->freq, d.dim / 2 * sizeof(float)))
                break;
        }
        if (rope == m->ropes.size()) {
            RopeTable t;
            t.freq.assign(r->freq, r->freq + d.dim / 2);
            t.dim = d.dim;
            t.scale_bits = scale;
            t.freq_dev = dev_alloc<float>(m, d.dim / 2);
            if (!t.freq_dev ||
                hipMemcpy(t.freq_dev, r->freq, d.dim / 2 * 4, hipMemcpyHostToDevice) != hipSuccess) {
                (void)hipGetLastError();
                release_model(m);
                return problem(m, "cannot copy RoPE frequencies");
            }
            m->ropes.push_back(std::move(t));
        }
        d.rope = (uint32_t)rope;
        uint64_t want = std::min<uint64_t>(c->capacity, kInitialRows);
        if (!ensure_rope_rows(m, m->ropes[rope], want) || !ensure_kv_rows(m, d, want)) {
            release_model(m);
            return 0;
        }
        d.synced = false;
        d.last_kv.assign(2 * probe_floats(d.width), 0.0f);
        m->max_width = std::max<uint64_t>(m->max_width, d.width);
        m->max_qkv = std::max<uint64_t>(m->max_qkv, (uint64_t)(d.qh + 2 * d.kh) * d.dim);
        m->max_attention = std::max<uint64_t>(m->max_attention, (uint64_t)d.qh * d.dim);
        m->max_inter = std::max<uint64_t>(m->max_inter, d.inter);
        m->max_partial = std::max<uint64_t>(m->max_partial, (uint64_t)d.qh * (d.dim + 2));
        m->max_splits = std::max(m->max_splits, decode_attention_splits(d.capacity));
        m->max_cols = std::max<uint64_t>(m->max_cols, std::max<uint64_t>(d.inter, (uint64_t)d.qh * d.dim));
    }
    // The embedding is read one row per token on the device: keep the table
    // resident even when the engine did not preload it (runtime/engine.c:293-296
    // skips it on purpose for Apple's shared memory).
    if (!add_range(m, model->embedding, model->vocab * h * 2)) {
        release_model(m);
        return 0;
    }
    m->embedding = (const uint16_t *)resolve(m, model->embedding, model->vocab * h * 2);
    m->final_norm = dev_alloc<uint16_t>(m, h);
    if (!m->final_norm ||
        hipMemcpy(m->final_norm, model->norm, h * 2, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        release_model(m);
        return problem(m, "cannot copy the final norm");
    }
    if (configure_gemv(m->max_cols) != hipSuccess) {
        (void)hipGetLastError();
        release_model(m);
        return problem(m, "projection width %llu exceeds the LDS budget",
                       (unsigned long long)m->max_cols);
    }
    // Decode workspace.
    uint64_t L = model->count, V = model->vocab;
    dev_free(m, m->state_a);
    dev_free(m, m->state_b);
    dev_free(m, m->qkv);
    dev_free(m, m->q);
    dev_free(m, m->attn);
    dev_free(m, m->branch);
    dev_free(m, m->act);
    dev_free(m, m->down_out);
    dev_free(m, m->partial);
    dev_free(m, m->counters);
    dev_free(m, m->attention_flags);
    dev_free(m, m->outbox);
    if (m->outbox_host) (void)hipHostFree(m->outbox_host);
    m->outbox_host = nullptr;
    m->state_a = dev_alloc<float>(m, h);
    m->state_b = dev_alloc<float>(m, h);
    m->qkv = dev_alloc<float>(m, m->max_qkv);
    m->q = dev_alloc<float>(m, m->max_attention);
    m->attn = dev_alloc<float>(m, m->max_attention);
    m->branch = dev_alloc<float>(m, h);
    m->act = dev_alloc<float>(m, m->max_inter);
    m->down_out = dev_alloc<float>(m, h);
    m->partial = dev_alloc<float>(m, m->max_partial * m->max_splits);
    m->counters = dev_alloc<uint32_t>(m, 256);
    m->attention_flags = dev_alloc<uint32_t>(m, L * kAttentionFlags);
    m->outbox_floats = V + 2 * h + L * 3 * m->max_width;
    m->outbox = dev_alloc<float>(m, m->outbox_floats);
    if (!m->state_a || !m->state_b || !m->qkv || !m->q || !m->attn || !m->branch || !m->act ||
        !m->down_out || !m->partial || !m->counters || !m->attention_flags || !m->outbox ||
        hipHostMalloc((void **)&m->outbox_host, m->outbox_floats * 4, hipHostMallocDefault) !=
            hipSuccess ||
        hipMemset(m->counters, 0, 256 * 4) != hipSuccess ||
        hipMemset(m->attention_flags, 0, L * kAttentionFlags * 4) != hipSuccess) {
        (void)hipGetLastError();
        release_model(m);
        return problem(m, "cannot allocate decode workspace");
    }
    m->model = model;
    m->fingerprint = std::move(f);
    find_host_views(m, model);
    ++m->epoch;
    return 1;
}

// Projections must already be resident (preloaded or mapped); a miss declines.
bool resolve_layers(plamo_metal *m, struct model *model) {
    uint64_t h = model->hidden;
    for (uint64_t i = 0; i < model->count; ++i) {
        Layer &d = m->layers[i];
        if (d.qkv && d.o && d.gu && d.down) continue;
        const struct layer *l = model->layers[i];
        const struct qkv *q = l->mixer->qkv;
        d.qkv = (const uint16_t *)resolve(m, q->weight, (uint64_t)(d.qh + 2 * d.kh) * d.dim * h * 2);
        d.o = (const uint16_t *)resolve(m, l->mixer->weight, h * d.qh * d.dim * 2);
        d.gu = (const uint16_t *)resolve(m, l->mlp->gu, 2 * (uint64_t)d.inter * h * 2);
        d.down = (const uint16_t *)resolve(m, l->mlp->down, (uint64_t)d.inter * h * 2);
        if (!d.qkv || !d.o || !d.gu || !d.down) {
            d.qkv = d.o = d.gu = d.down = nullptr;
            return false;
        }
    }
    if (!m->head) m->head = (const uint16_t *)resolve(m, model->head, model->vocab * h * 2);
    return m->head != nullptr;
}

// ---------------------------------------------------------------- host <-> device KV
// Longest fixed prompt prefix the engine snapshots and restores
// (PLAMO_PROMPT_PREFIX_LIMIT, runtime/prompt_cache.h:8).
constexpr uint64_t kPromptPrefixLimit = 64;

// Detects host-side KV edits since this backend's last return (prompt-prefix
// restore, draft restore, request reset, a CPU step) and uploads the host rows.
// Sets stale[i] when the device rotated rows must be rebuilt.
//
// A prompt-prefix restore can leave every counter and the last rows as they
// were: the engine prepares both translation prefixes in turn
// (runtime/engine.c:357-381) and a request then restores the other one
// (runtime/prompt_cache.c:62-82). The two template prefixes differ only in a
// middle id (the target language) and end in the same id, and a layer-0 row
// depends only on its token, so the sampled last rows agree too. So at prompt
// entry (`prompt_entry`) a layer whose host count is a prefix length
// (1..PLAMO_PROMPT_PREFIX_LIMIT) is always uploaded in full.
//
// When the host arrays are device-visible (pinned), the uploads run as one
// copy kernel reading them through their device views: a restored prefix is
// 3 arrays x layers segments, and as many DMA copies cost ~0.9 ms of a C4
// 128-token TTFT against ~0.1 ms for the kernel.
int sync_from_host(plamo_metal *m, struct model *model, std::vector<char> &stale,
                   bool prompt_entry) {
    stale.assign(model->count, 0);
    uint32_t entries = 0;
    for (uint64_t i = 0; i < model->count; ++i) {
        Layer &d = m->layers[i];
        const struct mixer *mx = model->layers[i]->mixer;
        const struct cache *c = mx->cache;
        const struct rotation *r = mx->rotation;
        uint32_t scale = float_bits(model->scales[i]);
        const uint64_t last = c->count ? (c->count - 1) * c->width : 0, pf = probe_floats(c->width);
        const bool restorable = prompt_entry && c->count && c->count <= kPromptPrefixLimit;
        bool same = !restorable && d.synced && d.count == c->count &&
                    d.processed == r->processed_count &&
                    d.scale_bits == r->scale_bits &&
                    (!c->count || (probe_equal(c->k + last, c->width, d.last_kv.data()) &&
                                   probe_equal(c->v + last, c->width, d.last_kv.data() + pf)));
        if (same) {
            stale[i] = r->processed_count != c->count || r->scale_bits != scale;
            continue;
        }
        if (!ensure_kv_rows(m, d, c->count)) return 0;
        const uint64_t floats = c->count * c->width, bytes = floats * 4;
        const bool rotated = r->processed_count == c->count && r->scale_bits == scale;
        const bool viewed = m->host_direct && d.host_k && d.host_v && d.host_rot;
        if (bytes && viewed) {
            // A call that returned early may have left its upload running:
            // it reads this table until it finishes.
            if (!entries) {
                HIP_TRY(m, hipStreamSynchronize(m->copy_stream));
                HIP_TRY(m, hipStreamSynchronize(m->stream));
            }
            m->upload_table[entries++] = CopyRow{d.host_k, d.k, floats};
            m->upload_table[entries++] = CopyRow{d.host_v, d.v, floats};
            if (rotated) m->upload_table[entries++] = CopyRow{d.host_rot, d.rot, floats};
        } else if (bytes) {
            HIP_TRY(m, hipMemcpyAsync(d.k, c->k, bytes, hipMemcpyHostToDevice, m->stream));
            HIP_TRY(m, hipMemcpyAsync(d.v, c->v, bytes, hipMemcpyHostToDevice, m->stream));
            if (rotated)
                HIP_TRY(m, hipMemcpyAsync(d.rot, r->out, bytes, hipMemcpyHostToDevice, m->stream));
        }
        stale[i] = !rotated && c->count;
        d.synced = false;
    }
    // The kernel reads the table on the stream; the previous call's upload has
    // completed, since every call waits for its work. At prompt entry it runs
    // on copy_stream, after whatever the stream holds (reallocation copies of
    // the same rows), while the prompt's embedding, norm and first
    // projection need no cached row (C4 128-token prompt: the 4.7 MB of a
    // restored 12-token prefix cross the bus in ~80 us).
    m->upload_pending = false;
    if (prompt_entry && entries) {
        HIP_TRY(m, hipEventRecord(m->upload_event, m->stream));
        HIP_TRY(m, hipStreamWaitEvent(m->copy_stream, m->upload_event, 0));
        HIP_TRY(m, launch_copy_rows(m->copy_stream, m->upload_view, entries));
        HIP_TRY(m, hipEventRecord(m->upload_event, m->copy_stream));
        m->upload_pending = true;
        return 1;
    }
    HIP_TRY(m, launch_copy_rows(m->stream, m->upload_view, entries));
    return 1;
}

void remember(plamo_metal *m, struct model *model) {
    for (uint64_t i = 0; i < model->count; ++i) {
        Layer &d = m->layers[i];
        const struct mixer *mx = model->layers[i]->mixer;
        const struct cache *c = mx->cache;
        d.count = c->count;
        d.processed = mx->rotation->processed_count;
        d.scale_bits = mx->rotation->scale_bits;
        if (c->count) {
            const uint64_t last = (c->count - 1) * c->width;
            probe_row(c->k + last, c->width, d.last_kv.data());
            probe_row(c->v + last, c->width, d.last_kv.data() + probe_floats(c->width));
        }
        d.synced = true;
    }
}

// `start` only timestamps the call (created without the system-scope fence:
// the fence's cache write-back held the call's first launch back, C4 decode
// 2.918-2.920 against 2.915-2.916 ms/step); `stop` keeps it, since the host
// reads the call's results once it has completed.
void begin_timing(plamo_metal *m) { (void)hipEventRecord(m->start, m->stream); }
int end_timing(plamo_metal *m) {
    HIP_TRY(m, hipEventRecord(m->stop, m->stream));
    HIP_TRY(m, hipEventSynchronize(m->stop));
    float ms = 0;
    if (hipEventElapsedTime(&ms, m->start, m->stop) == hipSuccess) m->info.gpu_seconds += ms * 1e-3;
    ++m->info.command_buffers;
    return 1;
}

// A kernel of the call gave up a bounded wait (runtime/metal.h:63-67: the
// call then fails with -1 after partial writes).
bool device_failed(plamo_metal *m) {
    if (!*m->status_host) return false;
    problem(m, "a bounded device wait gave up (error word %u)", *m->status_host);
    return true;
}

// ---------------------------------------------------------------- decode
struct DecodePlan {
    std::vector<char> stale, shift;
    bool special = false;
    bool direct = false;  // host arrays written in place by the step itself
    // Nonzero: every layer's rows stay below this count for the step, and the
    // decode attention sees at most this many allocated rows (its
    // short-context blocks).
    uint32_t row_cap = 0;
};

// Enqueues one decode step: embedding, every layer, final norm + head, and the
// copy of logits/state/normalized/new KV rows to the pinned outbox.
int encode_decode(plamo_metal *m, struct model *model, const DecodePlan &plan, int *dispatches) {
    const uint64_t h = model->hidden, V = model->vocab, L = model->count;
    hipStream_t s = m->stream;
    int n = 0;
    float *logits = m->outbox, *state_out = m->outbox + V, *norm_out = m->outbox + V + h;
    float *stage = m->outbox + V + 2 * h;
    // The embedding reads the host's parameter block and publishes it to the
    // device copy the later kernels read (no separate upload node).
    HIP_TRY(m, launch_embed(s, m->embedding, nullptr, m->params_view, 1, (uint32_t)h, m->state_a,
                            m->params_dev));
    ++n;
    float *cur = m->state_a, *nxt = m->state_b;
    const int blocks = 2 * m->cus;
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        const uint16_t *pre = d.norms, *post = d.norms + h, *mpre = d.norms + 2 * h,
                       *mpost = d.norms + 3 * h, *qn = d.norms + 4 * h, *kn = qn + d.dim;
        const RopeTable &rope = m->ropes[d.rope];
        Prologue p1{};
        p1.src = cur;
        p1.w = pre;
        p1.offset = 1.0f;
        if (i) {
            p1.branch = m->down_out;
            p1.rw = m->layers[i - 1].norms + 3 * h;
            p1.roffset = kMlpOffset;
            p1.state_out = nxt;
        }
        uint64_t qkv_rows = (uint64_t)(d.qh + 2 * d.kh) * d.dim;
        const bool shift = plan.shift[i], stale = plan.stale[i];
        float *layer_stage = stage + i * 3 * m->max_width;
        // Attention over the materialized rotated rows (no sliding shift).
        auto attention_args = [&]() {
            DecodeAttention da{};
            da.qkv = m->qkv;
            da.qn = qn;
            da.kn = kn;
            da.freq = rope.freq_dev;
            memcpy(&da.rope_scale, &rope.scale_bits, 4);
            da.k_raw = d.k;
            da.rows = (uint32_t)(plan.row_cap ? std::min<uint64_t>(d.rows, plan.row_cap) : d.rows);
            da.v = d.v;
            da.k_rot = d.rot;
            da.stage = plan.direct ? nullptr : layer_stage;
            if (plan.direct) {
                da.host_k = d.host_k;
                da.host_v = d.host_v;
                da.host_rot = d.host_rot;
            }
            da.out = m->attn;
            da.partial = m->partial;
            da.counters = m->counters;
            da.params = m->params_dev;
            da.layer = (uint32_t)i;
            da.qh = d.qh;
            da.kh = d.kh;
            da.dim = d.dim;
            da.splits = decode_attention_splits(da.rows);
            return da;
        };
        HIP_TRY(m, launch_gemv(s, d.qkv, qkv_rows, h, p1, m->qkv, 0, blocks));
        ++n;
        if (i) std::swap(cur, nxt);
        if (stale && !shift) {
            uint32_t rows = m->params_host->count[i];
            HIP_TRY(m, launch_rerotate(s, d.k, d.rot, rope.table, rows, d.kh, d.dim));
            ++n;
        }
        bool fused_o = false;
        if (!shift && d.fused) {
            DecodeAttention da = attention_args();
            if (attention_o_supported(d.dim, d.qh / d.kh, (uint64_t)d.qh * d.dim) &&
                !((uintptr_t)d.o & 15)) {
                AttentionO ao{};
                ao.a = da;
                ao.w = d.o;
                ao.x = m->attn;
                ao.y = m->branch;
                ao.rows = (uint32_t)h;
                ao.cols = d.qh * d.dim;
                ao.heads = d.kh;
                ao.done = m->params_dev->done + i;
                ao.error = &m->params_dev->error;
                ao.flags = m->attention_flags + i * kAttentionFlags;
                HIP_TRY(m, launch_attention_o(s, ao));
                fused_o = true;
            } else {
                HIP_TRY(m, launch_decode_attention(s, da));
            }
            ++n;
        } else {
            // General path (eager only: its arguments depend on the row count).
            const uint32_t count = m->params_host->count[i];
            QkvPost qp{};
            qp.qkv = m->qkv;
            qp.q_out = m->q;
            qp.qn = qn;
            qp.kn = kn;
            qp.table = rope.table;
            qp.params = m->params_dev;
            qp.layer = (uint32_t)i;
            qp.qh = d.qh;
            qp.kh = d.kh;
            qp.dim = d.dim;
            qp.tokens = 1;
            qp.capacity = (uint32_t)d.capacity;
            qp.stage = layer_stage;
            qp.k_raw = shift ? as<float>(m->p_side_k) : d.k;
            qp.v = shift ? as<float>(m->p_side_v) : d.v;
            qp.k_rot = shift ? nullptr : d.rot;
            qp.rows_from_count = !shift;
            qp.rotate_k = !shift;
            HIP_TRY(m, launch_qkv_post(s, qp));
            PromptAttention pa{};
            pa.q = m->q;
            pa.table = rope.table;
            pa.out = m->attn;
            pa.prefix = count;
            pa.tokens = 1;
            pa.qh = d.qh;
            pa.kh = d.kh;
            pa.dim = d.dim;
            if (shift) {
                pa.k_cache = d.k;
                pa.v_cache = d.v;
                pa.k_new = as<float>(m->p_side_k);
                pa.v_new = as<float>(m->p_side_v);
                pa.window = (uint32_t)d.capacity;
            } else {
                pa.k_cache = d.rot;
                pa.v_cache = d.v;
                pa.k_new = d.rot + (uint64_t)count * d.width;
                pa.v_new = d.v + (uint64_t)count * d.width;
            }
            HIP_TRY(m, launch_prompt_attention(s, pa));
            n += 2;
            if (shift) {
                HIP_TRY(m, launch_window_store(s, d.k, d.v, d.rot, as<float>(m->p_side_k),
                                               as<float>(m->p_side_v), d.width, rope.table,
                                               as<float>(m->p_window), d.capacity, 1, d.capacity,
                                               d.kh, d.dim));
                n += 2;
            }
        }
        if (!fused_o) {
            Prologue po{};
            po.src = m->attn;
            HIP_TRY(m, launch_gemv(s, d.o, h, (uint64_t)d.qh * d.dim, po, m->branch, 0, blocks));
            ++n;
        }
        Prologue pg{};
        pg.src = cur;
        pg.w = mpre;
        pg.offset = 1.0f;
        pg.branch = m->branch;
        pg.rw = post;
        pg.roffset = kAttentionOffset;
        pg.state_out = nxt;
        HIP_TRY(m, launch_gemv(s, d.gu, 2 * (uint64_t)d.inter, h, pg, m->act, d.inter, blocks));
        std::swap(cur, nxt);
        Prologue pd{};
        pd.src = m->act;
        HIP_TRY(m, launch_gemv(s, d.down, h, d.inter, pd, m->down_out, 0, blocks));
        n += 2;
        (void)mpost;
    }
    Prologue ph{};
    ph.src = cur;
    ph.w = m->final_norm;
    ph.offset = 1.0f;
    ph.branch = m->down_out;
    ph.rw = m->layers[L - 1].norms + 3 * h;
    ph.roffset = kMlpOffset;
    ph.state_out = plan.direct ? m->host_state : state_out;
    ph.norm_out = plan.direct ? m->host_norm : norm_out;
    ph.status = &m->params_dev->error;
    ph.status_out = m->status_dev;
    // Direct: the head's rows go straight to the host logits as they are
    // computed (the PCIe writes overlap the head's weight stream; a copy
    // after the head would add its transfer to the step).
    HIP_TRY(m, launch_gemv(s, m->head, V, h, ph, plan.direct ? m->host_logits : logits, 0, blocks));
    ++n;
    if (!plan.direct)
        HIP_TRY(m, hipMemcpyAsync(m->outbox_host, m->outbox, m->outbox_floats * 4,
                                  hipMemcpyDeviceToHost, s));
    *dispatches = n;
    return 1;
}

int ensure_prompt(plamo_metal *m, struct model *model, uint64_t rows) {
    if (rows <= m->prompt_rows && m->p_state.ptr) return 1;
    uint64_t r = std::max<uint64_t>(rows, 16);
    uint64_t h = model->hidden;
    bool ok = ensure(m, m->p_state, r * h * 4) && ensure(m, m->p_norm, r * h * 4) &&
              ensure(m, m->p_qkv, r * m->max_qkv * 4) && ensure(m, m->p_q, r * m->max_attention * 4) &&
              ensure(m, m->p_attn, r * m->max_attention * 4) && ensure(m, m->p_branch, r * h * 4) &&
              ensure(m, m->p_gu, r * 2 * m->max_inter * 4) && ensure(m, m->p_act, r * m->max_inter * 4) &&
              ensure(m, m->p_side_k, r * m->max_width * 4) &&
              ensure(m, m->p_side_v, r * m->max_width * 4) && ensure(m, m->p_ids, r * 4);
    if (!ok) return 0;
    if (m->ids_host) (void)hipHostFree(m->ids_host);
    m->ids_host = nullptr;
    if (hipHostMalloc((void **)&m->ids_host, r * 4, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return problem(m, "cannot allocate pinned id staging");
    }
    m->prompt_rows = r;
    return 1;
}

// Scratch of the prompt GEMMs for up to `tokens` rows of `cols` columns: the
// split-K partials and counters are allocated once (the counters start at
// zero and every GEMM leaves them zero), the BF16 planes of X grow on demand.
const GemmWorkspace *gemm_workspace(plamo_metal *m, uint64_t tokens, uint64_t cols) {
    if (!m->gemm.partial) {
        float *partial = dev_alloc<float>(m, kGemmPartialFloats);
        uint32_t *counters = dev_alloc<uint32_t>(m, kGemmCounters);
        if (!partial || !counters || hipMemset(counters, 0, kGemmCounters * 4) != hipSuccess) {
            (void)hipGetLastError();
            dev_free(m, partial);
            dev_free(m, counters);
            problem(m, "cannot allocate GEMM scratch");
            return nullptr;
        }
        m->gemm.partial = partial;
        m->gemm.partial_floats = kGemmPartialFloats;
        m->gemm.counter_base = counters;
        m->gemm.counters = kGemmCounters;
        m->gemm.cus = (uint32_t)m->cus;
    }
    const uint64_t need = gemm_plane_elems(std::max<uint64_t>(tokens, 128), cols);
    if (need > m->gemm.plane_elems) {
        dev_free(m, m->gemm.planes);
        m->gemm.planes = dev_alloc<uint16_t>(m, need);
        m->gemm.plane_elems = m->gemm.planes ? need : 0;
        if (!m->gemm.planes) return nullptr;
    }
    return &m->gemm;
}

int ensure_window_scratch(plamo_metal *m, struct model *model) {
    uint64_t need = 0;
    for (uint64_t i = 0; i < model->count; ++i)
        if (m->layers[i].sliding)
            need = std::max<uint64_t>(need, 2 * m->layers[i].capacity * m->layers[i].width * 4);
    return !need || ensure(m, m->p_window, need);
}

}  // namespace

// ================================================================ public API
extern "C" {

static int forward_hook(struct model *model, uint64_t token, void *context) {
    return plamo_metal_forward((struct plamo_metal *)context, model, token);
}
static int prefill_hook(struct model *model, const uint32_t *ids, uint64_t n, float *states,
                        void *context) {
    return plamo_metal_prefill((struct plamo_metal *)context, model, ids, n, states);
}
static int mlp_hook(const struct mlp *mlp, float *states, uint64_t tokens, void *context) {
    return plamo_metal_mlp((struct plamo_metal *)context, mlp, states, tokens);
}
static void matvec_hook(const uint16_t *w, const float *x, float *y, uint64_t rows,
                        uint64_t cols, void *context) {
    struct plamo_metal *m = (struct plamo_metal *)context;
    struct plamo_matmul mm = {w, x, y, rows, cols, 1, cols, rows};
    if (plamo_metal_linear(m, &mm)) return;
    ++m->info.cpu_fallbacks;
    if (plamo_bf16_matvec_serial)
        plamo_bf16_matvec_serial(w, x, y, rows, cols);
    else
        problem(m, "projection not resident and no CPU kernel is linked");
}
static void matmul_hook(const struct plamo_matmul *mm, void *context) {
    struct plamo_metal *m = (struct plamo_metal *)context;
    if (plamo_metal_linear(m, mm)) return;
    ++m->info.cpu_fallbacks;
    if (plamo_bf16_matmul_core)
        plamo_bf16_matmul_core(mm);
    else
        problem(m, "projection not resident and no CPU kernel is linked");
}
static const void *identity_provider(const void *p, uint64_t, void *) { return p; }

struct plamo_metal *plamo_metal_open(const struct plamo_metal_config *config, char *error,
                                     size_t cap) {
    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1) {
        (void)hipGetLastError();
        if (error && cap) snprintf(error, cap, "HIP requires an available MI355X (gfx950) GPU");
        return nullptr;
    }
    plamo_metal *m = new plamo_metal();
    if (config) m->config = *config;
    hipDeviceProp_t prop;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        (void)hipGetLastError();
        if (error && cap) snprintf(error, cap, "cannot open HIP device 0");
        delete m;
        return nullptr;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (error && cap)
            snprintf(error, cap, "device %s is not gfx950; this backend is built for MI355X",
                     prop.gcnArchName);
        delete m;
        return nullptr;
    }
    m->cus = prop.multiProcessorCount;
    // The device address of this GPU's static scratch (once per device).
    if (m->device < kMaxDevices && !static_scratch[m->device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess && ptr)
            static_scratch[m->device] = ptr;
        else
            (void)hipGetLastError();
    }
    snprintf(m->info.device, sizeof m->info.device, "%s (%s, %d CUs)", prop.name,
             prop.gcnArchName, prop.multiProcessorCount);
    snprintf(m->info.precision, sizeof m->info.precision, "fp32");
    snprintf(m->info.weight_storage, sizeof m->info.weight_storage, "hbm-bf16");
    m->info.recommended_working_set_bytes = prop.totalGlobalMem;
    bool events = hipEventCreateWithFlags(&m->upload_event, hipEventDisableTiming) == hipSuccess;
    for (hipEvent_t &e : m->layer_events)
        events = events && hipEventCreateWithFlags(&e, hipEventDisableTiming) == hipSuccess;
    if (!events || hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&m->copy_stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&m->start, hipEventDisableSystemFence) != hipSuccess ||
        hipEventCreate(&m->stop) != hipSuccess ||
        hipHostMalloc((void **)&m->params_host, sizeof(StepParams), hipHostMallocDefault) !=
            hipSuccess ||
        !(m->params_view = (StepParams *)device_view(m->params_host)) ||
        hipHostMalloc((void **)&m->status_host, 64, hipHostMallocDefault) != hipSuccess ||
        !(m->status_dev = (uint32_t *)device_view(m->status_host)) ||
        hipHostMalloc((void **)&m->upload_table, 3 * kMaxLayers * sizeof(CopyRow),
                      hipHostMallocDefault) != hipSuccess ||
        !(m->upload_view = (const CopyRow *)device_view(m->upload_table)) ||
        hipMalloc((void **)&m->params_dev, sizeof(StepParams)) != hipSuccess) {
        (void)hipGetLastError();
        if (error && cap) snprintf(error, cap, "cannot create HIP stream or staging");
        plamo_metal_close(m);
        return nullptr;
    }
    memset(m->params_host, 0, sizeof(StepParams));
    *m->status_host = 0;
    const char *eager = getenv("PLAMO_HIP_EAGER_DECODE");
    m->eager_decode = eager && *eager && strcmp(eager, "0") != 0;
    if (m->config.memory != PLAMO_METAL_STREAM)
        for (size_t i = 0; i < m->config.count && m->config.maps; ++i)
            if (!add_range(m, m->config.maps[i].base, m->config.maps[i].bytes)) {
                if (error && cap) snprintf(error, cap, "%s", m->info.note);
                plamo_metal_close(m);
                return nullptr;
            }
    m->info.cache.budget_bytes = m->info.cache.max_budget_bytes = prop.totalGlobalMem;
    // runtime/metal.m:900-910: one process-owned backend installs the hooks.
    if (!plamo_compute_context && !plamo_weight_provider) {
        plamo_compute_context = m;
        plamo_matvec_kernel = matvec_hook;
        plamo_matmul_kernel = matmul_hook;
        plamo_mlp_kernel = mlp_hook;
        plamo_forward_kernel = forward_hook;
        plamo_prefill_kernel = prefill_hook;
        plamo_weight_provider = identity_provider;
        plamo_weight_context = nullptr;
        plamo_weight_chunk_bytes = 0;
        m->hooks = true;
    }
    return m;
}

void plamo_metal_close(struct plamo_metal *m) {
    if (!m) return;
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    if (m->copy_stream) (void)hipStreamSynchronize(m->copy_stream);
    // runtime/metal.m:938-948
    if (m->hooks && plamo_compute_context == m) {
        plamo_compute_context = nullptr;
        plamo_matvec_kernel = nullptr;
        plamo_matmul_kernel = nullptr;
        plamo_mlp_kernel = nullptr;
        plamo_forward_kernel = nullptr;
        plamo_prefill_kernel = nullptr;
        plamo_weight_provider = nullptr;
        plamo_weight_chunk_bytes = 0;
    }
    release_model(m);
    for (void *p : m->allocations) (void)hipFree(p);
    m->allocations.clear();
    if (m->outbox_host) (void)hipHostFree(m->outbox_host);
    if (m->ids_host) (void)hipHostFree(m->ids_host);
    if (m->v_host) (void)hipHostFree(m->v_host);
    if (m->v_next_host) (void)hipHostFree(m->v_next_host);
    if (m->copy_table_host) (void)hipHostFree(m->copy_table_host);
    if (m->params_host) (void)hipHostFree(m->params_host);
    if (m->status_host) (void)hipHostFree(m->status_host);
    if (m->upload_table) (void)hipHostFree(m->upload_table);
    if (m->params_dev) (void)hipFree(m->params_dev);
    if (m->start) (void)hipEventDestroy(m->start);
    if (m->stop) (void)hipEventDestroy(m->stop);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    if (m->copy_stream) (void)hipStreamDestroy(m->copy_stream);
    for (hipEvent_t e : m->layer_events)
        if (e) (void)hipEventDestroy(e);
    if (m->upload_event) (void)hipEventDestroy(m->upload_event);
    delete m;
}

void plamo_metal_maintain(struct plamo_metal *m) {
    if (m && m->stream) (void)hipStreamSynchronize(m->stream);
}

void plamo_metal_get_info(const struct plamo_metal *m, struct plamo_metal_info *out) {
    if (out) *out = m->info;
}

int plamo_metal_preload(struct plamo_metal *m, const void *ptr, uint64_t bytes) {
    if (m->config.memory == PLAMO_METAL_STREAM) return 1;
    if (resolve(m, ptr, bytes)) {
        ++m->info.cache.hits;
        m->info.cache.hit_bytes += bytes;
        return 1;
    }
    return add_range(m, ptr, bytes);
}

int plamo_metal_warm_cache(struct plamo_metal *m) {
    return hipStreamSynchronize(m->stream) == hipSuccess && hipDeviceSynchronize() == hipSuccess;
}

int plamo_metal_prepare_model(struct plamo_metal *m, struct model *model) {
    if (m->config.memory == PLAMO_METAL_STREAM) return 1;
    return prepare(m, model);
}

int plamo_metal_forward(struct plamo_metal *m, struct model *model, uint64_t token) {
    m->verification_tokens = 0;
    for (Layer &l : m->layers) l.verify_stale = false;
    if (token >= model->vocab) return -1;
    if (m->config.memory == PLAMO_METAL_STREAM) return 0;
    if (!prepare(m, model)) return -1;
    const uint64_t L = model->count, h = model->hidden, V = model->vocab;
    // Preflight before touching any state (runtime/metal_model.m:396-421).
    for (uint64_t i = 0; i < L; ++i) {
        const struct cache *c = model->layers[i]->mixer->cache;
        if (c->count > c->capacity || (c->count == c->capacity && !c->sliding)) return -1;
    }
    if (!resolve_layers(m, model)) return 0;
    DecodePlan plan;
    if (!sync_from_host(m, model, plan.stale, false)) return -1;
    plan.shift.assign(L, 0);
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        const struct cache *c = model->layers[i]->mixer->cache;
        plan.shift[i] = c->count == c->capacity;
        if (plan.shift[i] || plan.stale[i] || !d.fused) plan.special = true;
        uint64_t rows = std::min<uint64_t>(c->count + 1, c->capacity);
        if (!ensure_kv_rows(m, d, rows) || !ensure_rope_rows(m, m->ropes[d.rope], rows)) return -1;
        m->params_host->count[i] = (uint32_t)c->count;
    }
    if (plan.special && (!ensure_prompt(m, model, 1) || !ensure_window_scratch(m, model))) return -1;
    m->params_host->token = (uint32_t)token;
    m->params_host->tokens = 1;
    // A fresh tag per step (never 0, the flags' initial value).
    if (++m->step_tag == 0) m->step_tag = 1;
    m->params_host->step = m->step_tag;
    *m->status_host = 0;
    plan.direct = m->host_direct && !plan.special;
    bool short_ctx = true;
    for (uint64_t i = 0; i < L && short_ctx; ++i)
        short_ctx = model->layers[i]->mixer->cache->count + 1 <= kDecodeShortRows;
    plan.row_cap = short_ctx ? kDecodeShortRows : 0;
    int dispatches = 0;
    begin_timing(m);
    if (plan.special || m->eager_decode) {
        if (!encode_decode(m, model, plan, &dispatches)) return fail(m);
    } else {
        hipGraphExec_t &g = short_ctx ? m->graph_short : m->graph;
        uint64_t &g_epoch = short_ctx ? m->graph_short_epoch : m->graph_epoch;
        int &g_dispatches = short_ctx ? m->graph_short_dispatches : m->graph_dispatches;
        if (!g || g_epoch != m->epoch) {
            if (g) (void)hipGraphExecDestroy(g);
            g = nullptr;
            hipGraph_t graph = nullptr;
            int ok = hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal) == hipSuccess;
            int encoded = ok && encode_decode(m, model, plan, &dispatches);
            ok = hipStreamEndCapture(m->stream, &graph) == hipSuccess && encoded && graph;
            ok = ok && hipGraphInstantiate(&g, graph, nullptr, nullptr, 0) == hipSuccess;
            if (graph) (void)hipGraphDestroy(graph);
            if (!ok) {
                (void)hipGetLastError();
                g = nullptr;
                problem(m, "cannot capture the decode graph");
                return fail(m);
            }
            g_epoch = m->epoch;
            g_dispatches = dispatches;
        }
        dispatches = g_dispatches;
        if (hipGraphLaunch(g, m->stream) != hipSuccess) {
            (void)hipGetLastError();
            problem(m, "decode graph launch failed");
            return fail(m);
        }
    }
    if (!end_timing(m)) return fail(m);
    m->info.dispatches += dispatches;
    if (device_failed(m)) return fail(m);
    // Host mirror (runtime/metal_model.m:491-500); a direct step has written
    // logits, state, normalized and the new rows in place already.
    const float *out = m->outbox_host;
    if (!plan.direct) {
        memcpy(model->logits, out, V * 4);
        memcpy(model->state, out + V, h * 4);
        memcpy(model->normalized, out + V + h, h * 4);
    }
    const float *stage = out + V + 2 * h;
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        struct mixer *mx = model->layers[i]->mixer;
        struct cache *c = mx->cache;
        struct rotation *r = mx->rotation;
        const float *st = stage + i * 3 * m->max_width;
        uint64_t row = c->count;
        if (plan.shift[i]) {
            memmove(c->k, c->k + c->width, (c->capacity - 1) * c->width * 4);
            memmove(c->v, c->v + c->width, (c->capacity - 1) * c->width * 4);
            row = c->capacity - 1;
        }
        if (!plan.direct) {
            memcpy(c->k + row * c->width, st, c->width * 4);
            memcpy(c->v + row * c->width, st + c->width, c->width * 4);
        }
        uint64_t count = row + 1;
        if (plan.shift[i] || plan.stale[i]) {
            if (hipMemcpy(r->out, d.rot, count * c->width * 4, hipMemcpyDeviceToHost) != hipSuccess) {
                problem(m, "cannot mirror rotated keys");
                return fail(m);
            }
        } else if (!plan.direct) {
            memcpy(r->out + row * c->width, st + 2 * c->width, c->width * 4);
        }
        c->count = count;
        r->processed_count = count;
        r->scale_bits = float_bits(model->scales[i]);
    }
    remember(m, model);
    ++m->info.fused_decodes;
    m->info.fused_mlps += L;
    return 1;
}

}  // extern "C"

namespace {

// Layer-major prompt processing shared by prefill (verify == false) and
// candidate verification (verify == true). Returns 1, 0 (declined, nothing
// changed) or -1.
int run_prompt(plamo_metal *m, struct model *model, const uint32_t *ids, uint64_t T,
               float *states, bool verify) {
    m->verification_tokens = 0;
    for (Layer &l : m->layers) l.verify_stale = false;
    if (!model || !ids || !T) return -1;
    if (m->config.memory == PLAMO_METAL_STREAM || T > kMaxPrompt) return 0;
    for (uint64_t t = 0; t < T; ++t)
        if (ids[t] >= model->vocab) return -1;
    if (!prepare(m, model)) return -1;
    const uint64_t L = model->count, h = model->hidden, V = model->vocab;
    for (uint64_t i = 0; i < L; ++i) {
        const struct cache *c = model->layers[i]->mixer->cache;
        if (c->count > c->capacity || (!c->sliding && T > c->capacity - c->count)) return -1;
    }
    if (!resolve_layers(m, model)) return 0;
    std::vector<char> stale;
    if (!sync_from_host(m, model, stale, !verify)) return -1;
    if (!ensure_prompt(m, model, T) || !ensure_window_scratch(m, model)) return -1;
    // Planes room for the widest projection input, and for the gate/up
    // GEMM's input and activation planes side by side.
    const GemmWorkspace *ws = gemm_workspace(
        m, T, std::max({h, m->max_attention, m->max_inter, gemm_swiglu_cols(h, m->max_inter)}));
    if (!ws) return -1;
    if (verify && !m->v_state && !alloc_verify(m, L, h, V)) return -1;
    std::vector<char> overflow(L, 0);
    uint64_t split_floats = 0;
    for (uint64_t i = 0; i < L; ++i) {
        const Layer &d = m->layers[i];
        const struct cache *c = model->layers[i]->mixer->cache;
        const uint32_t window = c->count + T > c->capacity ? (uint32_t)c->capacity : 0;
        split_floats = std::max(split_floats,
                                prompt_attention_scratch((uint32_t)c->count, (uint32_t)T, d.qh,
                                                         d.kh, d.dim, window));
    }
    if (split_floats && !ensure(m, m->p_attn_split, split_floats * 4)) return -1;
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        const struct cache *c = model->layers[i]->mixer->cache;
        overflow[i] = c->count + T > c->capacity;
        uint64_t rows = std::min<uint64_t>(c->count + T, c->capacity);
        if (!ensure_kv_rows(m, d, rows) || !ensure_rope_rows(m, m->ropes[d.rope], rows)) return -1;
        m->params_host->count[i] = (uint32_t)c->count;
    }
    m->params_host->tokens = (uint32_t)T;
    *m->status_host = 0;
    memcpy(m->ids_host, ids, T * 4);
    hipStream_t s = m->stream;
    int n = 0;
    begin_timing(m);
    HIP_FAIL(m, hipMemcpyAsync(m->params_dev, m->params_host, sizeof(StepParams),
                              hipMemcpyHostToDevice, s));
    HIP_FAIL(m, hipMemcpyAsync(m->p_ids.ptr, m->ids_host, T * 4, hipMemcpyHostToDevice, s));
    float *state = as<float>(m->p_state), *norm = as<float>(m->p_norm), *qkv = as<float>(m->p_qkv),
          *q = as<float>(m->p_q), *attn = as<float>(m->p_attn), *branch = as<float>(m->p_branch),
          *gu = as<float>(m->p_gu), *act = as<float>(m->p_act);
    HIP_FAIL(m, launch_embed(s, m->embedding, as<uint32_t>(m->p_ids), nullptr, (uint32_t)T,
                            (uint32_t)h, state));
    ++n;
    // A residual followed by a norm of the same rows runs as one launch; then
    // `normed` says the next layer's input norm is already in `norm`.
    const bool fuse_rows = h <= 8192;
    bool normed = false, final_normed = false;
    // Prompts past 16 tokens take the matrix-core GEMM, which reads X as
    // three BF16 planes: the norms that feed QKV and gate/up write them as
    // they write their rows, so those projections skip their own split.
    // qkv_planes: the planes of the next QKV input are already written.
    uint16_t *const planes = ws->planes;
    bool qkv_planes = false;
    // Host-mirror copies of finished layers' cache rows not yet enqueued.
    struct MirrorRows {
        float *host;
        const float *dev;
        uint64_t bytes;
    };
    constexpr uint64_t kMirrorLayers = 4;
    std::vector<MirrorRows> mirror;
    mirror.reserve(3 * kMirrorLayers);
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        const struct cache *c = model->layers[i]->mixer->cache;
        const uint16_t *pre = d.norms, *post = d.norms + h, *mpre = d.norms + 2 * h,
                       *mpost = d.norms + 3 * h, *qn = d.norms + 4 * h, *kn = qn + d.dim;
        const RopeTable &rope = m->ropes[d.rope];
        const uint64_t qkv_w = (uint64_t)(d.qh + 2 * d.kh) * d.dim, aw = (uint64_t)d.qh * d.dim;
        if (!normed) {
            const uint32_t tp = gemm_planes_rows(T, h, ws);
            HIP_FAIL(m, launch_norm_rows(s, state, h, pre, 1.0f, norm, h, h, T, tp ? planes : nullptr,
                                         tp));
            qkv_planes = tp != 0;
            ++n;
        }
        normed = false;
        HIP_FAIL(m, launch_gemm(s, norm, h, d.qkv, qkv_w, h, T, qkv, qkv_w, ws, qkv_planes));
        qkv_planes = false;
        ++n;
        if (m->upload_pending) {  // cached rows are read from here on
            HIP_FAIL(m, hipStreamWaitEvent(s, m->upload_event, 0));
            m->upload_pending = false;
        }
        if (stale[i] && (verify || !overflow[i])) {
            HIP_FAIL(m, launch_rerotate(s, d.k, d.rot, rope.table, c->count, d.kh, d.dim));
            d.verify_stale = verify;
            ++n;
        }
        float *prop_k = nullptr, *prop_v = nullptr, *prop_r = nullptr;
        if (verify) {  // [layer][K, V, rotated K][T][width]
            prop_k = m->v_prop + ((i * 3 + 0) * T) * m->max_width;
            prop_v = m->v_prop + ((i * 3 + 1) * T) * m->max_width;
            prop_r = m->v_prop + ((i * 3 + 2) * T) * m->max_width;
        }
        QkvPost qp{};
        qp.qkv = qkv;
        qp.q_out = q;
        qp.qn = qn;
        qp.kn = kn;
        qp.table = rope.table;
        qp.params = m->params_dev;
        qp.layer = (uint32_t)i;
        qp.qh = d.qh;
        qp.kh = d.kh;
        qp.dim = d.dim;
        qp.tokens = (uint32_t)T;
        qp.capacity = (uint32_t)d.capacity;
        if (verify) {
            qp.k_raw = prop_k;
            qp.v = prop_v;
            qp.k_rot = prop_r;
            qp.rows_from_count = 0;
            qp.rotate_k = 1;
        } else if (overflow[i]) {
            qp.k_raw = as<float>(m->p_side_k);
            qp.v = as<float>(m->p_side_v);
            qp.rows_from_count = 0;
            qp.rotate_k = 0;
        } else {
            qp.k_raw = d.k;
            qp.v = d.v;
            qp.k_rot = d.rot;
            qp.rows_from_count = 1;
            qp.rotate_k = 1;
        }
        HIP_FAIL(m, launch_qkv_post(s, qp));
        ++n;
        // With states == NULL only the final row feeds the logits; the last
        // layer's projection and MLP run for that row alone
        // (runtime/metal_model.m:761-770).
        const bool last_row_only = !verify && !states && i + 1 == L && T > 1;
        PromptAttention pa{};
        pa.q = q;
        pa.table = rope.table;
        pa.out = attn;
        pa.prefix = (uint32_t)c->count;
        pa.tokens = (uint32_t)T;
        pa.partial = split_floats ? as<float>(m->p_attn_split) : nullptr;
        pa.qh = d.qh;
        pa.kh = d.kh;
        pa.dim = d.dim;
        // The O projection over every row reads the attention output as BF16
        // planes, written by the attention itself.
        const uint32_t o_tp =
            !last_row_only && !overflow[i] &&
                    prompt_attention_writes_planes(d.dim, d.qh, d.kh, 0)
                ? gemm_planes_rows(T, aw, ws)
                : 0;
        pa.planes = o_tp ? planes : nullptr;
        pa.padded = o_tp;
        if (overflow[i]) {
            pa.k_cache = d.k;
            pa.v_cache = d.v;
            pa.k_new = verify ? prop_k : as<float>(m->p_side_k);
            pa.v_new = verify ? prop_v : as<float>(m->p_side_v);
            pa.window = (uint32_t)d.capacity;
        } else {
            pa.k_cache = d.rot;
            pa.v_cache = d.v;
            pa.k_new = verify ? prop_r : d.rot + c->count * d.width;
            pa.v_new = verify ? prop_v : d.v + c->count * d.width;
            pa.window = 0;
        }
        HIP_FAIL(m, launch_prompt_attention(s, pa));
        ++n;
        if (overflow[i] && !verify) {
            HIP_FAIL(m, launch_window_store(s, d.k, d.v, d.rot, as<float>(m->p_side_k),
                                           as<float>(m->p_side_v), d.width, rope.table,
                                           as<float>(m->p_window), c->count, T, d.capacity, d.kh,
                                           d.dim));
            n += 2;
        }
        if (!verify) {
            // This layer's cache rows are final: they cross to the host arrays
            // on the copy stream while the later layers compute (the appended
            // rows, the whole window after a sliding shift, and rotations the
            // device rebuilt). One event covers kMirrorLayers layers, except
            // for the last kMirrorLayers layers, whose copies would otherwise
            // run after the prompt's last launch: each event recorded on the
            // stream held the next launch back by about 7 us (C4, 116 tokens).
            const uint64_t first = overflow[i] ? 0 : c->count;
            const uint64_t end = std::min<uint64_t>(c->count + T, c->capacity);
            const uint64_t rot_first = (overflow[i] || stale[i]) ? 0 : first, w = d.width * 4;
            const struct mixer *mx = model->layers[i]->mixer;
            mirror.push_back(MirrorRows{c->k + first * d.width, d.k + first * d.width,
                                        (end - first) * w});
            mirror.push_back(MirrorRows{c->v + first * d.width, d.v + first * d.width,
                                        (end - first) * w});
            mirror.push_back(MirrorRows{mx->rotation->out + rot_first * d.width,
                                        d.rot + rot_first * d.width, (end - rot_first) * w});
            if (mirror.size() == 3 * kMirrorLayers || i + kMirrorLayers >= L) {
                HIP_FAIL(m, hipEventRecord(m->layer_events[i], s));
                HIP_FAIL(m, hipStreamWaitEvent(m->copy_stream, m->layer_events[i], 0));
                for (const MirrorRows &r : mirror)
                    HIP_FAIL(m, hipMemcpyAsync(r.host, r.dev, r.bytes, hipMemcpyDeviceToHost,
                                               m->copy_stream));
                mirror.clear();
            }
        }
        uint64_t first = 0, rows = T;
        if (last_row_only) {
            first = T - 1;
            rows = 1;
        }
        float *st = state + first * h;
        if (rows == 1 && !verify) {
            // One prompt row: the decode GEMVs (norm and SwiGLU fused) instead of
            // GEMM tiles. A one-candidate verify keeps the token GEMVs and the
            // fused residual norms: C5 verify(1) 12.9 against 14.1 ms this way.
            Prologue po{};
            po.src = attn + first * aw;
            HIP_FAIL(m, launch_gemv(s, d.o, h, aw, po, branch, 0, 2 * m->cus));
            HIP_FAIL(m, launch_residual_rows(s, st, branch, post, kAttentionOffset, h, 1));
            Prologue pg{};
            pg.src = st;
            pg.w = mpre;
            pg.offset = 1.0f;
            HIP_FAIL(m, launch_gemv(s, d.gu, 2 * (uint64_t)d.inter, h, pg, act, d.inter, 2 * m->cus));
            Prologue pd{};
            pd.src = act;
            HIP_FAIL(m, launch_gemv(s, d.down, h, d.inter, pd, branch, 0, 2 * m->cus));
            HIP_FAIL(m, launch_residual_rows(s, st, branch, mpost, kMlpOffset, h, 1));
            n += 5;
        } else {
            HIP_FAIL(m, launch_gemm(s, attn + first * aw, aw, d.o, h, aw, rows, branch, h, ws,
                                    o_tp != 0));
            bool gu_planes = false;
            if (fuse_rows) {
                const uint32_t tp = gemm_planes_rows(rows, h, ws);
                HIP_FAIL(m, launch_residual_norm_rows(s, st, branch, post, kAttentionOffset, mpre,
                                                     1.0f, norm, h, h, rows, tp ? planes : nullptr,
                                                     tp));
                gu_planes = tp != 0;
            } else {
                HIP_FAIL(m, launch_residual_rows(s, st, branch, post, kAttentionOffset, h, rows));
                HIP_FAIL(m, launch_norm_rows(s, st, h, mpre, 1.0f, norm, h, h, rows));
                ++n;
            }
            // The activation goes to down's GEMM as BF16 planes only, when
            // that GEMM takes the matrix-core route.
            const uint32_t act_planes = gemm_planes_rows(rows, d.inter, ws);
            uint16_t *act_at = nullptr;
            HIP_FAIL(m, launch_gemm_swiglu(s, norm, h, d.gu, d.inter, h, rows, act, gu, ws,
                                          gu_planes, act_planes, &act_at));
            // Down reads the activation planes where the gate/up launch put them.
            GemmWorkspace down_ws = *ws;
            if (act_planes) {
                down_ws.planes = act_at;
                down_ws.plane_elems = ws->plane_elems - (uint64_t)(act_at - ws->planes);
            }
            HIP_FAIL(m, launch_gemm(s, act, d.inter, d.down, h, d.inter, rows, branch, h,
                                    &down_ws, act_planes != 0));
            if (fuse_rows && i + 1 < L) {
                const uint32_t tp = gemm_planes_rows(rows, h, ws);
                HIP_FAIL(m, launch_residual_norm_rows(s, st, branch, mpost, kMlpOffset,
                                                     m->layers[i + 1].norms, 1.0f, norm, h, h,
                                                     rows, tp ? planes : nullptr, tp));
                normed = true;
                qkv_planes = tp != 0;
            } else if (fuse_rows && verify) {
                HIP_FAIL(m, launch_residual_norm_rows(s, st, branch, mpost, kMlpOffset,
                                                     m->final_norm, 1.0f, m->v_norm, h, h, rows));
                final_normed = true;
            } else {
                HIP_FAIL(m, launch_residual_rows(s, st, branch, mpost, kMlpOffset, h, rows));
            }
            n += act_planes && act_at != ws->planes ? 5 : 6;  // the SwiGLU in gate/up's epilogue
        }
    }
    if (verify) {
        if (!final_normed) HIP_FAIL(m, launch_norm_rows(s, state, h, m->final_norm, 1.0f, m->v_norm, h, h, T));
        HIP_FAIL(m, launch_gemm(s, m->v_norm, h, m->head, V, h, T, m->v_logits, V, ws));
        HIP_FAIL(m, launch_argmax_rows(s, m->v_logits, V, T, m->v_next, m->v_argmax));
        HIP_FAIL(m, hipMemcpyAsync(m->v_state, state, T * h * 4, hipMemcpyDeviceToDevice, s));
        HIP_FAIL(m, hipMemcpyAsync(m->v_host, m->v_state, T * h * 4, hipMemcpyDeviceToHost, s));
        HIP_FAIL(m, hipMemcpyAsync(m->v_host + kMaxVerify * h, m->v_norm, T * h * 4,
                                  hipMemcpyDeviceToHost, s));
        HIP_FAIL(m, hipMemcpyAsync(m->v_host + 2 * kMaxVerify * h, m->v_logits, T * V * 4,
                                  hipMemcpyDeviceToHost, s));
        // The candidates' cache rows reach the host at commit, for the
        // committed candidate only: written in place by the commit's copy
        // kernel when the host arrays are device-visible, else from this copy.
        m->prop_on_host = !m->host_direct;
        if (m->prop_on_host)
            HIP_FAIL(m, hipMemcpyAsync(m->v_host + kMaxVerify * (2 * h + V), m->v_prop,
                                      L * 3 * T * m->max_width * 4, hipMemcpyDeviceToHost, s));
        HIP_FAIL(m, hipMemcpyAsync(m->v_next_host, m->v_next, T * 4, hipMemcpyDeviceToHost, s));
        HIP_FAIL(m, hipMemcpyAsync(m->status_host, &m->params_dev->error, 4, hipMemcpyDeviceToHost, s));
        n += 3;
    } else {
        const float *last = state + (T - 1) * h;
        Prologue ph{};
        ph.src = last;
        ph.w = m->final_norm;
        ph.offset = 1.0f;
        ph.norm_out = m->outbox + V + h;
        ph.status = &m->params_dev->error;
        ph.status_out = m->status_dev;
        HIP_FAIL(m, launch_gemv(s, m->head, V, h, ph, m->outbox, 0, 2 * m->cus));
        HIP_FAIL(m, hipMemcpyAsync(m->outbox + V, last, h * 4, hipMemcpyDeviceToDevice, s));
        HIP_FAIL(m, hipMemcpyAsync(m->outbox_host, m->outbox, (V + 2 * h) * 4,
                                  hipMemcpyDeviceToHost, s));
        ++n;
    }
    if (!end_timing(m)) return fail(m);
    m->info.dispatches += n;
    if (device_failed(m)) return fail(m);
    if (verify) {
        m->verification_tokens = T;
        m->verification_index = 0;
        for (uint64_t i = 0; i < L; ++i) m->layers[i].verify_prefix = model->layers[i]->mixer->cache->count;
        ++m->info.verification_batches;
        m->info.verified_tokens += T;
        return 1;
    }
    // Host mirror: prompt states, final state / normalized / logits, new KV rows.
    if (states && hipMemcpy(states, state, T * h * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        problem(m, "cannot copy prompt states");
        return fail(m);
    }
    memcpy(model->logits, m->outbox_host, V * 4);
    memcpy(model->state, m->outbox_host + V, h * 4);
    memcpy(model->normalized, m->outbox_host + V + h, h * 4);
    if (hipStreamSynchronize(m->copy_stream) != hipSuccess) {
        problem(m, "cannot mirror prompt KV rows");
        return fail(m);
    }
    for (uint64_t i = 0; i < L; ++i) {
        struct mixer *mx = model->layers[i]->mixer;
        struct cache *c = mx->cache;
        struct rotation *r = mx->rotation;
        uint64_t end = std::min<uint64_t>(c->count + T, c->capacity);
        c->count = end;
        r->processed_count = end;
        r->scale_bits = float_bits(model->scales[i]);
    }
    remember(m, model);
    ++m->info.fused_prefills;
    m->info.fused_mlps += L;
    return 1;
}

}  // namespace

extern "C" {

int plamo_metal_prefill(struct plamo_metal *m, struct model *model, const uint32_t *ids,
                        uint64_t tokens, float *states) {
    return run_prompt(m, model, ids, tokens, states, false);
}

int plamo_metal_verify(struct plamo_metal *m, struct model *model, const uint32_t *ids,
                       uint64_t tokens, uint32_t *next) {
    if (!next || !tokens || tokens > PLAMO_VERIFY_MAX) return 0;
    int result = run_prompt(m, model, ids, tokens, nullptr, true);
    if (result == 1) memcpy(next, m->v_next_host, tokens * 4);
    return result;
}

int plamo_metal_commit(struct plamo_metal *m, struct model *model, uint64_t index) {
    if (m->model != model || index != m->verification_index || index >= m->verification_tokens)
        return 0;
    const uint64_t L = model->count, h = model->hidden, V = model->vocab;
    bool full = false;
    for (uint64_t i = 0; i < L; ++i) {
        const struct cache *c = model->layers[i]->mixer->cache;
        uint64_t count = std::min<uint64_t>(m->layers[i].verify_prefix + index, c->capacity);
        if (c->count != count) return 0;
        if (c->count == c->capacity) {
            if (!c->sliding) return 0;
            full = true;
        }
    }
    // Candidate rows were rotated at positions prefix + index; ordinary
    // appends only copy them (runtime/metal_model.m:881-900). A full sliding
    // window is rebased on the device instead.
    const uint64_t T = m->verification_tokens;
    const float *prop_host = m->v_host + kMaxVerify * (2 * h + V);
    uint32_t entries = 0;
    begin_timing(m);
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        const struct cache *c = model->layers[i]->mixer->cache;
        float *pk = m->v_prop + ((i * 3 + 0) * T + index) * m->max_width;
        float *pv = m->v_prop + ((i * 3 + 1) * T + index) * m->max_width;
        float *pr = m->v_prop + ((i * 3 + 2) * T + index) * m->max_width;
        if (c->count < c->capacity) {
            m->copy_table_host[entries++] = CopyRow{pk, d.k + c->count * d.width, d.width};
            m->copy_table_host[entries++] = CopyRow{pv, d.v + c->count * d.width, d.width};
            m->copy_table_host[entries++] = CopyRow{pr, d.rot + c->count * d.width, d.width};
            if (!m->prop_on_host) {
                const uint64_t o = c->count * d.width;
                m->copy_table_host[entries++] = CopyRow{pk, d.host_k + o, d.width};
                m->copy_table_host[entries++] = CopyRow{pv, d.host_v + o, d.width};
                m->copy_table_host[entries++] = CopyRow{pr, d.host_rot + o, d.width};
            }
        } else {
            HIP_FAIL(m, launch_window_store(m->stream, d.k, d.v, d.rot, pk, pv, d.width,
                                           m->ropes[d.rope].table, as<float>(m->p_window),
                                           c->capacity, 1, c->capacity, d.kh, d.dim));
            m->info.dispatches += 2;
        }
    }
    if (entries) {
        HIP_FAIL(m, hipMemcpyAsync(m->copy_table, m->copy_table_host, entries * sizeof(CopyRow),
                                  hipMemcpyHostToDevice, m->stream));
        HIP_FAIL(m, launch_copy_rows(m->stream, m->copy_table, entries));
        ++m->info.dispatches;
    }
    if (!end_timing(m)) return fail(m);
    for (uint64_t i = 0; i < L; ++i) {
        Layer &d = m->layers[i];
        struct mixer *mx = model->layers[i]->mixer;
        struct cache *c = mx->cache;
        struct rotation *r = mx->rotation;
        const float *hk = prop_host + ((i * 3 + 0) * T + index) * m->max_width;
        const float *hv = prop_host + ((i * 3 + 1) * T + index) * m->max_width;
        const float *hr = prop_host + ((i * 3 + 2) * T + index) * m->max_width;
        if (c->count < c->capacity) {
            if (m->prop_on_host) {
                memcpy(c->k + c->count * c->width, hk, c->width * 4);
                memcpy(c->v + c->count * c->width, hv, c->width * 4);
                memcpy(r->out + c->count * c->width, hr, c->width * 4);
            }
            ++c->count;
        } else {
            memmove(c->k, c->k + c->width, (c->capacity - 1) * c->width * 4);
            memmove(c->v, c->v + c->width, (c->capacity - 1) * c->width * 4);
            float *kk = c->k + (c->capacity - 1) * c->width, *vv = c->v + (c->capacity - 1) * c->width;
            if (m->prop_on_host) {
                memcpy(kk, hk, c->width * 4);
                memcpy(vv, hv, c->width * 4);
            } else if (hipMemcpy(kk, m->v_prop + ((i * 3 + 0) * T + index) * m->max_width,
                                 c->width * 4, hipMemcpyDeviceToHost) != hipSuccess ||
                       hipMemcpy(vv, m->v_prop + ((i * 3 + 1) * T + index) * m->max_width,
                                 c->width * 4, hipMemcpyDeviceToHost) != hipSuccess) {
                problem(m, "cannot mirror a committed row");
                return fail(m);
            }
            if (hipMemcpy(r->out, d.rot, c->capacity * c->width * 4, hipMemcpyDeviceToHost) !=
                hipSuccess) {
                problem(m, "cannot mirror rotated keys");
                return fail(m);
            }
        }
        if (d.verify_stale && c->count < c->capacity) {
            if (hipMemcpy(r->out, d.rot, c->count * c->width * 4, hipMemcpyDeviceToHost) !=
                hipSuccess) {
                problem(m, "cannot mirror rotated keys");
                return fail(m);
            }
        }
        d.verify_stale = false;
        r->processed_count = c->count;
        r->scale_bits = float_bits(model->scales[i]);
    }
    (void)full;
    memcpy(model->state, m->v_host + index * h, h * 4);
    memcpy(model->normalized, m->v_host + kMaxVerify * h + index * h, h * 4);
    memcpy(model->logits, m->v_host + 2 * kMaxVerify * h + index * V, V * 4);
    remember(m, model);
    ++m->verification_index;
    ++m->info.committed_tokens;
    return 1;
}

// Lowers every layer's count by `steps` on host and device. The rows below the
// new count are untouched by the undone steps unless a sliding window was full
// (its rows shifted each step), so nothing is uploaded: the shadow is moved
// with the host counts and the next step appends at the lower count. Rotated
// rows stay valid when they were (positions are row indices).
int plamo_hip_rewind(struct plamo_metal *m, struct model *model, uint64_t steps) {
    if (!m || !model) return 0;
    if (!steps) return 1;
    if (m->model != model || m->layers.size() != model->count) return 0;
    for (uint64_t i = 0; i < model->count; ++i) {
        const Layer &d = m->layers[i];
        const struct mixer *mx = model->layers[i]->mixer;
        const struct cache *c = mx->cache;
        if (!d.synced || d.count != c->count || d.processed != mx->rotation->processed_count ||
            d.scale_bits != mx->rotation->scale_bits || c->count < steps ||
            (c->sliding && c->count >= c->capacity))
            return 0;
    }
    m->verification_tokens = 0;
    for (uint64_t i = 0; i < model->count; ++i) {
        struct mixer *mx = model->layers[i]->mixer;
        struct cache *c = mx->cache;
        struct rotation *r = mx->rotation;
        bool rotated = r->processed_count == c->count;
        c->count -= steps;
        if (rotated) {
            r->processed_count = c->count;
        } else {
            r->processed_count = 0;
            r->scale_bits = 0;
        }
        mx->gqa->tokens = c->count;
    }
    remember(m, model);
    return 1;
}

int plamo_metal_linear(struct plamo_metal *m, const struct plamo_matmul *mm) {
    if (!mm || !mm->rows || !mm->columns || !mm->tokens || mm->input_stride < mm->columns ||
        mm->output_stride < mm->rows)
        return 0;
    const uint16_t *w =
        (const uint16_t *)resolve(m, mm->weights, mm->rows * mm->columns * 2);
    if (!w) return 0;
    uint64_t T = mm->tokens, K = mm->columns, N = mm->rows;
    Buffer &in = m->lin_in, &out = m->lin_out;
    if (!ensure(m, in, T * K * 4) || !ensure(m, out, T * N * 4)) return 0;
    if (configure_gemv(K) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int ok = hipMemcpy2DAsync(in.ptr, K * 4, mm->input, mm->input_stride * 4, K * 4, T,
                              hipMemcpyHostToDevice, m->stream) == hipSuccess;
    begin_timing(m);
    if (ok && T == 1) {
        Prologue p{};
        p.src = as<float>(in);
        ok = launch_gemv(m->stream, w, N, K, p, as<float>(out), 0, 2 * m->cus) == hipSuccess;
    } else if (ok) {
        const GemmWorkspace *ws = gemm_workspace(m, T, K);
        ok = ws && launch_gemm(m->stream, as<float>(in), K, w, N, K, T, as<float>(out), N, ws) ==
                       hipSuccess;
    }
    ok = ok && hipMemcpy2DAsync(mm->output, mm->output_stride * 4, out.ptr, N * 4, N * 4, T,
                                hipMemcpyDeviceToHost, m->stream) == hipSuccess;
    ok = ok && end_timing(m);
    if (!ok) {
        (void)hipGetLastError();
        return problem(m, "projection failed");
    }
    ++m->info.dispatches;
    return 1;
}

namespace {

// True when [p, p + bytes) lies inside one device allocation of this GPU
// (hipMalloc memory). Host memory, pinned or not, and pointers the runtime
// does not know are refused. Neither query allocates.
bool device_extent(int device, const void *p, uint64_t bytes) {
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, p) != hipSuccess || a.type != hipMemoryTypeDevice ||
        a.device != device) {
        (void)hipGetLastError();
        return false;
    }
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) != hipSuccess || !base) {
        (void)hipGetLastError();
        return false;
    }
    const uintptr_t b = (uintptr_t)base, q = (uintptr_t)p;
    return q >= b && bytes <= size && q - b <= size - bytes;
}

struct ScratchOwner {
    std::atomic<bool> *flag = nullptr;
    bool take(int device) {
        bool expected = false;
        if (!static_scratch_busy[device].compare_exchange_strong(expected, true)) return false;
        flag = &static_scratch_busy[device];
        return true;
    }
    ~ScratchOwner() {
        if (flag) flag->store(false);
    }
};

}  // namespace

int plamo_hip_linear_static(struct plamo_metal *m, const struct plamo_matmul *mm) {
    if (!m) return 0;
    if (!mm || !mm->input || !mm->output || !mm->rows || !mm->columns || !mm->tokens ||
        mm->input_stride < mm->columns || mm->output_stride < mm->rows)
        return problem(m, "static linear: invalid projection");
    const uint64_t T = mm->tokens, K = mm->columns, N = mm->rows;
    const uint16_t *w = (const uint16_t *)resolve(m, mm->weights, N * K * 2);
    if (!w) return problem(m, "static linear: weights not resident");
    char *base = m->device < kMaxDevices ? (char *)static_scratch[m->device] : nullptr;
    if (!base) return problem(m, "static linear: no static scratch on this device");
    // Kernels read the input and write the output directly: both must be
    // device memory of this GPU spanning every row the strides reach (a host
    // pointer would fault the GPU).
    if (!device_extent(m->device, mm->input, ((T - 1) * mm->input_stride + K) * 4) ||
        !device_extent(m->device, mm->output, ((T - 1) * mm->output_stride + N) * 4))
        return problem(m, "static linear: input and output must be device memory of this GPU "
                          "covering every strided row");
    ScratchOwner owner;
    if (!owner.take(m->device))
        return problem(m, "static linear: the static scratch of this GPU is in use by another "
                          "call");
    if (T > 1 && gemm_plane_elems(T, K) * 2 > PLAMO_HIP_STATIC_PLANE_BYTES)
        return problem(m,
                       "static linear: %llu tokens x %llu columns need %llu bytes of input "
                       "planes, above the static scratch's %llu",
                       (unsigned long long)T, (unsigned long long)K,
                       (unsigned long long)(gemm_plane_elems(T, K) * 2),
                       (unsigned long long)PLAMO_HIP_STATIC_PLANE_BYTES);
    if (configure_gemv(K) != hipSuccess) {
        (void)hipGetLastError();
        return problem(m, "static linear: %llu columns exceed the LDS budget",
                       (unsigned long long)K);
    }
    GemmWorkspace ws{};
    ws.counter_base = (uint32_t *)base;
    ws.counters = kGemmCounters;
    ws.partial = (float *)(base + kStaticCounterBytes);
    ws.partial_floats = kGemmPartialFloats;
    ws.planes = (uint16_t *)(base + kStaticCounterBytes + kStaticPartialBytes);
    ws.plane_elems = PLAMO_HIP_STATIC_PLANE_BYTES / 2;
    ws.cus = (uint32_t)m->cus;
    const float *x = (const float *)mm->input;
    float *y = mm->output;
    hipStream_t s = m->stream;
    begin_timing(m);
    // The previous call on this GPU may have ended without leaving the
    // counters at zero (a failed launch): clear them first.
    bool ok = launch_fill(s, ws.counter_base, kGemmCounters, 0) == hipSuccess;
    if (ok && T == 1) {
        Prologue p{};
        p.src = x;
        ok = launch_gemv(s, w, N, K, p, y, 0, 2 * m->cus) == hipSuccess;
    } else if (ok) {
        ok = launch_gemm(s, x, mm->input_stride, w, N, K, T, y, mm->output_stride, &ws) ==
             hipSuccess;
    }
    ok = ok && end_timing(m);
    if (!ok) {
        // Nothing of this call may still run when the scratch is released.
        (void)hipStreamSynchronize(s);
        (void)hipGetLastError();
        return problem(m, "static linear: launch failed");
    }
    m->info.dispatches += 2;
    return 1;
}

int plamo_metal_mlp(struct plamo_metal *m, const struct mlp *mlp, float *states, uint64_t tokens) {
    if (!mlp || !states || !tokens || !mlp->hidden || !mlp->intermediate) return 0;
    uint64_t h = mlp->hidden, I = mlp->intermediate, T = tokens;
    const uint16_t *gu = (const uint16_t *)resolve(m, mlp->gu, 2 * I * h * 2);
    const uint16_t *down = (const uint16_t *)resolve(m, mlp->down, I * h * 2);
    if (!gu || !down) return 0;
    if (configure_gemv(std::max<uint64_t>(h, I)) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    Buffer &st = m->mlp_state, &nrm = m->mlp_norm, &g = m->mlp_gu, &a = m->mlp_act,
           &b = m->mlp_branch, &norms = m->mlp_norms;
    const GemmWorkspace *ws = gemm_workspace(m, T, std::max(h, I));
    bool ok = ws && ensure(m, st, T * h * 4) && ensure(m, nrm, T * h * 4) &&
              ensure(m, g, T * 2 * I * 4) && ensure(m, a, T * I * 4) && ensure(m, b, T * h * 4) &&
              ensure(m, norms, 2 * h * 2);
    hipStream_t s = m->stream;
    ok = ok && hipMemcpyAsync(norms.ptr, mlp->pre, h * 2, hipMemcpyHostToDevice, s) == hipSuccess &&
         hipMemcpyAsync(as<uint16_t>(norms) + h, mlp->post, h * 2, hipMemcpyHostToDevice, s) ==
             hipSuccess &&
         hipMemcpyAsync(st.ptr, states, T * h * 4, hipMemcpyHostToDevice, s) == hipSuccess;
    if (ok) begin_timing(m);
    ok = ok && launch_norm_rows(s, as<float>(st), h, as<uint16_t>(norms), 1.0f, as<float>(nrm), h, h, T) == hipSuccess &&
         launch_gemm_swiglu(s, as<float>(nrm), h, gu, I, h, T, as<float>(a), as<float>(g), ws) == hipSuccess &&
         launch_gemm(s, as<float>(a), I, down, h, I, T, as<float>(b), h, ws) == hipSuccess &&
         launch_residual_rows(s, as<float>(st), as<float>(b), as<uint16_t>(norms) + h, kMlpOffset, h, T) == hipSuccess &&
         hipMemcpyAsync(states, st.ptr, T * h * 4, hipMemcpyDeviceToHost, s) == hipSuccess &&
         end_timing(m);
    if (!ok) {
        (void)hipGetLastError();
        return problem(m, "MLP failed");
    }
    m->info.dispatches += 5;
    ++m->info.fused_mlps;
    return 1;
}

}  // extern "C"

extern "C" void plamo_hip_invalidate(struct plamo_metal *m) {
    if (!m) return;
    for (Layer &l : m->layers) l.synced = false;
}

extern "C" void plamo_hip_debug_waits(struct plamo_metal *m, uint32_t extra, uint32_t polls) {
    if (!m) return;
    m->params_host->wait_extra = extra;
    m->params_host->wait_limit = polls;
}

extern "C" int plamo_hip_time_kernel(struct plamo_metal *m, struct model *model, uint64_t layer,
                                     int which, int reps, double *ms_per_launch,
                                     double *bytes_per_launch) {
    if (!m || m->model != model || !model || layer >= model->count || reps < 1 ||
        !ms_per_launch || !bytes_per_launch || !resolve_layers(m, model))
        return 0;
    const uint64_t h = model->hidden;
    Layer &d = m->layers[layer];
    const int blocks = 2 * m->cus;
    hipStream_t s = m->stream;
    double bytes = 0;
    // Same arguments as the decode graph uses for this kernel.
    auto launch = [&]() -> hipError_t {
        Prologue p{};
        switch (which) {
        case PLAMO_HIP_QKV:
            p.src = m->state_a;
            p.w = d.norms;
            p.offset = 1.0f;
            if (layer) {
                // After the first layer the prologue also adds the previous
                // layer's MLP branch (the decode step's state buffers are
                // rewritten from the embedding at every step).
                p.branch = m->down_out;
                p.rw = m->layers[layer - 1].norms + 3 * h;
                p.roffset = kMlpOffset;
                p.state_out = m->state_b;
            }
            return launch_gemv(s, d.qkv, (uint64_t)(d.qh + 2 * d.kh) * d.dim, h, p, m->qkv, 0,
                               blocks);
        case PLAMO_HIP_O:
            p.src = m->attn;
            return launch_gemv(s, d.o, h, (uint64_t)d.qh * d.dim, p, m->branch, 0, blocks);
        case PLAMO_HIP_GATE_UP:
            p.src = m->state_a;
            p.w = d.norms + 2 * h;
            p.offset = 1.0f;
            p.branch = m->branch;
            p.rw = d.norms + h;
            p.roffset = kAttentionOffset;
            p.state_out = m->state_b;
            return launch_gemv(s, d.gu, 2 * (uint64_t)d.inter, h, p, m->act, d.inter, blocks);
        case PLAMO_HIP_DOWN:
            p.src = m->act;
            return launch_gemv(s, d.down, h, d.inter, p, m->down_out, 0, blocks);
        case PLAMO_HIP_HEAD:
            p.src = m->state_a;
            p.w = m->final_norm;
            p.offset = 1.0f;
            return launch_gemv(s, m->head, model->vocab, h, p, m->outbox, 0, blocks);
        default: {
            if (!d.fused) return hipErrorInvalidValue;
            DecodeAttention da{};
            da.qkv = m->qkv;
            da.qn = d.norms + 4 * h;
            da.kn = d.norms + 4 * h + d.dim;
            da.freq = m->ropes[d.rope].freq_dev;
            memcpy(&da.rope_scale, &m->ropes[d.rope].scale_bits, 4);
            da.k_raw = d.k;
            da.rows = (uint32_t)d.rows;
            da.v = d.v;
            da.k_rot = d.rot;
            da.stage = nullptr;
            da.out = m->attn;
            da.partial = m->partial;
            da.counters = m->counters;
            da.params = m->params_dev;
            da.layer = (uint32_t)layer;
            da.qh = d.qh;
            da.kh = d.kh;
            da.dim = d.dim;
            da.splits = decode_attention_splits(d.rows);
            return launch_decode_attention(s, da);
        }
        }
    };
    switch (which) {
    case PLAMO_HIP_QKV: bytes = 2.0 * (d.qh + 2 * d.kh) * d.dim * h; break;
    case PLAMO_HIP_O: bytes = 2.0 * h * d.qh * d.dim; break;
    case PLAMO_HIP_GATE_UP: bytes = 2.0 * 2 * d.inter * h; break;
    case PLAMO_HIP_DOWN: bytes = 2.0 * d.inter * h; break;
    case PLAMO_HIP_HEAD: bytes = 2.0 * model->vocab * h; break;
    case PLAMO_HIP_ATTENTION: {
        // Rows the kernel reads: the count stored for this layer by the last step.
        uint64_t rows = (uint64_t)m->params_host->count[layer] + 1;
        bytes = 2.0 * 4.0 * rows * d.width;
        break;
    }
    default: return 0;
    }
    if (launch() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
        (void)hipGetLastError();
        return problem(m, "timed launch failed");
    }
    HIP_TRY(m, hipEventRecord(m->start, s));
    for (int i = 0; i < reps; ++i)
        if (launch() != hipSuccess) {
            (void)hipGetLastError();
            return problem(m, "timed launch failed");
        }
    HIP_TRY(m, hipEventRecord(m->stop, s));
    HIP_TRY(m, hipEventSynchronize(m->stop));
    float ms = 0;
    HIP_TRY(m, hipEventElapsedTime(&ms, m->start, m->stop));
    *ms_per_launch = ms / reps;
    *bytes_per_launch = bytes;
    // The attention kernel re-appended this layer's last row from whatever the
    // QKV buffer now holds: upload the host rows again at the next call.
    if (which == PLAMO_HIP_ATTENTION) d.synced = false;
    return 1;
}
