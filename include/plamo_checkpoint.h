/* Real PLaMo-3 checkpoints on Linux.
 *
 * The reference binds its weights from the original safetensors shards with
 * AArch64 assembly (src/load.s, src/json.s, src/tensor.s, src/find.s,
 * src/resolve.s, src/bind.s, src/model_open.s) and bakes the model's shape
 * into generated assembly (tools/weight_schema.py, tools/model_layout.py,
 * tools/rope_constants.py). This header restates that binder in C with the
 * same entry points and results, and evaluates the schema and descriptor
 * layout at run time from the checkpoint's config.json, so a Linux host can
 * open any profile (tools/profiles/{0.8b,2b,8b,31b}) without a generation
 * step. Tensors stay where the shards are mapped (no conversion, no copy);
 * plamo_metal_open() uploads them to HBM unchanged.
 */
#ifndef PLAMO_CHECKPOINT_H
#define PLAMO_CHECKPOINT_H
#include <stddef.h>

#include "plamo_model.h"
#include "plamo_synthetic.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- safetensors primitives (tests/load.c:4-13, tests/find.c:4-7) ---- */

struct plamo_safetensors_view {
    const char *header;
    uint64_t header_size;
    const void *data;
    uint64_t data_size;
};
struct plamo_number {
    const char *next;
    uint64_t value;
};
/* src/json.s:2: {next, start, length, value}; strings exclude the quotes and
 * keep escapes raw. */
struct plamo_json_token {
    const char *next;
    const char *start;
    uint64_t length;
    uint64_t value;
};
enum { PLAMO_JSON_END = 0, PLAMO_JSON_STRING = 256, PLAMO_JSON_UINT = 257, PLAMO_JSON_BAD = -1 };
/* src/tensor.s:3: {next, offset, byte_length, rank, dimensions[4]}. */
struct plamo_tensor_field {
    const char *next;
    uint64_t offset, bytes, rank, dims[4];
};
/* src/find.s:3: {data, bytes, rank, dimensions[4], reserved}. */
struct plamo_tensor {
    const uint16_t *data;
    uint64_t bytes, rank, dims[4], reserved;
};

/* src/load.s:3-44 (_plamo_safetensors_view): validates the envelope (an
 * 8-byte little-endian header length n with 2 <= n <= 100 MB and n <= size - 8,
 * a header that opens with '{' and, before trailing spaces, closes with '}')
 * without touching tensor data. 1 on success; 0 clears the output. */
int plamo_safetensors_view(const void *file, uint64_t size, struct plamo_safetensors_view *out);
/* src/load.s:46-80 (_plamo_parse_u64): a JSON unsigned integer in [p, end)
 * (no sign, no leading zero, no overflow). 0 clears the output. */
int plamo_parse_u64(const char *p, const char *end, struct plamo_number *out);
/* src/json.s:7 (_plamo_json_next): the next token of a restricted JSON lexer:
 * ASCII punctuation ({ } [ ] : ,), PLAMO_JSON_STRING, PLAMO_JSON_UINT,
 * PLAMO_JSON_END, or PLAMO_JSON_BAD. */
int plamo_json_next(const char *p, const char *end, struct plamo_json_token *out);
/* src/tensor.s:18 (_plamo_tensor_descriptor): one tensor's object, fields in
 * any order and each exactly once: "dtype" must be "BF16", "shape" at most 4
 * dimensions, "data_offsets" [b, e] with b <= e <= data_bytes and e - b equal
 * to 2 bytes per element. Any other key fails. 0 clears the output. */
int plamo_tensor_descriptor(const char *p, const char *end, uint64_t data_bytes,
                            struct plamo_tensor_field *out);
/* src/find.s:11 (_plamo_find_tensor): the tensor named exactly `name` in one
 * mapped safetensors file (string-to-string "__metadata__" skipped). 1 when
 * found; 0 (output cleared) when absent or when the header is invalid up to it. */
int plamo_find_tensor(const void *file, uint64_t size, const char *name, struct plamo_tensor *out);
/* src/resolve.s:6 (_plamo_resolve_weight): the first shard holding `name`
 * decides; its rank and dimensions must equal the expected ones. Rank <= 4.
 * The BF16 data pointer, or NULL. */
const uint16_t *plamo_resolve_weight(const struct plamo_mapping *shards, uint64_t count,
                                     const char *name, uint64_t rank, const uint64_t *dims);
/* src/bind.s:5 (_plamo_bind_weights): resolves every entry of a schema
 * terminated by a NULL name into its slot. 1 when all resolve; otherwise 0
 * with every slot cleared. */
int plamo_bind_weights(const struct plamo_mapping *shards, uint64_t count,
                       struct plamo_weight_spec *schema);

/* ---- checkpoints (no reference counterpart as an API: the reference
 * generates these tables at build time from the same config.json) ---- */

/* The fields of config.json the layout reads (tools/weight_schema.py:15-44,
 * tools/model_layout.py:71-199, tools/rope_constants.py:21-76). */
struct plamo_checkpoint_config {
    uint64_t hidden, layers, qh, kh, dim, intermediate, vocab;
    uint64_t window;                 /* window_size */
    uint64_t pattern;                /* sliding_window_pattern */
    uint64_t max_positions;          /* max_position_embeddings */
    int tied;                        /* tie_word_embeddings */
    double local_theta;              /* rope_parameters.sliding_attention.rope_theta */
    int global_yarn;                 /* full_attention.rope_type == "yarn" */
    double global_theta, factor, original, beta_fast, beta_slow;
};

struct plamo_checkpoint;

/* Opens a checkpoint directory: reads config.json, maps every *.safetensors
 * shard read-only (sorted by name), binds the schema of tools/weight_schema.py
 * (the head is the embedding when tied) and derives the RoPE tables. Global
 * layers get min(max_positions, global_capacity) rows (0: 8192, the engine's
 * 4096 + 4096 request limit, runtime/engine.c:432-448). NULL with a message. */
struct plamo_checkpoint *plamo_checkpoint_open(const char *directory, uint64_t global_capacity,
                                               char *error, size_t cap);
void plamo_checkpoint_close(struct plamo_checkpoint *);
const struct plamo_checkpoint_config *plamo_checkpoint_config(const struct plamo_checkpoint *);
/* The shard mappings (for plamo_metal_config.maps) and their count. */
const struct plamo_mapping *plamo_checkpoint_mappings(const struct plamo_checkpoint *,
                                                      size_t *count);
/* The bound schema, terminated by a NULL name (for plamo_metal_config.schema). */
const struct plamo_weight_spec *plamo_checkpoint_schema(const struct plamo_checkpoint *);
/* A model instance over the checkpoint's weights (descriptors, workspace, KV
 * caches); released with plamo_synthetic_release(). */
struct plamo_synthetic_instance *plamo_checkpoint_instantiate(const struct plamo_checkpoint *,
                                                              int pinned, char *error, size_t cap);

/* ---- the engine's model globals (declared in plamo_model.h) ----
 * plamo_model_open() opens the directory set by plamo_model_set_directory(), or
 * else $PLAMO_MODEL_DIR, and fills plamo_model, the weight tables, the schema
 * (at most PLAMO_MAX_SCHEMA entries with its terminator) and the patch table.
 * plamo_model_set_directory() also sets the profile strings at once (the
 * engine opens the tokenizer before the model, runtime/engine.c:113); 0 when
 * the path is too long or a model is already open. */
enum { PLAMO_MAX_SCHEMA = 3 + 10 * 128 + 1 };
int plamo_model_set_directory(const char *directory);

#ifdef __cplusplus
}
#endif
#endif
