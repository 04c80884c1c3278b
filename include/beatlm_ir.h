/*
 * The host side above the backend's C ABI: a C++ restatement of the parts of
 * the reference's core (Rust, crates/beatlm-core) that produce and consume
 * kernel specs for the ViT encoder block, and of its graph builder for the
 * block (crates/beatlm/src/model/depth_anything_v2.rs), behind a C API.
 *
 *   reference                                         here
 *   ------------------------------------------------  -------------------------------
 *   Graph::{new, tensor, push}   kernel.rs:1137-1245  bli_graph_new/_tensor/_push
 *   OpKind::output_elements      kernel.rs:977-1005   bli_op_output_elements
 *   Graph::lower(Fusion)         kernel.rs:1285-1343  bli_graph_lower
 *   Program::split(parts)        kernel.rs:2384-2408  bli_program_split
 *   Program::parts_within        kernel.rs:2350-2366  bli_program_parts_within
 *   Program::tensors / role      kernel.rs:2415-2425  bli_program_tensors / _role
 *   Program::stand_in            kernel.rs:2427-2451  bli_program_stand_in
 *   KernelSpec::{name, bindings, part, max_parts, output_range, epilogue}
 *                                kernel.rs:1911-2115  bli_program_kernel / _kernel_name
 *   MemoryPlan::new / placement / arenas / peak_live_bytes / total_bytes / valid_on
 *                                memory.rs:285-429    bli_plan_*
 *   block() / layer_of           depth_anything_v2.rs:252-424  bli_vit_block
 *   encoder() (embeddings)       depth_anything_v2.rs:435-498  bli_vit_embeddings
 *
 * plus one backend-level rewrite with no reference counterpart,
 * bli_program_fuse_attention: attention_scores+scale -> softmax ->
 * attention_values over one qkv tensor becomes one flash-attention kernel, and
 * the two [T][H][T] tensors leave the program (and so the memory plan).
 *
 * Errors: negative codes, the variants of KernelError (kernel.rs:2453-2576)
 * and PlanError (memory.rs:190-245); bli_last_error() gives the message of
 * the last failure on the calling thread.
 */
#ifndef BEATLM_IR_H
#define BEATLM_IR_H

#include <stdint.h>

#include "beatlm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

#define BLI_NONE 0xffffffffu

enum { BLI_INPUT = 0, BLI_WEIGHT = 1, BLI_ACTIVATION = 2, BLI_OUTPUT = 3 }; /* TensorRole */
enum { BLI_FUSION_ON = 0, BLI_FUSION_OFF = 1 };                              /* Fusion */

/* OpKind (kernel.rs:818-916): the encoder block's variants and the DPT head's. */
enum {
    BLI_OP_CONV3X3 = 9,          /* t: image, weights [3][3][cin][cout], bias|NONE; d: height, width, cin, cout, stride */
    BLI_OP_CONV1X1 = 10,         /* t: image, weights [cin][cout], bias|NONE; d: height, width, cin, cout */
    BLI_OP_CONV_TRANSPOSE = 11,  /* t: image, weights [f][f][cin][cout], bias|NONE; d: height, width, cin, cout, factor */
    BLI_OP_RESIZE_BILINEAR = 12, /* t: map; d: in_height, in_width, out_height, out_width, channels */
    BLI_OP_LAYER_NORM = 1,       /* t: input, gamma, beta; d: rows, channels; f: epsilon */
    BLI_OP_MATMUL = 2,           /* t: a, b, bias|NONE; d: m, k, n */
    BLI_OP_ATTENTION_SCORES = 3, /* t: qkv; d: tokens, heads, head_dim */
    BLI_OP_SOFTMAX = 4,          /* t: input; d: rows, cols */
    BLI_OP_ATTENTION_VALUES = 5, /* t: probs, qkv; d: tokens, heads, head_dim */
    BLI_OP_PATCH_EMBED = 6,      /* t: image, weights, bias|NONE; d: grid_h, grid_w, patch, cin, cout */
    BLI_OP_PREPEND_TOKEN = 7,    /* t: token, tokens; d: rows, channels */
    BLI_OP_TOKENS_TO_MAP = 8,    /* t: input; d: height, width, channels */
    BLI_OP_ADD = 20,             /* t: a, b; d: elements */
    BLI_OP_RELU = 21,            /* t: input; d: elements */
    BLI_OP_GELU = 22,            /* t: input; d: elements */
    BLI_OP_GELU_ERF = 23,        /* t: input; d: elements */
    BLI_OP_SCALE = 24,           /* t: input; d: elements; f: factor */
    BLI_OP_CHANNEL_SCALE = 25    /* t: input, scale; d: rows, channels */
};

/* KernelError and PlanError variants. */
enum {
    BLI_ERR_DUPLICATE_TENSOR = -100,
    BLI_ERR_EMPTY_TENSOR = -101,
    BLI_ERR_TENSOR_TOO_LARGE = -102,
    BLI_ERR_UNKNOWN_TENSOR = -103,
    BLI_ERR_ELEMENT_COUNT = -104,
    BLI_ERR_READ_BEFORE_WRITTEN = -105,
    BLI_ERR_WRITTEN_TWICE = -106,
    BLI_ERR_NOT_WRITABLE = -107,
    BLI_ERR_ZERO_DIMENSION = -108,
    BLI_ERR_OP_TOO_LARGE = -109,
    BLI_ERR_NON_FINITE_SCALE = -110,
    BLI_ERR_INVALID_EPSILON = -111,
    BLI_ERR_TOO_MANY_OPS = -112,
    BLI_ERR_EMPTY_GRAPH = -113,
    BLI_ERR_NEVER_WRITTEN = -114,
    BLI_ERR_NOT_INPUT_OR_OUTPUT = -115,
    BLI_ERR_EXCEEDS_LIMIT = -116,
    BLI_ERR_PART_COUNTS = -117,
    BLI_ERR_ALREADY_SPLIT = -118,
    BLI_ERR_ZERO_BOUND = -119,
    BLI_ERR_UNKNOWN_OP = -120,
    /* PlanError */
    BLI_ERR_PLAN_DUPLICATE_TENSOR = -130,
    BLI_ERR_PLAN_INVALID_LIFETIME = -131,
    BLI_ERR_PLAN_EMPTY_TENSOR = -132,
    BLI_ERR_PLAN_SIZE_OVERFLOW = -133,
    BLI_ERR_PLAN_TENSOR_TOO_LARGE = -134,
    BLI_ERR_PLAN_INVALID_PROFILE = -135,
    BLI_ERR_PLAN_TOO_MANY_TENSORS = -136,
    BLI_ERR_NO_PLACEMENT = -137
};

typedef struct {
    uint32_t kind;
    uint32_t t[4];
    uint32_t d[6];
    float f;
} bli_op;

typedef struct {
    uint32_t id;
    uint32_t dtype;      /* BL_F32 / BL_F16 */
    uint64_t elements;
    uint32_t first_use, last_use;
} bli_tensor_desc;

/* The limits the planner and the launch checks read (DeviceProfile). */
typedef struct {
    uint64_t max_storage_buffer_binding_size;
    uint64_t max_buffer_size;
    uint32_t min_storage_buffer_offset_alignment;
    uint32_t max_compute_workgroup_storage_size;
    uint32_t max_compute_invocations_per_workgroup;
    uint32_t max_compute_workgroups_per_dimension;
    uint32_t max_storage_buffers_per_shader_stage;
} bli_profile;

typedef struct {
    uint32_t arena;
    uint32_t reserved;
    uint64_t offset, size;
} bli_placement;

/* One kernel of a program, as KernelSpec's accessors report it. */
typedef struct {
    uint32_t main;          /* BL_MAIN_* */
    uint32_t dims[6];
    float epsilon, scale;
    bl_part part;
    uint32_t max_parts;
    uint32_t tile_rows;     /* the reference tile's rows (the part grain), 0 when untiled */
    uint64_t output_start, output_end;  /* KernelSpec::output_range */
    uint32_t n_reads;
    uint32_t reads[4];      /* binding index of each main-op read */
    uint32_t n_epilogue;
    bl_epilogue epilogue[BL_MAX_EPILOGUE];   /* operand: binding index */
    uint32_t n_bindings;
    uint32_t bindings[BL_MAX_BINDINGS];      /* tensor ids, output last */
    uint32_t first_op, end_op;               /* KernelSpec::ops */
    uint32_t prologue;                       /* BL_PRO_* or 0 */
} bli_kernel_info;

typedef struct bli_graph bli_graph;
typedef struct bli_program bli_program;
typedef struct bli_plan bli_plan;

const char *bli_last_error(void);

/* profiles */
void bli_profile_webgpu_baseline(bli_profile *out); /* device.rs:97-113 */
void bli_profile_mi355x(bli_profile *out);          /* what the HIP backend runs */

/* graph */
int bli_graph_new(bli_graph **out);
void bli_graph_free(bli_graph *g);
int bli_graph_tensor(bli_graph *g, uint32_t id, uint32_t role, uint64_t elements);
int bli_graph_push(bli_graph *g, const bli_op *op, uint32_t output);
uint64_t bli_op_output_elements(const bli_op *op);
uint32_t bli_graph_ops(const bli_graph *g);
int bli_graph_lower(const bli_graph *g, uint32_t fusion, bli_program **out);

/* program */
void bli_program_free(bli_program *p);
int bli_program_split(const bli_program *p, const uint32_t *parts, uint32_t n, bli_program **out);
int bli_program_parts_within(const bli_program *p, const uint64_t *durations_us, uint32_t n,
                             uint64_t bound_us, uint32_t *parts_out);
int bli_program_fuse_attention(const bli_program *p, bli_program **out);
/* Every tensor stored as `dtype` (BL_F16 for the half-precision configurations). */
int bli_program_set_dtype(bli_program *p, uint32_t dtype);
uint32_t bli_program_len(const bli_program *p);
int bli_program_kernel(const bli_program *p, uint32_t k, bli_kernel_info *out);
int bli_program_kernel_name(const bli_program *p, uint32_t k, char *buf, uint32_t cap);
uint32_t bli_program_tensors(const bli_program *p, bli_tensor_desc *out, uint32_t cap);
int bli_program_role(const bli_program *p, uint32_t id);
int bli_program_stand_in(const bli_program *p, uint32_t of, uint32_t id, bli_tensor_desc *out);
/* Kernel k of the program as the backend's spec, its bindings placed by `plan`. */
int bli_program_spec(const bli_program *p, uint32_t k, const bli_plan *plan, bl_spec *out);

/* memory plan */
int bli_plan_new(const bli_tensor_desc *tensors, uint32_t n, const bli_profile *profile, bli_plan **out);
void bli_plan_free(bli_plan *plan);
uint32_t bli_plan_arenas(const bli_plan *plan, uint64_t *sizes, uint32_t cap);
int bli_plan_placement(const bli_plan *plan, uint32_t id, bli_placement *out);
uint64_t bli_plan_peak_live_bytes(const bli_plan *plan);
uint64_t bli_plan_total_bytes(const bli_plan *plan);
int bli_plan_valid_on(const bli_plan *plan, const bli_profile *profile);

/* model: the pre-norm DINOv2 block and the embeddings in front of the blocks */
typedef struct {
    uint32_t tokens, width, heads, mlp;
    float epsilon;
} bli_vit_dims;

/* The weights of one block, in the order the reference's builder declares
 * them (depth_anything_v2.rs:272-330), and its output. */
typedef struct {
    uint32_t norm1_g, norm1_b, qkv_w, qkv_b, proj_w, proj_b, ls1;
    uint32_t norm2_g, norm2_b, fc1_w, fc1_b, fc2_w, fc2_b, ls2;
    uint32_t output;
    uint32_t next_id;   /* the first id the block did not use */
} bli_block_ids;

int bli_vit_block(bli_graph *g, const bli_vit_dims *d, uint32_t x, uint32_t first_id, uint32_t out_role,
                  bli_block_ids *out);

typedef struct {
    uint32_t image, patch_w, patch_b, cls, pos;
    uint32_t output;
    uint32_t next_id;
} bli_embed_ids;

/* patch embedding (p x p, stride p) -> class token -> + positions */
int bli_vit_embeddings(bli_graph *g, uint32_t grid, uint32_t patch, uint32_t channels, uint32_t width,
                       uint32_t first_id, bli_embed_ids *out);

#ifdef __cplusplus
}
#endif
#endif
