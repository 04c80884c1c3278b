/* beatlm_load.h — the model-file side of the backend: a safetensors reader,
 * tensor inventories and their check against a file, the Depth Anything V2
 * inventory, and the conversions from a checkpoint's layouts to the IR's.
 *
 * Replaces, one for one, crates/beatlm/src/load/ and the conversion half of
 * crates/beatlm/src/model/ (mod.rs:140-353, positions.rs): a host that is not
 * Rust reads a checkpoint here and writes the converted numbers into the
 * arenas (bl_arenas_write). Host code only; nothing here touches the GPU.
 *
 * Every call returns BLF_OK or an error code; blf_last_error() is the
 * message of the calling thread's last error.
 */
#ifndef BEATLM_LOAD_H
#define BEATLM_LOAD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* LoadError / ConfigError / ModelError (load/error.rs:11-43,
 * load/depth_anything_v2.rs:254-300, model/mod.rs:52-136). */
enum {
    BLF_OK = 0,
    BLF_ERR_FORMAT = 1,           /* LoadError::Format: not a valid safetensors file */
    BLF_ERR_IO = 2,               /* LoadError::Io: the file cannot be read (message names the path) */
    BLF_ERR_MISSING_TENSOR = 3,   /* LoadError::MissingTensor */
    BLF_ERR_DUPLICATE_NAME = 4,   /* LoadError::DuplicateName */
    BLF_ERR_INVALID_ARGUMENT = 5, /* a null pointer, an index out of range, a buffer too small */
    BLF_ERR_CONFIG = 6,           /* ConfigError: the call's variant argument says which */
    BLF_ERR_UNKNOWN_ROLE = 7,     /* ModelError::UnknownRole */
    BLF_ERR_LAYOUT = 8,           /* ModelError::Layout: stored with another type or shape */
    BLF_ERR_CONVERT = 9,          /* ModelError::Convert: the conversion does not apply to the shape */
    BLF_ERR_SOURCE_SIZE = 10      /* ModelError::SourceSize: the parts do not add up to the weight */
};

/* StoredType (load/reader.rs:43-120). */
enum {
    BLF_F32 = 0,
    BLF_F16 = 1,
    BLF_BF16 = 2,
    BLF_F64 = 3,
    BLF_U8 = 4,
    BLF_I32 = 5,
    BLF_I64 = 6,
    BLF_OTHER = 7
};

const char *blf_last_error(void);
/* StoredType::size_bytes (reader.rs:65-74): bytes per element, 0 for OTHER. */
uint32_t blf_stored_type_size(uint32_t dtype);
/* The type's name as the reference prints it ("F32", "BF16", "other"). */
const char *blf_stored_type_name(uint32_t dtype);

/* ---- the reader (load/reader.rs) ---- */

typedef struct blf_archive blf_archive;

/* Tensor (reader.rs:124-160): name, type, shape (rank extents, outermost
 * first) and stored bytes. The pointers stay valid while the archive (or the
 * report that handed it out) exists. */
typedef struct {
    const char *name;
    uint32_t dtype;
    uint32_t rank;
    const uint64_t *shape;
    const uint8_t *data;
    uint64_t bytes;
} blf_tensor;

/* Archive::parse (reader.rs:183-199): the whole file in `bytes`, which must
 * outlive the archive (tensors borrow from it). BLF_ERR_FORMAT when the
 * header is malformed or disagrees with the buffer. */
int blf_archive_parse(const uint8_t *bytes, uint64_t len, blf_archive **out);
/* read_file + Archive::parse (reader.rs:252-258): the archive owns the bytes
 * it read. BLF_ERR_IO names the path. */
int blf_archive_open(const char *path, blf_archive **out);
void blf_archive_destroy(blf_archive *a);
uint64_t blf_archive_len(const blf_archive *a);
/* The index-th tensor in name order (Archive::iter, reader.rs:227-232). */
int blf_archive_at(const blf_archive *a, uint64_t index, blf_tensor *out);
/* Archive::require (reader.rs:220-225): BLF_ERR_MISSING_TENSOR when absent. */
int blf_archive_get(const blf_archive *a, const char *name, blf_tensor *out);
/* Archive::parameter_count (reader.rs:234-239), saturating. */
uint64_t blf_archive_parameter_count(const blf_archive *a);

/* ---- inventories (load/inventory.rs) ---- */

/* A tensor's role: a model's own vocabulary, compared field by field. The
 * Depth Anything V2 roles (depth_anything_v2.rs:324-460) use the BLF_ROLE_*,
 * BLF_BLOCK_*, BLF_PART_* and BLF_PARAM_* values below; unused fields are 0. */
typedef struct {
    uint32_t kind;
    uint32_t index; /* layer (Block, Fusion) or stage (Reassemble, NeckConv) */
    uint32_t part;
    uint32_t param;
    uint32_t unit;  /* Fusion residual unit: 0 first, 1 second */
    uint32_t conv;  /* Fusion residual conv (0, 1) or head conv (0, 1, 2) */
} blf_role;

enum {
    BLF_ROLE_CLASS_TOKEN = 0,
    BLF_ROLE_MASK_TOKEN = 1,
    BLF_ROLE_POSITION_EMBEDDING = 2,
    BLF_ROLE_PATCH_PROJECTION = 3,
    BLF_ROLE_BLOCK = 4,
    BLF_ROLE_FINAL_NORM = 5,
    BLF_ROLE_REASSEMBLE = 6,
    BLF_ROLE_NECK_CONV = 7,
    BLF_ROLE_FUSION = 8,
    BLF_ROLE_HEAD = 9
};
enum { BLF_PARAM_WEIGHT = 0, BLF_PARAM_BIAS = 1 };
enum {
    BLF_BLOCK_NORM1 = 0,
    BLF_BLOCK_QUERY = 1,
    BLF_BLOCK_KEY = 2,
    BLF_BLOCK_VALUE = 3,
    BLF_BLOCK_ATTENTION_OUTPUT = 4,
    BLF_BLOCK_LAYER_SCALE1 = 5,
    BLF_BLOCK_NORM2 = 6,
    BLF_BLOCK_MLP_FC1 = 7,
    BLF_BLOCK_MLP_FC2 = 8,
    BLF_BLOCK_LAYER_SCALE2 = 9
};
/* Reassemble parts; Fusion parts. */
enum { BLF_PART_PROJECTION = 0, BLF_PART_RESIZE = 1, BLF_PART_RESIDUAL = 1 };

/* TensorSpec (inventory.rs:31-48). Given to blf_inventory_new, the name and
 * shape are copied; handed out, they point into the inventory. */
typedef struct {
    const char *name;
    uint32_t dtype;
    uint32_t rank;
    const uint64_t *shape;
    blf_role role;
} blf_spec;

typedef struct blf_inventory blf_inventory;

/* Inventory::new (inventory.rs:62-75): BLF_ERR_DUPLICATE_NAME names the
 * repeated name. The names are copied. */
int blf_inventory_new(const blf_spec *specs, uint64_t count, blf_inventory **out);
void blf_inventory_destroy(blf_inventory *inv);
uint64_t blf_inventory_len(const blf_inventory *inv);
/* The index-th spec in the order given (Inventory::iter). */
int blf_inventory_at(const blf_inventory *inv, uint64_t index, blf_spec *out);
/* Inventory::get: BLF_ERR_MISSING_TENSOR when the name is not listed. */
int blf_inventory_get(const blf_inventory *inv, const char *name, blf_spec *out);
/* Inventory::by_role: the first spec of the role, BLF_ERR_UNKNOWN_ROLE when none. */
int blf_inventory_by_role(const blf_inventory *inv, const blf_role *role, blf_spec *out);
uint64_t blf_inventory_parameter_count(const blf_inventory *inv);

/* Inventory::check (inventory.rs:117-160) and its CheckReport (:189-207). */
typedef struct blf_report blf_report;
int blf_inventory_check(const blf_inventory *inv, const blf_archive *a, blf_report **out);
void blf_report_destroy(blf_report *r);
int blf_report_is_exact(const blf_report *r);
/* Missing names in inventory order; unexpected names in file (name) order;
 * mismatches in inventory order. */
uint64_t blf_report_missing_len(const blf_report *r);
const char *blf_report_missing(const blf_report *r, uint64_t i);
uint64_t blf_report_unexpected_len(const blf_report *r);
const char *blf_report_unexpected(const blf_report *r, uint64_t i);
uint64_t blf_report_mismatched_len(const blf_report *r);
/* Mismatch i: its name, then the expected and found layouts (dtype, rank
 * and shape set; no data). */
int blf_report_mismatch(const blf_report *r, uint64_t i, const char **name, blf_tensor *expected, blf_tensor *found);
uint64_t blf_report_expected_parameters(const blf_report *r);
uint64_t blf_report_file_parameters(const blf_report *r);
/* The report as the reference's Display renders it (inventory.rs:210-245). */
const char *blf_report_text(const blf_report *r);

/* ---- Depth Anything V2 (load/depth_anything_v2.rs) ---- */

enum { BLF_KEEP = 0, BLF_UP = 1, BLF_DOWN = 2 };
#define BLF_MAX_STAGES 8

/* Config (depth_anything_v2.rs:92-124). */
typedef struct {
    uint32_t image_size, patch_size, num_channels, hidden_size, num_layers, num_heads, mlp_ratio;
    uint32_t mask_token; /* 1: the file holds backbone.embeddings.mask_token */
    uint32_t stages;
    uint32_t out_indices[BLF_MAX_STAGES];
    uint32_t neck_hidden_sizes[BLF_MAX_STAGES];
    uint32_t resample[BLF_MAX_STAGES]; /* BLF_KEEP, BLF_UP or BLF_DOWN */
    uint32_t factor[BLF_MAX_STAGES];   /* Up or Down's factor */
    uint32_t fusion_hidden_size, head_hidden_size;
} blf_dav2_config;

/* ConfigError's variants (depth_anything_v2.rs:254-300). */
enum {
    BLF_CONFIG_ZERO = 1,
    BLF_CONFIG_HEADS_DO_NOT_DIVIDE_HIDDEN = 2,
    BLF_CONFIG_IMAGE_NOT_WHOLE_PATCHES = 3,
    BLF_CONFIG_FUSION_WIDTH_ODD = 4,
    BLF_CONFIG_STAGE_COUNT_MISMATCH = 5,
    BLF_CONFIG_OUT_INDEX_OUT_OF_RANGE = 6,
    BLF_CONFIG_OUT_INDICES_NOT_INCREASING = 7,
    BLF_CONFIG_RESAMPLE_BY_ONE = 8
};

/* Config::small (depth_anything_v2.rs:126-150). */
void blf_dav2_small(blf_dav2_config *out);
/* Config::validate (depth_anything_v2.rs:170-250): BLF_ERR_CONFIG, with the
 * variant in *variant (may be null) and its fields in the message. */
int blf_dav2_validate(const blf_dav2_config *c, uint32_t *variant);
/* inventory() (depth_anything_v2.rs:462-620): every tensor of the checkpoint,
 * F32, with its role, in the reference's order. */
int blf_dav2_inventory(const blf_dav2_config *c, blf_inventory **out, uint32_t *variant);

/* ---- conversions (model/mod.rs:130-353, positions.rs) ---- */

/* Convert (model/mod.rs:140-170). */
enum {
    BLF_AS_STORED = 0,
    BLF_LINEAR = 1,          /* [out][in] -> [in][out] */
    BLF_CONV = 2,            /* OIHW -> HWIO */
    BLF_CONV_TRANSPOSE = 3,  /* [in][out][kh][kw] -> HWIO */
    BLF_INTERPOLATE_POSITIONS = 4 /* [1][1 + g g][C]: the grid resampled bicubically to height x width */
};

/* convert() (model/mod.rs:274-335): `values` of `shape` rearranged, into
 * `out` (out_len elements at least: the input's, or 1 + height * width rows
 * for positions); *written and *cols (the result's last dimension) set.
 * BLF_ERR_CONVERT for a shape the conversion does not apply to. */
int blf_convert(uint32_t how, const float *values, const uint64_t *shape, uint32_t rank, uint32_t height,
                uint32_t width, float *out, uint64_t out_len, uint64_t *written, uint64_t *cols);

/* Weight::numbers (model/mod.rs:218-262): the tensors of `parts` roles (found
 * through the inventory, checked as F32 of the inventory's shape), each
 * converted, laid side by side along their last dimension, `elements`
 * numbers in all. */
int blf_weight_numbers(const blf_inventory *inv, const blf_archive *a, const blf_role *parts, uint32_t n_parts,
                       uint32_t how, uint32_t height, uint32_t width, float *out, uint64_t elements);

#ifdef __cplusplus
}
#endif

#endif
