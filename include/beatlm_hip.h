/*
 * beatlm HIP backend: the C ABI that replaces the reference's wgpu backend for
 * one lowered program (a list of kernel specs over a memory plan) on one AMD
 * Instinct MI355X (gfx950).
 *
 * The reference's boundary is everything below `&[KernelSpec] + &MemoryPlan`:
 *
 *   reference (Rust, crates/beatlm)                       this ABI
 *   ---------------------------------------------------   ----------------------------
 *   gpu::profile(limits, features)      gpu/profile.rs:24  bl_device_profile
 *   Arenas::new(device, plan)           gpu/arenas.rs:88   bl_arenas_create
 *   queue.write_buffer(arena, off, ..)  bench harness.rs:145-149  bl_arenas_write
 *   (map_async readback, tests only)    bench harness.rs:95-121   bl_arenas_read
 *   Kernels::new(device, plan, arenas,  codegen/kernels.rs:63-184 bl_kernels_create
 *                specs, sets)
 *   Kernels::encode(enc, k, set, ts)    codegen/kernels.rs:217-233 bl_kernels_encode
 *   Kernels::{len, sets, label}         codegen/kernels.rs:188-209 bl_kernels_len/_sets/_label
 *   SliceTimer::new(device, queue, n)   gpu/timer.rs:208    bl_timer_create
 *   SliceTimer::begin_frame(frame)      gpu/timer.rs:272    bl_timer_begin_frame
 *   FrameTimestamps::compute_pass(tag)  gpu/timer.rs:507    (timer argument of bl_kernels_encode)
 *   FrameTimestamps::resolve(encoder)   gpu/timer.rs:561    bl_timer_resolve
 *   SliceTimer::submitted(resolved)     gpu/timer.rs:307    bl_timer_submitted
 *   SliceTimer::submitted_held(resolved) gpu/timer.rs:332   bl_timer_submitted_held
 *   HeldFrame::accept / reject          gpu/timer.rs:674-684 bl_timer_verdict
 *   drop(ResolvedFrame)                 gpu/ring.rs:113-140 bl_timer_abandon
 *   SliceTimer::in_flight()             gpu/timer.rs:452    bl_timer_in_flight
 *   SliceTimer::collect_ready()         gpu/timer.rs:371    bl_timer_collect
 *   SliceTimer::invalidate_submitted()  gpu/timer.rs:445    bl_timer_invalidate_submitted
 *   SliceTimer::stats()                 gpu/timer.rs:458    bl_timer_stats
 *
 * A `bl_spec` is the reference's `KernelSpec` (crates/beatlm-core/src/kernel.rs
 * :1939-1947) flattened: main operation and its dimensions, the `Part` of the
 * split dimension one dispatch computes, the epilogue steps in order, and the
 * bindings in `KernelSpec::bindings` order (main reads, epilogue operands,
 * output last; kernel.rs:2096-2113), each resolved through the memory plan to
 * (arena, offset, size) as `Arenas::binding` does (gpu/arenas.rs:127-155).
 *
 * Conventions: every call returns a status, 0 = ok, negative = the error enum
 * below (mirroring CodegenError, ArenaError, TimerError and KernelError);
 * bl_last_error(ctx) gives the message of the last failure on that context.
 * Handles are opaque and destroyed by the caller. A context is used from one
 * thread at a time. Everything that allocates happens in the create calls;
 * bl_kernels_encode allocates nothing and never waits for the GPU.
 */
#ifndef BEATLM_HIP_H
#define BEATLM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BL_ABI_VERSION 4u
#define BL_MAX_EPILOGUE 8
#define BL_MAX_BINDINGS 8

/* ---- status codes ---- */
enum {
    BL_OK = 0,
    BL_ERR_HIP = -1,                   /* a HIP runtime call failed (device lost, OOM, ...) */
    BL_ERR_INVALID_ARGUMENT = -2,      /* null pointer, zero count, bad enum */
    /* ArenaError (gpu/arenas.rs:18-48) */
    BL_ERR_PLAN_NOT_VALID_ON_DEVICE = -10,
    BL_ERR_UNKNOWN_ARENA = -11,
    BL_ERR_PLACEMENT_OUT_OF_RANGE = -12,
    BL_ERR_MISALIGNED_PLACEMENT = -13,
    /* CodegenError (codegen/mod.rs:85-154) */
    BL_ERR_KERNEL = -20,               /* the spec has no variant that runs here */
    BL_ERR_MISSING_PLACEMENT = -21,
    BL_ERR_STAND_IN_SIZE = -22,
    BL_ERR_NO_SUCH_KERNEL = -23,
    BL_ERR_NO_SUCH_SET = -24,
    BL_ERR_TOO_LARGE = -25,            /* the shape needs more than a fixed-size buffer holds */
    /* TimerError (gpu/timer.rs:61-89) */
    BL_ERR_TIMER_TOO_MANY_SLICES = -30,
    BL_ERR_TIMER_NO_FRAME = -31,
    BL_ERR_TIMER_CAPACITY = -32,
    BL_ERR_TIMER_RENDER_TWICE = -33    /* TimerError::RenderPassAlreadyTimed */
};

/* ---- main operations (MainOp, kernel.rs:1393-1445) ---- */
enum {
    BL_MAIN_LAYER_NORM = 1,       /* dims: rows, channels; epsilon */
    BL_MAIN_MATMUL = 2,           /* dims: m, k, n, has_bias */
    BL_MAIN_ATTENTION_SCORES = 3, /* dims: tokens, heads, head_dim */
    BL_MAIN_SOFTMAX = 4,          /* dims: rows, cols */
    BL_MAIN_ATTENTION_VALUES = 5, /* dims: tokens, heads, head_dim */
    BL_MAIN_PATCH_EMBED = 6,      /* dims: grid_h, grid_w, patch, cin, cout, has_bias */
    BL_MAIN_PREPEND_TOKEN = 7,    /* dims: rows, channels */
    BL_MAIN_TOKENS_TO_MAP = 8,    /* dims: height, width, channels */
    BL_MAIN_MAP = 9,              /* dims: elements */
    /* The DPT head's operations: MainOp::Conv2d3x3, ConvTranspose2d, ResizeBilinear
     * (kernel.rs:1412-1417; the ops at kernel.rs:447-631). */
    BL_MAIN_CONV3X3 = 10,         /* dims: height, width, cin, cout, stride, has_bias; NHWC, HWIO weights, padding 1;
                                   * split along output pixels; prologue BL_PRO_RELU allowed */
    BL_MAIN_CONV_TRANSPOSE = 11,  /* dims: height, width, cin, cout, factor, has_bias; kernel = stride = factor;
                                   * split along output pixels */
    BL_MAIN_RESIZE_BILINEAR = 12, /* dims: in_height, in_width, out_height, out_width, channels; corners aligned;
                                   * split along output pixels */
    /* Backend-level main op with no MainOp counterpart: the three kernels
     * attention_scores+scale -> softmax -> attention_values over one qkv tensor
     * fused into one flash-attention kernel (online softmax, no [T][H][T]
     * tensors). dims: tokens, heads, head_dim; scale = the Scale epilogue's
     * factor. Bindings: qkv, output. Parts split along query rows. */
    BL_MAIN_FLASH_ATTENTION = 100
};

/* ---- prologue steps (Prologue, kernel.rs:1639-1659): applied to every
 * value of the main input as it is loaded; only BL_MAIN_CONV3X3 takes one ---- */
enum { BL_PRO_RELU = 1 };

/* ---- epilogue steps (Epilogue, kernel.rs:1593-1615) ---- */
enum {
    BL_EPI_ADD = 1,           /* v + operand[index] */
    BL_EPI_RELU = 2,
    BL_EPI_GELU = 3,          /* tanh approximation */
    BL_EPI_GELU_ERF = 4,
    BL_EPI_SCALE = 5,         /* v * factor */
    BL_EPI_CHANNEL_SCALE = 6  /* v * operand[index % channels] */
};

/* ---- element types (DType, memory.rs:133-150) ---- */
enum { BL_F32 = 0, BL_F16 = 1 };

/* ---- how f32 products run on the matrix cores ---- */
enum {
    BL_F32_MATH_SPLIT_BF16 = 0, /* each f32 operand as hi + lo bf16, three bf16 MFMAs, f32 accumulate */
    BL_F32_MATH_MFMA_F32 = 1    /* v_mfma_f32_*_f32: f32 operands, f32 accumulate */
};

typedef struct {
    uint32_t kind;       /* BL_EPI_* */
    float factor;        /* BL_EPI_SCALE */
    uint32_t channels;   /* BL_EPI_CHANNEL_SCALE */
    uint32_t operand;    /* binding index of the tensor read (ADD, CHANNEL_SCALE) */
} bl_epilogue;

typedef struct {
    uint32_t tensor;     /* TensorId; what a binding set substitutes by */
    uint32_t arena;      /* Placement::arena */
    uint64_t offset;     /* Placement::offset (bytes) */
    uint64_t size;       /* Placement::size (bytes) */
    uint32_t dtype;      /* BL_F32 / BL_F16 */
    uint32_t reserved;
} bl_binding;

typedef struct {
    uint32_t index, count; /* Part::index, Part::count */
    uint32_t start, end;   /* Part::range, in units of the split dimension */
} bl_part;

typedef struct {
    uint32_t main;                 /* BL_MAIN_* */
    uint32_t dims[6];              /* per main op, see the enum */
    float epsilon;                 /* layer norm */
    float scale;                   /* flash attention */
    bl_part part;
    /* Binding index of each tensor the main operation reads, in MainOp::reads
     * order (kernel.rs:1447-1474); duplicates in `bindings` are allowed to
     * collapse, as KernelSpec::bindings does. */
    uint32_t n_reads;
    uint32_t reads[4];
    uint32_t n_epilogue;
    bl_epilogue epilogue[BL_MAX_EPILOGUE];
    uint32_t n_bindings;
    bl_binding bindings[BL_MAX_BINDINGS];
    uint32_t prologue;             /* BL_PRO_* or 0 (KernelSpec::prologue, kernel.rs:1947) */
} bl_spec;

/* One binding set: tensors of the specs bound to stand-ins (Substitution,
 * codegen/kernels.rs:22-26), each given with the stand-in's placement. */
typedef struct {
    uint32_t original;   /* TensorId of the spec's binding */
    uint32_t stand_in;   /* TensorId bound in its place */
    uint32_t arena;
    uint32_t reserved;
    uint64_t offset, size;
} bl_substitution;

typedef struct {
    const bl_substitution *items;
    uint32_t count;
} bl_binding_set;

/* DeviceProfile (crates/beatlm-core/src/device.rs:62-95) as the device reports it. */
typedef struct {
    uint64_t max_storage_buffer_binding_size;
    uint64_t max_buffer_size;
    uint32_t min_storage_buffer_offset_alignment;
    uint32_t max_compute_workgroup_storage_size;
    uint32_t max_compute_invocations_per_workgroup;
    uint32_t max_compute_workgroup_size[3];
    uint32_t max_compute_workgroups_per_dimension;
    uint32_t max_storage_buffers_per_shader_stage;
    uint32_t shader_f16, subgroups, timestamp_query;
    /* what the core profile has no field for */
    uint32_t compute_units;
    uint32_t wave_size;
    uint64_t total_memory;
    char name[64];
    char arch[32];
} bl_device_profile_t;

typedef struct bl_ctx bl_ctx;
typedef struct bl_arenas bl_arenas;
typedef struct bl_kernels bl_kernels;
typedef struct bl_timer bl_timer;

/* ---- context ---- */
uint32_t bl_abi_version(void);
int bl_ctx_create(int device_ordinal, bl_ctx **out);
/* Arenas, kernels and timers keep their context alive: destroying the context
 * first is allowed, and it is released when the last of them is destroyed. */
void bl_ctx_destroy(bl_ctx *ctx);
const char *bl_last_error(const bl_ctx *ctx);
int bl_device_profile(bl_ctx *ctx, bl_device_profile_t *out);
/* BL_F32_MATH_*; applies to kernels created afterwards. */
int bl_ctx_set_f32_math(bl_ctx *ctx, uint32_t mode);
/* Waits for everything submitted on the context's stream (tests and hosts
 * outside the frame loop only). */
int bl_ctx_synchronize(bl_ctx *ctx);
/* Device allocations the context has made (arenas, scratch, events): the
 * frame loop's count must not move. */
uint64_t bl_ctx_allocations(const bl_ctx *ctx);
/* Bytes of device memory the context's live arenas and kernels hold now: the
 * arenas' one allocation each plus each kernels' workspace
 * (bl_kernels_workspace_bytes). No counterpart in the reference. */
uint64_t bl_ctx_device_bytes(const bl_ctx *ctx);
/* The context's HIP stream (hipStream_t), for hosts that order their own work
 * (e.g. a render pass) on it. */
void *bl_ctx_stream(bl_ctx *ctx);

/* ---- arenas: one hipMalloc for every arena of a plan ---- */
int bl_arenas_create(bl_ctx *ctx, const uint64_t *arena_sizes, uint32_t n,
                     bl_arenas **out);
/* Kernels made over the arenas keep them alive (as the reference's Kernels
 * keep their buffers): destroying the arenas first is allowed, and their
 * memory is freed when the last of those kernels is destroyed. */
void bl_arenas_destroy(bl_arenas *arenas);
/* Ordered on the context's stream; returns when the source may be reused.
 * Packed copies of weights made from the written bytes are remade before the
 * next launch that reads them; nothing else is repacked. */
int bl_arenas_write(bl_arenas *arenas, uint32_t arena, uint64_t offset,
                    const void *src, uint64_t bytes);
/* The host changed bytes [offset, offset + bytes) of an arena without
 * bl_arenas_write (through bl_arenas_device_ptr): what the kernels derived
 * from those bytes (packed weights, attention operands) is remade before its
 * next use, as after bl_arenas_write. No counterpart in the reference, whose
 * host writes only through queue.write_buffer. */
int bl_arenas_invalidate(bl_arenas *arenas, uint32_t arena, uint64_t offset,
                         uint64_t bytes);
/* Waits for the stream, then copies out. */
int bl_arenas_read(bl_arenas *arenas, uint32_t arena, uint64_t offset, void *dst,
                   uint64_t bytes);
/* Device address of a byte of an arena (for hosts that bind their own work).
 * A host that writes through it calls bl_arenas_invalidate for those bytes. */
int bl_arenas_device_ptr(bl_arenas *arenas, uint32_t arena, uint64_t offset,
                         void **out);

/* ---- kernels ---- */
int bl_kernels_create(bl_ctx *ctx, bl_arenas *arenas, const bl_spec *specs,
                      uint32_t n_specs, const bl_binding_set *sets,
                      uint32_t n_sets, bl_kernels **out);
/* bl_kernels_create, told which tensors (bl_binding.tensor ids) the host
 * never reads or writes itself: the program's activations, which only its
 * kernels produce and consume. The backend may keep those in a layout of its
 * own; with bf16x3 f32 math, an activation every reader of which is a GEMM
 * reading it as its A operand is stored as hi and lo bf16 planes, written
 * split by its producer, so the GEMMs multiply it without splitting it.
 * No counterpart in the reference (Kernels::new has no such hint); a host
 * passes its plan's activation tensors, or calls bl_kernels_create. */
int bl_kernels_create_internal(bl_ctx *ctx, bl_arenas *arenas, const bl_spec *specs,
                               uint32_t n_specs, const bl_binding_set *sets,
                               uint32_t n_sets, const uint32_t *internal,
                               uint32_t n_internal, bl_kernels **out);
/* Waits for the context's stream; frees the arenas too when they were
 * destroyed before and these were their last kernels. */
void bl_kernels_destroy(bl_kernels *kernels);
uint32_t bl_kernels_len(const bl_kernels *kernels);
uint32_t bl_kernels_sets(const bl_kernels *kernels);
/* The spec's name (e.g. "matmul+channel_scale+add"), followed for a part of a
 * split kernel by " part i/n"; the variant chosen after " @ ". */
const char *bl_kernels_label(const bl_kernels *kernels, uint32_t kernel);
/* Launches kernel `kernel` with binding set `set` on the context's stream.
 * With a timer, the launch is bracketed by that timer's events for the
 * current frame under `tag`. No allocation, no wait.
 * Each kernel's result depends only on its bindings, whatever was encoded
 * before it: a flash-attention kernel whose K and V operands its QKV
 * projection's epilogue wrote into the backend's scratch reads them from
 * there only when nothing has written qkv since; otherwise (the kernel
 * encoded alone, a host write, another kernel over those bytes) it makes
 * them from qkv itself first. Under bl_kernels_create_internal, a qkv that is
 * internal, written by nothing but its projections from an internal x and
 * read by nothing but flash kernels holds the queries alone (the label of each
 * projection ends in " > queries only"): such a flash kernel runs its
 * projections again instead, from x as it is, which in program order is the
 * x they read before. Kernels of bl_kernels_create_internal whose work
 * another kernel does launch nothing: a LayerNorm folded into the product
 * that reads it, and a class-token prepend fused into the patch embedding
 * before it (which writes the prepend's output; the internal patches tensor
 * between them is never written). */
int bl_kernels_encode(bl_kernels *kernels, uint32_t kernel, uint32_t set,
                      bl_timer *timer, uint32_t tag);
/* Launches kernels [first, first + count) in order with binding set `set`.
 * The first call for a (first, count, set) captures the launches as a HIP
 * graph; later calls replay it (weights packs that went stale since are
 * remade first, outside the graph). Programs whose kernels rewrite a packed
 * weight's source, a process with BL_NO_GRAPH set, or one run under
 * rocprofv3 launch one by one. */
int bl_kernels_encode_range(bl_kernels *kernels, uint32_t first, uint32_t count,
                            uint32_t set);

/* The average duration of one launch of `kernel`, from a hipEvent pair on the
 * context's stream around `repeats` back-to-back launches (after one untimed
 * launch). Blocks until they finish. No counterpart in the reference, which
 * times kernels only through the slice timer: a measurement aid for per-kernel
 * rooflines, free of the launch gaps a per-slice event pair includes. */
int bl_kernels_time(bl_kernels *kernels, uint32_t kernel, uint32_t set, uint32_t repeats, float *micros_per_launch);
/* How many packed weight copies the kernels have made so far (once per
 * weight at first use, again after the host writes its bytes). No
 * counterpart in the reference: lets a host check its frame loop repacks
 * nothing. */
uint64_t bl_kernels_packs_made(const bl_kernels *kernels);
/* Bytes of device memory the kernels hold beside the plan's arenas, in one
 * allocation made by bl_kernels_create (0: none): packed weights, split-k
 * partial sums, attention scratch, the folded LayerNorms' statistics and
 * planes, placed by lifetime as the plan places tensors in an arena (items of
 * disjoint kernel spans share bytes). No counterpart in the reference, whose
 * kernels hold no memory of their own; with the arenas' one allocation, a
 * program's device memory is these two allocations. */
uint64_t bl_kernels_workspace_bytes(const bl_kernels *kernels);
/* A LayerNorm whose output only a later product reads, as its A, while its
 * input x was last written by an earlier product, is folded into the reader:
 * LN(x) W + b = rstd ((x - mean) (gamma W)) + d with d = beta W + b, the
 * writer of x leaving each row's 32-column block statistics (mean, sum of
 * squared deviations) and the LayerNorm launching nothing. In f32 storage the
 * writer also leaves x centred per block (x less its block's mean, the
 * "shadow"), and the reader adds sum_b (mean_b - mean) cb[b] with cb[b] the
 * column sums of gamma W over block b, so no product carries x's common
 * offset; in f16 storage the reader computes x (gamma W) - mean c with c the
 * column sums. bl_kernels_fold_read copies fold `fold`'s device buffers out
 * after waiting for the stream: what = 0 the statistics of set `set`
 * ([rows][cols / 32] pairs of floats), 1 the vectors c, d (each padded to the
 * pack's columns n_pad) and cb ([n_pad][32]), 2 the shadow of set `set`
 * (hi then lo bf16 planes for bf16x3 math, f32 for the f32 matrix cores).
 * Folds are numbered in kernel order. Folds whose producer-to-consumer spans
 * do not overlap share bytes, so a fold's buffers hold what the last writer
 * of those bytes left. A diagnostic with no counterpart in
 * the reference (whose kernels run one per spec); the fold itself changes no
 * kernel's bindings or results beyond rounding. */
int bl_kernels_fold_read(bl_kernels *kernels, uint32_t fold, uint32_t set, uint32_t what, void *dst, uint64_t bytes);
/* The GPU kernel launches behind one bl_kernels_encode_range(first, count,
 * set) call, counted as the kernel nodes of the HIP graph that call replays
 * (a folded LayerNorm adds none; a flash attention adds its prep launch when
 * no projection writes its operands, and a merge launch only under
 * BL_FLASH_MERGE_LAUNCH). BL_ERR_INVALID_ARGUMENT when that range has no captured graph
 * (graphs off, or the range not yet encoded). A measurement aid with no
 * counterpart in the reference. */
int bl_kernels_range_launches(bl_kernels *kernels, uint32_t first, uint32_t count, uint32_t set, uint32_t *launches);

/* ---- flash attention that allocates nothing ----
 * No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, hosts that
 * forbid hipMalloc): the computation of a BL_MAIN_FLASH_ATTENTION kernel,
 * whole, as bl_kernels_encode runs it when no projection wrote its operands:
 * qkv [tokens][3][heads][64] (dtype BL_F32, with the context's f32 math, or
 * BL_F16) into out [tokens][heads * 64], scale as the Scale epilogue's, on
 * the context's stream. The caller passes device pointers to both. Its
 * scratch (the K and Vt operands, partial results of split key ranges and
 * the arrival counters of their in-kernel merge, zero between calls) is a
 * static device array of BL_STATIC_SCRATCH_BYTES that the library holds on
 * each GPU it has run this on until the process ends; a shape needing more
 * is refused with BL_ERR_TOO_LARGE and a message. Nothing is allocated, the
 * first call on a device aside, which looks the array's address up (and so
 * loads the code object holding it; a failed lookup is tried again on the
 * next call). The call makes the context's device current and restores the
 * caller's current device before it returns. Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU race. */
#define BL_STATIC_SCRATCH_BYTES (64ull << 20)
int bl_flash_attention_static(bl_ctx *ctx, const void *qkv, void *out, uint32_t tokens,
                              uint32_t heads, float scale, uint32_t dtype);

/* Diagnostic (no GPU work, no context): checks the flash kernel's plan for
 * tokens x heads on compute_units CUs (dtype BL_F32 with bf16x3 math, or
 * BL_F16): the (head, query tile, key tile) units of each XCD are covered by
 * its runs of workgroups in order, each unit by exactly one run. BL_OK with
 * *units the units planned, BL_ERR_TOO_LARGE when the shape is beyond the
 * kernel's 32-bit run arithmetic (kernels for it are refused the same way),
 * BL_ERR_KERNEL when the runs are wrong. No counterpart in the reference. */
int bl_flash_plan_check(uint32_t tokens, uint32_t heads, uint32_t compute_units, uint32_t dtype, uint64_t *units);

/* ---- slice timer: hipEvent pairs per slice, a ring of frames ---- */
#define BL_TIMER_RING_DEPTH 3
typedef struct {
    uint64_t frame;       /* FrameIndex given to begin_frame */
    uint32_t n_slices;
    uint32_t failed;      /* 1: the frame was invalidated and carries no times */
    const uint32_t *tags; /* n_slices tags, valid until the next collect */
    const float *micros;  /* n_slices durations in microseconds */
    uint32_t has_render;  /* 1: the frame timed its render pass (FrameTiming::render) */
    float render_micros;
} bl_frame_timing;

typedef struct {
    uint64_t frames_begun, frames_timed, frames_skipped, frames_failed, frames_dropped;
} bl_timer_stats_t;

int bl_timer_create(bl_ctx *ctx, uint32_t max_slices, bl_timer **out);
void bl_timer_destroy(bl_timer *timer);
/* Opens a frame. `*timed` is 0 when its ring slot is still in flight: the
 * frame then runs untimed and counts as skipped (FrameTimestamps::is_timed). */
int bl_timer_begin_frame(bl_timer *timer, uint64_t frame, uint32_t *timed);
/* FrameTimestamps::render_pass (gpu/timer.rs:527-560): the frame's render
 * pass, the host's own work on the context's stream enqueued between these
 * two calls, timed apart from the compute passes (at most once a frame;
 * nothing is recorded when the frame is untimed). */
int bl_timer_render_begin(bl_timer *timer);
int bl_timer_render_end(bl_timer *timer);
/* Closes the open frame. `*resolved` is its ticket (0 for an untimed frame),
 * spent by exactly one of bl_timer_submitted, bl_timer_submitted_held or
 * bl_timer_abandon; until then the frame keeps its slot, and tickets may come
 * back in any order. A frame begun while another is open drops the open one
 * unread (frames_dropped). */
int bl_timer_resolve(bl_timer *timer, uint64_t *resolved);
/* The host says the frame's work reached the stream: only now may it be read.
 * A ticket of 0, from another timer or an earlier lap is accepted and ignored
 * (another timer's frame then goes untimed). */
int bl_timer_submitted(bl_timer *timer, uint64_t resolved);
/* bl_timer_submitted for a host that learns later whether the submission
 * ran: the frame is read only once bl_timer_verdict accepts `*hold` (0 when
 * there is nothing to hold), and frames submitted after it wait for it. */
int bl_timer_submitted_held(bl_timer *timer, uint64_t resolved, uint64_t *hold);
/* The verdict on a held frame: accepted (read once its events completed) or
 * rejected (dropped unread, holding back nothing). Returns 1 when it reached
 * the frame, 0 when the frame had been invalidated meanwhile. A hold never
 * given a verdict waits, and holds back every later frame, until
 * bl_timer_invalidate_submitted. */
int bl_timer_verdict(bl_timer *timer, uint64_t hold, uint32_t accepted);
/* The frame's work was never submitted (an error path): its slot is freed
 * unread at the next begin_frame and counted in frames_dropped. */
int bl_timer_abandon(bl_timer *timer, uint64_t resolved);
/* Frames recorded or submitted and not yet collected (an abandoned one is not). */
uint32_t bl_timer_in_flight(const bl_timer *timer);
/* The frames ready to read, in submission order, without blocking
 * (hipEventQuery): a frame waits while one submitted before it is held or
 * still running; invalid and failed frames are freed and hold back nothing.
 * Fills up to `cap` entries. */
int bl_timer_collect(bl_timer *timer, bl_frame_timing *out, uint32_t cap,
                     uint32_t *n_out);
/* Every submitted or held frame not yet collected is marked failed: never
 * decoded, freed once its events complete. Returns how many were marked. */
int bl_timer_invalidate_submitted(bl_timer *timer);
int bl_timer_stats(const bl_timer *timer, bl_timer_stats_t *out);

/* ---- a fixed amount of GPU time (a synthetic render load) ---- */
/* Launches one kernel on the context's stream that spins every CU for
 * `micros` microseconds of the device's constant-rate wall clock. */
int bl_spin(bl_ctx *ctx, uint32_t micros);

#ifdef __cplusplus
}
#endif
#endif
