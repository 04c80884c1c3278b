// The C ABI of include/beatlm_hip.h: context, arenas and kernels.
//
// bl_kernels_create is the HIP counterpart of the reference's Kernels::new
// (crates/beatlm/src/codegen/kernels.rs:63-184): it checks every spec once,
// resolves each binding set's bindings to device addresses inside the
// arenas, picks the kernel variant and launch shape, and allocates the
// scratch any kernel needs, so that bl_kernels_encode (Kernels::encode,
// :217-233) is a launch over prepared arguments and nothing else.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "spec.hpp"
#include "timer.hpp"

using namespace bl;

struct bl_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string error;
    uint64_t allocations = 0;
    uint64_t device_bytes = 0;  // held now by the context's arenas and kernels
    uint32_t f32_math = BL_F32_MATH_SPLIT_BF16;
    uint32_t compute_units = 0;
    uint32_t wall_clock_khz = 0;
    bl_device_profile_t profile{};
    // Arenas, kernels and timers made from this context and not yet destroyed;
    // bl_ctx_destroy waits for the last of them before releasing the stream.
    uint32_t children = 0;
    bool closed = false;
};

namespace {

int fail(bl_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->error = buf;
    }
    return code;
}

int hip_fail(bl_ctx *ctx, hipError_t e, const char *what) {
    return fail(ctx, BL_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

// The placement alignment every plan made for this backend uses: HBM
// transactions are 128-byte lines and the kernels' 16-byte vector loads need
// 16; 256 matches the reference's baseline (device.rs:97-113), so a baseline
// plan is valid here unchanged.
constexpr uint32_t PLACEMENT_ALIGNMENT = 256;

// Whether the process runs under rocprofv3, which sets these for the program
// it starts. HIP-graph capture and replay is not used there, so that profiled
// runs are not the ones that ended in a host segmentation fault under
// rocprofv3 with the depth model's programs captured. A second such fault
// came with graphs off, on a thread this library never runs on, so capture is
// not known to be the cause; that case is simply not repeated.
bool profiler_attached() {
    static const bool attached = [] {
        const bool on = getenv("ROCPROF_OUTPUT_PATH") || getenv("ROCPROFILER_LIBRARY_CTOR");
        if (on) fprintf(stderr, "beatlm: running under rocprofv3: kernel ranges launch one by one, not as HIP graphs\n");
        return on;
    }();
    return attached;
}

}  // namespace

struct bl_arenas {
    bl_ctx *ctx = nullptr;
    char *base = nullptr;
    std::vector<uint64_t> offset, size;
    uint64_t total = 0;
    // Kernels made over these arenas and not yet destroyed. Each holds the
    // arenas (bl_arenas_destroy frees the memory only after the last of them
    // is gone, since their launches point into it) and is told of every host
    // write, so that it remakes the packed copies a write made stale.
    std::vector<bl_kernels *> users;
    bool closed = false;
};

// A host write to bytes [offset, offset + bytes) of an arena.
static void kernels_written(bl_kernels *k, uint32_t arena, uint64_t offset, uint64_t bytes);

// ---- context ----

extern "C" uint32_t bl_abi_version(void) { return BL_ABI_VERSION; }

extern "C" int bl_ctx_create(int device_ordinal, bl_ctx **out) {
    if (!out) return BL_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return BL_ERR_HIP;
    if (device_ordinal < 0 || device_ordinal >= count) return BL_ERR_INVALID_ARGUMENT;
    bl_ctx *ctx = new bl_ctx();
    ctx->device = device_ordinal;
    // Messages are formatted into 512 bytes: with this capacity, setting one
    // allocates nothing (the allocation-free entry point reports through it).
    ctx->error.reserve(512);
    if ((e = hipSetDevice(device_ordinal)) != hipSuccess) { delete ctx; return BL_ERR_HIP; }
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device_ordinal)) != hipSuccess) { delete ctx; return BL_ERR_HIP; }
    // One stream at the default priority; the frame loop's work is ordered on it.
    if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete ctx;
        return BL_ERR_HIP;
    }
    int khz = 0;
    hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device_ordinal);
    ctx->wall_clock_khz = (uint32_t)khz;
    ctx->compute_units = (uint32_t)prop.multiProcessorCount;
    bl_device_profile_t &p = ctx->profile;
    // A hipMalloc'd arena is addressed by 64-bit pointers: no binding limit
    // below the device's memory (kernels index elements with 32-bit rows and
    // 64-bit offsets).
    p.max_storage_buffer_binding_size = prop.totalGlobalMem;
    p.max_buffer_size = prop.totalGlobalMem;
    p.min_storage_buffer_offset_alignment = PLACEMENT_ALIGNMENT;
    p.max_compute_workgroup_storage_size = (uint32_t)prop.sharedMemPerBlock;
    p.max_compute_invocations_per_workgroup = (uint32_t)prop.maxThreadsPerBlock;
    p.max_compute_workgroup_size[0] = (uint32_t)prop.maxThreadsDim[0];
    p.max_compute_workgroup_size[1] = (uint32_t)prop.maxThreadsDim[1];
    p.max_compute_workgroup_size[2] = (uint32_t)prop.maxThreadsDim[2];
    p.max_compute_workgroups_per_dimension = (uint32_t)std::min<int>(prop.maxGridSize[1], prop.maxGridSize[2]);
    p.max_storage_buffers_per_shader_stage = BL_MAX_BINDINGS;
    p.shader_f16 = 1;
    p.subgroups = 1;
    p.timestamp_query = 1;
    p.compute_units = ctx->compute_units;
    p.wave_size = (uint32_t)prop.warpSize;
    p.total_memory = prop.totalGlobalMem;
    snprintf(p.name, sizeof p.name, "%s", prop.name);
    snprintf(p.arch, sizeof p.arch, "%s", prop.gcnArchName);
    *out = ctx;
    return BL_OK;
}

static void ctx_free(bl_ctx *ctx) {
    hipSetDevice(ctx->device);
    if (ctx->stream) {
        hipStreamSynchronize(ctx->stream);
        hipStreamDestroy(ctx->stream);
    }
    delete ctx;
}

extern "C" void bl_ctx_destroy(bl_ctx *ctx) {
    if (!ctx || ctx->closed) return;
    ctx->closed = true;
    if (ctx->children == 0) ctx_free(ctx);
}

void bl_ctx_retain(bl_ctx *ctx) { ctx->children++; }

void bl_ctx_release(bl_ctx *ctx) {
    if (--ctx->children == 0 && ctx->closed) ctx_free(ctx);
}

extern "C" const char *bl_last_error(const bl_ctx *ctx) { return ctx ? ctx->error.c_str() : "no context"; }

extern "C" int bl_device_profile(bl_ctx *ctx, bl_device_profile_t *out) {
    if (!ctx || !out) return BL_ERR_INVALID_ARGUMENT;
    *out = ctx->profile;
    return BL_OK;
}

extern "C" int bl_ctx_set_f32_math(bl_ctx *ctx, uint32_t mode) {
    if (!ctx) return BL_ERR_INVALID_ARGUMENT;
    if (mode != BL_F32_MATH_SPLIT_BF16 && mode != BL_F32_MATH_MFMA_F32)
        return fail(ctx, BL_ERR_INVALID_ARGUMENT, "unknown f32 math mode %u", mode);
    ctx->f32_math = mode;
    return BL_OK;
}

extern "C" int bl_ctx_synchronize(bl_ctx *ctx) {
    if (!ctx) return BL_ERR_INVALID_ARGUMENT;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? BL_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

extern "C" uint64_t bl_ctx_allocations(const bl_ctx *ctx) { return ctx ? ctx->allocations : 0; }
extern "C" uint64_t bl_ctx_device_bytes(const bl_ctx *ctx) { return ctx ? ctx->device_bytes : 0; }

extern "C" void *bl_ctx_stream(bl_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

// Device memory the backend owns, counted so a host can check the frame loop
// allocates nothing.
void *bl_device_alloc(bl_ctx *ctx, uint64_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    ctx->allocations++;
    ctx->device_bytes += bytes;
    return p;
}

void bl_device_free(bl_ctx *ctx, void *p, uint64_t bytes) {
    if (!p) return;
    hipFree(p);
    ctx->device_bytes -= bytes;
}

bool bl_events_counted(bl_ctx *ctx, uint64_t n) {
    ctx->allocations += n;
    return true;
}

hipStream_t bl_stream_of(bl_ctx *ctx) { return ctx->stream; }
int bl_device_of(const bl_ctx *ctx) { return ctx->device; }
uint32_t bl_compute_units_of(const bl_ctx *ctx) { return ctx->compute_units; }
uint32_t bl_f32_math_of(const bl_ctx *ctx) { return ctx->f32_math; }
int bl_fail(bl_ctx *ctx, int code, const char *msg) { return fail(ctx, code, "%s", msg); }

// ---- arenas ----

extern "C" int bl_arenas_create(bl_ctx *ctx, const uint64_t *sizes, uint32_t n, bl_arenas **out) {
    if (!ctx || !out || (n && !sizes)) return BL_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    hipSetDevice(ctx->device);
    bl_arenas *a = new bl_arenas();
    a->ctx = ctx;
    uint64_t total = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (sizes[i] > ctx->profile.max_buffer_size) {
            delete a;
            return fail(ctx, BL_ERR_PLAN_NOT_VALID_ON_DEVICE,
                        "arena %u of %llu bytes exceeds the device's %llu", i,
                        (unsigned long long)sizes[i], (unsigned long long)ctx->profile.max_buffer_size);
        }
        total = (total + PLACEMENT_ALIGNMENT - 1) / PLACEMENT_ALIGNMENT * PLACEMENT_ALIGNMENT;
        a->offset.push_back(total);
        a->size.push_back(sizes[i]);
        total += sizes[i];
    }
    a->total = total;
    if (total) {
        // One allocation for every arena of the plan.
        a->base = (char *)bl_device_alloc(ctx, total);
        if (!a->base) {
            delete a;
            return fail(ctx, BL_ERR_HIP, "hipMalloc of %llu bytes of arenas", (unsigned long long)total);
        }
    }
    bl_ctx_retain(ctx);
    *out = a;
    return BL_OK;
}

static void arenas_free(bl_arenas *a) {
    if (a->base) {
        hipSetDevice(a->ctx->device);
        hipStreamSynchronize(a->ctx->stream);
        bl_device_free(a->ctx, a->base, a->total);
    }
    bl_ctx *ctx = a->ctx;
    delete a;
    bl_ctx_release(ctx);
}

extern "C" void bl_arenas_destroy(bl_arenas *a) {
    if (!a || a->closed) return;
    a->closed = true;
    if (a->users.empty()) arenas_free(a);
}

static void arenas_written(bl_arenas *a, uint32_t arena, uint64_t offset, uint64_t bytes) {
    for (bl_kernels *k : a->users) kernels_written(k, arena, offset, bytes);
}

static int check_range(bl_arenas *a, uint32_t arena, uint64_t offset, uint64_t bytes) {
    if (arena >= a->size.size())
        return fail(a->ctx, BL_ERR_UNKNOWN_ARENA, "arena %u does not exist in this set", arena);
    if (offset > a->size[arena] || bytes > a->size[arena] - offset)
        return fail(a->ctx, BL_ERR_PLACEMENT_OUT_OF_RANGE,
                    "placement at offset %llu of %llu bytes does not lie inside arena %u",
                    (unsigned long long)offset, (unsigned long long)bytes, arena);
    return BL_OK;
}

extern "C" int bl_arenas_write(bl_arenas *a, uint32_t arena, uint64_t offset, const void *src, uint64_t bytes) {
    if (!a || (bytes && !src)) return BL_ERR_INVALID_ARGUMENT;
    if (int r = check_range(a, arena, offset, bytes)) return r;
    if (!bytes) return BL_OK;
    hipSetDevice(a->ctx->device);
    hipError_t e = hipMemcpyAsync(a->base + a->offset[arena] + offset, src, bytes, hipMemcpyHostToDevice,
                                  a->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(a->ctx->stream);
    arenas_written(a, arena, offset, bytes);
    return e == hipSuccess ? BL_OK : hip_fail(a->ctx, e, "arena write");
}

extern "C" int bl_arenas_invalidate(bl_arenas *a, uint32_t arena, uint64_t offset, uint64_t bytes) {
    if (!a) return BL_ERR_INVALID_ARGUMENT;
    if (int r = check_range(a, arena, offset, bytes)) return r;
    if (bytes) arenas_written(a, arena, offset, bytes);
    return BL_OK;
}

extern "C" int bl_arenas_read(bl_arenas *a, uint32_t arena, uint64_t offset, void *dst, uint64_t bytes) {
    if (!a || (bytes && !dst)) return BL_ERR_INVALID_ARGUMENT;
    if (int r = check_range(a, arena, offset, bytes)) return r;
    if (!bytes) return BL_OK;
    hipSetDevice(a->ctx->device);
    hipError_t e = hipMemcpyAsync(dst, a->base + a->offset[arena] + offset, bytes, hipMemcpyDeviceToHost,
                                  a->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(a->ctx->stream);
    return e == hipSuccess ? BL_OK : hip_fail(a->ctx, e, "arena read");
}

extern "C" int bl_arenas_device_ptr(bl_arenas *a, uint32_t arena, uint64_t offset, void **out) {
    if (!a || !out) return BL_ERR_INVALID_ARGUMENT;
    if (int r = check_range(a, arena, offset, 0)) return r;
    *out = a->base + a->offset[arena] + offset;
    return BL_OK;
}

// ---- kernels ----

namespace {

enum class Family { LAYER_NORM, GEMM, GATHER, SOFTMAX, FLASH, ELEMENT, DPT, GEMV };

struct Launch {
    Family family;
    Math math = Math::F32;
    int tile = 0;
    int pack = -1;  // the packed B a GEMM reads
    bool f16 = false;
    Gather gather = Gather::SCORES;
    PerElement element = PerElement::MAP;
    LayerNormArgs ln;
    GemmArgs gemm;
    GatherArgs ga;
    SoftmaxArgs sm;
    FlashArgs fl;
    ElementArgs el;
    Dpt dpt = Dpt::RESIZE;
    DptArgs dp;
    GemvArgs gv;
    // The output's bytes (what the launch writes, the scratch aside).
    const char *out_lo = nullptr, *out_hi = nullptr;
    // A flash kernel whose QKV projections write its K and Vt (fl.prepped):
    // those projection kernels (one per part). kv_rerun: they store qkv's
    // queries alone, so the flash kernel cannot make K and Vt from qkv and
    // runs them again when the scratch does not hold its operands.
    std::vector<uint32_t> kv_producers;
    bool kv_rerun = false;
    // A LayerNorm folded into the product that reads it (fold >= 0): the
    // LayerNorm itself launches nothing, the product applies it (FOLD_CONSUMER),
    // and the product that wrote its input leaves the input's statistics
    // (FOLD_PRODUCER). Both the LayerNorm and the consumer first make the
    // statistics from x when the producer has not written them since x changed.
    int fold = -1;
    int fold_role = 0;
    // A class-token prepend fused into the patch embedding before it: it
    // launches nothing (the product writes its output).
    bool fused = false;
};
enum FoldRole : int { FOLD_NONE = 0, FOLD_LAYER_NORM = 1, FOLD_CONSUMER = 2, FOLD_PRODUCER = 3 };

struct Kernel {
    std::string label;
    std::vector<Launch> per_set;
};

// A packed copy of one B operand (a weight matrix), remade before the next
// launch that reads it once the host has written (or invalidated) any of the
// bytes it is packed from, or before every launch when a kernel of the
// program writes those bytes.
struct Pack {
    Math math;
    const void *src;
    uint32_t arena;
    uint64_t offset, size;
    uint32_t k, n, k_pad, n_pad;
    uint64_t dst_offset;  // into the kernels' pack buffer
    bool stale = true;
    bool dynamic = false;
    // A folded LayerNorm's pack: B's rows scaled by gamma, then the column
    // vectors c and d (PackArgs) at vec_offset. Its sources: gamma, beta and
    // the bias (null when the product has none), each an arena range.
    struct Source {
        const void *ptr = nullptr;
        uint32_t arena = 0;
        uint64_t offset = 0, size = 0;
    };
    Source gamma, beta, bias;
    uint64_t vec_offset = 0;
    bool used = false;
    bool frag = false;  // fragment-major (packed_at): every reader takes B in registers
    bool folded() const { return gamma.ptr != nullptr; }
    bool reads(uint32_t a, uint64_t off, uint64_t bytes) const {
        auto hit = [&](uint32_t ar, uint64_t o, uint64_t sz) { return sz && ar == a && off < o + sz && o < off + bytes; };
        return hit(arena, offset, size) || hit(gamma.arena, gamma.offset, gamma.size) ||
               hit(beta.arena, beta.offset, beta.size) || hit(bias.arena, bias.offset, bias.size);
    }
};

// Bytes of a folded pack's column vectors: c [n_pad], d [n_pad], then the
// per-block column sums cb [n_pad][32].
inline uint64_t fold_vec_bytes(uint32_t n_pad) { return (uint64_t)(2 + 32) * n_pad * sizeof(float); }

// One LayerNorm folded into the product that reads its output. Per binding
// set: x's bytes (the LayerNorm's input) and the statistics launch that makes
// the fold's buffers from x.
struct Fold {
    uint32_t ln, consumer, producer;
    std::vector<const char *> x_lo, x_hi;
    std::vector<LnStatsArgs> stats;
};

const char *main_name(uint32_t m) {
    switch (m) {
    case BL_MAIN_LAYER_NORM: return "layernorm";
    case BL_MAIN_MATMUL: return "matmul";
    case BL_MAIN_ATTENTION_SCORES: return "attention_scores";
    case BL_MAIN_SOFTMAX: return "softmax";
    case BL_MAIN_ATTENTION_VALUES: return "attention_values";
    case BL_MAIN_PATCH_EMBED: return "patch_embed";
    case BL_MAIN_PREPEND_TOKEN: return "prepend_token";
    case BL_MAIN_TOKENS_TO_MAP: return "tokens_to_map";
    case BL_MAIN_MAP: return "map";
    case BL_MAIN_FLASH_ATTENTION: return "flash_attention";
    case BL_MAIN_CONV3X3: return "conv2d3x3";
    case BL_MAIN_CONV_TRANSPOSE: return "conv_transpose2d";
    case BL_MAIN_RESIZE_BILINEAR: return "resize_bilinear";
    default: return nullptr;
    }
}

const char *epi_name(uint32_t k) {
    switch (k) {
    case BL_EPI_ADD: return "add";
    case BL_EPI_RELU: return "relu";
    case BL_EPI_GELU: return "gelu";
    case BL_EPI_GELU_ERF: return "gelu_erf";
    case BL_EPI_SCALE: return "scale";
    case BL_EPI_CHANNEL_SCALE: return "channel_scale";
    default: return nullptr;
    }
}

uint64_t mul(std::initializer_list<uint64_t> v) {
    uint64_t r = 1;
    for (uint64_t x : v) r *= x;
    return r;
}

// What a spec's main operation reads and writes, in elements; its split
// extent and grain (MainOp::split_extent / split_grain, kernel.rs:1521-1543).
struct Shape {
    std::vector<uint64_t> reads;
    uint64_t out = 0;
    uint32_t extent = 0;
    uint32_t grain = 1;
    uint64_t per_unit = 1;  // output elements per unit of the split dimension
};

bool shape_of(const bl_spec &s, Shape &sh, std::string &why) {
    const uint32_t *d = s.dims;
    switch (s.main) {
    case BL_MAIN_LAYER_NORM:
        sh.reads = {mul({d[0], d[1]}), d[1], d[1]};
        sh.out = mul({d[0], d[1]});
        sh.extent = d[0];
        sh.per_unit = d[1];
        if (!(s.epsilon > 0.0f && s.epsilon < 1e30f)) { why = "layer norm epsilon is not finite and positive"; return false; }
        return d[0] && d[1];
    case BL_MAIN_MATMUL:
        sh.reads = {mul({d[0], d[1]}), mul({d[1], d[2]})};
        if (d[3]) sh.reads.push_back(d[2]);
        sh.out = mul({d[0], d[2]});
        sh.extent = d[0];
        sh.grain = 64;
        sh.per_unit = d[2];
        return d[0] && d[1] && d[2];
    case BL_MAIN_ATTENTION_SCORES:
        sh.reads = {mul({d[0], 3, d[1], d[2]})};
        sh.out = mul({d[0], d[1], d[0]});
        sh.extent = d[0];
        sh.grain = 64;
        sh.per_unit = mul({d[1], d[0]});
        return d[0] && d[1] && d[2];
    case BL_MAIN_SOFTMAX:
        sh.reads = {mul({d[0], d[1]})};
        sh.out = mul({d[0], d[1]});
        sh.extent = d[0];
        sh.per_unit = d[1];
        return d[0] && d[1];
    case BL_MAIN_ATTENTION_VALUES:
        sh.reads = {mul({d[0], d[1], d[0]}), mul({d[0], 3, d[1], d[2]})};
        sh.out = mul({d[0], d[1], d[2]});
        sh.extent = d[0];
        sh.grain = 64;
        sh.per_unit = mul({d[1], d[2]});
        return d[0] && d[1] && d[2];
    case BL_MAIN_PATCH_EMBED:
        sh.reads = {mul({d[0], d[2], d[1], d[2], d[3]}), mul({d[2], d[2], d[3], d[4]})};
        if (d[5]) sh.reads.push_back(d[4]);
        sh.out = mul({d[0], d[1], d[4]});
        sh.extent = d[0] * d[1];
        sh.grain = 64;
        sh.per_unit = d[4];
        return d[0] && d[1] && d[2] && d[3] && d[4];
    case BL_MAIN_PREPEND_TOKEN:
        sh.reads = {d[1], mul({d[0], d[1]})};
        sh.out = mul({(uint64_t)d[0] + 1, d[1]});
        sh.extent = (uint32_t)sh.out;
        return d[0] && d[1];
    case BL_MAIN_TOKENS_TO_MAP:
        sh.reads = {(mul({d[0], d[1]}) + 1) * d[2]};
        sh.out = mul({d[0], d[1], d[2]});
        sh.extent = (uint32_t)sh.out;
        return d[0] && d[1] && d[2];
    case BL_MAIN_MAP:
        sh.reads = {d[0]};
        sh.out = d[0];
        sh.extent = d[0];
        return d[0] != 0;
    case BL_MAIN_CONV3X3: {
        if (!d[4]) { why = "a stride of zero"; return false; }
        const uint64_t oh = (d[0] - 1) / d[4] + 1, ow = (d[1] - 1) / d[4] + 1;
        sh.reads = {mul({d[0], d[1], d[2]}), mul({9, d[2], d[3]})};
        if (d[5]) sh.reads.push_back(d[3]);
        sh.out = mul({oh, ow, d[3]});
        sh.extent = (uint32_t)std::min<uint64_t>(oh * ow, UINT32_MAX);
        sh.grain = 64;
        sh.per_unit = d[3];
        return d[0] && d[1] && d[2] && d[3];
    }
    case BL_MAIN_CONV_TRANSPOSE:
        sh.reads = {mul({d[0], d[1], d[2]}), mul({d[4], d[4], d[2], d[3]})};
        if (d[5]) sh.reads.push_back(d[3]);
        sh.out = mul({d[0], d[4], d[1], d[4], d[3]});
        sh.extent = (uint32_t)std::min<uint64_t>(mul({d[0], d[4], d[1], d[4]}), UINT32_MAX);
        sh.per_unit = d[3];
        return d[0] && d[1] && d[2] && d[3] && d[4];
    case BL_MAIN_RESIZE_BILINEAR:
        sh.reads = {mul({d[0], d[1], d[4]})};
        sh.out = mul({d[2], d[3], d[4]});
        sh.extent = (uint32_t)std::min<uint64_t>(mul({d[2], d[3]}), UINT32_MAX);
        sh.per_unit = d[4];
        return d[0] && d[1] && d[2] && d[3] && d[4];
    case BL_MAIN_FLASH_ATTENTION:
        sh.reads = {mul({d[0], 3, d[1], d[2]})};
        sh.out = mul({d[0], d[1], d[2]});
        sh.extent = d[0];
        sh.grain = 64;
        sh.per_unit = mul({d[1], d[2]});
        if (d[2] != FLASH_HEAD_DIM) { why = "the flash kernel needs a head width of 64"; return false; }
        if (!(s.scale == s.scale) || s.scale == INFINITY || s.scale == -INFINITY) { why = "non-finite scale"; return false; }
        return d[0] && d[1];
    default:
        why = "unknown main operation";
        return false;
    }
}

uint64_t round4(uint64_t bytes) { return (bytes + 3) / 4 * 4; }

}  // namespace

// What the shared attention scratch holds: the K and Vt operands made from
// the qkv tensor at `qkv` (null: nothing known), written by the projection
// kernels in `done` (each writes its part's rows) or, when `whole`, by a flash
// kernel's own prep from all of qkv. Nothing has written qkv's bytes since.
struct KvState {
    const void *qkv = nullptr;
    const char *lo = nullptr, *hi = nullptr;  // qkv's bytes
    bool whole = false;
    std::vector<uint32_t> done;
};

// A range of kernels captured once as a HIP graph and replayed by
// bl_kernels_encode_range: one submission instead of one per launch. `kv`
// is what the attention scratch holds after a replay.
// Whether each (fold, set)'s statistics describe x as it now is, and which
// entries a range of launches set (what a graph replay of the range does).
struct FoldState {
    std::vector<uint8_t> valid, touched;
};

struct RangeGraph {
    uint32_t first, count, set;
    hipGraphExec_t exec;
    KvState entry;  // what the scratch held when the range was captured
    KvState kv;
    FoldState folds;  // the entries the range sets (touched) and their values after it
    uint32_t launches;  // kernel nodes of the captured graph
};

struct bl_kernels {
    bl_ctx *ctx = nullptr;
    bl_arenas *arenas = nullptr;
    std::vector<Kernel> kernels;
    uint32_t sets = 1;
    // The one allocation holding the packed weights, the attention scratch,
    // the split-k partial sums and the folds' buffers, placed by lifetime.
    char *workspace = nullptr;
    uint64_t workspace_bytes = 0;
    void *scratch = nullptr;
    std::vector<Pack> packs;
    void *pack_buffer = nullptr;
    uint64_t packs_made = 0;
    KvState kv;
    std::vector<Fold> folds;
    FoldState fold_state;  // [fold * sets + set]
    // Fold entries ([fold * sets + set]) whose workspace bytes another entry
    // shares (their lifetimes are disjoint), and per kernel the entries its
    // split-k partial sums overwrite: writing one makes the others stale.
    std::vector<std::vector<uint32_t>> fold_alias, kernel_clobbers;
    std::vector<RangeGraph> graphs;
    // Graphs replay fixed launches: not used when a kernel of the program
    // rewrites a packed weight's source (the pack must rerun in between),
    // when BL_NO_GRAPH is set, or under rocprofv3.
    bool graphs_ok = true;
};

static void kernels_written(bl_kernels *k, uint32_t arena, uint64_t offset, uint64_t bytes) {
    for (Pack &pk : k->packs)
        if (pk.reads(arena, offset, bytes)) pk.stale = true;
    // The attention scratch is made from qkv: any host write may have changed it.
    k->kv = KvState{};
    // So may any folded LayerNorm's input.
    std::fill(k->fold_state.valid.begin(), k->fold_state.valid.end(), 0);
}

namespace {

// Activations stored as hi and lo bf16 planes (bf16x3 math): tensors the host
// named internal, written by a LayerNorm, a GEMM or a flash attention kernel,
// and read by nothing but the pipelined GEMM as its A operand. Each producer
// launch gets the plane distance of its output, each reader of its A.
void keep_split_activations(bl_kernels *ks, const bl_spec *specs, uint32_t n, const uint32_t *internal,
                            uint32_t n_internal) {
    struct Use {
        std::vector<uint32_t> producers, readers;
        bool other = false;
    };
    std::vector<uint32_t> ids(internal, internal + n_internal);
    std::sort(ids.begin(), ids.end());
    auto is_internal = [&](uint32_t t) { return std::binary_search(ids.begin(), ids.end(), t); };
    std::vector<std::pair<uint32_t, Use>> uses;
    auto use_of = [&](uint32_t t) -> Use & {
        for (auto &u : uses)
            if (u.first == t) return u.second;
        uses.push_back({t, Use{}});
        return uses.back().second;
    };
    for (uint32_t ki = 0; ki < n; ki++) {
        const bl_spec &s = specs[ki];
        const uint32_t last = s.n_bindings - 1;
        const uint32_t out_t = s.bindings[last].tensor;
        for (uint32_t b = 0; b < last; b++) {
            const uint32_t t = s.bindings[b].tensor;
            if (!is_internal(t)) continue;
            Use &u = use_of(t);
            // A pipelined GEMM's A, or a 3x3 convolution's image when its
            // ring kernel takes the fast window gather (channels a whole
            // k-step, the image under 2^31 elements, 9 cin under 2^16).
            const bool conv = s.main == BL_MAIN_CONV3X3;
            bool ok = (s.main == BL_MAIN_MATMUL || conv) && b == s.reads[0] && t != out_t;
            for (uint32_t c = 0; c < last && ok; c++)
                if (c != b && s.bindings[c].tensor == t) ok = false;  // also an epilogue operand or B
            for (uint32_t si = 0; si < ks->sets && ok; si++) {
                const Launch &L = ks->kernels[ki].per_set[si];
                const GemmArgs &g = L.gemm;
                ok = L.family == Family::GEMM && L.math == Math::SPLIT && L.gemm.pipeline &&
                     (conv ? g.load == 3 && gemm_tile_cols(L.tile) >= 64 && g.p2 % 32 == 0 &&
                                 (uint64_t)(g.p0 + 1) * (g.p1 + 1) * g.p2 < (1ull << 31) && 9ull * g.p2 < (1u << 16) &&
                                 !getenv("BL_CONV_NO_SPLIT_INPUT")
                          : g.load == 0 && g.k % 32 == 0);
            }
            if (ok) u.readers.push_back(ki);
            else u.other = true;
        }
        if (!is_internal(out_t)) continue;
        Use &u = use_of(out_t);
        bool ok = true;
        for (uint32_t si = 0; si < ks->sets && ok; si++) {
            const Launch &L = ks->kernels[ki].per_set[si];
            ok = L.math == Math::SPLIT && !L.f16 &&
                 (L.family == Family::LAYER_NORM || L.family == Family::FLASH ||
                  (L.family == Family::GEMM && L.gemm.load != 2 && !L.gemm.flash_ops));
        }
        if (ok) u.producers.push_back(ki);
        else u.other = true;
    }
    for (auto &[t, u] : uses) {
        if (u.other || u.producers.empty() || u.readers.empty()) continue;
        for (uint32_t ki : u.producers) {
            ks->kernels[ki].label += " > split";
            for (Launch &L : ks->kernels[ki].per_set) {
                if (L.family == Family::LAYER_NORM) L.ln.y_planes = (uint64_t)L.ln.rows * L.ln.channels;
                else if (L.family == Family::GEMM) L.gemm.c_planes = (uint64_t)L.gemm.m * L.gemm.n;
                else L.fl.out_planes = (uint64_t)L.fl.tokens * L.fl.heads * FLASH_HEAD_DIM;
            }
        }
        for (uint32_t ki : u.readers) {
            Kernel &K = ks->kernels[ki];
            K.label += " < split";
            for (Launch &L : K.per_set) {
                // The planes split the whole tensor: the image of a convolution.
                L.gemm.a_planes = L.gemm.load == 3 ? (uint64_t)L.gemm.p0 * L.gemm.p1 * L.gemm.p2 : (uint64_t)L.gemm.m * L.gemm.k;
                if (L.gemm.load == 3) continue;
                // Without the split in its k-steps the 32 x 64 tile with 64-wide
                // steps in a 3-stage ring beats the long-k rule's 64 x 64 tile
                // with four groups (fc2: 15.7 against 18.8 us).
                if (L.tile == TILE_64x64 && L.gemm.kgroups == 4 && !getenv("BL_GEMM_TILE") && !getenv("BL_GEMM_KGROUPS")) {
                    L.tile = TILE_32x64;
                    L.gemm.kgroups = 1;
                    L.gemm.stages = 3;
                    if (const char *force = getenv("BL_GEMM_STAGES")) L.gemm.stages = (uint32_t)atoi(force);
                    L.gemm.kslices = L.gemm.k % 64 == 0 ? 2 : 1;
                    const size_t at = K.label.find(" 64x64 k4");
                    if (at != std::string::npos) K.label.replace(at, 9, L.gemm.kslices == 2 ? " 32x64 bk64" : " 32x64");
                }
            }
        }
    }
}

// Resolves binding `b` of spec `s` through binding set `set`'s substitutions.
bl_binding resolve(const bl_spec &s, uint32_t b, const bl_binding_set &set) {
    bl_binding bd = s.bindings[b];
    for (uint32_t t = 0; t < set.count; t++)
        if (set.items[t].original == bd.tensor) {
            bd.arena = set.items[t].arena;
            bd.offset = set.items[t].offset;
        }
    return bd;
}

// The class-token prepend fused into the patch embedding that makes its rows
// (the embeddings' x = [token; patches] + pos): a prepend Q (whole) whose rows
// are an internal tensor written by nothing but the patch embedding P just
// before it (whole, no epilogue, not split) and read by nothing but Q. P then
// writes x's rows 1 .. m itself through Q's epilogue (its added tensors read
// one row on), its first row band also writes x's first row from the token,
// and Q launches nothing. Q's epilogue steps must not depend on where a row
// lies: adds of x-shaped tensors, scales, activations, channel scales over a
// divisor of the row.
void plan_prepends(bl_kernels *ks, const bl_spec *specs, uint32_t n, const uint32_t *internal, uint32_t n_internal) {
    if (!n_internal || getenv("BL_NO_PREPEND_FUSION")) return;
    std::vector<uint32_t> ids(internal, internal + n_internal);
    std::sort(ids.begin(), ids.end());
    for (uint32_t qi = 1; qi < n; qi++) {
        const bl_spec &qs = specs[qi];
        const uint32_t pi = qi - 1;
        const bl_spec &ps = specs[pi];
        if (qs.main != BL_MAIN_PREPEND_TOKEN || qs.part.count != 1 || ps.main != BL_MAIN_PATCH_EMBED ||
            ps.part.count != 1 || ps.n_epilogue)
            continue;
        const uint32_t rows_t = qs.bindings[qs.reads[1]].tensor;
        if (!std::binary_search(ids.begin(), ids.end(), rows_t) || ps.bindings[ps.n_bindings - 1].tensor != rows_t) continue;
        bool ok = true;
        for (uint32_t ki = 0; ki < n && ok; ki++) {
            const bl_spec &s = specs[ki];
            const uint32_t last = s.n_bindings - 1;
            if (ki != pi && s.bindings[last].tensor == rows_t) ok = false;
            for (uint32_t b = 0; b < last; b++)
                if (s.bindings[b].tensor == rows_t && !(ki == qi && b == qs.reads[1])) ok = false;
        }
        for (uint32_t si = 0; si < ks->sets && ok; si++) {
            const Launch &P = ks->kernels[pi].per_set[si];
            const Launch &Q = ks->kernels[qi].per_set[si];
            const GemmArgs &g = P.gemm;
            ok = P.family == Family::GEMM && Q.family == Family::ELEMENT && Q.element == PerElement::PREPEND &&
                 g.load == 2 && g.ksplit <= 1 && !g.flash_ops && !g.c_planes && g.epi_mode == 0 && g.row0 == 0 &&
                 g.row1 == g.m && g.n == Q.el.channels && Q.el.start == 0 &&
                 Q.el.end == (uint64_t)(g.m + 1) * g.n && P.out_lo == (const char *)Q.el.b && P.f16 == Q.f16;
            for (int k = 0; k < Q.el.epi.n && ok; k++) {
                const int kind = Q.el.epi.kind[k];
                ok = kind == BL_EPI_ADD || kind == BL_EPI_RELU || kind == BL_EPI_GELU || kind == BL_EPI_GELU_ERF ||
                     kind == BL_EPI_SCALE || (kind == BL_EPI_CHANNEL_SCALE && Q.el.epi.channels[k] && g.n % Q.el.epi.channels[k] == 0);
            }
        }
        if (!ok) continue;
        for (uint32_t si = 0; si < ks->sets; si++) {
            Launch &P = ks->kernels[pi].per_set[si];
            Launch &Q = ks->kernels[qi].per_set[si];
            GemmArgs &g = P.gemm;
            const uint64_t row_bytes = (uint64_t)g.n * (P.f16 ? 2 : 4);
            g.c = (char *)Q.el.y + row_bytes;
            g.epi = Q.el.epi;
            for (int k = 0; k < g.epi.n; k++)
                if (g.epi.kind[k] == BL_EPI_ADD) g.epi.operand[k] = (const char *)g.epi.operand[k] + row_bytes;
            g.epi_mode = 3;
            g.cls_token = Q.el.a;
            g.cls_out = Q.el.y;
            g.cls_epi = Q.el.epi;
            P.out_lo = Q.out_lo;
            P.out_hi = Q.out_hi;
            Q.fused = true;
            Q.out_lo = Q.out_hi = nullptr;
        }
        ks->kernels[qi].label += " > fused into " + std::to_string(pi);
        ks->kernels[pi].label += " < prepend " + std::to_string(qi);
    }
}

// LayerNorms folded into the products that read them. A LayerNorm L (no
// epilogue, whole) over x [rows][D] whose output n is internal and read by
// nothing but one later product G, as G's A (G whole, the ring kernel, plain
// rows, k = D, D a multiple of 32), while x was last written before L by a
// product P (whole, no split k, its output exactly x, whole 32-column blocks
// per wave) or by the class-token prepend (whole, the token whole blocks), and
// nothing writes x between L and G:
//   LN(x) W + b = rstd (x (gamma W) - mean c) + d,  c = column sums of gamma W,
//   d = beta W + b,
// so G reads x itself (its bf16 planes for bf16x3) with a pack of gamma W and
// applies mean and rstd per row in its epilogue; P (its epilogue, or the
// prepend's stats kernel) leaves each row's 32-column block statistics (and
// the planes). L launches nothing.
void plan_folds(bl_kernels *ks, const bl_spec *specs, uint32_t n, const bl_binding_set *sets, uint32_t n_sets,
                const uint32_t *internal, uint32_t n_internal) {
    if (!n_internal || getenv("BL_NO_LN_FOLD")) return;
    std::vector<uint32_t> ids(internal, internal + n_internal);
    std::sort(ids.begin(), ids.end());
    auto is_internal = [&](uint32_t t) { return std::binary_search(ids.begin(), ids.end(), t); };
    auto overlaps = [](const Launch &L, const char *lo, const char *hi) { return L.out_lo < hi && lo < L.out_hi; };
    std::vector<uint8_t> producing(n, 0);
    for (uint32_t li = 0; li < n; li++) {
        const bl_spec &ls = specs[li];
        if (ls.main != BL_MAIN_LAYER_NORM || ls.n_epilogue || ls.part.count != 1) continue;
        const uint32_t out_t = ls.bindings[ls.n_bindings - 1].tensor;
        if (!is_internal(out_t)) continue;
        const uint32_t D = ls.dims[1];
        if (D % 32 != 0 || ls.part.start != 0 || ls.part.end != ls.dims[0]) continue;
        // The one reader of the LayerNorm's output: a later product's A.
        int gi = -1;
        bool ok = true;
        for (uint32_t ki = 0; ki < n && ok; ki++) {
            const bl_spec &s = specs[ki];
            for (uint32_t b = 0; b + 1 < s.n_bindings; b++) {
                if (s.bindings[b].tensor != out_t) continue;
                if (gi >= 0 || ki <= li || s.main != BL_MAIN_MATMUL || b != s.reads[0]) ok = false;
                else gi = (int)ki;
            }
        }
        if (!ok || gi < 0) continue;
        const bl_spec &gs = specs[gi];
        if (gs.part.count != 1) continue;
        for (uint32_t b = 0; b + 1 < gs.n_bindings; b++)
            if (b != gs.reads[0] && gs.bindings[b].tensor == out_t) ok = false;
        int pi = -1;
        for (uint32_t si = 0; si < n_sets && ok; si++) {
            const Launch &Ln = ks->kernels[li].per_set[si];
            const Launch &G = ks->kernels[gi].per_set[si];
            // The consumer's prologue takes one quad of invocations per tile row
            // (in two passes for an f16 tile of 128 rows) and whole pairs of
            // 32-column blocks, at most 16 of them.
            const int fold_rows = G.math == Math::F16 ? 128 : 64;
            if (Ln.family != Family::LAYER_NORM || G.family != Family::GEMM || !G.gemm.pipeline || G.gemm.load != 0 ||
                gemm_tile_rows(G.tile) > fold_rows || D > 1024 || D % 64 != 0 ||
                G.gemm.ksplit > 1 || G.gemm.k != D || G.gemm.m != ls.dims[0] || G.gemm.row0 != 0 || G.gemm.row1 != G.gemm.m) {
                ok = false;
                break;
            }
            const bl_binding xb = resolve(ls, ls.reads[0], sets[si]);
            const char *x_lo = (const char *)Ln.ln.x, *x_hi = x_lo + xb.size;
            // Nothing writes x between the LayerNorm and its reader.
            for (uint32_t j = li + 1; j < (uint32_t)gi && ok; j++)
                if (overlaps(ks->kernels[j].per_set[si], x_lo, x_hi)) ok = false;
            // x's last writer before the LayerNorm, a product writing exactly x.
            int p = -1;
            for (uint32_t j = li; j-- > 0;)
                if (overlaps(ks->kernels[j].per_set[si], x_lo, x_hi)) {
                    p = (int)j;
                    break;
                }
            if (p < 0 || (pi >= 0 && p != pi) || producing[p]) {
                ok = false;
                break;
            }
            pi = p;
            const Launch &P = ks->kernels[p].per_set[si];
            const bl_spec &ps = specs[p];
            if (P.family == Family::ELEMENT) {
                // The class-token prepend writing all of x (its token whole blocks).
                // Its stats kernel loads and stores 16 bytes at a time.
                auto a16 = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
                bool al = a16(P.el.a) && a16(P.el.b) && a16(P.el.y);
                for (int k = 0; k < P.el.epi.n; k++)
                    if (P.el.epi.kind[k] == BL_EPI_ADD) al = al && a16(P.el.epi.operand[k]);
                if (P.element != PerElement::PREPEND || ps.part.count != 1 || P.out_lo != x_lo || P.out_hi != x_hi ||
                    P.el.start != 0 || P.el.end != (uint64_t)ls.dims[0] * D || P.el.channels % 32 != 0 || P.f16 != G.f16 ||
                    !al)
                    ok = false;
            } else if (P.family != Family::GEMM || ps.part.count != 1 || P.gemm.ksplit > 1 || P.gemm.flash_ops ||
                       P.gemm.c_planes || P.out_lo != x_lo || P.out_hi != x_hi || P.gemm.n != D ||
                       P.gemm.m + (P.gemm.cls_out ? 1 : 0) != ls.dims[0] || P.gemm.row0 != 0 || P.gemm.row1 != P.gemm.m ||
                       (gemm_tile_cols(P.tile) / 2) % 32 != 0 || P.math != G.math) {
                ok = false;
            }
        }
        if (!ok || pi < 0) continue;
        const uint32_t f = (uint32_t)ks->folds.size();
        Fold fo{li, (uint32_t)gi, (uint32_t)pi, {}, {}, {}};
        producing[pi] = 1;
        for (uint32_t si = 0; si < n_sets; si++) {
            Launch &Ln = ks->kernels[li].per_set[si];
            Launch &G = ks->kernels[gi].per_set[si];
            Launch &P = ks->kernels[pi].per_set[si];
            const bl_binding xb = resolve(ls, ls.reads[0], sets[si]);
            fo.x_lo.push_back((const char *)Ln.ln.x);
            fo.x_hi.push_back((const char *)Ln.ln.x + xb.size);
            LnStatsArgs sa{};
            sa.x = Ln.ln.x;
            sa.rows = ls.dims[0];
            sa.cols = D;
            fo.stats.push_back(sa);
            Ln.fold = G.fold = P.fold = (int)f;
            Ln.fold_role = FOLD_LAYER_NORM;
            G.fold_role = FOLD_CONSUMER;
            P.fold_role = FOLD_PRODUCER;
            // The consumer's own pack: gamma W with the column vectors.
            Pack pk = ks->packs[G.pack];
            pk.stale = true;
            pk.dynamic = false;
            auto src = [&](const bl_spec &sp, uint32_t b, const void *ptr) {
                const bl_binding bd = resolve(sp, b, sets[si]);
                Pack::Source so;
                so.ptr = ptr;
                so.arena = bd.arena;
                so.offset = bd.offset;
                so.size = bd.size;
                return so;
            };
            pk.gamma = src(ls, ls.reads[1], Ln.ln.gamma);
            pk.beta = src(ls, ls.reads[2], Ln.ln.beta);
            pk.bias = G.gemm.bias ? src(gs, gs.reads[2], G.gemm.bias) : Pack::Source{};
            int found = -1;
            for (size_t q = 0; q < ks->packs.size(); q++) {
                const Pack &o = ks->packs[q];
                if (o.folded() && o.math == pk.math && o.arena == pk.arena && o.offset == pk.offset && o.k == pk.k &&
                    o.n == pk.n && o.gamma.ptr == pk.gamma.ptr && o.beta.ptr == pk.beta.ptr && o.bias.ptr == pk.bias.ptr)
                    found = (int)q;
            }
            if (found < 0) {
                ks->packs.push_back(pk);
                found = (int)ks->packs.size() - 1;
            }
            G.pack = found;
        }
        ks->folds.push_back(std::move(fo));
        ks->kernels[li].label += " > folded into " + std::to_string(gi);
        ks->kernels[gi].label += " < layernorm " + std::to_string(li);
        ks->kernels[pi].label += " > row statistics";
    }
    ks->fold_state.valid.assign(ks->folds.size() * n_sets, 0);
    ks->fold_state.touched.assign(ks->folds.size() * n_sets, 0);
}

// Bytes of a fold's buffers for one binding set: the statistics, then (f32
// storage) x centred per block, as bf16 planes (bf16x3) or f32.
uint64_t fold_stats_bytes(const Fold &f) { return (uint64_t)f.stats[0].rows * (f.stats[0].cols / 32) * 8; }
uint64_t fold_plane_bytes(const Fold &f, const Launch &G) {
    return G.math != Math::F16 ? (uint64_t)f.stats[0].rows * f.stats[0].cols * 4 : 0;
}

// Points the folds' launches at their buffers (after the split activations
// are chosen: the consumer reads x, or x's planes, whatever it read before).
void apply_folds(bl_kernels *ks) {
    for (Fold &f : ks->folds) {
        for (uint32_t si = 0; si < ks->sets; si++) {
            Launch &G = ks->kernels[f.consumer].per_set[si];
            Launch &P = ks->kernels[f.producer].per_set[si];
            const Launch &Ln = ks->kernels[f.ln].per_set[si];
            const LnStatsArgs &sa = f.stats[si];
            const Pack &pk = ks->packs[G.pack];
            // The shadow (f32 storage): x centred per block, as bf16 planes
            // sa.planes elements apart (bf16x3) or as f32 (sa.planes 0).
            const uint64_t shadow_elt = sa.planes ? 2 : 4;
            if (P.family == Family::ELEMENT) {
                P.el.ln_out = sa.stats;
                P.el.ln_shadow = sa.shadow;
                P.el.ln_cols = sa.cols;
                P.el.ln_plane = sa.planes;
            } else if (P.gemm.cls_out) {
                // The product's rows are x's rows 1 .. m; its first row band writes row 0.
                P.gemm.ln_out = sa.stats + 2 * (sa.cols / 32);
                P.gemm.ln_shadow = sa.shadow ? (char *)sa.shadow + (uint64_t)sa.cols * shadow_elt : nullptr;
                P.gemm.ln_plane = sa.planes;
                P.gemm.cls_ln_out = sa.stats;
                P.gemm.cls_shadow = sa.shadow;
            } else {
                P.gemm.ln_out = sa.stats;
                P.gemm.ln_shadow = sa.shadow;
                P.gemm.ln_plane = sa.planes;
            }
            G.gemm.a = sa.shadow ? sa.shadow : sa.x;
            G.gemm.a_planes = sa.shadow ? sa.planes : 0;
            G.gemm.ln_stats = sa.stats;
            G.gemm.ln_c = (const float *)((char *)ks->pack_buffer + pk.vec_offset);
            G.gemm.ln_d = G.gemm.ln_c + pk.n_pad;
            G.gemm.ln_cb = sa.shadow ? G.gemm.ln_c + 2 * (uint64_t)pk.n_pad : nullptr;
            G.gemm.ln_blocks = sa.cols / 32;
            G.gemm.ln_eps = Ln.ln.eps;
            G.gemm.bias = nullptr;
        }
    }
}

}  // namespace

extern "C" int bl_kernels_create(bl_ctx *ctx, bl_arenas *arenas, const bl_spec *specs, uint32_t n,
                                 const bl_binding_set *sets, uint32_t n_sets, bl_kernels **out) {
    return bl_kernels_create_internal(ctx, arenas, specs, n, sets, n_sets, nullptr, 0, out);
}

namespace {

// One item of the backend's workspace: its bytes, the kernels from its first
// writer to its last reader (inclusive), its binding set (-1: any), and its
// offset once placed.
struct WsItem {
    uint64_t size;
    uint32_t first, last;
    int set;
    uint64_t at;
};

// Places the items as the memory plan places tensors in an arena
// (memory.rs:285-338): by size, descending (ties in item order), each at the
// lowest 256-byte aligned offset clear of every placed item it may be live
// with. Items of two different binding sets are taken to be live together
// (a frame loop may interleave the sets' ranges); otherwise two items are
// live together when their kernel intervals overlap. Returns the bytes the
// placement spans.
uint64_t place_workspace(std::vector<WsItem> &items) {
    std::vector<size_t> order(items.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = i;
    std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return items[a].size > items[b].size; });
    auto together = [&](const WsItem &a, const WsItem &b) {
        if (a.set >= 0 && b.set >= 0 && a.set != b.set) return true;
        return a.first <= b.last && b.first <= a.last;
    };
    std::vector<size_t> placed;
    uint64_t total = 0;
    for (size_t i : order) {
        WsItem &it = items[i];
        std::vector<std::pair<uint64_t, uint64_t>> busy;
        for (size_t j : placed)
            if (together(it, items[j])) busy.push_back({items[j].at, items[j].at + items[j].size});
        std::sort(busy.begin(), busy.end());
        uint64_t at = 0;
        for (auto [lo, hi] : busy) {
            if (at + it.size <= lo) break;
            at = std::max(at, (hi + 255) / 256 * 256);
        }
        it.at = at;
        total = std::max(total, at + it.size);
        placed.push_back(i);
    }
    return total;
}

}  // namespace

extern "C" int bl_kernels_create_internal(bl_ctx *ctx, bl_arenas *arenas, const bl_spec *specs, uint32_t n,
                                          const bl_binding_set *sets, uint32_t n_sets, const uint32_t *internal,
                                          uint32_t n_internal, bl_kernels **out) {
    if (!ctx || !arenas || !out || (n && !specs) || (n_sets && !sets) || (n_internal && !internal))
        return BL_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    hipSetDevice(ctx->device);
    const bl_binding_set identity{nullptr, 0};
    if (n_sets == 0) {
        sets = &identity;
        n_sets = 1;
    }
    auto *ks = new bl_kernels();
    ks->ctx = ctx;
    ks->arenas = arenas;
    ks->sets = n_sets;
    uint64_t scratch_bytes = 0;
    uint64_t flash_counter_bytes = 0;  // the largest in-kernel merge's arrival counters
    std::vector<std::pair<size_t, size_t>> flash_users;  // (kernel, set) whose FlashArgs need scratch
    std::vector<std::pair<size_t, size_t>> split_users;  // (kernel, set) of split-k GEMMs

    auto bad = [&](int code, const char *fmt, auto... args) {
        bl_device_free(ctx, ks->workspace, ks->workspace_bytes);
        delete ks;
        return fail(ctx, code, fmt, args...);
    };

    for (uint32_t ki = 0; ki < n; ki++) {
        const bl_spec &s = specs[ki];
        const char *mname = main_name(s.main);
        if (!mname) return bad(BL_ERR_KERNEL, "kernel %u: unknown main operation %u", ki, s.main);
        std::string name = mname;
        for (uint32_t e = 0; e < s.n_epilogue && e < BL_MAX_EPILOGUE; e++) {
            const char *en = epi_name(s.epilogue[e].kind);
            if (!en) return bad(BL_ERR_KERNEL, "kernel %u: unknown epilogue step %u", ki, s.epilogue[e].kind);
            name += "+";
            name += en;
        }
        Shape sh;
        std::string why;
        if (!shape_of(s, sh, why))
            return bad(BL_ERR_KERNEL, "kernel %s: %s", name.c_str(), why.empty() ? "a zero dimension" : why.c_str());
        if (s.n_bindings < 2 || s.n_bindings > BL_MAX_BINDINGS || s.n_epilogue > BL_MAX_EPILOGUE)
            return bad(BL_ERR_KERNEL, "kernel %s: %u bindings", name.c_str(), s.n_bindings);
        if (s.n_reads != sh.reads.size())
            return bad(BL_ERR_KERNEL, "kernel %s: main operation reads %zu tensors, spec names %u", name.c_str(),
                       sh.reads.size(), s.n_reads);
        const uint32_t dtype = s.bindings[0].dtype;
        if (dtype != BL_F32 && dtype != BL_F16) return bad(BL_ERR_KERNEL, "kernel %s: unknown dtype", name.c_str());
        const uint64_t esz = dtype == BL_F16 ? 2 : 4;
        for (uint32_t b = 0; b < s.n_bindings; b++)
            if (s.bindings[b].dtype != dtype)
                return bad(BL_ERR_KERNEL, "kernel %s: bindings of mixed element types", name.c_str());
        // Every binding's placement holds what the operation's shape says.
        std::vector<uint64_t> need(s.n_bindings, 0);
        for (uint32_t r = 0; r < s.n_reads; r++) {
            if (s.reads[r] >= s.n_bindings - 1)
                return bad(BL_ERR_KERNEL, "kernel %s: read %u names binding %u", name.c_str(), r, s.reads[r]);
            need[s.reads[r]] = round4(sh.reads[r] * esz);
        }
        need[s.n_bindings - 1] = round4(sh.out * esz);
        for (uint32_t e = 0; e < s.n_epilogue; e++) {
            const bl_epilogue &ep = s.epilogue[e];
            if (ep.kind == BL_EPI_ADD || ep.kind == BL_EPI_CHANNEL_SCALE) {
                if (ep.operand >= s.n_bindings - 1)
                    return bad(BL_ERR_KERNEL, "kernel %s: epilogue step %u names binding %u", name.c_str(), e,
                               ep.operand);
                uint64_t el = sh.out;
                if (ep.kind == BL_EPI_CHANNEL_SCALE) {
                    if (!ep.channels || sh.out % ep.channels)
                        return bad(BL_ERR_KERNEL, "kernel %s: channel scale of %u channels", name.c_str(), ep.channels);
                    el = ep.channels;
                }
                need[ep.operand] = round4(el * esz);
            }
        }
        for (uint32_t b = 0; b < s.n_bindings; b++)
            if (need[b] == 0 || s.bindings[b].size != need[b])
                return bad(BL_ERR_KERNEL, "kernel %s: binding %u (tensor %u) is %llu bytes, the shape needs %llu",
                           name.c_str(), b, s.bindings[b].tensor, (unsigned long long)s.bindings[b].size,
                           (unsigned long long)need[b]);
        // The part: a non-empty range of the split dimension, starting on the grain.
        const bl_part &pt = s.part;
        if (pt.count == 0 || pt.index >= pt.count || pt.start >= pt.end || pt.end > sh.extent ||
            pt.start % sh.grain != 0)
            return bad(BL_ERR_KERNEL, "kernel %s: part %u/%u covers %u..%u of %u (grain %u)", name.c_str(),
                       pt.index + 1, pt.count, pt.start, pt.end, sh.extent, sh.grain);

        if (s.prologue && !(s.prologue == BL_PRO_RELU && s.main == BL_MAIN_CONV3X3))
            return bad(BL_ERR_KERNEL, "kernel %s: prologue %u on a main operation that takes none", name.c_str(), s.prologue);
        if (s.prologue == BL_PRO_RELU) name = "relu-" + name;
        Kernel k;
        k.label = name;
        if (pt.count > 1) k.label += " part " + std::to_string(pt.index + 1) + "/" + std::to_string(pt.count);

        for (uint32_t si = 0; si < n_sets; si++) {
            // Resolve every binding of this set to a device address.
            void *ptr[BL_MAX_BINDINGS];
            for (uint32_t b = 0; b < s.n_bindings; b++) {
                bl_binding bd = s.bindings[b];
                for (uint32_t t = 0; t < sets[si].count; t++) {
                    const bl_substitution &sub = sets[si].items[t];
                    if (sub.original == bd.tensor) {
                        if (sub.size != bd.size)
                            return bad(BL_ERR_STAND_IN_SIZE,
                                       "tensor %u stands in for tensor %u but its placement is %llu bytes, not %llu",
                                       sub.stand_in, sub.original, (unsigned long long)sub.size,
                                       (unsigned long long)bd.size);
                        bd.arena = sub.arena;
                        bd.offset = sub.offset;
                    }
                }
                if (bd.arena >= arenas->size.size())
                    return bad(BL_ERR_UNKNOWN_ARENA, "arena %u does not exist in this set", bd.arena);
                if (bd.offset > arenas->size[bd.arena] || bd.size > arenas->size[bd.arena] - bd.offset)
                    return bad(BL_ERR_PLACEMENT_OUT_OF_RANGE,
                               "placement at offset %llu of %llu bytes does not lie inside its arena",
                               (unsigned long long)bd.offset, (unsigned long long)bd.size);
                if (bd.offset % PLACEMENT_ALIGNMENT)
                    return bad(BL_ERR_MISALIGNED_PLACEMENT, "placement at offset %llu is not aligned to %u bytes",
                               (unsigned long long)bd.offset, PLACEMENT_ALIGNMENT);
                ptr[b] = arenas->base + arenas->offset[bd.arena] + bd.offset;
            }
            EpilogueArgs epi{};
            epi.n = (int)s.n_epilogue;
            for (uint32_t e = 0; e < s.n_epilogue; e++) {
                epi.kind[e] = (int)s.epilogue[e].kind;
                epi.factor[e] = s.epilogue[e].factor;
                epi.channels[e] = s.epilogue[e].channels;
                epi.operand[e] = (s.epilogue[e].kind == BL_EPI_ADD || s.epilogue[e].kind == BL_EPI_CHANNEL_SCALE)
                                     ? ptr[s.epilogue[e].operand]
                                     : nullptr;
            }
            void *out_ptr = ptr[s.n_bindings - 1];
            auto rd = [&](int i) -> const void * { return ptr[s.reads[i]]; };
            const bool f16 = dtype == BL_F16;
            const Math fmath = f16 ? Math::F16 : (ctx->f32_math == BL_F32_MATH_MFMA_F32 ? Math::F32 : Math::SPLIT);
            const uint32_t *d = s.dims;
            Launch L{};
            L.f16 = f16;
            L.math = fmath;
            std::string variant;
            switch (s.main) {
            case BL_MAIN_LAYER_NORM:
                L.family = Family::LAYER_NORM;
                L.ln = LayerNormArgs{rd(0), rd(1), rd(2), out_ptr, d[0], d[1], pt.start, pt.end, s.epsilon, epi};
                variant = "wave-per-row";
                break;
            case BL_MAIN_MATMUL:
            case BL_MAIN_PATCH_EMBED:
            case BL_MAIN_CONV3X3: {
                // At most 4 output columns (the head's 1x1 convolution to one
                // channel): a 64-wide MFMA tile would be all padding.
                if (s.main == BL_MAIN_MATMUL && d[2] <= 4 && d[1] % 4 == 0 && !getenv("BL_NO_GEMV")) {
                    L.family = Family::GEMV;
                    L.gv = GemvArgs{rd(0), rd(1), d[3] ? rd(2) : nullptr, out_ptr, d[1], d[2], pt.start, pt.end, epi};
                    variant = "valu-gemv";
                    break;
                }
                L.family = Family::GEMM;
                const bool patch = s.main == BL_MAIN_PATCH_EMBED, conv = s.main == BL_MAIN_CONV3X3;
                const uint32_t conv_oh = conv ? (d[0] - 1) / d[4] + 1 : 0, conv_ow = conv ? (d[1] - 1) / d[4] + 1 : 0;
                const uint32_t gm = patch ? d[0] * d[1] : conv ? conv_oh * conv_ow : d[0];
                const uint32_t gk = patch ? d[2] * d[2] * d[3] : conv ? 9 * d[2] : d[1];
                const uint32_t gn = patch ? d[4] : conv ? d[3] : d[2];
                const bool has_bias = (patch || conv) ? d[5] != 0 : d[3] != 0;
                GemmArgs ga{};
                ga.a = rd(0);
                ga.bias = has_bias ? rd(2) : nullptr;
                ga.c = out_ptr;
                ga.m = gm;
                ga.n = gn;
                ga.k = gk;
                ga.k_pad = (gk + PACK_K - 1) / PACK_K * PACK_K;
                ga.n_pad = (gn + PACK_N - 1) / PACK_N * PACK_N;
                ga.row0 = pt.start;
                ga.row1 = pt.end;
                ga.load = patch ? 2 : conv ? 3 : 0;
                ga.pipeline = getenv("BL_GEMM_NO_PIPELINE") || (conv && getenv("BL_CONV_NO_PIPELINE")) ? 0 : 1;
                if (patch) {
                    ga.p0 = d[1];
                    ga.p1 = d[2];
                    ga.p2 = d[3];
                    ga.p3 = d[1] * d[2];
                }
                if (conv) {
                    ga.p0 = d[0];
                    ga.p1 = d[1];
                    ga.p2 = d[2];
                    ga.p3 = d[4];
                    ga.p4 = conv_ow;
                    ga.p5 = s.prologue == BL_PRO_RELU ? 1 : 0;
                }
                ga.epi = epi;
                // Epilogues with a kernel of their own: GELU (erf); LayerScale over the
                // output's columns followed by the residual add; anything else runs the
                // steps in order.
                if (s.n_epilogue == 0) ga.epi_mode = 0;
                else if (s.n_epilogue == 1 && s.epilogue[0].kind == BL_EPI_GELU_ERF) ga.epi_mode = 1;
                else if (s.n_epilogue == 2 && s.epilogue[0].kind == BL_EPI_CHANNEL_SCALE &&
                         s.epilogue[0].channels == gn && s.epilogue[1].kind == BL_EPI_ADD) ga.epi_mode = 2;
                else ga.epi_mode = 3;
                // The packed B: one per distinct weight placement and math.
                const bl_binding &bb = s.bindings[s.reads[1]];
                uint32_t barena = bb.arena;
                uint64_t boff = bb.offset;
                for (uint32_t t = 0; t < sets[si].count; t++)
                    if (sets[si].items[t].original == bb.tensor) {
                        barena = sets[si].items[t].arena;
                        boff = sets[si].items[t].offset;
                    }
                int pack = -1;
                for (size_t q = 0; q < ks->packs.size(); q++) {
                    const Pack &pk = ks->packs[q];
                    if (pk.arena == barena && pk.offset == boff && pk.math == fmath && pk.k == gk && pk.n == gn) pack = (int)q;
                }
                if (pack < 0) {
                    Pack pk{};
                    pk.math = fmath;
                    pk.src = rd(1);
                    pk.arena = barena;
                    pk.offset = boff;
                    pk.size = bb.size;
                    pk.k = gk;
                    pk.n = gn;
                    pk.k_pad = ga.k_pad;
                    pk.n_pad = ga.n_pad;
                    ks->packs.push_back(pk);
                    pack = (int)ks->packs.size() - 1;
                }
                L.pack = pack;
                const uint32_t rows = pt.end - pt.start;
                auto wgs_of = [&](int t) {
                    return (uint64_t)((rows + gemm_tile_rows(t) - 1) / gemm_tile_rows(t)) *
                           ((gn + gemm_tile_cols(t) - 1) / gemm_tile_cols(t));
                };
                // 64 x 64 tiles when they fill every CU in one round (two
                // workgroups per CU at most), else 32 x 64: at the encoder's
                // sizes the smaller tile's extra workgroups hide its per-step
                // waits better than a second round or idle CUs would.
                const uint64_t w64 = wgs_of(TILE_64x64);
                int chosen = (w64 >= ctx->compute_units && w64 <= 2ull * ctx->compute_units) ? TILE_64x64 : TILE_32x64;
                ga.kgroups = 1;
                ga.stages = 4;
                // A long k with too few 64 x 64 tiles to go round (fc2 at the
                // encoder's sizes: 132 tiles, 48 k-steps): 64 x 64 tiles with
                // four groups of waves splitting k, two-stage rings each.
                if (w64 <= ctx->compute_units && gk / 32 >= 32) {
                    chosen = TILE_64x64;
                    ga.kgroups = 4;
                    ga.stages = 2;
                }
                // Products of plain rows in f16 or bf16x3 otherwise take 64-wide
                // k-steps, so that every staged row is whole 128-byte lines: a
                // wave's load touching 16 half lines reads a third as fast as
                // one touching 8 whole lines (15 against 48 bytes per clock per
                // CU from L2, measured). Two-stage rings in bf16x3, so that 2
                // to 3 workgroups fit a CU. The tiles follow the rounds of
                // workgroups the chip runs: bf16x3 takes 64 x 64 for wide
                // outputs whose tiles fit one round at two per CU (QKV: 11.4
                // -> 9.1 us), else 32 x 64 (fc1 17.9 -> 14.5); f16 takes 64 x
                // 64, or 32 x 64 for square projections of few rows (ViT-L's
                // QKV 38.4 -> 24.1 us, fc1 54.4 -> 33.0). An f16 product's
                // tiles wait on L2 latency rather than bandwidth, so its ring
                // deepens with the k-steps it has to hide it over: 2 stages
                // below 12 steps, 3 below 24, else 4 (ViT-L at 518: QKV 25.9
                // -> 24.5 us, fc2 30.1 -> 27.3; ViT-B: fc2 22.4 -> 21.0; ViT-S
                // at 1036: fc2 26.2 -> 21.8). Its square projections of few
                // rows keep 2 (ViT-L's out-projection: 9.5 against 10.8 with
                // 3), and so do grids of more than 5 tiles per CU (ViT-L's fc1,
                // 1408 tiles: 30.4 us against 32.9 to 34.0 with 3). With fewer
                // 32 x 64 tiles than CUs (small images) the deeper rings of
                // 32-wide steps hide more latency and stay.
                uint32_t kslices = 1;
                if ((fmath == Math::F16 || fmath == Math::SPLIT) && !patch && !conv && gk % 64 == 0 &&
                    wgs_of(TILE_32x64) >= ctx->compute_units) {
                    kslices = 2;
                    ga.kgroups = 1;
                    ga.stages = 2;
                    if (fmath == Math::F16) {
                        const bool square_few = gn <= 1024 && gk <= 1024 && rows <= 2048;
                        chosen = square_few ? TILE_32x64 : TILE_64x64;
                        if (!square_few)
                            ga.stages = gk / 64 >= 24 ? 4 : gk / 64 >= 12 && wgs_of(TILE_64x64) <= 5ull * ctx->compute_units ? 3 : 2;
                        // Wide products of 12 to 16 k-steps: 128 x 64 tiles
                        // in a two-stage ring (half the B bytes per output)
                        // when they leave no CU idle and their last round of
                        // two workgroups per CU is not a sliver of a round
                        // (in-encoder with the LayerNorm folded, µs: ViT-B
                        // QKV 18.6 -> 14.8, ViT-L fc1 30.6 -> 29.3). Products
                        // of 528 such tiles (a round and 16: ViT-B fc1, ViT-L
                        // QKV) measured slower, and those of 6 k-steps gained
                        // nothing once the fold's prologue took two passes
                        // (ViT-S 1036 QKV 18.3 -> 18.6; ViT-S fc1 in f16):
                        // they keep 64 x 64.
                        const uint64_t t128 = wgs_of(TILE_128x64), slots = 2ull * ctx->compute_units;
                        if (!square_few && gn >= 1024 && gk >= 768 && gk <= 1024 && t128 >= ctx->compute_units &&
                            (t128 % slots == 0 || t128 % slots >= slots / 8) && !getenv("BL_GEMM_NO_128")) {
                            chosen = TILE_128x64;
                            ga.stages = 2;
                        }
                    }
                    else chosen = (gn >= 1024 && w64 <= 2ull * ctx->compute_units) ? TILE_64x64 : TILE_32x64;
                    // bf16x3 outputs of whole 96-column tiles, at least 1536
                    // wide, that fit one round at two 64 x 96 workgroups per CU
                    // (fc1 at the encoder's sizes: 13.3 -> 12.3 us against 32 x
                    // 64 in two rounds; QKV's 1152 columns measured slower
                    // than its 64 x 64 tiles, 11.3 -> 12.1).
                    if (fmath == Math::SPLIT && gn >= 1536 && gn % 96 == 0 &&
                        wgs_of(TILE_64x96) <= 2ull * ctx->compute_units && !getenv("BL_GEMM_NO_96"))
                        chosen = TILE_64x96;
                }
                bool tile_forced = false;
                if (const char *force = getenv("BL_GEMM_TILE")) {
                    // "t" for every product, "t@n" for the products n columns wide.
                    const int t = atoi(force);
                    const char *at = strchr(force, '@');
                    if (t >= 0 && t < TILE_COUNT && (!at || (uint32_t)atoi(at + 1) == gn)) {
                        chosen = t;
                        tile_forced = true;
                    }
                }
                if (const char *force = getenv("BL_GEMM_KGROUPS")) ga.kgroups = (uint32_t)atoi(force);
                if (const char *force = getenv("BL_GEMM_STAGES")) ga.stages = (uint32_t)atoi(force);
                ga.kslices = kslices;
                ga.lane_epilogue = getenv("BL_GEMM_LANE_EPILOGUE") ? 1 : 0;
                if (const char *force = getenv("BL_GEMM_KSLICES")) ga.kslices = (uint32_t)atoi(force);
                // A 3x3 convolution with fewer tiles than CUs (the decoder's deep,
                // narrow stages: 6 tiles and 108 k-steps at 19 x 19 x 384 -> 64)
                // is bound by its serial k-loop: split k over up to two
                // workgroups per CU, at least two k-steps each.
                // A convolution to 32 channels or fewer over many pixels (the
                // head's): 128 x 32 tiles, so B is not half padding and A is
                // read by a quarter as many workgroups.
                // Otherwise 32 x 64: a convolution's window loads wait longer than
                // a plain row's, and the smaller tile's extra workgroups hide it
                // (148 x 148 x 64 -> 64: 19.8 us against 24.6 with 64 x 64).
                if (conv && !tile_forced)
                    chosen = gn <= 32 && wgs_of(TILE_128x32) >= ctx->compute_units ? TILE_128x32 : TILE_32x64;
                // A stride-1 convolution over an image with at least a tile per
                // CU: the direct kernel, which stages each input window once
                // for all nine taps (k_conv_direct.inc).
                if (conv && fmath != Math::F32 && (!tile_forced || chosen == TILE_CONV3) && !getenv("BL_CONV_NO_DIRECT") &&
                    conv_direct_fits(ga)) {
                    uint32_t oy_first, trows, tcols, nbs;
                    conv_direct_tiles(ga, oy_first, trows, tcols, nbs);
                    uint64_t min_tiles = ctx->compute_units;
                    if (const char *force = getenv("BL_CONV_DIRECT_MIN_TILES")) min_tiles = (uint64_t)atoll(force);
                    if ((uint64_t)trows * tcols * nbs >= min_tiles) chosen = TILE_CONV3;
                    else if (chosen == TILE_CONV3) chosen = TILE_32x64;
                }
                if (chosen == TILE_CONV3) {
                    // Weights resident in LDS when one chunk of 32 input
                    // channels holds them (the LDS of a per-tile chunk): more
                    // chunks resident cost a workgroup per CU, which measured
                    // slower than restaging (148 x 148 x 64 -> 64: 20.4 us
                    // resident at one per CU, 14.5 restaged at two; 518 x 518
                    // x 32 -> 32: 35.2 resident, 37.6 restaged). As many
                    // workgroups per CU as LDS holds (at most 4), persistent
                    // over the tiles.
                    const uint32_t chunks = (ga.p2 + CD_CC - 1) / CD_CC;
                    const char *res = getenv("BL_CONV_DIRECT_RESIDENT");
                    ga.cd_resident = (res ? atoi(res) != 0 && chunks <= 3 : chunks == 1) ? chunks : 0;
                    const uint32_t lds = conv_direct_lds(fmath, ga.cd_resident);
                    const uint32_t per_cu = std::max<uint32_t>(1, std::min<uint32_t>(4, 160 * 1024 / lds));
                    ga.cd_grid = per_cu * ctx->compute_units;
                    if (const char *force = getenv("BL_CONV_DIRECT_GRID")) ga.cd_grid = (uint32_t)atoi(force);
                }
                if (chosen == TILE_CONV3 && !(conv && fmath != Math::F32 && conv_direct_fits(ga))) chosen = TILE_32x64;
                ga.ksplit = 1;
                if (conv && chosen != TILE_CONV3 && !getenv("BL_CONV_NO_SPLIT_K")) {
                    const uint64_t wgs = wgs_of(chosen);
                    const uint32_t steps = ga.k_pad / 32;
                    if (wgs < ctx->compute_units && steps >= 4) {
                        uint64_t want = std::min<uint64_t>(steps / 2, (2ull * ctx->compute_units + wgs - 1) / wgs);
                        if (const char *force = getenv("BL_CONV_SPLIT_K")) want = (uint64_t)atoi(force);
                        if (want >= 2) {
                            // No empty split: ceil(steps / per) runs of per steps.
                            const uint32_t per = (uint32_t)((steps + want - 1) / want);
                            ga.ksplit = (steps + per - 1) / per;
                        }
                    }
                }
                // (Split k for plain products with few tiles measured slower: the
                // reduce launch and the partial sums cost more than the shorter
                // k-loops save, 1.00 -> 1.07 ms for the model at 182 pixels.)
                if (ga.ksplit > 1) split_users.push_back({ki, si});
                L.gemm = ga;
                L.tile = chosen;
                variant = std::string(fmath == Math::F16 ? "mfma-f16" : fmath == Math::F32 ? "mfma-f32" : "mfma-bf16x3") +
                          (chosen == TILE_CONV3 ? std::string(" direct ") + std::to_string(CD_TH) + "x" + std::to_string(CD_TW) + "x" +
                                                      std::to_string(CD_NB)
                                                : " " + std::to_string(gemm_tile_rows(chosen)) + "x" +
                                                      std::to_string(gemm_tile_cols(chosen))) +
                          (ga.kslices == 2 ? " bk64" : "") +
                          (ga.kgroups > 1 && !conv ? " k" + std::to_string(ga.kgroups) : std::string()) +
                          (ga.ksplit > 1 ? " splitk" + std::to_string(ga.ksplit) : std::string());
                break;
            }
            case BL_MAIN_ATTENTION_SCORES:
                L.family = Family::GATHER;
                L.gather = Gather::SCORES;
                L.ga = GatherArgs{rd(0), rd(0), nullptr, out_ptr, d[0], d[2], d[1], pt.start, pt.end, d[0], d[1], d[2], 0, epi};
                variant = "valu-tiled";
                break;
            case BL_MAIN_ATTENTION_VALUES:
                L.family = Family::GATHER;
                L.gather = Gather::VALUES;
                L.ga = GatherArgs{rd(0), rd(1), nullptr, out_ptr, d[2], d[0], d[1], pt.start, pt.end, d[0], d[1], d[2], 0, epi};
                variant = "valu-tiled";
                break;
            case BL_MAIN_SOFTMAX:
                L.family = Family::SOFTMAX;
                L.sm = SoftmaxArgs{rd(0), out_ptr, d[1], pt.start, pt.end, epi};
                variant = "workgroup-per-row";
                break;
            case BL_MAIN_PREPEND_TOKEN:
                L.family = Family::ELEMENT;
                L.element = PerElement::PREPEND;
                L.el = ElementArgs{rd(0), rd(1), out_ptr, pt.start, pt.end, d[1], epi};
                variant = "per-element";
                break;
            case BL_MAIN_TOKENS_TO_MAP:
                L.family = Family::ELEMENT;
                L.element = PerElement::DROP_FIRST;
                L.el = ElementArgs{rd(0), nullptr, out_ptr, pt.start, pt.end, d[2], epi};
                variant = "per-element";
                break;
            case BL_MAIN_MAP:
                L.family = Family::ELEMENT;
                L.element = PerElement::MAP;
                L.el = ElementArgs{rd(0), nullptr, out_ptr, pt.start, pt.end, 0, epi};
                variant = "per-element";
                break;
            case BL_MAIN_CONV_TRANSPOSE:
            case BL_MAIN_RESIZE_BILINEAR: {
                L.family = Family::DPT;
                const bool ct = s.main == BL_MAIN_CONV_TRANSPOSE;
                L.dpt = ct ? Dpt::CONV_TRANSPOSE : Dpt::RESIZE;
                L.dp = DptArgs{};
                L.dp.x = rd(0);
                L.dp.w = ct ? rd(1) : nullptr;
                L.dp.bias = ct && d[5] ? rd(2) : nullptr;
                L.dp.y = out_ptr;
                for (int i = 0; i < 6; i++) L.dp.d[i] = d[i];
                // ResizeBilinear::ratios (kernel.rs:614-631): (in - 1) / (out - 1)
                // in f32, zero for one output row or column.
                if (!ct) {
                    L.dp.ry = d[2] > 1 ? (float)(d[0] - 1) / (float)(d[2] - 1) : 0.0f;
                    L.dp.rx = d[3] > 1 ? (float)(d[1] - 1) / (float)(d[3] - 1) : 0.0f;
                }
                L.dp.start = (uint64_t)pt.start * sh.per_unit;
                L.dp.end = (uint64_t)pt.end * sh.per_unit;
                L.dp.epi = epi;
                variant = "per-element";
                break;
            }
            case BL_MAIN_FLASH_ATTENTION: {
                if (s.n_epilogue) return bad(BL_ERR_KERNEL, "kernel %s: the flash kernel takes no epilogue", name.c_str());
                L.family = Family::FLASH;
                const uint32_t t_pad = (d[0] + 63) / 64 * 64;
                const FlashPlan fp = plan_flash(fmath, d[0], d[1], pt.start, pt.end, ctx->compute_units);
                if (!fp.fits)
                    return bad(BL_ERR_TOO_LARGE, "kernel %s: %u tokens x %u heads is beyond the flash kernel's run arithmetic",
                               name.c_str(), d[0], d[1]);
                L.fl = FlashArgs{};
                L.fl.qkv = rd(0);
                L.fl.out = out_ptr;
                L.fl.tokens = d[0];
                L.fl.heads = d[1];
                L.fl.t_pad = t_pad;
                L.fl.row0 = pt.start;
                L.fl.row1 = pt.end;
                L.fl.splits = fp.splits;
                L.fl.scale = s.scale;
                L.fl.qtiles = fp.qtiles;
                L.fl.wgs = fp.wgs;
                L.fl.units = fp.units;
                L.fl.merge = fp.merge;
                L.fl.merge_inline = fp.merge && fp.counters && !getenv("BL_FLASH_MERGE_LAUNCH");
                scratch_bytes = std::max(scratch_bytes, fp.scratch_bytes);
                flash_counter_bytes = std::max(flash_counter_bytes, fp.counter_bytes);
                flash_users.push_back({ki, si});
                variant = fmath == Math::F32 ? "mfma-f32 splits=" + std::to_string(fp.splits)
                                             : std::string(fmath == Math::F16 ? "mfma-f16" : "mfma-bf16x3") + " 32x32 runs=" +
                                                   std::to_string(fp.wgs) +
                                                   (L.fl.merge_inline ? " merged in-kernel" : fp.merge ? " merged" : "");
                break;
            }
            }
            if (si == 0) k.label += " @ " + variant;
            L.out_lo = (const char *)out_ptr;
            L.out_hi = L.out_lo + s.bindings[s.n_bindings - 1].size;
            k.per_set.push_back(L);
        }
        ks->kernels.push_back(std::move(k));
    }
    plan_prepends(ks, specs, n, internal, n_internal);
    plan_folds(ks, specs, n, sets, n_sets, internal, n_internal);
    // The backend's own device memory, one allocation beside the plan's
    // arenas, laid out by lifetime (place_workspace): the packed weights and
    // the attention scratch for the whole program, each split-k GEMM's
    // partial sums for its own launch, each folded LayerNorm's statistics and
    // planes from its producer to its consumer.
    auto align256 = [](uint64_t b) { return (b + 255) / 256 * 256; };
    // B in registers (GemmArgs::breg) for ring-kernel products of 64-column
    // tiles of at most 64 rows, one group of waves and 64-wide k-steps whose
    // k is long against their width (the MLP's second product, k = 4 n: at
    // 1370 tokens 16.1 -> 15.4 us in bf16x3, 21.6 -> 19.5 at ViT-B, 28.3 ->
    // 27.8 at ViT-L, and at 5477 tokens 22.3 -> 18.0 in f16). The other
    // encoder products measured slower so (QKV 12.8 -> 15.8 us in bf16x3,
    // 24.3 -> 27.5 at ViT-L; out-projections +0.2 to +0.8 us; fc1 +0.5 to
    // +3.9 us), as did rings of 6 and 8 stages for every product. BL_GEMM_BREG=1 takes B in registers wherever it
    // applies, BL_GEMM_BREG=0 nowhere. A pack goes fragment-major when every
    // launch that reads it takes B in registers; the others read their B
    // through the ring.
    {
        const char *knob = getenv("BL_GEMM_BREG");
        const int breg_mode = knob ? atoi(knob) : -1;  // -1: long products only
        std::vector<int> all(ks->packs.size(), -1);
        for (Kernel &k : ks->kernels)
            for (Launch &L : k.per_set) {
                if (L.pack < 0) continue;
                const GemmArgs &g = L.gemm;
                L.gemm.breg = breg_mode != 0 && L.family == Family::GEMM && (L.math == Math::SPLIT || L.math == Math::F16) &&
                              g.pipeline && g.load == 0 && g.kgroups == 1 && g.kslices == 2 && g.ksplit <= 1 &&
                              g.k % 64 == 0 && g.k >= 64 && g.k_pad == g.k && (L.tile == TILE_32x64 || L.tile == TILE_64x64) &&
                              (breg_mode == 1 || (g.k >= 2 * g.n && g.k / 64 >= 12));
                int &v = all[L.pack];
                v = v < 0 ? (int)L.gemm.breg : (v && L.gemm.breg);
            }
        for (size_t q = 0; q < ks->packs.size(); q++) ks->packs[q].frag = all[q] == 1;
        for (Kernel &k : ks->kernels) {
            for (Launch &L : k.per_set) {
                if (L.pack >= 0 && !ks->packs[L.pack].frag) L.gemm.breg = 0;
                if (L.gemm.breg) L.gemm.stages = 4;
            }
            if (!k.per_set.empty() && k.per_set[0].gemm.breg) k.label += " breg";
        }
    }
    for (const Kernel &k : ks->kernels)
        for (const Launch &L : k.per_set)
            if (L.pack >= 0) ks->packs[L.pack].used = true;
    uint64_t pack_total = 0;
    for (Pack &pk : ks->packs) {
        if (!pk.used) continue;  // a plain pack every reader of which took a folded one
        pk.dst_offset = pack_total;
        pack_total += align256(packed_bytes(pk.math, pk.k_pad, pk.n_pad));
        if (pk.folded()) {
            pk.vec_offset = pack_total;
            pack_total += align256(fold_vec_bytes(pk.n_pad));
        }
        // Written by a kernel of this program: packed again before every launch.
        for (uint32_t ki = 0; ki < n && !pk.dynamic; ki++) {
            const bl_binding &o = specs[ki].bindings[specs[ki].n_bindings - 1];
            if (pk.reads(o.arena, o.offset, o.size)) pk.dynamic = true;
        }
    }
    for (const Pack &pk : ks->packs)
        if (pk.used && pk.dynamic) ks->graphs_ok = false;
    std::vector<WsItem> items;
    const uint32_t whole = n ? n - 1 : 0;
    const size_t pack_item = items.size();
    if (pack_total) items.push_back({pack_total, 0, whole, -1, 0});
    // The attention scratch: the in-kernel merge's arrival counters in front
    // (every flash kernel's at the same bytes, zero between launches), then
    // the largest flash kernel's operands and partial results.
    const uint64_t counter_bytes = align256(flash_counter_bytes);
    if (scratch_bytes) scratch_bytes = counter_bytes + align256(scratch_bytes);
    const size_t scratch_item = items.size();
    if (scratch_bytes) items.push_back({align256(scratch_bytes), 0, whole, -1, 0});
    // Each split-k GEMM's partial sums: the largest over its binding sets,
    // written and read within its own launch.
    std::map<size_t, size_t> partial_item;  // kernel -> item
    for (auto [ki, si] : split_users) {
        const GemmArgs &ga = ks->kernels[ki].per_set[si].gemm;
        const uint64_t b = align256((uint64_t)ga.ksplit * (ga.row1 - ga.row0) * ga.n * sizeof(float));
        auto it = partial_item.find(ki);
        if (it == partial_item.end()) {
            partial_item[ki] = items.size();
            items.push_back({b, (uint32_t)ki, (uint32_t)ki, -1, 0});
        } else {
            items[it->second].size = std::max(items[it->second].size, b);
        }
    }
    const size_t fold_item = items.size();
    for (const Fold &f : ks->folds)
        for (uint32_t si = 0; si < ks->sets; si++)
            items.push_back({align256(fold_stats_bytes(f)) + align256(fold_plane_bytes(f, ks->kernels[f.consumer].per_set[si])),
                             f.producer, f.consumer, (int)si, 0});
    const uint64_t workspace = place_workspace(items);
    if (workspace) {
        ks->workspace = (char *)bl_device_alloc(ctx, workspace);
        if (!ks->workspace)
            return bad(BL_ERR_HIP, "hipMalloc of %llu bytes of workspace (packed weights, partial sums, attention scratch, folds)",
                       (unsigned long long)workspace);
        ks->workspace_bytes = workspace;
    }
    if (pack_total) {
        ks->pack_buffer = ks->workspace + items[pack_item].at;
        for (Kernel &k : ks->kernels)
            for (Launch &L : k.per_set)
                if (L.pack >= 0) L.gemm.b = (char *)ks->pack_buffer + ks->packs[L.pack].dst_offset;
    }
    // A split-k GEMM's partial sums, every element written by its split
    // before the reduce reads it, share bytes with folds of disjoint
    // lifetimes: its launch makes their statistics stale.
    ks->kernel_clobbers.assign(n, {});
    ks->fold_alias.assign(ks->folds.size() * ks->sets, {});
    auto overlap = [&](size_t a, size_t b) {
        return items[a].at < items[b].at + items[b].size && items[b].at < items[a].at + items[a].size;
    };
    for (auto [ki, item] : partial_item) {
        for (auto [kj, sj] : split_users)
            if (kj == ki) ks->kernels[kj].per_set[sj].gemm.partials = (float *)(ks->workspace + items[item].at);
        for (size_t e = 0; e < ks->fold_alias.size(); e++)
            if (overlap(item, fold_item + e)) ks->kernel_clobbers[ki].push_back((uint32_t)e);
    }
    for (size_t e = 0; e < ks->fold_alias.size(); e++)
        for (size_t g = 0; g < ks->fold_alias.size(); g++)
            if (g != e && overlap(fold_item + e, fold_item + g)) ks->fold_alias[e].push_back((uint32_t)g);
    if (scratch_bytes) {
        ks->scratch = ks->workspace + items[scratch_item].at;
        // Kernels run one after another on the stream, so every flash kernel
        // uses the same scratch: operands, then partial outputs and statistics.
        for (auto [ki, si] : flash_users)
            bind_flash_scratch(ks->kernels[ki].per_set[si].fl, ks->kernels[ki].per_set[si].math, ks->scratch, counter_bytes);
        // Zeroed once: the operands' padding keys (past the last token) are
        // never written by a fused QKV projection and must stay finite, and the
        // merge's arrival counters start at zero (each launch leaves them so).
        if (hipMemset(ks->scratch, 0, scratch_bytes) != hipSuccess)
            return bad(BL_ERR_HIP, "clearing %llu bytes of attention scratch", (unsigned long long)scratch_bytes);
        // A flash kernel (f16 or bf16x3) whose qkv comes straight from QKV
        // projection kernels (no epilogue steps) gets its K and Vt from their
        // epilogues and skips its own prep launch. Parts of the flash kernel
        // reading the same qkv share the producers.
        if (!getenv("BL_NO_FUSED_PREP")) {
            for (auto [ki, si] : flash_users) {
                Launch &F = ks->kernels[ki].per_set[si];
                if (F.math == Math::F32) continue;
                std::vector<size_t> producers;
                bool ok = true;
                for (size_t j = ki; j-- > 0;) {
                    Launch &P = ks->kernels[j].per_set[si];
                    if (P.family == Family::FLASH && P.fl.qkv == F.fl.qkv) continue;
                    if (P.family != Family::GEMM || P.gemm.c != F.fl.qkv) break;
                    if (P.gemm.load != 0 || P.gemm.epi_mode != 0 || P.gemm.ksplit > 1 || P.math != F.math || P.gemm.m != F.fl.tokens ||
                        P.gemm.n != 3 * F.fl.heads * FLASH_HEAD_DIM)
                        ok = false;
                    producers.push_back(j);
                }
                if (!ok || producers.empty()) continue;
                for (size_t j : producers) {
                    GemmArgs &ga = ks->kernels[j].per_set[si].gemm;
                    ga.flash_ops = 1;
                    ga.fl_kp = F.fl.kp;
                    ga.fl_vt = F.fl.vt;
                    ga.fl_tpad = F.fl.t_pad;
                }
                F.fl.prepped = 1;
                F.kv_producers.assign(producers.begin(), producers.end());
                std::sort(F.kv_producers.begin(), F.kv_producers.end());
            }
            // A qkv the host never touches, written by nothing but those
            // projections and read by nothing but these flash kernels, from
            // an x the host never touches either: the projections store its
            // queries alone (the flash kernels read K and Vt from the
            // operands), and a flash kernel whose operands the scratch does
            // not hold runs its projections again, from the same x, instead of
            // its own prep (ViT-S/14 518: QKV 11.9 -> 11.3 us).
            std::vector<uint32_t> ids(internal, internal + n_internal);
            std::sort(ids.begin(), ids.end());
            auto is_internal = [&](uint32_t t) { return std::binary_search(ids.begin(), ids.end(), t); };
            for (auto [ki, si] : flash_users) {
                Launch &F = ks->kernels[ki].per_set[si];
                if (!F.fl.prepped || F.kv_producers.empty() || getenv("BL_QKV_WHOLE")) continue;
                const bl_spec &fsp = specs[ki];
                const uint32_t t = fsp.bindings[fsp.reads[0]].tensor;
                bool ok = is_internal(t);
                for (uint32_t kj = 0; kj < n && ok; kj++) {
                    const bl_spec &s = specs[kj];
                    const uint32_t last = s.n_bindings - 1;
                    const bool writer = s.bindings[last].tensor == t;
                    bool reader = false;
                    for (uint32_t b = 0; b < last; b++) reader = reader || s.bindings[b].tensor == t;
                    if (writer && reader) ok = false;
                    if (writer) ok = ok && is_internal(s.bindings[s.reads[0]].tensor);
                    for (uint32_t sj = 0; sj < ks->sets && ok && (writer || reader); sj++) {
                        const Launch &L = ks->kernels[kj].per_set[sj];
                        ok = writer ? L.family == Family::GEMM && L.gemm.flash_ops != 0
                                    : L.family == Family::FLASH && L.fl.prepped && !L.kv_producers.empty();
                    }
                }
                if (!ok) continue;
                F.kv_rerun = true;
                for (uint32_t j : F.kv_producers) {
                    ks->kernels[j].per_set[si].gemm.flash_ops = 2;
                    if (si == 0) ks->kernels[j].label += " > queries only";
                }
            }
        }
    }
    if (n_internal && !getenv("BL_NO_SPLIT_ACTIVATIONS")) keep_split_activations(ks, specs, n, internal, n_internal);
    if (!ks->folds.empty()) {
        for (size_t fi = 0; fi < ks->folds.size(); fi++)
            for (uint32_t si = 0; si < ks->sets; si++) {
                Fold &f = ks->folds[fi];
                const uint64_t at = items[fold_item + fi * ks->sets + si].at;
                LnStatsArgs &sa = f.stats[si];
                sa.stats = (float *)(ks->workspace + at);
                const Launch &G = ks->kernels[f.consumer].per_set[si];
                const uint64_t planes = fold_plane_bytes(f, G);
                sa.shadow = planes ? ks->workspace + at + align256(fold_stats_bytes(f)) : nullptr;
                sa.planes = planes && G.math == Math::SPLIT ? (uint64_t)sa.rows * sa.cols : 0;
            }
        apply_folds(ks);
    }
    if (getenv("BL_NO_GRAPH") || profiler_attached()) ks->graphs_ok = false;
    bl_ctx_retain(ctx);
    arenas->users.push_back(ks);
    *out = ks;
    return BL_OK;
}

extern "C" void bl_kernels_destroy(bl_kernels *k) {
    if (!k) return;
    hipSetDevice(k->ctx->device);
    hipStreamSynchronize(k->ctx->stream);
    for (RangeGraph &g : k->graphs) hipGraphExecDestroy(g.exec);
    bl_device_free(k->ctx, k->workspace, k->workspace_bytes);
    bl_ctx *ctx = k->ctx;
    bl_arenas *a = k->arenas;
    a->users.erase(std::find(a->users.begin(), a->users.end(), k));
    delete k;
    // The arenas outlive every kernel pointing into them.
    if (a->closed && a->users.empty()) arenas_free(a);
    bl_ctx_release(ctx);
}

extern "C" uint64_t bl_kernels_packs_made(const bl_kernels *k) { return k ? k->packs_made : 0; }

// Test hook: a fold's device buffers copied out (synchronously): what = 0 its
// statistics for binding set `set`, 1 the column vectors of its pack (c, d,
// then the per-block column sums [n_pad][32]), 2 its shadow (x centred per
// block) for binding set `set`.
extern "C" int bl_kernels_fold_read(bl_kernels *k, uint32_t fold, uint32_t set, uint32_t what, void *dst, uint64_t bytes) {
    if (!k || !dst || fold >= k->folds.size() || set >= k->sets) return BL_ERR_INVALID_ARGUMENT;
    const Fold &f = k->folds[fold];
    const Launch &G = k->kernels[f.consumer].per_set[set];
    const void *src = nullptr;
    uint64_t have = 0;
    if (what == 0) {
        src = f.stats[set].stats;
        have = fold_stats_bytes(f);
    } else if (what == 2) {
        src = f.stats[set].shadow;
        have = src ? fold_plane_bytes(f, G) : 0;
    } else {
        const Pack &pk = k->packs[G.pack];
        src = (const char *)k->pack_buffer + pk.vec_offset;
        have = fold_vec_bytes(pk.n_pad);
    }
    if (bytes > have) return BL_ERR_INVALID_ARGUMENT;
    hipSetDevice(k->ctx->device);
    hipError_t e = hipStreamSynchronize(k->ctx->stream);
    if (e == hipSuccess) e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    return e == hipSuccess ? BL_OK : hip_fail(k->ctx, e, "fold read");
}
extern "C" uint64_t bl_kernels_workspace_bytes(const bl_kernels *k) { return k ? k->workspace_bytes : 0; }

extern "C" uint32_t bl_kernels_len(const bl_kernels *k) { return k ? (uint32_t)k->kernels.size() : 0; }
extern "C" uint32_t bl_kernels_sets(const bl_kernels *k) { return k ? k->sets : 0; }
extern "C" const char *bl_kernels_label(const bl_kernels *k, uint32_t i) {
    return (k && i < k->kernels.size()) ? k->kernels[i].label.c_str() : nullptr;
}

// Packs a GEMM's B when its source may have changed since the last pack.
static hipError_t refresh_pack(bl_kernels *k, const Launch &L, hipStream_t s) {
    Pack &pk = k->packs[L.pack];
    if (!pk.dynamic && !pk.stale) return hipSuccess;
    PackArgs pa{pk.src, (char *)k->pack_buffer + pk.dst_offset, pk.k, pk.n, pk.k_pad, pk.n_pad,
                pk.gamma.ptr, pk.beta.ptr, pk.bias.ptr,
                pk.folded() ? (float *)((char *)k->pack_buffer + pk.vec_offset) : nullptr, pk.frag ? 1u : 0u};
    hipError_t e = launch_pack(pa, pk.math, s);
    if (e == hipSuccess) {
        pk.stale = false;
        k->packs_made++;
    }
    return e;
}

static hipError_t launch(const Launch &L, hipStream_t s) {
    if (L.fused) return hipSuccess;  // the product before it does its work
    switch (L.family) {
    case Family::LAYER_NORM: return L.fold_role == FOLD_LAYER_NORM ? hipSuccess : launch_layernorm(L.ln, L.f16, s);
    case Family::GEMM: {
        const hipError_t e = launch_gemm(L.gemm, L.math, L.tile, s);
        return e == hipSuccess && L.gemm.ksplit > 1 ? launch_gemm_reduce(L.gemm, L.f16, s) : e;
    }
    case Family::GATHER: return launch_gather(L.ga, L.gather, L.f16, s);
    case Family::SOFTMAX: return launch_softmax(L.sm, L.f16, s);
    case Family::FLASH: return launch_flash(L.fl, L.math, s);
    case Family::ELEMENT: return launch_element(L.el, L.element, L.f16, s);
    case Family::DPT: return launch_dpt(L.dp, L.dpt, L.f16, s);
    case Family::GEMV: return launch_gemv(L.gv, L.f16, s);
    }
    return hipErrorInvalidValue;
}

// Kernel `i`'s launch `L` as the attention scratch's state `kv` requires it,
// and that state after it. A flash kernel whose K and Vt its projections
// write (fl.prepped) reads them from the scratch; when the scratch does not
// hold them (the flash kernel encoded alone, qkv written since by the host
// or another kernel, or another flash kernel's operands in between) it runs
// its own prep instead, which makes them from all of qkv (a kv_rerun flash
// kernel has its projections run again first: run_one).
static bool kv_held(const Launch &L, const KvState &kv) {
    if (kv.qkv != L.fl.qkv) return false;
    if (kv.whole) return true;
    for (uint32_t p : L.kv_producers)
        if (std::find(kv.done.begin(), kv.done.end(), p) == kv.done.end()) return false;
    return true;
}

static Launch with_kv(const Launch &L, uint32_t i, KvState &kv) {
    Launch run = L;
    if (L.family == Family::FLASH && L.fl.prepped) {
        if (!kv_held(L, kv)) {
            run.fl.prepped = 0;
            kv = KvState{};
            kv.qkv = L.fl.qkv;
            kv.lo = (const char *)L.fl.qkv;
            kv.hi = kv.lo + (uint64_t)3 * L.fl.tokens * L.fl.heads * FLASH_HEAD_DIM * (L.math == Math::F16 ? 2 : 4);
            kv.whole = true;
        }
        return run;
    }
    if (L.family == Family::FLASH) {
        // A flash kernel's own prep overwrites the scratch's operands.
        if (kv.qkv != L.fl.qkv) kv = KvState{};
        return run;
    }
    if (L.family == Family::GEMM && L.gemm.flash_ops) {
        if (kv.qkv != L.gemm.c) {
            kv = KvState{};
            kv.qkv = L.gemm.c;
            kv.lo = (const char *)L.gemm.c;
            kv.hi = kv.lo + (uint64_t)L.gemm.m * L.gemm.n * (L.math == Math::F16 ? 2 : 4);
        }
        kv.done.push_back(i);
        return run;
    }
    if (kv.qkv && L.out_lo < kv.hi && kv.lo < L.out_hi) kv = KvState{};
    return run;
}

static void stale(FoldState &fs, const std::vector<uint32_t> &entries) {
    for (uint32_t e : entries) {
        fs.valid[e] = 0;
        fs.touched[e] = 1;
    }
}

// Kernel i of binding set `set` as the attention scratch (kv) and the folded
// LayerNorms' statistics (fs) require it, and their state after it: a folded
// LayerNorm, or its consumer, whose statistics do not describe x as it now is
// first makes them from x; the fold's producer makes them valid; any other
// write over a fold's x makes them stale.
static hipError_t run_one(bl_kernels *k, uint32_t i, uint32_t set, hipStream_t s, KvState &kv, FoldState &fs) {
    const Launch &L = k->kernels[i].per_set[set];
    const uint32_t sets = k->sets;
    if (L.fused) return hipSuccess;
    if (L.fold >= 0 && (L.fold_role == FOLD_LAYER_NORM || L.fold_role == FOLD_CONSUMER)) {
        const size_t at = (size_t)L.fold * sets + set;
        if (!fs.valid[at]) {
            const hipError_t e = launch_ln_stats(k->folds[L.fold].stats[set], L.f16, s);
            if (e != hipSuccess) return e;
            fs.valid[at] = 1;
            fs.touched[at] = 1;
            stale(fs, k->fold_alias[at]);
        }
        if (L.fold_role == FOLD_LAYER_NORM) return hipSuccess;
    }
    if (L.family == Family::FLASH && L.fl.prepped && L.kv_rerun && !kv_held(L, kv)) {
        // qkv holds the queries alone: its projections make K and Vt again,
        // from the x they read before (nothing but they write qkv, and the
        // host touches neither).
        for (uint32_t p : L.kv_producers) {
            const hipError_t e = run_one(k, p, set, s, kv, fs);
            if (e != hipSuccess) return e;
        }
        if (!kv_held(L, kv)) return hipErrorInvalidValue;
    }
    const hipError_t e = launch(with_kv(L, i, kv), s);
    if (e != hipSuccess) return e;
    for (size_t f = 0; f < k->folds.size(); f++) {
        const Fold &fo = k->folds[f];
        for (uint32_t si = 0; si < sets; si++) {
            if (!(L.out_lo < fo.x_hi[si] && fo.x_lo[si] < L.out_hi)) continue;
            const size_t at = f * sets + si;
            fs.valid[at] = (L.fold == (int)f && L.fold_role == FOLD_PRODUCER && si == set) ? 1 : 0;
            fs.touched[at] = 1;
        }
    }
    // The producer's statistics and the split-k partial sums overwrite the
    // folds that share their bytes.
    if (L.fold >= 0 && L.fold_role == FOLD_PRODUCER) stale(fs, k->fold_alias[(size_t)L.fold * sets + set]);
    stale(fs, k->kernel_clobbers[i]);
    return hipSuccess;
}

extern "C" int bl_kernels_encode(bl_kernels *k, uint32_t kernel, uint32_t set, bl_timer *timer, uint32_t tag) {
    if (!k) return BL_ERR_INVALID_ARGUMENT;
    if (kernel >= k->kernels.size()) return fail(k->ctx, BL_ERR_NO_SUCH_KERNEL, "there is no kernel %u", kernel);
    if (set >= k->sets) return fail(k->ctx, BL_ERR_NO_SUCH_SET, "there is no binding set %u", set);
    hipStream_t s = k->ctx->stream;
    int slice = -1;
    if (timer) {
        int r = bl_timer_slice_begin(timer, tag, s, &slice);
        if (r) return r;
    }
    const Launch &L = k->kernels[kernel].per_set[set];
    hipError_t e = L.pack >= 0 ? refresh_pack(k, L, s) : hipSuccess;
    if (e == hipSuccess) e = run_one(k, kernel, set, s, k->kv, k->fold_state);
    if (e != hipSuccess) return hip_fail(k->ctx, e, k->kernels[kernel].label.c_str());
    if (timer && slice >= 0) bl_timer_slice_end(timer, slice, s);
    return BL_OK;
}

// What a replay of the range may take the attention scratch to hold when it
// starts: the operands of the range's first flash kernel whose projections
// all precede the range and store qkv's queries alone, when the scratch now
// holds them (else a capture would run those projections again); nothing
// otherwise, so that the graph is right whatever ran before it.
static KvState range_entry(const bl_kernels *k, uint32_t first, uint32_t count, uint32_t set) {
    for (uint32_t i = first; i < first + count; i++) {
        const Launch &L = k->kernels[i].per_set[set];
        if (L.family != Family::FLASH) continue;
        if (!L.kv_rerun || L.kv_producers.empty() || L.kv_producers.back() >= first || !kv_held(L, k->kv)) break;
        return k->kv;
    }
    return KvState{};
}

static bool same_kv(const KvState &a, const KvState &b) {
    return a.qkv == b.qkv && a.lo == b.lo && a.hi == b.hi && a.whole == b.whole && a.done == b.done;
}

// The range's launches captured on the context's stream, or null when the
// capture failed (the caller then launches one by one). The attention
// scratch is taken to hold `entry` when a replay starts (the caller replays
// the graph only then); `kv` is what it holds after a replay.
static hipGraphExec_t capture_range(bl_kernels *k, uint32_t first, uint32_t count, uint32_t set, const KvState &entry,
                                     KvState &kv, FoldState &fs, uint32_t &launches) {
    launches = 0;
    hipStream_t s = k->ctx->stream;
    kv = entry;
    // Likewise no fold's statistics are taken as valid when a replay starts.
    fs.valid.assign(k->fold_state.valid.size(), 0);
    fs.touched.assign(k->fold_state.valid.size(), 0);
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return nullptr;
    hipError_t e = hipSuccess;
    for (uint32_t i = first; i < first + count && e == hipSuccess; i++) e = run_one(k, i, set, s, kv, fs);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(s, &g);
    hipGraphExec_t exec = nullptr;
    if (e == hipSuccess && end == hipSuccess && g) {
        if (hipGraphInstantiate(&exec, g, nullptr, nullptr, 0) != hipSuccess) exec = nullptr;
        size_t nodes = 0;
        if (exec && hipGraphGetNodes(g, nullptr, &nodes) == hipSuccess && nodes) {
            std::vector<hipGraphNode_t> list(nodes);
            if (hipGraphGetNodes(g, list.data(), &nodes) == hipSuccess)
                for (size_t q = 0; q < nodes; q++) {
                    hipGraphNodeType type;
                    if (hipGraphNodeGetType(list[q], &type) == hipSuccess && type == hipGraphNodeTypeKernel) launches++;
                }
        }
    }
    if (g) hipGraphDestroy(g);
    (void)hipGetLastError();
    return exec;
}

extern "C" int bl_kernels_encode_range(bl_kernels *k, uint32_t first, uint32_t count, uint32_t set) {
    if (!k) return BL_ERR_INVALID_ARGUMENT;
    if ((uint64_t)first + count > k->kernels.size())
        return fail(k->ctx, BL_ERR_NO_SUCH_KERNEL, "there is no kernel %u", first + count - 1);
    if (set >= k->sets) return fail(k->ctx, BL_ERR_NO_SUCH_SET, "there is no binding set %u", set);
    hipStream_t s = k->ctx->stream;
    if (k->graphs_ok && count > 1) {
        // Stale packs are remade first, outside the graph (the graph holds the
        // program's own launches only).
        for (uint32_t i = first; i < first + count; i++) {
            const Launch &L = k->kernels[i].per_set[set];
            hipError_t e = L.pack >= 0 ? refresh_pack(k, L, s) : hipSuccess;
            if (e != hipSuccess) return hip_fail(k->ctx, e, k->kernels[i].label.c_str());
        }
        const KvState entry = range_entry(k, first, count, set);
        const RangeGraph *found = nullptr;
        for (const RangeGraph &g : k->graphs)
            if (g.first == first && g.count == count && g.set == set && same_kv(g.entry, entry)) found = &g;
        if (!found) {
            KvState after;
            FoldState folds_after;
            uint32_t launches = 0;
            hipGraphExec_t exec = capture_range(k, first, count, set, entry, after, folds_after, launches);
            if (exec) {
                k->graphs.push_back({first, count, set, exec, entry, after, folds_after, launches});
                found = &k->graphs.back();
            } else {
                k->graphs_ok = false;
            }
        }
        if (found) {
            hipError_t e = hipGraphLaunch(found->exec, s);
            if (e != hipSuccess) return hip_fail(k->ctx, e, "graph launch");
            k->kv = found->kv;
            for (size_t q = 0; q < found->folds.touched.size(); q++)
                if (found->folds.touched[q]) k->fold_state.valid[q] = found->folds.valid[q];
            return BL_OK;
        }
    }
    for (uint32_t i = first; i < first + count; i++) {
        const Launch &L = k->kernels[i].per_set[set];
        hipError_t e = L.pack >= 0 ? refresh_pack(k, L, s) : hipSuccess;
        if (e == hipSuccess) e = run_one(k, i, set, s, k->kv, k->fold_state);
        if (e != hipSuccess) return hip_fail(k->ctx, e, k->kernels[i].label.c_str());
    }
    return BL_OK;
}

extern "C" int bl_kernels_range_launches(bl_kernels *k, uint32_t first, uint32_t count, uint32_t set, uint32_t *launches) {
    if (!k || !launches) return BL_ERR_INVALID_ARGUMENT;
    for (const RangeGraph &g : k->graphs)
        if (g.first == first && g.count == count && g.set == set) {
            *launches = g.launches;
            return BL_OK;
        }
    return fail(k->ctx, BL_ERR_INVALID_ARGUMENT, "kernels %u..%u of set %u have no captured graph", first,
                first + count - 1, set);
}

extern "C" int bl_kernels_time(bl_kernels *k, uint32_t kernel, uint32_t set, uint32_t repeats, float *micros) {
    if (!k || !micros || repeats == 0) return BL_ERR_INVALID_ARGUMENT;
    if (kernel >= k->kernels.size()) return fail(k->ctx, BL_ERR_NO_SUCH_KERNEL, "there is no kernel %u", kernel);
    if (set >= k->sets) return fail(k->ctx, BL_ERR_NO_SUCH_SET, "there is no binding set %u", set);
    hipStream_t s = k->ctx->stream;
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipError_t e = hipEventCreate(&ev[0]);
    if (e == hipSuccess) e = hipEventCreate(&ev[1]);
    const Launch &L = k->kernels[kernel].per_set[set];
    // The first launch refreshes a packed operand when it must (and a flash
    // kernel's scratch operands); the timed ones then run the kernel alone,
    // back to back, as it runs in its program.
    if (e == hipSuccess && L.pack >= 0) e = refresh_pack(k, L, s);
    if (e == hipSuccess) e = run_one(k, kernel, set, s, k->kv, k->fold_state);
    if (e == hipSuccess) e = hipEventRecord(ev[0], s);
    for (uint32_t r = 0; r < repeats && e == hipSuccess; r++) e = launch(L, s);
    if (e == hipSuccess) e = hipEventRecord(ev[1], s);
    if (e == hipSuccess) e = hipEventSynchronize(ev[1]);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev[0], ev[1]);
    for (hipEvent_t x : ev)
        if (x) hipEventDestroy(x);
    if (e != hipSuccess) return hip_fail(k->ctx, e, k->kernels[kernel].label.c_str());
    *micros = ms * 1000.0f / (float)repeats;
    return BL_OK;
}

extern "C" int bl_spin(bl_ctx *ctx, uint32_t micros) {
    if (!ctx) return BL_ERR_INVALID_ARGUMENT;
    if (!ctx->wall_clock_khz) return fail(ctx, BL_ERR_HIP, "the device reports no wall clock rate");
    uint64_t ticks = (uint64_t)micros * ctx->wall_clock_khz / 1000;
    hipError_t e = launch_spin(ticks, ctx->compute_units * 4, ctx->stream);
    return e == hipSuccess ? BL_OK : hip_fail(ctx, e, "spin");
}
