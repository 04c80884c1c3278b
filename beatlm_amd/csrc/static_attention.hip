// Flash attention that allocates nothing: bl_flash_attention_static.
//
// The same computation as a BL_MAIN_FLASH_ATTENTION kernel encoded by
// bl_kernels_encode (its own prep of K and Vt, the flash kernel, the merge of
// split key ranges; k_flash.hip), for callers that cannot allocate device
// memory. What bl_kernels_create allocates for that kernel (the K and Vt
// operands, the partial results of split key ranges and their statistics)
// lives here in one file-scope device array, `scratch`, of
// BL_STATIC_SCRATCH_BYTES. Each GPU the library runs on holds its own copy
// of the array until the process ends; the code object that holds it is
// loaded on a device the first time this entry point runs there.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// the array's address on a device comes from hipGetSymbolAddress, called
// once per device (with that device current) on the entry point's first call
// there (kept once found; a failed lookup is tried again on the next call),
// and only that address is handed to kernels. The call makes the context's
// device current and restores the caller's current device before returning.
//
// Every call on a GPU shares that GPU's array: calls that overlap on one GPU
// (two streams, two contexts) race. The array's first COUNTER_BYTES hold the
// in-kernel merge's arrival counters (one per (head, query tile) pair, at the
// same bytes for every shape): they start at zero, as the whole array does
// when its code object is loaded, and every call leaves them at zero. The
// rest needs no initial value: the prep launch writes every K and Vt element
// the flash kernel reads (padding keys included), and each split key range
// writes its partial result before the merge reads it, within the same call.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "ctx.hpp"
#include "spec.hpp"

namespace {

static __device__ __align__(256) char scratch[BL_STATIC_SCRATCH_BYTES];
constexpr uint64_t COUNTER_BYTES = 1 << 20;  // 8192 (head, query tile) pairs, 128 bytes each

constexpr int MAX_DEVICES = 64;
void *device_scratch[MAX_DEVICES];
std::mutex device_mutex;

// The array's address on `device` (current): looked up on the first call
// there and kept once found; a failed lookup is tried again next call.
hipError_t scratch_on(int device, void **out) {
    std::lock_guard<std::mutex> lock(device_mutex);
    if (!device_scratch[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        device_scratch[device] = p;
    }
    *out = device_scratch[device];
    return hipSuccess;
}

// Makes `device` current for the call and restores the caller's device after.
struct DeviceScope {
    int prev = -1;
    hipError_t status = hipSuccess;
    explicit DeviceScope(int device) {
        status = hipGetDevice(&prev);
        if (status == hipSuccess && prev != device) status = hipSetDevice(device);
        else if (status == hipSuccess) prev = -1;  // already current: nothing to restore
    }
    ~DeviceScope() {
        if (prev >= 0) hipSetDevice(prev);
    }
};

int fail(bl_ctx *ctx, int code, const char *fmt, unsigned long long a, unsigned long long b) {
    char msg[256];
    snprintf(msg, sizeof msg, fmt, a, b);
    return bl_fail(ctx, code, msg);
}

}  // namespace

extern "C" int bl_flash_attention_static(bl_ctx *ctx, const void *qkv, void *out, uint32_t tokens, uint32_t heads,
                                         float scale, uint32_t dtype) {
    if (!ctx) return BL_ERR_INVALID_ARGUMENT;
    if (!qkv || !out || tokens == 0 || heads == 0 || (dtype != BL_F32 && dtype != BL_F16))
        return bl_fail(ctx, BL_ERR_INVALID_ARGUMENT, "flash attention (static): null tensor, zero size or unknown dtype");
    if (!(scale == scale) || scale == INFINITY || scale == -INFINITY)
        return bl_fail(ctx, BL_ERR_INVALID_ARGUMENT, "flash attention (static): non-finite scale");
    const int device = bl_device_of(ctx);
    if (device < 0 || device >= MAX_DEVICES)
        return bl_fail(ctx, BL_ERR_INVALID_ARGUMENT, "flash attention (static): device ordinal beyond the library's table");
    const bl::Math m = dtype == BL_F16 ? bl::Math::F16
                     : bl_f32_math_of(ctx) == BL_F32_MATH_MFMA_F32 ? bl::Math::F32 : bl::Math::SPLIT;
    const bl::FlashPlan plan = bl::plan_flash(m, tokens, heads, 0, tokens, bl_compute_units_of(ctx));
    if (!plan.fits)
        return fail(ctx, BL_ERR_TOO_LARGE, "flash attention (static): %llu tokens x %llu heads is beyond the kernel's run arithmetic",
                    (unsigned long long)tokens, (unsigned long long)heads);
    if (plan.counter_bytes > COUNTER_BYTES)
        return fail(ctx, BL_ERR_TOO_LARGE,
                    "flash attention (static): this shape has %llu (head, query tile) pairs, the static array holds counters for %llu",
                    (unsigned long long)plan.counters, (unsigned long long)(COUNTER_BYTES * plan.counters / plan.counter_bytes));
    if (COUNTER_BYTES + plan.scratch_bytes > BL_STATIC_SCRATCH_BYTES)
        return fail(ctx, BL_ERR_TOO_LARGE,
                    "flash attention (static): this shape needs %llu bytes of scratch, the static array holds %llu",
                    (unsigned long long)(COUNTER_BYTES + plan.scratch_bytes), (unsigned long long)BL_STATIC_SCRATCH_BYTES);
    const DeviceScope scope(device);
    hipError_t e = scope.status;
    void *base = nullptr;
    if (e == hipSuccess) e = scratch_on(device, &base);
    if (e != hipSuccess || !base) return bl_fail(ctx, BL_ERR_HIP, "flash attention (static): no address for the scratch array");

    bl::FlashArgs a{};
    a.qkv = qkv;
    a.out = out;
    a.tokens = tokens;
    a.heads = heads;
    a.t_pad = (tokens + 63) / 64 * 64;
    a.row0 = 0;
    a.row1 = tokens;
    a.splits = plan.splits;
    a.scale = scale;
    a.qtiles = plan.qtiles;
    a.wgs = plan.wgs;
    a.units = plan.units;
    a.merge = plan.merge;
    a.merge_inline = plan.merge && plan.counters;
    a.prepped = 0;  // the prep launch writes K and Vt into the scratch
    bl::bind_flash_scratch(a, m, base, COUNTER_BYTES);
    e = bl::launch_flash(a, m, bl_stream_of(ctx));
    return e == hipSuccess ? BL_OK : bl_fail(ctx, BL_ERR_HIP, hipGetErrorString(e));
}
