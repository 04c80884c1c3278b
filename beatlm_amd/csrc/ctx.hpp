// Internal: what the backend's other source files need of a context (its
// device, stream and compute units, error reporting, lifetime and the
// allocation count).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/beatlm_hip.h"

// Handles made from a context hold it: it is released after the last of them.
void bl_ctx_retain(bl_ctx *ctx);
void bl_ctx_release(bl_ctx *ctx);
bool bl_events_counted(bl_ctx *ctx, uint64_t n);
hipStream_t bl_stream_of(bl_ctx *ctx);
int bl_device_of(const bl_ctx *ctx);
uint32_t bl_compute_units_of(const bl_ctx *ctx);
uint32_t bl_f32_math_of(const bl_ctx *ctx);
// Sets the context's message (no allocation for messages under 512 bytes).
int bl_fail(bl_ctx *ctx, int code, const char *msg);
