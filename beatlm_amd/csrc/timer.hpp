// Internal: the hooks bl_kernels_encode uses to bracket a launch with the
// timer's events, and the allocation counter the timer reports its events to.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/beatlm_hip.h"

// Records the slice's start event on `stream` for the open frame; `*slice` is
// -1 when the frame is untimed (its ring slot was busy).
int bl_timer_slice_begin(bl_timer *timer, uint32_t tag, hipStream_t stream, int *slice);
void bl_timer_slice_end(bl_timer *timer, int slice, hipStream_t stream);

bool bl_events_counted(bl_ctx *ctx, uint64_t n);
// Handles made from a context hold it: it is released after the last of them.
void bl_ctx_retain(bl_ctx *ctx);
void bl_ctx_release(bl_ctx *ctx);
hipStream_t bl_stream_of(bl_ctx *ctx);
int bl_fail(bl_ctx *ctx, int code, const char *msg);
