// Internal: the hooks bl_kernels_encode uses to bracket a launch with the
// timer's events.
#pragma once

#include <hip/hip_runtime.h>

#include "ctx.hpp"

// Records the slice's start event on `stream` for the open frame; `*slice` is
// -1 when the frame is untimed (its ring slot was busy).
int bl_timer_slice_begin(bl_timer *timer, uint32_t tag, hipStream_t stream, int *slice);
void bl_timer_slice_end(bl_timer *timer, int slice, hipStream_t stream);
