// The slice timer: per-slice GPU durations from hipEvent pairs, read back
// without ever blocking. The HIP counterpart of the reference's SliceTimer
// (crates/beatlm/src/gpu/timer.rs:185-464); which slot a frame uses and when
// its events may be read is the ring's bookkeeping (ring.hpp), and this file
// holds only the events:
//
//  - BL_TIMER_RING_DEPTH slots, each with an event pair per slice, a pair for
//    the render pass and one event closing the frame, all created once;
//  - a frame whose slot is still in flight when it begins is not timed, and
//    is counted skipped; nothing waits;
//  - a resolved frame is read only once the host hands its ticket back as
//    submitted, frames come back in submission order, and a ticket given up
//    (bl_timer_abandon) frees its slot unread;
//  - held frames are read only once the host's verdict accepts them;
//  - frames the host marks (bl_timer_invalidate_submitted) are never
//    decoded: they free their slot once their events completed and count as
//    failed;
//  - a slot's work stands where hipEventQuery of its closing event says, so
//    collecting never blocks.
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "ring.hpp"
#include "timer.hpp"
#include "../../include/beatlm_schedule.h"

namespace {

struct Slot {
    uint64_t frame = 0;
    uint32_t used = 0;
    std::vector<hipEvent_t> events;  // 2 per slice
    hipEvent_t render[2] = {nullptr, nullptr};
    int render_state = 0;            // 0 not timed, 1 begun, 2 ended
    hipEvent_t done = nullptr;       // recorded at resolve
    std::vector<uint32_t> tags;
};

}  // namespace

struct bl_timer {
    bl_ctx *ctx = nullptr;
    bool retained = false;         // holds a reference on ctx (set once created)
    uint32_t max_slices = 0;
    bl::Ring ring{BL_TIMER_RING_DEPTH};
    std::vector<Slot> slots;
    int open = -1;                 // slot of the frame being recorded, -1 when untimed
    bool frame_open = false;
    bool render_begun = false;     // the open frame's render pass was requested
    bl_timer_stats_t stats{};
    // What the last collect returned; valid until the next collect.
    std::vector<std::vector<uint32_t>> out_tags;
    std::vector<std::vector<float>> out_micros;
};

// The most slices one frame can time.
static constexpr uint32_t TIMER_MAX_SLICES = BLS_TIMER_MAX_SLICES;  // what timer_capacity checks against

extern "C" int bl_timer_create(bl_ctx *ctx, uint32_t max_slices, bl_timer **out) {
    if (!ctx || !out) return BL_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    if (max_slices == 0 || max_slices > TIMER_MAX_SLICES)
        return bl_fail(ctx, BL_ERR_INVALID_ARGUMENT, "slice capacity outside 1..=4096");
    auto *t = new bl_timer();
    t->ctx = ctx;
    t->max_slices = max_slices;
    t->slots.resize(BL_TIMER_RING_DEPTH);
    uint64_t created = 0;
    for (Slot &s : t->slots) {
        s.events.resize(2 * (size_t)max_slices, nullptr);
        s.tags.resize(max_slices, 0);
        for (hipEvent_t &e : s.events) {
            if (hipEventCreate(&e) != hipSuccess) {
                bl_timer_destroy(t);
                return bl_fail(ctx, BL_ERR_HIP, "hipEventCreate");
            }
            created++;
        }
        for (hipEvent_t *e : {&s.done, &s.render[0], &s.render[1]}) {
            if (hipEventCreate(e) != hipSuccess) {
                bl_timer_destroy(t);
                return bl_fail(ctx, BL_ERR_HIP, "hipEventCreate");
            }
            created++;
        }
    }
    bl_events_counted(ctx, created);
    bl_ctx_retain(ctx);
    t->retained = true;
    *out = t;
    return BL_OK;
}

extern "C" void bl_timer_destroy(bl_timer *t) {
    if (!t) return;
    hipStreamSynchronize(bl_stream_of(t->ctx));
    for (Slot &s : t->slots) {
        for (hipEvent_t e : s.events)
            if (e) hipEventDestroy(e);
        for (hipEvent_t e : {s.done, s.render[0], s.render[1]})
            if (e) hipEventDestroy(e);
    }
    bl_ctx *ctx = t->retained ? t->ctx : nullptr;
    delete t;
    if (ctx) bl_ctx_release(ctx);
}

extern "C" int bl_timer_begin_frame(bl_timer *t, uint64_t frame, uint32_t *timed) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    // A frame still open (begun, never resolved) gives its slot back unread.
    if (t->frame_open && t->open >= 0) {
        t->ring.release((uint32_t)t->open);
        t->stats.frames_dropped++;
    }
    const uint64_t reclaimed = t->ring.reclaimed();
    t->open = t->ring.claim();
    t->stats.frames_dropped += t->ring.reclaimed() - reclaimed;  // tickets given up
    t->stats.frames_begun++;
    t->frame_open = true;
    t->render_begun = false;
    if (t->open < 0) {
        t->stats.frames_skipped++;
    } else {
        Slot &s = t->slots[t->open];
        s.frame = frame;
        s.used = 0;
        s.render_state = 0;
    }
    if (timed) *timed = t->open >= 0 ? 1u : 0u;
    return BL_OK;
}

int bl_timer_slice_begin(bl_timer *t, uint32_t tag, hipStream_t stream, int *slice) {
    *slice = -1;
    if (!t->frame_open) return bl_fail(t->ctx, BL_ERR_TIMER_NO_FRAME, "no frame is open on the timer");
    if (t->open < 0) return BL_OK;  // untimed frame
    Slot &s = t->slots[t->open];
    if (s.used >= t->max_slices) {
        std::string msg = "more than " + std::to_string(t->max_slices) + " slices timed in one frame";
        return bl_fail(t->ctx, BL_ERR_TIMER_TOO_MANY_SLICES, msg.c_str());
    }
    const uint32_t i = s.used++;
    s.tags[i] = tag;
    if (hipEventRecord(s.events[2 * i], stream) != hipSuccess)
        return bl_fail(t->ctx, BL_ERR_HIP, "hipEventRecord");
    *slice = (int)i;
    return BL_OK;
}

void bl_timer_slice_end(bl_timer *t, int slice, hipStream_t stream) {
    Slot &s = t->slots[t->open];
    hipEventRecord(s.events[2 * slice + 1], stream);
}

extern "C" int bl_timer_render_begin(bl_timer *t) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    if (!t->frame_open) return bl_fail(t->ctx, BL_ERR_TIMER_NO_FRAME, "no frame is open on the timer");
    if (t->render_begun) return bl_fail(t->ctx, BL_ERR_TIMER_RENDER_TWICE, "the frame's render pass is already timed");
    t->render_begun = true;
    if (t->open < 0) return BL_OK;  // untimed frame
    Slot &s = t->slots[t->open];
    if (hipEventRecord(s.render[0], bl_stream_of(t->ctx)) != hipSuccess)
        return bl_fail(t->ctx, BL_ERR_HIP, "hipEventRecord");
    s.render_state = 1;
    return BL_OK;
}

extern "C" int bl_timer_render_end(bl_timer *t) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    if (!t->frame_open) return bl_fail(t->ctx, BL_ERR_TIMER_NO_FRAME, "no frame is open on the timer");
    if (t->open < 0) return BL_OK;
    Slot &s = t->slots[t->open];
    if (s.render_state != 1) return bl_fail(t->ctx, BL_ERR_INVALID_ARGUMENT, "the render pass was not begun");
    if (hipEventRecord(s.render[1], bl_stream_of(t->ctx)) != hipSuccess)
        return bl_fail(t->ctx, BL_ERR_HIP, "hipEventRecord");
    s.render_state = 2;
    return BL_OK;
}

extern "C" int bl_timer_resolve(bl_timer *t, uint64_t *resolved) {
    if (!t || !resolved) return BL_ERR_INVALID_ARGUMENT;
    *resolved = 0;  // untimed: handing it back is accepted and ignored
    if (!t->frame_open) return bl_fail(t->ctx, BL_ERR_TIMER_NO_FRAME, "no frame is open on the timer");
    t->frame_open = false;
    if (t->open < 0) return BL_OK;
    const uint32_t i = (uint32_t)t->open;
    t->open = -1;
    if (hipEventRecord(t->slots[i].done, bl_stream_of(t->ctx)) != hipSuccess) {
        t->ring.release(i);
        return bl_fail(t->ctx, BL_ERR_HIP, "hipEventRecord");
    }
    *resolved = t->ring.encode(i);
    return BL_OK;
}

extern "C" int bl_timer_submitted(bl_timer *t, uint64_t resolved) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    if (resolved) t->ring.submit(resolved);  // another timer's frame goes untimed
    return BL_OK;
}

extern "C" int bl_timer_submitted_held(bl_timer *t, uint64_t resolved, uint64_t *hold) {
    if (!t || !hold) return BL_ERR_INVALID_ARGUMENT;
    *hold = 0;
    if (resolved) t->ring.submit_held(resolved, hold);
    return BL_OK;
}

extern "C" int bl_timer_verdict(bl_timer *t, uint64_t hold, uint32_t accepted) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    return hold && bl::give_verdict(hold, accepted != 0) ? 1 : 0;
}

extern "C" int bl_timer_abandon(bl_timer *t, uint64_t resolved) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    if (resolved) bl::drop_ticket(resolved);
    return BL_OK;
}

extern "C" uint32_t bl_timer_in_flight(const bl_timer *t) { return t ? t->ring.in_flight() : 0; }

// Reads slot `i`'s slice and render durations into out[*n_out]; false when
// an elapsed time cannot be read.
static bool read_slot(bl_timer *t, uint32_t i, bl_frame_timing *out, uint32_t *n_out) {
    Slot &s = t->slots[i];
    std::vector<uint32_t> tags(s.tags.begin(), s.tags.begin() + s.used);
    std::vector<float> micros(s.used, 0.0f);
    for (uint32_t j = 0; j < s.used; j++) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, s.events[2 * j], s.events[2 * j + 1]) != hipSuccess) return false;
        micros[j] = ms * 1000.0f;
    }
    t->out_tags.push_back(std::move(tags));
    t->out_micros.push_back(std::move(micros));
    bl_frame_timing &f = out[*n_out];
    f.frame = s.frame;
    f.n_slices = s.used;
    f.failed = 0;
    f.tags = t->out_tags.back().data();
    f.micros = t->out_micros.back().data();
    f.has_render = 0;
    f.render_micros = 0.0f;
    float ms = 0.0f;
    if (s.render_state == 2 && hipEventElapsedTime(&ms, s.render[0], s.render[1]) == hipSuccess) {
        f.has_render = 1;
        f.render_micros = ms * 1000.0f;
    }
    (*n_out)++;
    return true;
}

extern "C" int bl_timer_collect(bl_timer *t, bl_frame_timing *out, uint32_t cap, uint32_t *n_out) {
    if (!t || !n_out || (cap && !out)) return BL_ERR_INVALID_ARGUMENT;
    *n_out = 0;
    t->out_tags.clear();
    t->out_micros.clear();
    t->out_tags.reserve(cap);
    t->out_micros.reserve(cap);
    t->ring.settle();
    uint32_t slots[bl::RING_MAX_DEPTH];
    bl::Action actions[bl::RING_MAX_DEPTH];
    const uint32_t n = t->ring.ready(
        [t](uint32_t i) {
            const hipError_t q = hipEventQuery(t->slots[i].done);
            return q == hipSuccess ? bl::Done::OK : q == hipErrorNotReady ? bl::Done::PENDING : bl::Done::FAILED;
        },
        slots, actions);
    for (uint32_t j = 0; j < n; j++) {
        const uint32_t i = slots[j];
        if (actions[j] == bl::Action::READ) {
            if (*n_out >= cap) break;  // no room: it and what follows wait for the next call
            if (read_slot(t, i, out, n_out)) t->stats.frames_timed++;
            else t->stats.frames_failed++;
        } else {
            t->stats.frames_failed++;
        }
        t->ring.release(i);
    }
    return BL_OK;
}

extern "C" int bl_timer_invalidate_submitted(bl_timer *t) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    return (int)t->ring.invalidate();
}

extern "C" int bl_timer_stats(const bl_timer *t, bl_timer_stats_t *out) {
    if (!t || !out) return BL_ERR_INVALID_ARGUMENT;
    *out = t->stats;
    return BL_OK;
}
