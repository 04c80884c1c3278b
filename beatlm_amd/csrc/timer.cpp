// The slice timer: per-slice GPU durations from hipEvent pairs, read back
// without ever blocking. The HIP counterpart of the reference's SliceTimer
// (crates/beatlm/src/gpu/timer.rs:185-464) and its ring
// (crates/beatlm/src/gpu/ring.rs):
//
//  - a ring of BL_TIMER_RING_DEPTH frames in flight, each with an event pair
//    per slice and one event closing the frame, all created once;
//  - a frame whose slot is still in flight when it begins is not timed, and
//    is counted skipped; nothing waits;
//  - only frames the host hands back as submitted are read, in submission
//    order; a resolved frame never handed back frees its slot unread;
//  - frames the host marks (bl_timer_invalidate_submitted) are never
//    decoded: they free their slot and count as failed;
//  - completion is polled with hipEventQuery, so collecting never blocks.
#include <hip/hip_runtime.h>

#include <deque>
#include <string>
#include <vector>

#include "timer.hpp"
#include "../../include/beatlm_schedule.h"

namespace {

enum class State { FREE, RECORDING, RESOLVED, SUBMITTED };

struct Slot {
    State state = State::FREE;
    bool invalid = false;
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
    std::vector<Slot> slots;
    int open = -1;                 // slot of the frame being recorded, -1 when untimed
    bool frame_open = false;
    bool render_begun = false;     // the open frame's render pass was requested
    std::deque<int> submitted;     // submission order
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
    // A frame still open, or resolved and never handed back, is dropped unread.
    for (Slot &s : t->slots) {
        if (s.state == State::RECORDING || s.state == State::RESOLVED) {
            s.state = State::FREE;
            t->stats.frames_dropped++;
        }
    }
    t->stats.frames_begun++;
    t->frame_open = true;
    t->render_begun = false;
    t->open = -1;
    for (size_t i = 0; i < t->slots.size(); i++) {
        if (t->slots[i].state == State::FREE) {
            t->open = (int)i;
            break;
        }
    }
    if (t->open < 0) {
        t->stats.frames_skipped++;
    } else {
        Slot &s = t->slots[t->open];
        s.state = State::RECORDING;
        s.invalid = false;
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

extern "C" int bl_timer_resolve(bl_timer *t, uint32_t *resolved) {
    if (!t || !resolved) return BL_ERR_INVALID_ARGUMENT;
    if (!t->frame_open) return bl_fail(t->ctx, BL_ERR_TIMER_NO_FRAME, "no frame is open on the timer");
    t->frame_open = false;
    if (t->open < 0) {
        *resolved = UINT32_MAX;  // untimed: handing it back is accepted and ignored
        return BL_OK;
    }
    Slot &s = t->slots[t->open];
    if (hipEventRecord(s.done, bl_stream_of(t->ctx)) != hipSuccess)
        return bl_fail(t->ctx, BL_ERR_HIP, "hipEventRecord");
    s.state = State::RESOLVED;
    *resolved = (uint32_t)t->open;
    t->open = -1;
    return BL_OK;
}

extern "C" int bl_timer_submitted(bl_timer *t, uint32_t resolved) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    if (resolved >= t->slots.size()) return BL_OK;
    Slot &s = t->slots[resolved];
    if (s.state != State::RESOLVED) return BL_OK;
    s.state = State::SUBMITTED;
    t->submitted.push_back((int)resolved);
    return BL_OK;
}

extern "C" int bl_timer_collect(bl_timer *t, bl_frame_timing *out, uint32_t cap, uint32_t *n_out) {
    if (!t || !n_out || (cap && !out)) return BL_ERR_INVALID_ARGUMENT;
    *n_out = 0;
    t->out_tags.clear();
    t->out_micros.clear();
    t->out_tags.reserve(cap);
    t->out_micros.reserve(cap);
    while (!t->submitted.empty()) {
        Slot &s = t->slots[t->submitted.front()];
        hipError_t q = hipEventQuery(s.done);
        if (q == hipErrorNotReady) break;  // later frames wait: submission order
        bool ok = q == hipSuccess && !s.invalid;
        if (ok && *n_out >= cap) break;   // no room: leave it for the next call
        if (ok) {
            std::vector<uint32_t> tags(s.tags.begin(), s.tags.begin() + s.used);
            std::vector<float> micros(s.used, 0.0f);
            for (uint32_t i = 0; i < s.used && ok; i++) {
                float ms = 0.0f;
                if (hipEventElapsedTime(&ms, s.events[2 * i], s.events[2 * i + 1]) != hipSuccess) ok = false;
                micros[i] = ms * 1000.0f;
            }
            if (ok) {
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
                t->stats.frames_timed++;
            }
        }
        if (!ok) t->stats.frames_failed++;
        s.state = State::FREE;
        t->submitted.pop_front();
    }
    return BL_OK;
}

extern "C" int bl_timer_invalidate_submitted(bl_timer *t) {
    if (!t) return BL_ERR_INVALID_ARGUMENT;
    int marked = 0;
    for (int i : t->submitted) {
        if (!t->slots[i].invalid) marked++;
        t->slots[i].invalid = true;
    }
    return marked;
}

extern "C" int bl_timer_stats(const bl_timer *t, bl_timer_stats_t *out) {
    if (!t || !out) return BL_ERR_INVALID_ARGUMENT;
    *out = t->stats;
    return BL_OK;
}
