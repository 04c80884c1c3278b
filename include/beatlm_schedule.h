/*
 * The frame-budget slice scheduler, its cost model and the host's frame step:
 * the caller of the backend for the high-resolution configuration (a job's
 * kernels handed out as slices across frames inside a per-frame budget). A
 * C++ restatement of the reference's pure logic, behind a C API. No clock and
 * no GPU: the host measures, these decide.
 *
 *   reference                                                     here
 *   ------------------------------------------------------------  -------------------------------
 *   beatlm-core/src/budget.rs:32   Budget::for_frame               bls_budget_for_frame
 *   beatlm-core/src/cost.rs:339    Estimator (4 kinds)             bls_estimator
 *   cost.rs:748                    CostModel::new                  bls_cost_new_with (bls_cost_new:
 *                                                                  the windowed quantile)
 *   cost.rs:779-794                record / record_calibration     bls_cost_record / _record_calibration
 *   cost.rs:851-911                frame_estimate / record_frame / bls_cost_frame_estimate / _record_frame /
 *                                  frame_scale / frames_recorded   _frame_scale / _frames_recorded
 *   cost.rs:927-966                planning_estimate / estimate /  bls_cost_planning_estimate / _estimate /
 *                                  samples                         _samples
 *   cost.rs:666                    nearest_rank                    bls_nearest_rank
 *   beatlm-core/src/time.rs:158-183 BeatGrid                       bls_beat_grid_next
 *   time.rs:194-260                BeatMap                         bls_beat_map_*
 *   beatlm-core/src/sync.rs        SyncPolicy, MissPolicy          bls_policy, BLS_MISS_*
 *   beatlm-core/src/schedule.rs:205 Due                            bls_due
 *   schedule.rs:525-785            Scheduler                       bls_scheduler_*
 *   beatlm-host/src/frame.rs:89-160 RenderCost                     bls_render_cost_*
 *   frame.rs:163-240               Submit, Admission               BLS_SUBMIT_*, inside bls_step
 *   frame.rs:264-283               timer_capacity, jobs_with_slices bls_timer_capacity, bls_jobs_with_slices
 *   beatlm-host/src/step.rs:78-540 StepConfig, FrameStep, Tally    bls_step_*
 *   beatlm/src/gpu/ring.rs:98-111  collect                         bls_collect_action
 *   ring.rs:184-412                Ring (claim, encode, submit,    bls_ring_*
 *                                  submit_held, settle, invalidate,
 *                                  ready, release, in_flight)
 *   ring.rs:113-182                Ticket / Verdict drop, accept,  bls_ticket_drop, bls_hold_verdict
 *                                  reject
 *
 * Times are microseconds (Micros, TimePoint), frames are FrameIndex values.
 * Every call is deterministic. Handles are not thread-safe; one handle may
 * move between threads.
 */
#ifndef BEATLM_SCHEDULE_H
#define BEATLM_SCHEDULE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    BLS_OK = 0,
    BLS_ERR_INVALID = -1,
    BLS_ERR_EMPTY_JOB = -2,            /* ScheduleError::EmptyJob */
    BLS_ERR_INVALID_WINDOW = -3,       /* CostError::InvalidWindow */
    BLS_ERR_INVALID_QUANTILE = -4,     /* CostError::InvalidQuantile */
    BLS_ERR_NO_SUCH_JOB = -5,          /* Scheduler::due gave None */
    BLS_ERR_INVALID_ALPHA = -6,        /* CostError::InvalidAlpha */
    BLS_ERR_INVALID_SIGMAS = -7,       /* CostError::InvalidSigmas */
    BLS_ERR_INVALID_CAP = -8,          /* CostError::InvalidCap */
    BLS_ERR_INVALID_FRAME_WINDOW = -9, /* CostError::InvalidFrameWindow */
    BLS_ERR_NOT_ON_BEAT = -10,         /* ScheduleError::NotOnBeat */
    BLS_ERR_ZERO_BEAT = -11,           /* TimeError::ZeroBeat */
    BLS_ERR_NOT_COUNTED = -12,         /* FrameStep::plan: the frame planned before was never through after_submit */
    BLS_ERR_NOT_PLANNED = -13,         /* after_submit / complete of a frame the step has not planned / counted */
    BLS_ERR_FINISHED = -14             /* the step was closed by bls_step_finish */
};
enum { BLS_MISS_HOLD_PREVIOUS = 0, BLS_MISS_DROP = 1 };   /* MissPolicy */
#define BLS_MAX_WINDOW 4096u                             /* cost.rs:295 MAX_WINDOW */
#define BLS_WARM_SAMPLES 5u                              /* cost.rs:685 WARM_SAMPLES */
#define BLS_TIMER_MAX_SLICES 4096u                       /* slices one bl_timer times in a frame */
#define BLS_RENDER_PRIOR 2000u                           /* beatlm-host/src/presets.rs:47 */
#define BLS_RENDER_WINDOW 32u                            /* presets.rs:52 */
#define BLS_STARTUP_FRAMES 64u                           /* presets.rs:62 */

typedef struct bls_cost bls_cost;
typedef struct bls_scheduler bls_scheduler;
typedef struct bls_beat_map bls_beat_map;
typedef struct bls_render_cost bls_render_cost;
typedef struct bls_step bls_step;

/* FrameInfo (time.rs:121). */
typedef struct {
    uint64_t index;   /* FrameIndex */
    uint64_t start;   /* TimePoint */
    uint64_t period;  /* to the next frame's start */
} bls_frame;

uint64_t bls_budget_for_frame(uint64_t period, uint64_t render, uint64_t margin);
uint32_t bls_nearest_rank(double quantile, uint32_t n);

/* ---- cost model ---------------------------------------------------------- */

enum {
    BLS_EST_MEAN_PLUS_SIGMAS = 0,   /* alpha, sigmas */
    BLS_EST_WINDOWED_QUANTILE = 1,  /* window, quantile */
    BLS_EST_CAPPED_DEVIATION = 2,   /* alpha, sigmas, cap */
    BLS_EST_FRAME_SCALED = 3        /* window, frame_window, quantile (the frame quantile) */
};
typedef struct {
    uint32_t kind;
    uint32_t window;
    uint32_t frame_window;
    uint32_t reserved;
    double alpha;
    double sigmas;
    double cap;
    double quantile;
} bls_estimator;

enum { BLS_SCALE_NONE = 0, BLS_SCALE_WARMING_UP = 1, BLS_SCALE_MEASURED = 2 };  /* FrameScale */
typedef struct {
    uint32_t kind;
    uint32_t reserved;
    uint64_t recorded;   /* WarmingUp */
    uint64_t needed;     /* WarmingUp */
    double scale;        /* Measured */
} bls_frame_scale;

/* The windowed quantile of the last `window` measurements. */
int bls_cost_new(uint64_t prior, uint32_t window, double quantile, bls_cost **out);
int bls_cost_new_with(uint64_t prior, const bls_estimator *estimator, bls_cost **out);
int bls_cost_clone(const bls_cost *c, bls_cost **out);
void bls_cost_free(bls_cost *c);
void bls_cost_estimator(const bls_cost *c, bls_estimator *out);
void bls_cost_record(bls_cost *c, uint32_t slice, uint64_t measured);
void bls_cost_record_calibration(bls_cost *c, uint32_t slice, uint64_t measured);
uint64_t bls_cost_estimate(const bls_cost *c, uint32_t slice);
uint64_t bls_cost_planning_estimate(const bls_cost *c, uint32_t slice);
uint32_t bls_cost_samples(const bls_cost *c, uint32_t slice);
/* 1 and *out set when the slice takes part in a frame's ratio, 0 (None) when not. */
int bls_cost_frame_estimate(const bls_cost *c, uint32_t slice, uint64_t *out);
void bls_cost_record_frame(bls_cost *c, uint64_t predicted, uint64_t measured);
void bls_cost_frame_scale(const bls_cost *c, bls_frame_scale *out);
uint64_t bls_cost_frames_recorded(const bls_cost *c);

/* ---- beats ------------------------------------------------------------- */

/* BeatGrid::next_beat_at_or_after for the grid (origin, beat). */
int bls_beat_grid_next(uint64_t origin, uint64_t beat, uint64_t t, uint64_t *out);
int bls_beat_map_new(uint64_t origin, uint64_t beat, bls_beat_map **out);
void bls_beat_map_free(bls_beat_map *m);
int bls_beat_map_replace_from(bls_beat_map *m, uint64_t from, uint64_t origin, uint64_t beat);
uint64_t bls_beat_map_next(const bls_beat_map *m, uint64_t t);
void bls_beat_map_forget_before(bls_beat_map *m, uint64_t t);
uint32_t bls_beat_map_grids(const bls_beat_map *m);

/* ---- scheduler --------------------------------------------------------- */

enum { BLS_POLICY_FIXED_LATENCY = 0, BLS_POLICY_SAME_FRAME = 1, BLS_POLICY_ON_BEAT = 2 };
typedef struct {
    uint32_t kind;
    uint32_t frames;        /* FixedLatency */
    uint64_t margin;        /* OnBeat */
    uint64_t grid_origin;   /* OnBeat */
    uint64_t grid_beat;     /* OnBeat */
} bls_policy;
/* SyncPolicy::source_delay / max_in_flight: 1 and *out set, or 0 (None). */
int bls_policy_source_delay(const bls_policy *p, uint32_t *out);
int bls_policy_max_in_flight(const bls_policy *p, uint32_t *out);

enum { BLS_DUE_FRAME = 0, BLS_DUE_BEAT = 1 };
typedef struct { uint32_t kind; uint32_t reserved; uint64_t at; } bls_due;  /* a FrameIndex or a TimePoint */

typedef struct { uint64_t job; uint32_t slice; uint32_t position; } bls_run;          /* SliceRun */
typedef struct { uint64_t job; uint64_t input; } bls_delivery;                        /* Delivery */
typedef struct { uint64_t job; uint64_t input; bls_due due; uint32_t policy; uint32_t reserved; } bls_missed;

/* FramePlan. The arrays stay valid until the next plan of the scheduler (or,
 * for a step, as bls_step_plan and bls_step_complete say). */
typedef struct {
    uint32_t n_runs, n_delivered, n_missed, reserved;
    const bls_run *runs;
    const bls_delivery *delivered;
    const bls_missed *missed;
    uint64_t spent_estimate;
    uint64_t budget;
} bls_frame_plan;

/* FixedLatency { frames } (SameFrame is 0 frames). */
int bls_scheduler_new(uint32_t latency_frames, uint32_t miss_policy, uint64_t expected_budget, bls_scheduler **out);
int bls_scheduler_new_policy(const bls_policy *policy, uint32_t miss_policy, uint64_t expected_budget,
                             bls_scheduler **out);
void bls_scheduler_free(bls_scheduler *s);
void bls_scheduler_set_expected_budget(bls_scheduler *s, uint64_t expected);
uint64_t bls_scheduler_expected_budget(const bls_scheduler *s);
int bls_scheduler_replace_beat_grid(bls_scheduler *s, uint64_t from, uint64_t origin, uint64_t beat);
int bls_scheduler_submit(bls_scheduler *s, const bls_frame *input, const uint32_t *slices, uint32_t n,
                         const bls_cost *cost, uint64_t *job_out);
int bls_scheduler_plan_frame(bls_scheduler *s, const bls_frame *frame, uint64_t budget, const bls_cost *cost,
                             bls_frame_plan *out);
uint32_t bls_scheduler_pending(const bls_scheduler *s);
int bls_scheduler_due(const bls_scheduler *s, uint64_t job, bls_due *out);

/* ---- the slice timer's ring (no GPU in it) ------------------------------- */
/* Which ring slot a frame's timing uses and when it may be read; the HIP
 * slice timer (bl_timer_*) runs one ring per timer. A slot goes FREE ->
 * RECORDING (bls_ring_claim) -> ENCODED (bls_ring_encode hands out a ticket)
 * -> SUBMITTED (the ticket came back through bls_ring_submit) or HELD
 * (bls_ring_submit_held: read only once its verdict accepts it) -> FREE
 * (bls_ring_release, once collected). INVALID: submitted or held, then marked
 * by bls_ring_invalidate or rejected; freed unread once its work completes.
 *
 * Tickets and holds are nonzero 64-bit values naming the ring, the slot and
 * the lap: one from an earlier lap is refused, and one handed to another ring
 * is refused there and dropped in its own ring. A ticket is spent by exactly
 * one of bls_ring_submit, bls_ring_submit_held or bls_ticket_drop; a ticket
 * dropped frees its slot unread at the ring's next claim. A hold is spent by
 * bls_hold_verdict (the C form of Verdict::accept / reject; a verdict never
 * given keeps its slot, and every later read, waiting until the ring is
 * invalidated). bls_ticket_drop and bls_hold_verdict may be called from any
 * thread; a ring from one thread at a time. */
typedef struct bls_ring bls_ring;
enum { BLS_PHASE_FREE = 0, BLS_PHASE_RECORDING = 1, BLS_PHASE_ENCODED = 2, BLS_PHASE_SUBMITTED = 3,
       BLS_PHASE_HELD = 4, BLS_PHASE_INVALID = 5 };
/* Where a slot's work stands (its closing event: pending, completed, failed). */
enum { BLS_DONE_PENDING = 0, BLS_DONE_OK = 1, BLS_DONE_FAILED = 2 };
enum { BLS_COLLECT_WAIT = 0, BLS_COLLECT_READ = 1, BLS_COLLECT_DROP = 2 };
#define BLS_RING_MAX_DEPTH 64

/* collect (ring.rs:98-111): READ only SUBMITTED with its work completed;
 * DROP an INVALID slot once its work completed or failed, and a SUBMITTED
 * one whose work failed; WAIT otherwise (HELD always). */
uint32_t bls_collect_action(uint32_t phase, uint32_t done);
/* `depth` free slots (0 is raised to 1); BLS_ERR_INVALID above BLS_RING_MAX_DEPTH. */
int bls_ring_new(uint32_t depth, bls_ring **out);
void bls_ring_free(bls_ring *r);
uint32_t bls_ring_depth(const bls_ring *r);
/* Frees slots whose ticket was dropped, then takes the slot at the cursor if
 * it is free and moves the cursor on; -1 when it is busy (the cursor stays). */
int32_t bls_ring_claim(bls_ring *r);
/* The RECORDING slot's frame is closed: its ticket, 0 if not recording. */
uint64_t bls_ring_encode(bls_ring *r, uint32_t slot);
/* The ticket comes back after its work was submitted: the slot, now
 * SUBMITTED, or -1 (not this ring's, an earlier lap's, or dropped). */
int32_t bls_ring_submit(bls_ring *r, uint64_t ticket);
/* bls_ring_submit, but the slot is HELD; *hold names it for bls_hold_verdict. */
int32_t bls_ring_submit_held(bls_ring *r, uint64_t ticket, uint64_t *hold);
/* The frame's work was never submitted (or the host cannot tell). */
void bls_ticket_drop(uint64_t ticket);
/* 1 when the verdict reached its HELD slot; 0 when the slot moved on
 * (invalidated, released, held again by a later frame) or the ring is gone.
 * The slot moves at the ring's next bls_ring_settle. */
int bls_hold_verdict(uint64_t hold, uint32_t accepted);
void bls_ring_settle(bls_ring *r);
/* Every SUBMITTED or HELD slot -> INVALID; returns how many moved. */
uint32_t bls_ring_invalidate(bls_ring *r);
/* The slots to collect now, oldest submission first, given `done[slot]`
 * (BLS_DONE_*, one per slot of the ring): a READ waits while a slot
 * submitted before it is HELD or SUBMITTED with its work pending; DROPs
 * never wait. Writes up to depth entries to `slots` and `actions`. */
uint32_t bls_ring_ready(const bls_ring *r, const uint8_t *done, uint32_t *slots, uint8_t *actions);
void bls_ring_release(bls_ring *r, uint32_t slot);
/* Slots neither FREE nor waiting on a dropped ticket. */
uint32_t bls_ring_in_flight(const bls_ring *r);
/* BLS_PHASE_*, -1 for a slot the ring does not have. */
int32_t bls_ring_phase(const bls_ring *r, uint32_t slot);
/* Slots freed so far because their ticket was dropped. */
uint64_t bls_ring_reclaimed(const bls_ring *r);

/* ---- the host's frame step ---------------------------------------------- */

int bls_render_cost_new(bls_render_cost **out);
void bls_render_cost_free(bls_render_cost *r);
void bls_render_cost_record(bls_render_cost *r, uint64_t render);
uint64_t bls_render_cost_last(const bls_render_cost *r);
uint64_t bls_render_cost_forecast(const bls_render_cost *r);
uint64_t bls_render_cost_budget(const bls_render_cost *r, uint64_t period, uint64_t margin);
uint64_t bls_render_cost_expected(const bls_render_cost *r, uint64_t period, uint64_t margin);

enum { BLS_SUBMIT_EVERY = 0, BLS_SUBMIT_FREE = 1 };
enum { BLS_IN_FLIGHT_LATENCY = 0, BLS_IN_FLIGHT_BOUNDED = 1 };
/* 1 and *out set, or 0 (None: over BLS_TIMER_MAX_SLICES, or overflow). */
int bls_timer_capacity(uint32_t slices, uint32_t jobs, uint32_t *out);
int bls_jobs_with_slices(uint32_t submit, uint32_t in_flight_kind, uint32_t in_flight, uint32_t *out);

typedef struct {
    bls_policy policy;
    uint32_t miss;
    uint32_t slices;        /* per job */
    uint64_t margin;
    uint64_t prior_period;
    uint32_t submit;
    uint32_t reserved;
} bls_step_config;

/* Planned. Its plan's arrays stay valid until the frame's bls_step_complete. */
typedef struct {
    bls_frame frame;
    bls_frame_plan plan;
    uint64_t job;
    uint32_t has_job;
    uint32_t has_due;
    bls_due due;            /* read between the submission and the plan */
    uint64_t budget;
    uint64_t expected;
} bls_planned;

/* One timed compute pass, labelled with its Tag (frame.rs:28). */
typedef struct {
    uint64_t job;
    uint32_t slice;
    uint32_t has_planned;
    uint64_t planned;       /* the frame estimate the pass was tagged with */
    uint64_t duration;
} bls_timed_slice;

/* FrameTiming, without the pass timestamps. */
typedef struct {
    uint64_t frame;
    const bls_timed_slice *compute;
    uint32_t n_compute;
    uint32_t has_render;
    uint64_t render;
} bls_frame_timing;

typedef struct { uint64_t frame; uint32_t has_render; uint32_t ran_slices; uint64_t render; } bls_absorbed;

typedef struct { uint32_t slice; uint32_t reserved; uint64_t sum; uint64_t count; } bls_slice_measured;
typedef struct { uint32_t slice; uint32_t reserved; uint64_t estimate; } bls_slice_estimate;

/* Tally. The arrays stay valid until bls_step_free. `timed_frames` counts the
 * frames absorbed (the reference keeps their passes for its overlap report). */
typedef struct {
    uint64_t submitted, delivered, missed, startup_missed, violations, pending_at_end;
    uint64_t n_latencies, n_dispatches_per_frame, n_dispatches_per_job, n_gpu_frame_us, n_longest_dispatch_us;
    const uint64_t *latencies, *dispatches_per_frame, *dispatches_per_job, *gpu_frame_us, *longest_dispatch_us;
    uint64_t n_measured, n_estimates, n_frame_ratios, n_frame_scales;
    const bls_slice_measured *measured;
    const bls_slice_estimate *estimates;
    const double *frame_ratios;
    const double *frame_scales;
    bls_frame_scale frame_scale;
    uint64_t frames_recorded;
    uint64_t timed_frames;
} bls_tally;

/* FrameStep::new; the step keeps a copy of `cost`. */
int bls_step_new(const bls_step_config *config, const bls_cost *cost, bls_step **out);
void bls_step_free(bls_step *s);
int bls_step_replace_beat_grid(bls_step *s, uint64_t from, uint64_t origin, uint64_t beat);
const bls_cost *bls_step_cost(const bls_step *s);
uint64_t bls_step_submitted(const bls_step *s);
uint64_t bls_step_dispatched(const bls_step *s, uint64_t job);
/* BLS_ERR_NOT_COUNTED when the frame planned before (written to *unsubmitted
 * when given) was never through bls_step_after_submit: the step is over. */
int bls_step_plan(bls_step *s, const bls_frame *frame, int owed, bls_planned *out, uint64_t *unsubmitted);
/* FrameStep::tag: the frame estimate a pass of `slice` is labelled with. */
int bls_step_tag(const bls_step *s, uint32_t slice, uint64_t *planned);
int bls_step_after_submit(bls_step *s, uint64_t frame_index);
int bls_step_absorb(bls_step *s, const bls_frame_timing *timing, bls_absorbed *out);
/* Counts the frame's deliveries and misses; *out's arrays stay valid until
 * the next bls_step_complete. */
int bls_step_complete(bls_step *s, uint64_t frame_index, bls_frame_plan *out);
int bls_step_finish(bls_step *s, bls_tally *out);

#ifdef __cplusplus
}
#endif
#endif
