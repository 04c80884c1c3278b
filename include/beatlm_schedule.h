/*
 * The frame-budget slice scheduler and its cost model, the caller of the
 * backend for the high-resolution configuration (a job's kernels handed out
 * as slices across frames inside a per-frame budget). A C++ restatement of
 * the reference core's pure logic, behind a C API:
 *
 *   reference (crates/beatlm-core/src)                  here
 *   --------------------------------------------------  ----------------------------
 *   Budget::for_frame               budget.rs:32        bls_budget_for_frame
 *   CostModel::new(prior, WindowedQuantile{window, q})  cost.rs:748  bls_cost_new
 *   CostModel::record / record_calibration cost.rs:779-794  bls_cost_record / _record_calibration
 *   CostModel::estimate / planning_estimate cost.rs:927-964  bls_cost_estimate / _planning_estimate
 *   CostModel::samples              cost.rs:966         bls_cost_samples
 *   nearest_rank                    cost.rs:666         bls_nearest_rank
 *   Scheduler::new(FixedLatency|SameFrame, miss, expected)  schedule.rs:525  bls_scheduler_new
 *   Scheduler::submit               schedule.rs:618     bls_scheduler_submit
 *   Scheduler::plan_frame           schedule.rs:706     bls_scheduler_plan_frame
 *   Scheduler::set_expected_budget / pending / due  schedule.rs:553, :773, :779
 *
 * Times are microseconds (Micros), frames are FrameIndex values. The OnBeat
 * policy and the other estimators are not restated.
 */
#ifndef BEATLM_SCHEDULE_H
#define BEATLM_SCHEDULE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BLS_OK = 0, BLS_ERR_INVALID = -1, BLS_ERR_EMPTY_JOB = -2, BLS_ERR_INVALID_WINDOW = -3,
       BLS_ERR_INVALID_QUANTILE = -4, BLS_ERR_NO_SUCH_JOB = -5 };
enum { BLS_MISS_HOLD_PREVIOUS = 0, BLS_MISS_DROP = 1 };   /* MissPolicy */
#define BLS_MAX_WINDOW 4096u                             /* cost.rs:295 */

typedef struct bls_cost bls_cost;
typedef struct bls_scheduler bls_scheduler;

typedef struct {
    uint64_t index;   /* FrameIndex */
    uint64_t start;   /* TimePoint, microseconds */
    uint64_t period;  /* microseconds to the next frame's start */
} bls_frame;

typedef struct { uint64_t job; uint32_t slice; uint32_t position; } bls_run;          /* SliceRun */
typedef struct { uint64_t job; uint64_t input; } bls_delivery;                        /* Delivery */
typedef struct { uint64_t job; uint64_t input; uint64_t due_frame; uint32_t policy; uint32_t reserved; } bls_missed;

/* FramePlan; the arrays stay valid until the scheduler's next plan. */
typedef struct {
    uint32_t n_runs, n_delivered, n_missed, reserved;
    const bls_run *runs;
    const bls_delivery *delivered;
    const bls_missed *missed;
    uint64_t spent_estimate;
    uint64_t budget;
} bls_frame_plan;

uint64_t bls_budget_for_frame(uint64_t period, uint64_t render, uint64_t margin);
uint32_t bls_nearest_rank(double quantile, uint32_t n);

int bls_cost_new(uint64_t prior, uint32_t window, double quantile, bls_cost **out);
void bls_cost_free(bls_cost *c);
void bls_cost_record(bls_cost *c, uint32_t slice, uint64_t measured);
void bls_cost_record_calibration(bls_cost *c, uint32_t slice, uint64_t measured);
uint64_t bls_cost_estimate(const bls_cost *c, uint32_t slice);
uint64_t bls_cost_planning_estimate(const bls_cost *c, uint32_t slice);
uint32_t bls_cost_samples(const bls_cost *c, uint32_t slice);

/* FixedLatency { frames } (SameFrame is 0 frames). */
int bls_scheduler_new(uint32_t latency_frames, uint32_t miss_policy, uint64_t expected_budget, bls_scheduler **out);
void bls_scheduler_free(bls_scheduler *s);
void bls_scheduler_set_expected_budget(bls_scheduler *s, uint64_t expected);
uint64_t bls_scheduler_expected_budget(const bls_scheduler *s);
int bls_scheduler_submit(bls_scheduler *s, const bls_frame *input, const uint32_t *slices, uint32_t n,
                         const bls_cost *cost, uint64_t *job_out);
int bls_scheduler_plan_frame(bls_scheduler *s, const bls_frame *frame, uint64_t budget, const bls_cost *cost,
                             bls_frame_plan *out);
uint32_t bls_scheduler_pending(const bls_scheduler *s);
int bls_scheduler_due(const bls_scheduler *s, uint64_t job, uint64_t *due_frame);

#ifdef __cplusplus
}
#endif
#endif
