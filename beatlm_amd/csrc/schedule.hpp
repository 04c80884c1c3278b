// Internal classes behind include/beatlm_schedule.h: the cost model
// (cost.cpp), beats and the scheduler (schedule.cpp) and the host's frame step
// (step.cpp). Pure logic: no clock, no GPU.
#pragma once

#include "../../include/beatlm_schedule.h"

#include <cstddef>
#include <cstdint>
#include <deque>
#include <map>
#include <optional>
#include <vector>

namespace bls {

inline uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
inline uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }
inline uint64_t sat_mul(uint64_t a, uint64_t b) { return (b != 0 && a > UINT64_MAX / b) ? UINT64_MAX : a * b; }

size_t nearest_rank(double q, size_t n);

// ---- cost model (crates/beatlm-core/src/cost.rs) ----

// A slice's last `capacity` measurements with the quantile(s) read from them
// at each fold (cost.rs:521-576).
struct Window {
    std::vector<uint64_t> ring;
    size_t next = 0;
    uint64_t estimate = 0;
    uint64_t second = 0;  // a second quantile; the estimate when none is asked
    uint32_t samples = 0;
    void fold(uint64_t x, size_t capacity, double q, std::optional<double> second_q);
};

struct SliceStats {
    // MeanPlusSigmas / CappedDeviation: exponentially weighted mean and variance.
    double mean = 0.0, var = 0.0;
    uint32_t ewma_samples = 0;
    // WindowedQuantile uses `all`; FrameScaled keeps every measurement in
    // `all` (estimate: the frame quantile; second: the median) and the loop's
    // alone in `looped` (estimate: the median).
    Window all, looped;
    bool warm() const { return looped.samples >= BLS_WARM_SAMPLES; }
};

class CostModel {
public:
    static int make(uint64_t prior, const bls_estimator &e, CostModel &out);
    const bls_estimator &estimator() const { return est_; }
    void record(uint32_t slice, uint64_t measured) { fold(slice, measured, true); }
    void record_calibration(uint32_t slice, uint64_t measured) { fold(slice, measured, false); }
    uint64_t estimate(uint32_t slice) const;
    uint64_t planning_estimate(uint32_t slice) const;
    uint32_t samples(uint32_t slice) const;
    std::optional<uint64_t> frame_estimate(uint32_t slice) const;
    void record_frame(uint64_t predicted, uint64_t measured);
    bls_frame_scale frame_scale() const;
    uint64_t frames_recorded() const { return frames_recorded_; }

private:
    void fold(uint32_t slice, uint64_t measured, bool in_loop);
    const SliceStats *find(uint32_t slice) const;

    uint64_t prior_ = 0;
    bls_estimator est_{};
    std::map<uint32_t, SliceStats> stats_;  // ordered: identical inputs, identical estimates
    // FrameScaled: the last frames' (ratio, weight) and the scale read from a full window.
    std::vector<std::pair<double, double>> frames_;
    size_t frames_next_ = 0;
    double scale_ = 1.0;
    uint64_t frames_recorded_ = 0;
};

}  // namespace bls

// A cost-model handle of the C API.
struct bls_cost {
    bls::CostModel m;
};

namespace bls {

inline const CostModel &model_of(const bls_cost *c) { return c->m; }

// ---- beats (crates/beatlm-core/src/time.rs) ----

struct BeatGrid {
    uint64_t origin = 0, beat = 1;
    uint64_t next_at_or_after(uint64_t t) const;
};

class BeatMap {
public:
    explicit BeatMap(BeatGrid g) : grids_{{0, g}} {}
    void replace_from(uint64_t from, BeatGrid g);
    uint64_t next_at_or_after(uint64_t t) const;
    void forget_before(uint64_t t);
    size_t size() const { return grids_.size(); }

private:
    size_t in_effect(uint64_t t) const;             // index of the grid in effect at t
    std::vector<std::pair<uint64_t, BeatGrid>> grids_;  // (from, grid), strictly increasing from
};

// ---- scheduler (crates/beatlm-core/src/schedule.rs) ----

struct Due {
    uint32_t kind = BLS_DUE_FRAME;
    uint64_t at = 0;
    bool reached(const bls_frame &f) const;
    bool on_time(const bls_frame &f) const;
    std::optional<uint64_t> frames_left(const bls_frame &f) const;
};

struct FramePlan {
    std::vector<bls_run> runs;
    std::vector<bls_delivery> delivered;
    std::vector<bls_missed> missed;
    uint64_t spent = 0, budget = 0;
    void expose(bls_frame_plan &out) const;
};

class Scheduler {
public:
    Scheduler(const bls_policy &policy, uint32_t miss, uint64_t expected);
    void set_expected_budget(uint64_t e) { expected_ = e; }
    uint64_t expected_budget() const { return expected_; }
    int replace_beat_grid(uint64_t from, BeatGrid g);
    int submit(const bls_frame &input, const uint32_t *slices, size_t n, const CostModel &cost, uint64_t &job);
    void plan_frame(const bls_frame &frame, uint64_t budget, const CostModel &cost, FramePlan &out);
    size_t pending() const { return pending_.size(); }
    std::optional<Due> due(uint64_t job) const;

    struct Cursor {
        uint64_t frame = 0, spent = 0;
    };
    struct Budgets {
        uint64_t now, later;
        uint64_t of(uint64_t frame) const { return frame == 0 ? now : later; }
    };
    struct Job {
        uint64_t id, input;
        std::vector<uint32_t> slices;
        size_t scheduled = 0;
        Due deadline;
        bool abandoned = false;
    };

private:
    Cursor projected_end(const bls_frame &frame, Budgets b, const CostModel &cost) const;

    bool on_beat_;
    uint32_t frames_ = 0;
    uint64_t margin_ = 0;
    BeatMap beats_;
    uint32_t miss_;
    uint64_t expected_;
    uint64_t next_job_ = 0;
    std::vector<Job> pending_;
};

}  // namespace bls
