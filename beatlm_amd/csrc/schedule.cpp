// The frame-budget slice scheduler (FixedLatency) and the windowed-quantile
// cost model: a C++ restatement of crates/beatlm-core/src/{schedule,cost,
// budget}.rs behind include/beatlm_schedule.h. Pure logic: no clock, no GPU.
#include "../../include/beatlm_schedule.h"

#include <algorithm>
#include <cmath>
#include <map>
#include <vector>

namespace {

uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }
uint64_t sat_sub(uint64_t a, uint64_t b) { return a > b ? a - b : 0; }

// nearest_rank (cost.rs:666-679): ceil(q n), a product within 1e-9 of a whole
// number taken as that number, clamped to 1..=n.
size_t nearest_rank(double q, size_t n) {
    const double product = q * (double)n;
    const double nearest = std::round(product);
    const double rank = std::fabs(product - nearest) < 1e-9 ? nearest : std::ceil(product);
    size_t r = (size_t)rank;
    return std::min(std::max<size_t>(r, 1), std::max<size_t>(n, 1));
}

// One slice's last `window` measurements and the quantile read from them
// (cost.rs:521-576).
struct Window {
    std::vector<uint64_t> ring;
    size_t next = 0;
    uint64_t estimate = 0;
    uint32_t samples = 0;

    void fold(uint64_t x, size_t capacity, double q) {
        if (ring.size() < capacity) ring.push_back(x);
        else ring[next] = x;
        next = (next + 1) % capacity;
        if (samples < UINT32_MAX) samples++;
        std::vector<uint64_t> scratch(ring);
        const size_t rank = nearest_rank(q, scratch.size());
        std::nth_element(scratch.begin(), scratch.begin() + (rank - 1), scratch.end());
        estimate = scratch[rank - 1];
    }
};

}  // namespace

struct bls_cost {
    uint64_t prior;
    size_t window;
    double quantile;
    std::map<uint32_t, Window> stats;  // ordered: identical measurements, identical estimates
};

extern "C" uint32_t bls_nearest_rank(double quantile, uint32_t n) { return (uint32_t)nearest_rank(quantile, n); }

extern "C" uint64_t bls_budget_for_frame(uint64_t period, uint64_t render, uint64_t margin) {
    return sat_sub(sat_sub(period, render), margin);
}

extern "C" int bls_cost_new(uint64_t prior, uint32_t window, double quantile, bls_cost **out) {
    if (window == 0 || window > BLS_MAX_WINDOW) return BLS_ERR_INVALID_WINDOW;
    if (!(std::isfinite(quantile) && quantile >= 0.0 && quantile <= 1.0)) return BLS_ERR_INVALID_QUANTILE;
    *out = new bls_cost{prior, window, quantile, {}};
    return BLS_OK;
}
extern "C" void bls_cost_free(bls_cost *c) { delete c; }
extern "C" void bls_cost_record(bls_cost *c, uint32_t slice, uint64_t measured) {
    c->stats[slice].fold(measured, c->window, c->quantile);
}
// The windowed quantile folds a calibration measurement as a loop one (cost.rs:792-797).
extern "C" void bls_cost_record_calibration(bls_cost *c, uint32_t slice, uint64_t measured) {
    bls_cost_record(c, slice, measured);
}
extern "C" uint64_t bls_cost_estimate(const bls_cost *c, uint32_t slice) {
    auto it = c->stats.find(slice);
    return it == c->stats.end() ? c->prior : it->second.estimate;
}
extern "C" uint64_t bls_cost_planning_estimate(const bls_cost *c, uint32_t slice) { return bls_cost_estimate(c, slice); }
extern "C" uint32_t bls_cost_samples(const bls_cost *c, uint32_t slice) {
    auto it = c->stats.find(slice);
    return it == c->stats.end() ? 0 : it->second.samples;
}

namespace {

// Where projected work ends: a frame counted from the planned one and the
// estimate already placed in it (schedule.rs:322-345).
struct Cursor {
    uint64_t frame = 0;
    uint64_t spent = 0;
};

struct Placed {
    bool fits;   // false: a slice fits no frame after the planned one
    Cursor end;
    size_t now;  // leading slices that landed in the planned frame
};

struct Budgets {
    uint64_t now, later;
    uint64_t of(uint64_t frame) const { return frame == 0 ? now : later; }

    // Budgets::place (schedule.rs:381-406): slices in order onto frames; a
    // frame takes slices while they fit, the first that does not opens the next.
    Placed place(Cursor at, const uint32_t *slices, size_t n, const bls_cost *cost) const {
        size_t now_count = 0;
        for (size_t i = 0; i < n; i++) {
            const uint64_t estimate = bls_cost_planning_estimate(cost, slices[i]);
            for (;;) {
                const uint64_t after = sat_add(at.spent, estimate);
                if (after <= of(at.frame)) {
                    at.spent = after;
                    break;
                }
                if (at.frame > 0 && at.spent == 0) return Placed{false, at, now_count};
                at = Cursor{sat_add(at.frame, 1), 0};
            }
            if (at.frame == 0) now_count++;
        }
        return Placed{true, at, now_count};
    }
};

enum class Fate { Passed, Abandoned, Late, Kept };

struct Job {
    uint64_t id;
    uint64_t input;
    std::vector<uint32_t> slices;
    size_t scheduled = 0;
    uint64_t deadline;  // Due::Frame
    bool abandoned = false;

    bool complete() const { return scheduled >= slices.size(); }
    // Due::frames_left (schedule.rs:245-251): none once the deadline is behind.
    bool frames_left(uint64_t frame, uint64_t &left) const {
        if (deadline < frame) return false;
        left = deadline - frame;
        return true;
    }
    bool passed(uint64_t frame) const { return deadline < frame; }

    // Job::fate (schedule.rs:447-471).
    Fate fate(Cursor from, uint64_t frame, Budgets b, const bls_cost *cost, bool behind, size_t &now, Cursor &end) const {
        uint64_t left;
        if (!frames_left(frame, left)) return Fate::Passed;
        if (scheduled >= slices.size()) {
            now = 0;
            end = from;
            return Fate::Kept;
        }
        Placed p = b.place(from, slices.data() + scheduled, slices.size() - scheduled, cost);
        if (p.fits && p.end.frame <= left) {
            now = p.now;
            end = p.end;
            return Fate::Kept;
        }
        if (behind) return Fate::Abandoned;
        now = p.now;
        return Fate::Late;
    }

    void hand_out(size_t count, const bls_cost *cost, std::vector<bls_run> &runs, uint64_t &spent) {
        for (size_t i = 0; i < count && scheduled < slices.size(); i++) {
            runs.push_back(bls_run{id, slices[scheduled], (uint32_t)scheduled});
            spent = sat_add(spent, bls_cost_planning_estimate(cost, slices[scheduled]));
            scheduled++;
        }
    }
};

}  // namespace

struct bls_scheduler {
    uint32_t frames;
    uint32_t miss;
    uint64_t expected;
    uint64_t next_job = 0;
    std::vector<Job> pending;
    std::vector<bls_run> runs;
    std::vector<bls_delivery> delivered;
    std::vector<bls_missed> missed;
};

extern "C" int bls_scheduler_new(uint32_t latency_frames, uint32_t miss_policy, uint64_t expected, bls_scheduler **out) {
    if (miss_policy > BLS_MISS_DROP) return BLS_ERR_INVALID;
    *out = new bls_scheduler{latency_frames, miss_policy, expected};
    return BLS_OK;
}
extern "C" void bls_scheduler_free(bls_scheduler *s) { delete s; }
extern "C" void bls_scheduler_set_expected_budget(bls_scheduler *s, uint64_t e) { s->expected = e; }
extern "C" uint64_t bls_scheduler_expected_budget(const bls_scheduler *s) { return s->expected; }

// Scheduler::submit (schedule.rs:618-661), FixedLatency: due `frames` after the input.
extern "C" int bls_scheduler_submit(bls_scheduler *s, const bls_frame *input, const uint32_t *slices, uint32_t n,
                                    const bls_cost *, uint64_t *job_out) {
    if (n == 0) return BLS_ERR_EMPTY_JOB;
    Job j;
    j.id = s->next_job;
    s->next_job = sat_add(s->next_job, 1);
    j.input = input->index;
    j.slices.assign(slices, slices + n);
    j.deadline = sat_add(input->index, s->frames);
    s->pending.push_back(std::move(j));
    if (job_out) *job_out = s->pending.back().id;
    return BLS_OK;
}

// Scheduler::plan_frame (schedule.rs:706-769).
extern "C" int bls_scheduler_plan_frame(bls_scheduler *s, const bls_frame *frame, uint64_t budget, const bls_cost *cost,
                                        bls_frame_plan *out) {
    const Budgets budgets{budget, s->expected};
    s->runs.clear();
    s->delivered.clear();
    s->missed.clear();
    uint64_t spent = 0;
    Cursor at;
    // A job waits behind another when it comes after it and this plan does
    // not report it missed for a deadline already behind the frame.
    long last_waiting = -1;
    for (long i = (long)s->pending.size() - 1; i >= 0; i--)
        if (!s->pending[i].passed(frame->index)) {
            last_waiting = i;
            break;
        }
    for (size_t i = 0; i < s->pending.size(); i++) {
        Job &job = s->pending[i];
        const bool behind = last_waiting >= 0 && (long)i < last_waiting;
        size_t now = 0;
        Cursor end;
        switch (job.fate(at, frame->index, budgets, cost, behind, now, end)) {
        case Fate::Passed: break;
        case Fate::Abandoned: job.abandoned = true; break;
        case Fate::Late: job.hand_out(now, cost, s->runs, spent); break;
        case Fate::Kept:
            job.hand_out(now, cost, s->runs, spent);
            at = end;
            break;
        }
    }
    // Deliver or report the jobs whose deadline arrives or that were abandoned.
    std::vector<Job> keep;
    for (Job &job : s->pending) {
        const bool reached = frame->index >= job.deadline;
        if (job.abandoned || reached) {
            if (!job.abandoned && job.complete() && frame->index == job.deadline)
                s->delivered.push_back(bls_delivery{job.id, job.input});
            else
                s->missed.push_back(bls_missed{job.id, job.input, job.deadline, s->miss, 0});
        } else {
            keep.push_back(std::move(job));
        }
    }
    s->pending.swap(keep);
    out->n_runs = (uint32_t)s->runs.size();
    out->n_delivered = (uint32_t)s->delivered.size();
    out->n_missed = (uint32_t)s->missed.size();
    out->reserved = 0;
    out->runs = s->runs.data();
    out->delivered = s->delivered.data();
    out->missed = s->missed.data();
    out->spent_estimate = spent;
    out->budget = budget;
    return BLS_OK;
}

extern "C" uint32_t bls_scheduler_pending(const bls_scheduler *s) { return (uint32_t)s->pending.size(); }

extern "C" int bls_scheduler_due(const bls_scheduler *s, uint64_t job, uint64_t *due) {
    for (const Job &j : s->pending)
        if (j.id == job) {
            *due = j.deadline;
            return BLS_OK;
        }
    return BLS_ERR_NO_SUCH_JOB;
}
