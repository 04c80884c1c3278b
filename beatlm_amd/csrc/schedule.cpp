// Beats and the frame-budget slice scheduler: a C++ restatement of
// crates/beatlm-core/src/{time,sync,schedule}.rs behind
// include/beatlm_schedule.h. A job's deadline is fixed at submission by the
// sync policy: a frame (FixedLatency, SameFrame) or, OnBeat, the first beat
// at or after the job's projected finish plus the margin. Each plan spends the
// frame's budget on pending jobs in submission order; a job projected late is
// abandoned when a job waits behind it, kept to its deadline otherwise
// (schedule.rs:1-150).
#include "schedule.hpp"

#include <algorithm>

namespace bls {

// BeatGrid::next_beat_at_or_after (time.rs:171-183).
uint64_t BeatGrid::next_at_or_after(uint64_t t) const {
    if (t <= origin) return origin;
    const uint64_t into = (t - origin) % beat;
    return into == 0 ? t : sat_add(t, beat - into);
}

size_t BeatMap::in_effect(uint64_t t) const {
    size_t n = 0;  // grids whose `from` is at or before t
    while (n < grids_.size() && grids_[n].first <= t) n++;
    return n == 0 ? 0 : n - 1;
}

// BeatMap::replace_from (time.rs:213-216): later announcements are dropped.
void BeatMap::replace_from(uint64_t from, BeatGrid g) {
    grids_.erase(std::remove_if(grids_.begin(), grids_.end(), [&](const auto &e) { return e.first >= from; }),
                 grids_.end());
    grids_.emplace_back(from, g);
}

// BeatMap::next_beat_at_or_after (time.rs:226-246): a grid's beats exist only
// from its `from` to the next grid's; a beat past that hands over.
uint64_t BeatMap::next_at_or_after(uint64_t t) const {
    for (size_t i = in_effect(t); i < grids_.size(); i++) {
        const uint64_t beat = grids_[i].second.next_at_or_after(std::max(t, grids_[i].first));
        if (i + 1 < grids_.size() && beat >= grids_[i + 1].first) {
            t = grids_[i + 1].first;
            continue;
        }
        return beat;
    }
    return t;
}

// BeatMap::forget_before (time.rs:252-258).
void BeatMap::forget_before(uint64_t t) { grids_.erase(grids_.begin(), grids_.begin() + in_effect(t)); }

// Due::reached / on_time / frames_left (schedule.rs:212-252).
bool Due::reached(const bls_frame &f) const { return kind == BLS_DUE_FRAME ? f.index >= at : f.start >= at; }

bool Due::on_time(const bls_frame &f) const {
    if (kind == BLS_DUE_FRAME) return f.index == at;
    return f.start == at || (f.start > at && f.start - at < f.period);
}

std::optional<uint64_t> Due::frames_left(const bls_frame &f) const {
    if (kind == BLS_DUE_FRAME) {
        if (at < f.index) return std::nullopt;
        return at - f.index;
    }
    if (at <= f.start) return on_time(f) ? std::optional<uint64_t>(0) : std::nullopt;
    const uint64_t ahead = at - f.start;
    if (f.period == 0) return UINT64_MAX;
    return ahead / f.period + (ahead % f.period != 0);
}

void FramePlan::expose(bls_frame_plan &out) const {
    out.n_runs = (uint32_t)runs.size();
    out.n_delivered = (uint32_t)delivered.size();
    out.n_missed = (uint32_t)missed.size();
    out.reserved = 0;
    out.runs = runs.data();
    out.delivered = delivered.data();
    out.missed = missed.data();
    out.spent_estimate = spent;
    out.budget = budget;
}

namespace {

using Cursor = Scheduler::Cursor;
using Budgets = Scheduler::Budgets;
using Job = Scheduler::Job;

// When the work up to `c` is projected to finish, the frames from `planned`
// on following each other at its period (schedule.rs:336-344).
uint64_t instant(Cursor c, const bls_frame &planned) {
    return sat_add(sat_add(planned.start, sat_mul(c.frame, planned.period)), c.spent);
}

// Budgets::place (schedule.rs:381-406): slices in order onto frames from
// `at`; a frame takes slices while they fit, the first that does not opens
// the next frame. `fits` is false when a slice fits no empty frame after the
// planned one; `now` counts the slices that landed in the planned frame.
struct Placed {
    bool fits;
    Cursor end;
    size_t now;
};

Placed place(Budgets b, Cursor at, const uint32_t *slices, size_t n, const CostModel &cost) {
    size_t now = 0;
    for (size_t i = 0; i < n; i++) {
        const uint64_t estimate = cost.planning_estimate(slices[i]);
        for (;;) {
            const uint64_t after = sat_add(at.spent, estimate);
            if (after <= b.of(at.frame)) {
                at.spent = after;
                break;
            }
            if (at.frame > 0 && at.spent == 0) return Placed{false, at, now};
            at = Cursor{sat_add(at.frame, 1), 0};
        }
        if (at.frame == 0) now++;
    }
    return Placed{true, at, now};
}

enum class Fate { Passed, Abandoned, Late, Kept };

// Job::fate (schedule.rs:447-471): what the projection decides for `job` when
// the work kept ahead of it ends at `from`, and `behind` says whether a job
// waits behind it.
Fate fate(const Job &job, Cursor from, const bls_frame &frame, Budgets b, const CostModel &cost, bool behind,
          size_t &now, Cursor &end) {
    const auto left = job.deadline.frames_left(frame);
    if (!left) return Fate::Passed;
    now = 0;
    end = from;
    if (job.scheduled >= job.slices.size()) return Fate::Kept;
    const Placed p = place(b, from, job.slices.data() + job.scheduled, job.slices.size() - job.scheduled, cost);
    if (p.fits && p.end.frame <= *left) {
        now = p.now;
        end = p.end;
        return Fate::Kept;
    }
    if (behind) return Fate::Abandoned;
    now = p.now;
    return Fate::Late;
}

void hand_out(Job &job, size_t count, const CostModel &cost, FramePlan &plan) {
    for (size_t i = 0; i < count && job.scheduled < job.slices.size(); i++) {
        const uint32_t slice = job.slices[job.scheduled];
        plan.runs.push_back(bls_run{job.id, slice, (uint32_t)job.scheduled});
        plan.spent = sat_add(plan.spent, cost.planning_estimate(slice));
        job.scheduled++;
    }
}

BeatGrid grid_of(const bls_policy &p) { return BeatGrid{p.grid_origin, p.grid_beat ? p.grid_beat : 1}; }

}  // namespace

Scheduler::Scheduler(const bls_policy &policy, uint32_t miss, uint64_t expected)
    : on_beat_(policy.kind == BLS_POLICY_ON_BEAT),
      frames_(policy.kind == BLS_POLICY_FIXED_LATENCY ? policy.frames : 0),
      margin_(policy.kind == BLS_POLICY_ON_BEAT ? policy.margin : 0),
      beats_(grid_of(policy)),
      miss_(miss),
      expected_(expected) {}

int Scheduler::replace_beat_grid(uint64_t from, BeatGrid g) {
    if (!on_beat_) return BLS_ERR_NOT_ON_BEAT;
    if (g.beat == 0) return BLS_ERR_ZERO_BEAT;
    beats_.replace_from(from, g);
    return BLS_OK;
}

// Scheduler::projected_end (schedule.rs:671-678): every pending job is seen
// as the plan of the same frame sees it once the submitted job queues behind
// it, so a late one is abandoned and adds nothing.
Cursor Scheduler::projected_end(const bls_frame &frame, Budgets b, const CostModel &cost) const {
    Cursor at;
    for (const Job &job : pending_) {
        size_t now;
        Cursor end;
        if (fate(job, at, frame, b, cost, true, now, end) == Fate::Kept) at = end;
    }
    return at;
}

// Scheduler::submit (schedule.rs:618-665).
int Scheduler::submit(const bls_frame &input, const uint32_t *slices, size_t n, const CostModel &cost,
                      uint64_t &job_id) {
    if (n == 0) return BLS_ERR_EMPTY_JOB;
    Due deadline;
    if (!on_beat_) {
        deadline = Due{BLS_DUE_FRAME, sat_add(input.index, frames_)};
    } else {
        const Budgets b{expected_, expected_};
        const Placed p = place(b, projected_end(input, b, cost), slices, n, cost);
        uint64_t finish;
        if (p.fits) {
            finish = instant(p.end, input);
        } else {
            // No frame of the expected budget holds a slice: the earliest any
            // budget could make, the work back to back from the input.
            finish = input.start;
            for (size_t i = 0; i < n; i++) finish = sat_add(finish, cost.planning_estimate(slices[i]));
        }
        deadline = Due{BLS_DUE_BEAT, beats_.next_at_or_after(sat_add(finish, margin_))};
    }
    Job j;
    j.id = next_job_;
    next_job_ = sat_add(next_job_, 1);
    j.input = input.index;
    j.slices.assign(slices, slices + n);
    j.deadline = deadline;
    pending_.push_back(std::move(j));
    job_id = pending_.back().id;
    return BLS_OK;
}

// Scheduler::plan_frame (schedule.rs:706-769).
void Scheduler::plan_frame(const bls_frame &frame, uint64_t budget, const CostModel &cost, FramePlan &plan) {
    // Inputs are submitted in their frame, so no grid whose span ended before
    // this frame's start is read again.
    if (on_beat_) beats_.forget_before(frame.start);
    const Budgets b{budget, expected_};
    plan.runs.clear();
    plan.delivered.clear();
    plan.missed.clear();
    plan.spent = 0;
    plan.budget = budget;
    // A job waits behind another when it comes after it and this plan does
    // not report it missed for a deadline already behind the frame.
    long last_waiting = -1;
    for (long i = (long)pending_.size() - 1; i >= 0; i--)
        if (pending_[i].deadline.frames_left(frame)) {
            last_waiting = i;
            break;
        }
    Cursor at;
    for (size_t i = 0; i < pending_.size(); i++) {
        Job &job = pending_[i];
        size_t now = 0;
        Cursor end;
        switch (fate(job, at, frame, b, cost, (long)i < last_waiting, now, end)) {
        case Fate::Passed: break;
        case Fate::Abandoned: job.abandoned = true; break;
        case Fate::Late: hand_out(job, now, cost, plan); break;
        case Fate::Kept:
            hand_out(job, now, cost, plan);
            at = end;
            break;
        }
    }
    // Deliver or report the jobs whose deadline arrives or that were abandoned.
    std::vector<Job> keep;
    keep.reserve(pending_.size());
    for (Job &job : pending_) {
        if (!job.abandoned && !job.deadline.reached(frame)) {
            keep.push_back(std::move(job));
            continue;
        }
        if (!job.abandoned && job.scheduled >= job.slices.size() && job.deadline.on_time(frame))
            plan.delivered.push_back(bls_delivery{job.id, job.input});
        else
            plan.missed.push_back(bls_missed{job.id, job.input, bls_due{job.deadline.kind, 0, job.deadline.at}, miss_, 0});
    }
    pending_.swap(keep);
}

std::optional<Due> Scheduler::due(uint64_t job) const {
    auto it = std::lower_bound(pending_.begin(), pending_.end(), job, [](const Job &j, uint64_t id) { return j.id < id; });
    if (it == pending_.end() || it->id != job) return std::nullopt;
    return it->deadline;
}

}  // namespace bls

struct bls_scheduler {
    bls::Scheduler s;
    bls::FramePlan plan;
};

struct bls_beat_map {
    bls::BeatMap m;
};

namespace {
bool valid_policy(const bls_policy *p) {
    return p && (p->kind == BLS_POLICY_FIXED_LATENCY || p->kind == BLS_POLICY_SAME_FRAME || p->kind == BLS_POLICY_ON_BEAT);
}
}  // namespace

extern "C" int bls_beat_grid_next(uint64_t origin, uint64_t beat, uint64_t t, uint64_t *out) {
    if (beat == 0) return BLS_ERR_ZERO_BEAT;
    *out = bls::BeatGrid{origin, beat}.next_at_or_after(t);
    return BLS_OK;
}
extern "C" int bls_beat_map_new(uint64_t origin, uint64_t beat, bls_beat_map **out) {
    if (beat == 0) return BLS_ERR_ZERO_BEAT;
    *out = new bls_beat_map{bls::BeatMap(bls::BeatGrid{origin, beat})};
    return BLS_OK;
}
extern "C" void bls_beat_map_free(bls_beat_map *m) { delete m; }
extern "C" int bls_beat_map_replace_from(bls_beat_map *m, uint64_t from, uint64_t origin, uint64_t beat) {
    if (beat == 0) return BLS_ERR_ZERO_BEAT;
    m->m.replace_from(from, bls::BeatGrid{origin, beat});
    return BLS_OK;
}
extern "C" uint64_t bls_beat_map_next(const bls_beat_map *m, uint64_t t) { return m->m.next_at_or_after(t); }
extern "C" void bls_beat_map_forget_before(bls_beat_map *m, uint64_t t) { m->m.forget_before(t); }
extern "C" uint32_t bls_beat_map_grids(const bls_beat_map *m) { return (uint32_t)m->m.size(); }

// SyncPolicy::source_delay / max_in_flight (sync.rs).
extern "C" int bls_policy_source_delay(const bls_policy *p, uint32_t *out) {
    if (!valid_policy(p) || p->kind == BLS_POLICY_ON_BEAT) return 0;
    *out = p->kind == BLS_POLICY_FIXED_LATENCY ? p->frames : 0;
    return 1;
}
extern "C" int bls_policy_max_in_flight(const bls_policy *p, uint32_t *out) {
    if (!valid_policy(p) || p->kind == BLS_POLICY_ON_BEAT) return 0;
    *out = p->kind == BLS_POLICY_FIXED_LATENCY ? (p->frames == UINT32_MAX ? UINT32_MAX : p->frames + 1) : 1;
    return 1;
}

extern "C" int bls_scheduler_new_policy(const bls_policy *policy, uint32_t miss, uint64_t expected,
                                        bls_scheduler **out) {
    if (!valid_policy(policy) || miss > BLS_MISS_DROP || !out) return BLS_ERR_INVALID;
    if (policy->kind == BLS_POLICY_ON_BEAT && policy->grid_beat == 0) return BLS_ERR_ZERO_BEAT;
    *out = new bls_scheduler{bls::Scheduler(*policy, miss, expected), {}};
    return BLS_OK;
}
extern "C" int bls_scheduler_new(uint32_t latency_frames, uint32_t miss, uint64_t expected, bls_scheduler **out) {
    bls_policy p{};
    p.kind = BLS_POLICY_FIXED_LATENCY;
    p.frames = latency_frames;
    return bls_scheduler_new_policy(&p, miss, expected, out);
}
extern "C" void bls_scheduler_free(bls_scheduler *s) { delete s; }
extern "C" void bls_scheduler_set_expected_budget(bls_scheduler *s, uint64_t e) { s->s.set_expected_budget(e); }
extern "C" uint64_t bls_scheduler_expected_budget(const bls_scheduler *s) { return s->s.expected_budget(); }
extern "C" int bls_scheduler_replace_beat_grid(bls_scheduler *s, uint64_t from, uint64_t origin, uint64_t beat) {
    return s->s.replace_beat_grid(from, bls::BeatGrid{origin, beat});
}
extern "C" int bls_scheduler_submit(bls_scheduler *s, const bls_frame *input, const uint32_t *slices, uint32_t n,
                                    const bls_cost *cost, uint64_t *job_out) {
    if (!input || !cost || (n && !slices)) return BLS_ERR_INVALID;
    uint64_t job = 0;
    const int rc = s->s.submit(*input, slices, n, bls::model_of(cost), job);
    if (rc == BLS_OK && job_out) *job_out = job;
    return rc;
}
extern "C" int bls_scheduler_plan_frame(bls_scheduler *s, const bls_frame *frame, uint64_t budget, const bls_cost *cost,
                                        bls_frame_plan *out) {
    if (!frame || !cost || !out) return BLS_ERR_INVALID;
    s->s.plan_frame(*frame, budget, bls::model_of(cost), s->plan);
    s->plan.expose(*out);
    return BLS_OK;
}
extern "C" uint32_t bls_scheduler_pending(const bls_scheduler *s) { return (uint32_t)s->s.pending(); }
extern "C" int bls_scheduler_due(const bls_scheduler *s, uint64_t job, bls_due *out) {
    const auto d = s->s.due(job);
    if (!d) return BLS_ERR_NO_SUCH_JOB;
    if (out) *out = bls_due{d->kind, 0, d->at};
    return BLS_OK;
}
