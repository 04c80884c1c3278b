// A frame's step as the host takes it, reading no clock: plan the frame (its
// budget from the render measured last, the forecast of the frames to come
// from the median of the recent renders, the input's admission, the plan),
// count what was submitted, take the timings that come back into the cost
// model, count the frame's deliveries and misses, and close the run into a
// tally. A C++ restatement of crates/beatlm-host/src/step.rs:78-540 and the
// rules it takes from frame.rs:89-283, behind include/beatlm_schedule.h.
//
// The reference holds a frame's order (plan, after_submit, complete) in its
// types; through a C ABI it is held at run time: a plan is refused while the
// frame planned before has not been counted, and after_submit and complete
// name the frame they act on.
#include "schedule.hpp"

#include <algorithm>

namespace bls {
namespace {

// RenderCost (frame.rs:89-158): the budget reads the render measured last,
// the forecast the upper median of the last RENDER_WINDOW.
struct RenderCost {
    uint64_t last = BLS_RENDER_PRIOR;
    std::deque<uint64_t> recent;

    void record(uint64_t render) {
        last = render;
        if (recent.size() == BLS_RENDER_WINDOW) recent.pop_front();
        recent.push_back(render);
    }
    uint64_t forecast() const {
        if (recent.empty()) return BLS_RENDER_PRIOR;
        std::vector<uint64_t> w(recent.begin(), recent.end());
        const size_t middle = w.size() / 2;
        std::nth_element(w.begin(), w.begin() + middle, w.end());
        return w[middle];
    }
    uint64_t budget(uint64_t period, uint64_t margin) const { return bls_budget_for_frame(period, last, margin); }
    uint64_t expected(uint64_t period, uint64_t margin) const {
        return bls_budget_for_frame(period, forecast(), margin);
    }
};

// Admission (frame.rs:190-238): under Free a frame takes an input only once
// the job submitted last has had every slice handed out or has left.
struct Admission {
    uint32_t submit = BLS_SUBMIT_EVERY;
    bool busy = false;
    uint64_t busy_job = 0;
    size_t left = 0;

    bool takes_input() const { return submit == BLS_SUBMIT_EVERY || !busy; }
    void planned(const std::optional<uint64_t> &job, size_t slices, const FramePlan &plan) {
        if (submit == BLS_SUBMIT_EVERY) return;
        if (job) {
            busy = true;
            busy_job = *job;
            left = slices;
        }
        if (!busy) return;
        size_t handed = 0;
        for (const bls_run &r : plan.runs) handed += r.job == busy_job;
        left = left > handed ? left - handed : 0;
        bool gone = false;
        for (const bls_delivery &d : plan.delivered) gone |= d.job == busy_job;
        for (const bls_missed &m : plan.missed) gone |= m.job == busy_job;
        if (left == 0 || gone) busy = false;
    }
};

struct Planned {
    bls_frame frame{};
    FramePlan plan;
    std::optional<uint64_t> job;
    std::optional<Due> due;
    uint64_t budget = 0, expected = 0;
};

}  // namespace

struct Step {
    Scheduler scheduler;
    bls_cost cost_handle;  // the cost model, as a handle bls_step_cost can return
    RenderCost render;
    std::vector<uint32_t> slices;
    uint64_t margin;
    std::optional<uint32_t> promised;  // the latency deliveries are held to
    Admission admission;
    std::map<uint64_t, uint64_t> job_dispatches;
    std::optional<Planned> unsubmitted;  // planned, not yet through after_submit
    std::deque<Planned> submitted;       // counted, not yet completed
    FramePlan completed;                 // the plan complete returned last
    bool finished = false;

    // Tally (step.rs:161-233).
    uint64_t n_submitted = 0, delivered = 0, missed = 0, startup_missed = 0, violations = 0, pending_at_end = 0;
    std::vector<uint64_t> latencies, dispatches_per_frame, dispatches_per_job, gpu_frame_us, longest_dispatch_us;
    std::map<uint32_t, std::pair<uint64_t, uint64_t>> measured;
    std::vector<bls_slice_measured> measured_out;
    std::vector<bls_slice_estimate> estimates;
    std::vector<double> frame_ratios, frame_scales;
    uint64_t timed_frames = 0;

    Step(const bls_step_config &c, const CostModel &m)
        : scheduler(c.policy, c.miss, bls_budget_for_frame(c.prior_period, BLS_RENDER_PRIOR, c.margin)),
          cost_handle{m},
          margin(c.margin) {
        for (uint32_t i = 0; i < c.slices; i++) slices.push_back(i);
        uint32_t d;
        if (bls_policy_source_delay(&c.policy, &d)) promised = d;
        admission.submit = c.submit;
    }
};

}  // namespace bls

struct bls_render_cost {
    bls::RenderCost r;
};
struct bls_step {
    bls::Step s;
};

using bls::Step;

extern "C" int bls_render_cost_new(bls_render_cost **out) {
    *out = new bls_render_cost{};
    return BLS_OK;
}
extern "C" void bls_render_cost_free(bls_render_cost *r) { delete r; }
extern "C" void bls_render_cost_record(bls_render_cost *r, uint64_t render) { r->r.record(render); }
extern "C" uint64_t bls_render_cost_last(const bls_render_cost *r) { return r->r.last; }
extern "C" uint64_t bls_render_cost_forecast(const bls_render_cost *r) { return r->r.forecast(); }
extern "C" uint64_t bls_render_cost_budget(const bls_render_cost *r, uint64_t period, uint64_t margin) {
    return r->r.budget(period, margin);
}
extern "C" uint64_t bls_render_cost_expected(const bls_render_cost *r, uint64_t period, uint64_t margin) {
    return r->r.expected(period, margin);
}

// timer_capacity / jobs_with_slices (frame.rs:264-283).
extern "C" int bls_timer_capacity(uint32_t slices, uint32_t jobs, uint32_t *out) {
    const uint64_t capacity = (uint64_t)slices * jobs;
    if (capacity > BLS_TIMER_MAX_SLICES) return 0;
    *out = (uint32_t)capacity;
    return 1;
}
extern "C" int bls_jobs_with_slices(uint32_t submit, uint32_t in_flight_kind, uint32_t in_flight, uint32_t *out) {
    if (submit == BLS_SUBMIT_FREE) {
        *out = 1;
        return 1;
    }
    if (in_flight_kind == BLS_IN_FLIGHT_BOUNDED) {
        *out = in_flight;
        return 1;
    }
    if (in_flight == UINT32_MAX) return 0;
    *out = in_flight + 1;
    return 1;
}

extern "C" int bls_step_new(const bls_step_config *c, const bls_cost *cost, bls_step **out) {
    if (!c || !cost || !out || c->miss > BLS_MISS_DROP || c->submit > BLS_SUBMIT_FREE) return BLS_ERR_INVALID;
    if (c->policy.kind > BLS_POLICY_ON_BEAT) return BLS_ERR_INVALID;
    if (c->policy.kind == BLS_POLICY_ON_BEAT && c->policy.grid_beat == 0) return BLS_ERR_ZERO_BEAT;
    *out = new bls_step{Step(*c, bls::model_of(cost))};
    return BLS_OK;
}
extern "C" void bls_step_free(bls_step *s) { delete s; }
extern "C" int bls_step_replace_beat_grid(bls_step *s, uint64_t from, uint64_t origin, uint64_t beat) {
    return s->s.scheduler.replace_beat_grid(from, bls::BeatGrid{origin, beat});
}

// The cost model as the next plan reads it; a handle the caller does not free.
extern "C" const bls_cost *bls_step_cost(const bls_step *s) { return &s->s.cost_handle; }
extern "C" uint64_t bls_step_submitted(const bls_step *s) { return s->s.n_submitted; }
extern "C" uint64_t bls_step_dispatched(const bls_step *s, uint64_t job) {
    auto it = s->s.job_dispatches.find(job);
    return it == s->s.job_dispatches.end() ? 0 : it->second;
}

// FrameStep::plan (step.rs:348-383).
extern "C" int bls_step_plan(bls_step *h, const bls_frame *frame, int owed, bls_planned *out, uint64_t *unsubmitted) {
    Step &s = h->s;
    if (s.finished) return BLS_ERR_FINISHED;
    if (!frame || !out) return BLS_ERR_INVALID;
    if (s.unsubmitted) {
        if (unsubmitted) *unsubmitted = s.unsubmitted->frame.index;
        return BLS_ERR_NOT_COUNTED;
    }
    bls::Planned p;
    p.frame = *frame;
    p.budget = s.render.budget(frame->period, s.margin);
    p.expected = s.render.expected(frame->period, s.margin);
    s.scheduler.set_expected_budget(p.expected);
    if (owed && s.admission.takes_input()) {
        uint64_t job = 0;
        const int rc = s.scheduler.submit(*frame, s.slices.data(), s.slices.size(), s.cost_handle.m, job);
        if (rc != BLS_OK) return rc;
        p.job = job;
        p.due = s.scheduler.due(job);  // read before the plan, which can deliver or miss the job
    }
    s.scheduler.plan_frame(*frame, p.budget, s.cost_handle.m, p.plan);
    s.unsubmitted = std::move(p);
    const bls::Planned &q = *s.unsubmitted;
    *out = bls_planned{};
    out->frame = q.frame;
    q.plan.expose(out->plan);
    out->has_job = q.job.has_value();
    out->job = q.job.value_or(0);
    out->has_due = q.due.has_value();
    if (q.due) out->due = bls_due{q.due->kind, 0, q.due->at};
    out->budget = q.budget;
    out->expected = q.expected;
    return BLS_OK;
}

extern "C" int bls_step_tag(const bls_step *s, uint32_t slice, uint64_t *planned) {
    const auto v = s->s.cost_handle.m.frame_estimate(slice);
    if (v && planned) *planned = *v;
    return v ? 1 : 0;
}

// FrameStep::after_submit (step.rs:401-425).
extern "C" int bls_step_after_submit(bls_step *h, uint64_t frame_index) {
    Step &s = h->s;
    if (s.finished) return BLS_ERR_FINISHED;
    if (!s.unsubmitted || s.unsubmitted->frame.index != frame_index) return BLS_ERR_NOT_PLANNED;
    const bls::Planned &p = *s.unsubmitted;
    s.dispatches_per_frame.push_back(p.plan.runs.size());
    const bls_frame_scale f = s.cost_handle.m.frame_scale();
    if (f.kind == BLS_SCALE_MEASURED) s.frame_scales.push_back(f.scale);
    if (p.job) s.n_submitted++;
    s.admission.planned(p.job, s.slices.size(), p.plan);
    for (const bls_run &r : p.plan.runs) s.job_dispatches[r.job]++;
    s.submitted.push_back(std::move(*s.unsubmitted));
    s.unsubmitted.reset();
    return BLS_OK;
}

// FrameStep::absorb (step.rs:430-470).
extern "C" int bls_step_absorb(bls_step *h, const bls_frame_timing *t, bls_absorbed *out) {
    Step &s = h->s;
    if (s.finished) return BLS_ERR_FINISHED;
    if (!t || (t->n_compute && !t->compute)) return BLS_ERR_INVALID;
    s.timed_frames++;
    uint64_t gpu = 0, predicted = 0, in_ratio = 0, longest = 0;
    for (uint32_t i = 0; i < t->n_compute; i++) {
        const bls_timed_slice &c = t->compute[i];
        s.cost_handle.m.record(c.slice, c.duration);
        auto &m = s.measured[c.slice];
        m.first = bls::sat_add(m.first, c.duration);
        m.second++;
        gpu = bls::sat_add(gpu, c.duration);
        if (c.has_planned) {
            predicted = bls::sat_add(predicted, c.planned);
            in_ratio = bls::sat_add(in_ratio, c.duration);
        }
        longest = std::max(longest, c.duration);
    }
    if (t->n_compute) {
        s.cost_handle.m.record_frame(predicted, in_ratio);
        if (predicted > 0) s.frame_ratios.push_back((double)in_ratio / (double)predicted);
        s.longest_dispatch_us.push_back(longest);
    }
    if (t->has_render) {
        s.render.record(t->render);
        s.gpu_frame_us.push_back(bls::sat_add(gpu, t->render));
    }
    if (out) *out = bls_absorbed{t->frame, t->has_render ? 1u : 0u, t->n_compute ? 1u : 0u, t->has_render ? t->render : 0};
    return BLS_OK;
}

// FrameStep::complete (step.rs:474-500).
extern "C" int bls_step_complete(bls_step *h, uint64_t frame_index, bls_frame_plan *out) {
    Step &s = h->s;
    if (s.finished) return BLS_ERR_FINISHED;
    auto it = std::find_if(s.submitted.begin(), s.submitted.end(),
                           [&](const bls::Planned &p) { return p.frame.index == frame_index; });
    if (it == s.submitted.end()) return BLS_ERR_NOT_PLANNED;
    const bls::FramePlan &plan = it->plan;
    for (const bls_delivery &d : plan.delivered) {
        const uint64_t latency = bls::sat_sub(frame_index, d.input);
        s.latencies.push_back(latency);
        s.delivered++;
        if (s.promised && latency != *s.promised) s.violations++;
        auto j = s.job_dispatches.find(d.job);
        s.dispatches_per_job.push_back(j == s.job_dispatches.end() ? 0 : j->second);
        if (j != s.job_dispatches.end()) s.job_dispatches.erase(j);
    }
    for (const bls_missed &m : plan.missed) {
        s.job_dispatches.erase(m.job);
        if (m.input < BLS_STARTUP_FRAMES) s.startup_missed++;
    }
    s.missed += plan.missed.size();
    s.completed = std::move(it->plan);
    s.submitted.erase(it);
    if (out) s.completed.expose(*out);
    return BLS_OK;
}

// FrameStep::finish (step.rs:504-516). The step takes no frame after it.
extern "C" int bls_step_finish(bls_step *h, bls_tally *out) {
    Step &s = h->s;
    if (!out) return BLS_ERR_INVALID;
    if (!s.finished) {
        s.finished = true;
        s.pending_at_end = s.scheduler.pending();
        for (uint32_t slice : s.slices) s.estimates.push_back(bls_slice_estimate{slice, 0, s.cost_handle.m.estimate(slice)});
        for (const auto &kv : s.measured) s.measured_out.push_back(bls_slice_measured{kv.first, 0, kv.second.first, kv.second.second});
    }
    *out = bls_tally{};
    out->submitted = s.n_submitted;
    out->delivered = s.delivered;
    out->missed = s.missed;
    out->startup_missed = s.startup_missed;
    out->violations = s.violations;
    out->pending_at_end = s.pending_at_end;
    out->n_latencies = s.latencies.size();
    out->latencies = s.latencies.data();
    out->n_dispatches_per_frame = s.dispatches_per_frame.size();
    out->dispatches_per_frame = s.dispatches_per_frame.data();
    out->n_dispatches_per_job = s.dispatches_per_job.size();
    out->dispatches_per_job = s.dispatches_per_job.data();
    out->n_gpu_frame_us = s.gpu_frame_us.size();
    out->gpu_frame_us = s.gpu_frame_us.data();
    out->n_longest_dispatch_us = s.longest_dispatch_us.size();
    out->longest_dispatch_us = s.longest_dispatch_us.data();
    out->n_measured = s.measured_out.size();
    out->measured = s.measured_out.data();
    out->n_estimates = s.estimates.size();
    out->estimates = s.estimates.data();
    out->n_frame_ratios = s.frame_ratios.size();
    out->frame_ratios = s.frame_ratios.data();
    out->n_frame_scales = s.frame_scales.size();
    out->frame_scales = s.frame_scales.data();
    out->frame_scale = s.cost_handle.m.frame_scale();
    out->frames_recorded = s.cost_handle.m.frames_recorded();
    out->timed_frames = s.timed_frames;
    return BLS_OK;
}
