// The cost model: measured slice durations read as the estimate the scheduler
// plans with. A C++ restatement of crates/beatlm-core/src/cost.rs behind
// include/beatlm_schedule.h, with its four estimators:
//   mean plus sigmas and capped deviation (exponentially weighted mean and
//   variance, cost.rs:487-514, 927-960), the windowed quantile (nearest rank
//   of the last `window` measurements, cost.rs:521-576) and the frame-scaled
//   median (loop median times a weighted quantile of recent frames' measured
//   over planned time, never below 1, cost.rs:590-720, 851-941).
#include "schedule.hpp"

#include <algorithm>
#include <cmath>

namespace bls {

// nearest_rank (cost.rs:666-679): ceil(q n), a product within 1e-9 of a whole
// number taken as that number, clamped to 1..=n.
size_t nearest_rank(double q, size_t n) {
    const double product = q * (double)n;
    const double nearest = std::round(product);
    const double rank = std::fabs(product - nearest) < 1e-9 ? nearest : std::ceil(product);
    const size_t r = rank <= 0.0 ? 0 : (size_t)rank;
    return std::min(std::max<size_t>(r, 1), std::max<size_t>(n, 1));
}

namespace {

// Rounds up to whole microseconds; NaN and negatives are zero, values at or
// above 2^64 saturate (cost.rs:1002-1012).
uint64_t micros_ceil(double v) {
    v = std::ceil(std::fmax(v, 0.0));
    return v >= 18446744073709551616.0 ? UINT64_MAX : (uint64_t)v;
}

// median * scale rounded up, a product within a billionth of itself of a
// whole number taken as that number (cost.rs:988-999).
uint64_t scaled_ceil(uint64_t median, double scale) {
    const double product = (double)median * scale;
    const double nearest = std::round(product);
    return micros_ceil(std::fabs(product - nearest) <= std::fabs(product) * 1e-9 ? nearest : product);
}

// The value at q's nearest rank among `values` (reordered in place).
uint64_t select_rank(std::vector<uint64_t> &values, double q) {
    const size_t rank = nearest_rank(q, values.size());
    std::nth_element(values.begin(), values.begin() + (rank - 1), values.end());
    return values[rank - 1];
}

bool unit_interval(double x) { return std::isfinite(x) && x > 0.0 && x <= 1.0; }
bool non_negative(double x) { return std::isfinite(x) && x >= 0.0; }
bool rank_in_range(double q) { return std::isfinite(q) && q >= 0.0 && q <= 1.0; }
bool window_in_range(uint32_t w) { return w >= 1 && w <= BLS_MAX_WINDOW; }

// Estimator::validate (cost.rs:433-485): the first parameter out of range.
int validate(const bls_estimator &e) {
    switch (e.kind) {
    case BLS_EST_MEAN_PLUS_SIGMAS:
        if (!unit_interval(e.alpha)) return BLS_ERR_INVALID_ALPHA;
        if (!non_negative(e.sigmas)) return BLS_ERR_INVALID_SIGMAS;
        return BLS_OK;
    case BLS_EST_WINDOWED_QUANTILE:
        if (!window_in_range(e.window)) return BLS_ERR_INVALID_WINDOW;
        if (!rank_in_range(e.quantile)) return BLS_ERR_INVALID_QUANTILE;
        return BLS_OK;
    case BLS_EST_FRAME_SCALED:
        if (!window_in_range(e.window)) return BLS_ERR_INVALID_WINDOW;
        if (!window_in_range(e.frame_window)) return BLS_ERR_INVALID_FRAME_WINDOW;
        if (!rank_in_range(e.quantile)) return BLS_ERR_INVALID_QUANTILE;
        return BLS_OK;
    case BLS_EST_CAPPED_DEVIATION:
        if (!unit_interval(e.alpha)) return BLS_ERR_INVALID_ALPHA;
        if (!non_negative(e.sigmas)) return BLS_ERR_INVALID_SIGMAS;
        if (!non_negative(e.cap)) return BLS_ERR_INVALID_CAP;
        return BLS_OK;
    default: return BLS_ERR_INVALID;
    }
}

// The weighted nearest rank of q among (ratio, weight) sorted by ratio: the
// first ratio at which the cumulative weight reaches q of the total, less the
// rounding tolerance nearest_rank allows (cost.rs:646-660).
double weighted_rank(const std::vector<std::pair<double, double>> &sorted, double q) {
    double total = 0.0;
    for (const auto &r : sorted) total += r.second;
    const double target = std::fma(q, total, -(total * 1e-9));
    double reached = 0.0;
    for (const auto &r : sorted) {
        reached += r.second;
        if (reached >= target) return r.first;
    }
    return sorted.empty() ? 1.0 : sorted.back().first;
}

}  // namespace

void Window::fold(uint64_t x, size_t capacity, double q, std::optional<double> second_q) {
    if (ring.size() < capacity) ring.push_back(x);
    else ring[next] = x;
    next = (next + 1) % capacity;
    if (samples < UINT32_MAX) samples++;
    std::vector<uint64_t> scratch(ring);
    estimate = select_rank(scratch, q);
    second = second_q ? select_rank(scratch, *second_q) : estimate;
}

int CostModel::make(uint64_t prior, const bls_estimator &e, CostModel &out) {
    const int rc = validate(e);
    if (rc != BLS_OK) return rc;
    out = CostModel();
    out.prior_ = prior;
    out.est_ = e;
    out.est_.reserved = 0;
    if (e.kind == BLS_EST_FRAME_SCALED) out.frames_.reserve(e.frame_window);
    return BLS_OK;
}

const SliceStats *CostModel::find(uint32_t slice) const {
    auto it = stats_.find(slice);
    return it == stats_.end() ? nullptr : &it->second;
}

// CostModel::fold (cost.rs:796-842).
void CostModel::fold(uint32_t slice, uint64_t measured, bool in_loop) {
    SliceStats &s = stats_[slice];
    switch (est_.kind) {
    case BLS_EST_MEAN_PLUS_SIGMAS:
    case BLS_EST_CAPPED_DEVIATION: {
        const double x = (double)measured;
        if (s.ewma_samples == 0) {
            s.mean = x;
            s.var = 0.0;
            s.ewma_samples = 1;
        } else {
            const double diff = x - s.mean;
            const double incr = est_.alpha * diff;
            s.mean += incr;
            s.var = (1.0 - est_.alpha) * (s.var + diff * incr);
            if (s.ewma_samples < UINT32_MAX) s.ewma_samples++;
        }
        break;
    }
    case BLS_EST_WINDOWED_QUANTILE:
        s.all.fold(measured, est_.window, est_.quantile, std::nullopt);
        break;
    case BLS_EST_FRAME_SCALED:
        s.all.fold(measured, est_.window, est_.quantile, 0.5);
        if (in_loop) s.looped.fold(measured, est_.window, 0.5, std::nullopt);
        break;
    }
}

// CostModel::estimate (cost.rs:944-964).
uint64_t CostModel::estimate(uint32_t slice) const {
    const SliceStats *s = find(slice);
    if (!s) return prior_;
    switch (est_.kind) {
    case BLS_EST_MEAN_PLUS_SIGMAS:
        return micros_ceil(std::fma(est_.sigmas, std::sqrt(std::fmax(s->var, 0.0)), s->mean));
    case BLS_EST_CAPPED_DEVIATION: {
        const double padding =
            std::fmin(est_.sigmas * std::sqrt(std::fmax(s->var, 0.0)), est_.cap * std::fmax(s->mean, 0.0));
        return micros_ceil(s->mean + padding);
    }
    case BLS_EST_WINDOWED_QUANTILE: return s->all.estimate;
    case BLS_EST_FRAME_SCALED: return s->warm() ? s->looped.estimate : s->all.second;
    }
    return prior_;
}

// CostModel::planning_estimate (cost.rs:927-941): only the frame-scaled
// estimator plans away from its estimate.
uint64_t CostModel::planning_estimate(uint32_t slice) const {
    const SliceStats *s = find(slice);
    if (!s || est_.kind != BLS_EST_FRAME_SCALED) return estimate(slice);
    const bls_frame_scale f = frame_scale();
    if (f.kind == BLS_SCALE_MEASURED && s->warm()) return scaled_ceil(s->looped.estimate, f.scale);
    return s->all.estimate;
}

uint32_t CostModel::samples(uint32_t slice) const {
    const SliceStats *s = find(slice);
    if (!s) return 0;
    switch (est_.kind) {
    case BLS_EST_MEAN_PLUS_SIGMAS:
    case BLS_EST_CAPPED_DEVIATION: return s->ewma_samples;
    default: return s->all.samples;
    }
}

// CostModel::frame_estimate (cost.rs:851-858).
std::optional<uint64_t> CostModel::frame_estimate(uint32_t slice) const {
    if (est_.kind != BLS_EST_FRAME_SCALED) return estimate(slice);
    const SliceStats *s = find(slice);
    if (s && s->warm()) return s->looped.estimate;
    return std::nullopt;
}

// CostModel::record_frame (cost.rs:871-893) and Frames::fold (cost.rs:609-627).
void CostModel::record_frame(uint64_t predicted, uint64_t measured) {
    if (est_.kind != BLS_EST_FRAME_SCALED || predicted == 0) return;
    const double weight = (double)predicted;
    const std::pair<double, double> frame{(double)measured / weight, weight};
    const size_t capacity = est_.frame_window;
    if (frames_.size() < capacity) frames_.push_back(frame);
    else frames_[frames_next_] = frame;
    frames_next_ = (frames_next_ + 1) % capacity;
    if (frames_recorded_ < UINT64_MAX) frames_recorded_++;
    if (frames_.size() < capacity) return;  // the scale is read only from a full window
    std::vector<std::pair<double, double>> sorted(frames_);
    std::sort(sorted.begin(), sorted.end(), [](const auto &a, const auto &b) { return a.first < b.first; });
    scale_ = std::fmax(weighted_rank(sorted, est_.quantile), 1.0);
}

bls_frame_scale CostModel::frame_scale() const {
    bls_frame_scale f{};
    if (est_.kind != BLS_EST_FRAME_SCALED) return f;
    if (frames_.size() < est_.frame_window) {
        f.kind = BLS_SCALE_WARMING_UP;
        f.recorded = frames_.size();
        f.needed = est_.frame_window;
    } else {
        f.kind = BLS_SCALE_MEASURED;
        f.scale = scale_;
    }
    return f;
}

}  // namespace bls

extern "C" uint32_t bls_nearest_rank(double quantile, uint32_t n) { return (uint32_t)bls::nearest_rank(quantile, n); }

extern "C" uint64_t bls_budget_for_frame(uint64_t period, uint64_t render, uint64_t margin) {
    return bls::sat_sub(bls::sat_sub(period, render), margin);
}

extern "C" int bls_cost_new_with(uint64_t prior, const bls_estimator *e, bls_cost **out) {
    if (!e || !out) return BLS_ERR_INVALID;
    bls::CostModel m;
    const int rc = bls::CostModel::make(prior, *e, m);
    if (rc != BLS_OK) return rc;
    *out = new bls_cost{std::move(m)};
    return BLS_OK;
}

extern "C" int bls_cost_new(uint64_t prior, uint32_t window, double quantile, bls_cost **out) {
    bls_estimator e{};
    e.kind = BLS_EST_WINDOWED_QUANTILE;
    e.window = window;
    e.quantile = quantile;
    return bls_cost_new_with(prior, &e, out);
}

extern "C" int bls_cost_clone(const bls_cost *c, bls_cost **out) {
    if (!c || !out) return BLS_ERR_INVALID;
    *out = new bls_cost{c->m};
    return BLS_OK;
}
extern "C" void bls_cost_free(bls_cost *c) { delete c; }
extern "C" void bls_cost_estimator(const bls_cost *c, bls_estimator *out) { *out = c->m.estimator(); }
extern "C" void bls_cost_record(bls_cost *c, uint32_t slice, uint64_t measured) { c->m.record(slice, measured); }
extern "C" void bls_cost_record_calibration(bls_cost *c, uint32_t slice, uint64_t measured) {
    c->m.record_calibration(slice, measured);
}
extern "C" uint64_t bls_cost_estimate(const bls_cost *c, uint32_t slice) { return c->m.estimate(slice); }
extern "C" uint64_t bls_cost_planning_estimate(const bls_cost *c, uint32_t slice) {
    return c->m.planning_estimate(slice);
}
extern "C" uint32_t bls_cost_samples(const bls_cost *c, uint32_t slice) { return c->m.samples(slice); }
extern "C" int bls_cost_frame_estimate(const bls_cost *c, uint32_t slice, uint64_t *out) {
    const auto v = c->m.frame_estimate(slice);
    if (v && out) *out = *v;
    return v ? 1 : 0;
}
extern "C" void bls_cost_record_frame(bls_cost *c, uint64_t predicted, uint64_t measured) {
    c->m.record_frame(predicted, measured);
}
extern "C" void bls_cost_frame_scale(const bls_cost *c, bls_frame_scale *out) { *out = c->m.frame_scale(); }
extern "C" uint64_t bls_cost_frames_recorded(const bls_cost *c) { return c->m.frames_recorded(); }
