"""The rest of the scheduler's caller restated in C++ (beatlm_amd/csrc/
{cost,schedule,step}.cpp): the four cost estimators, beat grids and maps, the
OnBeat and SameFrame policies, the host's render cost and frame step. Each
case is one of the reference's own tests, with its numbers:
crates/beatlm-core/src/cost.rs:1014-1380, time.rs (tests), sync.rs (tests),
schedule.rs:787-1640, crates/beatlm-host/src/frame.rs (tests) and
step.rs (tests). CPU only.
"""

import math

import pytest

from beatlm_amd import schedule as S

E = S.Estimator
SL = 0  # the slice most cases measure


def mean_sigmas(prior, alpha, sigmas):
    return S.CostModel(prior, estimator=E.mean_plus_sigmas(alpha, sigmas))


def quantile(prior, window, q):
    return S.CostModel(prior, estimator=E.windowed_quantile(window, q))


def capped(prior, alpha, sigmas, cap):
    return S.CostModel(prior, estimator=E.capped_deviation(alpha, sigmas, cap))


def frame_scaled(prior, window, frame_window, q):
    return S.CostModel(prior, estimator=E.frame_scaled(window, frame_window, q))


def rejected(est):
    with pytest.raises(S.ScheduleError) as e:
        S.CostModel(0, estimator=est)
    return e.value.code


# ---- cost model (cost.rs tests) ---------------------------------------------------


def test_invalid_alpha_sigmas_and_cap_are_rejected():
    for alpha in (0.0, -0.5, 1.5, math.nan, math.inf):
        assert rejected(E.mean_plus_sigmas(alpha, 1.0)) == S.ERR_INVALID_ALPHA
        assert rejected(E.capped_deviation(alpha, 1.0, 1.0)) == S.ERR_INVALID_ALPHA
    for sigmas in (-0.1, math.nan, math.inf):
        assert rejected(E.mean_plus_sigmas(0.5, sigmas)) == S.ERR_INVALID_SIGMAS
        assert rejected(E.capped_deviation(0.5, sigmas, 1.0)) == S.ERR_INVALID_SIGMAS
    for cap in (-0.1, math.nan, math.inf):
        assert rejected(E.capped_deviation(0.5, 1.0, cap)) == S.ERR_INVALID_CAP


def test_invalid_frame_scaled_parameters_are_rejected():
    for window in (0, S.MAX_WINDOW + 1):
        assert rejected(E.frame_scaled(window, 8, 0.9)) == S.ERR_INVALID_WINDOW
    for fw in (0, S.MAX_WINDOW + 1):
        assert rejected(E.frame_scaled(8, fw, 0.9)) == S.ERR_INVALID_FRAME_WINDOW
    for q in (-0.1, 1.1, math.nan, math.inf):
        assert rejected(E.frame_scaled(8, 8, q)) == S.ERR_INVALID_QUANTILE
    for w, fw, q in ((1, 1, 0.0), (S.MAX_WINDOW, S.MAX_WINDOW, 1.0)):
        frame_scaled(0, w, fw, q)


def test_prior_is_used_without_samples_by_every_estimator():
    for m in (mean_sigmas(123, 0.5, 2.0), quantile(123, 8, 0.9), capped(123, 0.5, 2.0, 0.5),
              frame_scaled(123, 8, 4, 0.9)):
        assert m.estimate(SL) == 123 and m.samples(SL) == 0
        m.record(1, 5)
        assert m.estimate(SL) == 123


def test_the_model_reports_its_estimator():
    e = E.windowed_quantile(4, 0.5)
    assert S.CostModel(0, estimator=e).estimator() == e


def test_alpha_one_tracks_the_last_sample():
    m = mean_sigmas(1, 1.0, 3.0)
    for x in (100, 400, 250):
        m.record(SL, x)
    assert m.estimate(SL) == 250


def test_estimate_pads_the_mean_by_sigmas():
    m = mean_sigmas(1, 0.5, 2.0)
    m.record(SL, 100)
    assert m.estimate(SL) == 100
    m.record(SL, 120)
    m.record(SL, 80)
    # mean 95, var 275: ceil(95 + 2 sqrt(275)) = 129.
    assert m.estimate(SL) == 129


def test_samples_count_per_slice_for_every_estimator():
    for m in (mean_sigmas(1, 0.5, 0.0), quantile(1, 3, 0.5), capped(1, 0.5, 0.0, 0.0), frame_scaled(1, 3, 2, 0.5)):
        m.record(SL, 10)
        m.record(SL, 10)
        m.record(8, 10)
        assert (m.samples(SL), m.samples(8), m.samples(9)) == (2, 1, 0)


def test_huge_estimates_saturate():
    top = 2**64 - 1
    for m in (mean_sigmas(0, 1.0, 0.0), capped(0, 1.0, 0.0, 0.0), quantile(0, 2, 1.0)):
        m.record(SL, top)
        assert m.estimate(SL) == top


def test_capped_pads_by_the_smaller_of_sigmas_and_the_cap():
    for cap, want in ((1.0, 129), (0.1, 105), (0.0, 95)):
        m = capped(1, 0.5, 2.0, cap)
        for x in (100, 120, 80):
            m.record(SL, x)
        assert m.estimate(SL) == want, cap


def test_estimates_change_only_through_record_and_clones_agree():
    for m in (mean_sigmas(1, 0.2, 2.0), quantile(1, 8, 0.9), capped(1, 0.2, 2.0, 0.5)):
        m.record(SL, 100)
        m.record(SL, 300)
        before = m.estimate(SL)
        assert m.estimate(SL) == before and m.clone().estimate(SL) == before


def test_identical_measurements_give_identical_estimates():
    for e in (E.mean_plus_sigmas(0.2, 2.0), E.windowed_quantile(6, 0.9), E.capped_deviation(0.2, 2.0, 0.5)):
        a, b = S.CostModel(9, estimator=e), S.CostModel(9, estimator=e)
        for i in range(40):
            x = 100 + (i * 37) % 11 * 13
            a.record(SL, x)
            b.record(SL, x)
            assert a.estimate(SL) == b.estimate(SL)


def _peak(m):
    peak = 0
    for i in range(200):
        m.record(SL, 8_000 if i % 10 == 9 else 1_000 + (i % 5) * 10)
        if i >= 30:
            peak = max(peak, m.estimate(SL))
    return peak


def test_noise_inflates_mean_plus_sigmas_but_not_the_robust_estimators():
    inflated = _peak(mean_sigmas(1, 0.05, 2.0))
    windowed = _peak(quantile(1, 20, 0.9))
    bounded = _peak(capped(1, 0.05, 2.0, 0.5))
    assert windowed <= 1_040 and bounded <= 3_000 and inflated >= 6_000
    assert windowed < bounded < inflated


def frames(m, pairs):
    for predicted, measured in pairs:
        m.record_frame(predicted, measured)


def test_frame_scaled_estimates_the_median_and_warms_up_at_the_frame_quantile():
    m = frame_scaled(123, 8, 3, 0.9)
    assert m.estimate(SL) == 123 and m.planning_estimate(SL) == 123
    for x in (50, 10, 40, 20, 30):
        m.record(SL, x)
    assert m.estimate(SL) == 30
    assert m.frame_scale() == S.FrameScale(S.SCALE_WARMING_UP, recorded=0, needed=3)
    assert m.planning_estimate(SL) == 50
    frames(m, [(100, 150), (100, 150)])
    assert m.frame_scale() == S.FrameScale(S.SCALE_WARMING_UP, recorded=2, needed=3)
    assert m.planning_estimate(SL) == 50
    frames(m, [(100, 150)])
    assert m.frame_scale() == S.FrameScale(S.SCALE_MEASURED, scale=1.5)
    assert m.planning_estimate(SL) == 45 and m.estimate(SL) == 30
    assert m.planning_estimate(1) == 123
    assert m.frames_recorded() == 3


def test_the_frame_scale_is_the_nearest_rank_of_the_last_frames():
    m = frame_scaled(1, 4, 4, 0.75)
    frames(m, [(100, 150), (100, 120), (100, 200), (100, 110)])
    assert m.frame_scale().scale == 1.5
    frames(m, [(100, 130)])
    assert m.frame_scale().scale == 1.3
    for q, want in ((0.0, 1.1), (1.0, 2.0)):
        m = frame_scaled(1, 4, 4, q)
        frames(m, [(100, 150), (100, 120), (100, 200), (100, 110)])
        assert m.frame_scale().scale == want, q
    m = frame_scaled(1, 4, 100, 0.55)
    frames(m, [(100, 100 + i) for i in range(1, 101)])
    assert m.frame_scale().scale == 1.55


def test_the_planning_estimate_is_the_median_times_the_scale_rounded_up():
    m = frame_scaled(1, 5, 1, 1.0)
    for _ in range(5):
        m.record(SL, 101)
    frames(m, [(1_000, 1_234)])
    assert m.planning_estimate(SL) == 125 >= m.estimate(SL)
    m = frame_scaled(1, 5, 1, 1.0)
    for _ in range(5):
        m.record(SL, 100)
    frames(m, [(1_000, 1_100)])
    assert m.planning_estimate(SL) == 110


def test_the_frame_scale_never_plans_a_slice_below_its_median():
    m = frame_scaled(1, 8, 4, 0.9)
    for _ in range(5):
        m.record(SL, 200)
    frames(m, [(400, 200)] * 4)
    assert m.frame_scale().scale == 1.0
    assert m.planning_estimate(SL) == m.estimate(SL) == 200


def test_a_frame_counts_as_much_as_its_predicted_time():
    m = frame_scaled(1, 4, 25, 0.9)
    frames(m, [(4_000, 4_800)] * 20 + [(20, 200)] * 5)
    assert m.frame_scale().scale == 1.2 and m.frames_recorded() == 25
    u = frame_scaled(1, 4, 25, 0.9)
    frames(u, [(100, 120)] * 20 + [(100, 1_000)] * 5)
    assert u.frame_scale().scale == 10.0


def test_a_frame_predicted_at_zero_is_not_recorded():
    m = frame_scaled(1, 4, 2, 0.9)
    frames(m, [(0, 500), (0, 0)])
    assert m.frames_recorded() == 0
    assert m.frame_scale() == S.FrameScale(S.SCALE_WARMING_UP, recorded=0, needed=2)
    frames(m, [(100, 0), (100, 0)])
    assert m.frame_scale() == S.FrameScale(S.SCALE_MEASURED, scale=1.0)


def test_the_other_estimators_ignore_frames_and_plan_at_their_estimate():
    for m in (mean_sigmas(1, 0.2, 2.0), quantile(1, 8, 0.9), capped(1, 0.2, 2.0, 0.5)):
        for x in (100, 300, 200, 900):
            m.record(SL, x)
        before = m.estimate(SL)
        frames(m, [(100, 300)] * 50)
        assert m.frame_scale() == S.FrameScale(S.SCALE_NONE) and m.frames_recorded() == 0
        assert m.estimate(SL) == before == m.planning_estimate(SL)
        assert m.planning_estimate(1) == 1


def test_calibration_does_not_seed_the_frame_scaled_median():
    m = frame_scaled(1, 32, 1, 0.9)
    for _ in range(20):
        m.record_calibration(SL, 100)
    assert m.samples(SL) == 20 and m.frame_estimate(SL) is None
    assert m.planning_estimate(SL) == 100 == m.estimate(SL)
    m.record_frame(100, 150)
    assert m.frame_scale().scale == 1.5
    for _ in range(4):
        m.record(SL, 300)
    assert m.frame_estimate(SL) is None and m.planning_estimate(SL) == 300
    m.record(SL, 300)
    assert m.frame_estimate(SL) == 300 == m.estimate(SL)
    assert m.planning_estimate(SL) == 450 and m.samples(SL) == 25


def test_the_frame_scale_reads_warm_slices_and_not_stale_ones():
    a, b = 1, 2
    m = frame_scaled(1, 32, 8, 0.9)
    for _ in range(S.WARM_SAMPLES):
        m.record(a, 100)
    for _ in range(10):
        m.record_calibration(b, 50)
    m.record(b, 200)
    m.record(b, 200)
    for _ in range(8):
        predicted = measured = 0
        for sl, took in ((a, 100), (b, 200)):
            planned = m.frame_estimate(sl)
            if planned is not None:
                predicted += planned
                measured += took
        m.record_frame(predicted, measured)
    assert m.frame_scale().scale == 1.0
    assert m.planning_estimate(a) == 100 and m.estimate(b) == 50


def test_the_other_estimators_fold_calibration_as_the_loop():
    for e in (E.mean_plus_sigmas(0.2, 2.0), E.windowed_quantile(6, 0.9), E.capped_deviation(0.2, 2.0, 0.5)):
        by_record, by_cal = S.CostModel(9, estimator=e), S.CostModel(9, estimator=e)
        for i in range(40):
            x = 100 + (i * 37) % 11 * 13
            by_record.record(SL, x)
            (by_cal.record_calibration if i < 20 else by_cal.record)(SL, x)
            assert by_record.estimate(SL) == by_cal.estimate(SL)
            assert by_cal.frame_estimate(SL) == by_cal.estimate(SL)
        assert by_record.samples(SL) == by_cal.samples(SL)
        assert by_cal.frame_estimate(3) == 9
    assert frame_scaled(9, 4, 4, 0.9).frame_estimate(SL) is None


def test_frame_scaled_is_deterministic_and_changes_only_through_records():
    e = E.frame_scaled(6, 5, 0.9)
    a, b = S.CostModel(9, estimator=e), S.CostModel(9, estimator=e)
    for i in range(40):
        x = 100 + (i * 37) % 11 * 13
        measured = 1_000 + (i * 53) % 17 * 31
        for m in (a, b):
            m.record(SL, x)
            m.record_frame(1_000, measured)
        assert (a.estimate(SL), a.planning_estimate(SL), a.frame_scale()) == (
            b.estimate(SL), b.planning_estimate(SL), b.frame_scale())
        assert a.clone().planning_estimate(SL) == a.planning_estimate(SL)


# ---- beats (time.rs tests) ----------------------------------------------------------


def test_beat_grid():
    with pytest.raises(S.ScheduleError) as e:
        S.beat_grid_next(0, 0, 5)
    assert e.value.code == S.ERR_ZERO_BEAT
    assert S.beat_grid_next(1_000, 500, 10) == 1_000
    assert S.beat_grid_next(1_000, 500, 1_000) == 1_000
    assert S.beat_grid_next(1_000, 500, 2_500) == 2_500
    assert S.beat_grid_next(1_000, 500, 1_001) == 1_500
    assert S.beat_grid_next(1_000, 500, 1_999) == 2_000
    assert S.beat_grid_next(0, 1_000, 2**64 - 2) == 2**64 - 1


def changed():
    m = S.BeatMap(0, 1_000)
    m.replace_from(2_500, 2_600, 300)
    return m


def test_beat_map_uses_the_old_grid_before_the_change_and_the_new_one_after():
    m = changed()
    assert m.next_beat_at_or_after(1_200) == 2_000
    assert m.next_beat_at_or_after(2_700) == 2_900
    # The old grid's beat at 3000 lies past the change: the new grid's 2600.
    assert m.next_beat_at_or_after(2_100) == 2_600


def test_replacing_drops_the_grids_announced_at_or_after_it():
    m = changed()
    m.replace_from(2_000, 0, 250)
    assert m.next_beat_at_or_after(2_700) == 2_750
    assert m.next_beat_at_or_after(1_500) == 2_000


def test_forgetting_keeps_every_beat_from_then_on():
    m = changed()
    before = [m.next_beat_at_or_after(t) for t in range(2_500, 4_000, 7)]
    m.forget_before(2_500)
    assert m.grids() == 1
    assert [m.next_beat_at_or_after(t) for t in range(2_500, 4_000, 7)] == before
    assert m.next_beat_at_or_after(1_200) == 2_600
    m = changed()
    m.forget_before(2_499)
    assert m.grids() == 2


# ---- sync policies (sync.rs tests) -------------------------------------------------


def on_beat(margin, beat=1_000):
    return S.Policy.on_beat(0, beat, margin)


def test_source_delay_and_max_in_flight_follow_the_policy():
    assert S.Policy.fixed_latency(3).source_delay() == 3
    assert S.Policy.same_frame().source_delay() == 0
    assert on_beat(0, 500_000).source_delay() is None
    assert S.Policy.fixed_latency(0).max_in_flight() == 1
    assert S.Policy.fixed_latency(2).max_in_flight() == 3
    assert S.Policy.fixed_latency(2**32 - 1).max_in_flight() == 2**32 - 1
    assert S.Policy.same_frame().max_in_flight() == 1
    assert on_beat(0, 500_000).max_in_flight() is None


# ---- scheduler: SameFrame and OnBeat (schedule.rs tests) ---------------------------

PERIOD = 1_000


def frame(i):
    return S.frame(i, PERIOD)


def at(start):
    return S.Frame(start // PERIOD, start, PERIOD)


def cost():
    """Every unmeasured slice costs 100 µs; a measured one its last measurement."""
    return mean_sigmas(100, 1.0, 0.0)


def beat(t):
    return S.Due.beat(t)


def test_replacing_beats_needs_an_on_beat_scheduler():
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_DROP, 100)
    with pytest.raises(S.ScheduleError) as e:
        s.replace_beat_grid(0, 0, 1_000)
    assert e.value.code == S.ERR_NOT_ON_BEAT
    S.Scheduler(on_beat(0), S.MISS_DROP, 100).replace_beat_grid(0, 0, 1_000)


def test_a_missed_job_does_not_hold_up_the_jobs_after_it():
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_DROP, 100)
    c = cost()
    a = s.submit(frame(0), [0, 1], c)
    b = s.submit(frame(1), [0], c)
    p = s.plan_frame(frame(1), 1_000, c)
    assert [r.job for r in p.runs] == [b]
    assert [m.job for m in p.missed] == [a] and [d.job for d in p.delivered] == [b]


def test_equal_deadlines_go_to_the_lower_job_id():
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_DROP, 100)
    c = cost()
    first = s.submit(frame(0), [0], c)
    s.submit(frame(0), [0], c)
    p = s.plan_frame(frame(0), 100, c)
    assert [r.job for r in p.runs] == [first] and len(p.delivered) == 1 and len(p.missed) == 1


def test_same_frame_fitting_job_is_delivered_in_the_same_plan():
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_HOLD_PREVIOUS, 200)
    c = cost()
    job = s.submit(frame(4), [0, 1], c)
    p = s.plan_frame(frame(4), 200, c)
    assert len(p.runs) == 2 and p.delivered == [S.Delivery(job, 4)] and not p.missed and s.pending() == 0


def test_same_frame_oversized_job_is_missed_in_the_same_plan():
    c = cost()
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_DROP, 150)
    job = s.submit(frame(4), [0, 1], c)
    p = s.plan_frame(frame(4), 150, c)
    assert len(p.runs) == 1 and p.spent_estimate == 100 and not p.delivered
    missed = S.Missed(job, 4, S.Due.frame(4), S.MISS_DROP)
    assert p.missed == [missed] and s.pending() == 0
    s = S.Scheduler(S.Policy.same_frame(), S.MISS_DROP, 150)
    job = s.submit(frame(4), [0, 1], c)
    nxt = s.submit(frame(4), [2], c)
    p = s.plan_frame(frame(4), 150, c)
    assert [r.job for r in p.runs] == [nxt] and p.missed == [missed] and len(p.delivered) == 1


def test_on_beat_deadline_follows_the_grid():
    c = cost()
    s = S.Scheduler(on_beat(50), S.MISS_DROP, 1_000)
    job = s.submit(at(250), [0, 1], c)
    assert s.due(job) == beat(1_000)
    assert len(s.plan_frame(at(250), 1_000, c).runs) == 2
    for start in (500, 750, 999):
        p = s.plan_frame(at(start), 1_000, c)
        assert not p.delivered and not p.missed, start
    assert s.pending() == 1
    assert s.plan_frame(at(1_000), 1_000, c).delivered == [S.Delivery(job, 0)]
    assert s.pending() == 0


def test_on_beat_skips_to_the_next_beat_when_work_does_not_fit_before_it():
    c = cost()
    s = S.Scheduler(on_beat(50), S.MISS_DROP, 1_000)
    job = s.submit(at(900), [0], c)
    s.plan_frame(at(900), 1_000, c)
    for start in (1_000, 1_999):
        p = s.plan_frame(at(start), 1_000, c)
        assert not p.delivered and not p.missed
    assert [d.job for d in s.plan_frame(at(2_000), 1_000, c).delivered] == [job]


def test_on_beat_multi_frame_job_gets_a_beat_it_can_make():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_DROP, 100)
    job = s.submit(frame(0), [0, 1, 2], c)
    assert s.due(job) == beat(3_000)
    for f in range(3):
        p = s.plan_frame(frame(f), 100, c)
        assert len(p.runs) == 1 and not p.delivered and not p.missed, f
    p = s.plan_frame(frame(3), 100, c)
    assert [d.job for d in p.delivered] == [job] and not p.missed


def test_on_beat_work_queued_ahead_pushes_the_beat_later():
    c = cost()
    alone = S.Scheduler(on_beat(0), S.MISS_DROP, 100)
    assert alone.due(alone.submit(frame(0), [3], c)) == beat(1_000)
    s = S.Scheduler(on_beat(0), S.MISS_DROP, 100)
    a = s.submit(frame(0), [0, 1, 2], c)
    b = s.submit(frame(0), [3], c)
    assert (s.due(a), s.due(b)) == (beat(3_000), beat(4_000))
    delivered = []
    for f in range(5):
        p = s.plan_frame(frame(f), 100, c)
        assert not p.missed, f
        delivered += [(f, d.job) for d in p.delivered]
    assert delivered == [(3, a), (4, b)]


def test_on_beat_job_no_frame_can_run_is_decided_at_its_beat():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_HOLD_PREVIOUS, 50)
    job = s.submit(at(0), [0], c)
    assert s.due(job) == beat(1_000)
    p = s.plan_frame(at(500), 50, c)
    assert not p.runs and not p.missed and not p.delivered
    p = s.plan_frame(at(1_000), 50, c)
    assert not p.runs and not p.delivered
    assert [(m.job, m.due) for m in p.missed] == [(job, beat(1_000))]
    s = S.Scheduler(on_beat(0), S.MISS_HOLD_PREVIOUS, 50)
    job = s.submit(at(0), [0], c)
    s.plan_frame(at(500), 50, c)
    p = s.plan_frame(at(1_000), 100, c)
    assert len(p.runs) == 1 and [d.job for d in p.delivered] == [job]


def test_on_beat_lone_job_a_dip_makes_late_is_kept_and_delivered_on_its_beat():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_HOLD_PREVIOUS, 100)
    job = s.submit(frame(0), [0, 1, 2], c)
    assert s.due(job) == beat(3_000)
    for f, b, ran in ((0, 0, 0), (1, 0, 0), (2, 100, 1)):
        p = s.plan_frame(frame(f), b, c)
        assert len(p.runs) == ran and not p.missed and not p.delivered, f
    p = s.plan_frame(frame(3), 200, c)
    assert len(p.runs) == 2 and [d.job for d in p.delivered] == [job] and not p.missed


def test_on_beat_job_queued_behind_a_late_one_is_placed_as_the_plan_runs_it():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_DROP, 100)
    a = s.submit(frame(0), [0, 1, 2], c)
    for f in range(2):
        assert not s.plan_frame(frame(f), 0, c).missed, f
    b = s.submit(frame(2), [3], c)
    assert s.due(b) == beat(3_000)
    p2 = s.plan_frame(frame(2), 100, c)
    assert [r.job for r in p2.runs] == [b]
    assert p2.missed == [S.Missed(a, 0, beat(3_000), S.MISS_DROP)]
    p3 = s.plan_frame(frame(3), 100, c)
    assert [d.job for d in p3.delivered] == [b] and not p3.missed


def test_on_beat_miss_is_reported_at_the_beat():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_HOLD_PREVIOUS, 1_000)
    job = s.submit(at(0), [0], c)
    assert not s.plan_frame(at(500), 50, c).missed
    assert [m.job for m in s.plan_frame(at(1_000), 50, c).missed] == [job]


def test_on_beat_frame_starting_after_the_beat_still_runs_and_delivers():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_DROP, 200)
    job = s.submit(at(10), [0, 1], c)
    assert s.due(job) == beat(1_000)
    p = s.plan_frame(at(10), 100, c)
    assert len(p.runs) == 1 and not p.missed
    p = s.plan_frame(at(1_010), 100, c)
    assert len(p.runs) == 1 and [d.job for d in p.delivered] == [job] and not p.missed


def test_on_beat_result_seen_after_a_skipped_beat_frame_is_missed():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_HOLD_PREVIOUS, 100)
    job = s.submit(at(10), [0], c)
    assert len(s.plan_frame(at(10), 100, c).runs) == 1
    p = s.plan_frame(at(2_010), 100, c)
    assert not p.delivered and [m.job for m in p.missed] == [job]


def test_a_tempo_change_moves_only_the_deadlines_fixed_after_it():
    c = cost()
    s = S.Scheduler(on_beat(0), S.MISS_DROP, 1_000)
    a = s.submit(at(0), [0], c)
    assert s.due(a) == beat(1_000)
    s.plan_frame(at(0), 1_000, c)
    s.replace_beat_grid(500, 500, 300)
    assert s.due(a) == beat(1_000)
    b = s.submit(at(600), [1], c)
    assert s.due(b) == beat(800)
    p = s.plan_frame(at(600), 1_000, c)
    assert not p.delivered and not p.missed
    assert [d.job for d in s.plan_frame(at(800), 1_000, c).delivered] == [b]
    p = s.plan_frame(at(1_000), 1_000, c)
    assert [d.job for d in p.delivered] == [a] and not p.missed


def test_a_slice_no_frame_holds_runs_the_slices_before_it_alone_and_is_abandoned_for_a_job_behind():
    c = cost()
    c.record(0, 500)
    s = S.Scheduler(1, S.MISS_DROP, 499)
    job = s.submit(frame(0), [1, 0], c)
    p0 = s.plan_frame(frame(0), 499, c)
    assert [(r.job, r.position) for r in p0.runs] == [(job, 0)] and not p0.missed and not p0.delivered
    p1 = s.plan_frame(frame(1), 499, c)
    assert not p1.runs and not p1.delivered and [m.job for m in p1.missed] == [job]
    s = S.Scheduler(1, S.MISS_DROP, 499)
    late = s.submit(frame(0), [1, 0], c)
    nxt = s.submit(frame(0), [2], c)
    p0 = s.plan_frame(frame(0), 499, c)
    assert [r.job for r in p0.runs] == [nxt]
    assert [(m.job, m.due) for m in p0.missed] == [(late, S.Due.frame(1))]


# ---- the host's render cost and frame step (frame.rs, step.rs tests) ---------------


def test_the_budget_follows_the_last_render_and_the_forecast_the_median():
    r = S.RenderCost()
    assert r.budget(8_300, 2_000) == 4_300
    for us in (1_900, 1_900, 9_000):
        r.record(us)
    assert r.last() == 9_000 and r.budget(8_300, 2_000) == 0
    assert r.forecast() == 1_900 and r.expected(8_300, 2_000) == 4_400
    for _ in range(S.RENDER_WINDOW):
        r.record(2_000)
    assert r.forecast() == 2_000


def test_the_timer_must_hold_the_slices_of_every_job_with_slices_left():
    cap = S.TIMER_MAX_SLICES
    assert S.timer_capacity(6, 3) == 18
    assert S.timer_capacity(cap, 1) == cap
    assert S.timer_capacity(cap, 2) is None
    assert S.timer_capacity(1, 2**32 - 1) is None and S.timer_capacity(2**32 - 1, 3) is None
    every = lambda k: S.jobs_with_slices(S.SUBMIT_EVERY, S.IN_FLIGHT_LATENCY, k)  # noqa: E731
    free = lambda k: S.jobs_with_slices(S.SUBMIT_FREE, S.IN_FLIGHT_LATENCY, k)  # noqa: E731
    assert every(2) == 3 and every(2**32 - 1) is None and free(17) == 1
    assert S.jobs_with_slices(S.SUBMIT_EVERY, S.IN_FLIGHT_BOUNDED, 3) == 3
    assert S.jobs_with_slices(S.SUBMIT_FREE, S.IN_FLIGHT_BOUNDED, 3) == 1
    assert S.timer_capacity(300, free(17)) == 300 and S.timer_capacity(300, every(17)) is None
    assert S.timer_capacity(cap + 1, free(10)) is None


def frame_at(index, period):
    return S.Frame(index, index * period, period)


def run_frame(step, index, period, owed, slice_us=None, render_us=None):
    """Plan, count, absorb (slices timed at slice_us each unless None) and
    complete one frame; returns (planned, completed plan)."""
    planned = step.plan(frame_at(index, period), owed)
    compute = []
    if slice_us is not None:
        compute = [S.TimedSlice(r.job, r.slice, slice_us, step.tag(r.slice)) for r in planned.plan.runs]
    step.after_submit(index)
    step.absorb(index, compute, render_us)
    return planned, step.complete(index)


def test_the_tally_counts_what_a_scripted_run_planned_delivered_and_missed():
    period = 16_667
    c = S.CostModel(2_000)  # the default estimator: 0.9 of the last 32
    step = S.FrameStep(S.Policy.fixed_latency(1), S.MISS_HOLD_PREVIOUS, 1, 2_000, period, c)
    slow = {2, 3, 65, 66}
    for index in range(70):
        run_frame(step, index, period, True, 1_500, 20_000 if index in slow else 1_000)
    t = step.finish()
    assert (t.submitted, t.delivered, t.missed, t.startup_missed, t.violations, t.pending_at_end) == (70, 67, 2, 1, 0, 1)
    assert t.latencies == [1] * 67 and t.dispatches_per_job == [1] * 67
    per_frame = [1] * 70
    for f, d in ((3, 0), (4, 0), (5, 2), (66, 0), (67, 0), (68, 2)):
        per_frame[f] = d
    assert t.dispatches_per_frame == per_frame
    assert len(t.gpu_frame_us) == 70 and t.gpu_frame_us[0] == 2_500 and t.gpu_frame_us[3] == 20_000
    assert t.gpu_frame_us[5] == 4_000
    assert t.longest_dispatch_us == [1_500] * 66
    assert t.measured == {0: (68 * 1_500, 68)}
    assert len(t.frame_ratios) == 66 and t.timed_frames == 70 and len(t.estimates) == 1


def test_a_frame_planned_before_the_last_was_counted_is_refused():
    period = 16_667
    step = S.FrameStep(S.Policy.fixed_latency(2), S.MISS_HOLD_PREVIOUS, 2, 2_000, period, S.CostModel(2_000))
    first = step.plan(frame_at(0, period), True)
    assert len(first.plan.runs) == 2 and step.dispatched(first.job) == 0
    with pytest.raises(S.ScheduleError) as e:
        step.plan(frame_at(1, period), True)
    assert e.value.code == S.ERR_NOT_COUNTED and e.value.unsubmitted == 0
    step.after_submit(0)
    assert step.dispatched(first.job) == 2 and step.submitted() == 1
    step.complete(0)
    step.plan(frame_at(1, period), True)


def test_the_tally_counts_what_a_scripted_on_beat_run_delivered_and_missed():
    period, beat_us = 10_000, 50_000
    c = mean_sigmas(2_000, 1.0, 0.0)
    step = S.FrameStep(S.Policy.on_beat(0, 1_000_000, 1_000), S.MISS_HOLD_PREVIOUS, 3, 3_000, period, c)
    step.replace_beat_grid(0, 0, beat_us)
    due, delivered, missed = {}, [], []
    for index in range(21):
        planned = step.plan(frame_at(index, period), index % 5 == 0)
        budget = 0 if 10 <= index <= 15 else 5_000
        assert (planned.budget, planned.expected) == (budget, 5_000), index
        if planned.job is not None:
            assert planned.due == S.Due.beat(index * period + beat_us), index
            due[planned.job] = planned.due
        step.after_submit(index)
        step.absorb(index, [], 20_000 if 9 <= index <= 14 else 2_000)
        plan = step.complete(index)
        for d in plan.delivered:
            assert due[d.job] == S.Due.beat(index * period)
            delivered.append((d.job, index))
        for m in plan.missed:
            assert due[m.job] == m.due
            missed.append((m.job, index))
    assert delivered == [(0, 5), (1, 10), (3, 20)] and missed == [(2, 15)]
    t = step.finish()
    assert (t.submitted, t.delivered, t.missed, t.startup_missed, t.violations, t.pending_at_end) == (5, 3, 1, 1, 0, 1)
    assert t.latencies == [5] * 3 and t.dispatches_per_job == [3] * 3
    per_frame = [0] * 21
    for f, d in ((0, 2), (1, 1), (5, 2), (6, 1), (16, 2), (17, 1), (20, 2)):
        per_frame[f] = d
    assert t.dispatches_per_frame == per_frame


def test_a_job_its_own_frame_delivers_keeps_the_beat_read_before_the_plan():
    period = 10_000
    step = S.FrameStep(S.Policy.on_beat(0, 50_000, 0), S.MISS_HOLD_PREVIOUS, 1, 3_000, period,
                       mean_sigmas(0, 1.0, 0.0))
    planned = step.plan(frame_at(5, period), True)
    assert planned.due == S.Due.beat(50_000)
    assert [d.job for d in planned.plan.delivered] == [planned.job]
    step.after_submit(5)
    step.complete(5)
    t = step.finish()
    assert (t.delivered, t.latencies) == (1, [0])


def _simulate(waits, frames):
    period, margin, render_us = 8_300, 2_000, 1_900
    costs = [(60, 120, 180, 240, 300)[i % 5] for i in range(160)]
    c = S.CostModel(2_000)
    for _ in range(32):
        for sl, us in enumerate(costs):
            c.record(sl, us)
    step = S.FrameStep(S.Policy.fixed_latency(25), S.MISS_HOLD_PREVIOUS, 160, margin, period, c, S.SUBMIT_FREE)
    for index in range(frames):
        planned = step.plan(frame_at(index, period), True)
        ran = sum(costs[r.slice] for r in planned.plan.runs)
        step.after_submit(index)
        step.absorb(index, [], render_us + (ran if waits else 0))
        step.complete(index)
    t = step.finish()
    return t.delivered, t.missed


def test_a_render_that_waits_for_the_slices_slows_the_jobs():
    assert _simulate(False, 3_000) == (425, 0)
    assert _simulate(True, 3_000) == (218, 0)


def _schedule_alone(submit, slices, k, frames):
    period = 16_667
    margin = period - S.RENDER_PRIOR - 10_000
    step = S.FrameStep(S.Policy.fixed_latency(k), S.MISS_HOLD_PREVIOUS, slices, margin, period,
                       mean_sigmas(1_000, 1.0, 0.0), submit)
    for i in range(frames):
        planned = step.plan(frame_at(i, period), True)
        assert planned.budget == planned.expected == 10_000
        step.after_submit(i)
        step.complete(i)
    t = step.finish()
    return t.submitted, t.delivered, t.missed


def test_a_job_longer_than_a_frame_misses_most_inputs_when_every_frame_submits_and_none_when_free():
    assert _schedule_alone(S.SUBMIT_EVERY, 45, 5, 120) == (120, 26, 92)
    assert _schedule_alone(S.SUBMIT_FREE, 45, 5, 120) == (24, 23, 0)
    assert _schedule_alone(S.SUBMIT_FREE, 45, 3, 120) == (30, 0, 30)


def test_a_finished_step_takes_no_frame():
    step = S.FrameStep(S.Policy.fixed_latency(1), S.MISS_DROP, 1, 0, 1_000, S.CostModel(10))
    step.finish()
    with pytest.raises(S.ScheduleError) as e:
        step.plan(frame_at(0, 1_000), True)
    assert e.value.code == S.ERR_FINISHED
