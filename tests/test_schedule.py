"""The slice scheduler and cost model restated in C++ (beatlm_amd/csrc/
schedule.cpp), checked with the cases of the reference core's own tests:
crates/beatlm-core/src/budget.rs:43-55, cost.rs:1088-1380 (windowed quantile)
and schedule.rs:856-1240 (FixedLatency / SameFrame). The reference's
scheduler tests price unmeasured slices at a 100 µs prior and measured ones at
their one measurement, which the windowed quantile gives as well. CPU only.
"""

import math

import pytest

from beatlm_amd import schedule as S

PERIOD = 1000
SLICE = 7


def frame(i):
    return S.frame(i, PERIOD)


def cost():
    return S.CostModel(100, 32, 0.9)


def test_budget_for_frame_subtracts_render_and_margin():
    assert S.budget_for_frame(16_000, 10_000, 1_000) == 5_000


def test_budget_for_frame_saturates_at_zero():
    assert S.budget_for_frame(16_000, 15_000, 2_000) == 0
    assert S.budget_for_frame(1, 2**64 - 1, 2**64 - 1) == 0


def test_invalid_window_and_quantile_are_rejected():
    for window in (0, S.MAX_WINDOW + 1):
        with pytest.raises(S.ScheduleError) as e:
            S.CostModel(0, window, 0.9)
        assert e.value.code == S.ERR_INVALID_WINDOW
    for q in (-0.1, 1.1, math.nan, math.inf):
        with pytest.raises(S.ScheduleError) as e:
            S.CostModel(0, 8, q)
        assert e.value.code == S.ERR_INVALID_QUANTILE
    for window, q in ((1, 0.0), (S.MAX_WINDOW, 1.0), (8, 0.5)):
        S.CostModel(0, window, q)


def test_prior_is_used_without_samples():
    m = S.CostModel(123, 8, 0.9)
    assert m.estimate(SLICE) == 123 and m.samples(SLICE) == 0
    m.record(SLICE + 1, 5)
    assert m.estimate(SLICE) == 123


def test_quantile_reads_the_nearest_rank_of_the_window():
    for q, expected in ((0.0, 10), (0.2, 10), (0.5, 30), (0.9, 50), (1.0, 50)):
        m = S.CostModel(1, 8, q)
        for x in (50, 10, 40, 20, 30):
            m.record(SLICE, x)
        assert m.estimate(SLICE) == expected, q


def test_a_whole_rank_is_not_pushed_up_by_rounding():
    assert S.nearest_rank(0.55, 100) == 55
    assert S.nearest_rank(0.9, 32) == 29
    assert S.nearest_rank(0.0, 5) == 1
    assert S.nearest_rank(1.0, 5) == 5


def test_nearest_rank_is_the_textbook_definition_off_the_whole_numbers():
    # Away from products within 1e-9 of an integer the rank is ceil(q n).
    for n in (1, 2, 3, 7, 32, 100, 4096):
        for q in (0.013, 0.25, 0.333, 0.9, 0.999):
            p = q * n
            if abs(p - round(p)) < 1e-6:
                continue
            assert S.nearest_rank(q, n) == min(max(math.ceil(p), 1), n), (q, n)


def test_quantile_forgets_what_leaves_the_window():
    m = S.CostModel(1, 3, 1.0)
    for x in (900, 10, 20):
        m.record(SLICE, x)
    assert m.estimate(SLICE) == 900
    m.record(SLICE, 30)
    assert m.estimate(SLICE) == 30
    m.record(SLICE, 5)
    assert m.estimate(SLICE) == 30
    m.record(SLICE, 6)
    m.record(SLICE, 7)
    assert m.estimate(SLICE) == 7
    assert m.samples(SLICE) == 7


def test_a_window_of_one_tracks_the_last_sample():
    m = S.CostModel(1, 1, 0.9)
    m.record(SLICE, 100)
    m.record(SLICE, 400)
    assert m.estimate(SLICE) == 400


def test_windows_are_per_slice_and_samples_count_per_slice():
    m = S.CostModel(1, 2, 1.0)
    m.record(SLICE, 100)
    m.record(SLICE, 90)
    m.record(8, 5)
    assert m.estimate(SLICE) == 100 and m.estimate(8) == 5
    assert (m.samples(SLICE), m.samples(8), m.samples(9)) == (2, 1, 0)


def test_calibration_folds_as_the_loop_does():
    a, b = S.CostModel(9, 4, 0.9), S.CostModel(9, 4, 0.9)
    for x in (5, 50, 500, 7, 70):
        a.record(SLICE, x)
        b.record_calibration(SLICE, x)
        assert a.estimate(SLICE) == b.estimate(SLICE) == b.planning_estimate(SLICE)
    assert a.samples(SLICE) == b.samples(SLICE)


def test_the_windowed_quantile_is_robust_to_outliers():
    # Bulk 1000-1040 µs, one slow 8000 µs outlier in ten (cost.rs:1344-1378).
    m = S.CostModel(1, 20, 0.9)
    peak = 0
    for i in range(200):
        m.record(SLICE, 8000 if i % 10 == 9 else 1000 + (i % 5) * 10)
        if i >= 30:
            peak = max(peak, m.estimate(SLICE))
    assert peak <= 1040


def test_the_window_matches_a_brute_force_quantile():
    import random

    rng = random.Random(5)
    for window, q in ((1, 0.5), (5, 0.9), (32, 0.9), (17, 0.3)):
        m = S.CostModel(0, window, q)
        seen = []
        for _ in range(80):
            x = rng.randrange(0, 10_000)
            m.record(SLICE, x)
            seen.append(x)
            w = sorted(seen[-window:])
            assert m.estimate(SLICE) == w[S.nearest_rank(q, len(w)) - 1]


def test_an_empty_job_is_rejected():
    s = S.Scheduler(0, S.MISS_DROP, 100)
    with pytest.raises(S.ScheduleError) as e:
        s.submit(frame(0), [], cost())
    assert e.value.code == S.ERR_EMPTY_JOB and s.pending() == 0


def test_job_ids_count_from_zero():
    s = S.Scheduler(0, S.MISS_DROP, 100)
    c = cost()
    assert (s.submit(frame(0), [0], c), s.submit(frame(0), [0], c)) == (0, 1)


def test_fixed_latency_delivers_exactly_on_its_frame():
    s = S.Scheduler(2, S.MISS_DROP, 1000)
    c = cost()
    job = s.submit(frame(10), [0], c)
    assert s.due(job) == S.Due.frame(12)
    p10 = s.plan_frame(frame(10), 1000, c)
    assert len(p10.runs) == 1 and not p10.delivered and not p10.missed
    p11 = s.plan_frame(frame(11), 1000, c)
    assert not p11.runs and not p11.delivered and not p11.missed and s.pending() == 1
    p12 = s.plan_frame(frame(12), 1000, c)
    assert p12.delivered == [S.Delivery(job, 10)] and not p12.missed
    assert s.pending() == 0 and s.due(job) is None


def test_a_lone_job_that_cannot_finish_runs_to_its_deadline_and_is_missed_there():
    s = S.Scheduler(2, S.MISS_HOLD_PREVIOUS, 100)
    c = cost()
    job = s.submit(frame(0), [0, 1, 2, 3], c)
    for f in range(2):
        p = s.plan_frame(frame(f), 100, c)
        assert len(p.runs) == 1 and not p.delivered and not p.missed, f
    p = s.plan_frame(frame(2), 100, c)
    assert len(p.runs) == 1 and p.runs[0].position == 2 and not p.delivered
    assert p.missed == [S.Missed(job, 0, S.Due.frame(2), S.MISS_HOLD_PREVIOUS)]
    assert s.pending() == 0
    for f in range(3, 6):
        later = s.plan_frame(frame(f), 100, c)
        assert not later.runs and not later.delivered and not later.missed


def test_a_forecast_above_the_real_budget_delays_the_miss_to_its_deadline():
    s = S.Scheduler(2, S.MISS_HOLD_PREVIOUS, 200)
    c = cost()
    job = s.submit(frame(0), [0, 1, 2, 3], c)
    ran = 0
    for f in range(2):
        p = s.plan_frame(frame(f), 100, c)
        ran += len(p.runs)
        assert not p.delivered and not p.missed
    p = s.plan_frame(frame(2), 100, c)
    assert ran == 2 and len(p.runs) == 1 and not p.delivered
    assert [(m.job, m.due) for m in p.missed] == [(job, S.Due.frame(2))]


def test_a_dip_in_one_frame_does_not_abandon_a_job_the_later_frames_finish():
    s = S.Scheduler(2, S.MISS_DROP, 200)
    c = cost()
    job = s.submit(frame(0), [0, 1, 2, 3], c)
    ran = 0
    for f, b in ((0, 100), (1, 200)):
        p = s.plan_frame(frame(f), b, c)
        ran += len(p.runs)
        assert not p.missed
    p = s.plan_frame(frame(2), 200, c)
    ran += len(p.runs)
    assert ran == 4 and [d.job for d in p.delivered] == [job]


def test_an_abandoned_job_frees_the_job_behind_it():
    s = S.Scheduler(1, S.MISS_DROP, 100)
    c = cost()
    a = s.submit(frame(0), [0, 1, 2], c)
    b = s.submit(frame(0), [3], c)
    p0 = s.plan_frame(frame(0), 100, c)
    assert [r.job for r in p0.runs] == [b]
    assert p0.missed == [S.Missed(a, 0, S.Due.frame(1), S.MISS_DROP)]
    p1 = s.plan_frame(frame(1), 100, c)
    assert [d.job for d in p1.delivered] == [b]
    for f in range(2, 5):
        p = s.plan_frame(frame(f), 100, c)
        assert not p.delivered and not p.missed


def test_a_late_lone_job_is_abandoned_once_a_job_queues_behind_it():
    s = S.Scheduler(2, S.MISS_DROP, 100)
    c = cost()
    a = s.submit(frame(0), [0, 1, 2, 3], c)
    p0 = s.plan_frame(frame(0), 100, c)
    assert [(r.job, r.position) for r in p0.runs] == [(a, 0)] and not p0.missed
    b = s.submit(frame(1), [4], c)
    p1 = s.plan_frame(frame(1), 100, c)
    assert [(r.job, r.position) for r in p1.runs] == [(b, 0)]
    assert p1.missed == [S.Missed(a, 0, S.Due.frame(2), S.MISS_DROP)]
    delivered = []
    for f in range(2, 6):
        p = s.plan_frame(frame(f), 100, c)
        assert not p.runs and not p.missed, f
        delivered += [(f, d.job) for d in p.delivered]
    assert delivered == [(3, b)]


def test_a_job_whose_deadline_has_passed_is_not_waiting_behind_a_late_one():
    s = S.Scheduler(2, S.MISS_DROP, 100)
    c = cost()
    a = s.submit(frame(2), [0, 1, 2, 3], c)
    b = s.submit(frame(0), [4], c)
    p3 = s.plan_frame(frame(3), 100, c)
    assert [r.job for r in p3.runs] == [a]
    assert [m.job for m in p3.missed] == [b]
    p4 = s.plan_frame(frame(4), 100, c)
    assert len(p4.runs) == 1 and [(m.job, m.due) for m in p4.missed] == [(a, S.Due.frame(4))] and not p4.delivered


def test_miss_policy_is_carried_through():
    s = S.Scheduler(0, S.MISS_DROP, 50)
    c = cost()
    s.submit(frame(0), [0], c)
    assert s.plan_frame(frame(0), 50, c).missed[0].policy == S.MISS_DROP


def test_budget_is_never_exceeded_and_leftover_is_not_given_to_a_later_job():
    c = cost()
    c.record(2, 40)
    s = S.Scheduler(5, S.MISS_DROP, 150)
    a = s.submit(frame(0), [0, 1], c)
    b = s.submit(frame(1), [2], c)
    p = s.plan_frame(frame(1), 150, c)
    assert [(r.job, r.position) for r in p.runs] == [(a, 0)]
    assert p.spent_estimate == 100 <= p.budget
    p = s.plan_frame(frame(2), 150, c)
    assert [(r.job, r.position) for r in p.runs] == [(a, 1), (b, 0)]
    assert p.spent_estimate == 140 == sum(c.estimate(r.slice) for r in p.runs)


def test_budget_holds_across_many_frames():
    c = cost()
    s = S.Scheduler(20, S.MISS_DROP, 250)
    for i in range(4):
        s.submit(frame(i), [0, 1, 2], c)
    for f in range(25):
        p = s.plan_frame(frame(f), 250, c)
        assert p.spent_estimate <= 250 and len(p.runs) <= 2 and not p.missed, f
    assert s.pending() == 0


def test_oldest_job_gets_slices_first_even_with_the_later_deadline():
    s = S.Scheduler(5, S.MISS_DROP, 100)
    c = cost()
    first = s.submit(frame(3), [0], c)
    second = s.submit(frame(1), [0], c)
    assert first < second
    p = s.plan_frame(frame(3), 100, c)
    assert [r.job for r in p.runs] == [first]


def test_later_job_never_gets_a_slice_while_an_earlier_job_has_slices_left():
    c = cost()
    c.record(10, 10)
    c.record(11, 10)
    s = S.Scheduler(6, S.MISS_DROP, 250)
    a = s.submit(frame(0), [0, 1, 2, 3], c)
    b = s.submit(frame(1), [10, 11], c)
    a_left, b_ran = 4, 0
    for f in range(1, 8):
        p = s.plan_frame(frame(f), 250, c)
        for run in p.runs:
            if run.job == a:
                a_left -= 1
            else:
                assert run.job == b and a_left == 0, f
                b_ran += 1
    assert (a_left, b_ran) == (0, 2)


def test_a_slice_above_every_budget_never_runs_and_is_missed_at_its_deadline():
    # A slice estimated above the expected budget fits no frame: the job is
    # late, nothing runs, and the deadline frame reports it.
    c = cost()
    c.record(0, 5000)
    s = S.Scheduler(1, S.MISS_DROP, 1000)
    job = s.submit(frame(0), [0], c)
    p0 = s.plan_frame(frame(0), 1000, c)
    assert not p0.runs and not p0.missed
    p1 = s.plan_frame(frame(1), 1000, c)
    assert not p1.runs and [m.job for m in p1.missed] == [job]


def test_the_high_resolution_loop_spreads_a_block_chain_over_frames():
    # 12 encoder blocks as 24 slices of ~600 µs against a 16 667 µs frame
    # with an 8 000 µs render pass: 8 667 µs a frame holds 14 slices, so a
    # job finishes in its second frame and latency 1 delivers every input.
    budget = S.budget_for_frame(16_667, 8_000, 0)
    c = S.CostModel(100, 32, 0.9)
    for sl in range(24):
        c.record_calibration(sl, 600)
    s = S.Scheduler(1, S.MISS_HOLD_PREVIOUS, budget)
    delivered, missed = [], []
    for f in range(12):
        if f % 2 == 0:
            s.submit(S.frame(f, 16_667), list(range(24)), c)
        p = s.plan_frame(S.frame(f, 16_667), budget, c)
        assert p.spent_estimate <= budget
        delivered += p.delivered
        missed += p.missed
    assert len(delivered) == 6 and not missed


def test_the_frame_loop_helpers():
    from beatlm_amd import frameloop as F

    # The second half of the calibration frames count (calibration.rs:29).
    assert [f for f in range(F.CALIBRATION_FRAMES + 1) if F.counted(f)][0] == F.CALIBRATION_FRAMES // 2 + 1
    # The upper middle (stats.rs:145).
    assert F.median_upper([4, 1, 3, 2]) == 3 and F.median_upper([5]) == 5
    # The latency a lone job needs is where the scheduler's projection ends,
    # and a scheduler with that latency delivers it, one frame less misses.
    for est, budget in (([100] * 24, 1000), ([600] * 24, 8667), ([30, 500, 30, 470], 500)):
        k = F.latency_for(est, budget, budget)
        for latency, ok in ((k, True), (k - 1, False)):
            if latency < 0:
                continue
            c = S.CostModel(1, 32, 0.9)
            for i, e in enumerate(est):
                c.record(i, e)
            s = S.Scheduler(latency, S.MISS_DROP, budget)
            s.submit(frame(0), list(range(len(est))), c)
            got = []
            for f in range(latency + 1):
                p = s.plan_frame(frame(f), budget, c)
                got += p.delivered
            assert bool(got) == ok, (est, latency)
    with pytest.raises(ValueError):
        F.latency_for([600], 500, 500)
