"""The slice timer (hipEvent pairs, crates/beatlm/src/gpu/timer.rs:185-464 and
its tests), the fixed-time render load, and the frame-budget loop of the
high-resolution encoder (calibrate -> parts_within -> split -> scheduled
slices), on a small block so each test takes seconds."""

import time

import numpy as np
import pytest

import oracle
from beatlm_amd import frameloop, hip, ir
from tests.blockdata import block_graph, block_values, block_weights

pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def small(ctx):
    t, d, h, mlp = 257, 384, 6, 1536
    x = oracle.uniform(31, t * d, -2.0, 2.0)
    w = block_weights(d, mlp, 100, "reference")
    g, ids = block_graph(t, d, h, mlp, EPS)
    vals = block_values(ids, x, w)
    prep = ir.prepare(ctx, g)
    for tid, v in vals.items():
        prep.write(tid, v)
    yield g, ids, vals, prep
    prep.kernels.close()
    prep.arenas.close()


def encode_frame(prep, timer, frame, tags=None):
    timed = timer.begin_frame(frame)
    for k in range(len(prep.kernels)):
        prep.kernels.encode(k, 0, timer, k if tags is None else tags[k])
    return timed, timer.resolve()


def test_frames_come_back_in_submission_order_with_every_slice(ctx, small):
    _, _, _, prep = small
    n = len(prep.kernels)
    timer = hip.Timer(ctx, n)
    try:
        got = []
        for f in range(3):
            timed, r = encode_frame(prep, timer, 10 + f, tags=[100 * f + k for k in range(n)])
            assert timed
            timer.submitted(r)
        ctx.synchronize()
        got = timer.collect()
        assert [f for f, _ in got] == [10, 11, 12]
        for i, (_, slices) in enumerate(got):
            assert [t for t, _ in slices] == [100 * i + k for k in range(n)]
            assert all(us > 0.0 for _, us in slices)
        s = timer.stats()
        assert (s.frames_begun, s.frames_timed, s.frames_skipped, s.frames_failed, s.frames_dropped) == (3, 3, 0, 0, 0)
    finally:
        timer.close()


def test_a_frame_whose_slot_is_in_flight_is_skipped_not_waited_for(ctx, small):
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))
    try:
        for f in range(hip.RING_DEPTH):
            timed, r = encode_frame(prep, timer, f)
            assert timed
            timer.submitted(r)
        timed, r = encode_frame(prep, timer, hip.RING_DEPTH)
        assert not timed
        timer.submitted(r)  # handing back an untimed frame is accepted and ignored
        ctx.synchronize()
        assert [f for f, _ in timer.collect()] == list(range(hip.RING_DEPTH))
        assert timer.stats().frames_skipped == 1
        timed, r = encode_frame(prep, timer, 99)
        assert timed
        timer.submitted(r)
        ctx.synchronize()
        assert [f for f, _ in timer.collect()] == [99]
    finally:
        timer.close()


def test_invalidated_frames_are_never_decoded_and_count_as_failed(ctx, small):
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))
    try:
        for f in range(2):
            _, r = encode_frame(prep, timer, f)
            timer.submitted(r)
        assert timer.invalidate_submitted() == 2
        assert timer.invalidate_submitted() == 0  # already marked
        ctx.synchronize()
        assert timer.collect() == []
        s = timer.stats()
        assert (s.frames_failed, s.frames_timed) == (2, 0)
        _, r = encode_frame(prep, timer, 5)
        timer.submitted(r)
        ctx.synchronize()
        assert [f for f, _ in timer.collect()] == [5]
    finally:
        timer.close()


def run_frame(ctx, prep, timer, frame):
    """One frame through the timer: encode, hand back, wait, collect."""
    _, r = encode_frame(prep, timer, frame, tags=[1000 + frame] * len(prep.kernels))
    timer.submitted(r)
    ctx.synchronize()
    return timer.collect()


def test_an_abandoned_frame_is_never_read_and_its_slot_comes_back(ctx, small):
    """gpu/timer.rs:964-1017: after a lap every slot's events hold real
    times; a frame resolved and then given up (its work never handed back)
    is not read, the next frame is reported as itself, and the freed slot
    serves a further lap."""
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))
    try:
        for f in range(hip.RING_DEPTH):
            assert [x for x, _ in run_frame(ctx, prep, timer, f)] == [f]
        dropped = hip.RING_DEPTH
        _, r = encode_frame(prep, timer, dropped)
        assert r != 0
        timer.abandon(r)
        assert timer.in_flight() == 0
        timer.submitted(r)  # spent: handing it back afterwards is ignored
        nxt = dropped + 1
        got = run_frame(ctx, prep, timer, nxt)
        assert [x for x, _ in got] == [nxt]
        assert {t for t, _ in got[0][1]} == {1000 + nxt}
        assert timer.in_flight() == 0
        for f in range(nxt + 1, nxt + 1 + hip.RING_DEPTH):
            got = run_frame(ctx, prep, timer, f)
            assert [x for x, _ in got] == [f] and {t for t, _ in got[0][1]} == {1000 + f}
        s = timer.stats()
        assert (s.frames_timed, s.frames_failed, s.frames_skipped, s.frames_dropped) == (2 * hip.RING_DEPTH + 1, 0, 0, 1)
    finally:
        timer.close()


def test_tickets_may_come_back_out_of_order_and_are_read_in_submission_order(ctx, small):
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))
    try:
        _, a = encode_frame(prep, timer, 1)
        _, b = encode_frame(prep, timer, 2)
        assert timer.in_flight() == 2
        timer.submitted(b)
        timer.submitted(a)
        ctx.synchronize()
        assert [f for f, _ in timer.collect()] == [2, 1]
    finally:
        timer.close()


def test_an_invalidated_frame_after_a_lap_is_counted_and_never_read(ctx, small):
    """gpu/timer.rs:1020-1083: the frame lands on a slot whose events hold an
    earlier lap's times; marked before collection, it is dropped unread, and
    the frames after it are reported as themselves."""
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))
    try:
        for f in range(hip.RING_DEPTH):
            assert len(run_frame(ctx, prep, timer, f)) == 1
        marked = hip.RING_DEPTH
        _, r = encode_frame(prep, timer, marked)
        timer.submitted(r)
        ctx.synchronize()
        assert timer.invalidate_submitted() == 1
        assert timer.in_flight() == 1
        assert timer.collect() == []
        assert timer.in_flight() == 0
        for f in range(marked + 1, marked + 2 + hip.RING_DEPTH):
            got = run_frame(ctx, prep, timer, f)
            assert [x for x, _ in got] == [f] and {t for t, _ in got[0][1]} == {1000 + f}
        s = timer.stats()
        assert (s.frames_failed, s.frames_timed, s.frames_skipped) == (1, 2 * hip.RING_DEPTH + 1, 0)
    finally:
        timer.close()


def test_a_held_frame_is_read_only_once_accepted(ctx, small):
    """gpu/timer.rs:1086-1160: held frames are read only once accepted and in
    submission order; the rejected one between two accepted ones is dropped
    unread and holds back nothing."""
    _, _, _, prep = small
    timer = hip.Timer(ctx, len(prep.kernels))

    def held(frame):
        _, r = encode_frame(prep, timer, frame, tags=[1000 + frame] * len(prep.kernels))
        h = timer.submitted_held(r)
        assert h != 0
        return h

    try:
        for f in range(hip.RING_DEPTH):
            h = held(f)
            ctx.synchronize()
            assert timer.collect() == []  # completed, not accepted
            assert timer.verdict(h, True)
            assert [x for x, _ in timer.collect()] == [f]
        first = hip.RING_DEPTH
        before, rejected, after = held(first), held(first + 1), held(first + 2)
        ctx.synchronize()
        assert timer.collect() == [] and timer.in_flight() == 3
        assert timer.verdict(after, True)
        assert timer.collect() == [] and timer.in_flight() == 3
        assert timer.verdict(rejected, False)
        assert timer.verdict(before, True)
        got = timer.collect()
        assert [x for x, _ in got] == [first, first + 2]
        assert {t for t, _ in got[0][1]} == {1000 + first} and {t for t, _ in got[1][1]} == {1000 + first + 2}
        assert timer.in_flight() == 0
        assert not timer.verdict(before, False)  # spent
        s = timer.stats()
        assert (s.frames_failed, s.frames_timed, s.frames_skipped) == (1, hip.RING_DEPTH + 2, 0)
    finally:
        timer.close()


def test_too_many_slices_in_a_frame_is_an_error(ctx, small):
    _, _, _, prep = small
    timer = hip.Timer(ctx, 2)
    try:
        timer.begin_frame(0)
        prep.kernels.encode(0, 0, timer, 0)
        prep.kernels.encode(1, 0, timer, 1)
        with pytest.raises(hip.BackendError) as e:
            prep.kernels.encode(2, 0, timer, 2)
        assert e.value.code == hip.ERR_TIMER_TOO_MANY_SLICES
        timer.submitted(timer.resolve())
        ctx.synchronize()
        timer.collect()
    finally:
        timer.close()


def test_the_render_load_spins_for_its_time(ctx):
    ctx.synchronize()
    for us in (2000, 8000):
        t0 = time.perf_counter()
        ctx.spin(us)
        ctx.synchronize()
        took = (time.perf_counter() - t0) * 1e6
        assert us * 0.98 <= took <= us + 3000, (us, took)


def test_the_slice_timer_sees_the_render_load_it_runs_behind(ctx, small):
    # A slice encoded after the spin starts only when the spin ends, so the
    # frame's wall time covers both and the slice's own time stays short.
    _, _, _, prep = small
    timer = hip.Timer(ctx, 1)
    try:
        ctx.synchronize()
        t0 = time.perf_counter()
        timer.begin_frame(0)
        ctx.spin(3000)
        prep.kernels.encode(0, 0, timer, 7)
        timer.submitted(timer.resolve())
        ctx.synchronize()
        wall = (time.perf_counter() - t0) * 1e6
        [(frame, [(tag, us)])] = timer.collect()
        assert (frame, tag) == (0, 7) and 0 < us < 1000 and wall >= 2900
    finally:
        timer.close()


@pytest.mark.parametrize("bound_us", [frameloop.DEFAULT_MAX_DISPATCH_US, 4])
def test_the_frame_loop_delivers_every_frame_within_its_latency(ctx, small, bound_us):
    g, ids, vals, _ = small
    frames = 24
    report = frameloop.run(ctx, g, vals, ids.output, hip.F32, frames=frames, period_us=4000, render_us=1500,
                           bound_us=bound_us, tolerance=1e-4)
    k = report["latency_frames_k"]
    assert report["budget_us"] == 2500
    if report["dropped_periods"] == 0:  # a host that lost whole periods misses their deadlines
        assert report["missed"] == 0, report
        assert report["delivered"] == frames - k, report
    assert report["spent_estimate_us_per_frame_max"] <= report["budget_us"]
    assert report["output_within_tolerance"], report
    if bound_us == 4:
        # Some kernel of this block takes longer than 4 µs: it was split, and
        # the split program's result still matches the whole one.
        assert report["kernels_split"] > 0 and report["slices_per_job"] > report["kernels_unsplit"]
    else:
        assert report["slices_per_job"] == report["kernels_unsplit"]


def test_on_beat_delivers_every_job_on_its_beat_at_the_high_resolution_shape(ctx):
    """Config 5's encoder (ViT-S/14 at 1036 pixels: 5477 tokens, 12 f16
    blocks) driven by the host's frame step with the OnBeat policy at 60
    frames per second beside an 8 ms render load: an input every 6 frames,
    beats every 6 frames, each job delivered by the frame that starts on the
    beat after its submission (beatlm-host/src/step.rs:686-760 scripts the
    same), none missed; kernels longer than 40 us split into parts, and each
    of the two job slots' outputs equals the unsplit program's for its input."""
    import bench
    from beatlm_amd import schedule as S

    cfg = bench.CONFIGS["vit-s-1036"]
    g, emb, ids, tokens = bench.build_encoder(cfg)
    vals = bench.synthetic_values(cfg, emb, ids, tokens, np.float16)
    period = 16_667
    beat = 6 * period
    frames = 42
    policy = S.Policy.on_beat(0, beat, 1_000)
    images = [bench.frame_image(cfg, f, np.float16) for f in range(2)]
    report = frameloop.run(ctx, g, vals, ids[-1].output, hip.F16, frames=frames, period_us=period, render_us=8_000,
                           bound_us=40, tolerance=2e-2, policy=policy, owed_every=6, slots=2,
                           input_tid=emb.image, slot_inputs=images)
    print({k: report[k] for k in ("policy", "kernels_split", "slices_per_job", "delivered", "missed", "submitted",
                                  "pending_at_end", "latencies_frames", "output_max_abs_vs_unsplit")})
    assert report["kernels_split"] > 0 and report["slices_per_job"] > report["kernels_unsplit"]
    assert report["submitted"] == frames // 6
    assert report["missed"] == 0, report["misses"]
    # Every job but the last (due after the run) is delivered, on a beat frame,
    # six frames after its submission.
    assert report["delivered"] == report["submitted"] - report["pending_at_end"] >= frames // 6 - 1
    assert all(frame % 6 == 0 for _, frame in report["deliveries"]), report["deliveries"]
    assert report["latencies_frames"] == [6]
    assert report["output_within_tolerance"], report["output_max_abs_vs_unsplit"]
