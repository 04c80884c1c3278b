"""The frame-budget loop of the high-resolution encoder: the encoder's kernels
run as slices inside each frame's budget, beside a fixed-time render load, at a
fixed frame period.

It follows the reference bench's flow (crates/beatlm-bench/src/calibrate.rs
and engine.rs):

1. Calibration pass 1: the unsplit program runs whole once per paced frame,
   followed by the render load, for CALIBRATION_FRAMES timed frames after one
   untimed frame; each kernel's duration is the median (the upper middle,
   beatlm-host/src/stats.rs:145) of its slice-timer measurements in the second
   half (beatlm-host/src/calibration.rs:29).
2. `Program.parts_within(durations, bound)` decides the parts
   (kernel.rs:2350-2408) and `Program.split` makes them.
3. Calibration pass 2: the split program runs the same way and every part's
   measurements of the second half go into the cost model as calibration
   (CostModel::record_calibration).
4. The loop: every frame submits the frame's input as a job of all the split
   program's slices (Submit::Every, beatlm-host/src/frame.rs:163-170), plans it
   with the FixedLatency scheduler against Budget::for_frame(period, render,
   margin), encodes the runs with the slice timer, then the render load, and
   feeds the timer's durations back into the cost model.

Durations reach the cost model in whole microseconds rounded to nearest, as
the reference timer rounds (gpu/timer.rs:781-799). Every GPU call goes through
the backend's C ABI; this module only decides and paces.
"""

from __future__ import annotations

import statistics
import time
from dataclasses import dataclass

import numpy as np

from . import hip, ir
from . import schedule as S

WINDOW = 32                         # presets.rs: the quantile estimator's window
CALIBRATION_FRAMES = 2 * WINDOW     # presets.rs:71
SLICE_PRIOR_US = 2_000              # presets.rs:44
DEFAULT_MAX_DISPATCH_US = 1_000     # beatlm-bench/src/args.rs:72
FRAME_PERIOD_US = 16_667            # 60 frames per second


def counted(frame: int) -> bool:
    """The calibration frames whose measurements count: the second half."""
    return frame > CALIBRATION_FRAMES // 2


def median_upper(samples) -> int:
    s = sorted(samples)
    return s[len(s) // 2]


class Pacer:
    """Frame boundaries every `period_us` from the first call; a frame that
    begins a whole period late gives up the periods it missed."""

    def __init__(self, period_us: int):
        self.period = period_us / 1e6
        self.t0 = None
        self.index = 0
        self.dropped = 0
        self.lateness_us: list[float] = []

    def next(self) -> tuple[int, int]:
        now = time.perf_counter()
        if self.t0 is None:
            self.t0 = now
            return 0, 0
        self.index += 1
        boundary = self.t0 + self.index * self.period
        if now > boundary + self.period:
            skipped = int((now - boundary) / self.period)
            self.index += skipped
            self.dropped += skipped
            boundary = self.t0 + self.index * self.period
        while True:
            now = time.perf_counter()
            if now >= boundary:
                break
            time.sleep(min(boundary - now, 0.001))
        self.lateness_us.append((now - boundary) * 1e6)
        return self.index, int(round((boundary - self.t0) * 1e6))


def _release(prep: ir.Prepared) -> None:
    prep.kernels.close()
    prep.arenas.close()


def _measure(prep: ir.Prepared, period_us: int, render_us: int, record) -> None:
    """One untimed frame, then CALIBRATION_FRAMES timed ones, each the whole
    program followed by the render load, paced at the frame period; `record`
    receives (frame, kernel, µs) for every measurement."""
    ctx = prep.ctx
    n = len(prep.kernels)
    timer = hip.Timer(ctx, n)
    pacer = Pacer(period_us)
    try:
        for f in range(CALIBRATION_FRAMES + 1):
            pacer.next()
            if f == 0:  # pays for first use
                prep.run()
                ctx.spin(render_us)
                ctx.synchronize()
                continue
            timer.begin_frame(f)
            for k in range(n):
                prep.kernels.encode(k, 0, timer, k)
            ctx.spin(render_us)
            timer.submitted(timer.resolve())
            ctx.synchronize()
            for frame, slices in timer.collect():
                for tag, us in slices:
                    record(frame, tag, int(round(us)))
    finally:
        timer.close()


@dataclass
class Calibration:
    durations: list        # µs per kernel of the unsplit program
    parts: list            # parts per kernel
    program: ir.Program    # the split program
    cost: S.CostModel      # slice i = kernel i of `program`
    reference_output: np.ndarray


def calibrate(ctx, graph, values, output_tid, dtype, period_us, render_us, bound_us) -> Calibration:
    whole = ir.prepare(ctx, graph, dtype=dtype)
    for tid, v in values.items():
        whole.write(tid, v)
    samples = [[] for _ in range(len(whole.kernels))]

    def first(frame, k, us):
        if counted(frame):
            samples[k].append(us)

    _measure(whole, period_us, render_us, first)
    missing = [whole.program.name(k) for k, s in enumerate(samples) if not s]
    if missing:
        raise RuntimeError(f"calibration never measured {missing}")
    durations = [median_upper(s) for s in samples]
    reference_output = whole.read(output_tid).astype(np.float32)
    parts = whole.program.parts_within(durations, bound_us) if bound_us else [1] * len(durations)
    _release(whole)

    program = graph.lower(ir.FUSION_ON).fuse_attention()
    program = program.split(parts)
    split = ir.realise(ctx, program, dtype)
    for tid, v in values.items():
        split.write(tid, v)
    cost = S.CostModel(SLICE_PRIOR_US, WINDOW, 0.9)

    def second(frame, k, us):
        if counted(frame):
            cost.record_calibration(k, us)

    _measure(split, period_us, render_us, second)
    _release(split)
    return Calibration(durations, parts, program, cost, reference_output)


def latency_for(estimates, budget_us: int, expected_us: int) -> int:
    """The smallest FixedLatency that keeps a lone job of slices priced at
    `estimates`: the last frame the scheduler's projection (schedule.rs:381-406)
    places them on, counting from the submission frame."""
    frame, spent = 0, 0
    for e in estimates:
        while True:
            cap = budget_us if frame == 0 else expected_us
            if spent + e <= cap:
                spent += e
                break
            if frame > 0 and spent == 0:
                raise ValueError(f"a slice of {e} µs fits no frame of {expected_us} µs")
            frame, spent = frame + 1, 0
    return frame


def run(ctx, graph, values, output_tid, dtype, frames=120, period_us=FRAME_PERIOD_US, render_us=8_000,
        margin_us=0, bound_us=DEFAULT_MAX_DISPATCH_US, tolerance=2e-2) -> dict:
    """Calibrates, then runs `frames` paced frames; returns the report."""
    budget = S.budget_for_frame(period_us, render_us, margin_us)
    cal = calibrate(ctx, graph, values, output_tid, dtype, period_us, render_us, bound_us)
    n = len(cal.program)
    estimates = [cal.cost.planning_estimate(i) for i in range(n)]
    k = latency_for(estimates, budget, budget)

    prep = ir.realise(ctx, cal.program, dtype)
    for tid, v in values.items():
        prep.write(tid, v)
    timer = hip.Timer(ctx, min(4096, n * (k + 1)))
    sched = S.Scheduler(k, S.MISS_HOLD_PREVIOUS, budget)
    pacer = Pacer(period_us)
    runs_per_frame, spent, gpu_us_per_frame, frame_wall_us = [], [], [], []
    delivered = missed = 0
    job_slices: dict[int, int] = {}
    job_gpu: dict[int, float] = {}
    job_of_frame: dict[int, list] = {}
    allocs = ctx.allocations()
    try:
        for _ in range(frames):
            index, start = pacer.next()
            began = time.perf_counter()
            info = S.Frame(index, start, period_us)
            job = sched.submit(info, list(range(n)), cal.cost)
            plan = sched.plan_frame(info, budget, cal.cost)
            timer.begin_frame(index)
            job_of_frame[index] = []
            for r in plan.runs:
                prep.kernels.encode(r.slice, 0, timer, r.slice)
                job_of_frame[index].append(r.job)
            ctx.spin(render_us)
            timer.submitted(timer.resolve())
            ctx.synchronize()
            frame_wall_us.append((time.perf_counter() - began) * 1e6)
            runs_per_frame.append(len(plan.runs))
            spent.append(plan.spent_estimate)
            delivered += len(plan.delivered)
            missed += len(plan.missed)
            job_slices[job] = n
            for frame, slices in timer.collect():
                owners = job_of_frame.pop(frame, [])
                gpu_us_per_frame.append(sum(us for _, us in slices))
                for (tag, us), owner in zip(slices, owners):
                    cal.cost.record(tag, int(round(us)))
                    job_gpu[owner] = job_gpu.get(owner, 0.0) + us
        stats = timer.stats()
        assert ctx.allocations() == allocs, "the frame loop allocated device memory"
        out = prep.read(output_tid).astype(np.float32)
    finally:
        timer.close()
        _release(prep)
    err = float(np.max(np.abs(out - cal.reference_output)))
    job_times = [v for j, v in job_gpu.items() if j < max(job_gpu, default=0)]
    split_kernels = sum(1 for p in cal.parts if p > 1)
    return {
        "workload": "frame-budget slices at a fixed frame period beside a fixed-time render load",
        "frame_period_us": period_us,
        "render_load_us": render_us,
        "margin_us": margin_us,
        "budget_us": budget,
        "max_dispatch_us": bound_us,
        "kernels_unsplit": len(cal.durations),
        "kernels_split": split_kernels,
        "slices_per_job": n,
        "calibrated_job_us": sum(cal.durations),
        "planned_job_us": sum(estimates),
        "latency_frames_k": k,
        "submit": "every frame",
        "frames": frames,
        "slices_per_frame": {
            "mean": round(statistics.mean(runs_per_frame), 2),
            "min": min(runs_per_frame),
            "max": max(runs_per_frame),
        },
        "spent_estimate_us_per_frame_max": max(spent),
        "measured_slice_us_per_frame_median": round(statistics.median(gpu_us_per_frame), 1) if gpu_us_per_frame else None,
        "measured_job_us_median": round(statistics.median(job_times), 1) if job_times else None,
        "frame_wall_us_median": round(statistics.median(frame_wall_us), 1),
        "delivered": delivered,
        "missed": missed,
        "dropped_periods": pacer.dropped,
        "timer": {"frames_timed": int(stats.frames_timed), "frames_skipped": int(stats.frames_skipped),
                  "frames_failed": int(stats.frames_failed), "frames_dropped": int(stats.frames_dropped)},
        "output_max_abs_vs_unsplit": err,
        "output_within_tolerance": bool(err <= tolerance),
    }
