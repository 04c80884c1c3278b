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


def reference_outputs(ctx, graph, values, output_tid, dtype, input_tid, inputs) -> list:
    """The unsplit program's output for each of `inputs` (one job slot each)."""
    whole = ir.prepare(ctx, graph, dtype=dtype, slots=len(inputs))
    try:
        for tid, v in values.items():
            whole.write(tid, v)
        for j, x in enumerate(inputs):
            whole.write(input_tid, x, slot=j)
            whole.run(j)
        ctx.synchronize()
        return [whole.read(output_tid, slot=j).astype(np.float32) for j in range(len(inputs))]
    finally:
        _release(whole)


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
        margin_us=0, bound_us=DEFAULT_MAX_DISPATCH_US, tolerance=2e-2, policy: S.Policy | None = None,
        owed_every: int = 1, slots: int | None = None, input_tid: int | None = None, slot_inputs=None) -> dict:
    """Calibrates, then runs `frames` paced frames through the host's frame
    step (S.FrameStep, beatlm-host/src/step.rs:347-467), as the reference
    bench's engine ticks (crates/beatlm-bench/src/engine.rs:351-470):

      plan(frame, owed) -> encode each run into its job's slot, every compute
      pass and the render pass timed -> resolve, submit -> after_submit ->
      collect the frames whose timings have come back (never waiting) ->
      absorb each -> complete(frame).

    `policy` is FixedLatency{k} by default, with k the smallest that keeps a
    lone job of the calibrated costs (the latency the bench reports); an
    OnBeat policy delivers each job on the beat after its submission. A frame
    owes an input when its index is a multiple of `owed_every`. Jobs run in
    `slots` job slots (binding sets of the program's input and output, job j
    in slot j mod slots), by default as many as jobs can be in flight;
    `slot_inputs` gives each slot's input tensor `input_tid` its own values.
    Returns the report, with every slot's output against the unsplit
    program's for the same input."""
    budget = S.budget_for_frame(period_us, render_us, margin_us)
    cal = calibrate(ctx, graph, values, output_tid, dtype, period_us, render_us, bound_us)
    n = len(cal.program)
    estimates = [cal.cost.planning_estimate(i) for i in range(n)]
    k = latency_for(estimates, budget, budget)
    if policy is None:
        policy = S.Policy.fixed_latency(k)
    if slots is None:
        in_flight = policy.max_in_flight()
        slots = (S.jobs_with_slices(S.SUBMIT_EVERY, S.IN_FLIGHT_LATENCY, in_flight) if in_flight is not None else None) or 2
    slots = max(1, min(slots, 64))
    capacity = S.timer_capacity(n, slots)
    if capacity is None:
        raise ValueError(f"{n} slices of {slots} jobs exceed the slice timer")

    prep = ir.realise(ctx, cal.program, dtype, slots=slots)
    for tid, v in values.items():
        prep.write(tid, v)
    # Every slot's inputs (the program's INPUT tensors), as slot 0's.
    program_inputs = [t.id for t in cal.program.tensors() if cal.program.role(t.id) == ir.INPUT]
    for j in range(1, slots):
        for tid in program_inputs:
            prep.write(tid, values[tid], slot=j)
    inputs = [values[input_tid]] * slots if input_tid is not None else None
    if slot_inputs is not None:
        inputs = [slot_inputs[j % len(slot_inputs)] for j in range(slots)]
        for j in range(slots):
            prep.write(input_tid, inputs[j], slot=j)
    timer = hip.Timer(ctx, min(4096, capacity + 1))
    step = S.FrameStep(policy, S.MISS_HOLD_PREVIOUS, n, margin_us, period_us, cal.cost, S.SUBMIT_EVERY)
    pacer = Pacer(period_us)
    runs_per_frame, frame_wall_us, deliveries, misses, spent = [], [], [], [], []
    tags: dict[int, list] = {}
    # First use (packing the weights) before the loop, as the reference's
    # engine warms up before its first frame.
    prep.run(0)
    ctx.synchronize()
    allocs = ctx.allocations()
    packs = prep.kernels.packs_made()

    def absorb_ready():
        for frame, slices, render in timer.collect(render=True):
            owners = tags.pop(frame, [])
            compute = []
            for tag, us in slices:
                job, slice_id, planned = owners[tag]
                compute.append(S.TimedSlice(job, slice_id, int(round(us)), planned))
            step.absorb(frame, compute, None if render is None else int(round(render)))

    try:
        for f in range(frames):
            index, start = pacer.next()
            began = time.perf_counter()
            planned = step.plan(S.Frame(index, index * period_us, period_us), index % owed_every == 0)
            spent.append(planned.plan.spent_estimate)
            timer.begin_frame(index)
            owners = []
            for r in planned.plan.runs:
                owners.append((r.job, r.slice, step.tag(r.slice)))
                prep.kernels.encode(r.slice, r.job % slots, timer, len(owners) - 1)
            tags[index] = owners
            # The render pass, timed apart from the compute passes.
            timer.render_begin()
            ctx.spin(render_us)
            timer.render_end()
            timer.submitted(timer.resolve())
            step.after_submit(index)
            absorb_ready()
            plan = step.complete(index)
            runs_per_frame.append(len(plan.runs))
            deliveries += [(d.job, index) for d in plan.delivered]
            misses += [(m.job, index) for m in plan.missed]
            frame_wall_us.append((time.perf_counter() - began) * 1e6)
        ctx.synchronize()
        absorb_ready()
        tally = step.finish()
        stats = timer.stats()
        assert ctx.allocations() == allocs, "the frame loop allocated device memory"
        assert prep.kernels.packs_made() == packs, "the frame loop repacked weights"
        outs = [prep.read(output_tid, slot=j).astype(np.float32) for j in range(slots)]
    finally:
        timer.close()
        _release(prep)
    if inputs is not None and slot_inputs is not None:
        wants = reference_outputs(ctx, graph, values, output_tid, dtype, input_tid, inputs)
    else:
        wants = [cal.reference_output] * slots
    err = max(float(np.max(np.abs(o - w))) for o, w in zip(outs, wants))
    split_kernels = sum(1 for p in cal.parts if p > 1)
    kind = {S.POLICY_FIXED_LATENCY: f"FixedLatency {policy.frames}", S.POLICY_SAME_FRAME: "SameFrame",
            S.POLICY_ON_BEAT: f"OnBeat (beat {policy.grid_beat} us, margin {policy.margin} us)"}[policy.kind]
    return {
        "workload": "frame-budget slices at a fixed frame period beside a fixed-time render load, "
                    "driven by the host's frame step",
        "policy": kind,
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
        "job_slots": slots,
        "submit": "every frame" if owed_every == 1 else f"every {owed_every} frames",
        "frames": frames,
        "slices_per_frame": {
            "mean": round(statistics.mean(runs_per_frame), 2),
            "min": min(runs_per_frame),
            "max": max(runs_per_frame),
        },
        "spent_estimate_us_per_frame_max": max(spent),
        "frame_wall_us_median": round(statistics.median(frame_wall_us), 1),
        "submitted": int(tally.submitted),
        "delivered": int(tally.delivered),
        "missed": int(tally.missed),
        "startup_missed": int(tally.startup_missed),
        "latency_violations": int(tally.violations),
        "pending_at_end": int(tally.pending_at_end),
        "latencies_frames": sorted(set(int(x) for x in tally.latencies)),
        "dispatches_per_job": sorted(set(int(x) for x in tally.dispatches_per_job)),
        "gpu_frame_us_median": round(statistics.median(tally.gpu_frame_us), 1) if tally.gpu_frame_us else None,
        "longest_dispatch_us_max": max(tally.longest_dispatch_us) if tally.longest_dispatch_us else None,
        "deliveries": deliveries,
        "misses": misses,
        "dropped_periods": pacer.dropped,
        "timer": {"frames_timed": int(stats.frames_timed), "frames_skipped": int(stats.frames_skipped),
                  "frames_failed": int(stats.frames_failed), "frames_dropped": int(stats.frames_dropped)},
        "output_max_abs_vs_unsplit": err,
        "output_within_tolerance": bool(err <= tolerance),
    }
