"""ctypes binding of the slice scheduler, its cost model and the host's frame
step (include/beatlm_schedule.h), shaped like the reference's API:
`Budget::for_frame` (crates/beatlm-core/src/budget.rs:32), `CostModel` with
its four estimators (cost.rs:339-966), `BeatGrid`/`BeatMap`
(time.rs:158-260), `SyncPolicy` (sync.rs), `Scheduler` with the
FixedLatency / SameFrame / OnBeat policies (schedule.rs:525-785), and the
host's `RenderCost` and `FrameStep` (beatlm-host/src/frame.rs:89-283,
step.rs:78-540).

Times are integer microseconds and frames integer indices. The logic lives in
the native library; this module only converts.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from .hip import lib

OK = 0
ERR_INVALID = -1
ERR_EMPTY_JOB = -2
ERR_INVALID_WINDOW = -3
ERR_INVALID_QUANTILE = -4
ERR_NO_SUCH_JOB = -5
ERR_INVALID_ALPHA = -6
ERR_INVALID_SIGMAS = -7
ERR_INVALID_CAP = -8
ERR_INVALID_FRAME_WINDOW = -9
ERR_NOT_ON_BEAT = -10
ERR_ZERO_BEAT = -11
ERR_NOT_COUNTED = -12
ERR_NOT_PLANNED = -13
ERR_FINISHED = -14
MISS_HOLD_PREVIOUS = 0
MISS_DROP = 1
MAX_WINDOW = 4096
WARM_SAMPLES = 5
TIMER_MAX_SLICES = 4096
RENDER_PRIOR = 2000
RENDER_WINDOW = 32
STARTUP_FRAMES = 64

EST_MEAN_PLUS_SIGMAS = 0
EST_WINDOWED_QUANTILE = 1
EST_CAPPED_DEVIATION = 2
EST_FRAME_SCALED = 3
SCALE_NONE = 0
SCALE_WARMING_UP = 1
SCALE_MEASURED = 2
POLICY_FIXED_LATENCY = 0
POLICY_SAME_FRAME = 1
POLICY_ON_BEAT = 2
DUE_FRAME = 0
DUE_BEAT = 1
SUBMIT_EVERY = 0
SUBMIT_FREE = 1
IN_FLIGHT_LATENCY = 0
IN_FLIGHT_BOUNDED = 1

_ERRORS = {
    ERR_INVALID: "invalid argument",
    ERR_EMPTY_JOB: "a job needs at least one slice",
    ERR_INVALID_WINDOW: "window must be in 1..=4096",
    ERR_INVALID_QUANTILE: "quantile must be a finite value in [0, 1]",
    ERR_NO_SUCH_JOB: "no such pending job",
    ERR_INVALID_ALPHA: "alpha must be a finite value in (0, 1]",
    ERR_INVALID_SIGMAS: "sigmas must be finite and not negative",
    ERR_INVALID_CAP: "cap must be finite and not negative",
    ERR_INVALID_FRAME_WINDOW: "frame window must be in 1..=4096",
    ERR_NOT_ON_BEAT: "the scheduler's policy is not OnBeat",
    ERR_ZERO_BEAT: "a beat grid needs a beat longer than zero",
    ERR_NOT_COUNTED: "the frame planned before was never counted (after_submit)",
    ERR_NOT_PLANNED: "no such planned frame",
    ERR_FINISHED: "the step is finished",
}


class ScheduleError(ValueError):
    def __init__(self, code: int):
        self.code = code
        super().__init__(_ERRORS.get(code, str(code)))


def _check(rc: int) -> None:
    if rc != OK:
        raise ScheduleError(rc)


class Frame(C.Structure):
    _fields_ = [("index", C.c_uint64), ("start", C.c_uint64), ("period", C.c_uint64)]


class _Estimator(C.Structure):
    _fields_ = [
        ("kind", C.c_uint32), ("window", C.c_uint32), ("frame_window", C.c_uint32), ("reserved", C.c_uint32),
        ("alpha", C.c_double), ("sigmas", C.c_double), ("cap", C.c_double), ("quantile", C.c_double),
    ]


class _FrameScale(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("reserved", C.c_uint32), ("recorded", C.c_uint64),
                ("needed", C.c_uint64), ("scale", C.c_double)]


class _Policy(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("frames", C.c_uint32), ("margin", C.c_uint64),
                ("grid_origin", C.c_uint64), ("grid_beat", C.c_uint64)]


class _Due(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("reserved", C.c_uint32), ("at", C.c_uint64)]


class _Run(C.Structure):
    _fields_ = [("job", C.c_uint64), ("slice", C.c_uint32), ("position", C.c_uint32)]


class _Delivery(C.Structure):
    _fields_ = [("job", C.c_uint64), ("input", C.c_uint64)]


class _Missed(C.Structure):
    _fields_ = [("job", C.c_uint64), ("input", C.c_uint64), ("due", _Due),
                ("policy", C.c_uint32), ("reserved", C.c_uint32)]


class _Plan(C.Structure):
    _fields_ = [
        ("n_runs", C.c_uint32), ("n_delivered", C.c_uint32), ("n_missed", C.c_uint32), ("reserved", C.c_uint32),
        ("runs", C.POINTER(_Run)), ("delivered", C.POINTER(_Delivery)), ("missed", C.POINTER(_Missed)),
        ("spent_estimate", C.c_uint64), ("budget", C.c_uint64),
    ]


class _StepConfig(C.Structure):
    _fields_ = [("policy", _Policy), ("miss", C.c_uint32), ("slices", C.c_uint32), ("margin", C.c_uint64),
                ("prior_period", C.c_uint64), ("submit", C.c_uint32), ("reserved", C.c_uint32)]


class _Planned(C.Structure):
    _fields_ = [("frame", Frame), ("plan", _Plan), ("job", C.c_uint64), ("has_job", C.c_uint32),
                ("has_due", C.c_uint32), ("due", _Due), ("budget", C.c_uint64), ("expected", C.c_uint64)]


class _TimedSlice(C.Structure):
    _fields_ = [("job", C.c_uint64), ("slice", C.c_uint32), ("has_planned", C.c_uint32),
                ("planned", C.c_uint64), ("duration", C.c_uint64)]


class _FrameTiming(C.Structure):
    _fields_ = [("frame", C.c_uint64), ("compute", C.POINTER(_TimedSlice)), ("n_compute", C.c_uint32),
                ("has_render", C.c_uint32), ("render", C.c_uint64)]


class _Absorbed(C.Structure):
    _fields_ = [("frame", C.c_uint64), ("has_render", C.c_uint32), ("ran_slices", C.c_uint32),
                ("render", C.c_uint64)]


class _SliceMeasured(C.Structure):
    _fields_ = [("slice", C.c_uint32), ("reserved", C.c_uint32), ("sum", C.c_uint64), ("count", C.c_uint64)]


class _SliceEstimate(C.Structure):
    _fields_ = [("slice", C.c_uint32), ("reserved", C.c_uint32), ("estimate", C.c_uint64)]


_P64 = C.POINTER(C.c_uint64)


class _Tally(C.Structure):
    _fields_ = [
        ("submitted", C.c_uint64), ("delivered", C.c_uint64), ("missed", C.c_uint64),
        ("startup_missed", C.c_uint64), ("violations", C.c_uint64), ("pending_at_end", C.c_uint64),
        ("n_latencies", C.c_uint64), ("n_dispatches_per_frame", C.c_uint64), ("n_dispatches_per_job", C.c_uint64),
        ("n_gpu_frame_us", C.c_uint64), ("n_longest_dispatch_us", C.c_uint64),
        ("latencies", _P64), ("dispatches_per_frame", _P64), ("dispatches_per_job", _P64),
        ("gpu_frame_us", _P64), ("longest_dispatch_us", _P64),
        ("n_measured", C.c_uint64), ("n_estimates", C.c_uint64), ("n_frame_ratios", C.c_uint64),
        ("n_frame_scales", C.c_uint64),
        ("measured", C.POINTER(_SliceMeasured)), ("estimates", C.POINTER(_SliceEstimate)),
        ("frame_ratios", C.POINTER(C.c_double)), ("frame_scales", C.POINTER(C.c_double)),
        ("frame_scale", _FrameScale), ("frames_recorded", C.c_uint64), ("timed_frames", C.c_uint64),
    ]


_VP = C.c_void_p
_U64 = C.c_uint64
_U32 = C.c_uint32
_I = C.c_int
_PU32 = C.POINTER(_U32)
_SIG = {
    "bls_budget_for_frame": (_U64, [_U64, _U64, _U64]),
    "bls_nearest_rank": (_U32, [C.c_double, _U32]),
    "bls_cost_new": (_I, [_U64, _U32, C.c_double, C.POINTER(_VP)]),
    "bls_cost_new_with": (_I, [_U64, C.POINTER(_Estimator), C.POINTER(_VP)]),
    "bls_cost_clone": (_I, [_VP, C.POINTER(_VP)]),
    "bls_cost_free": (None, [_VP]),
    "bls_cost_estimator": (None, [_VP, C.POINTER(_Estimator)]),
    "bls_cost_record": (None, [_VP, _U32, _U64]),
    "bls_cost_record_calibration": (None, [_VP, _U32, _U64]),
    "bls_cost_estimate": (_U64, [_VP, _U32]),
    "bls_cost_planning_estimate": (_U64, [_VP, _U32]),
    "bls_cost_samples": (_U32, [_VP, _U32]),
    "bls_cost_frame_estimate": (_I, [_VP, _U32, _P64]),
    "bls_cost_record_frame": (None, [_VP, _U64, _U64]),
    "bls_cost_frame_scale": (None, [_VP, C.POINTER(_FrameScale)]),
    "bls_cost_frames_recorded": (_U64, [_VP]),
    "bls_beat_grid_next": (_I, [_U64, _U64, _U64, _P64]),
    "bls_beat_map_new": (_I, [_U64, _U64, C.POINTER(_VP)]),
    "bls_beat_map_free": (None, [_VP]),
    "bls_beat_map_replace_from": (_I, [_VP, _U64, _U64, _U64]),
    "bls_beat_map_next": (_U64, [_VP, _U64]),
    "bls_beat_map_forget_before": (None, [_VP, _U64]),
    "bls_beat_map_grids": (_U32, [_VP]),
    "bls_policy_source_delay": (_I, [C.POINTER(_Policy), _PU32]),
    "bls_policy_max_in_flight": (_I, [C.POINTER(_Policy), _PU32]),
    "bls_scheduler_new": (_I, [_U32, _U32, _U64, C.POINTER(_VP)]),
    "bls_scheduler_new_policy": (_I, [C.POINTER(_Policy), _U32, _U64, C.POINTER(_VP)]),
    "bls_scheduler_free": (None, [_VP]),
    "bls_scheduler_set_expected_budget": (None, [_VP, _U64]),
    "bls_scheduler_expected_budget": (_U64, [_VP]),
    "bls_scheduler_replace_beat_grid": (_I, [_VP, _U64, _U64, _U64]),
    "bls_scheduler_submit": (_I, [_VP, C.POINTER(Frame), _PU32, _U32, _VP, _P64]),
    "bls_scheduler_plan_frame": (_I, [_VP, C.POINTER(Frame), _U64, _VP, C.POINTER(_Plan)]),
    "bls_scheduler_pending": (_U32, [_VP]),
    "bls_scheduler_due": (_I, [_VP, _U64, C.POINTER(_Due)]),
    "bls_render_cost_new": (_I, [C.POINTER(_VP)]),
    "bls_render_cost_free": (None, [_VP]),
    "bls_render_cost_record": (None, [_VP, _U64]),
    "bls_render_cost_last": (_U64, [_VP]),
    "bls_render_cost_forecast": (_U64, [_VP]),
    "bls_render_cost_budget": (_U64, [_VP, _U64, _U64]),
    "bls_render_cost_expected": (_U64, [_VP, _U64, _U64]),
    "bls_timer_capacity": (_I, [_U32, _U32, _PU32]),
    "bls_jobs_with_slices": (_I, [_U32, _U32, _U32, _PU32]),
    "bls_step_new": (_I, [C.POINTER(_StepConfig), _VP, C.POINTER(_VP)]),
    "bls_step_free": (None, [_VP]),
    "bls_step_replace_beat_grid": (_I, [_VP, _U64, _U64, _U64]),
    "bls_step_cost": (_VP, [_VP]),
    "bls_step_submitted": (_U64, [_VP]),
    "bls_step_dispatched": (_U64, [_VP, _U64]),
    "bls_step_plan": (_I, [_VP, C.POINTER(Frame), _I, C.POINTER(_Planned), _P64]),
    "bls_step_tag": (_I, [_VP, _U32, _P64]),
    "bls_step_after_submit": (_I, [_VP, _U64]),
    "bls_step_absorb": (_I, [_VP, C.POINTER(_FrameTiming), C.POINTER(_Absorbed)]),
    "bls_step_complete": (_I, [_VP, _U64, C.POINTER(_Plan)]),
    "bls_step_finish": (_I, [_VP, C.POINTER(_Tally)]),
    "bls_collect_action": (_U32, [_U32, _U32]),
    "bls_ring_new": (_I, [_U32, C.POINTER(_VP)]),
    "bls_ring_free": (None, [_VP]),
    "bls_ring_depth": (_U32, [_VP]),
    "bls_ring_claim": (C.c_int32, [_VP]),
    "bls_ring_encode": (_U64, [_VP, _U32]),
    "bls_ring_submit": (C.c_int32, [_VP, _U64]),
    "bls_ring_submit_held": (C.c_int32, [_VP, _U64, _P64]),
    "bls_ticket_drop": (None, [_U64]),
    "bls_hold_verdict": (_I, [_U64, _U32]),
    "bls_ring_settle": (None, [_VP]),
    "bls_ring_invalidate": (_U32, [_VP]),
    "bls_ring_ready": (_U32, [_VP, C.POINTER(C.c_uint8), _PU32, C.POINTER(C.c_uint8)]),
    "bls_ring_release": (None, [_VP, _U32]),
    "bls_ring_in_flight": (_U32, [_VP]),
    "bls_ring_phase": (C.c_int32, [_VP, _U32]),
    "bls_ring_reclaimed": (_U64, [_VP]),
}
_bound = False


def _lib():
    global _bound
    h = lib()
    if not _bound:
        for name, (res, args) in _SIG.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _bound = True
    return h


def budget_for_frame(period: int, render: int, margin: int) -> int:
    """`Budget::for_frame`: period − render − margin, saturating at zero."""
    return int(_lib().bls_budget_for_frame(period, render, margin))


def nearest_rank(quantile: float, n: int) -> int:
    return int(_lib().bls_nearest_rank(quantile, n))


def frame(index: int, period: int, start: int | None = None) -> Frame:
    return Frame(index, index * period if start is None else start, period)


# ---- cost model --------------------------------------------------------------


@dataclass(frozen=True)
class Estimator:
    """`Estimator` (cost.rs:339-416). Build with the class methods."""

    kind: int
    window: int = 0
    frame_window: int = 0
    alpha: float = 0.0
    sigmas: float = 0.0
    cap: float = 0.0
    quantile: float = 0.0

    @classmethod
    def mean_plus_sigmas(cls, alpha: float, sigmas: float) -> "Estimator":
        return cls(EST_MEAN_PLUS_SIGMAS, alpha=alpha, sigmas=sigmas)

    @classmethod
    def windowed_quantile(cls, window: int, quantile: float) -> "Estimator":
        return cls(EST_WINDOWED_QUANTILE, window=window, quantile=quantile)

    @classmethod
    def capped_deviation(cls, alpha: float, sigmas: float, cap: float) -> "Estimator":
        return cls(EST_CAPPED_DEVIATION, alpha=alpha, sigmas=sigmas, cap=cap)

    @classmethod
    def frame_scaled(cls, window: int, frame_window: int, quantile: float) -> "Estimator":
        return cls(EST_FRAME_SCALED, window=window, frame_window=frame_window, quantile=quantile)

    def _c(self) -> _Estimator:
        return _Estimator(self.kind, self.window, self.frame_window, 0, self.alpha, self.sigmas, self.cap,
                          self.quantile)


@dataclass(frozen=True)
class FrameScale:
    """`FrameScale`: None (another estimator), WarmingUp{recorded, needed}
    or Measured(scale)."""

    kind: int
    recorded: int = 0
    needed: int = 0
    scale: float = 0.0


def _scale(f: _FrameScale) -> FrameScale:
    if f.kind == SCALE_WARMING_UP:
        return FrameScale(SCALE_WARMING_UP, recorded=int(f.recorded), needed=int(f.needed))
    if f.kind == SCALE_MEASURED:
        return FrameScale(SCALE_MEASURED, scale=float(f.scale))
    return FrameScale(SCALE_NONE)


class CostModel:
    """Per-slice cost estimates: the prior until a slice is measured, then
    what the estimator reads from its measurements. The default is the
    windowed quantile (the `quantile` nearest rank of the last `window`)."""

    def __init__(self, prior: int, window: int = 32, quantile: float = 0.9, estimator: Estimator | None = None,
                 _handle=None):
        if _handle is not None:
            self.handle = _handle
            self._owned = False
            return
        est = estimator or Estimator.windowed_quantile(window, quantile)
        h = C.c_void_p()
        _check(_lib().bls_cost_new_with(prior, C.byref(est._c()), C.byref(h)))
        self.handle = h
        self._owned = True

    def clone(self) -> "CostModel":
        h = C.c_void_p()
        _check(_lib().bls_cost_clone(self.handle, C.byref(h)))
        return CostModel(0, _handle=h)._own()

    def _own(self) -> "CostModel":
        self._owned = True
        return self

    def estimator(self) -> Estimator:
        e = _Estimator()
        _lib().bls_cost_estimator(self.handle, C.byref(e))
        return Estimator(e.kind, e.window, e.frame_window, e.alpha, e.sigmas, e.cap, e.quantile)

    def record(self, slice_id: int, measured: int) -> None:
        _lib().bls_cost_record(self.handle, slice_id, measured)

    def record_calibration(self, slice_id: int, measured: int) -> None:
        _lib().bls_cost_record_calibration(self.handle, slice_id, measured)

    def estimate(self, slice_id: int) -> int:
        return int(_lib().bls_cost_estimate(self.handle, slice_id))

    def planning_estimate(self, slice_id: int) -> int:
        return int(_lib().bls_cost_planning_estimate(self.handle, slice_id))

    def samples(self, slice_id: int) -> int:
        return int(_lib().bls_cost_samples(self.handle, slice_id))

    def frame_estimate(self, slice_id: int):
        v = C.c_uint64()
        return int(v.value) if _lib().bls_cost_frame_estimate(self.handle, slice_id, C.byref(v)) else None

    def record_frame(self, predicted: int, measured: int) -> None:
        _lib().bls_cost_record_frame(self.handle, predicted, measured)

    def frame_scale(self) -> FrameScale:
        f = _FrameScale()
        _lib().bls_cost_frame_scale(self.handle, C.byref(f))
        return _scale(f)

    def frames_recorded(self) -> int:
        return int(_lib().bls_cost_frames_recorded(self.handle))

    def __del__(self):
        if getattr(self, "handle", None) and getattr(self, "_owned", False):
            _lib().bls_cost_free(self.handle)
        self.handle = None


# ---- beats ---------------------------------------------------------------------


def beat_grid_next(origin: int, beat: int, t: int) -> int:
    """`BeatGrid::next_beat_at_or_after` for the grid (origin, beat)."""
    v = C.c_uint64()
    _check(_lib().bls_beat_grid_next(origin, beat, t, C.byref(v)))
    return int(v.value)


class BeatMap:
    """`BeatMap`: beat grids each in effect from its `from` instant."""

    def __init__(self, origin: int, beat: int):
        h = C.c_void_p()
        _check(_lib().bls_beat_map_new(origin, beat, C.byref(h)))
        self.handle = h

    def replace_from(self, from_: int, origin: int, beat: int) -> None:
        _check(_lib().bls_beat_map_replace_from(self.handle, from_, origin, beat))

    def next_beat_at_or_after(self, t: int) -> int:
        return int(_lib().bls_beat_map_next(self.handle, t))

    def forget_before(self, t: int) -> None:
        _lib().bls_beat_map_forget_before(self.handle, t)

    def grids(self) -> int:
        return int(_lib().bls_beat_map_grids(self.handle))

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_beat_map_free(self.handle)
            self.handle = None


# ---- policies and the scheduler ----------------------------------------------


@dataclass(frozen=True)
class Policy:
    """`SyncPolicy`: FixedLatency{frames}, SameFrame, OnBeat{grid, margin}."""

    kind: int
    frames: int = 0
    margin: int = 0
    grid_origin: int = 0
    grid_beat: int = 0

    @classmethod
    def fixed_latency(cls, frames: int) -> "Policy":
        return cls(POLICY_FIXED_LATENCY, frames=frames)

    @classmethod
    def same_frame(cls) -> "Policy":
        return cls(POLICY_SAME_FRAME)

    @classmethod
    def on_beat(cls, origin: int, beat: int, margin: int) -> "Policy":
        return cls(POLICY_ON_BEAT, margin=margin, grid_origin=origin, grid_beat=beat)

    def _c(self) -> _Policy:
        return _Policy(self.kind, self.frames, self.margin, self.grid_origin, self.grid_beat)

    def source_delay(self):
        v = C.c_uint32()
        return int(v.value) if _lib().bls_policy_source_delay(C.byref(self._c()), C.byref(v)) else None

    def max_in_flight(self):
        v = C.c_uint32()
        return int(v.value) if _lib().bls_policy_max_in_flight(C.byref(self._c()), C.byref(v)) else None


@dataclass(frozen=True)
class Due:
    """`Due`: a frame index (Frame) or an instant (Beat)."""

    kind: int
    at: int

    @classmethod
    def frame(cls, index: int) -> "Due":
        return cls(DUE_FRAME, index)

    @classmethod
    def beat(cls, t: int) -> "Due":
        return cls(DUE_BEAT, t)


def _due(d: _Due) -> Due:
    return Due(int(d.kind), int(d.at))


@dataclass(frozen=True)
class Run:
    job: int
    slice: int
    position: int


@dataclass(frozen=True)
class Delivery:
    job: int
    input: int


@dataclass(frozen=True)
class Missed:
    job: int
    input: int
    due: Due
    policy: int


@dataclass
class FramePlan:
    runs: list = field(default_factory=list)
    delivered: list = field(default_factory=list)
    missed: list = field(default_factory=list)
    spent_estimate: int = 0
    budget: int = 0


def _plan(p: _Plan) -> FramePlan:
    return FramePlan(
        runs=[Run(p.runs[i].job, p.runs[i].slice, p.runs[i].position) for i in range(p.n_runs)],
        delivered=[Delivery(p.delivered[i].job, p.delivered[i].input) for i in range(p.n_delivered)],
        missed=[Missed(p.missed[i].job, p.missed[i].input, _due(p.missed[i].due), p.missed[i].policy)
                for i in range(p.n_missed)],
        spent_estimate=int(p.spent_estimate),
        budget=int(p.budget),
    )


class Scheduler:
    """Jobs run in submission order inside each frame's budget. Built from a
    latency in frames (FixedLatency; SameFrame is 0) or from a `Policy`."""

    def __init__(self, latency_frames: int | Policy, miss: int, expected_budget: int):
        h = C.c_void_p()
        if isinstance(latency_frames, Policy):
            _check(_lib().bls_scheduler_new_policy(C.byref(latency_frames._c()), miss, expected_budget,
                                                   C.byref(h)))
        else:
            _check(_lib().bls_scheduler_new(latency_frames, miss, expected_budget, C.byref(h)))
        self.handle = h

    def set_expected_budget(self, expected: int) -> None:
        _lib().bls_scheduler_set_expected_budget(self.handle, expected)

    def expected_budget(self) -> int:
        return int(_lib().bls_scheduler_expected_budget(self.handle))

    def replace_beat_grid(self, from_: int, origin: int, beat: int) -> None:
        _check(_lib().bls_scheduler_replace_beat_grid(self.handle, from_, origin, beat))

    def submit(self, input_frame: Frame, slices, cost: CostModel) -> int:
        arr = (C.c_uint32 * max(len(slices), 1))(*slices)
        job = C.c_uint64()
        _check(_lib().bls_scheduler_submit(self.handle, C.byref(input_frame), arr, len(slices), cost.handle,
                                           C.byref(job)))
        return int(job.value)

    def plan_frame(self, f: Frame, budget: int, cost: CostModel) -> FramePlan:
        p = _Plan()
        _check(_lib().bls_scheduler_plan_frame(self.handle, C.byref(f), budget, cost.handle, C.byref(p)))
        return _plan(p)

    def pending(self) -> int:
        return int(_lib().bls_scheduler_pending(self.handle))

    def due(self, job: int):
        d = _Due()
        return _due(d) if _lib().bls_scheduler_due(self.handle, job, C.byref(d)) == OK else None

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_scheduler_free(self.handle)
            self.handle = None


# ---- the host's frame step ------------------------------------------------------


class RenderCost:
    """`RenderCost` (frame.rs:89-158): the budget reads the render measured
    last, the expected budget the upper median of the last 32."""

    def __init__(self):
        h = C.c_void_p()
        _check(_lib().bls_render_cost_new(C.byref(h)))
        self.handle = h

    def record(self, render: int) -> None:
        _lib().bls_render_cost_record(self.handle, render)

    def last(self) -> int:
        return int(_lib().bls_render_cost_last(self.handle))

    def forecast(self) -> int:
        return int(_lib().bls_render_cost_forecast(self.handle))

    def budget(self, period: int, margin: int) -> int:
        return int(_lib().bls_render_cost_budget(self.handle, period, margin))

    def expected(self, period: int, margin: int) -> int:
        return int(_lib().bls_render_cost_expected(self.handle, period, margin))

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_render_cost_free(self.handle)
            self.handle = None


def timer_capacity(slices: int, jobs: int):
    v = C.c_uint32()
    return int(v.value) if _lib().bls_timer_capacity(slices, jobs, C.byref(v)) else None


def jobs_with_slices(submit: int, in_flight_kind: int, in_flight: int):
    v = C.c_uint32()
    return int(v.value) if _lib().bls_jobs_with_slices(submit, in_flight_kind, in_flight, C.byref(v)) else None


@dataclass(frozen=True)
class TimedSlice:
    job: int
    slice: int
    duration: int
    planned: int | None = None


@dataclass
class Planned:
    frame: Frame
    plan: FramePlan
    job: int | None
    due: Due | None
    budget: int
    expected: int


@dataclass
class Tally:
    submitted: int
    delivered: int
    missed: int
    startup_missed: int
    violations: int
    pending_at_end: int
    latencies: list
    dispatches_per_frame: list
    dispatches_per_job: list
    gpu_frame_us: list
    longest_dispatch_us: list
    measured: dict
    estimates: dict
    frame_ratios: list
    frame_scales: list
    frame_scale: FrameScale
    frames_recorded: int
    timed_frames: int


class FrameStep:
    """`FrameStep` (beatlm-host/src/step.rs:78-540): plan a frame, count what
    was submitted, absorb the timings that come back, count the frame's
    deliveries and misses, and close the run into a tally."""

    def __init__(self, policy: Policy, miss: int, slices: int, margin: int, prior_period: int,
                 cost: CostModel, submit: int = SUBMIT_EVERY):
        cfg = _StepConfig(policy._c(), miss, slices, margin, prior_period, submit, 0)
        h = C.c_void_p()
        _check(_lib().bls_step_new(C.byref(cfg), cost.handle, C.byref(h)))
        self.handle = h

    def replace_beat_grid(self, from_: int, origin: int, beat: int) -> None:
        _check(_lib().bls_step_replace_beat_grid(self.handle, from_, origin, beat))

    def cost(self) -> CostModel:
        """The step's cost model (a view that lives as long as the step)."""
        view = CostModel(0, _handle=C.c_void_p(_lib().bls_step_cost(self.handle)))
        view._keep = self
        return view

    def submitted(self) -> int:
        return int(_lib().bls_step_submitted(self.handle))

    def dispatched(self, job: int) -> int:
        return int(_lib().bls_step_dispatched(self.handle, job))

    def plan(self, f: Frame, owed: bool) -> Planned:
        out = _Planned()
        un = C.c_uint64()
        rc = _lib().bls_step_plan(self.handle, C.byref(f), 1 if owed else 0, C.byref(out), C.byref(un))
        if rc == ERR_NOT_COUNTED:
            e = ScheduleError(rc)
            e.unsubmitted = int(un.value)
            raise e
        _check(rc)
        return Planned(
            frame=Frame(out.frame.index, out.frame.start, out.frame.period),
            plan=_plan(out.plan),
            job=int(out.job) if out.has_job else None,
            due=_due(out.due) if out.has_due else None,
            budget=int(out.budget),
            expected=int(out.expected),
        )

    def tag(self, slice_id: int):
        v = C.c_uint64()
        return int(v.value) if _lib().bls_step_tag(self.handle, slice_id, C.byref(v)) else None

    def after_submit(self, frame_index: int) -> None:
        _check(_lib().bls_step_after_submit(self.handle, frame_index))

    def absorb(self, frame_index: int, compute, render: int | None):
        arr = (_TimedSlice * max(len(compute), 1))(
            *[_TimedSlice(c.job, c.slice, 0 if c.planned is None else 1, c.planned or 0, c.duration)
              for c in compute])
        t = _FrameTiming(frame_index, arr, len(compute), 0 if render is None else 1, render or 0)
        out = _Absorbed()
        _check(_lib().bls_step_absorb(self.handle, C.byref(t), C.byref(out)))
        return int(out.frame), (int(out.render) if out.has_render else None), bool(out.ran_slices)

    def complete(self, frame_index: int) -> FramePlan:
        p = _Plan()
        _check(_lib().bls_step_complete(self.handle, frame_index, C.byref(p)))
        return _plan(p)

    def finish(self) -> Tally:
        t = _Tally()
        _check(_lib().bls_step_finish(self.handle, C.byref(t)))

        def arr(ptr, n):
            return [ptr[i] for i in range(n)]

        return Tally(
            submitted=int(t.submitted), delivered=int(t.delivered), missed=int(t.missed),
            startup_missed=int(t.startup_missed), violations=int(t.violations),
            pending_at_end=int(t.pending_at_end),
            latencies=arr(t.latencies, t.n_latencies),
            dispatches_per_frame=arr(t.dispatches_per_frame, t.n_dispatches_per_frame),
            dispatches_per_job=arr(t.dispatches_per_job, t.n_dispatches_per_job),
            gpu_frame_us=arr(t.gpu_frame_us, t.n_gpu_frame_us),
            longest_dispatch_us=arr(t.longest_dispatch_us, t.n_longest_dispatch_us),
            measured={t.measured[i].slice: (int(t.measured[i].sum), int(t.measured[i].count))
                      for i in range(t.n_measured)},
            estimates={t.estimates[i].slice: int(t.estimates[i].estimate) for i in range(t.n_estimates)},
            frame_ratios=arr(t.frame_ratios, t.n_frame_ratios),
            frame_scales=arr(t.frame_scales, t.n_frame_scales),
            frame_scale=_scale(t.frame_scale),
            frames_recorded=int(t.frames_recorded),
            timed_frames=int(t.timed_frames),
        )

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_step_free(self.handle)
            self.handle = None


# ---- the slice timer's ring (crates/beatlm/src/gpu/ring.rs) ------------------

PHASE_FREE, PHASE_RECORDING, PHASE_ENCODED, PHASE_SUBMITTED, PHASE_HELD, PHASE_INVALID = range(6)
DONE_PENDING, DONE_OK, DONE_FAILED = range(3)
COLLECT_WAIT, COLLECT_READ, COLLECT_DROP = range(3)
RING_MAX_DEPTH = 64


def collect_action(phase: int, done: int) -> int:
    """`collect` (ring.rs:98-111): what collecting a slot does now."""
    return int(_lib().bls_collect_action(phase, done))


def drop_ticket(ticket: int) -> None:
    """Dropping a `Ticket`: its slot is freed unread at its ring's next claim."""
    _lib().bls_ticket_drop(ticket)


def verdict(hold: int, accepted: bool) -> bool:
    """`Verdict::accept` / `reject`; False when it reached no held slot."""
    return bool(_lib().bls_hold_verdict(hold, 1 if accepted else 0))


class Ring:
    """`Ring` (ring.rs:184-412). Tickets and holds are ints (never 0); a
    method that gives None where the reference gives None."""

    def __init__(self, depth: int):
        h = _VP()
        _check(_lib().bls_ring_new(depth, C.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            _lib().bls_ring_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def depth(self) -> int:
        return int(_lib().bls_ring_depth(self.handle))

    def claim(self) -> int | None:
        s = _lib().bls_ring_claim(self.handle)
        return None if s < 0 else int(s)

    def encode(self, slot: int) -> int | None:
        t = _lib().bls_ring_encode(self.handle, slot)
        return None if t == 0 else int(t)

    def submit(self, ticket: int) -> int | None:
        s = _lib().bls_ring_submit(self.handle, ticket)
        return None if s < 0 else int(s)

    def submit_held(self, ticket: int) -> tuple[int, int] | None:
        h = C.c_uint64()
        s = _lib().bls_ring_submit_held(self.handle, ticket, C.byref(h))
        return None if s < 0 else (int(s), int(h.value))

    def settle(self) -> None:
        _lib().bls_ring_settle(self.handle)

    def invalidate(self) -> int:
        return int(_lib().bls_ring_invalidate(self.handle))

    def ready(self, done) -> list[tuple[int, int]]:
        """(slot, COLLECT_*) pairs to collect now, oldest submission first;
        `done(slot)` gives DONE_* for each slot."""
        n = self.depth()
        d = (C.c_uint8 * n)(*[done(i) for i in range(n)])
        slots = (C.c_uint32 * n)()
        acts = (C.c_uint8 * n)()
        k = _lib().bls_ring_ready(self.handle, d, slots, acts)
        return [(int(slots[i]), int(acts[i])) for i in range(k)]

    def release(self, slot: int) -> None:
        _lib().bls_ring_release(self.handle, slot)

    def in_flight(self) -> int:
        return int(_lib().bls_ring_in_flight(self.handle))

    def phase(self, slot: int) -> int | None:
        p = _lib().bls_ring_phase(self.handle, slot)
        return None if p < 0 else int(p)

    def slots_in(self, phase: int) -> list[int]:
        return [i for i in range(self.depth()) if self.phase(i) == phase]

    def reclaimed(self) -> int:
        return int(_lib().bls_ring_reclaimed(self.handle))
