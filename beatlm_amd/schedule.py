"""ctypes binding of the slice scheduler and cost model
(include/beatlm_schedule.h), shaped like the reference core's API:
`Budget::for_frame` (crates/beatlm-core/src/budget.rs:32), `CostModel` with
the windowed-quantile estimator (cost.rs:748-966) and `Scheduler` with the
FixedLatency / SameFrame policies (schedule.rs:525-785).

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
MISS_HOLD_PREVIOUS = 0
MISS_DROP = 1
MAX_WINDOW = 4096

_ERRORS = {
    ERR_INVALID: "invalid argument",
    ERR_EMPTY_JOB: "a job needs at least one slice",
    ERR_INVALID_WINDOW: "window must be in 1..=4096",
    ERR_INVALID_QUANTILE: "quantile must be a finite value in [0, 1]",
    ERR_NO_SUCH_JOB: "no such pending job",
}


class ScheduleError(ValueError):
    def __init__(self, code: int):
        self.code = code
        super().__init__(_ERRORS.get(code, str(code)))


class Frame(C.Structure):
    _fields_ = [("index", C.c_uint64), ("start", C.c_uint64), ("period", C.c_uint64)]


class _Run(C.Structure):
    _fields_ = [("job", C.c_uint64), ("slice", C.c_uint32), ("position", C.c_uint32)]


class _Delivery(C.Structure):
    _fields_ = [("job", C.c_uint64), ("input", C.c_uint64)]


class _Missed(C.Structure):
    _fields_ = [("job", C.c_uint64), ("input", C.c_uint64), ("due_frame", C.c_uint64),
                ("policy", C.c_uint32), ("reserved", C.c_uint32)]


class _Plan(C.Structure):
    _fields_ = [
        ("n_runs", C.c_uint32), ("n_delivered", C.c_uint32), ("n_missed", C.c_uint32), ("reserved", C.c_uint32),
        ("runs", C.POINTER(_Run)), ("delivered", C.POINTER(_Delivery)), ("missed", C.POINTER(_Missed)),
        ("spent_estimate", C.c_uint64), ("budget", C.c_uint64),
    ]


_VP = C.c_void_p
_U64 = C.c_uint64
_U32 = C.c_uint32
_SIG = {
    "bls_budget_for_frame": (_U64, [_U64, _U64, _U64]),
    "bls_nearest_rank": (_U32, [C.c_double, _U32]),
    "bls_cost_new": (C.c_int, [_U64, _U32, C.c_double, C.POINTER(_VP)]),
    "bls_cost_free": (None, [_VP]),
    "bls_cost_record": (None, [_VP, _U32, _U64]),
    "bls_cost_record_calibration": (None, [_VP, _U32, _U64]),
    "bls_cost_estimate": (_U64, [_VP, _U32]),
    "bls_cost_planning_estimate": (_U64, [_VP, _U32]),
    "bls_cost_samples": (_U32, [_VP, _U32]),
    "bls_scheduler_new": (C.c_int, [_U32, _U32, _U64, C.POINTER(_VP)]),
    "bls_scheduler_free": (None, [_VP]),
    "bls_scheduler_set_expected_budget": (None, [_VP, _U64]),
    "bls_scheduler_expected_budget": (_U64, [_VP]),
    "bls_scheduler_submit": (C.c_int, [_VP, C.POINTER(Frame), C.POINTER(_U32), _U32, _VP, C.POINTER(_U64)]),
    "bls_scheduler_plan_frame": (C.c_int, [_VP, C.POINTER(Frame), _U64, _VP, C.POINTER(_Plan)]),
    "bls_scheduler_pending": (_U32, [_VP]),
    "bls_scheduler_due": (C.c_int, [_VP, _U64, C.POINTER(_U64)]),
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


class CostModel:
    """Per-slice cost estimates: the prior until a slice is measured, then
    the `quantile` nearest rank of its last `window` measurements."""

    def __init__(self, prior: int, window: int = 32, quantile: float = 0.9):
        h = C.c_void_p()
        rc = _lib().bls_cost_new(prior, window, quantile, C.byref(h))
        if rc != OK:
            raise ScheduleError(rc)
        self.handle = h

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

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_cost_free(self.handle)
            self.handle = None


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
    due: int
    policy: int


@dataclass
class FramePlan:
    runs: list = field(default_factory=list)
    delivered: list = field(default_factory=list)
    missed: list = field(default_factory=list)
    spent_estimate: int = 0
    budget: int = 0


class Scheduler:
    """FixedLatency { frames } (SameFrame is frames=0): jobs run in
    submission order, each due `frames` after its input frame."""

    def __init__(self, latency_frames: int, miss: int, expected_budget: int):
        h = C.c_void_p()
        rc = _lib().bls_scheduler_new(latency_frames, miss, expected_budget, C.byref(h))
        if rc != OK:
            raise ScheduleError(rc)
        self.handle = h

    def set_expected_budget(self, expected: int) -> None:
        _lib().bls_scheduler_set_expected_budget(self.handle, expected)

    def expected_budget(self) -> int:
        return int(_lib().bls_scheduler_expected_budget(self.handle))

    def submit(self, input_frame: Frame, slices, cost: CostModel) -> int:
        arr = (C.c_uint32 * max(len(slices), 1))(*slices)
        job = C.c_uint64()
        rc = _lib().bls_scheduler_submit(self.handle, C.byref(input_frame), arr, len(slices), cost.handle, C.byref(job))
        if rc != OK:
            raise ScheduleError(rc)
        return int(job.value)

    def plan_frame(self, f: Frame, budget: int, cost: CostModel) -> FramePlan:
        p = _Plan()
        rc = _lib().bls_scheduler_plan_frame(self.handle, C.byref(f), budget, cost.handle, C.byref(p))
        if rc != OK:
            raise ScheduleError(rc)
        return FramePlan(
            runs=[Run(p.runs[i].job, p.runs[i].slice, p.runs[i].position) for i in range(p.n_runs)],
            delivered=[Delivery(p.delivered[i].job, p.delivered[i].input) for i in range(p.n_delivered)],
            missed=[Missed(p.missed[i].job, p.missed[i].input, p.missed[i].due_frame, p.missed[i].policy)
                    for i in range(p.n_missed)],
            spent_estimate=int(p.spent_estimate),
            budget=int(p.budget),
        )

    def pending(self) -> int:
        return int(_lib().bls_scheduler_pending(self.handle))

    def due(self, job: int):
        d = C.c_uint64()
        return int(d.value) if _lib().bls_scheduler_due(self.handle, job, C.byref(d)) == OK else None

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bls_scheduler_free(self.handle)
            self.handle = None
