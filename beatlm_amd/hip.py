"""ctypes binding of the backend's C ABI (include/beatlm_hip.h).

This is host plumbing for tests and the bench: it loads the in-tree
libbeatlm_hip.so and fails loudly when it is missing. There is no other
implementation of the kernels to fall back to.
"""

from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libbeatlm_hip.so"

MAX_EPILOGUE = 8
MAX_BINDINGS = 8
RING_DEPTH = 3

# status codes
OK = 0
ERR_HIP = -1
ERR_INVALID_ARGUMENT = -2
ERR_PLAN_NOT_VALID_ON_DEVICE = -10
ERR_UNKNOWN_ARENA = -11
ERR_PLACEMENT_OUT_OF_RANGE = -12
ERR_MISALIGNED_PLACEMENT = -13
ERR_KERNEL = -20
ERR_MISSING_PLACEMENT = -21
ERR_STAND_IN_SIZE = -22
ERR_NO_SUCH_KERNEL = -23
ERR_NO_SUCH_SET = -24
ERR_TOO_LARGE = -25
ERR_TIMER_TOO_MANY_SLICES = -30
ERR_TIMER_NO_FRAME = -31
ERR_TIMER_CAPACITY = -32
ERR_TIMER_RENDER_TWICE = -33

# main operations
MAIN_LAYER_NORM = 1
MAIN_MATMUL = 2
MAIN_ATTENTION_SCORES = 3
MAIN_SOFTMAX = 4
MAIN_ATTENTION_VALUES = 5
MAIN_PATCH_EMBED = 6
MAIN_PREPEND_TOKEN = 7
MAIN_TOKENS_TO_MAP = 8
MAIN_MAP = 9
MAIN_CONV3X3 = 10
MAIN_CONV_TRANSPOSE = 11
MAIN_RESIZE_BILINEAR = 12
MAIN_FLASH_ATTENTION = 100
PRO_RELU = 1

# epilogue steps
EPI_ADD = 1
EPI_RELU = 2
EPI_GELU = 3
EPI_GELU_ERF = 4
EPI_SCALE = 5
EPI_CHANNEL_SCALE = 6

F32 = 0
F16 = 1

F32_MATH_SPLIT_BF16 = 0
F32_MATH_MFMA_F32 = 1


class Epilogue(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("factor", C.c_float), ("channels", C.c_uint32), ("operand", C.c_uint32)]


class Binding(C.Structure):
    _fields_ = [
        ("tensor", C.c_uint32),
        ("arena", C.c_uint32),
        ("offset", C.c_uint64),
        ("size", C.c_uint64),
        ("dtype", C.c_uint32),
        ("reserved", C.c_uint32),
    ]


class Part(C.Structure):
    _fields_ = [("index", C.c_uint32), ("count", C.c_uint32), ("start", C.c_uint32), ("end", C.c_uint32)]


class Spec(C.Structure):
    _fields_ = [
        ("main", C.c_uint32),
        ("dims", C.c_uint32 * 6),
        ("epsilon", C.c_float),
        ("scale", C.c_float),
        ("part", Part),
        ("n_reads", C.c_uint32),
        ("reads", C.c_uint32 * 4),
        ("n_epilogue", C.c_uint32),
        ("epilogue", Epilogue * MAX_EPILOGUE),
        ("n_bindings", C.c_uint32),
        ("bindings", Binding * MAX_BINDINGS),
        ("prologue", C.c_uint32),
    ]


class Substitution(C.Structure):
    _fields_ = [
        ("original", C.c_uint32),
        ("stand_in", C.c_uint32),
        ("arena", C.c_uint32),
        ("reserved", C.c_uint32),
        ("offset", C.c_uint64),
        ("size", C.c_uint64),
    ]


class BindingSet(C.Structure):
    _fields_ = [("items", C.POINTER(Substitution)), ("count", C.c_uint32)]


class DeviceProfile(C.Structure):
    _fields_ = [
        ("max_storage_buffer_binding_size", C.c_uint64),
        ("max_buffer_size", C.c_uint64),
        ("min_storage_buffer_offset_alignment", C.c_uint32),
        ("max_compute_workgroup_storage_size", C.c_uint32),
        ("max_compute_invocations_per_workgroup", C.c_uint32),
        ("max_compute_workgroup_size", C.c_uint32 * 3),
        ("max_compute_workgroups_per_dimension", C.c_uint32),
        ("max_storage_buffers_per_shader_stage", C.c_uint32),
        ("shader_f16", C.c_uint32),
        ("subgroups", C.c_uint32),
        ("timestamp_query", C.c_uint32),
        ("compute_units", C.c_uint32),
        ("wave_size", C.c_uint32),
        ("total_memory", C.c_uint64),
        ("name", C.c_char * 64),
        ("arch", C.c_char * 32),
    ]


class FrameTiming(C.Structure):
    _fields_ = [
        ("frame", C.c_uint64),
        ("n_slices", C.c_uint32),
        ("failed", C.c_uint32),
        ("tags", C.POINTER(C.c_uint32)),
        ("micros", C.POINTER(C.c_float)),
        ("has_render", C.c_uint32),
        ("render_micros", C.c_float),
    ]


class TimerStats(C.Structure):
    _fields_ = [
        ("frames_begun", C.c_uint64),
        ("frames_timed", C.c_uint64),
        ("frames_skipped", C.c_uint64),
        ("frames_failed", C.c_uint64),
        ("frames_dropped", C.c_uint64),
    ]


# Every symbol include/beatlm_hip.h declares, with its signature.
_VP = C.c_void_p
_SIGNATURES = {
    "bl_abi_version": (C.c_uint32, []),
    "bl_ctx_create": (C.c_int, [C.c_int, C.POINTER(_VP)]),
    "bl_ctx_destroy": (None, [_VP]),
    "bl_last_error": (C.c_char_p, [_VP]),
    "bl_device_profile": (C.c_int, [_VP, C.POINTER(DeviceProfile)]),
    "bl_ctx_set_f32_math": (C.c_int, [_VP, C.c_uint32]),
    "bl_ctx_synchronize": (C.c_int, [_VP]),
    "bl_ctx_allocations": (C.c_uint64, [_VP]),
    "bl_ctx_device_bytes": (C.c_uint64, [_VP]),
    "bl_ctx_stream": (_VP, [_VP]),
    "bl_arenas_create": (C.c_int, [_VP, C.POINTER(C.c_uint64), C.c_uint32, C.POINTER(_VP)]),
    "bl_arenas_destroy": (None, [_VP]),
    "bl_arenas_write": (C.c_int, [_VP, C.c_uint32, C.c_uint64, _VP, C.c_uint64]),
    "bl_arenas_read": (C.c_int, [_VP, C.c_uint32, C.c_uint64, _VP, C.c_uint64]),
    "bl_arenas_device_ptr": (C.c_int, [_VP, C.c_uint32, C.c_uint64, C.POINTER(_VP)]),
    "bl_arenas_invalidate": (C.c_int, [_VP, C.c_uint32, C.c_uint64, C.c_uint64]),
    "bl_kernels_create": (
        C.c_int,
        [_VP, _VP, C.POINTER(Spec), C.c_uint32, C.POINTER(BindingSet), C.c_uint32, C.POINTER(_VP)],
    ),
    "bl_kernels_create_internal": (
        C.c_int,
        [_VP, _VP, C.POINTER(Spec), C.c_uint32, C.POINTER(BindingSet), C.c_uint32, C.POINTER(C.c_uint32), C.c_uint32,
         C.POINTER(_VP)],
    ),
    "bl_kernels_destroy": (None, [_VP]),
    "bl_kernels_len": (C.c_uint32, [_VP]),
    "bl_kernels_sets": (C.c_uint32, [_VP]),
    "bl_kernels_label": (C.c_char_p, [_VP, C.c_uint32]),
    "bl_kernels_encode": (C.c_int, [_VP, C.c_uint32, C.c_uint32, _VP, C.c_uint32]),
    "bl_kernels_encode_range": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint32]),
    "bl_timer_create": (C.c_int, [_VP, C.c_uint32, C.POINTER(_VP)]),
    "bl_timer_destroy": (None, [_VP]),
    "bl_timer_begin_frame": (C.c_int, [_VP, C.c_uint64, C.POINTER(C.c_uint32)]),
    "bl_timer_resolve": (C.c_int, [_VP, C.POINTER(C.c_uint64)]),
    "bl_timer_render_begin": (C.c_int, [_VP]),
    "bl_timer_render_end": (C.c_int, [_VP]),
    "bl_timer_submitted": (C.c_int, [_VP, C.c_uint64]),
    "bl_timer_submitted_held": (C.c_int, [_VP, C.c_uint64, C.POINTER(C.c_uint64)]),
    "bl_timer_verdict": (C.c_int, [_VP, C.c_uint64, C.c_uint32]),
    "bl_timer_abandon": (C.c_int, [_VP, C.c_uint64]),
    "bl_timer_in_flight": (C.c_uint32, [_VP]),
    "bl_timer_collect": (C.c_int, [_VP, C.POINTER(FrameTiming), C.c_uint32, C.POINTER(C.c_uint32)]),
    "bl_timer_invalidate_submitted": (C.c_int, [_VP]),
    "bl_timer_stats": (C.c_int, [_VP, C.POINTER(TimerStats)]),
    "bl_kernels_time": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_float)]),
    "bl_kernels_packs_made": (C.c_uint64, [_VP]),
    "bl_kernels_workspace_bytes": (C.c_uint64, [_VP]),
    "bl_kernels_fold_read": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint32, _VP, C.c_uint64]),
    "bl_kernels_range_launches": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint32)]),
    "bl_spin": (C.c_int, [_VP, C.c_uint32]),
    "bl_flash_attention_static": (C.c_int, [_VP, _VP, _VP, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32]),
    "bl_flash_plan_check": (C.c_int, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]),
}

_lib = None


def lib() -> C.CDLL:
    """The backend library; raises when it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m beatlm_amd.build` "
                "(the backend has no fallback implementation)"
            )
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


class BackendError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class Context:
    """One device, one stream (bl_ctx)."""

    def __init__(self, device: int = 0):
        self._lib = lib()
        h = C.c_void_p()
        rc = self._lib.bl_ctx_create(device, C.byref(h))
        if rc != OK:
            raise BackendError(rc, f"bl_ctx_create({device}) failed")
        self.handle = h

    def check(self, rc: int) -> int:
        if rc < 0:
            raise BackendError(rc, self._lib.bl_last_error(self.handle).decode())
        return rc

    def profile(self) -> DeviceProfile:
        p = DeviceProfile()
        self.check(self._lib.bl_device_profile(self.handle, C.byref(p)))
        return p

    def set_f32_math(self, mode: int) -> None:
        self.check(self._lib.bl_ctx_set_f32_math(self.handle, mode))

    def synchronize(self) -> None:
        self.check(self._lib.bl_ctx_synchronize(self.handle))

    def allocations(self) -> int:
        return int(self._lib.bl_ctx_allocations(self.handle))

    def device_bytes(self) -> int:
        """Device bytes held now by this context's arenas and kernels."""
        return int(self._lib.bl_ctx_device_bytes(self.handle))

    def spin(self, micros: int) -> None:
        self.check(self._lib.bl_spin(self.handle, micros))

    def close(self) -> None:
        if self.handle:
            self._lib.bl_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Arenas:
    """Every arena of a plan in one device allocation (bl_arenas)."""

    def __init__(self, ctx: Context, sizes: list[int]):
        self.ctx = ctx
        arr = (C.c_uint64 * max(1, len(sizes)))(*sizes)
        h = C.c_void_p()
        ctx.check(ctx._lib.bl_arenas_create(ctx.handle, arr, len(sizes), C.byref(h)))
        self.handle = h

    def write(self, arena: int, offset: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        self.ctx.check(
            self.ctx._lib.bl_arenas_write(self.handle, arena, offset, data.ctypes.data, data.nbytes)
        )

    def read(self, arena: int, offset: int, count: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        self.ctx.check(self.ctx._lib.bl_arenas_read(self.handle, arena, offset, out.ctypes.data, out.nbytes))
        return out

    def device_ptr(self, arena: int, offset: int) -> int:
        p = C.c_void_p()
        self.ctx.check(self.ctx._lib.bl_arenas_device_ptr(self.handle, arena, offset, C.byref(p)))
        return int(p.value or 0)

    def invalidate(self, arena: int, offset: int, nbytes: int) -> None:
        """The host changed these bytes without write() (through device_ptr)."""
        self.ctx.check(self.ctx._lib.bl_arenas_invalidate(self.handle, arena, offset, nbytes))

    def close(self) -> None:
        if self.handle:
            self.ctx._lib.bl_arenas_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Kernels:
    """A program's kernels, checked and prepared once (bl_kernels)."""

    def __init__(
        self,
        ctx: Context,
        arenas: Arenas,
        specs: list[Spec],
        sets: list[list[Substitution]] | None = None,
        internal: list[int] | None = None,
    ):
        """`internal`: tensor ids the host never reads or writes (the program's
        activations); the backend may keep them in a layout of its own. The
        kernels hold `arenas` (the C side frees them after the kernels)."""
        self.ctx = ctx
        self.arenas = arenas
        arr = (Spec * max(1, len(specs)))(*specs)
        sets = sets or []
        keep = []
        set_arr = (BindingSet * max(1, len(sets)))()
        for i, subs in enumerate(sets):
            items = (Substitution * max(1, len(subs)))(*subs)
            keep.append(items)
            set_arr[i].items = C.cast(items, C.POINTER(Substitution))
            set_arr[i].count = len(subs)
        self._keep = keep
        h = C.c_void_p()
        internal = list(internal or [])
        ids = (C.c_uint32 * max(1, len(internal)))(*internal)
        ctx.check(
            ctx._lib.bl_kernels_create_internal(
                ctx.handle, arenas.handle, arr, len(specs), set_arr, len(sets), ids, len(internal), C.byref(h)
            )
        )
        self.handle = h

    def __len__(self) -> int:
        return int(self.ctx._lib.bl_kernels_len(self.handle))

    def sets(self) -> int:
        return int(self.ctx._lib.bl_kernels_sets(self.handle))

    def label(self, i: int) -> str | None:
        s = self.ctx._lib.bl_kernels_label(self.handle, i)
        return s.decode() if s is not None else None

    def encode(self, kernel: int, set_index: int = 0, timer: "Timer | None" = None, tag: int = 0) -> None:
        self.ctx.check(
            self.ctx._lib.bl_kernels_encode(self.handle, kernel, set_index, timer.handle if timer else None, tag)
        )

    def encode_all(self, set_index: int = 0) -> None:
        self.ctx.check(self.ctx._lib.bl_kernels_encode_range(self.handle, 0, len(self), set_index))

    def range_launches(self, first: int, count: int, set_index: int = 0) -> int:
        """GPU kernel launches of the captured graph that encode_range(first,
        count, set_index) replays (raises when that range has no graph)."""
        n = C.c_uint32()
        self.ctx.check(self.ctx._lib.bl_kernels_range_launches(self.handle, first, count, set_index, C.byref(n)))
        return int(n.value)

    def workspace_bytes(self) -> int:
        """Device bytes the kernels hold beside the arenas (one allocation)."""
        return int(self.ctx._lib.bl_kernels_workspace_bytes(self.handle))

    def packs_made(self) -> int:
        return int(self.ctx._lib.bl_kernels_packs_made(self.handle))

    def encode_range(self, first: int, count: int, set_index: int = 0) -> None:
        self.ctx.check(self.ctx._lib.bl_kernels_encode_range(self.handle, first, count, set_index))

    def fold_read(self, fold: int, what: int, floats: int, set_index: int = 0) -> np.ndarray:
        """A folded LayerNorm's buffers: what = 0 the statistics, 1 the column
        vectors c, d and the per-block column sums, 2 the centred shadow of x
        (diagnostics; `floats` counts 4-byte words)."""
        out = np.zeros(floats, np.float32)
        self.ctx.check(
            self.ctx._lib.bl_kernels_fold_read(self.handle, fold, set_index, what, out.ctypes.data_as(C.c_void_p), out.nbytes)
        )
        return out

    def time(self, kernel: int, repeats: int = 20, set_index: int = 0) -> float:
        """Average µs of one launch over `repeats` back-to-back launches."""
        us = C.c_float()
        self.ctx.check(self.ctx._lib.bl_kernels_time(self.handle, kernel, set_index, repeats, C.byref(us)))
        return float(us.value)

    def close(self) -> None:
        if self.handle:
            self.ctx._lib.bl_kernels_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Timer:
    """The slice timer (bl_timer)."""

    def __init__(self, ctx: Context, max_slices: int):
        self.ctx = ctx
        h = C.c_void_p()
        ctx.check(ctx._lib.bl_timer_create(ctx.handle, max_slices, C.byref(h)))
        self.handle = h

    def begin_frame(self, frame: int) -> bool:
        timed = C.c_uint32()
        self.ctx.check(self.ctx._lib.bl_timer_begin_frame(self.handle, frame, C.byref(timed)))
        return bool(timed.value)

    def resolve(self) -> int:
        """Closes the open frame; returns its ticket (0: untimed)."""
        r = C.c_uint64()
        self.ctx.check(self.ctx._lib.bl_timer_resolve(self.handle, C.byref(r)))
        return r.value

    def submitted(self, resolved: int) -> None:
        self.ctx.check(self.ctx._lib.bl_timer_submitted(self.handle, resolved))

    def submitted_held(self, resolved: int) -> int:
        """Hands the ticket back held; returns the hold for verdict() (0: nothing held)."""
        h = C.c_uint64()
        self.ctx.check(self.ctx._lib.bl_timer_submitted_held(self.handle, resolved, C.byref(h)))
        return h.value

    def verdict(self, hold: int, accepted: bool) -> bool:
        """HeldFrame::accept / reject; False when the frame had moved on."""
        return self.ctx.check(self.ctx._lib.bl_timer_verdict(self.handle, hold, 1 if accepted else 0)) == 1

    def abandon(self, resolved: int) -> None:
        """The frame's work was never submitted: its slot is freed unread."""
        self.ctx.check(self.ctx._lib.bl_timer_abandon(self.handle, resolved))

    def in_flight(self) -> int:
        return int(self.ctx._lib.bl_timer_in_flight(self.handle))

    def render_begin(self) -> None:
        self.ctx.check(self.ctx._lib.bl_timer_render_begin(self.handle))

    def render_end(self) -> None:
        self.ctx.check(self.ctx._lib.bl_timer_render_end(self.handle))

    def collect(self, cap: int = 16, render: bool = False):
        """The frames whose timings came back: (frame, [(tag, µs)]), or with
        `render` (frame, [(tag, µs)], render µs or None)."""
        out = (FrameTiming * cap)()
        n = C.c_uint32()
        self.ctx.check(self.ctx._lib.bl_timer_collect(self.handle, out, cap, C.byref(n)))
        frames = []
        for f in out[: n.value]:
            slices = [(int(f.tags[i]), float(f.micros[i])) for i in range(f.n_slices)]
            if render:
                frames.append((int(f.frame), slices, float(f.render_micros) if f.has_render else None))
            else:
                frames.append((int(f.frame), slices))
        return frames

    def invalidate_submitted(self) -> int:
        return self.ctx.check(self.ctx._lib.bl_timer_invalidate_submitted(self.handle))

    def stats(self) -> TimerStats:
        s = TimerStats()
        self.ctx.check(self.ctx._lib.bl_timer_stats(self.handle, C.byref(s)))
        return s

    def close(self) -> None:
        if self.handle:
            self.ctx._lib.bl_timer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
