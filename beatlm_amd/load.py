"""ctypes binding of the model-file side (include/beatlm_load.h), shaped like
the reference's `load` module and the conversion half of `model`:
`Archive` / `Tensor` / `StoredType` / `read_file` (crates/beatlm/src/load/
reader.rs:43-258), `Inventory` / `TensorSpec` / `CheckReport`
(load/inventory.rs:31-245), the Depth Anything V2 `inventory()` and
`Config::validate` (load/depth_anything_v2.rs:92-620), `Convert` and
`Weight::numbers` (model/mod.rs:140-353) with the bicubic position resampling
(model/positions.rs).

`depth_weights` is the step after it: every weight of a graph built by
`ir.depth_model`, read from a checkpoint through the inventory and converted
to the IR's layouts, ready for `Prepared.write`.

The parsing, checking and arithmetic live in the native library; this module
only converts.
"""

from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass, field

import numpy as np

from .hip import lib

OK = 0
ERR_FORMAT = 1
ERR_IO = 2
ERR_MISSING_TENSOR = 3
ERR_DUPLICATE_NAME = 4
ERR_INVALID_ARGUMENT = 5
ERR_CONFIG = 6
ERR_UNKNOWN_ROLE = 7
ERR_LAYOUT = 8
ERR_CONVERT = 9
ERR_SOURCE_SIZE = 10

AS_STORED = 0
LINEAR = 1
CONV = 2
CONV_TRANSPOSE = 3
INTERPOLATE_POSITIONS = 4

MAX_STAGES = 8


class LoadError(Exception):
    """LoadError (load/error.rs:11-43) and ModelError (model/mod.rs:52-136):
    `code` is the ERR_* value, the message the library's."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class FormatError(LoadError):
    pass


class IoError(LoadError):
    pass


class MissingTensor(LoadError):
    pass


class DuplicateName(LoadError):
    pass


class ModelError(LoadError):
    pass


class ConfigError(Exception):
    """ConfigError (depth_anything_v2.rs:254-300); `variant` names it."""

    VARIANTS = {1: "Zero", 2: "HeadsDoNotDivideHidden", 3: "ImageNotWholePatches", 4: "FusionWidthOdd",
                5: "StageCountMismatch", 6: "OutIndexOutOfRange", 7: "OutIndicesNotIncreasing", 8: "ResampleByOne"}

    def __init__(self, variant: str, message: str):
        super().__init__(message)
        self.variant = variant


_CLASSES = {ERR_FORMAT: FormatError, ERR_IO: IoError, ERR_MISSING_TENSOR: MissingTensor,
            ERR_DUPLICATE_NAME: DuplicateName, ERR_UNKNOWN_ROLE: ModelError, ERR_LAYOUT: ModelError,
            ERR_CONVERT: ModelError, ERR_SOURCE_SIZE: ModelError}


class StoredType(enum.IntEnum):
    """StoredType (reader.rs:43-120)."""

    F32 = 0
    F16 = 1
    BF16 = 2
    F64 = 3
    U8 = 4
    I32 = 5
    I64 = 6
    OTHER = 7

    def size_bytes(self):
        n = _l().blf_stored_type_size(int(self))
        return n or None

    def to_planned(self):
        """The storage the backend plans for a tensor stored as this one, or
        None: only F32 and F16 are planned as stored (reader.rs:76-90)."""
        from . import hip

        return {StoredType.F32: hip.F32, StoredType.F16: hip.F16}.get(self)

    def __str__(self):
        return _l().blf_stored_type_name(int(self)).decode()


_NUMPY = {StoredType.F32: np.float32, StoredType.F16: np.float16, StoredType.F64: np.float64,
          StoredType.U8: np.uint8, StoredType.I32: np.int32, StoredType.I64: np.int64}


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_uint32), ("rank", C.c_uint32),
                ("shape", C.POINTER(C.c_uint64)), ("data", C.POINTER(C.c_uint8)), ("bytes", C.c_uint64)]


class _Role(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("index", C.c_uint32), ("part", C.c_uint32), ("param", C.c_uint32),
                ("unit", C.c_uint32), ("conv", C.c_uint32)]


class _Spec(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_uint32), ("rank", C.c_uint32),
                ("shape", C.POINTER(C.c_uint64)), ("role", _Role)]


class _Config(C.Structure):
    _fields_ = [("image_size", C.c_uint32), ("patch_size", C.c_uint32), ("num_channels", C.c_uint32),
                ("hidden_size", C.c_uint32), ("num_layers", C.c_uint32), ("num_heads", C.c_uint32),
                ("mlp_ratio", C.c_uint32), ("mask_token", C.c_uint32), ("stages", C.c_uint32),
                ("out_indices", C.c_uint32 * MAX_STAGES), ("neck_hidden_sizes", C.c_uint32 * MAX_STAGES),
                ("resample", C.c_uint32 * MAX_STAGES), ("factor", C.c_uint32 * MAX_STAGES),
                ("fusion_hidden_size", C.c_uint32), ("head_hidden_size", C.c_uint32)]


_P = C.c_void_p
_SIGS = {
    "blf_last_error": (C.c_char_p, []),
    "blf_stored_type_size": (C.c_uint32, [C.c_uint32]),
    "blf_stored_type_name": (C.c_char_p, [C.c_uint32]),
    "blf_archive_parse": (C.c_int, [_P, C.c_uint64, C.POINTER(_P)]),
    "blf_archive_open": (C.c_int, [C.c_char_p, C.POINTER(_P)]),
    "blf_archive_destroy": (None, [_P]),
    "blf_archive_len": (C.c_uint64, [_P]),
    "blf_archive_at": (C.c_int, [_P, C.c_uint64, C.POINTER(_Tensor)]),
    "blf_archive_get": (C.c_int, [_P, C.c_char_p, C.POINTER(_Tensor)]),
    "blf_archive_parameter_count": (C.c_uint64, [_P]),
    "blf_inventory_new": (C.c_int, [C.POINTER(_Spec), C.c_uint64, C.POINTER(_P)]),
    "blf_inventory_destroy": (None, [_P]),
    "blf_inventory_len": (C.c_uint64, [_P]),
    "blf_inventory_at": (C.c_int, [_P, C.c_uint64, C.POINTER(_Spec)]),
    "blf_inventory_get": (C.c_int, [_P, C.c_char_p, C.POINTER(_Spec)]),
    "blf_inventory_by_role": (C.c_int, [_P, C.POINTER(_Role), C.POINTER(_Spec)]),
    "blf_inventory_parameter_count": (C.c_uint64, [_P]),
    "blf_inventory_check": (C.c_int, [_P, _P, C.POINTER(_P)]),
    "blf_report_destroy": (None, [_P]),
    "blf_report_is_exact": (C.c_int, [_P]),
    "blf_report_missing_len": (C.c_uint64, [_P]),
    "blf_report_missing": (C.c_char_p, [_P, C.c_uint64]),
    "blf_report_unexpected_len": (C.c_uint64, [_P]),
    "blf_report_unexpected": (C.c_char_p, [_P, C.c_uint64]),
    "blf_report_mismatched_len": (C.c_uint64, [_P]),
    "blf_report_mismatch": (C.c_int, [_P, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(_Tensor), C.POINTER(_Tensor)]),
    "blf_report_expected_parameters": (C.c_uint64, [_P]),
    "blf_report_file_parameters": (C.c_uint64, [_P]),
    "blf_report_text": (C.c_char_p, [_P]),
    "blf_dav2_small": (None, [C.POINTER(_Config)]),
    "blf_dav2_validate": (C.c_int, [C.POINTER(_Config), C.POINTER(C.c_uint32)]),
    "blf_dav2_inventory": (C.c_int, [C.POINTER(_Config), C.POINTER(_P), C.POINTER(C.c_uint32)]),
    "blf_convert": (C.c_int, [C.c_uint32, C.POINTER(C.c_float), C.POINTER(C.c_uint64), C.c_uint32, C.c_uint32,
                               C.c_uint32, C.POINTER(C.c_float), C.c_uint64, C.POINTER(C.c_uint64),
                               C.POINTER(C.c_uint64)]),
    "blf_weight_numbers": (C.c_int, [_P, _P, C.POINTER(_Role), C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                     C.POINTER(C.c_float), C.c_uint64]),
}
_bound = None


def _l():
    global _bound
    if _bound is None:
        h = lib()
        for name, (res, args) in _SIGS.items():
            f = getattr(h, name)
            f.restype = res
            f.argtypes = args
        _bound = h
    return _bound


def _check(rc: int) -> None:
    if rc != OK:
        msg = _l().blf_last_error().decode(errors="replace")
        raise _CLASSES.get(rc, LoadError)(rc, msg)


def _shape(ptr, rank) -> tuple:
    return tuple(int(ptr[i]) for i in range(rank))


def element_count(shape) -> int:
    """The product of a shape's extents (a scalar is one element),
    saturating at 2**64 - 1 (reader.rs:160-167)."""
    n = 1
    for e in shape:
        n = min(n * int(e), 2**64 - 1)
    return n


# ---- the reader ----------------------------------------------------------------


@dataclass(frozen=True)
class Tensor:
    """One tensor of an Archive: element type, shape and its stored bytes,
    which borrow from the archive's buffer."""

    dtype: StoredType
    shape: tuple
    data: memoryview
    owner: object = field(default=None, repr=False, compare=False)  # the archive the bytes borrow from

    def element_count(self) -> int:
        return element_count(self.shape)

    def numpy(self) -> np.ndarray:
        """The stored values as a little-endian array of the shape (a view)."""
        t = _NUMPY.get(self.dtype)
        if t is None:
            raise TypeError(f"no array type for {self.dtype}")
        return np.frombuffer(self.data, dtype=np.dtype(t).newbyteorder("<")).reshape(self.shape)


class Archive:
    """The tensors of one safetensors file, by name, iterated in name order."""

    def __init__(self, handle, keep):
        self._h = handle
        self._keep = keep  # the bytes the tensors borrow from

    @classmethod
    def parse(cls, data) -> "Archive":
        """Archive::parse: the whole file's bytes. FormatError when the header
        is malformed or disagrees with the buffer."""
        buf = bytes(data) if not isinstance(data, bytes) else data
        h = _P()
        _check(_l().blf_archive_parse(buf, len(buf), C.byref(h)))
        return cls(h, buf)

    @classmethod
    def open(cls, path) -> "Archive":
        """read_file + Archive::parse: IoError names the path."""
        h = _P()
        _check(_l().blf_archive_open(str(path).encode(), C.byref(h)))
        return cls(h, None)

    def __del__(self):
        if getattr(self, "_h", None):
            _l().blf_archive_destroy(self._h)
            self._h = None

    def __len__(self) -> int:
        return int(_l().blf_archive_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    def _tensor(self, t: _Tensor) -> Tensor:
        n = int(t.bytes)
        view = memoryview((C.c_uint8 * n).from_address(C.addressof(t.data.contents))) if n else memoryview(b"")
        return Tensor(StoredType(t.dtype), _shape(t.shape, t.rank), view.cast("B"), self)

    def get(self, name: str) -> Tensor | None:
        try:
            return self.require(name)
        except MissingTensor:
            return None

    def require(self, name: str) -> Tensor:
        t = _Tensor()
        _check(_l().blf_archive_get(self._h, name.encode(), C.byref(t)))
        return self._tensor(t)

    def iter(self):
        """Every tensor with its name, in name order."""
        for i in range(len(self)):
            t = _Tensor()
            _check(_l().blf_archive_at(self._h, i, C.byref(t)))
            yield t.name.decode(), self._tensor(t)

    __iter__ = iter

    def parameter_count(self) -> int:
        return int(_l().blf_archive_parameter_count(self._h))


def read_file(path) -> bytes:
    """The whole file (reader.rs:252-258); IoError names the path."""
    try:
        with open(path, "rb") as f:
            return f.read()
    except OSError as e:
        raise IoError(ERR_IO, f"cannot read {path}: {e.strerror}") from e


# ---- inventories ---------------------------------------------------------------


@dataclass(frozen=True)
class Role:
    """A tensor's role, compared field by field (the Depth Anything V2 roles:
    depth_anything_v2.rs:408-460; see the constructors below)."""

    kind: int
    index: int = 0
    part: int = 0
    param: int = 0
    unit: int = 0
    conv: int = 0

    def _c(self) -> _Role:
        return _Role(self.kind, self.index, self.part, self.param, self.unit, self.conv)


# Role kinds, block parts, params (include/beatlm_load.h).
CLASS_TOKEN, MASK_TOKEN, POSITION_EMBEDDING, PATCH_PROJECTION, BLOCK, FINAL_NORM, REASSEMBLE, NECK_CONV, FUSION, HEAD = \
    range(10)
WEIGHT, BIAS = 0, 1
NORM1, QUERY, KEY, VALUE, ATTENTION_OUTPUT, LAYER_SCALE1, NORM2, MLP_FC1, MLP_FC2, LAYER_SCALE2 = range(10)
PROJECTION, RESIZE, RESIDUAL = 0, 1, 1


def block_role(layer: int, part: int, param: int = 0) -> Role:
    return Role(BLOCK, layer, part, param if part not in (LAYER_SCALE1, LAYER_SCALE2) else 0)


@dataclass(frozen=True)
class TensorSpec:
    name: str
    dtype: StoredType
    shape: tuple
    role: Role

    def element_count(self) -> int:
        return element_count(self.shape)


@dataclass(frozen=True)
class Layout:
    dtype: StoredType
    shape: tuple

    def __str__(self):
        return f"{self.dtype} [{', '.join(str(e) for e in self.shape)}]"


@dataclass(frozen=True)
class Mismatch:
    name: str
    expected: Layout
    found: Layout


@dataclass(frozen=True)
class CheckReport:
    missing: list
    unexpected: list
    mismatched: list
    expected_parameters: int
    file_parameters: int
    text: str

    def is_exact(self) -> bool:
        return not (self.missing or self.unexpected or self.mismatched)

    def __str__(self):
        return self.text


def _spec_from(s: _Spec) -> TensorSpec:
    r = s.role
    return TensorSpec(s.name.decode(), StoredType(s.dtype), _shape(s.shape, s.rank),
                      Role(r.kind, r.index, r.part, r.param, r.unit, r.conv))


class Inventory:
    """The tensors a model expects: names, types, shapes and roles, in order.
    DuplicateName when a name repeats."""

    def __init__(self, specs=None, _handle=None):
        if _handle is not None:
            self._h = _handle
            return
        specs = list(specs)
        shapes = [(C.c_uint64 * max(1, len(s.shape)))(*s.shape) for s in specs]
        arr = (_Spec * max(1, len(specs)))()
        for i, s in enumerate(specs):
            arr[i] = _Spec(s.name.encode(), int(s.dtype), len(s.shape), C.cast(shapes[i], C.POINTER(C.c_uint64)),
                           s.role._c())
        h = _P()
        _check(_l().blf_inventory_new(arr, len(specs), C.byref(h)))
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            _l().blf_inventory_destroy(self._h)
            self._h = None

    def __len__(self) -> int:
        return int(_l().blf_inventory_len(self._h))

    def is_empty(self) -> bool:
        return len(self) == 0

    def iter(self):
        for i in range(len(self)):
            s = _Spec()
            _check(_l().blf_inventory_at(self._h, i, C.byref(s)))
            yield _spec_from(s)

    __iter__ = iter

    def get(self, name: str) -> TensorSpec | None:
        s = _Spec()
        if _l().blf_inventory_get(self._h, name.encode(), C.byref(s)) != OK:
            return None
        return _spec_from(s)

    def by_role(self, role: Role) -> TensorSpec | None:
        s = _Spec()
        r = role._c()
        if _l().blf_inventory_by_role(self._h, C.byref(r), C.byref(s)) != OK:
            return None
        return _spec_from(s)

    def parameter_count(self) -> int:
        return int(_l().blf_inventory_parameter_count(self._h))

    def check(self, archive: Archive) -> CheckReport:
        """Every difference between the inventory and the file
        (inventory.rs:117-160)."""
        L = _l()
        h = _P()
        _check(L.blf_inventory_check(self._h, archive._h, C.byref(h)))
        try:
            missing = [L.blf_report_missing(h, i).decode() for i in range(L.blf_report_missing_len(h))]
            unexpected = [L.blf_report_unexpected(h, i).decode() for i in range(L.blf_report_unexpected_len(h))]
            mismatched = []
            for i in range(L.blf_report_mismatched_len(h)):
                name, e, f = C.c_char_p(), _Tensor(), _Tensor()
                _check(L.blf_report_mismatch(h, i, C.byref(name), C.byref(e), C.byref(f)))
                mismatched.append(Mismatch(name.value.decode(), Layout(StoredType(e.dtype), _shape(e.shape, e.rank)),
                                           Layout(StoredType(f.dtype), _shape(f.shape, f.rank))))
            return CheckReport(missing, unexpected, mismatched, int(L.blf_report_expected_parameters(h)),
                               int(L.blf_report_file_parameters(h)), L.blf_report_text(h).decode())
        finally:
            L.blf_report_destroy(h)


# ---- Depth Anything V2 ---------------------------------------------------------


def _config(cfg) -> _Config:
    """An ir.DepthConfig as the library's struct; the stage lists' lengths
    must agree (StageCountMismatch otherwise, as Config::validate says)."""
    stages = len(cfg.out_indices)
    if stages == 0 or len(cfg.neck_hidden_sizes) != stages or len(cfg.reassemble) != stages:
        raise ConfigError("StageCountMismatch",
                          f"stage lists disagree: {stages} out indices, {len(cfg.neck_hidden_sizes)} neck sizes, "
                          f"{len(cfg.reassemble)} resamplings")
    if stages > MAX_STAGES:
        raise ValueError(f"at most {MAX_STAGES} stages")
    c = _Config()
    c.image_size, c.patch_size, c.num_channels = cfg.image_size, cfg.patch_size, cfg.num_channels
    c.hidden_size, c.num_layers, c.num_heads, c.mlp_ratio = cfg.hidden_size, cfg.num_layers, cfg.num_heads, cfg.mlp_ratio
    c.mask_token = 1 if getattr(cfg, "mask_token", True) else 0
    c.stages = stages
    for i in range(stages):
        c.out_indices[i] = cfg.out_indices[i]
        c.neck_hidden_sizes[i] = cfg.neck_hidden_sizes[i]
        kind = cfg.reassemble[i]
        c.resample[i] = {"keep": 0, "up": 1, "down": 2}[kind[0]]
        c.factor[i] = kind[1] if len(kind) > 1 else 0
    c.fusion_hidden_size, c.head_hidden_size = cfg.fusion_hidden_size, cfg.head_hidden_size
    return c


def validate(cfg) -> None:
    """Config::validate (depth_anything_v2.rs:170-250): ConfigError names the
    first rule the configuration breaks."""
    c = _config(cfg)
    v = C.c_uint32()
    rc = _l().blf_dav2_validate(C.byref(c), C.byref(v))
    if rc == ERR_CONFIG:
        raise ConfigError(ConfigError.VARIANTS.get(v.value, "?"), _l().blf_last_error().decode())
    _check(rc)


def inventory(cfg) -> Inventory:
    """inventory() (depth_anything_v2.rs:462-620): every tensor of a Depth
    Anything V2 checkpoint of this configuration, F32, with its role."""
    c = _config(cfg)
    v = C.c_uint32()
    h = _P()
    rc = _l().blf_dav2_inventory(C.byref(c), C.byref(h), C.byref(v))
    if rc == ERR_CONFIG:
        raise ConfigError(ConfigError.VARIANTS.get(v.value, "?"), _l().blf_last_error().decode())
    _check(rc)
    return Inventory(_handle=h)


# ---- conversions ---------------------------------------------------------------


def convert(values, shape, how: int, height: int = 0, width: int = 0):
    """convert() (model/mod.rs:274-335): (the rearranged f32 numbers, the
    result's last dimension). ModelError (ERR_CONVERT) for a shape the
    conversion does not apply to."""
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    sh = (C.c_uint64 * max(1, len(shape)))(*shape)
    cap = max(v.size, (1 + height * width) * (shape[-1] if shape else 1)) if how == INTERPOLATE_POSITIONS else v.size
    out = np.empty(max(1, cap), np.float32)
    written, cols = C.c_uint64(), C.c_uint64()
    _check(_l().blf_convert(how, v.ctypes.data_as(C.POINTER(C.c_float)), sh, len(shape), height, width,
                            out.ctypes.data_as(C.POINTER(C.c_float)), out.size, C.byref(written), C.byref(cols)))
    return out[: written.value].copy(), int(cols.value)


def weight_numbers(inv: Inventory, archive: Archive, parts, how: int, elements: int, height: int = 0,
                   width: int = 0) -> np.ndarray:
    """Weight::numbers (model/mod.rs:218-262): the parts' tensors, each
    converted, side by side along their last dimension."""
    roles = (_Role * max(1, len(parts)))(*[r._c() for r in parts])
    out = np.empty(max(1, elements), np.float32)
    _check(_l().blf_weight_numbers(inv._h, archive._h, roles, len(parts), how, height, width,
                                   out.ctypes.data_as(C.POINTER(C.c_float)), elements))
    return out[:elements]


def depth_weights(archive: Archive, cfg, model, side: int | None = None, check: bool = True) -> dict:
    """{tensor id: f32 numbers} for every weight of `model` (an
    ir.DepthModelIds built for an image of `side` pixels), read from a Depth
    Anything V2 checkpoint of configuration `cfg`: the encoder's weights
    converted as the reference's model() sources them (linear weights
    transposed, Q/K/V side by side, the patch projection as HWIO, the position
    embedding resampled to the graph's patch grid), the decoder's named as the
    checkpoint names them (3x3 and 1x1 convolutions as HWIO, transposed
    convolutions from [in][out][kh][kw]). With `check`, the file must match
    the inventory exactly (ModelError otherwise, with the report)."""
    inv = inventory(cfg)
    if check:
        report = inv.check(archive)
        if not report.is_exact():
            raise ModelError(ERR_LAYOUT, str(report))
    side = side or cfg.image_size
    grid = side // cfg.patch_size
    d, mlp = cfg.hidden_size, cfg.hidden_size * cfg.mlp_ratio
    enc = model.encoder
    e = enc.embed
    out = {}

    def take(tid, parts, how, elements, h=0, w=0):
        out[tid] = weight_numbers(inv, archive, parts, how, elements, h, w)

    take(e.patch_w, [Role(PATCH_PROJECTION, param=WEIGHT)], CONV, cfg.patch_size ** 2 * cfg.num_channels * d)
    take(e.patch_b, [Role(PATCH_PROJECTION, param=BIAS)], AS_STORED, d)
    take(e.cls, [Role(CLASS_TOKEN)], AS_STORED, d)
    take(e.pos, [Role(POSITION_EMBEDDING)], INTERPOLATE_POSITIONS, (grid * grid + 1) * d, grid, grid)
    for layer, ids in enumerate(enc.blocks):
        b = lambda part, param=0: block_role(layer, part, param)  # noqa: E731
        take(ids.norm1_g, [b(NORM1, WEIGHT)], AS_STORED, d)
        take(ids.norm1_b, [b(NORM1, BIAS)], AS_STORED, d)
        take(ids.qkv_w, [b(QUERY, WEIGHT), b(KEY, WEIGHT), b(VALUE, WEIGHT)], LINEAR, 3 * d * d)
        take(ids.qkv_b, [b(QUERY, BIAS), b(KEY, BIAS), b(VALUE, BIAS)], AS_STORED, 3 * d)
        take(ids.proj_w, [b(ATTENTION_OUTPUT, WEIGHT)], LINEAR, d * d)
        take(ids.proj_b, [b(ATTENTION_OUTPUT, BIAS)], AS_STORED, d)
        take(ids.ls1, [b(LAYER_SCALE1)], AS_STORED, d)
        take(ids.norm2_g, [b(NORM2, WEIGHT)], AS_STORED, d)
        take(ids.norm2_b, [b(NORM2, BIAS)], AS_STORED, d)
        take(ids.fc1_w, [b(MLP_FC1, WEIGHT)], LINEAR, d * mlp)
        take(ids.fc1_b, [b(MLP_FC1, BIAS)], AS_STORED, mlp)
        take(ids.fc2_w, [b(MLP_FC2, WEIGHT)], LINEAR, mlp * d)
        take(ids.fc2_b, [b(MLP_FC2, BIAS)], AS_STORED, d)
        take(ids.ls2, [b(LAYER_SCALE2)], AS_STORED, d)
    take(enc.final_g, [Role(FINAL_NORM, param=WEIGHT)], AS_STORED, d)
    take(enc.final_b, [Role(FINAL_NORM, param=BIAS)], AS_STORED, d)
    for tid, name, elements in model.decoder_weights:
        spec = inv.get(name)
        if spec is None:
            raise ModelError(ERR_UNKNOWN_ROLE, f"the inventory has no tensor `{name}`")
        if name.endswith(".bias"):
            how = AS_STORED
        elif ".resize." in name and cfg.reassemble[spec.role.index][0] == "up":
            how = CONV_TRANSPOSE
        else:
            how = CONV
        take(tid, [spec.role], how, elements)
    return out
