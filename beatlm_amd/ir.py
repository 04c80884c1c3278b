"""ctypes binding of the IR's C API (include/beatlm_ir.h) and the harness that
runs a graph through the backend, as the reference's
`harness::run_on_gpu` does (crates/beatlm-bench/src/harness.rs:133-172):
lower -> (fuse attention) -> split -> plan -> arenas -> write -> kernels ->
encode -> read.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import hip
from .hip import Spec, lib

NONE = 0xFFFFFFFF

INPUT, WEIGHT, ACTIVATION, OUTPUT = 0, 1, 2, 3
FUSION_ON, FUSION_OFF = 0, 1

OP_LAYER_NORM = 1
OP_MATMUL = 2
OP_ATTENTION_SCORES = 3
OP_SOFTMAX = 4
OP_ATTENTION_VALUES = 5
OP_PATCH_EMBED = 6
OP_PREPEND_TOKEN = 7
OP_TOKENS_TO_MAP = 8
OP_CONV3X3 = 9
OP_CONV1X1 = 10
OP_CONV_TRANSPOSE = 11
OP_RESIZE_BILINEAR = 12
OP_ADD = 20
OP_RELU = 21
OP_GELU = 22
OP_GELU_ERF = 23
OP_SCALE = 24
OP_CHANNEL_SCALE = 25

ERRORS = {
    -100: "DuplicateTensor", -101: "EmptyTensor", -102: "TensorTooLarge", -103: "UnknownTensor",
    -104: "ElementCount", -105: "ReadBeforeWritten", -106: "WrittenTwice", -107: "NotWritable",
    -108: "ZeroDimension", -109: "OpTooLarge", -110: "NonFiniteScale", -111: "InvalidEpsilon",
    -112: "TooManyOps", -113: "EmptyGraph", -114: "NeverWritten", -115: "NotInputOrOutput",
    -116: "ExceedsLimit", -117: "PartCounts", -118: "AlreadySplit", -119: "ZeroBound", -120: "UnknownOp",
    -130: "Plan.DuplicateTensor", -131: "Plan.InvalidLifetime", -132: "Plan.EmptyTensor",
    -133: "Plan.SizeOverflow", -134: "Plan.TensorTooLarge", -135: "Plan.InvalidProfile",
    -136: "Plan.TooManyTensors", -137: "NoPlacement",
}


class Op(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("t", C.c_uint32 * 4), ("d", C.c_uint32 * 6), ("f", C.c_float)]


def op(kind: int, tensors, dims, f: float = 0.0) -> Op:
    o = Op()
    o.kind = kind
    t = list(tensors) + [NONE] * (4 - len(tensors))
    d = list(dims) + [0] * (6 - len(dims))
    o.t = (C.c_uint32 * 4)(*t)
    o.d = (C.c_uint32 * 6)(*d)
    o.f = f
    return o


class TensorDesc(C.Structure):
    _fields_ = [
        ("id", C.c_uint32),
        ("dtype", C.c_uint32),
        ("elements", C.c_uint64),
        ("first_use", C.c_uint32),
        ("last_use", C.c_uint32),
    ]


class Profile(C.Structure):
    _fields_ = [
        ("max_storage_buffer_binding_size", C.c_uint64),
        ("max_buffer_size", C.c_uint64),
        ("min_storage_buffer_offset_alignment", C.c_uint32),
        ("max_compute_workgroup_storage_size", C.c_uint32),
        ("max_compute_invocations_per_workgroup", C.c_uint32),
        ("max_compute_workgroups_per_dimension", C.c_uint32),
        ("max_storage_buffers_per_shader_stage", C.c_uint32),
    ]


class Placement(C.Structure):
    _fields_ = [("arena", C.c_uint32), ("reserved", C.c_uint32), ("offset", C.c_uint64), ("size", C.c_uint64)]


class KernelInfo(C.Structure):
    _fields_ = [
        ("main", C.c_uint32),
        ("dims", C.c_uint32 * 6),
        ("epsilon", C.c_float),
        ("scale", C.c_float),
        ("part", hip.Part),
        ("max_parts", C.c_uint32),
        ("tile_rows", C.c_uint32),
        ("output_start", C.c_uint64),
        ("output_end", C.c_uint64),
        ("n_reads", C.c_uint32),
        ("reads", C.c_uint32 * 4),
        ("n_epilogue", C.c_uint32),
        ("epilogue", hip.Epilogue * hip.MAX_EPILOGUE),
        ("n_bindings", C.c_uint32),
        ("bindings", C.c_uint32 * hip.MAX_BINDINGS),
        ("first_op", C.c_uint32),
        ("end_op", C.c_uint32),
        ("prologue", C.c_uint32),
    ]


class VitDims(C.Structure):
    _fields_ = [
        ("tokens", C.c_uint32),
        ("width", C.c_uint32),
        ("heads", C.c_uint32),
        ("mlp", C.c_uint32),
        ("epsilon", C.c_float),
    ]


BLOCK_WEIGHTS = (
    "norm1_g", "norm1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "ls1",
    "norm2_g", "norm2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b", "ls2",
)


class BlockIds(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in BLOCK_WEIGHTS] + [("output", C.c_uint32), ("next_id", C.c_uint32)]


class EmbedIds(C.Structure):
    _fields_ = [
        (n, C.c_uint32) for n in ("image", "patch_w", "patch_b", "cls", "pos", "output", "next_id")
    ]


_VP = C.c_void_p
_SIG = {
    "bli_last_error": (C.c_char_p, []),
    "bli_profile_webgpu_baseline": (None, [C.POINTER(Profile)]),
    "bli_profile_mi355x": (None, [C.POINTER(Profile)]),
    "bli_graph_new": (C.c_int, [C.POINTER(_VP)]),
    "bli_graph_free": (None, [_VP]),
    "bli_graph_tensor": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint64]),
    "bli_graph_push": (C.c_int, [_VP, C.POINTER(Op), C.c_uint32]),
    "bli_op_output_elements": (C.c_uint64, [C.POINTER(Op)]),
    "bli_graph_ops": (C.c_uint32, [_VP]),
    "bli_graph_lower": (C.c_int, [_VP, C.c_uint32, C.POINTER(_VP)]),
    "bli_program_free": (None, [_VP]),
    "bli_program_split": (C.c_int, [_VP, C.POINTER(C.c_uint32), C.c_uint32, C.POINTER(_VP)]),
    "bli_program_parts_within": (
        C.c_int, [_VP, C.POINTER(C.c_uint64), C.c_uint32, C.c_uint64, C.POINTER(C.c_uint32)]
    ),
    "bli_program_fuse_attention": (C.c_int, [_VP, C.POINTER(_VP)]),
    "bli_program_set_dtype": (C.c_int, [_VP, C.c_uint32]),
    "bli_program_len": (C.c_uint32, [_VP]),
    "bli_program_kernel": (C.c_int, [_VP, C.c_uint32, C.POINTER(KernelInfo)]),
    "bli_program_kernel_name": (C.c_int, [_VP, C.c_uint32, C.c_char_p, C.c_uint32]),
    "bli_program_tensors": (C.c_uint32, [_VP, C.POINTER(TensorDesc), C.c_uint32]),
    "bli_program_role": (C.c_int, [_VP, C.c_uint32]),
    "bli_program_stand_in": (C.c_int, [_VP, C.c_uint32, C.c_uint32, C.POINTER(TensorDesc)]),
    "bli_program_spec": (C.c_int, [_VP, C.c_uint32, _VP, C.POINTER(Spec)]),
    "bli_plan_new": (C.c_int, [C.POINTER(TensorDesc), C.c_uint32, C.POINTER(Profile), C.POINTER(_VP)]),
    "bli_plan_free": (None, [_VP]),
    "bli_plan_arenas": (C.c_uint32, [_VP, C.POINTER(C.c_uint64), C.c_uint32]),
    "bli_plan_placement": (C.c_int, [_VP, C.c_uint32, C.POINTER(Placement)]),
    "bli_plan_peak_live_bytes": (C.c_uint64, [_VP]),
    "bli_plan_total_bytes": (C.c_uint64, [_VP]),
    "bli_plan_valid_on": (C.c_int, [_VP, C.POINTER(Profile)]),
    "bli_vit_block": (C.c_int, [_VP, C.POINTER(VitDims), C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(BlockIds)]),
    "bli_vit_embeddings": (
        C.c_int, [_VP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(EmbedIds)]
    ),
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


class IrError(RuntimeError):
    def __init__(self, code: int):
        self.code = code
        self.kind = ERRORS.get(code, str(code))
        super().__init__(f"{self.kind}: {_lib().bli_last_error().decode()}")


def _check(rc: int) -> int:
    if rc < 0:
        raise IrError(rc)
    return rc


def profile(kind: str = "mi355x") -> Profile:
    p = Profile()
    if kind == "baseline":
        _lib().bli_profile_webgpu_baseline(C.byref(p))
    else:
        _lib().bli_profile_mi355x(C.byref(p))
    return p


class Graph:
    def __init__(self):
        h = C.c_void_p()
        _check(_lib().bli_graph_new(C.byref(h)))
        self.handle = h

    def __del__(self):
        # At interpreter exit the module's globals may already be gone.
        if getattr(self, "handle", None) and callable(_lib):
            _lib().bli_graph_free(self.handle)
            self.handle = None

    def tensor(self, tid: int, role: int, elements: int) -> int:
        _check(_lib().bli_graph_tensor(self.handle, tid, role, elements))
        return tid

    def push(self, o: Op, output: int) -> int:
        _check(_lib().bli_graph_push(self.handle, C.byref(o), output))
        return output

    def ops(self) -> int:
        return int(_lib().bli_graph_ops(self.handle))

    def lower(self, fusion: int = FUSION_ON) -> "Program":
        h = C.c_void_p()
        _check(_lib().bli_graph_lower(self.handle, fusion, C.byref(h)))
        return Program(h)

    def vit_block(self, dims: VitDims, x: int, first_id: int, role: int = ACTIVATION) -> BlockIds:
        ids = BlockIds()
        _check(_lib().bli_vit_block(self.handle, C.byref(dims), x, first_id, role, C.byref(ids)))
        return ids

    def vit_embeddings(self, grid: int, patch: int, channels: int, width: int, first_id: int) -> EmbedIds:
        ids = EmbedIds()
        _check(_lib().bli_vit_embeddings(self.handle, grid, patch, channels, width, first_id, C.byref(ids)))
        return ids


class EncoderIds:
    """The tensors of an encoder built by Graph.vit_encoder."""

    def __init__(self, embed: EmbedIds, blocks: list, final_g: int, final_b: int, features: list, next_id: int):
        self.embed = embed
        self.blocks = blocks
        self.final_g, self.final_b = final_g, final_b
        self.features = features  # one [grid][grid][width] map per tapped layer, shallowest first
        self.next_id = next_id


def vit_encoder(
    g: "Graph",
    grid: int,
    patch: int,
    channels: int,
    width: int,
    heads: int,
    mlp: int,
    eps: float,
    out_indices,
    first_id: int = 0,
    features_role: int = OUTPUT,
) -> EncoderIds:
    """The reference's encoder() (crates/beatlm/src/model/depth_anything_v2.rs
    :434-527): patch embedding, class token and positions, the pre-LN blocks
    up to the deepest tapped layer, and for each layer in `out_indices`
    (1-based, as the checkpoint's config lists them) the shared final
    LayerNorm of its hidden state and the token-to-map that drops the class
    token, a [grid][grid][width] feature map of role `features_role`."""
    tokens = grid * grid + 1
    emb = g.vit_embeddings(grid, patch, channels, width, first_id)
    x, nid = emb.output, emb.next_id
    taps = set(out_indices)
    blocks, taken = [], []
    for layer in range(max(out_indices, default=0)):
        ids = g.vit_block(VitDims(tokens, width, heads, mlp, eps), x, nid, ACTIVATION)
        blocks.append(ids)
        x, nid = ids.output, ids.next_id
        if layer + 1 in taps:
            taken.append(x)
    final_g, final_b = nid, nid + 1
    g.tensor(final_g, WEIGHT, width)
    g.tensor(final_b, WEIGHT, width)
    nid += 2
    features = []
    for hidden in taken:
        normed, fmap = nid, nid + 1
        g.tensor(normed, ACTIVATION, tokens * width)
        g.push(op(OP_LAYER_NORM, [hidden, final_g, final_b], [tokens, width], eps), normed)
        g.tensor(fmap, features_role, grid * grid * width)
        g.push(op(OP_TOKENS_TO_MAP, [normed], [grid, grid, width]), fmap)
        features.append(fmap)
        nid += 2
    return EncoderIds(emb, blocks, final_g, final_b, features, nid)


@dataclass(frozen=True)
class DepthConfig:
    """The structure of a Depth Anything V2 model
    (crates/beatlm/src/load/depth_anything_v2.rs:85-152); `small()` is
    depth-anything/Depth-Anything-V2-Small-hf. `reassemble` per stage:
    ("up", f) a transposed convolution of kernel and stride f, ("keep",) or
    ("down", f) a 3x3 convolution at stride f."""

    image_size: int = 518
    patch_size: int = 14
    num_channels: int = 3
    hidden_size: int = 384
    num_layers: int = 12
    num_heads: int = 6
    mlp_ratio: int = 4
    out_indices: tuple = (3, 6, 9, 12)
    neck_hidden_sizes: tuple = (48, 96, 192, 384)
    reassemble: tuple = (("up", 4), ("up", 2), ("keep",), ("down", 2))
    fusion_hidden_size: int = 64
    head_hidden_size: int = 32
    eps: float = 1e-6
    mask_token: bool = True  # the checkpoint holds backbone.embeddings.mask_token (unused by inference)

    @classmethod
    def small(cls) -> "DepthConfig":
        return cls()

    def fan_in(self, name: str) -> int:
        """Inputs summed into one output of a decoder weight named as
        depth_decoder names it (a convolution's kh * kw * cin; a transposed
        convolution's cin), for scaling random weights."""
        parts = name.split(".")
        fusion = self.fusion_hidden_size
        if name.startswith("neck.reassemble_stage."):
            i = int(parts[3])
            ch = self.neck_hidden_sizes[i]
            if parts[4] == "projection":
                return self.hidden_size
            return ch if self.reassemble[i][0] == "up" else 9 * ch
        if name.startswith("neck.convs."):
            return 9 * self.neck_hidden_sizes[int(parts[2])]
        if name.startswith("neck.fusion_stage."):
            return fusion if parts[4] == "projection" else 9 * fusion
        return {"conv1": 9 * fusion, "conv2": 9 * (fusion // 2), "conv3": self.head_hidden_size}[parts[1]]


class _Ids:
    """Tensor ids handed out in order, as the reference's Builder does
    (crates/beatlm/src/model/mod.rs:360-444): every weight when an operation
    first needs it, then the operation's output."""

    def __init__(self, g: "Graph", first_id: int):
        self.g, self.next = g, first_id
        self.weights = []  # (id, name, elements) in declaration order

    def weight(self, name: str, elements: int) -> int:
        tid = self.next
        self.next += 1
        self.g.tensor(tid, WEIGHT, elements)
        self.weights.append((tid, name, elements))
        return tid

    def op(self, o: Op, role: int = ACTIVATION) -> int:
        tid = self.next
        self.next += 1
        self.g.tensor(tid, role, output_elements(o))
        self.g.push(o, tid)
        return tid


def _conv3x3(ids, x, name, size, cin, cout, stride=1, bias=True, role=ACTIVATION):
    w = ids.weight(name + ".weight", 9 * cin * cout)
    b = ids.weight(name + ".bias", cout) if bias else NONE
    return ids.op(op(OP_CONV3X3, [x, w, b], [size[0], size[1], cin, cout, stride]), role)


def _conv1x1(ids, x, name, size, cin, cout, role=ACTIVATION):
    w = ids.weight(name + ".weight", cin * cout)
    b = ids.weight(name + ".bias", cout)
    return ids.op(op(OP_CONV1X1, [x, w, b], [size[0], size[1], cin, cout]), role)


def _strided(extent, stride):
    return (extent - 1) // stride + 1


def _residual_unit(ids, x, name, size, c):
    """x + conv2(relu(conv1(relu(x)))): depth_anything_v2.rs:776-812."""
    n = size[0] * size[1] * c
    a = ids.op(op(OP_RELU, [x], [n]))
    first = _conv3x3(ids, a, name + ".convolution1", size, c, c)
    a2 = ids.op(op(OP_RELU, [first], [n]))
    second = _conv3x3(ids, a2, name + ".convolution2", size, c, c)
    return ids.op(op(OP_ADD, [second, x], [n]))


def depth_decoder(g: "Graph", cfg: DepthConfig, side: int, features, first_id: int, depth_role: int = OUTPUT):
    """The reference's decoder() (depth_anything_v2.rs:882-981): per stage a
    1x1 projection and its resampling, then a 3x3 convolution to the fusion
    width; the fusion layers deepest stage first (residual units, resampling,
    1x1 projection); the head (3x3, resample to the image side, 3x3 + ReLU,
    1x1 to one channel + ReLU). Returns (depth id, weights [(id, name,
    elements)], next id); depth is [side][side]."""
    ids = _Ids(g, first_id)
    grid = side // cfg.patch_size
    fusion = cfg.fusion_hidden_size
    stages = []
    for i, feat in enumerate(features):
        ch = cfg.neck_hidden_sizes[i]
        proj = _conv1x1(ids, feat, f"neck.reassemble_stage.layers.{i}.projection", (grid, grid), cfg.hidden_size, ch)
        kind = cfg.reassemble[i]
        if kind[0] == "up":
            f = kind[1]
            w = ids.weight(f"neck.reassemble_stage.layers.{i}.resize.weight", f * f * ch * ch)
            b = ids.weight(f"neck.reassemble_stage.layers.{i}.resize.bias", ch)
            m = ids.op(op(OP_CONV_TRANSPOSE, [proj, w, b], [grid, grid, ch, ch, f]))
            hw = (grid * f, grid * f)
        elif kind[0] == "down":
            m = _conv3x3(ids, proj, f"neck.reassemble_stage.layers.{i}.resize", (grid, grid), ch, ch, kind[1])
            hw = (_strided(grid, kind[1]), _strided(grid, kind[1]))
        else:
            m, hw = proj, (grid, grid)
        stages.append((_conv3x3(ids, m, f"neck.convs.{i}", hw, ch, fusion, bias=False), hw))
    fused = None
    for layer, (stage, hw) in enumerate(reversed(stages)):
        nxt = len(stages) - (layer + 2)
        out = stages[nxt][1] if nxt >= 0 else (hw[0] * 2, hw[1] * 2)
        name = f"neck.fusion_stage.layers.{layer}"
        x = stage
        n = hw[0] * hw[1] * fusion
        if fused is not None:
            unit = _residual_unit(ids, stage, name + ".residual_layer1", hw, fusion)
            x = ids.op(op(OP_ADD, [unit, fused[0]], [n]))
        x = _residual_unit(ids, x, name + ".residual_layer2", hw, fusion)
        resized = ids.op(op(OP_RESIZE_BILINEAR, [x], [hw[0], hw[1], out[0], out[1], fusion]))
        fused = (_conv1x1(ids, resized, name + ".projection", out, fusion, fusion), out)
    x, hw = fused
    half, width, full = fusion // 2, cfg.head_hidden_size, grid * cfg.patch_size
    first = _conv3x3(ids, x, "head.conv1", hw, fusion, half)
    resized = ids.op(op(OP_RESIZE_BILINEAR, [first], [hw[0], hw[1], full, full, half]))
    second = _conv3x3(ids, resized, "head.conv2", (full, full), half, width)
    act = ids.op(op(OP_RELU, [second], [full * full * width]))
    third = _conv1x1(ids, act, "head.conv3", (full, full), width, 1)
    depth = ids.op(op(OP_RELU, [third], [full * full]), depth_role)
    return depth, ids.weights, ids.next


@dataclass
class DepthModelIds:
    encoder: "EncoderIds"
    depth: int
    decoder_weights: list
    next_id: int


def depth_model(g: "Graph", cfg: DepthConfig, side: int | None = None, first_id: int = 0) -> DepthModelIds:
    """The reference's model() (depth_anything_v2.rs:984-995): the encoder,
    its features as activations, and the decoder reading them; the depth is
    the output."""
    side = side or cfg.image_size
    grid = side // cfg.patch_size
    enc = vit_encoder(g, grid, cfg.patch_size, cfg.num_channels, cfg.hidden_size, cfg.num_heads,
                      cfg.hidden_size * cfg.mlp_ratio, cfg.eps, cfg.out_indices, first_id, ACTIVATION)
    depth, weights, nid = depth_decoder(g, cfg, side, enc.features, enc.next_id)
    return DepthModelIds(enc, depth, weights, nid)


def output_elements(o: Op) -> int:
    return int(_lib().bli_op_output_elements(C.byref(o)))


class Program:
    def __init__(self, handle):
        self.handle = handle

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bli_program_free(self.handle)
            self.handle = None

    def __len__(self) -> int:
        return int(_lib().bli_program_len(self.handle))

    def split(self, parts) -> "Program":
        arr = (C.c_uint32 * max(1, len(parts)))(*parts)
        h = C.c_void_p()
        _check(_lib().bli_program_split(self.handle, arr, len(parts), C.byref(h)))
        return Program(h)

    def parts_within(self, durations_us, bound_us: int) -> list[int]:
        arr = (C.c_uint64 * max(1, len(durations_us)))(*durations_us)
        out = (C.c_uint32 * max(1, len(durations_us)))()
        _check(_lib().bli_program_parts_within(self.handle, arr, len(durations_us), bound_us, out))
        return list(out[: len(durations_us)])

    def fuse_attention(self) -> "Program":
        h = C.c_void_p()
        _check(_lib().bli_program_fuse_attention(self.handle, C.byref(h)))
        return Program(h)

    def set_dtype(self, dtype: int) -> "Program":
        _check(_lib().bli_program_set_dtype(self.handle, dtype))
        return self

    def kernel(self, k: int) -> KernelInfo:
        info = KernelInfo()
        _check(_lib().bli_program_kernel(self.handle, k, C.byref(info)))
        return info

    def name(self, k: int) -> str:
        buf = C.create_string_buffer(256)
        _check(_lib().bli_program_kernel_name(self.handle, k, buf, 256))
        return buf.value.decode()

    def names(self) -> list[str]:
        return [self.name(k) for k in range(len(self))]

    def bindings(self, k: int) -> list[int]:
        info = self.kernel(k)
        return list(info.bindings[: info.n_bindings])

    def tensors(self) -> list[TensorDesc]:
        n = _lib().bli_program_tensors(self.handle, None, 0)
        arr = (TensorDesc * max(1, n))()
        _lib().bli_program_tensors(self.handle, arr, n)
        return list(arr[:n])

    def lifetime(self, tid: int):
        for t in self.tensors():
            if t.id == tid:
                return (t.first_use, t.last_use)
        return None

    def role(self, tid: int) -> int:
        return int(_lib().bli_program_role(self.handle, tid))

    def stand_in(self, of: int, tid: int) -> TensorDesc:
        d = TensorDesc()
        _check(_lib().bli_program_stand_in(self.handle, of, tid, C.byref(d)))
        return d

    def spec(self, k: int, plan: "Plan") -> Spec:
        s = Spec()
        _check(_lib().bli_program_spec(self.handle, k, plan.handle, C.byref(s)))
        return s

    def specs(self, plan: "Plan") -> list[Spec]:
        return [self.spec(k, plan) for k in range(len(self))]


class Plan:
    def __init__(self, tensors, prof: Profile | None = None):
        prof = prof or profile("mi355x")
        arr = (TensorDesc * max(1, len(tensors)))(*tensors)
        h = C.c_void_p()
        _check(_lib().bli_plan_new(arr, len(tensors), C.byref(prof), C.byref(h)))
        self.handle = h

    def __del__(self):
        if getattr(self, "handle", None):
            _lib().bli_plan_free(self.handle)
            self.handle = None

    def arenas(self) -> list[int]:
        n = _lib().bli_plan_arenas(self.handle, None, 0)
        arr = (C.c_uint64 * max(1, n))()
        _lib().bli_plan_arenas(self.handle, arr, n)
        return list(arr[:n])

    def placement(self, tid: int) -> Placement | None:
        p = Placement()
        if _lib().bli_plan_placement(self.handle, tid, C.byref(p)) < 0:
            return None
        return p

    def peak_live_bytes(self) -> int:
        return int(_lib().bli_plan_peak_live_bytes(self.handle))

    def total_bytes(self) -> int:
        return int(_lib().bli_plan_total_bytes(self.handle))

    def valid_on(self, prof: Profile) -> bool:
        return bool(_lib().bli_plan_valid_on(self.handle, C.byref(prof)))


def tensor_desc(tid, dtype, elements, first, last) -> TensorDesc:
    return TensorDesc(tid, dtype, elements, first, last)


# ---------------------------------------------------------------------------
# running a graph on the device
# ---------------------------------------------------------------------------


# Job slots (crates/beatlm-host/src/slots.rs:41-151): slot 0 binds the
# program's own inputs and outputs; every later slot binds stand-ins for them
# (Program::stand_in), numbered from these bases so they never collide with
# the program's tensors. Each slot is one binding set of the kernels.
SLOT_INPUT_BASE = 1 << 16
SLOT_OUTPUT_BASE = 2 << 16
MAX_SLOTS = 1 << 16


@dataclass
class Prepared:
    """A program realised on the device once: plan, arenas, kernels, and the
    tensors each job slot reads and writes."""

    ctx: hip.Context
    program: Program
    plan: Plan
    arenas: hip.Arenas
    kernels: hip.Kernels
    dtype: int
    # slot -> {program tensor id: the tensor that slot binds in its place}
    slot_tensors: list = None
    elements: dict = None

    def np_dtype(self):
        return np.float16 if self.dtype == hip.F16 else np.float32

    def slots(self) -> int:
        return len(self.slot_tensors or [{}])

    def slot_tensor(self, tid: int, slot: int = 0) -> int:
        """The tensor slot `slot` binds for the program's input or output `tid`."""
        if not self.slot_tensors:
            if slot != 0:
                raise IndexError(f"slot {slot} of a program realised with one slot")
            return tid
        return self.slot_tensors[slot].get(tid, tid)

    def write(self, tid: int, values: np.ndarray, slot: int = 0) -> None:
        tid = self.slot_tensor(tid, slot)
        p = self.plan.placement(tid)
        if p is None:
            raise KeyError(f"tensor {tid} has no placement")
        self.arenas.write(p.arena, p.offset, np.ascontiguousarray(values, dtype=self.np_dtype()))

    def read(self, tid: int, slot: int = 0) -> np.ndarray:
        elements = self.elements[tid] if self.elements else next(t.elements for t in self.program.tensors() if t.id == tid)
        p = self.plan.placement(self.slot_tensor(tid, slot))
        return self.arenas.read(p.arena, p.offset, elements, self.np_dtype())

    def run(self, set_index: int = 0) -> None:
        self.kernels.encode_all(set_index)

    def close(self) -> None:
        """Kernels first, then the arenas they point into."""
        self.kernels.close()
        self.arenas.close()


def prepare(
    ctx: hip.Context,
    graph: Graph,
    fusion: int = FUSION_ON,
    parts: int = 1,
    flash: bool = True,
    dtype: int = hip.F32,
    slots: int = 1,
) -> Prepared:
    """Lower, optionally fuse attention, split every kernel into `parts`, plan
    against the MI355X profile (with `slots` job slots) and build the kernels."""
    program = graph.lower(fusion)
    if flash:
        program = program.fuse_attention()
    if parts != 1:
        program = program.split([parts] * len(program))
    return realise(ctx, program, dtype, slots)


def realise(ctx: hip.Context, program: Program, dtype: int = hip.F32, slots: int = 1) -> Prepared:
    """Plan `program` against the MI355X profile in `dtype` storage, allocate
    its arenas and build its kernels.

    With `slots` > 1, as the reference's Net::new (slots.rs:96-151,
    :185-240): every input and output of the program gets one stand-in per
    slot after the first, planned with the program's tensors (live for the
    whole program, so no slot shares bytes with an activation or another
    slot), and the kernels get one binding set per slot that rebinds the
    program's inputs and outputs to that slot's. Activations and weights are
    shared: jobs of different slots run one after another on the stream."""
    if not 1 <= slots <= MAX_SLOTS:
        raise ValueError(f"{slots} slots; a program has between 1 and {MAX_SLOTS}")
    program.set_dtype(dtype)
    tensors = program.tensors()
    io = [t.id for t in tensors if program.role(t.id) in (INPUT, OUTPUT)]
    descs = list(tensors)
    slot_tensors = [{tid: tid for tid in io}]
    for slot in range(1, slots):
        mine = {}
        for i, tid in enumerate(io):
            base = SLOT_INPUT_BASE if program.role(tid) == INPUT else SLOT_OUTPUT_BASE
            stand = base + slot * len(io) + i
            descs.append(program.stand_in(tid, stand))
            mine[tid] = stand
        slot_tensors.append(mine)
    plan = Plan(descs, profile("mi355x"))
    arenas = hip.Arenas(ctx, plan.arenas())
    sets = None
    if slots > 1:
        sets = []
        for mine in slot_tensors:
            subs = []
            for tid, stand in mine.items():
                p = plan.placement(stand)
                subs.append(hip.Substitution(tid, stand, p.arena, 0, p.offset, p.size))
            sets.append(subs)
    # The host never touches activations: the backend may store them its own way.
    activations = [t.id for t in tensors if program.role(t.id) == ACTIVATION]
    kernels = hip.Kernels(ctx, arenas, program.specs(plan), sets=sets, internal=activations)
    return Prepared(ctx, program, plan, arenas, kernels, dtype, slot_tensors if slots > 1 else None,
                    {t.id: t.elements for t in tensors})


def run_on_gpu(ctx, graph, values: dict[int, np.ndarray], fusion=FUSION_ON, parts=1, flash=True, dtype=hip.F32):
    """The reference's harness::run_on_gpu: every output tensor's numbers."""
    prep = prepare(ctx, graph, fusion, parts, flash, dtype)
    for tid, v in values.items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    outs = {}
    for t in prep.program.tensors():
        if prep.program.role(t.id) == OUTPUT:
            outs[t.id] = prep.read(t.id).astype(np.float32)
    return outs
