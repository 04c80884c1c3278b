"""The oracle: ctypes wrapper of oracle/build/liboracle.so.

TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it as the checker (or, for the CPU baseline, as the
reference path timed on the host). The product library never imports it.

`ref_*` are the reference's f64 CPU reference ops
(crates/beatlm-bench/src/reference.rs); `wg_*` the reference's WGSL kernels'
f32 arithmetic in their order (crates/beatlm/src/codegen/wgsl.rs).
"""

from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB = HERE / "build" / "liboracle.so"

# reference.rs:22-24
TOLERANCE_ABS = 1e-4
TOLERANCE_REL = 1e-4

_lib = None
_F = C.POINTER(C.c_float)
_S = C.c_size_t


class BlockWeights(C.Structure):
    _fields_ = [
        (n, _F)
        for n in (
            "norm1_g", "norm1_b", "qkv_w", "qkv_b", "proj_w", "proj_b", "ls1",
            "norm2_g", "norm2_b", "fc1_w", "fc1_b", "fc2_w", "fc2_b", "ls2",
        )
    ]


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        h = C.CDLL(str(LIB))
        sig = {
            "blo_uniform": [C.c_uint64, _S, C.c_float, C.c_float, _F],
            "blo_normal": [C.c_uint64, _S, C.c_float, C.c_float, _F],
            "blo_ref_layernorm": [_F, _F, _F, _S, _S, C.c_float, _F],
            "blo_ref_matmul": [_F, _F, _F, _S, _S, _S, _F],
            "blo_ref_add": [_F, _F, _S, _F],
            "blo_ref_relu": [_F, _S, _F],
            "blo_ref_gelu_tanh": [_F, _S, _F],
            "blo_ref_scale": [_F, _S, C.c_float, _F],
            "blo_ref_gelu_erf": [_F, _S, _F],
            "blo_ref_channel_scale": [_F, _F, _S, _S, _F],
            "blo_ref_attention_scores": [_F, _S, _S, _S, _F],
            "blo_ref_softmax": [_F, _S, _S, _F],
            "blo_ref_attention_values": [_F, _F, _S, _S, _S, _F],
            "blo_ref_attention": [_F, _S, _S, _S, C.c_float, _F],
            "blo_ref_patch_embed": [_F, _F, _F, _S, _S, _S, _S, _S, _F],
            "blo_ref_prepend_token": [_F, _F, _S, _S, _F],
            "blo_ref_conv3x3": [_F, _F, _F, _S, _S, _S, _S, _S, _F],
            "blo_ref_conv1x1": [_F, _F, _F, _S, _S, _S, _F],
            "blo_ref_conv_transpose": [_F, _F, _F, _S, _S, _S, _S, _S, _F],
            "blo_ref_resize_bilinear": [_F, _S, _S, _S, _S, _S, _F],
            "blo_ref_vit_block": [_F, C.POINTER(BlockWeights), _S, _S, _S, _S, C.c_float, C.c_int, _F],
            "blo_wg_layernorm": [_F, _F, _F, _S, _S, C.c_float, _F],
            "blo_wg_softmax": [_F, _S, _S, _F],
            "blo_wg_matmul": [_F, _F, _F, _S, _S, _S, _F],
            "blo_wg_block_scratch_floats": [_S, _S, _S, _S],
            "blo_wg_vit_block": [_F, C.POINTER(BlockWeights), _S, _S, _S, _S, C.c_float, C.c_int, _F, _F],
        }
        for name, args in sig.items():
            getattr(h, name).argtypes = args
            getattr(h, name).restype = None
        h.blo_erf.argtypes = [C.c_double]
        h.blo_erf.restype = C.c_double
        h.blo_wg_gelu_erf1.argtypes = [C.c_float]
        h.blo_wg_gelu_erf1.restype = C.c_float
        h.blo_wg_block_scratch_floats.restype = C.c_size_t
        _lib = h
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle arrays are contiguous f32"
    return a.ctypes.data_as(_F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- generators ----

def uniform(seed: int, count: int, low: float, high: float) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().blo_uniform(seed, count, low, high, _p(out))
    return out


def normal(seed: int, count: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().blo_normal(seed, count, mean, std, _p(out))
    return out


def fan_in_weights(seed: int, count: int, fan_in: int) -> np.ndarray:
    """U(+-1/sqrt(fan_in)), the reference's test weights (harness.rs:80-84)."""
    s = np.float32(1.0) / np.sqrt(np.float32(fan_in))
    return uniform(seed, count, -s, s)


def xavier(seed: int, fan_in: int, fan_out: int) -> np.ndarray:
    """Xavier-uniform U(+-sqrt(6 / (fan_in + fan_out)))."""
    a = float(np.sqrt(6.0 / (fan_in + fan_out)))
    return uniform(seed, fan_in * fan_out, -a, a)


# ---- f64 reference ops ----

def erf(x: float) -> float:
    return float(lib().blo_erf(x))


def layernorm(x, gamma, beta, rows, c, eps):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty(rows * c, np.float32)
    lib().blo_ref_layernorm(_p(x), _p(gamma), _p(beta), rows, c, eps, _p(out))
    return out


def matmul(a, b, bias, m, k, n):
    a, b = _f32(a), _f32(b)
    keep = _f32(bias) if bias is not None else None
    out = np.empty(m * n, np.float32)
    lib().blo_ref_matmul(_p(a), _p(b), _p(keep) if keep is not None else None, m, k, n, _p(out))
    return out


def add(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty(a.size, np.float32)
    lib().blo_ref_add(_p(a), _p(b), a.size, _p(out))
    return out


def relu(x):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_relu(_p(x), x.size, _p(out))
    return out


def gelu_tanh(x):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_gelu_tanh(_p(x), x.size, _p(out))
    return out


def scale(x, f):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_scale(_p(x), x.size, f, _p(out))
    return out


def gelu_erf(x):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_gelu_erf(_p(x), x.size, _p(out))
    return out


def channel_scale(x, s):
    x, s = _f32(x), _f32(s)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_channel_scale(_p(x), _p(s), x.size, s.size, _p(out))
    return out


def attention_scores(qkv, t, h, d):
    qkv = _f32(qkv)
    out = np.empty(t * h * t, np.float32)
    lib().blo_ref_attention_scores(_p(qkv), t, h, d, _p(out))
    return out


def softmax(x, cols):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_ref_softmax(_p(x), x.size // cols, cols, _p(out))
    return out


def attention_values(probs, qkv, t, h, d):
    probs, qkv = _f32(probs), _f32(qkv)
    out = np.empty(t * h * d, np.float32)
    lib().blo_ref_attention_values(_p(probs), _p(qkv), t, h, d, _p(out))
    return out


def attention(qkv, t, h, d, scale_factor):
    qkv = _f32(qkv)
    out = np.empty(t * h * d, np.float32)
    lib().blo_ref_attention(_p(qkv), t, h, d, scale_factor, _p(out))
    return out


def patch_embed(image, w, bias, gh, gw, p, cin, cout):
    image, w = _f32(image), _f32(w)
    out = np.empty(gh * gw * cout, np.float32)
    keep = _f32(bias) if bias is not None else None
    lib().blo_ref_patch_embed(_p(image), _p(w), _p(keep) if keep is not None else None, gh, gw, p, cin, cout, _p(out))
    return out


def prepend_token(token, tokens, rows, c):
    token, tokens = _f32(token), _f32(tokens)
    out = np.empty((rows + 1) * c, np.float32)
    lib().blo_ref_prepend_token(_p(token), _p(tokens), rows, c, _p(out))
    return out


def _opt(bias):
    return _f32(bias) if bias is not None else None


def conv3x3(x, w, bias, h, wd, cin, cout, stride=1):
    """reference.rs:31-81: NHWC x, HWIO w [3][3][cin][cout], padding 1."""
    x, w, b = _f32(x), _f32(w), _opt(bias)
    oh, ow = (h - 1) // stride + 1, (wd - 1) // stride + 1
    out = np.empty(oh * ow * cout, np.float32)
    lib().blo_ref_conv3x3(_p(x), _p(w), _p(b) if b is not None else None, h, wd, cin, cout, stride, _p(out))
    return out


def conv1x1(x, w, bias, pixels, cin, cout):
    """reference.rs:87-106."""
    x, w, b = _f32(x), _f32(w), _opt(bias)
    out = np.empty(pixels * cout, np.float32)
    lib().blo_ref_conv1x1(_p(x), _p(w), _p(b) if b is not None else None, pixels, cin, cout, _p(out))
    return out


def conv_transpose(x, w, bias, h, wd, cin, cout, f):
    """reference.rs:114-144: kernel = stride = f, HWIO w [f][f][cin][cout]."""
    x, w, b = _f32(x), _f32(w), _opt(bias)
    out = np.empty(h * f * wd * f * cout, np.float32)
    lib().blo_ref_conv_transpose(_p(x), _p(w), _p(b) if b is not None else None, h, wd, cin, cout, f, _p(out))
    return out


def resize_bilinear(x, ih, iw, oh, ow, c):
    """reference.rs:151-179: aligned corners."""
    x = _f32(x)
    out = np.empty(oh * ow * c, np.float32)
    lib().blo_ref_resize_bilinear(_p(x), ih, iw, oh, ow, c, _p(out))
    return out


def _weights_struct(w: dict):
    arrays = {k: _f32(v) for k, v in w.items()}
    s = BlockWeights(**{k: _p(v) for k, v in arrays.items()})
    return s, arrays


def vit_block(x, w: dict, t, h, d, mlp, eps, attention_rounded=True):
    x = _f32(x)
    s, keep = _weights_struct(w)
    out = np.empty(t * h * d, np.float32)
    lib().blo_ref_vit_block(_p(x), C.byref(s), t, h, d, mlp, eps, 1 if attention_rounded else 0, _p(out))
    del keep
    return out


def depth_decoder(cfg, side, features, w):
    """The DPT decoder composed from the ops above, as the reference composes
    it (crates/beatlm-bench/src/reference.rs:194-244 for the residual unit and
    fusion layer, crates/beatlm/src/model/depth_anything_v2.rs:882-981 for the
    stages and the head). `cfg` carries the configuration's fields (patch
    size, hidden size, neck sizes, resamplings, fusion and head widths);
    `features` the four [grid][grid][hidden] maps; `w` the weights by the
    checkpoint's names, convolutions HWIO. Returns the [side][side] depth."""
    grid, F = side // cfg.patch_size, cfg.fusion_hidden_size
    stages = []
    for i, feat in enumerate(features):
        ch = cfg.neck_hidden_sizes[i]
        pre = f"neck.reassemble_stage.layers.{i}"
        m = conv1x1(feat, w[pre + ".projection.weight"], w[pre + ".projection.bias"], grid * grid, cfg.hidden_size, ch)
        kind = cfg.reassemble[i]
        if kind[0] == "up":
            f = kind[1]
            m = conv_transpose(m, w[pre + ".resize.weight"], w[pre + ".resize.bias"], grid, grid, ch, ch, f)
            hw = (grid * f, grid * f)
        elif kind[0] == "down":
            m = conv3x3(m, w[pre + ".resize.weight"], w[pre + ".resize.bias"], grid, grid, ch, ch, kind[1])
            hw = ((grid - 1) // kind[1] + 1,) * 2
        else:
            hw = (grid, grid)
        stages.append((conv3x3(m, w[f"neck.convs.{i}.weight"], None, hw[0], hw[1], ch, F), hw))

    def unit(x, name, hw):
        a = conv3x3(relu(x), w[name + ".convolution1.weight"], w[name + ".convolution1.bias"], hw[0], hw[1], F, F)
        b = conv3x3(relu(a), w[name + ".convolution2.weight"], w[name + ".convolution2.bias"], hw[0], hw[1], F, F)
        return add(b, x)

    fused, hw_out = None, None
    for layer, (stage, hw) in enumerate(reversed(stages)):
        nxt = len(stages) - (layer + 2)
        out = stages[nxt][1] if nxt >= 0 else (hw[0] * 2, hw[1] * 2)
        name = f"neck.fusion_stage.layers.{layer}"
        x = stage if fused is None else add(unit(stage, name + ".residual_layer1", hw), fused)
        x = unit(x, name + ".residual_layer2", hw)
        r = resize_bilinear(x, hw[0], hw[1], out[0], out[1], F)
        fused = conv1x1(r, w[name + ".projection.weight"], w[name + ".projection.bias"], out[0] * out[1], F, F)
        hw_out = out
    full = grid * cfg.patch_size
    first = conv3x3(fused, w["head.conv1.weight"], w["head.conv1.bias"], hw_out[0], hw_out[1], F, F // 2)
    r = resize_bilinear(first, hw_out[0], hw_out[1], full, full, F // 2)
    second = relu(conv3x3(r, w["head.conv2.weight"], w["head.conv2.bias"], full, full, F // 2, cfg.head_hidden_size))
    third = conv1x1(second, w["head.conv3.weight"], w["head.conv3.bias"], full * full, cfg.head_hidden_size, 1)
    return relu(third)


# ---- WGSL-order emulation ----

def wg_gelu_erf(x):
    return np.array([lib().blo_wg_gelu_erf1(float(v)) for v in np.asarray(x, np.float32)], np.float32)


def wg_layernorm(x, gamma, beta, rows, c, eps):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty(rows * c, np.float32)
    lib().blo_wg_layernorm(_p(x), _p(gamma), _p(beta), rows, c, eps, _p(out))
    return out


def wg_softmax(x, cols):
    x = _f32(x)
    out = np.empty(x.size, np.float32)
    lib().blo_wg_softmax(_p(x), x.size // cols, cols, _p(out))
    return out


def wg_matmul(a, b, bias, m, k, n):
    a, b = _f32(a), _f32(b)
    keep = _f32(bias) if bias is not None else None
    out = np.empty(m * n, np.float32)
    lib().blo_wg_matmul(_p(a), _p(b), _p(keep) if keep is not None else None, m, k, n, _p(out))
    return out


class WgBlock:
    """The reference's 9 fused kernels of one block on the host, with its
    scratch allocated once so repeated runs time only the arithmetic."""

    def __init__(self, w: dict, t, h, d, mlp, eps, threads=0):
        self.s, self.keep = _weights_struct(w)
        self.t, self.h, self.d, self.mlp, self.eps, self.threads = t, h, d, mlp, eps, threads
        n = lib().blo_wg_block_scratch_floats(t, h, d, mlp)
        self.scratch = np.empty(n, np.float32)

    def __call__(self, x):
        x = _f32(x)
        out = np.empty(self.t * self.h * self.d, np.float32)
        lib().blo_wg_vit_block(
            _p(x), C.byref(self.s), self.t, self.h, self.d, self.mlp, self.eps, self.threads,
            _p(self.scratch), _p(out),
        )
        return out


def within_tolerance(got, want, abs_tol=TOLERANCE_ABS, rel_tol=TOLERANCE_REL) -> np.ndarray:
    """reference.rs:629-632; false for a NaN on either side."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    with np.errstate(invalid="ignore"):
        return np.abs(got - want) <= abs_tol + rel_tol * np.abs(want)


def first_mismatch(got, want, abs_tol=TOLERANCE_ABS, rel_tol=TOLERANCE_REL):
    """reference.rs:635-645: (index, got, want) of the first element outside
    the tolerance, or None."""
    got = np.asarray(got, np.float32).ravel()
    want = np.asarray(want, np.float32).ravel()
    if got.size != want.size:
        return (min(got.size, want.size), float("nan"), float("nan"))
    bad = np.flatnonzero(~within_tolerance(got, want, abs_tol, rel_tol))
    if bad.size == 0:
        return None
    i = int(bad[0])
    return (i, float(got[i]), float(want[i]))
