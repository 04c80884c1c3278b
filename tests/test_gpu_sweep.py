"""A seeded sweep of product and attention shapes on the GPU against the
oracle: rows, depths and widths drawn at random (ragged and whole tiles, few
and many tiles per CU, the depths and widths at which the tile rules switch
between 32x64, 64x64, 64x96, 128x64 tiles, split A, B in registers and ring
depths), in f32 storage (bf16x3 and f32 matrix math) and f16 storage, and flash attention at
random token and head counts (split and whole query tiles, runs within and
across pairs), so that every kernel the planners may pick for a shape is
checked, not only the encoder's; and the DPT head's 3x3 convolution at random
image sizes, channel counts and strides. The shapes are fixed by the seed and
named in each case's id.

Tolerance for f32 storage: |got - want| <= 1e-4 + 1e-4 |want|
(reference.rs:22-24); for f16 storage, max abs error <= 2e-2 against the
oracle on the same f16-rounded inputs.
"""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import CHAIN_OUT as Y, chain, max_abs_err

pytestmark = pytest.mark.gpu

X, W, B = 0, 1, 2
F16_TOL = 2e-2


def _matmul_shapes():
    rng = np.random.default_rng(20260)
    depths = [8, 24, 32, 64, 96, 192, 384, 640, 768, 1024, 1536, 3072]
    shapes = []
    while len(shapes) < 24:
        m = int(rng.integers(1, 5600))
        k = int(rng.choice(depths))
        n = int(rng.choice([int(rng.integers(1, 400)), 384, 768, 1024, 1152, 1536, 2304, 3072, 4096]))
        if m * k * n <= 3_000_000_000:
            shapes.append((m, k, n))
    # And shapes at the rules' edges: 128 x 64 f16 tiles (12-16 k-steps, wide),
    # with a ragged width; B in registers (long k); 64 x 96 bf16x3 tiles.
    return shapes + [(1370, 768, 2304), (1370, 1024, 4096), (2000, 1024, 1200), (1370, 3072, 768),
                     (700, 384, 1536), (1370, 4096, 1024), (333, 1024, 1056)]


def _conv_shapes():
    rng = np.random.default_rng(20262)
    shapes = []
    while len(shapes) < 14:
        h, w = int(rng.integers(1, 320)), int(rng.integers(1, 320))
        cin = int(rng.choice([3, 8, 16, 32, 48, 64, 96, 192, 384]))
        cout = int(rng.choice([1, 4, 16, 20, 32, 64, 256]))
        stride = int(rng.choice([1, 1, 2]))
        if h * w * cin * cout * 9 <= 2_000_000_000:
            shapes.append((h, w, cin, cout, stride))
    return shapes


def _attention_shapes():
    rng = np.random.default_rng(20261)
    return [(int(rng.integers(1, 2600)), int(rng.integers(1, 17))) for _ in range(10)]


MATMUL_SHAPES = _matmul_shapes()
CONV_SHAPES = _conv_shapes()
ATTENTION_SHAPES = _attention_shapes()


@pytest.mark.parametrize("m,k,n", MATMUL_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in MATMUL_SHAPES])
@pytest.mark.parametrize("math", ["bf16x3", "f32", "f16"])
def test_a_product_at_a_random_shape_matches_the_oracle(ctx, m, k, n, math):
    """f32 storage in bf16x3 and in f32 matrix math, and f16 storage."""
    f16 = math == "f16"
    if math == "f32":
        ctx.set_f32_math(hip.F32_MATH_MFMA_F32)
    a = oracle.uniform(m + 7 * k, m * k, -2.0, 2.0)
    b = oracle.fan_in_weights(n + 3 * k, k * n, k)
    bias = oracle.uniform(n + 11, n, -0.1, 0.1)
    if f16:
        a, b, bias = a.astype(np.float16), b.astype(np.float16), bias.astype(np.float16)
    g = chain({X: a, W: b, B: bias}, [ir.op(ir.OP_MATMUL, [X, W, B], [m, k, n])])
    want = oracle.matmul(a.astype(np.float32), b.astype(np.float32), bias.astype(np.float32), m, k, n)
    try:
        prep = ir.prepare(ctx, g, dtype=hip.F16 if f16 else hip.F32)
        try:
            label = prep.kernels.label(0)
            for tid, v in {X: a, W: b, B: bias}.items():
                prep.write(tid, v)
            prep.run()
            ctx.synchronize()
            got = prep.read(Y).astype(np.float32)
        finally:
            prep.close()
    finally:
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)
    if f16:
        err = max_abs_err(got, want)
        assert err <= F16_TOL, f"{m}x{k}x{n} f16 ({label}): max abs error {err:.3e}"
    else:
        bad = oracle.first_mismatch(got, want)
        assert bad is None, f"{m}x{k}x{n} {math} ({label}): element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"


@pytest.mark.parametrize("h,w,cin,cout,stride", CONV_SHAPES, ids=[f"{h}x{w}x{ci}to{co}s{st}" for h, w, ci, co, st in CONV_SHAPES])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_a_convolution_at_a_random_shape_matches_the_oracle(ctx, h, w, cin, cout, stride, f16):
    """The DPT head's 3x3 convolution (direct, implicit GEMM with or without
    split k, 128 x 32 tiles, the element-wise gather for narrow channels, as
    the planner picks for the shape), with bias."""
    x = oracle.uniform(h + w + cin, h * w * cin, -2.0, 2.0)
    wt = oracle.fan_in_weights(cout + 5 * cin, 9 * cin * cout, 9 * cin)
    b = oracle.uniform(cout + 17, cout, -0.1, 0.1)
    if f16:
        x, wt, b = x.astype(np.float16), wt.astype(np.float16), b.astype(np.float16)
    vals = {0: x, 1: wt, 2: b}
    g = chain(vals, [ir.op(ir.OP_CONV3X3, [0, 1, 2], [h, w, cin, cout, stride])])
    want = oracle.conv3x3(x.astype(np.float32), wt.astype(np.float32), b.astype(np.float32), h, w, cin, cout, stride)
    got = ir.run_on_gpu(ctx, g, vals, dtype=hip.F16 if f16 else hip.F32)[Y].astype(np.float32)
    if f16:
        err = max_abs_err(got, want)
        assert err <= F16_TOL, f"conv {h}x{w}x{cin}->{cout} s{stride} f16: max abs error {err:.3e}"
    else:
        bad = oracle.first_mismatch(got, want)
        assert bad is None, f"conv {h}x{w}x{cin}->{cout} s{stride}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"


def attention_graph(t, h, d):
    g = ir.Graph()
    g.tensor(X, ir.INPUT, t * 3 * h * d)
    g.tensor(10, ir.ACTIVATION, t * h * t)
    g.push(ir.op(ir.OP_ATTENTION_SCORES, [X], [t, h, d]), 10)
    g.tensor(11, ir.ACTIVATION, t * h * t)
    g.push(ir.op(ir.OP_SCALE, [10], [t * h * t], 1.0 / np.sqrt(d)), 11)
    g.tensor(12, ir.ACTIVATION, t * h * t)
    g.push(ir.op(ir.OP_SOFTMAX, [11], [t * h, t]), 12)
    g.tensor(Y, ir.OUTPUT, t * h * d)
    g.push(ir.op(ir.OP_ATTENTION_VALUES, [12, X], [t, h, d]), Y)
    return g


@pytest.mark.parametrize("t,h", ATTENTION_SHAPES, ids=[f"t{t}h{h}" for t, h in ATTENTION_SHAPES])
@pytest.mark.parametrize("f16", [False, True], ids=["f32", "f16"])
def test_flash_attention_at_a_random_shape_matches_the_oracle(ctx, t, h, f16):
    qkv = oracle.uniform(t + 100 * h, t * 3 * h * 64, -1.0, 1.0)
    if f16:
        qkv = qkv.astype(np.float16)
    g = attention_graph(t, h, 64)
    assert g.lower().fuse_attention().names() == ["flash_attention"]
    want = oracle.attention(qkv.astype(np.float32), t, h, 64, 0.125)
    got = ir.run_on_gpu(ctx, g, {X: qkv}, dtype=hip.F16 if f16 else hip.F32)[Y].astype(np.float32)
    if f16:
        err = max_abs_err(got, want)
        assert err <= F16_TOL, f"t={t} h={h} f16: max abs error {err:.3e}"
    else:
        bad = oracle.first_mismatch(got, want)
        assert bad is None, f"t={t} h={h}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"
