"""GPU parity of each kernel against the oracle, at the shapes of DINOv2 Small
at 518 pixels (1370 tokens, 384 channels, 6 heads of 64) and at small ragged
shapes, whole and split into parts, fused and unfused — the reference's
crates/beatlm-bench/src/vit.rs:53-203 through this backend's C ABI.

Tolerance for f32 storage: |got - want| <= 1e-4 + 1e-4 |want|
(reference.rs:22-24). For f16 storage: max abs error <= 2e-2 against the
oracle evaluated on the same f16-rounded inputs.
"""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import CHAIN as H_, CHAIN_OUT as Y, chain, max_abs_err

pytestmark = pytest.mark.gpu

TOKENS, WIDTH, HEADS, HEAD_DIM = 1370, 384, 6, 64
GRID, PATCH = 37, 14
X, W, B = 0, 1, 2
PARTS = [1, 3, 7, 22, 200]
F16_TOL = 2e-2


def assert_close(got, want, what):
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"


def assert_chain_matches(ctx, what, g, inputs, parts=PARTS, flash=True):
    """harness.rs:52-76: fused and unfused, whole and in parts, against the
    oracle and against the whole run."""
    want = inputs["__want__"]
    values = {k: v for k, v in inputs.items() if k != "__want__"}
    for fusion in (ir.FUSION_ON, ir.FUSION_OFF):
        whole = ir.run_on_gpu(ctx, g, values, fusion, 1, flash)[Y]
        for count in parts:
            got = ir.run_on_gpu(ctx, g, values, fusion, count, flash)[Y]
            case = f"{what}, fusion {fusion}, {count} parts"
            assert_close(got, want, case)
            assert_close(got, whole, case + ", against whole")


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
@pytest.mark.parametrize(
    "m,k,n",
    [(1370, 384, 1152), (1370, 384, 384), (1370, 384, 1536), (1370, 1536, 384), (257, 384, 1536), (17, 5, 7), (100, 40, 33), (1, 3, 1)],
)
def test_matmul_with_bias_matches_the_oracle(ctx, math, m, k, n):
    ctx.set_f32_math(math)
    try:
        a = oracle.uniform(1, m * k, -2.0, 2.0)
        b = oracle.fan_in_weights(2, k * n, k)
        bias = oracle.uniform(3, n, -0.1, 0.1)
        o = ir.op(ir.OP_MATMUL, [X, W, B], [m, k, n])
        g = chain({X: a, W: b, B: bias}, [o])
        want = oracle.matmul(a, b, bias, m, k, n)
        for parts in (1, 3):
            got = ir.run_on_gpu(ctx, g, {X: a, W: b, B: bias}, parts=parts)[Y]
            assert_close(got, want, f"matmul {m}x{k}x{n} math {math} parts {parts}")
    finally:
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)


@pytest.mark.parametrize("m,k,n", [(1370, 384, 1152), (1370, 1536, 384), (5477, 384, 1536), (17, 8, 24)])
def test_matmul_in_f16_is_within_its_tolerance(ctx, m, k, n):
    a = oracle.uniform(4, m * k, -2.0, 2.0).astype(np.float16)
    b = oracle.fan_in_weights(5, k * n, k).astype(np.float16)
    bias = oracle.uniform(6, n, -0.1, 0.1).astype(np.float16)
    o = ir.op(ir.OP_MATMUL, [X, W, B], [m, k, n])
    g = chain({X: a, W: b, B: bias}, [o])
    want = oracle.matmul(a.astype(np.float32), b.astype(np.float32), bias.astype(np.float32), m, k, n)
    got = ir.run_on_gpu(ctx, g, {X: a, W: b, B: bias}, dtype=hip.F16)[Y]
    assert max_abs_err(got, want) <= F16_TOL


def test_matmul_epilogues_channel_scale_then_add(ctx):
    m, k, n = 1370, 384, 384
    a = oracle.uniform(7, m * k, -2.0, 2.0)
    b = oracle.fan_in_weights(8, k * n, k)
    bias = oracle.uniform(9, n, -0.1, 0.1)
    ls = oracle.uniform(10, n, 0.1, 1.0)
    res = oracle.uniform(11, m * n, -2.0, 2.0)
    ops = [
        ir.op(ir.OP_MATMUL, [X, W, B], [m, k, n]),
        ir.op(ir.OP_CHANNEL_SCALE, [H_, 3], [m, n]),
        ir.op(ir.OP_ADD, [H_ + 1, 4], [m * n]),
    ]
    inputs = {X: a, W: b, B: bias, 3: ls, 4: res}
    g = chain(inputs, ops)
    assert g.lower().names() == ["matmul+channel_scale+add"]
    want = oracle.add(oracle.channel_scale(oracle.matmul(a, b, bias, m, k, n), ls), res)
    assert_chain_matches(ctx, "matmul+channel_scale+add", g, {**inputs, "__want__": want}, parts=[1, 3, 22])


def test_layernorm_matches_the_oracle_at_the_block_width(ctx):
    x = oracle.uniform(12, TOKENS * WIDTH, -2.0, 2.0)
    gamma = oracle.uniform(13, WIDTH, 0.8, 1.2)
    beta = oracle.uniform(14, WIDTH, -0.1, 0.1)
    o = ir.op(ir.OP_LAYER_NORM, [X, W, B], [TOKENS, WIDTH], 1e-6)
    inputs = {X: x, W: gamma, B: beta}
    g = chain(inputs, [o])
    want = oracle.layernorm(x, gamma, beta, TOKENS, WIDTH, 1e-6)
    assert_chain_matches(ctx, "layer norm", g, {**inputs, "__want__": want})


@pytest.mark.parametrize("rows,c", [(5, 1), (3, 7), (11, 1024), (2, 2000), (1370, 768)])
def test_layernorm_at_other_widths(ctx, rows, c):
    x = oracle.uniform(15, rows * c, -3.0, 3.0)
    gamma = oracle.uniform(16, c, 0.8, 1.2)
    beta = oracle.uniform(17, c, -0.1, 0.1)
    g = chain({X: x, W: gamma, B: beta}, [ir.op(ir.OP_LAYER_NORM, [X, W, B], [rows, c], 1e-5)])
    got = ir.run_on_gpu(ctx, g, {X: x, W: gamma, B: beta})[Y]
    if c == 1:
        # A constant row: (x - mean) is exactly zero, the output is beta.
        assert np.array_equal(got, np.tile(beta, rows))
    assert_close(got, oracle.layernorm(x, gamma, beta, rows, c, 1e-5), f"layer norm {rows}x{c}")


def test_the_scaled_attention_scores_match_the_oracle(ctx):
    qkv = oracle.uniform(7, TOKENS * 3 * WIDTH, -1.0, 1.0)
    ops = [
        ir.op(ir.OP_ATTENTION_SCORES, [X], [TOKENS, HEADS, HEAD_DIM]),
        ir.op(ir.OP_SCALE, [H_], [TOKENS * HEADS * TOKENS], 0.125),
    ]
    g = chain({X: qkv}, ops)
    want = oracle.scale(oracle.attention_scores(qkv, TOKENS, HEADS, HEAD_DIM), 0.125)
    assert_chain_matches(ctx, "attention scores", g, {X: qkv, "__want__": want}, parts=[1, 3, 22])


def test_the_softmax_matches_the_oracle_over_attention_rows(ctx):
    scores = oracle.uniform(8, TOKENS * HEADS * TOKENS, -8.0, 8.0)
    scores[::9973] = 120.0
    g = chain({X: scores}, [ir.op(ir.OP_SOFTMAX, [X], [TOKENS * HEADS, TOKENS])])
    want = oracle.softmax(scores, TOKENS)
    assert_chain_matches(ctx, "softmax", g, {X: scores, "__want__": want}, parts=[1, 7, 200])
    got = ir.run_on_gpu(ctx, g, {X: scores})[Y]
    assert np.isfinite(got).all()


def test_the_weighted_sum_of_the_values_matches_the_oracle(ctx):
    qkv = oracle.uniform(9, TOKENS * 3 * WIDTH, -1.0, 1.0)
    raw = oracle.uniform(10, TOKENS * HEADS * TOKENS, -4.0, 4.0)
    probs = oracle.softmax(raw, TOKENS)
    o = ir.op(ir.OP_ATTENTION_VALUES, [W, X], [TOKENS, HEADS, HEAD_DIM])
    g = chain({X: qkv, W: probs}, [o])
    want = oracle.attention_values(probs, qkv, TOKENS, HEADS, HEAD_DIM)
    assert_chain_matches(ctx, "attention values", g, {X: qkv, W: probs, "__want__": want}, parts=[1, 3, 22])


def attention_chain(t, h, d, qkv):
    ops = [
        ir.op(ir.OP_ATTENTION_SCORES, [X], [t, h, d]),
        ir.op(ir.OP_SCALE, [H_], [t * h * t], 1.0 / np.sqrt(d)),
        ir.op(ir.OP_SOFTMAX, [H_ + 1], [t * h, t]),
        ir.op(ir.OP_ATTENTION_VALUES, [H_ + 2, X], [t, h, d]),
    ]
    return chain({X: qkv}, ops)


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
@pytest.mark.parametrize("t,h", [(1370, 6), (257, 6), (17, 2), (64, 1), (65, 3), (1, 2), (5477, 6)])
def test_flash_attention_matches_the_oracle(ctx, math, t, h):
    ctx.set_f32_math(math)
    try:
        qkv = oracle.uniform(20 + t, t * 3 * h * 64, -1.0, 1.0)
        g = attention_chain(t, h, 64, qkv)
        prog = g.lower().fuse_attention()
        assert prog.names() == ["flash_attention"]
        want = oracle.attention(qkv, t, h, 64, 0.125)
        for parts in (1, 3):
            got = ir.run_on_gpu(ctx, g, {X: qkv}, parts=parts)[Y]
            assert_close(got, want, f"flash attention t={t} h={h} math {math} parts {parts}")
    finally:
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)


@pytest.mark.parametrize("t,h", [(1370, 6), (1370, 12), (5477, 6), (33, 2)])
def test_flash_attention_in_f16(ctx, t, h):
    qkv = oracle.uniform(40 + t, t * 3 * h * 64, -1.0, 1.0).astype(np.float16)
    g = attention_chain(t, h, 64, qkv)
    want = oracle.attention(qkv.astype(np.float32), t, h, 64, 0.125)
    got = ir.run_on_gpu(ctx, g, {X: qkv}, dtype=hip.F16)[Y]
    assert max_abs_err(got, want) <= F16_TOL


def test_unfused_attention_at_a_tiny_ragged_shape(ctx):
    # d = 5 has no flash kernel: the three kernels run as the reference's.
    t, h, d = 17, 2, 5
    qkv = oracle.uniform(50, t * 3 * h * d, -1.0, 1.0)
    g = attention_chain(t, h, d, qkv)
    assert len(g.lower().fuse_attention()) == 3
    want = oracle.attention_values(
        oracle.softmax(oracle.scale(oracle.attention_scores(qkv, t, h, d), np.float32(1 / np.sqrt(d))), t), qkv, t, h, d
    )
    assert_chain_matches(ctx, "attention t=17 d=5", g, {X: qkv, "__want__": want}, parts=[1, 3])


def test_gelu_erf_and_layerscale_match_the_oracle_at_the_mlp_width(ctx):
    mlp = 4 * WIDTH
    x = oracle.uniform(11, TOKENS * mlp, -6.0, 6.0)
    s = oracle.uniform(12, mlp, 0.1, 1.0)
    ops = [ir.op(ir.OP_GELU_ERF, [X], [TOKENS * mlp]), ir.op(ir.OP_CHANNEL_SCALE, [H_, W], [TOKENS, mlp])]
    want = oracle.channel_scale(oracle.gelu_erf(x), s)
    assert_chain_matches(ctx, "GELU (erf), LayerScale", chain({X: x, W: s}, ops), {X: x, W: s, "__want__": want})


def test_gelu_erf_on_the_gpu_is_within_its_stated_error(ctx):
    # vit.rs:179-204: the grid of kernel.rs:364-366 against GELU through f64 erf.
    grid = (-10.0 + np.arange(81921, dtype=np.float64) / 4096.0).astype(np.float32)
    g = chain({X: grid}, [ir.op(ir.OP_GELU_ERF, [X], [grid.size])])
    got = ir.run_on_gpu(ctx, g, {X: grid})[Y].astype(np.float64)
    exact = np.array([0.5 * v * (1.0 + oracle.erf(v / np.sqrt(2.0))) for v in grid.astype(np.float64)])
    err = np.abs(got - exact)
    assert err.max() <= 5e-7, f"{err.max():e} at x = {grid[err.argmax()]}"


def test_the_patch_embedding_matches_the_oracle_at_518_pixels(ctx):
    side = GRID * PATCH
    image = oracle.uniform(1, side * side * 3, -2.0, 2.0)
    w = oracle.fan_in_weights(2, PATCH * PATCH * 3 * WIDTH, PATCH * PATCH * 3)
    b = oracle.uniform(3, WIDTH, -0.1, 0.1)
    o = ir.op(ir.OP_PATCH_EMBED, [X, W, B], [GRID, GRID, PATCH, 3, WIDTH])
    inputs = {X: image, W: w, B: b}
    want = oracle.patch_embed(image, w, b, GRID, GRID, PATCH, 3, WIDTH)
    assert_chain_matches(ctx, "patch embedding", chain(inputs, [o]), {**inputs, "__want__": want}, parts=[1, 7, 22])


def test_the_class_token_position_add_and_token_drop_match_the_oracle(ctx):
    patches = oracle.uniform(4, (TOKENS - 1) * WIDTH, -1.0, 1.0)
    token = oracle.uniform(5, WIDTH, -1.0, 1.0)
    positions = oracle.uniform(6, TOKENS * WIDTH, -1.0, 1.0)
    ops = [
        ir.op(ir.OP_PREPEND_TOKEN, [W, X], [TOKENS - 1, WIDTH]),
        ir.op(ir.OP_ADD, [H_, B], [TOKENS * WIDTH]),
        ir.op(ir.OP_TOKENS_TO_MAP, [H_ + 1], [GRID, GRID, WIDTH]),
    ]
    inputs = {X: patches, W: token, B: positions}
    g = chain(inputs, ops)
    assert len(g.lower()) == 2
    want = oracle.add(oracle.prepend_token(token, patches, TOKENS - 1, WIDTH), positions)[WIDTH:]
    assert_chain_matches(ctx, "class token, position add, token drop", g, {**inputs, "__want__": want})


@pytest.mark.parametrize("m,k,n,bias", [(268324, 32, 1, True), (1000, 64, 4, True), (777, 12, 3, False),
                                        (5, 4, 2, True), (333, 10, 1, True)])
def test_products_with_few_columns_match_the_oracle(ctx, m, k, n, bias):
    """At most 4 columns with k a multiple of 4 take the GEMV kernel (the
    depth head's 1x1 convolution to one channel); k = 10 keeps the tiled
    GEMM. f32 (1e-4) and f16 (2e-2), whole and in parts, with ReLU after."""
    a = oracle.uniform(31, m * k, -2.0, 2.0)
    b = oracle.fan_in_weights(32, k * n, k)
    vals = {X: a, W: b}
    if bias:
        vals[B] = oracle.uniform(33, n, -0.1, 0.1)
    o = ir.op(ir.OP_MATMUL, [X, W, B if bias else ir.NONE], [m, k, n])
    g = chain(vals, [o, ir.op(ir.OP_RELU, [H_], [m * n])])
    labels = ir.prepare(ctx, g).program.names()
    assert labels == ["matmul+relu"]
    want = oracle.relu(oracle.matmul(a, b, vals.get(B), m, k, n))
    for parts in (1, 3):
        assert_close(ir.run_on_gpu(ctx, g, vals, parts=parts)[Y], want, f"matmul {m}x{k}x{n} parts {parts}")
    v16 = {t: v.astype(np.float16) for t, v in vals.items()}
    want16 = oracle.relu(oracle.matmul(*(v16[t].astype(np.float32) if t in v16 else None for t in (X, W, B)), m, k, n))
    assert max_abs_err(ir.run_on_gpu(ctx, g, v16, dtype=hip.F16)[Y], want16) <= F16_TOL


@pytest.mark.parametrize("t,h,f16", [(1370, 6, False), (1370, 12, True), (257, 6, False), (5477, 6, True)])
def test_flash_attention_merges_split_tiles_in_kernel_launch_after_launch(ctx, monkeypatch, t, h, f16):
    """The runs that split a query tile's key tiles merge it inside the flash
    kernel (arrival counters that every launch leaves at zero): six launches
    in a row give the same bits, and the same bits as the merge launched as a
    kernel of its own, both within tolerance of the oracle."""
    dtype = hip.F16 if f16 else hip.F32
    qkv = oracle.uniform(60 + t, t * 3 * h * 64, -1.0, 1.0)
    if f16:
        qkv = qkv.astype(np.float16)
    g = attention_chain(t, h, 64, qkv)
    want = oracle.attention(qkv.astype(np.float32), t, h, 64, 0.125)

    def outputs(runs):
        prep = ir.prepare(ctx, g, dtype=dtype)
        try:
            label = prep.kernels.label(0)
            prep.write(X, qkv)
            got = []
            for _ in range(runs):
                prep.run()
                ctx.synchronize()
                got.append(prep.read(Y))
            return label, got
        finally:
            prep.close()

    label, inline = outputs(6)
    assert "merged in-kernel" in label, label
    for i, o in enumerate(inline[1:]):
        assert np.array_equal(o, inline[0]), f"launch {i + 1} differs from launch 0"
    err = max_abs_err(inline[0], want)
    assert err <= (F16_TOL if f16 else 1e-4), f"max abs error {err}"
    monkeypatch.setenv("BL_FLASH_MERGE_LAUNCH", "1")
    label2, launched = outputs(1)
    assert "merged" in label2 and "in-kernel" not in label2, label2
    assert np.array_equal(launched[0], inline[0])


@pytest.mark.parametrize("m,k,n,f16,force", [(1370, 1536, 384, False, False), (1370, 3072, 768, True, False),
                                             (1370, 384, 1152, False, True), (1370, 384, 1536, True, True)])
def test_matmul_with_b_in_registers_matches_the_oracle(ctx, monkeypatch, m, k, n, f16, force):
    """Products whose k is long against their width take B straight into
    registers from a fragment-major pack (the MLP's second product); forced
    onto wide products too, the result is the oracle's."""
    if force:
        monkeypatch.setenv("BL_GEMM_BREG", "1")
        monkeypatch.setenv("BL_GEMM_TILE", "0")  # 64 x 64: a wide f16 product would take 128-row tiles
    a = oracle.uniform(70 + k, m * k, -2.0, 2.0)
    b = oracle.fan_in_weights(71 + k, k * n, k)
    bias = oracle.uniform(72 + k, n, -0.1, 0.1)
    if f16:
        a, b, bias = a.astype(np.float16), b.astype(np.float16), bias.astype(np.float16)
    g = chain({X: a, W: b, B: bias}, [ir.op(ir.OP_MATMUL, [X, W, B], [m, k, n])])
    want = oracle.matmul(a.astype(np.float32), b.astype(np.float32), bias.astype(np.float32), m, k, n)
    dtype = hip.F16 if f16 else hip.F32
    prep = ir.prepare(ctx, g, dtype=dtype)
    try:
        assert "breg" in prep.kernels.label(0), prep.kernels.label(0)
    finally:
        prep.close()
    got = ir.run_on_gpu(ctx, g, {X: a, W: b, B: bias}, dtype=dtype)[Y]
    if f16:
        assert max_abs_err(got, want) <= F16_TOL
    else:
        assert_close(got, want, f"matmul {m}x{k}x{n} with B in registers")
