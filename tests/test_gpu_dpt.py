"""GPU parity of the DPT head's kernels against the oracle, through the C ABI:
the 3x3 convolution (implicit GEMM on the matrix cores, strides 1 and 2, with
and without bias, the ReLU prologue, epilogues), the 1x1 convolution (a
matmul), the transposed convolution and the bilinear resampling, whole and
split into parts; then a whole decoder at a small side against the oracle's
composition of the same operations (reference.rs:194-244 for the residual unit
and fusion layer) — the reference's crates/beatlm-bench/src/dpt.rs cases.

Tolerance for f32 storage: |got - want| <= 1e-4 + 1e-4 |want|
(reference.rs:22-24); for f16 storage, max abs error <= 2e-2 against the
oracle on the same f16-rounded inputs.
"""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import CHAIN as H_, CHAIN_OUT as Y, chain, max_abs_err

pytestmark = pytest.mark.gpu

F16_TOL = 2e-2


def assert_close(got, want, what):
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"


def run(ctx, g, values, parts=1, dtype=hip.F32, fusion=ir.FUSION_ON):
    if dtype == hip.F16:
        values = {k: v.astype(np.float16) for k, v in values.items()}
    return ir.run_on_gpu(ctx, g, values, fusion, parts, True, dtype)[Y]


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("h,w,cin,cout,stride,bias", [
    (37, 37, 384, 64, 1, False),   # the neck's convolution at 518 pixels
    (37, 37, 384, 384, 2, True),   # the last stage's stride-2 resampling
    (19, 19, 64, 64, 1, True),
    (20, 13, 48, 32, 1, True),
    (5, 7, 3, 4, 1, True),         # channels not a whole vector: the element-wise gather
    (9, 9, 8, 6, 2, False),
    (1, 1, 32, 16, 1, True),
    (184, 184, 32, 32, 1, True),   # 32 channels over many pixels: the 128 x 32 tile
    (181, 181, 16, 20, 1, False),  # ... with ragged output channels
])
def test_conv3x3_matches_the_oracle(ctx, h, w, cin, cout, stride, bias):
    x = oracle.uniform(11, h * w * cin, -2.0, 2.0)
    wt = oracle.fan_in_weights(12, 9 * cin * cout, 9 * cin)
    b = oracle.uniform(13, cout, -0.1, 0.1) if bias else None
    vals = {0: x, 1: wt}
    if bias:
        vals[2] = b
    o = ir.op(ir.OP_CONV3X3, [0, 1, 2 if bias else ir.NONE], [h, w, cin, cout, stride])
    g = chain(vals, [o])
    want = oracle.conv3x3(x, wt, b, h, w, cin, cout, stride)
    for parts in (1, 3):
        assert_close(run(ctx, g, vals, parts), want, f"conv3x3 {h}x{w}x{cin}->{cout} s{stride}, {parts} parts")
    got16 = run(ctx, g, vals, 1, hip.F16)
    want16 = oracle.conv3x3(f16(x), f16(wt), f16(b) if bias else None, h, w, cin, cout, stride)
    assert max_abs_err(got16, want16) <= F16_TOL


@pytest.mark.parametrize("h,w,c", [(19, 21, 64), (148, 150, 64)])
def test_the_relu_prologue_and_epilogues_of_a_residual_unit(ctx, h, w, c):
    # x + conv2(relu(conv1(relu(x)))): the outer ReLU a prologue (x is read
    # twice), the inner an epilogue, the add fused into conv2. At 148 x 150
    # both convolutions take the direct kernel.
    x = oracle.uniform(21, h * w * c, -2.0, 2.0)
    w1, w2 = oracle.fan_in_weights(22, 9 * c * c, 9 * c), oracle.fan_in_weights(23, 9 * c * c, 9 * c)
    b1, b2 = oracle.uniform(24, c, -0.1, 0.1), oracle.uniform(25, c, -0.1, 0.1)
    vals = {0: x, 1: w1, 2: b1, 3: w2, 4: b2}
    n = h * w * c
    ops = [ir.op(ir.OP_RELU, [0], [n]), ir.op(ir.OP_CONV3X3, [H_, 1, 2], [h, w, c, c, 1]),
           ir.op(ir.OP_RELU, [H_ + 1], [n]), ir.op(ir.OP_CONV3X3, [H_ + 2, 3, 4], [h, w, c, c, 1]),
           ir.op(ir.OP_ADD, [H_ + 3, 0], [n])]
    g = chain(vals, ops)
    names = g.lower(ir.FUSION_ON).names()
    assert names == ["relu-conv2d3x3+relu", "conv2d3x3+add"]
    assert all((" direct " in lab) == (h > 100) for lab in labels_of(ctx, g)), labels_of(ctx, g)
    first = oracle.conv3x3(oracle.relu(x), w1, b1, h, w, c, c)
    want = oracle.add(oracle.conv3x3(oracle.relu(first), w2, b2, h, w, c, c), x)
    for fusion in (ir.FUSION_ON, ir.FUSION_OFF):
        for parts in (1, 4):
            assert_close(run(ctx, g, vals, parts, fusion=fusion), want, f"residual unit fusion {fusion} parts {parts}")


def labels_of(ctx, g, parts=1, dtype=hip.F32, fusion=ir.FUSION_ON):
    prep = ir.prepare(ctx, g, fusion, parts, True, dtype)
    labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
    prep.close()
    return labels


# Stride-1 convolutions over images with at least a tile (2 rows x 64 columns
# x 32 channels) per CU take the direct kernel, which stages each input window
# in LDS once for the nine taps: the decoder's 148 x 148 x 64 units and
# fusion convolutions, the head's 296 x 296 x 64 -> 32 and 518 x 518 x 32 ->
# 32 ones; ragged widths (tile columns past the image), odd tile-row counts,
# input channels not a whole 32-channel chunk, and parts.
@pytest.mark.parametrize("h,w,cin,cout,bias", [
    (148, 148, 64, 64, True),
    (148, 148, 48, 64, True),
    (296, 296, 64, 32, True),
    (201, 130, 40, 32, False),
    (518, 518, 32, 32, True),
])
def test_the_direct_convolution_matches_the_oracle(ctx, h, w, cin, cout, bias):
    x = oracle.uniform(31, h * w * cin, -2.0, 2.0)
    wt = oracle.fan_in_weights(32, 9 * cin * cout, 9 * cin)
    b = oracle.uniform(33, cout, -0.1, 0.1) if bias else None
    vals = {0: x, 1: wt}
    if bias:
        vals[2] = b
    g = chain(vals, [ir.op(ir.OP_CONV3X3, [0, 1, 2 if bias else ir.NONE], [h, w, cin, cout, 1])])
    labels = labels_of(ctx, g)
    assert len(labels) == 1 and " direct " in labels[0], labels
    want = oracle.conv3x3(x, wt, b, h, w, cin, cout, 1)
    for parts in (1, 3):
        assert_close(run(ctx, g, vals, parts), want, f"direct conv3x3 {h}x{w}x{cin}->{cout}, {parts} parts")
    assert " direct " in labels_of(ctx, g, dtype=hip.F16)[0]
    got16 = run(ctx, g, vals, 1, hip.F16)
    want16 = oracle.conv3x3(f16(x), f16(wt), f16(b) if bias else None, h, w, cin, cout, 1)
    err = max_abs_err(got16, want16)
    print(f"direct conv3x3 {h}x{w}x{cin}->{cout} f16: max abs error {err:.3e}")
    assert err <= F16_TOL


@pytest.mark.parametrize("h,w,cin,cout,f", [(37, 37, 48, 48, 4), (37, 37, 96, 96, 2), (3, 5, 7, 3, 2), (1, 2, 1, 1, 2)])
def test_conv_transpose_matches_the_oracle(ctx, h, w, cin, cout, f):
    x = oracle.uniform(31, h * w * cin, -2.0, 2.0)
    wt = oracle.fan_in_weights(32, f * f * cin * cout, cin)
    b = oracle.uniform(33, cout, -0.1, 0.1)
    vals = {0: x, 1: wt, 2: b}
    g = chain(vals, [ir.op(ir.OP_CONV_TRANSPOSE, [0, 1, 2], [h, w, cin, cout, f])])
    want = oracle.conv_transpose(x, wt, b, h, w, cin, cout, f)
    for parts in (1, 7):
        assert_close(run(ctx, g, vals, parts), want, f"conv transpose {h}x{w}x{cin} f{f}, {parts} parts")
    got16 = run(ctx, g, vals, 1, hip.F16)
    assert max_abs_err(got16, oracle.conv_transpose(f16(x), f16(wt), f16(b), h, w, cin, cout, f)) <= F16_TOL


@pytest.mark.parametrize("ih,iw,oh,ow,c", [(148, 148, 296, 296, 64), (19, 19, 37, 37, 64), (296, 296, 518, 518, 32),
                                           (4, 5, 9, 7, 3), (5, 5, 1, 1, 2), (2, 2, 3, 3, 1)])
def test_resize_bilinear_matches_the_oracle(ctx, ih, iw, oh, ow, c):
    x = oracle.uniform(41, ih * iw * c, -2.0, 2.0)
    vals = {0: x}
    g = chain(vals, [ir.op(ir.OP_RESIZE_BILINEAR, [0], [ih, iw, oh, ow, c])])
    want = oracle.resize_bilinear(x, ih, iw, oh, ow, c)
    for parts in (1, 5):
        assert_close(run(ctx, g, vals, parts), want, f"resize {ih}x{iw}->{oh}x{ow}x{c}, {parts} parts")
    assert max_abs_err(run(ctx, g, vals, 1, hip.F16), oracle.resize_bilinear(f16(x), ih, iw, oh, ow, c)) <= F16_TOL


def test_the_reference_known_answers_on_the_gpu(ctx):
    # reference.rs tests: a transposed convolution writes one block per input
    # pixel; aligned corners keep the corners and interpolate linearly.
    vals = {0: np.array([10.0, -1.0], np.float32), 1: np.array([1.0, 2.0, 3.0, 4.0], np.float32),
            2: np.array([0.5], np.float32)}
    g = chain(vals, [ir.op(ir.OP_CONV_TRANSPOSE, [0, 1, 2], [1, 2, 1, 1, 2])])
    assert np.array_equal(run(ctx, g, vals), [10.5, 20.5, -0.5, -1.5, 30.5, 40.5, -2.5, -3.5])
    vals = {0: np.array([0.0, 2.0, 4.0, 6.0], np.float32)}
    g = chain(vals, [ir.op(ir.OP_RESIZE_BILINEAR, [0], [2, 2, 3, 3, 1])])
    assert np.array_equal(run(ctx, g, vals), [0, 1, 2, 2, 3, 4, 4, 5, 6])
    vals = {0: np.ones(4, np.float32), 1: np.ones(9, np.float32), 2: np.array([0.5], np.float32)}
    g = chain(vals, [ir.op(ir.OP_CONV3X3, [0, 1, 2], [2, 2, 1, 1, 1])])
    assert np.array_equal(run(ctx, g, vals), [4.5] * 4)


# ---- the whole decoder -------------------------------------------------------


def decoder_values(weights, cfg, seed=500):
    """{id: values} and {name: values}: weights U(+-1/sqrt(fan_in)), biases
    U(-0.1, 0.1)."""
    by_id, by_name = {}, {}
    for i, (tid, name, n) in enumerate(weights):
        if name.endswith(".bias"):
            v = oracle.uniform(seed + i, n, -0.1, 0.1)
        else:
            v = oracle.fan_in_weights(seed + i, n, cfg.fan_in(name))
        by_id[tid] = by_name[name] = v
    return by_id, by_name


def oracle_decoder(cfg, side, features, w):
    return oracle.depth_decoder(cfg, side, features, w)


@pytest.mark.parametrize("side", [70, 98])
def test_a_whole_decoder_matches_the_oracle(ctx, side):
    cfg = ir.DepthConfig.small()
    grid = side // cfg.patch_size
    g = ir.Graph()
    for i in range(4):
        g.tensor(i, ir.INPUT, grid * grid * cfg.hidden_size)
    depth, weights, _ = ir.depth_decoder(g, cfg, side, [0, 1, 2, 3], 10)
    vals, named = decoder_values(weights, cfg)
    features = [oracle.normal(900 + i, grid * grid * cfg.hidden_size) for i in range(4)]
    vals.update(enumerate(features))
    want = oracle_decoder(cfg, side, features, named)
    assert float(np.max(want)) > 0.0  # the final ReLU leaves something to compare
    for parts in (1, 2):
        prep = ir.prepare(ctx, g, ir.FUSION_ON, parts)
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        # Residual units' second convolutions read their input as bf16 planes.
        assert any(lab.startswith("conv2d3x3+add") and "< split" in lab for lab in labels), labels
        for tid, v in vals.items():
            prep.write(tid, v)
        prep.run()
        ctx.synchronize()
        got = prep.read(depth)
        assert got.size == side * side
        assert_close(got, want, f"decoder at {side} pixels, {parts} parts")


# ---- the whole model ---------------------------------------------------------


def encoder_values(enc, cfg, grid, seed=60):
    """Image U[0,1], patch weights U(+-1/sqrt(588)), class token, positions and
    the final LayerNorm as the encoder test draws them, block weights by the
    reference's scheme (vit.rs:206-231)."""
    from tests.blockdata import block_weights

    d, t, p = cfg.hidden_size, grid * grid + 1, cfg.patch_size
    e = enc.embed
    vals = {e.image: oracle.uniform(seed, (grid * p) ** 2 * 3, 0.0, 1.0),
            e.patch_w: oracle.fan_in_weights(seed + 1, p * p * 3 * d, p * p * 3),
            e.patch_b: oracle.uniform(seed + 2, d, -0.1, 0.1), e.cls: oracle.uniform(seed + 3, d, -1.0, 1.0),
            e.pos: oracle.uniform(seed + 4, t * d, -0.5, 0.5), enc.final_g: oracle.uniform(seed + 5, d, 0.8, 1.2),
            enc.final_b: oracle.uniform(seed + 6, d, -0.1, 0.1)}
    for i, ids in enumerate(enc.blocks):
        w = block_weights(d, d * cfg.mlp_ratio, 100 + 20 * i, "reference")
        for name in ir.BLOCK_WEIGHTS:
            vals[getattr(ids, name)] = w[name]
    return vals


def oracle_encoder(enc, cfg, grid, f32):
    d, h, t = cfg.hidden_size, cfg.num_heads, grid * grid + 1
    e = enc.embed
    x = oracle.add(oracle.prepend_token(f32[e.cls], oracle.patch_embed(f32[e.image], f32[e.patch_w], f32[e.patch_b],
                                                                          grid, grid, cfg.patch_size, 3, d),
                                        grid * grid, d), f32[e.pos])
    features = []
    for i, ids in enumerate(enc.blocks):
        w = {name: f32[getattr(ids, name)] for name in ir.BLOCK_WEIGHTS}
        x = oracle.vit_block(x, w, t, h, d // h, d * cfg.mlp_ratio, cfg.eps)
        if i + 1 in cfg.out_indices:
            features.append(oracle.layernorm(x, f32[enc.final_g], f32[enc.final_b], t, d, cfg.eps)[d:])
    return features


@pytest.mark.parametrize("dtype", [hip.F32, hip.F16])
def test_the_whole_model_matches_the_oracle(ctx, dtype):
    """model() (depth_anything_v2.rs:984-995) at 70 pixels: the 12-layer
    encoder, its four tapped feature maps as activations, and the decoder."""
    cfg = ir.DepthConfig.small()
    side = 70
    grid = side // cfg.patch_size
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    vals = encoder_values(m.encoder, cfg, grid)
    dec, named = decoder_values(m.decoder_weights, cfg)
    vals.update(dec)
    if dtype == hip.F16:
        vals = {k: f16(v) for k, v in vals.items()}
        named = {n: vals[tid] for tid, n, _ in m.decoder_weights}
    want = oracle_decoder(cfg, side, oracle_encoder(m.encoder, cfg, grid, vals), named)
    got = ir.run_on_gpu(ctx, g, vals, dtype=dtype)
    assert list(got) == [m.depth]
    if dtype == hip.F16:
        assert max_abs_err(got[m.depth], want) <= F16_TOL
    else:
        assert_close(got[m.depth], want, "depth at 70 pixels")
