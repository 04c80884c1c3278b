"""One complete pre-norm encoder block on the GPU against the oracle's forward
pass (reference.rs:520-544), fused (flash attention), fused with the
reference's three attention kernels, unfused and split — the reference's
vit.rs:240-309 — plus the f16 configurations and a 12-block encoder."""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import block_graph, block_values, block_weights, max_abs_err

pytestmark = pytest.mark.gpu

EPS = 1e-6


def assert_close(got, want, what):
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}; max abs error {max_abs_err(got, want):.3e}"


@pytest.fixture(scope="module")
def small_block():
    t, d, h, mlp = 1370, 384, 6, 1536
    x = oracle.uniform(20, t * d, -2.0, 2.0)
    w = block_weights(d, mlp, 100, "reference")
    want = oracle.vit_block(x, w, t, h, d // h, mlp, EPS)
    return (t, d, h, mlp), x, w, want


@pytest.mark.parametrize(
    "fusion,parts,flash",
    [
        (ir.FUSION_ON, 1, True),
        (ir.FUSION_ON, 1, False),
        (ir.FUSION_OFF, 1, False),
        (ir.FUSION_ON, 3, True),
        (ir.FUSION_ON, 22, True),
        (ir.FUSION_ON, 3, False),
    ],
)
def test_one_encoder_block_with_random_weights_matches_the_oracle_block(ctx, small_block, fusion, parts, flash):
    (t, d, h, mlp), x, w, want = small_block
    g, ids = block_graph(t, d, h, mlp, EPS)
    got = ir.run_on_gpu(ctx, g, block_values(ids, x, w), fusion, parts, flash)[ids.output]
    assert_close(got, want, f"encoder block, fusion {fusion}, {parts} parts, flash {flash}")


def test_the_block_in_f32_matrix_core_math_matches_the_oracle(ctx, small_block):
    (t, d, h, mlp), x, w, want = small_block
    ctx.set_f32_math(hip.F32_MATH_MFMA_F32)
    try:
        g, ids = block_graph(t, d, h, mlp, EPS)
        got = ir.run_on_gpu(ctx, g, block_values(ids, x, w))[ids.output]
        assert_close(got, want, "encoder block, v_mfma_f32")
    finally:
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)


def test_the_benchmark_block_with_xavier_weights_and_normal_activations(ctx):
    t, d, h, mlp = 257, 384, 6, 1536
    x = oracle.normal(7, t * d)
    w = block_weights(d, mlp, 300, "xavier")
    want = oracle.vit_block(x, w, t, h, d // h, mlp, EPS)
    g, ids = block_graph(t, d, h, mlp, EPS)
    got = ir.run_on_gpu(ctx, g, block_values(ids, x, w))[ids.output]
    assert_close(got, want, "ViT-S block, 257 tokens")


@pytest.mark.parametrize("t,d,h", [(1370, 768, 12), (1370, 1024, 16), (5477, 384, 6)])
def test_the_f16_block_is_within_its_tolerance(ctx, t, d, h):
    mlp = 4 * d
    x = oracle.normal(9, t * d).astype(np.float16)
    w = {k: v.astype(np.float16) for k, v in block_weights(d, mlp, 500, "xavier").items()}
    want = oracle.vit_block(
        x.astype(np.float32), {k: v.astype(np.float32) for k, v in w.items()}, t, h, d // h, mlp, EPS,
        attention_rounded=False,
    )
    g, ids = block_graph(t, d, h, mlp, EPS)
    got = ir.run_on_gpu(ctx, g, block_values(ids, x, w), dtype=hip.F16)[ids.output]
    err = max_abs_err(got, want)
    assert err <= 2e-2, f"f16 block t={t} d={d}: max abs error {err:.3e}"


def test_graph_replays_match_launches_one_by_one(ctx):
    """encode_range replays a captured HIP graph of the block's kernels. Every
    replay, with host writes, reads and one-by-one launches in between, must
    equal the same kernels launched one by one on the same input, and the
    oracle's block."""
    t, d, h, mlp = 257, 384, 6, 1536
    w = block_weights(d, mlp, 300, "xavier")
    g, ids = block_graph(t, d, h, mlp, EPS)
    prep = ir.prepare(ctx, g)
    for tid, v in block_values(ids, oracle.normal(7, t * d), w).items():
        prep.write(tid, v)
    n = len(prep.kernels)
    for rep in range(4):
        x = oracle.normal(100 + rep, t * d)
        prep.write(0, x)
        for k in range(n):
            prep.kernels.encode(k)
        ctx.synchronize()
        one_by_one = prep.read(ids.output)
        prep.run()
        ctx.synchronize()
        replayed = prep.read(ids.output)
        assert np.array_equal(replayed, one_by_one), f"replay {rep} differs from one-by-one launches"
        assert_close(replayed, oracle.vit_block(x, w, t, h, d // h, mlp, EPS), f"replay {rep}")


@pytest.mark.parametrize("dtype,taps", [(hip.F32, [1, 2, 4]), (hip.F16, [1, 2])])
def test_the_encoders_feature_maps_match_the_oracle(ctx, dtype, taps):
    """encoder() (depth_anything_v2.rs:434-527) at 224 pixels: embeddings,
    blocks up to the deepest tap, and per tap the shared final LayerNorm and
    the token-to-map, against the oracle composed op by op."""
    grid, patch, d, h, mlp = 16, 14, 384, 6, 1536
    t = grid * grid + 1
    g = ir.Graph()
    enc = ir.vit_encoder(g, grid, patch, 3, d, h, mlp, EPS, taps)
    image = oracle.uniform(60, (grid * patch) ** 2 * 3, 0.0, 1.0)
    pw = oracle.fan_in_weights(61, patch * patch * 3 * d, patch * patch * 3)
    pb = oracle.uniform(62, d, -0.1, 0.1)
    cls = oracle.uniform(63, d, -1.0, 1.0)
    pos = oracle.uniform(64, t * d, -0.5, 0.5)
    fg, fb = oracle.uniform(65, d, 0.8, 1.2), oracle.uniform(66, d, -0.1, 0.1)
    weights = [block_weights(d, mlp, 100 + 20 * i, "reference") for i in range(len(enc.blocks))]
    vals = {enc.embed.image: image, enc.embed.patch_w: pw, enc.embed.patch_b: pb, enc.embed.cls: cls,
            enc.embed.pos: pos, enc.final_g: fg, enc.final_b: fb}
    for ids, w in zip(enc.blocks, weights):
        for name in ir.BLOCK_WEIGHTS:
            vals[getattr(ids, name)] = w[name]
    if dtype == hip.F16:
        vals = {k: v.astype(np.float16) for k, v in vals.items()}
    f32 = {k: v.astype(np.float32) for k, v in vals.items()}
    e = enc.embed
    x = oracle.add(oracle.prepend_token(f32[e.cls], oracle.patch_embed(f32[e.image], f32[e.patch_w], f32[e.patch_b],
                                                                          grid, grid, patch, 3, d), grid * grid, d),
                   f32[e.pos])
    want = []
    for i, ids in enumerate(enc.blocks):
        w = {name: f32[getattr(ids, name)] for name in ir.BLOCK_WEIGHTS}
        x = oracle.vit_block(x, w, t, h, d // h, mlp, EPS)
        if i + 1 in taps:
            want.append(oracle.layernorm(x, f32[enc.final_g], f32[enc.final_b], t, d, EPS)[d:])
    got = ir.run_on_gpu(ctx, g, vals, dtype=dtype)
    for tap, fmap, w in zip(taps, enc.features, want):
        case = f"feature map of layer {tap}, {'f16' if dtype == hip.F16 else 'f32'}"
        if dtype == hip.F16:
            assert max_abs_err(got[fmap], w) <= 2e-2, case
        else:
            assert_close(got[fmap], w, case)
