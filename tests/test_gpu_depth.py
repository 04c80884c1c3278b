"""The benchmark's encoders at full depth on the GPU against the oracle, at the
north star's bars: max abs error <= 1e-4 for f32 storage, <= 2e-2 for f16
storage with f32 accumulation.

- ViT-S/14 at 518 pixels: exactly the benchmark's workload (bench.py's
  build_encoder and synthetic_values): patch embedding, class token and
  positions, 12 f32 blocks of 1370 tokens; against the oracle's embeddings
  followed by 12 chained blocks (crates/beatlm-bench/src/reference.rs:388-425,
  :520-544; the reference's own encoder test, crates/beatlm-bench/src/vit.rs
  :240-309, runs one such block).
- ViT-B/14 at 518 pixels: 12 f16 blocks of 1370 tokens, width 768.
- ViT-S/14 at 1036 pixels (5477 tokens, f16): the first two blocks.
- ViT-L/14 at 518 pixels, four frames: four job slots of one program, each
  slot one binding set that rebinds the image and the output
  (crates/beatlm/src/codegen/kernels.rs:120-170, crates/beatlm-host/src/
  slots.rs:96-151). Each frame through its slot equals the same frame run
  alone, bit for bit, and the first two blocks of every frame are checked
  against the oracle.

Every test prints the maximum absolute error it measured."""

import numpy as np
import pytest

import bench
import oracle
from beatlm_amd import hip, ir
from tests.blockdata import max_abs_err

pytestmark = pytest.mark.gpu

PATCH = bench.PATCH


def oracle_encoder(cfg, emb, block_ids, tokens, vals, blocks=None):
    """The oracle's embeddings and the first `blocks` blocks, in f32 over the
    values the GPU was given (f16 values widened exactly)."""
    f = {k: np.asarray(v, np.float32) for k, v in vals.items()}
    grid, width, heads = cfg["grid"], cfg["width"], cfg["heads"]
    x = oracle.patch_embed(f[emb.image], f[emb.patch_w], f[emb.patch_b], grid, grid, PATCH, 3, width)
    x = oracle.add(oracle.prepend_token(f[emb.cls], x, grid * grid, width), f[emb.pos])
    for ids in block_ids[: blocks if blocks is not None else len(block_ids)]:
        w = {name: f[getattr(ids, name)] for name in ir.BLOCK_WEIGHTS}
        x = oracle.vit_block(x, w, tokens, heads, width // heads, 4 * width, bench.EPS,
                             attention_rounded=cfg["dtype"] == "f32")
    return x


def run_encoder(ctx, cfg, slots=1, blocks=None, seed=2024):
    cfg = dict(cfg)
    if blocks is not None:
        cfg["blocks"] = blocks
    g, emb, block_ids, tokens = bench.build_encoder(cfg)
    dtype = hip.F16 if cfg["dtype"] == "f16" else hip.F32
    vals = bench.synthetic_values(cfg, emb, block_ids, tokens, np.float16 if dtype == hip.F16 else np.float32, seed)
    prep = ir.prepare(ctx, g, dtype=dtype, slots=slots)
    for tid, v in vals.items():
        prep.write(tid, v)
    return prep, cfg, emb, block_ids, tokens, vals


def test_the_benchmark_workload_vit_s_518_f32_matches_the_oracle_within_1e_4(ctx):
    prep, cfg, emb, block_ids, tokens, vals = run_encoder(ctx, bench.CONFIGS["vit-s-518"])
    prep.run()
    ctx.synchronize()
    got = prep.read(block_ids[-1].output)
    want = oracle_encoder(cfg, emb, block_ids, tokens, vals)
    err = max_abs_err(got, want)
    print(f"vit-s-518, 12 f32 blocks, 1370 tokens: max abs error {err:.3e} (|want| max {np.abs(want).max():.2f})")
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"element {bad[0]} is {bad[1]}, the oracle says {bad[2]}"
    assert err <= 1e-4, f"max abs error {err:.3e} above 1e-4"
    prep.close()


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
def test_the_vit_s_518_workload_with_offset_rows_matches_the_oracle_within_1e_4(ctx, math):
    """The benchmark's ViT-S/14 518 workload with 30 added to every position
    embedding: every row of the residual stream then carries a common offset
    about 30 times its spread, which the reference's LayerNorm removes before
    anything multiplies it (crates/beatlm/src/codegen/wgsl.rs:519-585). All
    24 LayerNorms are folded into their products; the 12-block output stays
    within 1e-4 of the oracle in both f32 maths."""
    ctx.set_f32_math(math)
    try:
        cfg = dict(bench.CONFIGS["vit-s-518"])
        g, emb, block_ids, tokens = bench.build_encoder(cfg)
        vals = bench.synthetic_values(cfg, emb, block_ids, tokens, np.float32, 2024)
        vals[emb.pos] = (vals[emb.pos] + 30.0).astype(np.float32)
        prep = ir.prepare(ctx, g, dtype=hip.F32)
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        assert sum("folded into" in s for s in labels) == 24, labels
        for tid, v in vals.items():
            prep.write(tid, v)
        prep.run()
        ctx.synchronize()
        got = prep.read(block_ids[-1].output)
        prep.close()
    finally:
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)
    want = oracle_encoder(cfg, emb, block_ids, tokens, vals)
    rows = want.astype(np.float64).reshape(tokens, cfg["width"])
    err = max_abs_err(got, want)
    print(f"vit-s-518 with offset rows (row mean {rows.mean(1).mean():.1f}, spread {rows.std(1).mean():.2f}), "
          f"f32 math {math}: max abs error {err:.3e}")
    assert err <= 1e-4, f"max abs error {err:.3e} above 1e-4"


def test_the_vit_b_518_encoder_in_f16_is_within_2e_2_of_the_oracle(ctx):
    prep, cfg, emb, block_ids, tokens, vals = run_encoder(ctx, bench.CONFIGS["vit-b-518"])
    prep.run()
    ctx.synchronize()
    got = prep.read(block_ids[-1].output).astype(np.float32)
    want = oracle_encoder(cfg, emb, block_ids, tokens, vals)
    err = max_abs_err(got, want)
    print(f"vit-b-518, 12 f16 blocks, 1370 tokens x 768: max abs error {err:.3e} (|want| max {np.abs(want).max():.2f})")
    assert err <= 2e-2, f"max abs error {err:.3e} above 2e-2"
    prep.close()


def test_two_vit_s_1036_blocks_in_f16_are_within_2e_2_of_the_oracle(ctx):
    """Config 5's encoder (5477 tokens, f16) through its first two blocks,
    with the patch embedding, class token and positions, against the
    oracle's composition; its full 12-block depth is checked split against
    unsplit by the frame loop's test."""
    prep, cfg, emb, block_ids, tokens, vals = run_encoder(ctx, bench.CONFIGS["vit-s-1036"], blocks=2)
    assert tokens == 5477
    prep.run()
    ctx.synchronize()
    got = prep.read(block_ids[-1].output).astype(np.float32)
    prep.close()
    want = oracle_encoder(cfg, emb, block_ids, tokens, vals)
    err = max_abs_err(got, want)
    print(f"vit-s-1036, 2 f16 blocks, 5477 tokens: max abs error {err:.3e} (|want| max {np.abs(want).max():.2f})")
    assert err <= 2e-2, f"max abs error {err:.3e} above 2e-2"


def frame_images(cfg, frames):
    side = cfg["grid"] * PATCH
    mean = np.array([0.485, 0.456, 0.406], np.float32)
    std = np.array([0.229, 0.224, 0.225], np.float32)
    out = []
    for f in range(frames):
        rng = np.random.default_rng(700 + f)
        out.append((((rng.uniform(0, 1, (side, side, 3)).astype(np.float32) - mean) / std).ravel()).astype(np.float16))
    return out


@pytest.mark.parametrize("blocks", [2, 24])
def test_four_vit_l_frames_through_four_binding_sets(ctx, blocks):
    """Config 4's four frames as four job slots. Each slot's output equals the
    same frame run through a one-slot program, bit for bit, and writing one
    slot's image leaves the other slots' outputs as they were. At two blocks
    each frame is also checked against the oracle."""
    cfg = bench.CONFIGS["vit-l-518x4"]
    frames = cfg["frames"]
    prep, cfg2, emb, block_ids, tokens, vals = run_encoder(ctx, cfg, slots=frames, blocks=blocks)
    assert prep.slots() == frames and prep.kernels.sets() == frames
    images = frame_images(cfg, frames)
    for f, im in enumerate(images):
        prep.write(emb.image, im, slot=f)
    for f in range(frames):
        prep.run(f)
    ctx.synchronize()
    out = [prep.read(block_ids[-1].output, slot=f) for f in range(frames)]
    # The frames differ, so their outputs do.
    assert not np.array_equal(out[0], out[1])
    # Running slot 2 again after rewriting slot 0's image changes only slot 0's input.
    prep.write(emb.image, images[3], slot=0)
    prep.run(2)
    ctx.synchronize()
    assert np.array_equal(prep.read(block_ids[-1].output, slot=2), out[2])
    assert np.array_equal(prep.read(block_ids[-1].output, slot=1), out[1])
    prep.close()

    single, *_ = run_encoder(ctx, cfg, slots=1, blocks=blocks)
    for f, im in enumerate(images):
        single.write(emb.image, im)
        single.run()
        ctx.synchronize()
        alone = single.read(block_ids[-1].output)
        assert np.array_equal(alone, out[f]), f"frame {f}: its slot's output differs from the frame run alone"
        if blocks <= 2:
            v = dict(vals)
            v[emb.image] = im
            want = oracle_encoder(cfg2, emb, block_ids, tokens, v)
            err = max_abs_err(out[f].astype(np.float32), want)
            print(f"vit-l-518 frame {f}, {blocks} f16 blocks, 1370 tokens x 1024: max abs error {err:.3e}")
            assert err <= 2e-2, f"frame {f}: max abs error {err:.3e} above 2e-2"
    single.close()


def encoder_with_every_block_out(cfg):
    """bench.build_encoder with every block's output kept as an output of the
    program (readable after the run, never overwritten)."""
    grid, width, heads, blocks = cfg["grid"], cfg["width"], cfg["heads"], cfg["blocks"]
    tokens = grid * grid + 1
    g = ir.Graph()
    emb = g.vit_embeddings(grid, PATCH, 3, width, 0)
    x, next_id, block_ids = emb.output, emb.next_id, []
    for _ in range(blocks):
        ids = g.vit_block(ir.VitDims(tokens, width, heads, 4 * width, bench.EPS), x, next_id, ir.OUTPUT)
        block_ids.append(ids)
        x, next_id = ids.output, ids.next_id
    return g, emb, block_ids, tokens


@pytest.mark.parametrize("name", ["vit-s-1036", "vit-l-518x4", "vit-b-518"])
def test_every_block_of_the_f16_encoders_at_full_depth_is_within_2e_2_of_the_oracle(ctx, name):
    """Configs 3, 4 (one frame) and 5 at full depth (12, 24 and 12 f16
    blocks): every block's output on the GPU against the oracle's block
    applied to the same input the GPU block read (the GPU's own previous block
    output, exactly widened; the oracle's embeddings for the first), at the
    north star's bar for a block, 2e-2. The end-to-end error against the
    oracle's whole f32 encoder is printed too: f16 storage rounds the
    residual stream (|x| up to about 10, so half an f16 ulp is up to 4e-3)
    twice a block, and those roundings add up over the depth."""
    cfg = dict(bench.CONFIGS[name])
    g, emb, block_ids, tokens = encoder_with_every_block_out(cfg)
    vals = bench.synthetic_values(cfg, emb, block_ids, tokens, np.float16, 2024)
    prep = ir.prepare(ctx, g, dtype=hip.F16)
    for tid, v in vals.items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    outs = [prep.read(ids.output).astype(np.float32) for ids in block_ids]
    labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
    prep.close()
    f = {k: np.asarray(v, np.float32) for k, v in vals.items()}
    grid, width, heads = cfg["grid"], cfg["width"], cfg["heads"]
    x = oracle.add(oracle.prepend_token(
        f[emb.cls], oracle.patch_embed(f[emb.image], f[emb.patch_w], f[emb.patch_b], grid, grid, PATCH, 3, width),
        grid * grid, width), f[emb.pos])
    worst = 0.0
    for b, ids in enumerate(block_ids):
        w = {n: f[getattr(ids, n)] for n in ir.BLOCK_WEIGHTS}
        want = oracle.vit_block(x, w, tokens, heads, width // heads, 4 * width, bench.EPS, attention_rounded=False)
        err = max_abs_err(outs[b], want)
        worst = max(worst, err)
        assert err <= 2e-2, f"{name} block {b}: max abs error {err:.3e} above 2e-2"
        x = outs[b]
    end_to_end = max_abs_err(outs[-1], oracle_encoder(cfg, emb, block_ids, tokens, vals))
    print(f"{name}: {len(block_ids)} f16 blocks, {sum('folded into' in s for s in labels)} folded LayerNorms; "
          f"worst block against the oracle from the same input {worst:.3e}; "
          f"end to end against the oracle's f32 encoder {end_to_end:.3e}")
