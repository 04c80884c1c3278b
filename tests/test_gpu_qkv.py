"""QKV projections that store qkv's queries alone.

In an encoder whose qkv the host never touches (an internal activation,
written by the QKV projection from an internal x and read by nothing but the
flash kernel), the projection writes K and Vt to the flash kernel's operands
only and qkv receives the queries (its first third of columns). When the
attention scratch does not hold the operands as the flash kernel runs (a host
write in between, a range or a single launch that starts at the flash
kernel), the projection runs again from the same x. Every way of encoding the
program must then give the output of the program encoded whole, bit for bit
when no host write came in between, and that output must match the oracle
(1e-4 for f32 storage, 2e-2 for f16). A host write also makes each folded
LayerNorm's consumer remake its row statistics from x (in a launch of its
own, summed in another order than its producer's epilogue), so after one the
output is held to the oracle's bar instead, and to that bar against the
whole program's.
"""

import numpy as np
import pytest

import bench
import oracle
from beatlm_amd import hip, ir
from tests.blockdata import max_abs_err

pytestmark = pytest.mark.gpu

CFG = dict(grid=16, width=384, heads=6, blocks=2, frames=1)


def oracle_output(cfg, emb, block_ids, tokens, vals):
    f = {k: np.asarray(v, np.float32) for k, v in vals.items()}
    grid, width, heads = cfg["grid"], cfg["width"], cfg["heads"]
    x = oracle.patch_embed(f[emb.image], f[emb.patch_w], f[emb.patch_b], grid, grid, bench.PATCH, 3, width)
    x = oracle.add(oracle.prepend_token(f[emb.cls], x, grid * grid, width), f[emb.pos])
    for ids in block_ids:
        w = {name: f[getattr(ids, name)] for name in ir.BLOCK_WEIGHTS}
        x = oracle.vit_block(x, w, tokens, heads, width // heads, 4 * width, bench.EPS,
                             attention_rounded=cfg["dtype"] == "f32")
    return x


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_every_encoding_of_queries_only_projections_gives_the_whole_programs_output(ctx, dtype):
    cfg = dict(CFG, dtype=dtype)
    g, emb, block_ids, tokens = bench.build_encoder(cfg)
    f16 = dtype == "f16"
    vals = bench.synthetic_values(cfg, emb, block_ids, tokens, np.float16 if f16 else np.float32, 77)
    prep = ir.prepare(ctx, g, dtype=hip.F16 if f16 else hip.F32)
    try:
        for tid, v in vals.items():
            prep.write(tid, v)
        kernels = prep.kernels
        n = len(kernels)
        labels = [kernels.label(k) for k in range(n)]
        flash = [k for k, s in enumerate(labels) if s.startswith("flash_attention")]
        qonly = [k for k, s in enumerate(labels) if "> queries only" in s]
        print(labels)
        assert len(flash) == len(block_ids) and len(qonly) == len(block_ids), labels
        out = block_ids[-1].output
        image = vals[emb.image]

        prep.run()
        ctx.synchronize()
        whole = prep.read(out)
        want = oracle_output(cfg, emb, block_ids, tokens, vals)
        bar = 2e-2 if f16 else 1e-4
        err = max_abs_err(whole, want)
        print(f"{dtype}: max abs error {err:.3e} against the oracle")
        assert err <= bar, f"max abs error {err:.3e}"

        def check(what, exact=True):
            ctx.synchronize()
            got = prep.read(out)
            if exact:
                assert np.array_equal(got, whole), f"{what}: differs from the program encoded whole"
            else:
                e_whole, e_oracle = max_abs_err(got, whole), max_abs_err(got, want)
                print(f"{what}: {e_whole:.3e} from the whole program, {e_oracle:.3e} from the oracle")
                assert e_whole <= bar and e_oracle <= bar, f"{what}: {e_whole:.3e} / {e_oracle:.3e}"

        # One by one, with a host write (the same image) before every flash
        # kernel: the scratch is taken to hold nothing, so each projection runs
        # again before its attention.
        for k in range(n):
            if k in flash:
                prep.write(emb.image, image)
            kernels.encode(k)
        check("one by one, a host write before each flash kernel", exact=False)
        # Two ranges cut at the last flash kernel, in order: the second starts
        # with the operands the first left (a graph captured without the
        # projection), or, after a host write in between, with none (a graph
        # captured with the projection run again from the x the first range
        # left, which nothing has overwritten in program order).
        cut = flash[-1]
        for rep in range(4):
            ctx.check(ctx._lib.bl_kernels_encode_range(kernels.handle, 0, cut, 0))
            if rep % 2 == 1:
                prep.write(emb.image, image)
            ctx.check(ctx._lib.bl_kernels_encode_range(kernels.handle, cut, n - cut, 0))
            check(f"two ranges cut at the last flash kernel, pass {rep}", exact=rep % 2 == 0)
        # The whole program again, as a graph.
        prep.run()
        check("the program encoded whole again")
    finally:
        prep.close()
