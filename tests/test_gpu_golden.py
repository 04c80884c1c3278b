"""The GPU path, through the C ABI, against the committed golden fixtures
(tests/golden/, the oracle's outputs at small and ragged shapes): the block
fused and unfused, the fused attention alone and the embeddings.
Tolerance: the f32 bar, max abs error <= 1e-4 with a relative term for
large values (oracle.first_mismatch)."""

import numpy as np
import pytest

import oracle
from beatlm_amd import ir
from tests.blockdata import block_graph, block_values, chain
from tests.golden_data import ATTENTION, BLOCKS, EMBEDDINGS, attention_inputs, block_inputs, load

pytestmark = pytest.mark.gpu


def assert_close(got, want, what):
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the fixture says {bad[2]}"


@pytest.mark.parametrize("name", BLOCKS)
def test_the_block_matches_its_fixture(ctx, name):
    f = load(name)
    x, w = block_inputs(f)
    t, d, h, mlp = (int(f[k]) for k in ("t", "d", "h", "mlp"))
    g, ids = block_graph(t, d, h, mlp, float(f["eps"]))
    vals = block_values(ids, x, w)
    flash = d // h == 64
    for fuse in ([True, False] if flash else [False]):
        got = ir.run_on_gpu(ctx, g, vals, flash=fuse)[ids.output]
        assert_close(got, f["want"], f"{name}, flash {fuse}")


@pytest.mark.parametrize("name", ATTENTION)
def test_flash_attention_matches_its_fixture(ctx, name):
    f = load(name)
    t, h, d = int(f["t"]), int(f["h"]), int(f["d"])
    qkv = attention_inputs(f)
    X, Y = 1, 20
    ops = [
        ir.op(ir.OP_ATTENTION_SCORES, [X], [t, h, d]),
        ir.op(ir.OP_SCALE, [10], [t * h * t], 0.125),
        ir.op(ir.OP_SOFTMAX, [11], [t * h, t]),
        ir.op(ir.OP_ATTENTION_VALUES, [12, X], [t, h, d]),
    ]
    g = chain({X: qkv}, ops)
    for flash in (True, False):
        got = ir.run_on_gpu(ctx, g, {X: qkv}, flash=flash)[Y]
        assert_close(got, f["want"], f"{name}, flash {flash}")


@pytest.mark.parametrize("name", EMBEDDINGS)
def test_the_embeddings_match_their_fixture(ctx, name):
    f = load(name)
    gr, p, c = int(f["grid"]), int(f["patch"]), int(f["width"])
    g = ir.Graph()
    e = g.vit_embeddings(gr, p, 3, c, 0)
    g.tensor(e.next_id, ir.OUTPUT, (gr * gr + 1) * c)
    # x 1.0 is exact; it fuses into the class-token kernel's epilogue.
    g.push(ir.op(ir.OP_SCALE, [e.output], [(gr * gr + 1) * c], 1.0), e.next_id)
    vals = {e.image: f["image"], e.patch_w: f["patch_w"], e.patch_b: f["patch_b"], e.cls: f["cls"], e.pos: f["pos"]}
    got = ir.run_on_gpu(ctx, g, vals)[e.next_id]
    assert_close(got, np.asarray(f["want"]), name)
