"""The oracle still produces the committed golden fixtures (tests/golden/),
exactly. A change to the oracle or its generators that moves a single bit of
these outputs fails here. CPU only."""

import numpy as np
import pytest

import oracle
from tests.golden_data import ATTENTION, BLOCKS, EMBEDDINGS, attention_inputs, block_inputs, load


@pytest.mark.parametrize("name", BLOCKS)
def test_the_oracle_block_reproduces_its_fixture(name):
    f = load(name)
    x, w = block_inputs(f)
    t, d, h, mlp = (int(f[k]) for k in ("t", "d", "h", "mlp"))
    got = oracle.vit_block(x, w, t, h, d // h, mlp, float(f["eps"]))
    assert np.array_equal(got, f["want"])


@pytest.mark.parametrize("name", ATTENTION)
def test_the_oracle_attention_reproduces_its_fixture(name):
    f = load(name)
    t, h, d = int(f["t"]), int(f["h"]), int(f["d"])
    got = oracle.attention(attention_inputs(f), t, h, d, 0.125)
    assert np.array_equal(got, f["want"])


@pytest.mark.parametrize("name", EMBEDDINGS)
def test_the_oracle_embeddings_reproduce_their_fixture(name):
    f = load(name)
    g, p, c = int(f["grid"]), int(f["patch"]), int(f["width"])
    patches = oracle.patch_embed(f["image"], f["patch_w"], f["patch_b"], g, g, p, 3, c)
    got = oracle.add(oracle.prepend_token(f["cls"], patches, g * g, c), f["pos"])
    assert np.array_equal(got, f["want"])


def test_a_one_token_attention_fixture_is_its_value_rows():
    # Closed form: with one key, softmax is 1 and the output is V.
    f = load("attention_t1_h3.npz")
    qkv = attention_inputs(f).reshape(3, 3, 64)
    assert np.array_equal(f["want"].reshape(3, 64), qkv[2])
