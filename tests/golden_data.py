"""Loading the golden fixtures of tests/golden/ (written by
tests/golden/make_fixtures.py) and rebuilding their inputs."""

from __future__ import annotations

import os

import numpy as np

import oracle
from tests.blockdata import block_weights

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BLOCKS = ["block_t17_d10_h2.npz", "block_t41_d128_h2.npz"]
ATTENTION = ["attention_t65_h2.npz", "attention_t1_h3.npz"]
EMBEDDINGS = ["embeddings_grid3_w16.npz"]


def load(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def block_inputs(f: dict):
    """(x, weights) of a block fixture: stored, or regenerated from its seeds
    and checked against the stored checksums."""
    d, mlp = int(f["d"]), int(f["mlp"])
    if "x" in f:
        return f["x"], {k[2:]: f[k] for k in f if k.startswith("w_") and k != "w_seed" and k != "w_sum"}
    x = oracle.uniform(int(f["x_seed"]), int(f["t"]) * d, -2.0, 2.0)
    w = block_weights(d, mlp, int(f["w_seed"]), "reference")
    assert float(np.sum(x, dtype=np.float64)) == float(f["x_sum"]), "the input generator drifted"
    assert float(sum(np.sum(v, dtype=np.float64) for v in w.values())) == float(f["w_sum"]), "the weight generator drifted"
    return x, w


def attention_inputs(f: dict):
    t, h, d = int(f["t"]), int(f["h"]), int(f["d"])
    qkv = oracle.uniform(int(f["seed"]), t * 3 * h * d, -1.0, 1.0)
    assert float(np.sum(qkv, dtype=np.float64)) == float(f["qkv_sum"]), "the input generator drifted"
    return qkv
