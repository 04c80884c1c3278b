"""Writes the golden fixtures of this directory from the oracle
(oracle/oracle.c, the reference's CPU reference restated and pinned by
tests/test_oracle.py): small shapes of the encoder block, the fused attention
and the embeddings, with their expected outputs.

Inputs that are small are stored; large ones are stored as the seeds of the
reference's LCG generators (net.rs:183-203, pinned by tests/test_oracle.py)
together with a checksum of what the seeds produce, so a fixture notices a
generator that has drifted.

    python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests.blockdata import block_weights  # noqa: E402

EPS = 1e-6


def block_fixture(t, d, h, mlp, x_seed, w_seed, store_inputs):
    x = oracle.uniform(x_seed, t * d, -2.0, 2.0)
    w = block_weights(d, mlp, w_seed, "reference")
    y = oracle.vit_block(x, w, t, h, d // h, mlp, EPS)
    out = {"t": t, "d": d, "h": h, "mlp": mlp, "eps": EPS, "x_seed": x_seed, "w_seed": w_seed,
           "x_sum": float(np.sum(x, dtype=np.float64)),
           "w_sum": float(sum(np.sum(v, dtype=np.float64) for v in w.values())),
           "want": y}
    if store_inputs:
        out["x"] = x
        out.update({f"w_{k}": v for k, v in w.items()})
    return out


def attention_fixture(t, h, seed):
    d = 64
    qkv = oracle.uniform(seed, t * 3 * h * d, -1.0, 1.0)
    want = oracle.attention(qkv, t, h, d, 0.125)
    return {"t": t, "h": h, "d": d, "seed": seed, "qkv_sum": float(np.sum(qkv, dtype=np.float64)), "want": want}


def embedding_fixture(grid, patch, width):
    side = grid * patch
    image = oracle.uniform(41, side * side * 3, -2.0, 2.0)
    w = oracle.fan_in_weights(42, patch * patch * 3 * width, patch * patch * 3)
    b = oracle.uniform(43, width, -0.1, 0.1)
    cls = oracle.uniform(44, width, -1.0, 1.0)
    pos = oracle.uniform(45, (grid * grid + 1) * width, -0.5, 0.5)
    patches = oracle.patch_embed(image, w, b, grid, grid, patch, 3, width)
    want = oracle.add(oracle.prepend_token(cls, patches, grid * grid, width), pos)
    return {"grid": grid, "patch": patch, "width": width, "image": image, "patch_w": w, "patch_b": b,
            "cls": cls, "pos": pos, "want": want}


FIXTURES = {
    # d = 5 per head: the reference's tiny unfused shapes (kernel.rs:3241-3262)
    "block_t17_d10_h2.npz": lambda: block_fixture(17, 10, 2, 40, 11, 300, True),
    # d = 64, a ragged token count, the fused path
    "block_t41_d128_h2.npz": lambda: block_fixture(41, 128, 2, 512, 12, 400, False),
    "attention_t65_h2.npz": lambda: attention_fixture(65, 2, 13),
    "attention_t1_h3.npz": lambda: attention_fixture(1, 3, 14),
    "embeddings_grid3_w16.npz": lambda: embedding_fixture(3, 14, 16),
}


def main() -> None:
    for name, make in FIXTURES.items():
        data = make()
        np.savez_compressed(os.path.join(HERE, name), **{k: np.asarray(v) for k, v in data.items()})
        print(name, {k: np.asarray(v).shape for k, v in data.items()})


if __name__ == "__main__":
    main()
