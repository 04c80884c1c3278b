"""Seeded inputs and weights of one encoder block, as the reference's GPU test
draws them (crates/beatlm-bench/src/vit.rs:206-238) or as the benchmark
configurations state them, and graph construction helpers."""

from __future__ import annotations

import numpy as np

import oracle
from beatlm_amd import ir


def block_weights(d: int, mlp: int, seed: int = 100, scheme: str = "reference") -> dict[str, np.ndarray]:
    """The 14 weights of a block, keyed as oracle.BlockWeights.

    scheme "reference": vit.rs:206-231 — gamma U(0.8, 1.2), biases and betas
    U(-0.1, 0.1), linear weights U(+-1/sqrt(fan_in)), LayerScale U(0.1, 1).
    scheme "xavier": the benchmark's — linear weights Xavier-uniform, LN
    gamma 1 + 0.1 N(0,1), beta 0.1 N(0,1), biases U(-0.1, 0.1), LayerScale
    U(0.1, 1).
    """
    s = iter(range(seed, seed + 100))
    w = {}
    if scheme == "reference":
        w["norm1_g"] = oracle.uniform(next(s), d, 0.8, 1.2)
        w["norm1_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["qkv_w"] = oracle.fan_in_weights(next(s), d * 3 * d, d)
        w["qkv_b"] = oracle.uniform(next(s), 3 * d, -0.1, 0.1)
        w["proj_w"] = oracle.fan_in_weights(next(s), d * d, d)
        w["proj_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["ls1"] = oracle.uniform(next(s), d, 0.1, 1.0)
        w["norm2_g"] = oracle.uniform(next(s), d, 0.8, 1.2)
        w["norm2_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["fc1_w"] = oracle.fan_in_weights(next(s), d * mlp, d)
        w["fc1_b"] = oracle.uniform(next(s), mlp, -0.1, 0.1)
        w["fc2_w"] = oracle.fan_in_weights(next(s), mlp * d, mlp)
        w["fc2_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["ls2"] = oracle.uniform(next(s), d, 0.1, 1.0)
    else:
        w["norm1_g"] = oracle.normal(next(s), d, 1.0, 0.1)
        w["norm1_b"] = oracle.normal(next(s), d, 0.0, 0.1)
        w["qkv_w"] = oracle.xavier(next(s), d, 3 * d)
        w["qkv_b"] = oracle.uniform(next(s), 3 * d, -0.1, 0.1)
        w["proj_w"] = oracle.xavier(next(s), d, d)
        w["proj_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["ls1"] = oracle.uniform(next(s), d, 0.1, 1.0)
        w["norm2_g"] = oracle.normal(next(s), d, 1.0, 0.1)
        w["norm2_b"] = oracle.normal(next(s), d, 0.0, 0.1)
        w["fc1_w"] = oracle.xavier(next(s), d, mlp)
        w["fc1_b"] = oracle.uniform(next(s), mlp, -0.1, 0.1)
        w["fc2_w"] = oracle.xavier(next(s), mlp, d)
        w["fc2_b"] = oracle.uniform(next(s), d, -0.1, 0.1)
        w["ls2"] = oracle.uniform(next(s), d, 0.1, 1.0)
    return w


def block_graph(t: int, d: int, h: int, mlp: int, eps: float = 1e-6):
    """One block reading input 0 and writing an output: (graph, ids)."""
    g = ir.Graph()
    g.tensor(0, ir.INPUT, t * d)
    ids = g.vit_block(ir.VitDims(t, d, h, mlp, eps), 0, 100, ir.OUTPUT)
    return g, ids


def block_values(ids, x: np.ndarray, w: dict) -> dict[int, np.ndarray]:
    vals = {0: x}
    for name in ir.BLOCK_WEIGHTS:
        vals[getattr(ids, name)] = w[name]
    return vals


CHAIN = 10
CHAIN_OUT = 20


def chain(inputs: dict[int, np.ndarray], ops: list) -> ir.Graph:
    """harness.rs:26-47: inputs declared as weights, each op writing the next
    id from CHAIN, the last writing CHAIN_OUT (an output)."""
    g = ir.Graph()
    for tid, v in inputs.items():
        g.tensor(tid, ir.WEIGHT, v.size)
    for i, o in enumerate(ops):
        last = i + 1 == len(ops)
        out = CHAIN_OUT if last else CHAIN + i
        g.tensor(out, ir.OUTPUT if last else ir.ACTIVATION, ir.output_elements(o))
        g.push(o, out)
    return g


def max_abs_err(got, want) -> float:
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))))
