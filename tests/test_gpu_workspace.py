"""The backend's workspace laid out by lifetime: two folded LayerNorms whose
producer-to-consumer spans do not overlap share their statistics and planes,
so writing one fold's statistics must leave the other's stale. Encoded out of
order (the second fold's producer, then the first fold's, then the second
fold's consumer), the consumer must remake its statistics from its own x and
still match the oracle's LayerNorm, matmul and GELU."""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.test_gpu_fold import EPS, assert_close

pytestmark = pytest.mark.gpu

T, D, M = 1370, 384, 1536


def chain(g, base, t=T, d=D, m=M):
    """x1 = x + ls (.) (v Wo + bo), out = GELU(LN(x1) W1 + b1), tensor ids from
    `base`; x1 and out are outputs."""
    v, x, wo, bo, ls, g2, b2, w1, b1 = range(base, base + 9)
    g.tensor(v, ir.INPUT, t * d)
    g.tensor(x, ir.INPUT, t * d)
    for tid, n in [(wo, d * d), (bo, d), (ls, d), (g2, d), (b2, d), (w1, d * m), (b1, m)]:
        g.tensor(tid, ir.WEIGHT, n)
    g.tensor(base + 10, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_MATMUL, [v, wo, bo], [t, d, d]), base + 10)
    g.tensor(base + 11, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_CHANNEL_SCALE, [base + 10, ls], [t, d]), base + 11)
    g.tensor(base + 12, ir.OUTPUT, t * d)
    g.push(ir.op(ir.OP_ADD, [base + 11, x], [t * d]), base + 12)
    g.tensor(base + 13, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_LAYER_NORM, [base + 12, g2, b2], [t, d], EPS), base + 13)
    g.tensor(base + 14, ir.ACTIVATION, t * m)
    g.push(ir.op(ir.OP_MATMUL, [base + 13, w1, b1], [t, d, m]), base + 14)
    g.tensor(base + 15, ir.OUTPUT, t * m)
    g.push(ir.op(ir.OP_GELU_ERF, [base + 14], [t * m]), base + 15)


def chain_values(base, seed, t=T, d=D, m=M):
    rng = np.random.default_rng(seed)
    u = lambda lo, hi, n: rng.uniform(lo, hi, n).astype(np.float32)
    return {
        base: u(-1, 1, t * d), base + 1: u(-2, 2, t * d) + np.float32(seed),
        base + 2: u(-0.05, 0.05, d * d), base + 3: u(-0.1, 0.1, d), base + 4: u(0.1, 1.0, d),
        base + 5: (1 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        base + 6: (0.1 * rng.standard_normal(d)).astype(np.float32),
        base + 7: u(-0.05, 0.05, d * m), base + 8: u(-0.1, 0.1, m),
    }


def want(v, base, x1, t=T, d=D, m=M):
    n = oracle.layernorm(x1, v[base + 5], v[base + 6], t, d, EPS)
    return oracle.gelu_erf(oracle.matmul(n, v[base + 7], v[base + 8], t, d, m))


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
def test_folds_sharing_workspace_bytes_remake_their_statistics_when_run_out_of_order(ctx, math):
    ctx.set_f32_math(math)
    g = ir.Graph()
    chain(g, 0)
    chain(g, 100)
    prep = ir.prepare(ctx, g, dtype=hip.F32)
    try:
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        print(labels)
        prod = [k for k, s in enumerate(labels) if "> row statistics" in s]
        cons = [k for k, s in enumerate(labels) if "< layernorm" in s]
        assert len(prod) == 2 and len(cons) == 2 and prod[0] < cons[0] < prod[1] < cons[1], labels
        v = {**chain_values(0, 1), **chain_values(100, 2)}
        for tid, a in v.items():
            prep.write(tid, a)
        prep.run()
        ctx.synchronize()
        x1 = {b: prep.read(b + 12) for b in (0, 100)}
        for b in (0, 100):
            assert_close(prep.read(b + 15), want(v, b, x1[b]), f"chain {b}, in order")
        # The second fold's producer, then the first fold's, whose statistics
        # land on the bytes the second fold's consumer reads.
        prep.kernels.encode(prod[1])
        prep.kernels.encode(prod[0])
        ctx.synchronize()
        rows = T * (D // 32) * 2
        st0, st1 = prep.kernels.fold_read(0, 0, rows), prep.kernels.fold_read(1, 0, rows)
        assert np.array_equal(st0, st1), "the two folds are expected to share their workspace bytes"
        prep.kernels.encode(cons[1])
        ctx.synchronize()
        for b in (0, 100):
            assert np.array_equal(prep.read(b + 12), x1[b])
        assert_close(prep.read(115), want(v, 100, x1[100]), "chain 100, its consumer after the other fold's producer")
        st1 = prep.kernels.fold_read(1, 0, rows).reshape(T, D // 32, 2).astype(np.float64)
        blocks = x1[100].astype(np.float64).reshape(T, D // 32, 32)
        np.testing.assert_allclose(st1[:, :, 0], blocks.mean(2), atol=1e-5)
    finally:
        prep.close()
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)
