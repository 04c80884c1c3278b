"""LayerNorms folded into the products that read them: LN(x) W + b computed
inside the product from x's row statistics, which the product that wrote x
leaves: in f32 storage from x centred per 32-column block (the shadow) plus
the block means' correction, in f16 storage as rstd (x (gamma W) - mean c)
+ d. The fold must give the
LayerNorm-then-product result within the f32 bar (against the oracle's
LayerNorm and matmul), whatever order the host encodes the kernels in:
the LayerNorm or its reader encoded alone, x rewritten by the host in
between, ranges replayed as graphs."""

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir

pytestmark = pytest.mark.gpu

T, D, M = 1370, 384, 1536
EPS = 1e-6
# tensor ids of the three-kernel program below
V, X, WO, BO, LS, G2, B2, W1, B1 = 0, 1, 2, 3, 4, 5, 6, 7, 8
X1, N2, H, OUT = 12, 13, 14, 15


def values(seed=5, d=D, m=M, t=T, f16=False):
    rng = np.random.default_rng(seed)
    dt = np.float16 if f16 else np.float32
    return {
        V: rng.uniform(-1, 1, t * d).astype(dt),
        X: rng.uniform(-2, 2, t * d).astype(dt),
        WO: rng.uniform(-0.05, 0.05, d * d).astype(dt),
        BO: rng.uniform(-0.1, 0.1, d).astype(dt),
        LS: rng.uniform(0.1, 1.0, d).astype(dt),
        G2: (1 + 0.1 * rng.standard_normal(d)).astype(dt),
        B2: (0.1 * rng.standard_normal(d)).astype(dt),
        W1: rng.uniform(-0.05, 0.05, d * m).astype(dt),
        B1: rng.uniform(-0.1, 0.1, m).astype(dt),
    }


def graph(t=T, d=D, m=M):
    """x1 = x + ls (.) (v Wo + bo) (the fold's producer), n = LN(x1), out =
    GELU(n W1 + b1) (its consumer); x1 is an output, n internal."""
    g = ir.Graph()
    g.tensor(V, ir.INPUT, t * d)
    g.tensor(X, ir.INPUT, t * d)
    for tid, n in [(WO, d * d), (BO, d), (LS, d), (G2, d), (B2, d), (W1, d * m), (B1, m)]:
        g.tensor(tid, ir.WEIGHT, n)
    g.tensor(10, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_MATMUL, [V, WO, BO], [t, d, d]), 10)
    g.tensor(11, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_CHANNEL_SCALE, [10, LS], [t, d]), 11)
    g.tensor(X1, ir.OUTPUT, t * d)
    g.push(ir.op(ir.OP_ADD, [11, X], [t * d]), X1)
    g.tensor(N2, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_LAYER_NORM, [X1, G2, B2], [t, d], EPS), N2)
    g.tensor(H, ir.ACTIVATION, t * m)
    g.push(ir.op(ir.OP_MATMUL, [N2, W1, B1], [t, d, m]), H)
    g.tensor(OUT, ir.OUTPUT, t * m)
    g.push(ir.op(ir.OP_GELU_ERF, [H], [t * m]), OUT)
    return g


def want_out(x1, v, t=T, d=D, m=M):
    """The oracle's LayerNorm, matmul and GELU-erf over the given x1."""
    n = oracle.layernorm(x1, v[G2], v[B2], t, d, EPS)
    return oracle.gelu_erf(oracle.matmul(n, v[W1], v[B1], t, d, m))


def assert_close(got, want, what, abs_tol=oracle.TOLERANCE_ABS, rel_tol=oracle.TOLERANCE_REL):
    bad = oracle.first_mismatch(got, want, abs_tol, rel_tol)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    print(f"{what}: max abs error {err:.3e}")
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}; max abs error {err:.3e}"


@pytest.fixture()
def prepared(ctx):
    preps = []

    def make(math=hip.F32_MATH_SPLIT_BF16, dtype=hip.F32):
        ctx.set_f32_math(math)
        p = ir.prepare(ctx, graph(), dtype=dtype)
        preps.append(p)
        return p

    yield make
    for p in preps:
        p.close()
    ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
def test_a_folded_layernorm_matches_the_layernorm_then_the_product(ctx, prepared, math):
    prep = prepared(math)
    labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
    assert "folded into 2" in labels[1] and "row statistics" in labels[0] and "< layernorm 1" in labels[2], labels
    v = values()
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1)
    assert_close(prep.read(OUT), want_out(x1, v), f"folded LayerNorm, f32 math {math}")
    # The producer's statistics: per row and 32-column block, the mean and the
    # sum of squared deviations of x1 as stored.
    st = prep.kernels.fold_read(0, 0, T * (D // 32) * 2).reshape(T, D // 32, 2).astype(np.float64)
    blocks = x1.astype(np.float64).reshape(T, D // 32, 32)
    mean = blocks.mean(2)
    np.testing.assert_allclose(st[:, :, 0], mean, atol=1e-6)
    np.testing.assert_allclose(st[:, :, 1], ((blocks - mean[:, :, None]) ** 2).sum(2), rtol=1e-5, atol=1e-5)
    # The consumer's column vectors: c = column sums of gamma W, d = beta W + b.
    vec = prep.kernels.fold_read(0, 1, 2 * M).astype(np.float64)
    w1 = v[W1].astype(np.float64).reshape(D, M)
    np.testing.assert_allclose(vec[:M], (v[G2][:, None] * w1).sum(0), atol=2e-5)
    np.testing.assert_allclose(vec[M:], v[B2] @ w1 + v[B1], atol=2e-5)


def bf16_words(w: np.ndarray) -> np.ndarray:
    """bf16 values (as uint16 words) widened to float64."""
    return (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def read_shadow(prep, math, t=T, d=D) -> np.ndarray:
    """The fold's shadow as the consumer reads it: hi + lo of the bf16 planes
    for bf16x3, the f32 values for the f32 matrix cores."""
    raw = prep.kernels.fold_read(0, 2, t * d)
    if math == hip.F32_MATH_SPLIT_BF16:
        w = raw.view(np.uint16)
        return bf16_words(w[: t * d]) + bf16_words(w[t * d:])
    return raw.astype(np.float64)


def centred(x, t=T, d=D) -> np.ndarray:
    """x less each row's 32-column block means (float64)."""
    b = x.astype(np.float64).reshape(t, d // 32, 32)
    return (b - b.mean(2, keepdims=True)).reshape(-1)


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
@pytest.mark.parametrize("offset", [10.0, 30.0, 100.0])
def test_a_folded_layernorm_is_shift_invariant(ctx, prepared, math, offset):
    """Rows whose mean is 10, 30 and 100 times their spread: x1 = x + ls (.)
    (v Wo + bo) with x = offset + U(-1, 1). The reference normalises x - mean
    before anything multiplies it, two passes, mean first
    (crates/beatlm/src/codegen/wgsl.rs:519-585,
    crates/beatlm-bench/src/reference.rs:247-270), so its result does not
    depend on the offset; the fold must stay within the f32 bar (max abs
    error <= 1e-4 against the oracle's LayerNorm and matmul) at every offset,
    in both f32 maths. Its shadow holds x1 less each block's mean."""
    prep = prepared(math)
    v = values()
    v[X] = (offset + v[X] / 2).astype(np.float32)
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1)
    spread = float(np.std(x1.astype(np.float64).reshape(T, D), axis=1).mean())
    got = prep.read(OUT)
    want = want_out(x1, v)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    print(f"folded LayerNorm, rows at {offset} (mean / spread {offset / spread:.0f}), f32 math {math}: "
          f"max abs error {err:.3e}")
    assert_close(got, want, f"offset {offset}, f32 math {math}")
    assert err <= 1e-4
    # The shadow: x1 less its block means as the statistics hold them (the
    # f32 difference), as the consumer multiplies it: bf16x3's hi + lo within
    # 2^-16 of each value, the f32 matrix cores' exactly. The block means are
    # within an f32 rounding of x1's.
    st = prep.kernels.fold_read(0, 0, T * (D // 32) * 2).reshape(T, D // 32, 2)
    np.testing.assert_allclose(st[:, :, 0], x1.astype(np.float64).reshape(T, D // 32, 32).mean(2),
                               rtol=4e-7, atol=1e-6)
    cx = (x1.reshape(T, D // 32, 32) - st[:, :, :1]).astype(np.float64).ravel()
    sh = read_shadow(prep, math)
    if math == hip.F32_MATH_SPLIT_BF16:
        assert np.all(np.abs(sh - cx) <= 2.0 ** -16 * np.abs(cx)), float(np.max(np.abs(sh - cx)))
    else:
        assert np.array_equal(sh, cx)
    assert float(np.max(np.abs(cx - centred(x1)))) <= 2e-5 * offset


@pytest.mark.parametrize("math", [hip.F32_MATH_SPLIT_BF16, hip.F32_MATH_MFMA_F32])
def test_a_folded_layernorm_with_an_outlier_channel(ctx, prepared, math):
    """Every seventh row carries one channel 500 above the rest (a different
    channel each time): the row's variance is dominated by it, and the
    product after the fold stays within the f32 bar."""
    prep = prepared(math)
    v = values()
    x = v[X].reshape(T, D).copy()
    rows = np.arange(0, T, 7)
    x[rows, (rows * 37) % D] += 500.0
    v[X] = x.ravel()
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1)
    got = prep.read(OUT)
    want = want_out(x1, v)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    print(f"folded LayerNorm, outlier channels, f32 math {math}: max abs error {err:.3e}")
    assert_close(got, want, f"outlier channels, f32 math {math}")
    assert err <= 1e-4


def test_a_folded_layernorm_in_f16_storage_is_within_the_f16_bar(ctx, prepared):
    prep = prepared(dtype=hip.F16)
    v = values(f16=True)
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1).astype(np.float32)
    v32 = {k: a.astype(np.float32) for k, a in v.items()}
    got = prep.read(OUT).astype(np.float32)
    err = float(np.max(np.abs(got - want_out(x1, v32))))
    print(f"folded LayerNorm, f16 storage: max abs error {err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize("offset", [10.0, 30.0])
def test_a_folded_layernorm_in_f16_storage_with_offset_rows(ctx, prepared, offset):
    """f16 storage keeps x uncentred (the product reads x itself and
    subtracts mean c in f32): rows at 10 and 30 times their spread stay
    within the f16 bar."""
    prep = prepared(dtype=hip.F16)
    v = values(f16=True)
    v[X] = (offset + v[X].astype(np.float32) / 2).astype(np.float16)
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1).astype(np.float32)
    v32 = {k: a.astype(np.float32) for k, a in v.items()}
    got = prep.read(OUT).astype(np.float32)
    err = float(np.max(np.abs(got - want_out(x1, v32))))
    print(f"folded LayerNorm, f16 storage, rows at {offset}: max abs error {err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize("offset", [0.0, 30.0])
def test_an_f16_fold_into_tiles_of_128_rows(ctx, prepared, monkeypatch, offset):
    """An f16 product of 128 x 64 tiles takes its rows' statistics in two
    passes of its prologue (rows 0-63, then 64-127, 128 rows against the
    workgroup's 64 quads); the last tile is partial (1370 = 10 x 128 + 90)."""
    monkeypatch.setenv("BL_GEMM_TILE", "3@1536")
    prep = prepared(dtype=hip.F16)
    labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
    assert any("128x64" in lab and "< layernorm" in lab for lab in labels), labels
    v = values(f16=True)
    v[X] = (offset + v[X].astype(np.float32) / 2).astype(np.float16)
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    ctx.synchronize()
    x1 = prep.read(X1).astype(np.float32)
    v32 = {k: a.astype(np.float32) for k, a in v.items()}
    got = prep.read(OUT).astype(np.float32)
    err = float(np.max(np.abs(got - want_out(x1, v32))))
    print(f"folded LayerNorm into 128-row f16 tiles, rows at {offset}: max abs error {err:.3e}")
    assert err <= 2e-2


def test_the_folded_kernels_encoded_alone_after_the_host_rewrites_x(ctx, prepared):
    """x rewritten by the host: the producer's statistics are stale, so the
    LayerNorm (encoded alone) or its reader (encoded alone, or in a replayed
    range) makes them from x before the product reads them."""
    prep = prepared()
    v = values()
    for tid, a in v.items():
        prep.write(tid, a)
    prep.run()
    for step, encode in enumerate([
        lambda: (prep.kernels.encode(1), prep.kernels.encode(2)),  # the LayerNorm, then its reader
        lambda: prep.kernels.encode(2),  # the reader alone
        lambda: prep.kernels.encode_range(1, 2),  # a range from the LayerNorm (graph replay)
        lambda: prep.kernels.encode_range(1, 2),  # the same range again
    ]):
        x1 = oracle.uniform(40 + step, T * D, -3.0, 3.0)
        prep.write(X1, x1)
        encode()
        ctx.synchronize()
        assert_close(prep.read(OUT), want_out(x1, v), f"after a host write of x, encoding {step}")
    # The whole program again: the producer's own statistics are used.
    prep.run()
    ctx.synchronize()
    assert_close(prep.read(OUT), want_out(prep.read(X1), v), "the whole program after the host writes")
    # GPU launches of the replayed graphs: the folded LayerNorm launches
    # nothing; from the LayerNorm on, its statistics kernel takes the place of
    # the producer's.
    assert prep.kernels.range_launches(0, 3) == 2
    assert prep.kernels.range_launches(1, 2) == 2


def test_a_layernorm_whose_input_no_product_wrote_is_not_folded(ctx):
    """x is the program's input: no product leaves its statistics, and the
    LayerNorm runs as a kernel of its own."""
    g = ir.Graph()
    g.tensor(X1, ir.INPUT, T * D)
    for tid, n in [(G2, D), (B2, D), (W1, D * M), (B1, M)]:
        g.tensor(tid, ir.WEIGHT, n)
    g.tensor(N2, ir.ACTIVATION, T * D)
    g.push(ir.op(ir.OP_LAYER_NORM, [X1, G2, B2], [T, D], EPS), N2)
    g.tensor(OUT, ir.OUTPUT, T * M)
    g.push(ir.op(ir.OP_MATMUL, [N2, W1, B1], [T, D, M]), OUT)
    prep = ir.prepare(ctx, g)
    try:
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        assert not any("folded" in s for s in labels), labels
    finally:
        prep.close()


# tensor ids of the prepend program below
TOK, PAT, POS = 20, 21, 22
XP = 23


def prepend_graph(t=T, d=D, m=M):
    """x = prepend(token, patches) + pos (the class token and position add of
    the embeddings: the fold's producer), n = LN(x), out = GELU(n W1 + b1)."""
    g = ir.Graph()
    g.tensor(PAT, ir.INPUT, (t - 1) * d)
    for tid, n in [(TOK, d), (POS, t * d), (G2, d), (B2, d), (W1, d * m), (B1, m)]:
        g.tensor(tid, ir.WEIGHT, n)
    g.tensor(30, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_PREPEND_TOKEN, [TOK, PAT], [t - 1, d]), 30)
    g.tensor(XP, ir.OUTPUT, t * d)
    g.push(ir.op(ir.OP_ADD, [30, POS], [t * d]), XP)
    g.tensor(N2, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_LAYER_NORM, [XP, G2, B2], [t, d], EPS), N2)
    g.tensor(H, ir.ACTIVATION, t * m)
    g.push(ir.op(ir.OP_MATMUL, [N2, W1, B1], [t, d, m]), H)
    g.tensor(OUT, ir.OUTPUT, t * m)
    g.push(ir.op(ir.OP_GELU_ERF, [H], [t * m]), OUT)
    return g


def prepend_values(f16=False, seed=9):
    v = values(seed=seed, f16=f16)
    dt = np.float16 if f16 else np.float32
    rng = np.random.default_rng(seed + 1)
    v[TOK] = rng.uniform(-1, 1, D).astype(dt)
    v[PAT] = rng.uniform(-2, 2, (T - 1) * D).astype(dt)
    v[POS] = rng.uniform(-0.5, 0.5, T * D).astype(dt)
    return {k: a for k, a in v.items() if k in (TOK, PAT, POS, G2, B2, W1, B1)}


@pytest.mark.parametrize("dtype", [hip.F32, hip.F16])
def test_the_class_token_prepend_leaves_the_statistics_of_a_folded_layernorm(ctx, dtype):
    """The prepend (with its position add) writes x, its block statistics and,
    for bf16x3, x's planes: the LayerNorm launches nothing, and the product
    after it matches the oracle's prepend, add, LayerNorm, matmul and GELU;
    the same after the host rewrites x and the reader is encoded alone."""
    f16 = dtype == hip.F16
    prep = ir.prepare(ctx, prepend_graph(), dtype=dtype)
    try:
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        assert "row statistics" in labels[0] and "folded into 2" in labels[1] and "< layernorm 1" in labels[2], labels
        v = prepend_values(f16)
        for tid, a in v.items():
            prep.write(tid, a)
        prep.run()
        ctx.synchronize()
        assert prep.kernels.range_launches(0, 3) == 2
        v32 = {k: a.astype(np.float32) for k, a in v.items()}
        want_x = oracle.add(oracle.prepend_token(v32[TOK], v32[PAT], T - 1, D), v32[POS])
        x = prep.read(XP).astype(np.float32)
        if f16:
            assert np.array_equal(x, want_x.astype(np.float16).astype(np.float32))
            err = float(np.max(np.abs(prep.read(OUT).astype(np.float32) - want_out(x, v32))))
            print(f"prepend as the fold's producer, f16 storage: max abs error {err:.3e}")
            assert err <= 2e-2
            return
        assert np.array_equal(x, want_x)
        assert_close(prep.read(OUT), want_out(x, v), "prepend as the fold's producer")
        st = prep.kernels.fold_read(0, 0, T * (D // 32) * 2).reshape(T, D // 32, 2).astype(np.float64)
        blocks = x.astype(np.float64).reshape(T, D // 32, 32)
        mean = blocks.mean(2)
        np.testing.assert_allclose(st[:, :, 0], mean, atol=1e-6)
        np.testing.assert_allclose(st[:, :, 1], ((blocks - mean[:, :, None]) ** 2).sum(2), rtol=1e-5, atol=1e-5)
        x2 = oracle.uniform(77, T * D, -3.0, 3.0)
        prep.write(XP, x2)
        prep.kernels.encode(2)
        ctx.synchronize()
        assert_close(prep.read(OUT), want_out(x2, v), "the reader alone after a host write of x")
    finally:
        prep.close()


# tensor ids of the embeddings program below
IMG, PW, PB = 40, 41, 42


def embeddings_graph(grid, d, m, fold=True):
    """patches = patch_embed(image), x = prepend(token, patches) + pos (the
    prepend fused into the patch embedding), then n = LN(x) and out =
    GELU(n W1 + b1) (the LayerNorm folded, the patch embedding its producer)."""
    t = grid * grid + 1
    g = ir.Graph()
    g.tensor(IMG, ir.INPUT, (grid * 14) ** 2 * 3)
    for tid, n in [(PW, 14 * 14 * 3 * d), (PB, d), (TOK, d), (POS, t * d), (G2, d), (B2, d), (W1, d * m), (B1, m)]:
        g.tensor(tid, ir.WEIGHT, n)
    g.tensor(31, ir.ACTIVATION, (t - 1) * d)
    g.push(ir.op(ir.OP_PATCH_EMBED, [IMG, PW, PB], [grid, grid, 14, 3, d]), 31)
    g.tensor(30, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_PREPEND_TOKEN, [TOK, 31], [t - 1, d]), 30)
    g.tensor(XP, ir.OUTPUT, t * d)
    g.push(ir.op(ir.OP_ADD, [30, POS], [t * d]), XP)
    g.tensor(N2, ir.ACTIVATION, t * d)
    g.push(ir.op(ir.OP_LAYER_NORM, [XP, G2, B2], [t, d], EPS), N2)
    g.tensor(H, ir.ACTIVATION, t * m)
    g.push(ir.op(ir.OP_MATMUL, [N2, W1, B1], [t, d, m]), H)
    g.tensor(OUT, ir.OUTPUT, t * m)
    g.push(ir.op(ir.OP_GELU_ERF, [H], [t * m]), OUT)
    return g


@pytest.mark.parametrize("grid,dtype", [(10, hip.F32), (37, hip.F32), (10, hip.F16)])
def test_the_prepend_fused_into_the_patch_embedding_feeds_a_folded_layernorm(ctx, grid, dtype):
    """The patch embedding writes x = [token; patches] + pos itself (the prepend
    launches nothing) and x's row statistics and planes for the LayerNorm
    folded into the product after it: two launches for the four kernels, x
    and the product's output as the oracle's embeddings, LayerNorm, matmul
    and GELU give them."""
    d, m = 384, 512
    t = grid * grid + 1
    f16 = dtype == hip.F16
    prep = ir.prepare(ctx, embeddings_graph(grid, d, m), dtype=dtype)
    try:
        labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
        assert "< prepend 1" in labels[0] and "row statistics" in labels[0], labels
        assert "fused into 0" in labels[1] and "folded into 3" in labels[2], labels
        dt = np.float16 if f16 else np.float32
        rng = np.random.default_rng(grid)
        v = {
            IMG: rng.uniform(-2, 2, (grid * 14) ** 2 * 3).astype(dt),
            PW: rng.uniform(-0.05, 0.05, 14 * 14 * 3 * d).astype(dt),
            PB: rng.uniform(-0.1, 0.1, d).astype(dt),
            TOK: rng.uniform(-1, 1, d).astype(dt),
            POS: rng.uniform(-0.5, 0.5, t * d).astype(dt),
            G2: (1 + 0.1 * rng.standard_normal(d)).astype(dt),
            B2: (0.1 * rng.standard_normal(d)).astype(dt),
            W1: rng.uniform(-0.05, 0.05, d * m).astype(dt),
            B1: rng.uniform(-0.1, 0.1, m).astype(dt),
        }
        for tid, a in v.items():
            prep.write(tid, a)
        prep.run()
        ctx.synchronize()
        assert prep.kernels.range_launches(0, len(prep.kernels)) == 2
        v32 = {k: a.astype(np.float32) for k, a in v.items()}
        patches = oracle.patch_embed(v32[IMG], v32[PW], v32[PB], grid, grid, 14, 3, d)
        want_x = oracle.add(oracle.prepend_token(v32[TOK], patches, t - 1, d), v32[POS])
        x = prep.read(XP).astype(np.float32)
        n = oracle.layernorm(x, v32[G2], v32[B2], t, d, EPS)
        want = oracle.gelu_erf(oracle.matmul(n, v32[W1], v32[B1], t, d, m))
        got = prep.read(OUT).astype(np.float32)
        if f16:
            ex = float(np.max(np.abs(x - want_x)))
            eo = float(np.max(np.abs(got - want)))
            print(f"prepend fused, f16 storage, grid {grid}: x {ex:.3e}, output {eo:.3e}")
            assert ex <= 2e-2 and eo <= 2e-2
            return
        # The class row is exact; the patch rows are the product's.
        assert np.array_equal(x[:d], want_x[:d])
        # Timing the fused prepend on its own launches nothing, so x stays.
        prep.kernels.time(1, 3)
        ctx.synchronize()
        assert np.array_equal(prep.read(XP), x)
        assert_close(x, want_x, f"embeddings with the prepend fused, grid {grid}")
        assert_close(got, want, f"the folded LayerNorm's product after the fused prepend, grid {grid}")
        st = prep.kernels.fold_read(0, 0, t * (d // 32) * 2).reshape(t, d // 32, 2).astype(np.float64)
        blocks = x.astype(np.float64).reshape(t, d // 32, 32)
        mean = blocks.mean(2)
        np.testing.assert_allclose(st[:, :, 0], mean, atol=1e-6)
        np.testing.assert_allclose(st[:, :, 1], ((blocks - mean[:, :, None]) ** 2).sum(2), rtol=1e-5, atol=1e-5)
    finally:
        prep.close()
