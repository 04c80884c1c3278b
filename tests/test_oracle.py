"""The oracle pinned: the reference's own known-answer tests
(crates/beatlm-bench/src/reference.rs:652-896), library cross-checks against
torch's CPU float64 ops (a library, not the reference), the WGSL-order
emulation against the f64 ops within the reference's tolerance, and
properties the mathematics fixes. CPU only."""

import math

import numpy as np
import pytest

import oracle

torch = pytest.importorskip("torch")
F = torch.nn.functional


def t64(a):
    return torch.tensor(np.asarray(a, np.float64))


# ---- generators (net.rs:183-203) ----

def test_the_lcg_matches_its_formula():
    # x <- x * 6364136223846793005 + 1442695040888963407 (mod 2^64),
    # value (x >> 40) / 2^24; uniform = low + (high - low) * value in f32.
    x = 5
    want = []
    for _ in range(4):
        x = (x * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        u = np.float32((x >> 40) / float(1 << 24))
        want.append(np.float32(-1.0) + np.float32(np.float32(2.0) * u))
    assert np.array_equal(oracle.uniform(5, 4, -1.0, 1.0), np.array(want, np.float32))


def test_the_generators_have_their_moments():
    u = oracle.uniform(9, 1_000_000, 0.0, 1.0)
    assert 0.0 <= u.min() and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 2e-3 and abs(u.var() - 1 / 12) < 2e-3
    n = oracle.normal(9, 1_000_000)
    assert abs(n.mean()) < 5e-3 and abs(n.std() - 1.0) < 5e-3


# ---- reference.rs known answers ----

def test_matmul_multiplies_and_adds_the_bias_per_column():
    a, b = [1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]
    assert oracle.matmul(a, b, None, 2, 2, 2).tolist() == [19.0, 22.0, 43.0, 50.0]
    assert oracle.matmul(a, b, [1.0, -1.0], 2, 2, 2).tolist() == [20.0, 21.0, 44.0, 49.0]


def test_attention_reads_its_head_of_the_packed_rows():
    qkv = np.arange(1, 13, dtype=np.float32)
    assert oracle.attention_scores(qkv, 2, 2, 1).tolist() == [3, 9, 8, 20, 21, 63, 32, 80]
    p = np.array([0, 1, 1, 0, 0, 1, 1, 0], np.float32)
    assert oracle.attention_values(p, qkv, 2, 2, 1).tolist() == [11, 6, 11, 6]


def test_softmax_rows_sum_to_one_and_survive_large_scores():
    p = oracle.softmax([1.0, 2.0, 3.0, 1000.0, 1000.0, -1000.0], 3)
    assert abs(p[:3].sum() - 1.0) < 1e-6
    assert p[2] > p[1] > p[0]
    assert p[3:].tolist() == [0.5, 0.5, 0.0]


@pytest.mark.parametrize(
    "x,want",
    [(0.0, 0.0), (0.5, 0.5204998778130465), (1.0, 0.8427007929497149), (2.0, 0.9953222650189527),
     (2.999999, 0.999977909363748), (3.0, 0.9999779095030014), (4.0, 0.9999999845827421),
     (-1.0, -0.8427007929497149)],
)
def test_erf_has_its_tabulated_values_on_both_sides_of_the_switch(x, want):
    assert abs(oracle.erf(x) - want) < 1e-12


def test_erf_agrees_with_libm_and_saturates():
    assert oracle.erf(30.0) == 1.0
    for x in np.linspace(-6, 6, 2001):
        assert abs(oracle.erf(float(x)) - math.erf(float(x))) < 1e-13


def test_the_erf_approximation_is_within_its_stated_error():
    # GELU_ERF_MAX_ERROR = 5e-7 over [-10, 10] step 2^-12 (kernel.rs:355-372).
    grid = (-10.0 + np.arange(81921, dtype=np.float64) / 4096.0).astype(np.float32)
    got = oracle.wg_gelu_erf(grid).astype(np.float64)
    exact = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in grid.astype(np.float64)])
    err = np.abs(got - exact)
    assert err.max() <= 5e-7
    # A dropped 0.5 or a sign error in the negative branch is far outside it.
    assert abs(oracle.gelu_erf([1.0])[0] - 0.841344746068543) < 1e-7
    assert oracle.gelu_erf([0.0])[0] == 0.0


def test_layernorm_gives_zero_mean_unit_variance_before_gamma_and_beta():
    out = oracle.layernorm([1.0, 2.0, 3.0, 4.0], [1.0] * 4, [0.0] * 4, 1, 4, 1e-5)
    assert abs(out.mean()) < 1e-6 and abs(out.var() - 1.0) < 1e-3


def test_element_wise_operations_compute_what_they_say():
    assert oracle.add([1.0, -2.0], [0.5, 2.0]).tolist() == [1.5, 0.0]
    assert oracle.relu([-1.0, 0.0, 3.0]).tolist() == [0.0, 0.0, 3.0]
    assert oracle.scale([2.0, -4.0], 0.5).tolist() == [1.0, -2.0]
    g = oracle.gelu_tanh([0.0, 1.0, -1.0, 10.0, -10.0])
    assert g[0] == 0.0 and abs(g[1] - 0.841192) < 1e-5 and abs(g[2] + 0.158808) < 1e-5
    assert abs(g[3] - 10.0) < 1e-6 and abs(g[4]) < 1e-6
    assert oracle.channel_scale([1.0, 2.0, 3.0, 4.0], [2.0, -1.0]).tolist() == [2.0, -2.0, 6.0, -4.0]


def test_a_patch_embedding_of_one_hot_weights_picks_a_pixel_of_each_patch():
    image = np.arange(16, dtype=np.float32)
    w = np.zeros(8, np.float32)
    w[4] = 1.0
    w[3] = 1.0
    out = oracle.patch_embed(image, w, [0.5, 0.0], 2, 2, 2, 1, 2)
    assert out.tolist() == [4.5, 1.0, 6.5, 3.0, 12.5, 9.0, 14.5, 11.0]
    assert oracle.prepend_token([7.0, 7.0], out, 4, 2)[2:].tolist() == out.tolist()


def test_mismatches_are_found_and_lengths_compared():
    assert oracle.first_mismatch([1.0, 2.0], [1.0, 2.0]) is None
    assert oracle.first_mismatch([1.0, 2.5], [1.0, 2.0]) == (1, 2.5, 2.0)
    assert oracle.first_mismatch([1.0], [1.0, 2.0]) is not None
    assert oracle.first_mismatch([float("nan")], [1.0]) is not None


# ---- library cross-checks (torch CPU float64) ----

def test_layernorm_matches_torch():
    x = oracle.uniform(1, 37 * 384, -3, 3)
    g, b = oracle.uniform(2, 384, 0.8, 1.2), oracle.uniform(3, 384, -0.1, 0.1)
    want = F.layer_norm(t64(x).view(37, 384), (384,), t64(g), t64(b), 1e-6).numpy().ravel()
    assert np.abs(oracle.layernorm(x, g, b, 37, 384, 1e-6) - want).max() < 1e-6


def test_softmax_and_gelu_match_torch():
    x = oracle.uniform(4, 41 * 17, -8, 8)
    want = torch.softmax(t64(x).view(41, 17), -1).numpy().ravel()
    assert np.abs(oracle.softmax(x, 17) - want).max() < 1e-7
    y = oracle.uniform(5, 4096, -10, 10)
    assert np.abs(oracle.gelu_erf(y) - F.gelu(t64(y)).numpy()).max() < 1e-6
    assert np.abs(oracle.gelu_tanh(y) - F.gelu(t64(y), approximate="tanh").numpy()).max() < 1e-5


@pytest.mark.parametrize("t,h,d", [(17, 2, 5), (41, 3, 8), (1, 2, 4), (64, 1, 64)])
def test_attention_matches_torch_sdpa(t, h, d):
    qkv = oracle.uniform(6 + t, t * 3 * h * d, -1, 1)
    q, k, v = t64(qkv).view(t, 3, h, d).permute(1, 2, 0, 3)
    want = F.scaled_dot_product_attention(q, k, v, scale=1.0 / math.sqrt(d)).permute(1, 0, 2).reshape(-1).numpy()
    fused = oracle.attention(qkv, t, h, d, 1.0 / math.sqrt(d))
    assert np.abs(fused - want).max() < 1e-6
    unfused = oracle.attention_values(
        oracle.softmax(oracle.scale(oracle.attention_scores(qkv, t, h, d), np.float32(1 / math.sqrt(d))), t), qkv, t, h, d
    )
    assert np.abs(unfused - want).max() < 1e-5


def test_patch_embed_matches_torch_conv2d():
    gh, gw, p, cin, cout = 3, 4, 5, 3, 7
    img = oracle.uniform(7, gh * p * gw * p * cin, -1, 1)
    w = oracle.uniform(8, p * p * cin * cout, -1, 1)
    b = oracle.uniform(9, cout, -0.1, 0.1)
    x = t64(img).view(1, gh * p, gw * p, cin).permute(0, 3, 1, 2)
    wt = t64(w).view(p, p, cin, cout).permute(3, 2, 0, 1)
    want = F.conv2d(x, wt, t64(b), stride=p).permute(0, 2, 3, 1).reshape(-1).numpy()
    assert np.abs(oracle.patch_embed(img, w, b, gh, gw, p, cin, cout) - want).max() < 1e-5


def torch_block(x, w, t, h, d, mlp, eps):
    """The pre-norm block written with torch's float64 ops."""
    D = h * d
    W = {k: t64(v) for k, v in w.items()}
    X = t64(x).view(t, D)
    n1 = F.layer_norm(X, (D,), W["norm1_g"], W["norm1_b"], eps)
    qkv = n1 @ W["qkv_w"].view(D, 3 * D) + W["qkv_b"]
    q, k, v = qkv.view(t, 3, h, d).permute(1, 2, 0, 3)
    a = F.scaled_dot_product_attention(q, k, v).permute(1, 0, 2).reshape(t, D)
    x1 = X + W["ls1"] * (a @ W["proj_w"].view(D, D) + W["proj_b"])
    n2 = F.layer_norm(x1, (D,), W["norm2_g"], W["norm2_b"], eps)
    hid = F.gelu(n2 @ W["fc1_w"].view(D, mlp) + W["fc1_b"])
    return (x1 + W["ls2"] * (hid @ W["fc2_w"].view(mlp, D) + W["fc2_b"])).reshape(-1).numpy()


@pytest.mark.parametrize("t,h,d", [(17, 2, 8), (41, 3, 16)])
def test_the_oracle_block_matches_a_torch_forward_pass(t, h, d):
    from tests.blockdata import block_weights

    D, mlp = h * d, 4 * h * d
    x = oracle.uniform(20, t * D, -2, 2)
    w = block_weights(D, mlp, 100, "reference")
    want = torch_block(x, w, t, h, d, mlp, 1e-6)
    assert np.abs(oracle.vit_block(x, w, t, h, d, mlp, 1e-6) - want).max() < 1e-5
    assert np.abs(oracle.vit_block(x, w, t, h, d, mlp, 1e-6, attention_rounded=False) - want).max() < 1e-5


# ---- the reference's WGSL arithmetic against its f64 reference ----

def test_the_wgsl_order_kernels_are_within_the_reference_tolerance():
    from tests.blockdata import block_weights

    t, h, d, mlp = 41, 2, 32, 256
    D = h * d
    x = oracle.uniform(30, t * D, -2, 2)
    w = block_weights(D, mlp, 200, "reference")
    got = oracle.WgBlock(w, t, h, d, mlp, 1e-6, threads=2)(x)
    assert oracle.first_mismatch(got, oracle.vit_block(x, w, t, h, d, mlp, 1e-6)) is None
    a = oracle.uniform(31, 17 * 40, -2, 2)
    b = oracle.uniform(32, 40 * 9, -1, 1)
    assert oracle.first_mismatch(oracle.wg_matmul(a, b, None, 17, 40, 9), oracle.matmul(a, b, None, 17, 40, 9)) is None
    s = oracle.uniform(33, 7 * 300, -8, 8)
    assert oracle.first_mismatch(oracle.wg_softmax(s, 300), oracle.softmax(s, 300)) is None
    g, bb = oracle.uniform(34, 100, 0.8, 1.2), oracle.uniform(35, 100, -0.1, 0.1)
    xx = oracle.uniform(36, 5 * 100, -3, 3)
    assert oracle.first_mismatch(oracle.wg_layernorm(xx, g, bb, 5, 100, 1e-6), oracle.layernorm(xx, g, bb, 5, 100, 1e-6)) is None


# ---- what the mathematics fixes ----

def test_attention_over_one_token_returns_its_value():
    h, d = 3, 8
    qkv = oracle.uniform(40, 3 * h * d, -1, 1)
    assert np.array_equal(oracle.attention(qkv, 1, h, d, 0.125), qkv[2 * h * d:])


def test_attention_with_equal_keys_averages_the_values():
    t, h, d = 9, 1, 4
    qkv = oracle.uniform(41, t * 3 * h * d, -1, 1).reshape(t, 3, d)
    qkv[:, 1, :] = qkv[0, 1, :]
    out = oracle.attention(qkv.ravel(), t, h, d, 0.5).reshape(t, d)
    assert np.abs(out - qkv[:, 2, :].mean(0)).max() < 1e-6
