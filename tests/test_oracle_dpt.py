"""The oracle's DPT-head operations (oracle/oracle.c, blo_ref_conv3x3 /
conv1x1 / conv_transpose / resize_bilinear) pinned by the reference's own
known-answer tests (crates/beatlm-bench/src/reference.rs, tests of the same
names) and by torch float64 on the CPU (a library, not the reference).
CPU only."""

import numpy as np
import pytest
import torch

import oracle


def test_a_one_hot_kernel_copies_the_input_through_the_centre_tap():
    h, w, c = 3, 4, 2
    weights = np.zeros(9 * c * c, np.float32)
    for ci in range(c):
        weights[(4 * c + ci) * c + ci] = 1.0
    x = np.arange(h * w * c, dtype=np.float32)
    assert np.array_equal(oracle.conv3x3(x, weights, None, h, w, c, c), x)


def test_a_corner_pixel_sums_only_the_taps_inside_the_image():
    assert np.array_equal(oracle.conv3x3(np.ones(4), np.ones(9), None, 2, 2, 1, 1), [4.0] * 4)
    assert np.array_equal(oracle.conv3x3(np.ones(4), np.ones(9), [0.5], 2, 2, 1, 1), [4.5] * 4)


def test_a_strided_convolution_samples_every_stride_th_pixel():
    h, w = 5, 4
    weights = np.zeros(9, np.float32)
    weights[4] = 1.0
    x = np.arange(h * w, dtype=np.float32)
    assert np.array_equal(oracle.conv3x3(x, weights, None, h, w, 1, 1, 2), [0, 2, 8, 10, 16, 18])
    ones = oracle.conv3x3(np.ones(20), np.ones(9), [0.5], h, w, 1, 1, 2)
    assert np.array_equal(ones[:2], [4.5, 6.5])


def test_a_1x1_convolution_is_the_matrix_product_of_its_pixels():
    x = np.arange(15, dtype=np.float32) * 0.25 - 1.0
    w = 0.5 - np.arange(6, dtype=np.float32) * 0.3
    b = np.array([0.1, -0.2], np.float32)
    assert np.array_equal(oracle.conv1x1(x, w, b, 5, 3, 2), oracle.matmul(x, w, b, 5, 3, 2))


def test_a_transposed_convolution_writes_one_block_per_input_pixel():
    out = oracle.conv_transpose([10.0, -1.0], [1.0, 2.0, 3.0, 4.0], [0.5], 1, 2, 1, 1, 2)
    assert np.array_equal(out, [10.5, 20.5, -0.5, -1.5, 30.5, 40.5, -2.5, -3.5])


def test_aligned_corner_resampling_keeps_the_corners_and_interpolates_linearly():
    assert np.array_equal(oracle.resize_bilinear([0.0, 2.0, 4.0, 6.0], 2, 2, 3, 3, 1), [0, 1, 2, 2, 3, 4, 4, 5, 6])
    assert np.array_equal(oracle.resize_bilinear(np.arange(4, dtype=np.float32), 1, 4, 1, 7, 1),
                          [0, 0.5, 1, 1.5, 2, 2.5, 3])
    assert np.array_equal(oracle.resize_bilinear([1.0, 9.0], 2, 1, 1, 1, 1), [1.0])


def _nchw(x, h, w, c):
    return torch.tensor(x, dtype=torch.float64).reshape(1, h, w, c).permute(0, 3, 1, 2)


@pytest.mark.parametrize("h,w,cin,cout,stride", [(5, 7, 3, 4, 1), (9, 9, 8, 6, 2), (1, 1, 2, 3, 1), (4, 6, 5, 2, 3),
                                                 (19, 19, 16, 8, 2)])
def test_conv3x3_matches_torch(h, w, cin, cout, stride):
    rng = np.random.default_rng(h * 100 + cin)
    x = rng.standard_normal(h * w * cin).astype(np.float32)
    wt = rng.standard_normal(9 * cin * cout).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    got = oracle.conv3x3(x, wt, b, h, w, cin, cout, stride)
    tw = torch.tensor(wt, dtype=torch.float64).reshape(3, 3, cin, cout).permute(3, 2, 0, 1)
    want = torch.nn.functional.conv2d(_nchw(x, h, w, cin), tw, torch.tensor(b, dtype=torch.float64), stride=stride,
                                      padding=1).permute(0, 2, 3, 1).reshape(-1).numpy()
    assert got.shape == want.shape and np.max(np.abs(got - want)) < 1e-5


@pytest.mark.parametrize("h,w,cin,cout,f", [(3, 4, 5, 6, 2), (2, 2, 3, 3, 4), (5, 3, 8, 4, 2)])
def test_conv_transpose_matches_torch(h, w, cin, cout, f):
    rng = np.random.default_rng(f * 10 + cin)
    x = rng.standard_normal(h * w * cin).astype(np.float32)
    wt = rng.standard_normal(f * f * cin * cout).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    got = oracle.conv_transpose(x, wt, b, h, w, cin, cout, f)
    tw = torch.tensor(wt, dtype=torch.float64).reshape(f, f, cin, cout).permute(2, 3, 0, 1)
    want = torch.nn.functional.conv_transpose2d(_nchw(x, h, w, cin), tw, torch.tensor(b, dtype=torch.float64),
                                                stride=f).permute(0, 2, 3, 1).reshape(-1).numpy()
    assert np.max(np.abs(got - want)) < 1e-5


@pytest.mark.parametrize("ih,iw,oh,ow,c", [(4, 5, 9, 7, 3), (5, 5, 1, 1, 2), (3, 3, 3, 3, 1), (7, 6, 4, 3, 2),
                                           (19, 19, 37, 37, 4)])
def test_resize_bilinear_matches_torch(ih, iw, oh, ow, c):
    x = np.random.default_rng(ih + oh).standard_normal(ih * iw * c).astype(np.float32)
    got = oracle.resize_bilinear(x, ih, iw, oh, ow, c)
    want = torch.nn.functional.interpolate(_nchw(x, ih, iw, c), size=(oh, ow), mode="bilinear",
                                           align_corners=True).permute(0, 2, 3, 1).reshape(-1).numpy()
    assert np.max(np.abs(got - want)) < 1e-6
