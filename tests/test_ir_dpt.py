"""The DPT head in the IR restatement (beatlm_amd/csrc/ir.cpp, beatlm_amd/ir.py
depth_decoder / depth_model): lowering, the ReLU prologue rule and the memory
plan of the whole Depth Anything V2 Small model, checked with the numbers the
reference's own tests and tables pin
(crates/beatlm/src/model/depth_anything_v2.rs:1062-1318,
crates/beatlm-core/src/kernel.rs:242-319, crates/beatlm-bench/src/main.rs:383-389).
CPU only."""

import pytest

from beatlm_amd import hip, ir

ENCODER_KERNELS = 2 + 12 * 9 + 4 * 2


def small_model(side=518):
    g = ir.Graph()
    m = ir.depth_model(g, ir.DepthConfig.small(), side)
    return g, m


def test_the_small_decoder_lowers_to_the_kernels_the_fusion_rules_give():
    g, m = small_model()
    p = g.lower(ir.FUSION_ON)
    names = p.names()[ENCODER_KERNELS:]
    unit1 = ["relu-conv2d3x3+relu", "conv2d3x3+add+add"]
    unit2 = ["relu-conv2d3x3+relu", "conv2d3x3+add"]
    tail = ["resize_bilinear", "matmul"]
    want = ["matmul", "conv_transpose2d", "conv2d3x3", "matmul", "conv_transpose2d", "conv2d3x3", "matmul",
            "conv2d3x3", "matmul", "conv2d3x3", "conv2d3x3"] + unit2 + tail
    for _ in range(3):
        want += unit1 + unit2 + tail
    want += ["conv2d3x3", "resize_bilinear", "conv2d3x3+relu", "matmul+relu"]
    assert names == want
    assert len(want) == 37
    assert sum(1 for k in range(len(p)) if p.kernel(k).prologue == hip.PRO_RELU) == 7
    # Unfused, every operation is a kernel.
    assert len(g.lower(ir.FUSION_OFF)) == 3 + 12 * 15 + 4 * 2 + 11 + 7 + 3 * 13 + 6
    # The stride-2 convolution takes 37 pixels to 19; the last fusion layer doubles 148 to 296.
    strided = p.kernel(ENCODER_KERNELS + 9)
    assert strided.main == hip.MAIN_CONV3X3 and (strided.dims[4], (strided.dims[0] - 1) // strided.dims[4] + 1,
                                                 strided.dims[3]) == (2, 19, 384)
    last_resize = p.kernel(len(p) - 6)
    assert last_resize.main == hip.MAIN_RESIZE_BILINEAR
    assert (last_resize.dims[0], last_resize.dims[2], last_resize.dims[4]) == (148, 296, 64)


def test_a_relu_read_twice_is_not_a_prologue_and_an_unfused_program_has_none():
    g, _ = small_model(182)
    assert all(g.lower(ir.FUSION_OFF).kernel(k).prologue == 0 for k in range(len(g.lower(ir.FUSION_OFF))))
    # The prologue convolution binds the ReLU's input: its bindings are as many as before.
    p = g.lower(ir.FUSION_ON)
    for k in range(len(p)):
        info = p.kernel(k)
        if info.prologue:
            assert info.main == hip.MAIN_CONV3X3 and info.n_bindings == 4


def test_the_whole_model_plans_as_the_reference_publishes_at_every_side():
    # main.rs:383-389: the memory plan of the whole model, one slot, fused.
    for side, total in ((518, 207_959_172), (434, 156_838_788), (350, 131_021_828), (266, 116_541_700),
                        (182, 106_010_884)):
        g, _ = small_model(side)
        p = g.lower(ir.FUSION_ON)
        assert len(p) == 155
        plan = ir.Plan(p.tensors(), ir.profile("baseline"))
        assert plan.total_bytes() == total, side
        assert plan.valid_on(ir.profile("baseline"))


def test_the_whole_model_at_518_pixels_plans_fused_unfused_and_split():
    g, m = small_model()
    whole = g.lower(ir.FUSION_ON)
    tensors = whole.tensors()
    assert sum(1 for t in tensors if t.elements * 4 == 518 * 518 * 32 * 4) == 2
    assert max(t.elements * 4 for t in tensors) == 45_045_600
    depth = next(t for t in tensors if t.id == m.depth)
    assert (depth.first_use, depth.last_use) == (0, len(whole) - 1)
    for f in m.encoder.features:
        t = next(t for t in tensors if t.id == f)
        reader = whole.kernel(t.last_use)
        assert reader.main == hip.MAIN_MATMUL and whole.bindings(t.last_use)[0] == f
    base = ir.profile("baseline")
    for program in (whole, g.lower(ir.FUSION_OFF), whole.split([3] * len(whole))):
        plan = ir.Plan(program.tensors(), base)
        assert plan.valid_on(base)
        ts = program.tensors()
        for k in range(len(program)):
            for tid in program.bindings(k):
                d = next(t for t in ts if t.id == tid)
                assert d.first_use <= k <= d.last_use
        live = sorted(ts, key=lambda t: t.id)
        for i, a in enumerate(live):
            pa = plan.placement(a.id)
            for b in live[i + 1:]:
                if a.first_use <= b.last_use and b.first_use <= a.last_use:
                    pb = plan.placement(b.id)
                    assert pa.arena != pb.arena or pa.offset + pa.size <= pb.offset or pb.offset + pb.size <= pa.offset


def test_a_conv_transpose_and_resize_split_along_output_pixels():
    g, _ = small_model(182)
    p = g.lower(ir.FUSION_ON)
    for k in range(len(p)):
        info = p.kernel(k)
        if info.main in (hip.MAIN_CONV_TRANSPOSE, hip.MAIN_RESIZE_BILINEAR):
            d = info.dims
            pixels = d[0] * d[4] * d[1] * d[4] if info.main == hip.MAIN_CONV_TRANSPOSE else d[2] * d[3]
            assert info.max_parts == pixels and info.tile_rows == 0
        if info.main == hip.MAIN_CONV3X3:
            assert info.tile_rows == 64
