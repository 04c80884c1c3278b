"""The host side's restatement of the reference core (include/beatlm_ir.h),
tested as the reference tests its core: the block's lowering and lifetimes
(crates/beatlm-core/src/kernel.rs:3796-3884), the embeddings
(:3886-3956), split coverage (:3297-3401), part counts (:3403-3450), graph
errors, and the memory planner's rules (memory.rs:510-842). CPU only: the
IR lives in the backend library but makes no HIP call."""

import numpy as np
import pytest

from beatlm_amd import hip, ir
from beatlm_amd.ir import (
    ACTIVATION, FUSION_OFF, FUSION_ON, INPUT, OUTPUT, WEIGHT, Graph, IrError, Plan, op, profile, tensor_desc,
)

T, D, HEADS, HEAD_DIM, MLP = 1370, 384, 6, 64, 1536
X, Y = 0, 6
F32, F16 = hip.F32, hip.F16


def weight(g, tid, n):
    g.tensor(tid, WEIGHT, n)
    return tid


def add_op(g, o, tid, role=ACTIVATION):
    g.tensor(tid, role, ir.output_elements(o))
    g.push(o, tid)
    return tid


def encoder_block(g, x):
    """kernel.rs:3625-3752: one block at the real shapes, tensors from 100."""
    ln = lambda i, gm, bt: op(ir.OP_LAYER_NORM, [i, gm, bt], [T, D], 1e-6)
    mm = lambda a, b, bias, k, n: op(ir.OP_MATMUL, [a, b, bias], [T, k, n])
    g1, b1 = weight(g, 100, D), weight(g, 101, D)
    wqkv, bqkv = weight(g, 102, D * 3 * D), weight(g, 103, 3 * D)
    wo, bo = weight(g, 104, D * D), weight(g, 105, D)
    ls1 = weight(g, 106, D)
    g2, b2 = weight(g, 107, D), weight(g, 108, D)
    w1, bf1 = weight(g, 120, D * MLP), weight(g, 121, MLP)
    w2, bf2 = weight(g, 122, MLP * D), weight(g, 123, D)
    ls2 = weight(g, 124, D)
    n1 = add_op(g, ln(x, g1, b1), 109)
    qkv = add_op(g, mm(n1, wqkv, bqkv, D, 3 * D), 110)
    scores = add_op(g, op(ir.OP_ATTENTION_SCORES, [qkv], [T, HEADS, HEAD_DIM]), 111)
    scaled = add_op(g, op(ir.OP_SCALE, [scores], [T * HEADS * T], 0.125), 112)
    probs = add_op(g, op(ir.OP_SOFTMAX, [scaled], [T * HEADS, T]), 113)
    values = add_op(g, op(ir.OP_ATTENTION_VALUES, [probs, qkv], [T, HEADS, HEAD_DIM]), 114)
    projected = add_op(g, mm(values, wo, bo, D, D), 115)
    layer_scaled = add_op(g, op(ir.OP_CHANNEL_SCALE, [projected, ls1], [T, D]), 116)
    x1 = add_op(g, op(ir.OP_ADD, [layer_scaled, x], [T * D]), 118)
    n2 = add_op(g, ln(x1, g2, b2), 119)
    hidden = add_op(g, mm(n2, w1, bf1, D, MLP), 125)
    activated = add_op(g, op(ir.OP_GELU_ERF, [hidden], [T * MLP]), 126)
    out = add_op(g, mm(activated, w2, bf2, MLP, D), 127)
    ls_out = add_op(g, op(ir.OP_CHANNEL_SCALE, [out, ls2], [T, D]), 128)
    add_op(g, op(ir.OP_ADD, [x1, ls_out], [T * D]), Y, OUTPUT)


def block_graph():
    g = Graph()
    g.tensor(X, INPUT, T * D)
    encoder_block(g, X)
    return g


def assert_plan_holds(program, plan, prof):
    """kernel.rs:3764-3793: no two live-together tensors share a byte, every
    arena fits, and every kernel's tensors are live at that kernel."""
    assert plan.valid_on(prof)
    cap = min(prof.max_storage_buffer_binding_size, prof.max_buffer_size)
    assert all(a <= cap for a in plan.arenas())
    ts = program.tensors()
    for i, a in enumerate(ts):
        for b in ts[i + 1:]:
            if a.first_use <= b.last_use and b.first_use <= a.last_use:
                p, q = plan.placement(a.id), plan.placement(b.id)
                assert p.arena != q.arena or p.offset + p.size <= q.offset or q.offset + q.size <= p.offset
    life = {t.id: (t.first_use, t.last_use) for t in ts}
    for k in range(len(program)):
        for tid in program.bindings(k):
            f, l = life[tid]
            assert f <= k <= l


def test_an_encoder_block_fuses_layerscale_residuals_gelu_and_the_attention_scale():
    p = block_graph().lower(FUSION_ON)
    assert p.names() == [
        "layernorm", "matmul", "attention_scores+scale", "softmax", "attention_values",
        "matmul+channel_scale+add", "layernorm", "matmul+gelu_erf", "matmul+channel_scale+add",
    ]
    assert p.bindings(5) == [114, 104, 105, 106, X, 118]
    k5 = p.kernel(5)
    assert [(e.kind, e.channels) for e in k5.epilogue[: k5.n_epilogue]] == [(hip.EPI_CHANNEL_SCALE, D), (hip.EPI_ADD, 0)]
    assert p.bindings(5)[k5.epilogue[0].operand] == 106 and p.bindings(5)[k5.epilogue[1].operand] == X
    k2 = p.kernel(2)
    assert k2.n_epilogue == 1 and k2.epilogue[0].kind == hip.EPI_SCALE and k2.epilogue[0].factor == 0.125
    assert p.kernel(7).epilogue[0].kind == hip.EPI_GELU_ERF
    for gone in (111, 115, 116, 125, 127, 128):
        assert p.lifetime(gone) is None, gone
    unfused = block_graph().lower(FUSION_OFF)
    assert len(unfused) == 15
    assert unfused.name(3) == "map+scale"
    assert unfused.name(11) == "map+gelu_erf"
    assert unfused.name(7) == "map+channel_scale"
    assert unfused.bindings(7) == [115, 106, 116]


def test_an_encoder_blocks_lifetimes_come_from_its_kernels_and_its_plan_holds_split_or_whole():
    whole = block_graph().lower(FUSION_ON)
    assert whole.lifetime(110) == (1, 4)
    assert whole.lifetime(112) == (2, 3)
    assert whole.lifetime(113) == (3, 4)
    assert whole.lifetime(118) == (5, 8)
    assert whole.lifetime(X) == (0, 8)
    scores = next(t for t in whole.tensors() if t.id == 112)
    assert scores.elements * 4 == 45_045_600
    base = profile("baseline")
    assert_plan_holds(whole, Plan(whole.tensors(), base), base)
    for count in (2, 3, 7, 86, 200):
        split = whole.split([count] * len(whole))
        assert_plan_holds(split, Plan(split.tensors(), base), base)
        for k in range(len(split)):
            info = split.kernel(k)
            if info.main in (hip.MAIN_ATTENTION_SCORES, hip.MAIN_ATTENTION_VALUES):
                assert info.part.start % info.tile_rows == 0 and info.part.end <= T
    unfused = block_graph().lower(FUSION_OFF)
    assert_plan_holds(unfused, Plan(unfused.tensors(), base), base)


def test_the_embeddings_fuse_the_position_add_into_the_class_token_kernel():
    image, w, b, cls, pos = 0, 1, 2, 3, 4
    g = Graph()
    g.tensor(image, INPUT, 518 * 518 * 3)
    weight(g, 1, 14 * 14 * 3 * D)
    weight(g, 2, D)
    weight(g, 3, D)
    weight(g, 4, T * D)
    patches = add_op(g, op(ir.OP_PATCH_EMBED, [image, w, b], [37, 37, 14, 3, D]), 10)
    tokens = add_op(g, op(ir.OP_PREPEND_TOKEN, [cls, patches], [T - 1, D]), 11)
    embedded = add_op(g, op(ir.OP_ADD, [tokens, pos], [T * D]), 12)
    add_op(g, op(ir.OP_TOKENS_TO_MAP, [embedded], [37, 37, D]), 13, OUTPUT)
    p = g.lower(FUSION_ON)
    assert p.names() == ["patch_embed", "prepend_token+add", "tokens_to_map"]
    assert p.bindings(1) == [cls, patches, pos, 12]
    k0 = p.kernel(0)
    assert k0.output_end == (T - 1) * D
    assert k0.max_parts == -(-(T - 1) // 64)
    assert p.kernel(2).output_end == 37 * 37 * D
    assert len(g.lower(FUSION_OFF)) == 4


def test_the_model_builder_lowers_to_the_same_kernels():
    g = Graph()
    g.tensor(0, INPUT, T * D)
    ids = g.vit_block(ir.VitDims(T, D, HEADS, MLP, 1e-6), 0, 100, OUTPUT)
    assert g.lower().names() == block_graph().lower().names()
    assert ids.next_id == 100 + 14 + 15
    emb = Graph().vit_embeddings(37, 14, 3, D, 0)
    assert emb.next_id == 8


def test_the_encoder_taps_its_layers_through_the_final_norm_into_feature_maps():
    """encoder() (depth_anything_v2.rs:434-527): embeddings, the blocks up to
    the deepest tap, then per tap the shared final LayerNorm and the
    token-to-map, whose outputs are the features."""
    g = Graph()
    enc = ir.vit_encoder(g, 16, 14, 3, D, HEADS, MLP, 1e-6, [1, 2, 4])
    assert len(enc.blocks) == 4 and len(enc.features) == 3
    p = g.lower()
    names = p.names()
    assert names[:2] == ["patch_embed", "prepend_token+add"]
    assert names[-6:] == ["layernorm", "tokens_to_map"] * 3
    assert len(names) == 2 + 4 * 9 + 6
    assert all(p.role(f) == OUTPUT for f in enc.features)
    # Each tapped hidden state feeds the next block and the final norm; its
    # lifetime runs to the norm that reads it.
    tapped = [enc.blocks[i].output for i in (0, 1, 3)]
    assert all(p.role(t) == ACTIVATION for t in tapped)
    assert p.lifetime(tapped[0])[1] >= 2 + 4 * 9
    assert p.fuse_attention().names().count("flash_attention") == 4


def shapes():
    """One kernel of each kind the block uses, at small ragged sizes."""
    yield "layernorm", [(X, INPUT, 41 * 7), (1, WEIGHT, 7), (2, WEIGHT, 7)], op(ir.OP_LAYER_NORM, [X, 1, 2], [41, 7], 1e-5)
    yield "matmul", [(X, INPUT, 141 * 5), (1, WEIGHT, 5 * 9), (2, WEIGHT, 9)], op(ir.OP_MATMUL, [X, 1, 2], [141, 5, 9])
    yield "scores", [(X, INPUT, 130 * 3 * 2 * 5)], op(ir.OP_ATTENTION_SCORES, [X], [130, 2, 5])
    yield "softmax", [(X, INPUT, 41 * 17)], op(ir.OP_SOFTMAX, [X], [41, 17])
    yield "values", [(X, INPUT, 130 * 2 * 130), (1, INPUT, 130 * 3 * 2 * 5)], op(ir.OP_ATTENTION_VALUES, [X, 1], [130, 2, 5])
    yield "patch", [(X, INPUT, 10 * 2 * 7 * 2 * 3), (1, WEIGHT, 2 * 2 * 3 * 4), (2, WEIGHT, 4)], op(ir.OP_PATCH_EMBED, [X, 1, 2], [10, 7, 2, 3, 4])
    yield "prepend", [(X, WEIGHT, 6), (1, INPUT, 11 * 6)], op(ir.OP_PREPEND_TOKEN, [X, 1], [11, 6])
    yield "map", [(X, INPUT, 1000)], op(ir.OP_RELU, [X], [1000])


def single(tensors, o):
    g = Graph()
    for tid, role, n in tensors:
        g.tensor(tid, role, n)
    g.tensor(Y, OUTPUT, ir.output_elements(o))
    g.push(o, Y)
    return g


@pytest.mark.parametrize("name,tensors,o", list(shapes()), ids=[s[0] for s in shapes()])
def test_a_split_kernels_parts_cover_its_output_exactly_once(name, tensors, o):
    whole = single(tensors, o).lower(FUSION_ON)
    spec = whole.kernel(0)
    extent = spec.part.end
    grain = spec.tile_rows or 1
    assert spec.max_parts == -(-extent // grain)
    assert spec.part.count == 1 and spec.output_start == 0
    for count in sorted({1, 2, 3, spec.max_parts, spec.max_parts + 1, 1000}):
        split = whole.split([count])
        n = len(split)
        assert n == max(1, min(count, spec.max_parts))
        next_unit = next_el = 0
        sizes = []
        for i in range(n):
            part = split.kernel(i)
            assert (part.part.index, part.part.count) == (i, n)
            assert split.bindings(i) == whole.bindings(0)
            assert part.part.start == next_unit and part.part.end > part.part.start
            if part.part.end != extent:
                assert part.part.end % grain == 0
            assert part.output_start == next_el
            next_unit, next_el = part.part.end, part.output_end
            sizes.append(part.part.end - part.part.start)
        assert next_unit == extent and next_el == spec.output_end
        assert max(sizes) - min(sizes) <= 2 * grain


def test_the_part_count_is_the_duration_over_the_bound_rounded_up_and_clamped():
    small = single([(X, INPUT, 4 * 8), (1, WEIGHT, 8 * 4), (2, WEIGHT, 4)], op(ir.OP_MATMUL, [X, 1, 2], [4, 8, 4])).lower()
    assert small.kernel(0).max_parts == 1
    assert small.parts_within([10_000], 1_000) == [1]
    big = single([(X, INPUT, 1000)], op(ir.OP_RELU, [X], [1000])).lower()
    assert big.kernel(0).max_parts == 1000
    for duration, bound, parts in [(0, 1000, 1), (1, 1000, 1), (999, 1000, 1), (1000, 1000, 1), (1001, 1000, 2),
                                   (2700, 1000, 3), (3000, 1000, 3), (3001, 1000, 4), (5_000_000, 1, 1000),
                                   (2**64 - 1, 1, 1000)]:
        assert big.parts_within([duration], bound) == [parts], (duration, bound)
    with pytest.raises(IrError) as e:
        big.parts_within([1], 0)
    assert e.value.kind == "ZeroBound"
    with pytest.raises(IrError) as e:
        big.parts_within([], 1000)
    assert e.value.kind == "PartCounts"
    with pytest.raises(IrError) as e:
        big.split([2]).split([2, 2])
    assert e.value.kind == "AlreadySplit"


@pytest.mark.parametrize(
    "build,kind",
    [
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(1, INPUT, 4)), "DuplicateTensor"),
        (lambda g: g.tensor(1, INPUT, 0), "EmptyTensor"),
        (lambda g: g.tensor(1, INPUT, 2**31), "TensorTooLarge"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, ACTIVATION, 4), g.push(op(ir.OP_RELU, [9], [4]), 2)), "UnknownTensor"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, ACTIVATION, 5), g.push(op(ir.OP_RELU, [1], [4]), 2)), "ElementCount"),
        (lambda g: (g.tensor(1, ACTIVATION, 4), g.tensor(2, ACTIVATION, 4), g.push(op(ir.OP_RELU, [1], [4]), 2)), "ReadBeforeWritten"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, ACTIVATION, 4), g.push(op(ir.OP_RELU, [1], [4]), 2),
                    g.push(op(ir.OP_RELU, [1], [4]), 2)), "WrittenTwice"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, WEIGHT, 4), g.push(op(ir.OP_RELU, [1], [4]), 2)), "NotWritable"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, ACTIVATION, 4), g.push(op(ir.OP_SOFTMAX, [1], [0, 4]), 2)), "ZeroDimension"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, ACTIVATION, 4), g.push(op(ir.OP_SCALE, [1], [4], float("inf")), 2)), "NonFiniteScale"),
        (lambda g: (g.tensor(1, INPUT, 4), g.tensor(2, WEIGHT, 4), g.tensor(3, WEIGHT, 4), g.tensor(4, ACTIVATION, 4),
                    g.push(op(ir.OP_LAYER_NORM, [1, 2, 3], [1, 4], 0.0), 4)), "InvalidEpsilon"),
    ],
)
def test_malformed_graphs_are_errors_not_guesses(build, kind):
    g = Graph()
    with pytest.raises(IrError) as e:
        build(g)
    assert e.value.kind == kind


def test_lowering_refuses_empty_graphs_and_unwritten_tensors():
    with pytest.raises(IrError) as e:
        Graph().lower()
    assert e.value.kind == "EmptyGraph"
    g = Graph()
    g.tensor(1, INPUT, 4)
    g.tensor(2, ACTIVATION, 4)
    g.tensor(3, OUTPUT, 4)
    g.push(op(ir.OP_RELU, [1], [4]), 2)
    with pytest.raises(IrError) as e:
        g.lower()
    assert e.value.kind == "NeverWritten"


def test_a_stand_in_is_sized_and_timed_as_its_input_or_output():
    p = block_graph().lower()
    d = p.stand_in(X, 9000)
    assert (d.id, d.elements, d.first_use, d.last_use) == (9000, T * D, 0, 8)
    with pytest.raises(IrError):
        p.stand_in(110, 9001)  # an activation
    with pytest.raises(IrError):
        p.stand_in(X, 110)     # an id the program has


# ---- the backend's attention rewrite ----

def test_the_attention_triple_becomes_one_flash_kernel_and_its_scores_leave_the_plan():
    whole = block_graph().lower()
    fused = whole.fuse_attention()
    assert fused.names() == ["layernorm", "matmul", "flash_attention", "matmul+channel_scale+add", "layernorm",
                             "matmul+gelu_erf", "matmul+channel_scale+add"]
    k = fused.kernel(2)
    assert fused.bindings(2) == [110, 114] and k.scale == 0.125 and (k.first_op, k.end_op) == (2, 6)
    assert fused.lifetime(112) is None and fused.lifetime(113) is None
    mi = profile("mi355x")
    before, after = Plan(whole.tensors(), mi), Plan(fused.tensors(), mi)
    # The two 45 MB tensors of scores and probabilities were live together.
    assert after.total_bytes() <= before.total_bytes() - 2 * 45_045_600 + 24_000_000
    # Split after the rewrite: whole tiles of 64 query rows.
    split = fused.split([7] * len(fused))
    for i in range(len(split)):
        info = split.kernel(i)
        if info.main == hip.MAIN_FLASH_ATTENTION:
            assert info.part.start % 64 == 0


def test_the_high_resolution_block_is_plannable_only_with_flash_attention():
    t = 5477
    g = Graph()
    g.tensor(0, INPUT, t * D)
    g.vit_block(ir.VitDims(t, D, HEADS, MLP, 1e-6), 0, 100, OUTPUT)
    p = g.lower()
    # 5477 x 6 x 5477 f32 scores: 720 MB, past the baseline's 128 MiB binding (memory.rs:363-369).
    with pytest.raises(IrError) as e:
        Plan(p.tensors(), profile("baseline"))
    assert e.value.kind == "Plan.TensorTooLarge"
    fused = p.fuse_attention()
    plan = Plan(fused.set_dtype(F16).tensors(), profile("baseline"))
    assert plan.total_bytes() < 128 << 20


# ---- the memory planner (memory.rs:510-842) ----

def f32s(n, elements, first, last):
    return tensor_desc(n, F32, elements, first, last)


def test_disjoint_lifetimes_share_the_same_bytes():
    plan = Plan([f32s(0, 1024, 0, 1), f32s(1, 1024, 2, 3)], profile("baseline"))
    a, b = plan.placement(0), plan.placement(1)
    assert (a.arena, a.offset) == (b.arena, b.offset)
    assert plan.total_bytes() == 4096 and plan.peak_live_bytes() == 4096


def test_lifetimes_are_inclusive_at_both_ends():
    plan = Plan([f32s(0, 1024, 0, 2), f32s(1, 1024, 2, 4)], profile("baseline"))
    a, b = plan.placement(0), plan.placement(1)
    assert a.offset + a.size <= b.offset or b.offset + b.size <= a.offset
    assert plan.peak_live_bytes() == 8192


def test_offsets_are_aligned_and_sizes_rounded_to_four_bytes():
    plan = Plan([tensor_desc(0, F16, 3, 0, 1), tensor_desc(1, F16, 1, 0, 1)], profile("baseline"))
    a, b = plan.placement(0), plan.placement(1)
    assert (a.size, b.size) == (8, 4)
    assert (a.offset, b.offset) == (0, 256)
    assert plan.arenas() == [260]


def with_binding(size):
    p = profile("baseline")
    p.max_storage_buffer_binding_size = size
    return p


def test_arena_limits():
    with pytest.raises(IrError) as e:
        Plan([f32s(0, 256, 0, 0), f32s(1, 257, 0, 0)], with_binding(1024))
    assert e.value.kind == "Plan.TensorTooLarge"
    assert Plan([f32s(0, 256, 0, 0)], with_binding(1024)).arenas() == [1024]
    plan = Plan([f32s(0, 200, 0, 1), f32s(1, 200, 0, 1)], with_binding(1024))
    assert len(plan.arenas()) == 2 and plan.placement(0).arena != plan.placement(1).arena
    p = profile("baseline")
    p.max_buffer_size = 1024
    with pytest.raises(IrError):
        Plan([f32s(0, 257, 0, 0)], p)


@pytest.mark.parametrize(
    "tensors,kind",
    [
        ([f32s(7, 4, 0, 0), f32s(7, 8, 1, 1)], "Plan.DuplicateTensor"),
        ([f32s(3, 4, 5, 4)], "Plan.InvalidLifetime"),
        ([f32s(0, 0, 0, 0)], "Plan.EmptyTensor"),
        ([f32s(0, 2**64 - 1, 0, 0)], "Plan.SizeOverflow"),
    ],
)
def test_malformed_plans_are_errors(tensors, kind):
    with pytest.raises(IrError) as e:
        Plan(tensors, profile("baseline"))
    assert e.value.kind == kind


def test_bad_profiles_and_empty_plans():
    p = profile("baseline")
    p.min_storage_buffer_offset_alignment = 0
    with pytest.raises(IrError) as e:
        Plan([f32s(0, 1, 0, 0)], p)
    assert e.value.kind == "Plan.InvalidProfile"
    plan = Plan([], profile("baseline"))
    assert plan.arenas() == [] and plan.total_bytes() == 0 and plan.peak_live_bytes() == 0
    assert plan.placement(0) is None


def test_peak_live_bytes_is_the_most_live_at_one_operation():
    plan = Plan([f32s(0, 100, 0, 2), f32s(1, 50, 1, 1), f32s(2, 25, 3, 3)], profile("baseline"))
    assert plan.peak_live_bytes() == 600


def test_a_chain_of_operations_reuses_memory_down_to_two_activations():
    act = 1 << 20
    plan = Plan([f32s(n, act, n, n + 1) for n in range(8)], profile("baseline"))
    assert plan.peak_live_bytes() == 2 * act * 4 and plan.total_bytes() == 2 * act * 4


class Lcg:
    def __init__(self, s):
        self.s = s

    def next(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        return self.s >> 33

    def below(self, n):
        return self.next() % n


def random_graph(rng, max_elements):
    count, ops = 1 + rng.below(40), 1 + rng.below(30)
    out = []
    for n in range(count):
        first = rng.below(ops)
        last = first + rng.below(ops - first)
        dtype = F32 if rng.below(2) == 0 else F16
        out.append(tensor_desc(n, dtype, 1 + rng.below(max_elements), first, last))
    return out


def random_profile(rng):
    p = profile("baseline")
    p.min_storage_buffer_offset_alignment = [4, 16, 64, 256][rng.below(4)]
    p.max_storage_buffer_binding_size = 4096 * (1 + rng.below(8))
    p.max_buffer_size = p.max_storage_buffer_binding_size * 2
    return p


def check_rules(tensors, prof, plan):
    align = prof.min_storage_buffer_offset_alignment
    cap = min(prof.max_storage_buffer_binding_size, prof.max_buffer_size)
    arenas = plan.arenas()
    place = {t.id: plan.placement(t.id) for t in tensors}
    for t in tensors:
        p = place[t.id]
        nbytes = t.elements * (2 if t.dtype == F16 else 4)
        assert p.offset % align == 0 and p.size % 4 == 0 and nbytes <= p.size < nbytes + 4
        assert p.offset + p.size <= arenas[p.arena]
    assert all(a <= cap for a in arenas)
    for i, a in enumerate(tensors):
        for b in tensors[i + 1:]:
            pa, pb = place[a.id], place[b.id]
            if a.first_use <= b.last_use and b.first_use <= a.last_use and pa.arena == pb.arena:
                assert pa.offset + pa.size <= pb.offset or pb.offset + pb.size <= pa.offset
    assert plan.peak_live_bytes() <= plan.total_bytes()
    assert plan.valid_on(prof)


def test_rules_one_to_three_hold_on_many_generated_graphs():
    rng = Lcg(0x5EED)
    multi = reused = too_large = 0
    for _ in range(500):
        prof = random_profile(rng)
        tensors = random_graph(rng, 3000)
        try:
            plan = Plan(tensors, prof)
        except IrError as e:
            assert e.kind == "Plan.TensorTooLarge"
            too_large += 1
            continue
        check_rules(tensors, prof, plan)
        multi += len(plan.arenas()) > 1
        reused += plan.total_bytes() < sum(plan.placement(t.id).size for t in tensors)
    assert multi > 20 and reused > 20 and too_large > 5


def test_the_plan_does_not_depend_on_the_order_tensors_are_listed_in():
    rng = Lcg(7)
    for _ in range(50):
        prof = random_profile(rng)
        tensors = random_graph(rng, 600)
        try:
            fwd = Plan(tensors, prof)
        except IrError:
            continue
        bwd = Plan(list(reversed(tensors)), prof)
        assert fwd.arenas() == bwd.arenas()
        for t in tensors:
            a, b = fwd.placement(t.id), bwd.placement(t.id)
            assert (a.arena, a.offset, a.size) == (b.arena, b.offset, b.size)


def test_a_baseline_plan_is_valid_on_a_larger_device_but_not_the_reverse():
    base = profile("baseline")
    on_base = Plan([f32s(0, 1 << 20, 0, 1)], base)
    big = profile("baseline")
    big.max_storage_buffer_binding_size = 1 << 30
    big.max_buffer_size = 1 << 31
    big.min_storage_buffer_offset_alignment = 64
    assert on_base.valid_on(big)
    on_big = Plan([f32s(0, 40 << 20, 0, 1)], big)
    assert not on_big.valid_on(base)
    odd = profile("baseline")
    odd.min_storage_buffer_offset_alignment = 512
    assert not on_base.valid_on(odd)
