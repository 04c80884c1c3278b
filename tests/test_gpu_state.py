"""What the backend derives from the arenas stays true to them.

- Packed weights: writing a new input every frame repacks nothing; writing a
  weight (through bl_arenas_write, or through bl_arenas_device_ptr followed
  by bl_arenas_invalidate) repacks exactly that weight, and the output
  follows the new weight.
- The attention scratch: a flash kernel whose K and V operands its QKV
  projection writes gives the attention of whatever qkv holds when it runs,
  also when it is encoded alone or after the host rewrote qkv.
- Lifetime: kernels keep their arenas; destroying the arenas first leaves the
  kernels runnable, and the arenas' memory is released with the last kernels.
"""

import ctypes as C

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import block_graph, block_values, block_weights, max_abs_err

pytestmark = pytest.mark.gpu

EPS = 1e-6


def hip_runtime():
    rt = C.CDLL("libamdhip64.so")
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rt.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    return rt


def assert_close(got, want, what):
    bad = oracle.first_mismatch(got, want)
    assert bad is None, f"{what}: element {bad[0]} is {bad[1]}, the oracle says {bad[2]}; max {max_abs_err(got, want):.3e}"


def test_a_new_input_every_frame_repacks_nothing_and_a_new_weight_repacks_it(ctx):
    t, d, h, mlp = 257, 384, 6, 1536
    w = block_weights(d, mlp, 300, "xavier")
    g, ids = block_graph(t, d, h, mlp, EPS)
    prep = ir.prepare(ctx, g)
    for tid, v in block_values(ids, oracle.normal(7, t * d), w).items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    made = prep.kernels.packs_made()
    assert made == 4  # QKV, out-proj, fc1, fc2
    for frame in range(5):
        x = oracle.normal(40 + frame, t * d)
        prep.write(0, x)
        prep.run()
        ctx.synchronize()
        assert prep.kernels.packs_made() == made, f"frame {frame}: a new input repacked weights"
        assert_close(prep.read(ids.output), oracle.vit_block(x, w, t, h, d // h, mlp, EPS), f"frame {frame}")
    # A new fc1 weight: one repack, and the output follows it.
    w2 = dict(w)
    w2["fc1_w"] = oracle.xavier(999, d, mlp)
    prep.write(ids.fc1_w, w2["fc1_w"])
    prep.run()
    ctx.synchronize()
    assert prep.kernels.packs_made() == made + 1
    assert_close(prep.read(ids.output), oracle.vit_block(x, w2, t, h, d // h, mlp, EPS), "after a new fc1 weight")
    # Written behind the backend's back, then invalidated: the same.
    rt = hip_runtime()
    w3 = dict(w2)
    w3["proj_w"] = oracle.xavier(998, d, d)
    p = prep.plan.placement(ids.proj_w)
    dst = prep.arenas.device_ptr(p.arena, p.offset)
    src = np.ascontiguousarray(w3["proj_w"], np.float32)
    ctx.synchronize()
    assert rt.hipMemcpy(dst, src.ctypes.data, src.nbytes, 1) == 0  # hipMemcpyHostToDevice
    prep.arenas.invalidate(p.arena, p.offset, src.nbytes)
    prep.run()
    ctx.synchronize()
    assert prep.kernels.packs_made() == made + 2
    assert_close(prep.read(ids.output), oracle.vit_block(x, w3, t, h, d // h, mlp, EPS), "after an invalidated write")
    prep.close()


def attention_program(ctx, t, heads, dtype):
    """x -> qkv = x Wqkv + b -> flash attention -> out, with every tensor in
    the plain layout (no split activations), so qkv can be written and read."""
    d = heads * 64
    g = ir.Graph()
    X, Wq, Bq, QKV, OUT = 0, 1, 2, 10, 20
    g.tensor(X, ir.INPUT, t * d)
    g.tensor(Wq, ir.WEIGHT, d * 3 * d)
    g.tensor(Bq, ir.WEIGHT, 3 * d)
    g.tensor(QKV, ir.ACTIVATION, t * 3 * d)
    g.push(ir.op(ir.OP_MATMUL, [X, Wq, Bq], [t, d, 3 * d]), QKV)
    g.tensor(11, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_ATTENTION_SCORES, [QKV], [t, heads, 64]), 11)
    g.tensor(12, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_SCALE, [11], [t * heads * t], 0.125), 12)
    g.tensor(13, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_SOFTMAX, [12], [t * heads, t]), 13)
    g.tensor(OUT, ir.OUTPUT, t * d)
    g.push(ir.op(ir.OP_ATTENTION_VALUES, [13, QKV], [t, heads, 64]), OUT)
    program = g.lower(ir.FUSION_ON).fuse_attention()
    program.set_dtype(dtype)
    plan = ir.Plan(program.tensors(), ir.profile("mi355x"))
    arenas = hip.Arenas(ctx, plan.arenas())
    kernels = hip.Kernels(ctx, arenas, program.specs(plan))
    names = [program.name(k) for k in range(len(program))]
    assert names == ["matmul", "flash_attention"], names
    np_dtype = np.float16 if dtype == hip.F16 else np.float32

    def write(tid, v):
        p = plan.placement(tid)
        arenas.write(p.arena, p.offset, np.ascontiguousarray(v, np_dtype))

    def read(tid, n):
        p = plan.placement(tid)
        return arenas.read(p.arena, p.offset, n, np_dtype).astype(np.float32)

    return program, kernels, arenas, write, read, (X, Wq, Bq, QKV, OUT)


@pytest.mark.parametrize("dtype", [hip.F32, hip.F16])
def test_flash_attention_reads_qkv_as_it_is_when_it_runs(ctx, dtype):
    t, heads = 300, 2
    d = heads * 64
    program, kernels, arenas, write, read, (X, Wq, Bq, QKV, OUT) = attention_program(ctx, t, heads, dtype)
    wq = oracle.fan_in_weights(2, d * 3 * d, d)
    bq = oracle.uniform(3, 3 * d, -0.1, 0.1)
    write(Wq, wq)
    write(Bq, bq)
    tol = 1e-4 if dtype == hip.F32 else 2e-2

    def check(what, qkv):
        got = read(OUT, t * d)
        q = qkv.astype(np.float32)
        want = oracle.attention(q, t, heads, 64, 0.125)
        err = max_abs_err(got, want)
        assert err <= tol * (1 + np.abs(want).max()), f"{what}: max abs error {err:.3e}"

    cast = (lambda v: v.astype(np.float16).astype(np.float32)) if dtype == hip.F16 else (lambda v: v)
    # In program order.
    x1 = cast(oracle.uniform(4, t * d, -1.0, 1.0))
    write(X, x1)
    kernels.encode(0)
    kernels.encode(1)
    ctx.synchronize()
    qkv1 = read(QKV, t * 3 * d)
    check("projection then attention", qkv1)
    # The host rewrites qkv: the attention follows it, not the projection's operands.
    qkv2 = cast(oracle.uniform(5, t * 3 * d, -1.0, 1.0))
    write(QKV, qkv2)
    kernels.encode(1)
    ctx.synchronize()
    check("attention after a host write of qkv", qkv2)
    # Encoded alone again, twice: the same.
    kernels.encode(1)
    kernels.encode(1)
    ctx.synchronize()
    check("attention encoded alone", qkv2)
    # The projection again, then the attention as a range (a captured graph).
    x3 = cast(oracle.uniform(6, t * d, -1.0, 1.0))
    write(X, x3)
    kernels.encode_all()
    ctx.synchronize()
    check("range after a new input", read(QKV, t * 3 * d))
    # A range of the attention alone after the host rewrote qkv.
    qkv4 = cast(oracle.uniform(7, t * 3 * d, -1.0, 1.0))
    write(QKV, qkv4)
    ctx.check(ctx._lib.bl_kernels_encode_range(kernels.handle, 1, 1, 0))
    ctx.synchronize()
    check("one-kernel range after a host write", qkv4)
    kernels.close()
    arenas.close()


def test_kernels_keep_their_arenas(ctx):
    t, d, h, mlp = 257, 384, 6, 1536
    w = block_weights(d, mlp, 300, "xavier")
    g, ids = block_graph(t, d, h, mlp, EPS)
    rt = hip_runtime()
    free0, total = C.c_size_t(), C.c_size_t()
    ctx.synchronize()
    rt.hipMemGetInfo(C.byref(free0), C.byref(total))
    prep = ir.prepare(ctx, g)
    x = oracle.normal(7, t * d)
    for tid, v in block_values(ids, x, w).items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    first = prep.read(ids.output)
    p = prep.plan.placement(ids.output)
    out_ptr = prep.arenas.device_ptr(p.arena, p.offset)
    # The arenas' handle goes first; the kernels still run over their memory.
    prep.arenas.close()
    prep.kernels.encode_all()
    ctx.synchronize()
    again = np.empty_like(first)
    assert rt.hipMemcpy(again.ctypes.data, out_ptr, again.nbytes, 2) == 0  # hipMemcpyDeviceToHost
    assert np.array_equal(again, first)
    prep.kernels.close()
    ctx.synchronize()
    free1 = C.c_size_t()
    rt.hipMemGetInfo(C.byref(free1), C.byref(total))
    # Everything the program allocated is back (within allocator granularity).
    assert free1.value + (64 << 20) >= free0.value


def test_a_program_holds_two_allocations_that_do_not_move_over_100_frames(ctx):
    """The arenas are one allocation and the kernels' workspace (packed
    weights, split-k partials, attention scratch) another; the device bytes
    held are exactly the plan's arenas plus that workspace; 100 frames with a
    new input each allocate nothing and hold no more."""
    t, d, h, mlp = 1370, 384, 6, 1536
    w = block_weights(d, mlp, 301, "xavier")
    g, ids = block_graph(t, d, h, mlp, EPS)
    allocs0, bytes0 = ctx.allocations(), ctx.device_bytes()
    prep = ir.prepare(ctx, g)
    assert ctx.allocations() == allocs0 + 2, "arenas + workspace"
    ws = prep.kernels.workspace_bytes()
    assert ws > 0
    arenas = 0
    for size in prep.plan.arenas():
        arenas = (arenas + 255) // 256 * 256 + size
    assert ctx.device_bytes() == bytes0 + arenas + ws
    for tid, v in block_values(ids, oracle.normal(8, t * d), w).items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    held = ctx.allocations(), ctx.device_bytes()
    for frame in range(100):
        if frame % 10 == 0:
            prep.write(0, oracle.normal(500 + frame, t * d))
        prep.run()
    ctx.synchronize()
    assert (ctx.allocations(), ctx.device_bytes()) == held
    x = oracle.normal(590, t * d)
    assert_close(prep.read(ids.output), oracle.vit_block(x, w, t, h, d // h, mlp, EPS), "after 100 frames")
    prep.close()
    assert ctx.device_bytes() == bytes0
