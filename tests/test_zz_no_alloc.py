"""bl_flash_attention_static, the entry point that allocates nothing, against
bl_kernels_encode's flash attention on the same qkv (a program of one flash
kernel, which runs its own prep): bit-identical outputs on two calls in a row,
the second with a smaller input, in both f32 (bf16x3) and f16; no device
memory allocated by the calls; shapes beyond the static array refused."""

import ctypes as C

import numpy as np
import pytest

import oracle
from beatlm_amd import hip, ir
from tests.blockdata import max_abs_err

pytestmark = pytest.mark.gpu

SCALE = 0.125


def flash_program(ctx, t, heads, dtype):
    g = ir.Graph()
    QKV, S, SS, P, OUT = 0, 10, 11, 12, 20
    g.tensor(QKV, ir.INPUT, t * 3 * heads * 64)
    g.tensor(S, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_ATTENTION_SCORES, [QKV], [t, heads, 64]), S)
    g.tensor(SS, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_SCALE, [S], [t * heads * t], SCALE), SS)
    g.tensor(P, ir.ACTIVATION, t * heads * t)
    g.push(ir.op(ir.OP_SOFTMAX, [SS], [t * heads, t]), P)
    g.tensor(OUT, ir.OUTPUT, t * heads * 64)
    g.push(ir.op(ir.OP_ATTENTION_VALUES, [P, QKV], [t, heads, 64]), OUT)
    prep = ir.prepare(ctx, g, dtype=dtype)
    assert [prep.program.name(k) for k in range(len(prep.program))] == ["flash_attention"]
    return prep, QKV, OUT


def free_bytes():
    rt = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert rt.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


@pytest.mark.parametrize("dtype", [hip.F32, hip.F16])
def test_the_allocation_free_attention_equals_the_kernels_attention(ctx, dtype):
    np_dtype = np.float16 if dtype == hip.F16 else np.float32
    lib = ctx._lib
    for call, (t, heads) in enumerate([(1370, 6), (257, 6)]):
        prep, QKV, OUT = flash_program(ctx, t, heads, dtype)
        qkv = oracle.uniform(50 + call, t * 3 * heads * 64, -1.0, 1.0).astype(np_dtype)
        prep.write(QKV, qkv)
        prep.run()
        ctx.synchronize()
        want = prep.read(OUT).copy()
        pq = prep.plan.placement(QKV)
        po = prep.plan.placement(OUT)
        qkv_ptr = prep.arenas.device_ptr(pq.arena, pq.offset)
        out_ptr = prep.arenas.device_ptr(po.arena, po.offset)
        # Clear the output, so the static call must write every element.
        prep.write(OUT, np.full(t * heads * 64, np.nan, np_dtype))
        allocs = ctx.allocations()
        if call > 0:
            before = free_bytes()
        ctx.check(lib.bl_flash_attention_static(ctx.handle, qkv_ptr, out_ptr, t, heads, SCALE, dtype))
        ctx.synchronize()
        if call > 0:
            assert free_bytes() == before, "the static entry point allocated device memory"
        assert ctx.allocations() == allocs
        got = prep.read(OUT)
        print(f"call {call}: T={t} H={heads} {'f16' if dtype == hip.F16 else 'f32'}: "
              f"identical={np.array_equal(got, want)}")
        assert np.array_equal(got, want), f"call {call} (T={t}): the static entry point differs from bl_kernels_encode"
        ref = oracle.attention(qkv.astype(np.float32), t, heads, 64, SCALE)
        err = max_abs_err(got.astype(np.float32), ref)
        assert err <= (1e-4 if dtype == hip.F32 else 2e-2), f"call {call}: max abs error {err:.3e} against the oracle"
        prep.close()


def test_shapes_beyond_the_static_array_are_refused(ctx):
    prep, QKV, OUT = flash_program(ctx, 64, 1, hip.F32)
    pq = prep.plan.placement(QKV)
    po = prep.plan.placement(OUT)
    qkv_ptr = prep.arenas.device_ptr(pq.arena, pq.offset)
    out_ptr = prep.arenas.device_ptr(po.arena, po.offset)
    # 200 000 tokens of 16 heads need far more than the array holds; nothing runs.
    rc = ctx._lib.bl_flash_attention_static(ctx.handle, qkv_ptr, out_ptr, 200_000, 16, SCALE, hip.F32)
    assert rc == hip.ERR_TOO_LARGE
    assert "static array holds" in ctx._lib.bl_last_error(ctx.handle).decode()
    prep.close()
