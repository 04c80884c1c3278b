"""The C ABI as a drop-in boundary: the library loads without a GPU, exports
every function include/beatlm_hip.h, include/beatlm_ir.h,
include/beatlm_schedule.h and include/beatlm_load.h declare, and the
structs the host bindings pass have the C layout (checked against gcc
compiling the headers). CPU only; no compute call."""

import ctypes as C
import pathlib
import re
import subprocess

import pytest

from beatlm_amd import hip, ir, load, schedule

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADERS = [ROOT / "include" / "beatlm_hip.h", ROOT / "include" / "beatlm_ir.h", ROOT / "include" / "beatlm_schedule.h",
           ROOT / "include" / "beatlm_load.h"]


def declared_functions(path):
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(bl[isf]?_[a-z0-9_]+)\s*\(", text)) - {"bl_timer_stats_t"})


def test_the_library_exports_every_declared_function():
    lib = hip.lib()
    names = [n for h in HEADERS for n in declared_functions(h)]
    assert len(names) > 80 and sum(n.startswith("blf_") for n in names) == 34
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []


def test_the_abi_version():
    assert hip.lib().bl_abi_version() == 4


C_LAYOUT = r"""
#include <stddef.h>
#include <stdio.h>
#include "beatlm_ir.h"
#include "beatlm_schedule.h"
#include "beatlm_load.h"
#define P(T) printf(#T " %zu\n", sizeof(T));
#define O(T, f) printf(#T "." #f " %zu\n", offsetof(T, f));
int main(void) {
  P(bl_spec) O(bl_spec, part) O(bl_spec, n_reads) O(bl_spec, epilogue) O(bl_spec, bindings)
  P(bl_binding) P(bl_epilogue) P(bl_part) P(bl_substitution) P(bl_binding_set)
  P(bl_device_profile_t) O(bl_device_profile_t, compute_units) O(bl_device_profile_t, name)
  P(bl_frame_timing) P(bl_timer_stats_t)
  P(bli_op) P(bli_tensor_desc) P(bli_profile) P(bli_placement) P(bli_kernel_info)
  O(bli_kernel_info, output_start) O(bli_kernel_info, bindings) P(bli_vit_dims) P(bli_block_ids) P(bli_embed_ids)
  P(bls_frame) P(bls_frame_plan) O(bls_frame_plan, runs) O(bls_frame_plan, budget)
  P(blf_tensor) O(blf_tensor, shape) O(blf_tensor, bytes) P(blf_role) P(blf_spec) O(blf_spec, role)
  P(blf_dav2_config) O(blf_dav2_config, out_indices) O(blf_dav2_config, factor) O(blf_dav2_config, head_hidden_size)
  return 0;
}
"""


def test_the_host_structs_have_the_c_layout(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(C_LAYOUT)
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines())
    py = {
        "bl_spec": hip.Spec, "bl_binding": hip.Binding, "bl_epilogue": hip.Epilogue, "bl_part": hip.Part,
        "bl_substitution": hip.Substitution, "bl_binding_set": hip.BindingSet,
        "bl_device_profile_t": hip.DeviceProfile, "bl_frame_timing": hip.FrameTiming,
        "bl_timer_stats_t": hip.TimerStats, "bli_op": ir.Op, "bli_tensor_desc": ir.TensorDesc,
        "bli_profile": ir.Profile, "bli_placement": ir.Placement, "bli_kernel_info": ir.KernelInfo,
        "bli_vit_dims": ir.VitDims, "bli_block_ids": ir.BlockIds, "bli_embed_ids": ir.EmbedIds,
        "bls_frame": schedule.Frame, "bls_frame_plan": schedule._Plan,
        "blf_tensor": load._Tensor, "blf_role": load._Role, "blf_spec": load._Spec, "blf_dav2_config": load._Config,
    }
    for name, cls in py.items():
        assert int(got[name]) == C.sizeof(cls), name
    for key, value in got.items():
        if "." in key:
            struct, field = key.split(".")
            assert getattr(py[struct], field).offset == int(value), key


def test_without_a_device_a_context_is_an_error_not_a_crash():
    lib = hip.lib()
    h = C.c_void_p()
    rc = lib.bl_ctx_create(0, C.byref(h))
    if rc == hip.OK:
        lib.bl_ctx_destroy(h)
        pytest.skip("a GPU is visible")
    assert rc in (hip.ERR_HIP, hip.ERR_INVALID_ARGUMENT)
    assert lib.bl_ctx_create(-1, C.byref(h)) != hip.OK


@pytest.mark.parametrize("tokens,heads", [(1, 1), (17, 2), (257, 6), (1370, 6), (1370, 12), (1370, 16), (5477, 6),
                                          (65_536, 16), (1_000_000, 16), (3_000_000, 32)])
@pytest.mark.parametrize("dtype", [hip.F32, hip.F16])
def test_the_flash_plan_covers_every_unit_once(tokens, heads, dtype):
    """The flash kernel's (head, 256-query tile, 64-key tile) units, dealt in
    contiguous runs per XCD, are each covered by exactly one run, up to the
    longest sequences its 32-bit run arithmetic allows; beyond that the
    plan refuses the shape rather than overflow."""
    lib = hip.lib()
    units = C.c_uint64()
    rc = lib.bl_flash_plan_check(tokens, heads, 256, dtype, C.byref(units))
    want = heads * -(-tokens // 256) * -(-tokens // 64)
    if rc == hip.ERR_TOO_LARGE:
        assert want * 32 >= 2**32, (tokens, heads, want)
        return
    assert rc == hip.OK, rc
    assert units.value == want


@pytest.mark.parametrize("cus", [8, 80, 256, 304])
@pytest.mark.parametrize("tokens,heads", [(1, 1), (257, 6), (1370, 6), (1370, 16), (5477, 6), (40_000, 3)])
def test_the_in_kernel_merge_counts_every_split_tile_s_runs(cus, tokens, heads):
    """The in-kernel merge of split query tiles: the runs that split a tile,
    and only they, name it among their first and last segments (so each tile's
    arrival counter reaches exactly its run count), and their row shares cover
    the tile's rows once, on CU counts that divide the units unevenly."""
    lib = hip.lib()
    units = C.c_uint64()
    for dtype in (hip.F32, hip.F16):
        assert lib.bl_flash_plan_check(tokens, heads, cus, dtype, C.byref(units)) == hip.OK, (cus, tokens, heads, dtype)


def test_the_flash_plan_refuses_shapes_beyond_its_run_arithmetic():
    lib = hip.lib()
    units = C.c_uint64()
    assert lib.bl_flash_plan_check(2_000_000_000, 16, 256, hip.F16, C.byref(units)) == hip.ERR_TOO_LARGE
    assert lib.bl_flash_plan_check(0, 16, 256, hip.F16, C.byref(units)) == hip.ERR_INVALID_ARGUMENT
