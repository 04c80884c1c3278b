"""A static check of the built GEMM kernels' LDS fragment reads.

The ring GEMM (gemm_pipe_kernel) reads its fragments from LDS with inline
ds_read_b128, which the compiler does not track: it counts on every use of a
fragment register coming after the kernel's own `s_waitcnt lgkmcnt(0)`. A
compiler that copied or consumed such a register earlier would read stale
data on some shapes and not others. This test disassembles the gfx950 code
objects embedded in the built library (the repository's own build) and
checks every ring-GEMM kernel in program order: no instruction reads or
writes a register that an LDS read has not yet returned, where an
`s_waitcnt lgkmcnt(N)` returns all LDS operations but the N newest (LDS
operations complete in order; scalar loads, also counted, can only make
fewer of them complete).

The scan is linear within each kernel: an instruction after a conditional
branch inherits the state before it; one after an unconditional branch is
reached only by a jump and starts with nothing outstanding (the compiler's own
reads on paths that skip one another are not confused that way). Every ring
round ends with lgkmcnt(0) before its products, so a round's reads and their
uses lie in one straight stretch of code, which is what the scan covers.
"""

from __future__ import annotations

import os
import pathlib
import re
import struct
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
LIB = ROOT / "beatlm_amd" / "libbeatlm_hip.so"
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)\b)")
WAIT = re.compile(r"lgkmcnt\((\d+)\)")


def code_objects(lib: bytes) -> list[bytes]:
    """The gfx950 code objects of the clang offload bundles in a library."""
    out = []
    pos = 0
    while (i := lib.find(BUNDLE_MAGIC, pos)) >= 0:
        (entries,) = struct.unpack_from("<Q", lib, i + len(BUNDLE_MAGIC))
        p = i + len(BUNDLE_MAGIC) + 8
        for _ in range(entries):
            off, size, tlen = struct.unpack_from("<QQQ", lib, p)
            p += 24
            triple = lib[p:p + tlen].decode()
            p += tlen
            if "gfx950" in triple:
                out.append(lib[i + off:i + off + size])
        pos = i + len(BUNDLE_MAGIC)
    return out


def regs(text: str) -> set[tuple[str, int]]:
    found = set()
    for m in REG.finditer(text):
        kind = m.group(1)
        if m.group(4) is not None:
            found.add((kind, int(m.group(4))))
        else:
            for r in range(int(m.group(2)), int(m.group(3)) + 1):
                found.add((kind, r))
    return found


def check_kernel(name: str, lines: list[str]) -> list[str]:
    """Program-order scan of one kernel: the uses of LDS results before they
    are waited for."""
    pending: list[set] = []  # destination registers of outstanding LDS operations, oldest first
    problems = []
    for line in lines:
        text = line.split("//")[0].strip()
        if not text or text.endswith(":"):
            continue
        op, _, args = text.partition(" ")
        if op in ("s_branch", "s_endpgm"):
            pending = []
            continue
        if op == "s_waitcnt":
            m = WAIT.search(args)
            if m:
                keep = int(m.group(1))
                pending = pending[len(pending) - keep:] if keep else []
            continue
        operands = [a.strip() for a in args.split(",")] if args else []
        touched = regs(args)
        busy = set().union(*pending) if pending else set()
        hit = touched & busy
        if hit:
            problems.append(f"{name}: `{text}` touches {sorted(hit)[:4]} before its LDS read returned")
        if op.startswith("ds_"):
            # A DS operation with a result (reads, atomics with return) names
            # its destination first; stores name none.
            dest = regs(operands[0]) if operands and ("read" in op or "_rtn" in op or "bpermute" in op or "swizzle" in op) else set()
            pending.append(dest)
    return problems


@pytest.mark.skipif(not LIB.exists(), reason="the backend library is not built")
@pytest.mark.skipif(not os.path.exists(OBJDUMP), reason="ROCm's llvm-objdump is not installed")
def test_ring_gemm_fragment_registers_are_used_only_after_their_lds_reads_return(tmp_path):
    objects = [c for c in code_objects(LIB.read_bytes()) if b"gemm_pipe_kernel" in c]
    assert objects, "no code object with the ring GEMM in the library"
    procs = []
    for i, co in enumerate(objects):
        path = tmp_path / f"co{i}.o"
        path.write_bytes(co)
        procs.append(subprocess.Popen([OBJDUMP, "-d", "--mcpu=gfx950", "--no-show-raw-insn", str(path)],
                                      stdout=subprocess.PIPE, text=True))
    kernels = 0
    problems: list[str] = []
    for p in procs:
        name, body = None, []
        for line in p.stdout:
            if line.startswith("0") and line.rstrip().endswith(">:"):
                if name and "gemm_pipe_kernel" in name:
                    problems += check_kernel(name, body)
                    kernels += 1
                name, body = line.split("<", 1)[1].rstrip().rstrip(":").rstrip(">"), []
            elif name:
                body.append(line)
        if name and "gemm_pipe_kernel" in name:
            problems += check_kernel(name, body)
            kernels += 1
        assert p.wait() == 0
    assert kernels > 100, f"only {kernels} ring GEMM kernels found"
    assert not problems, f"{len(problems)} early uses, e.g.:\n" + "\n".join(problems[:10])


def test_the_scan_finds_an_early_use():
    """The checker itself: a fragment consumed before its wait is reported,
    the same code with the wait first is not, and lgkmcnt(1) retires all but
    the newest LDS read."""
    early = ["ds_read_b128 v[4:7], v1", "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]", "s_waitcnt lgkmcnt(0)"]
    assert check_kernel("k", early)
    late = ["ds_read_b128 v[4:7], v1", "s_waitcnt lgkmcnt(0)", "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]"]
    assert not check_kernel("k", late)
    partial = ["ds_read_b128 v[4:7], v1", "ds_read_b128 v[12:15], v2", "s_waitcnt lgkmcnt(1)",
               "v_add_f32_e32 v20, v4, v5"]
    assert not check_kernel("k", partial)
    partial_bad = partial[:3] + ["v_add_f32_e32 v20, v12, v5"]
    assert check_kernel("k", partial_bad)
    overwrite = ["ds_read_b128 v[4:7], v1", "v_mov_b32_e32 v5, 0", "s_waitcnt lgkmcnt(0)"]
    assert check_kernel("k", overwrite)
    jumped = ["ds_read_b64 v[4:5], v1", "s_branch 3", "v_mov_b32_e32 v5, 0"]
    assert not check_kernel("k", jumped)
