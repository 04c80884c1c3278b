"""Benchmark of the ViT encoder hot path on one MI355X.

Workload (the headline configuration): a ViT-S/14 encoder at 518 x 518 —
patch embedding (14 x 14, stride 14) of a normalised NHWC image, class token,
position embedding, then 12 pre-norm blocks of 1370 tokens, width 384, 6 heads
of 64, MLP 1536 with GELU (erf) — f32 activations and weights, random
Xavier-uniform weights, synthetic inputs from one seed. A step is one frame:
the whole encoder once. `value` is microseconds per block: the frame's time
over its 12 blocks (the patch embedding's time is counted in, conservatively).

Prints ONE JSON line. Everything is timed with inputs resident in HBM.

  python bench.py [--steps K] [--warmup W] [--config vit-s-518|vit-s-224|vit-b-518|vit-l-518x4|vit-s-1036]
                  [--f32-math split|mfma] [--no-cpu-baseline] [--frame-loop-frames N]

For an f32 workload timed with bf16x3 math (the default), the line also
carries `f32_mfma`: the same workload with the f32 matrix cores
(v_mfma_f32_16x16x4_f32), its µs/block, per-kernel times and dominant group
against their 157.3 TFLOP/s peak (--no-f32-mfma-line skips it).

The same line carries `frame_loop`: the high-resolution encoder (ViT-S/14 at
1036 x 1036, 5477 tokens, 12 blocks, f16) run as frame-budget slices at 60
frames per second beside a render load spinning the GPU for 8 ms a frame,
after calibration: slices per frame, the delivery latency k the calibrated
costs call for, deliveries and misses (--frame-loop-frames 0 skips it).

And `depth_model`: the whole Depth Anything V2 Small (the encoder with its four
tapped feature maps and the DPT decoder) in f32 at the reference's five image
sides, ms per run beside the reference's published per-run times; at 518
pixels the encoder's and decoder's kernel times, the decoder's dominant kernel
family against the matrix cores' peak, its CPU baseline (the oracle), the f16
model's time, and a full-size checkpoint read, checked and converted on the
host (--depth-runs 0 skips it).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from beatlm_amd import frameloop, hip, ir  # noqa: E402

METRIC = "µs per ViT encoder block + attention TFLOP/s (% MFMA peak), 1 MI355X"

# MI355X published dense peaks.
PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0, "f16": 2500.0}
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    # name: tokens grid, width, heads, blocks, frames, dtype
    "vit-s-224": dict(grid=16, width=384, heads=6, blocks=1, frames=1, dtype="f32"),
    "vit-s-518": dict(grid=37, width=384, heads=6, blocks=12, frames=1, dtype="f32"),
    "vit-b-518": dict(grid=37, width=768, heads=12, blocks=12, frames=1, dtype="f16"),
    "vit-l-518x4": dict(grid=37, width=1024, heads=16, blocks=24, frames=4, dtype="f16"),
    "vit-s-1036": dict(grid=74, width=384, heads=6, blocks=12, frames=1, dtype="f16"),
}
PATCH = 14
EPS = 1e-6


def build_encoder(cfg):
    grid, width, heads, blocks = cfg["grid"], cfg["width"], cfg["heads"], cfg["blocks"]
    tokens = grid * grid + 1
    g = ir.Graph()
    emb = g.vit_embeddings(grid, PATCH, 3, width, 0)
    x = emb.output
    next_id = emb.next_id
    block_ids = []
    for b in range(blocks):
        role = ir.OUTPUT if b == blocks - 1 else ir.ACTIVATION
        ids = g.vit_block(ir.VitDims(tokens, width, heads, 4 * width, EPS), x, next_id, role)
        block_ids.append(ids)
        x, next_id = ids.output, ids.next_id
    return g, emb, block_ids, tokens


def xavier(seed, fan_in, fan_out, rng_dtype):
    rng = np.random.default_rng(seed)
    a = np.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-a, a, fan_in * fan_out).astype(rng_dtype)


def synthetic_values(cfg, emb, block_ids, tokens, np_dtype, seed=2024):
    """Image U[0,1] normalised with the checkpoint's mean/std
    (load/depth_anything_v2/reference.rs:55-62), Xavier weights, LN gamma
    1 + 0.1 N(0,1), beta 0.1 N(0,1), biases U(-0.1, 0.1), LayerScale U(0.1, 1)."""
    rng = np.random.default_rng(seed)
    width, grid = cfg["width"], cfg["grid"]
    side = grid * PATCH
    mean = np.array([0.485, 0.456, 0.406], np.float32)
    std = np.array([0.229, 0.224, 0.225], np.float32)
    image = ((rng.uniform(0, 1, (side, side, 3)).astype(np.float32) - mean) / std).ravel()
    vals = {
        emb.image: image,
        emb.patch_w: xavier(seed + 1, PATCH * PATCH * 3, width, np.float32),
        emb.patch_b: rng.uniform(-0.1, 0.1, width),
        emb.cls: rng.normal(0, 1, width),
        emb.pos: rng.normal(0, 0.02, tokens * width),
    }
    mlp = 4 * width
    for b, ids in enumerate(block_ids):
        s = seed + 100 * (b + 1)
        vals[ids.norm1_g] = 1 + 0.1 * rng.normal(0, 1, width)
        vals[ids.norm1_b] = 0.1 * rng.normal(0, 1, width)
        vals[ids.qkv_w] = xavier(s + 1, width, 3 * width, np.float32)
        vals[ids.qkv_b] = rng.uniform(-0.1, 0.1, 3 * width)
        vals[ids.proj_w] = xavier(s + 2, width, width, np.float32)
        vals[ids.proj_b] = rng.uniform(-0.1, 0.1, width)
        vals[ids.ls1] = rng.uniform(0.1, 1.0, width)
        vals[ids.norm2_g] = 1 + 0.1 * rng.normal(0, 1, width)
        vals[ids.norm2_b] = 0.1 * rng.normal(0, 1, width)
        vals[ids.fc1_w] = xavier(s + 3, width, mlp, np.float32)
        vals[ids.fc1_b] = rng.uniform(-0.1, 0.1, mlp)
        vals[ids.fc2_w] = xavier(s + 4, mlp, width, np.float32)
        vals[ids.fc2_b] = rng.uniform(-0.1, 0.1, width)
        vals[ids.ls2] = rng.uniform(0.1, 1.0, width)
    return {k: np.asarray(v, np.float32).astype(np_dtype) for k, v in vals.items()}


def kernel_flops(info) -> float:
    """Algorithmic FLOP of one launch of a spec (2 per multiply-add of its
    products; the softmax's exponentials are not counted)."""
    d = list(info.dims)
    rows = info.part.end - info.part.start
    if info.main == hip.MAIN_MATMUL:
        return 2.0 * rows * d[1] * d[2]
    if info.main == hip.MAIN_FLASH_ATTENTION:
        return 4.0 * rows * d[0] * d[1] * d[2]
    if info.main == hip.MAIN_PATCH_EMBED:
        return 2.0 * rows * d[2] * d[2] * d[3] * d[4]
    if info.main == hip.MAIN_CONV3X3:  # rows are output pixels
        return 2.0 * rows * 9 * d[2] * d[3]
    if info.main == hip.MAIN_CONV_TRANSPOSE:  # rows are output pixels, each cin products per channel
        return 2.0 * rows * d[2] * d[3]
    return 0.0


def kernel_bytes(info, elt: int) -> float:
    """Algorithmic HBM bytes of one launch: each tensor read once, the output written once."""
    d = list(info.dims)
    rows = info.part.end - info.part.start
    if info.main == hip.MAIN_LAYER_NORM:
        return float(elt * (2 * rows * d[1] + 2 * d[1]))
    if info.main == hip.MAIN_FLASH_ATTENTION:
        return float(elt * 4 * rows * d[1] * d[2])
    if info.main == hip.MAIN_MATMUL:
        return float(elt * (rows * d[1] + d[1] * d[2] + rows * d[2]))
    if info.main == hip.MAIN_CONV3X3:
        # height, width, cin, cout, stride: the image, the 3 x 3 weights and the
        # part's output pixels (rows) once each.
        return float(elt * (d[0] * d[1] * d[2] + 9 * d[2] * d[3] + rows * d[3]))
    return 0.0


def step_distribution(ctx, step, n: int) -> dict:
    """`n` more steps, each between two hipEvents recorded on the backend's
    stream (no synchronisation between steps): the median, p10 and p90 of
    the per-step times in µs."""
    import ctypes as C

    rt = C.CDLL("libamdhip64.so")
    rt.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    rt.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    rt.hipEventSynchronize.argtypes = [C.c_void_p]
    rt.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    rt.hipEventDestroy.argtypes = [C.c_void_p]
    stream = ctx._lib.bl_ctx_stream(ctx.handle)
    events = [C.c_void_p() for _ in range(n + 1)]
    for e in events:
        assert rt.hipEventCreate(C.byref(e)) == 0
    ctx.synchronize()
    assert rt.hipEventRecord(events[0], stream) == 0
    for i in range(n):
        step()
        assert rt.hipEventRecord(events[i + 1], stream) == 0
    assert rt.hipEventSynchronize(events[n]) == 0
    us = []
    for i in range(n):
        ms = C.c_float()
        assert rt.hipEventElapsedTime(C.byref(ms), events[i], events[i + 1]) == 0
        us.append(ms.value * 1e3)
    for e in events:
        rt.hipEventDestroy(e)
    us.sort()
    pick = lambda q: us[min(n - 1, int(q * n))]
    return {"n": n, "median": round(pick(0.5), 2), "p10": round(pick(0.1), 2), "p90": round(pick(0.9), 2)}


def bracketed(ctx, prep, ks, repeats):
    """Per-launch µs of each kernel in `ks` (alone, back to back), between two
    zero-length spin launches that mark the span in a counter profile."""
    ctx.synchronize()
    ctx.spin(0)
    us = [prep.kernels.time(k, repeats) for k in ks]
    ctx.spin(0)
    ctx.synchronize()
    return us


TRAFFIC_DIR = os.path.join(ROOT, "profiles")


def traffic_file(config: str, math_name: str) -> str:
    return os.path.join(TRAFFIC_DIR, f"hbm_traffic_{config}_{math_name}.txt")


def read_traffic(config: str, math_name: str) -> dict:
    """Bytes per launch measured by the counter profile of this workload:
    {(tag, group): bytes}, from its `traffic` lines; empty when there is none."""
    out = {}
    try:
        with open(traffic_file(config, math_name)) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 4 and parts[0] == "traffic":
                    out[(parts[1], parts[2])] = float(parts[3])
    except FileNotFoundError:
        pass
    return out


def pmc_summary(directory: str) -> str:
    """The counter summary of a profile directory holding four rocprofv3 --pmc
    runs (pmc_FETCH_SIZE, pmc_WRITE_SIZE of this bench; copy_FETCH_SIZE,
    copy_WRITE_SIZE of a 256 MiB device copy) and the bench's JSON line in
    pmc_FETCH_SIZE.log (and pmc_WRITE_SIZE.log, when present, for that
    pass's brackets). Each counter is scaled by what it reads for the copy
    (bytes moved / counter KiB). The dispatches between the bench's marker
    launches (spin_kernel) are the bracketed group's: (repeats + 1) launches of
    each of its kernels, and any set-up launches the first of them needs (a
    flash kernel whose projections store the queries alone runs them again,
    with their LayerNorm statistics, when another block's operands are in the
    scratch): kernels launched a number of times that is not a multiple of
    repeats + 1 are those, listed but not counted."""
    import csv

    def rows(name):
        with open(os.path.join(directory, name, "run_counter_collection.csv")) as f:
            return sorted(csv.DictReader(f), key=lambda r: int(r["Dispatch_Id"]))

    copy_bytes = 256 << 20
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        vals = [float(r["Counter_Value"]) for r in rows(f"copy_{c}") if "copyBuffer" in r["Kernel_Name"]]
        vals.sort()
        scale[c] = copy_bytes / (vals[len(vals) // 2] * 1024.0)
    def brackets(c):
        # Each pass's own bench line: the groups it bracketed (the dominant
        # group is chosen per run) in the order of its marker launches.
        name = f"pmc_{c}.log"
        if c == "WRITE_SIZE" and not os.path.exists(os.path.join(directory, name)):
            name = "pmc_FETCH_SIZE.log"
        with open(os.path.join(directory, name)) as f:
            line = next(l for l in f if l.startswith("{") and '"metric"' in l)
        return json.loads(line)["brackets"]

    out = [f"# counter scale from a {copy_bytes >> 20} MiB copy: FETCH_SIZE x{scale['FETCH_SIZE']:.4f}, "
           f"WRITE_SIZE x{scale['WRITE_SIZE']:.4f} (bytes per counter KiB / 1024)"]
    per = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        bench = {"brackets": brackets(c)}
        rs = rows(f"pmc_{c}")
        marks = [i for i, r in enumerate(rs) if "spin_kernel" in r["Kernel_Name"]]
        spans = [rs[marks[2 * j] + 1: marks[2 * j + 1]] for j in range(len(marks) // 2)]
        for b, span in zip(bench["brackets"], spans):
            by_kernel = {}
            for r in span:
                by_kernel.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
            own = {n for n, v in by_kernel.items() if len(v) % (b["repeats"] + 1) == 0}
            if sum(len(by_kernel[n]) for n in own) != (b["repeats"] + 1) * b["kernels"]:
                own = set(by_kernel)
            kib = sum(sum(by_kernel[n]) for n in own)
            per.setdefault((b["tag"], b["group"]), {})[c] = (kib, len(span), b)
            for name, v in by_kernel.items():
                short = name.split("(bl::")[0].replace("void bl::(anonymous namespace)::", "")
                out.append(f"# {b['tag']:10s} {c:10s} {short:48s} dispatches {len(v):4d}  "
                           f"mean {sum(v) / len(v):12.1f} KiB" + ("" if name in own else "  (set-up, not counted)"))
    for (tag, group), cs in per.items():
        if len(cs) < 2:
            continue  # bracketed in one pass only
        b = cs["FETCH_SIZE"][2]
        launches = (b["repeats"] + 1) * b["kernels"]
        fetch = cs["FETCH_SIZE"][0] * 1024 * scale["FETCH_SIZE"] / launches
        write = cs["WRITE_SIZE"][0] * 1024 * scale["WRITE_SIZE"] / launches
        out.append(f"# {tag} {group}: per launch {fetch / 1e6:.3f} MB fetched + {write / 1e6:.3f} MB written")
        out.append(f"traffic {tag} {group} {fetch + write:.0f}")
    return "\n".join(out) + "\n"


def copy_calibration(copies: int = 4, nbytes: int = 256 << 20) -> None:
    """Device-to-device copies of `nbytes` (the runtime's copy kernel), the
    known traffic the HBM counters of a profile are scaled by."""
    import ctypes as C

    rt = C.CDLL("libamdhip64.so")
    rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    rt.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
    rt.hipFree.argtypes = [C.c_void_p]
    src, dst = C.c_void_p(), C.c_void_p()
    assert rt.hipMalloc(C.byref(src), nbytes) == 0 and rt.hipMalloc(C.byref(dst), nbytes) == 0
    assert rt.hipMemset(src, 1, nbytes) == 0
    for _ in range(copies):
        assert rt.hipMemcpy(dst, src, nbytes, 3) == 0  # hipMemcpyDeviceToDevice
    assert rt.hipDeviceSynchronize() == 0
    rt.hipFree(src)
    rt.hipFree(dst)


def trace_summary(directory: str) -> str:
    """The per-kernel statistics of a rocprofv3 --kernel-trace --stats run
    (its run_kernel_stats.csv): calls, mean, min and max duration per
    dispatch and share of the total, longest first."""
    import csv
    import glob

    files = glob.glob(os.path.join(directory, "**", "*kernel_stats.csv"), recursive=True)
    out = [f"{'kernel':100s} {'calls':>6s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s} {'pct':>6s}"]
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r["Name"].replace("void bl::(anonymous namespace)::", "")
                out.append(f"{name[:100]:100s} {r['Calls']:>6s} {float(r['AverageNs']) / 1e3:8.2f} "
                           f"{float(r['MinNs']) / 1e3:8.2f} {float(r['MaxNs']) / 1e3:8.2f} {float(r['Percentage']):6.2f}")
    return "\n".join(out) + "\n"


def _counter_rows(path: str):
    """(dispatch key, kernel name, counter, value, start ns, end ns) of a
    rocprofv3 --pmc run: its run_counter_collection.csv (csv output) or its
    run_results.db (the default rocpd database)."""
    import csv
    import glob
    import sqlite3

    for f in sorted(glob.glob(os.path.join(path, "**", "run_counter_collection.csv"), recursive=True)):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                yield ((f, int(r["Dispatch_Id"])), r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"]),
                       int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
    for f in sorted(glob.glob(os.path.join(path, "**", "*.db"), recursive=True)):
        db = sqlite3.connect(f)
        q = "select dispatch_id, kernel_name, counter_name, value, start, end from counters_collection"
        for d, name, c, v, t0, t1 in db.execute(q):
            yield (f, d), name, c, float(v), int(t0), int(t1)
        db.close()


def pmc_kernels(directories: list[str]) -> str:
    """Per-kernel counter summary of rocprofv3 --pmc runs of this bench (one
    directory per pass): for every kernel (by name and template arguments),
    its dispatches, mean duration, and each counter's mean per dispatch.
    MfmaUtil is rocprofv3's derived metric (MFMA busy cycles over GPU-active
    cycles of all SIMDs, %); MfmaFlops* its MOPS counters x 512, from which
    the matrix cores' rate follows; TA busy is TA_BUSY_avr over the GPU-active
    cycles of one XCD (GRBM_GUI_ACTIVE sums the 8)."""
    import re

    per: dict[str, dict] = {}
    for d in directories:
        for key, name, c, v, t0, t1 in _counter_rows(d):
            name = re.sub(r"^void ", "", name)
            name = re.sub(r"bl::\(anonymous namespace\)::", "", name)
            name = re.sub(r"\(bl::\w+\)$", "", name).replace("(bl::Math)", "M")
            k = per.setdefault(name, {"ns": {}, "counters": {}})
            k["ns"][key] = t1 - t0
            k["counters"].setdefault(c, []).append(v)
    lines = [f"{'kernel':64s} {'disp':>5s} {'us':>8s} {'MfmaUtil%':>9s} {'MFMA TFLOP/s':>12s} {'of 2.5P':>7s} {'TA busy':>7s}"]
    for name, k in sorted(per.items(), key=lambda kv: -sum(kv[1]["ns"].values())):
        ns = list(k["ns"].values())
        us = sum(ns) / len(ns) / 1e3
        cs = {c: sum(v) / len(v) for c, v in k["counters"].items()}
        # The derived metrics, or the same from the raw counters (MOPS x 512
        # flop; busy cycles over the GPU-active cycles of one XCD, which
        # GRBM_GUI_ACTIVE sums over the 8, times the 1024 SIMDs).
        flops = cs.get("MfmaFlopsBF16", 512.0 * cs.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)) + \
            cs.get("MfmaFlopsF16", 512.0 * cs.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0))
        tf = flops / us / 1e6
        ta = cs["TA_BUSY_avr"] / (cs["GRBM_GUI_ACTIVE"] / 8) if "TA_BUSY_avr" in cs and cs.get("GRBM_GUI_ACTIVE") else None
        util = cs.get("MfmaUtil")
        if util is None and "SQ_VALU_MFMA_BUSY_CYCLES" in cs and cs.get("GRBM_GUI_ACTIVE"):
            util = 100.0 * cs["SQ_VALU_MFMA_BUSY_CYCLES"] / (cs["GRBM_GUI_ACTIVE"] / 8 * 1024)
        lines.append(f"{name[:64]:64s} {len(ns):5d} {us:8.2f} " + (f"{util:9.2f} " if util is not None else f"{'':9s} ") +
                     (f"{tf:12.1f} {tf / PEAK_TFLOPS['bf16']:7.1%} " if flops else f"{'':12s} {'':7s} ") +
                     (f"{ta:7.1%}" if ta is not None else ""))
    return "\n".join(lines) + "\n"


def counter_table(directories: list[str]) -> str:
    """Every counter of rocprofv3 --pmc runs (one directory per pass), mean
    per dispatch, per kernel and grid size, with the shares the issue and wait
    counters give: SQ_WAIT_INST_ANY, SQ_WAIT_ANY and SQ_ACTIVE_INST_ANY over
    SQ_WAVE_CYCLES; SQ_VALU_MFMA_COEXEC_CYCLES over SQ_VALU_MFMA_BUSY_CYCLES."""
    import re

    per: dict[str, dict[str, list[float]]] = {}
    for d in directories:
        for key, name, c, v, t0, t1 in _counter_rows(d):
            name = re.sub(r"^void ", "", name)
            name = re.sub(r"bl::\(anonymous namespace\)::", "", name)
            name = re.sub(r"\(bl::\w+\)$", "", name).replace("(bl::Math)", "M")
            per.setdefault(name, {}).setdefault(c, []).append(v)
    lines = []
    for name, cs in per.items():
        if not any(k.startswith("SQ_") for k in cs):
            continue
        m = {c: sum(v) / len(v) for c, v in cs.items()}
        lines.append(name)
        for c in sorted(m):
            lines.append(f"    {c:32s} {m[c]:16.0f}")
        wc = m.get("SQ_WAVE_CYCLES")
        for c in ("SQ_WAIT_INST_ANY", "SQ_WAIT_ANY", "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
            if wc and c in m:
                lines.append(f"    {c + ' / SQ_WAVE_CYCLES':48s} {m[c] / wc:8.1%}")
        if m.get("SQ_VALU_MFMA_BUSY_CYCLES") and "SQ_VALU_MFMA_COEXEC_CYCLES" in m:
            lines.append(f"    {'COEXEC / MFMA_BUSY':48s} {m['SQ_VALU_MFMA_COEXEC_CYCLES'] / m['SQ_VALU_MFMA_BUSY_CYCLES']:8.1%}")
    return "\n".join(lines) + "\n"


def attention_only(ctx, cases: list[str], repeats: int) -> list[dict]:
    """The flash attention spec alone (T, H, f32 or f16 per case, d = 64,
    uniform qkv in [-1, 1]): per-launch time over `repeats` back-to-back
    launches and the rate of its 4 T^2 H d flop."""
    out = []
    for case in cases:
        t, h, dt = case.split(",")
        t, h = int(t), int(h)
        dtype = hip.F16 if dt == "f16" else hip.F32
        g = ir.Graph()
        g.tensor(0, ir.INPUT, t * 3 * h * 64)
        g.tensor(1, ir.ACTIVATION, t * h * t)
        g.push(ir.op(ir.OP_ATTENTION_SCORES, [0], [t, h, 64]), 1)
        g.tensor(2, ir.ACTIVATION, t * h * t)
        g.push(ir.op(ir.OP_SCALE, [1], [t * h * t], 0.125), 2)
        g.tensor(3, ir.ACTIVATION, t * h * t)
        g.push(ir.op(ir.OP_SOFTMAX, [2], [t * h, t]), 3)
        g.tensor(4, ir.OUTPUT, t * h * 64)
        g.push(ir.op(ir.OP_ATTENTION_VALUES, [3, 0], [t, h, 64]), 4)
        prep = ir.prepare(ctx, g, dtype=dtype)
        rng = np.random.default_rng(1)
        prep.write(0, rng.uniform(-1, 1, t * 3 * h * 64).astype(np.float16 if dtype == hip.F16 else np.float32))
        prep.kernels.time(0, repeats)  # clocks up
        us = prep.kernels.time(0, repeats)
        fl = 4.0 * t * t * h * 64
        out.append({"tokens": t, "heads": h, "dtype": dt, "kernel": prep.kernels.label(0), "us_per_launch": round(us, 2),
                    "TFLOP/s": round(fl / us / 1e6, 1)})
        prep.close()
    return out


def layernorm_hbm(ctx, rows: int, width: int, repeats: int = 20) -> dict:
    """One LayerNorm of `rows` x `width` f32 rows, larger than the caches, timed
    alone: algorithmic bytes (read x, write y, read gamma and beta) over the
    median launch time, against the HBM peak."""
    g = ir.Graph()
    g.tensor(1, ir.WEIGHT, rows * width)
    g.tensor(2, ir.WEIGHT, width)
    g.tensor(3, ir.WEIGHT, width)
    g.tensor(4, ir.OUTPUT, rows * width)
    g.push(ir.op(ir.OP_LAYER_NORM, [1, 2, 3], [rows, width], EPS), 4)
    prep = ir.prepare(ctx, g, flash=False)
    rng = np.random.default_rng(11)
    prep.write(1, rng.standard_normal(rows * width, dtype=np.float32))
    prep.write(2, 1 + 0.1 * rng.standard_normal(width, dtype=np.float32))
    prep.write(3, 0.1 * rng.standard_normal(width, dtype=np.float32))
    us = bracketed(ctx, prep, [0], repeats)[0]
    prep.close()
    nbytes = 4.0 * (2 * rows * width + 2 * width)
    gbs = nbytes / us / 1e3
    return {"rows": rows, "width": width, "dtype": "f32", "algorithmic_bytes_per_launch": int(nbytes),
            "us_per_launch": round(us, 2), "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4)}


# Whole Depth Anything V2 Small per run on an M1 Pro (Metal, f32), the
# reference's published figures (crates/beatlm-bench/src/main.rs:383-389).
DEPTH_SIDES_MS = {518: 202.3, 434: 137.8, 350: 85.6, 266: 53.2, 182: 35.0}


def depth_decoder_cpu(threads: int) -> dict:
    """The decoder of Depth Anything V2 Small at 518 pixels composed from the
    oracle's restatement of the reference's CPU ops (f64 accumulation, OpenMP
    over output pixels) on the host cores: 1 warm-up, median of 3."""
    import oracle

    cfg = ir.DepthConfig.small()
    side, grid = 518, 37
    g = ir.Graph()
    for i in range(4):
        g.tensor(i, ir.INPUT, grid * grid * cfg.hidden_size)
    _, weights, _ = ir.depth_decoder(g, cfg, side, [0, 1, 2, 3], 10)
    rng = np.random.default_rng(9)
    named = {name: (rng.uniform(-0.1, 0.1, n) if name.endswith(".bias") else
                    rng.uniform(-1, 1, n) / np.sqrt(cfg.fan_in(name))).astype(np.float32) for _, name, n in weights}
    features = [rng.standard_normal(grid * grid * cfg.hidden_size).astype(np.float32) for _ in range(4)]
    oracle.depth_decoder(cfg, side, features, named)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.depth_decoder(cfg, side, features, named)
        times.append(time.perf_counter() - t0)
    return {"value": round(statistics.median(times) * 1e3, 1), "unit": "ms/run (decoder)", "cores": threads,
            "kind": "port", "sample": "the DPT decoder at 518 pixels (37 x 37 features of 4 taps) in the reference's "
            "CPU ops restated in C (oracle, f64 accumulation), OpenMP; 1 warm-up, median of 3"}


def checkpoint_load() -> dict:
    """Reading a Depth Anything V2 Small checkpoint (24 785 089 f32
    parameters, 99 MB, random numbers under the checkpoint's names and
    shapes, written to a temporary file): ms to read and parse it, to check
    it against the inventory, and to convert every weight of the 518-pixel
    model (transposes, Q/K/V side by side, the position embedding through the
    bicubic resampling)."""
    import tempfile

    import safetensors.numpy as stn

    from beatlm_amd import load

    cfg = ir.DepthConfig.small()
    inv = load.inventory(cfg)
    rng = np.random.default_rng(3)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "dav2-small.safetensors")
        stn.save_file({sp.name: rng.standard_normal(sp.shape, dtype=np.float32) for sp in inv}, path)
        size = os.path.getsize(path)
        t0 = time.perf_counter()
        archive = load.Archive.open(path)
        t1 = time.perf_counter()
        report = inv.check(archive)
        t2 = time.perf_counter()
        g = ir.Graph()
        m = ir.depth_model(g, cfg, 518)
        weights = load.depth_weights(archive, cfg, m, 518, check=False)
        t3 = time.perf_counter()
    assert report.is_exact() and len(weights) > 0
    return {"file_bytes": size, "parameters": report.file_parameters, "read_and_parse_ms": round((t1 - t0) * 1e3, 1),
            "check_ms": round((t2 - t1) * 1e3, 2), "convert_ms": round((t3 - t2) * 1e3, 1),
            "workload": "a DAv2-Small checkpoint file read, checked against the inventory and converted for the "
                        "518-pixel graph on the host (one thread)"}


def depth_model_f16_ms(ctx, runs: int, side: int = 518) -> float:
    """ms per run of the whole model in f16 storage (f32 accumulation) at
    `side` pixels, random weights of the checkpoint's shapes."""
    cfg = ir.DepthConfig.small()
    g = ir.Graph()
    m = ir.depth_model(g, cfg, side)
    grid = side // PATCH
    vals = synthetic_values(dict(CONFIGS["vit-s-518"], grid=grid), m.encoder.embed, m.encoder.blocks, grid * grid + 1,
                            np.float16, seed=5000 + side)
    rng = np.random.default_rng(side + 1)
    vals[m.encoder.final_g] = (1 + 0.1 * rng.normal(0, 1, cfg.hidden_size)).astype(np.float16)
    vals[m.encoder.final_b] = (0.1 * rng.normal(0, 1, cfg.hidden_size)).astype(np.float16)
    for tid, name, n in m.decoder_weights:
        bound = 0.1 if name.endswith(".bias") else 1.0 / np.sqrt(cfg.fan_in(name))
        vals[tid] = rng.uniform(-bound, bound, n).astype(np.float16)
    prep = ir.prepare(ctx, g, dtype=hip.F16)
    for tid, v in vals.items():
        prep.write(tid, v)
    prep.run()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(runs):
        prep.run()
    ctx.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / runs
    d = prep.read(m.depth).astype(np.float32)
    prep.close()
    assert np.isfinite(d).all(), "non-finite f16 depth"
    return round(ms, 3)


def depth_model_runs(ctx, runs: int, repeats: int, dtype: int = hip.F32, brackets: list | None = None) -> dict:
    """The whole model (12-layer encoder, four tapped feature maps, DPT
    decoder) at each of the reference's five image sides: ms per run over
    `runs` back-to-back runs, and at 518 pixels the summed per-launch time of
    the encoder's and the decoder's kernels and the decoder's kernels by name.
    The decoder's dominant family is re-timed between marker launches (as the
    encoder's groups are, appended to `brackets`) for its HBM traffic, read
    from the committed counter profile of the model."""
    cfg = ir.DepthConfig.small()
    np_dtype = np.float16 if dtype == hip.F16 else np.float32
    out = {"workload": "Depth Anything V2 Small (ViT-S/14 encoder, taps 3/6/9/12, DPT decoder 48/96/192/384 -> "
                       f"64 -> 32 -> 1), {'f16' if dtype == hip.F16 else 'f32'}, random weights, synthetic image",
           "ms_per_run": {}, "reference_m1_pro_ms": {}}
    for side in DEPTH_SIDES_MS:
        grid = side // PATCH
        g = ir.Graph()
        enc = ir.vit_encoder(g, grid, PATCH, 3, cfg.hidden_size, cfg.num_heads, cfg.hidden_size * cfg.mlp_ratio,
                             cfg.eps, cfg.out_indices, 0, ir.ACTIVATION)
        encoder_ops = g.ops()
        depth, weights, _ = ir.depth_decoder(g, cfg, side, enc.features, enc.next_id)
        enc_cfg = dict(CONFIGS["vit-s-518"], grid=grid)
        vals = synthetic_values(enc_cfg, enc.embed, enc.blocks, grid * grid + 1, np_dtype, seed=3000 + side)
        rng = np.random.default_rng(side)
        vals[enc.final_g] = (1 + 0.1 * rng.normal(0, 1, cfg.hidden_size)).astype(np_dtype)
        vals[enc.final_b] = (0.1 * rng.normal(0, 1, cfg.hidden_size)).astype(np_dtype)
        for tid, name, n in weights:
            bound = 0.1 if name.endswith(".bias") else 1.0 / np.sqrt(cfg.fan_in(name))
            vals[tid] = rng.uniform(-bound, bound, n).astype(np_dtype)
        prep = ir.prepare(ctx, g, dtype=dtype)
        for tid, v in vals.items():
            prep.write(tid, v)
        prep.run()
        ctx.synchronize()
        allocs = ctx.allocations()
        t0 = time.perf_counter()
        for _ in range(runs):
            prep.run()
        ctx.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / runs
        assert ctx.allocations() == allocs, "the model's runs allocated device memory"
        d = prep.read(depth).astype(np.float32)
        assert d.size == side * side and np.isfinite(d).all(), "non-finite depth"
        out["ms_per_run"][str(side)] = round(ms, 3)
        out["reference_m1_pro_ms"][str(side)] = DEPTH_SIDES_MS[side]
        if side == 518:
            n = len(prep.kernels)
            us = [prep.kernels.time(k, repeats) for k in range(n)]
            dec = [k for k in range(n) if prep.program.kernel(k).first_op >= encoder_ops]
            by_name: dict[str, float] = {}
            for k in dec:
                by_name[prep.program.name(k)] = by_name.get(prep.program.name(k), 0.0) + us[k]
            out["kernels_at_518"] = len(prep.kernels)
            out["encoder_kernel_ms_at_518"] = round(sum(us[k] for k in range(n) if k not in dec) / 1e3, 3)
            out["decoder_kernel_ms_at_518"] = round(sum(us[k] for k in dec) / 1e3, 3)
            out["decoder_us_by_kernel_at_518"] = {k: round(v, 1) for k, v in sorted(by_name.items(), key=lambda x: -x[1])}
            out["plan_bytes_at_518"] = prep.plan.total_bytes()
            # The decoder's dominant kernel family (by main op; the 3 x 3
            # convolutions): their algorithmic flop over their summed
            # per-launch time against the matrix cores' peak.
            fam: dict[int, list[int]] = {}
            for k in dec:
                fam.setdefault(prep.program.kernel(k).main, []).append(k)
            main = max(fam, key=lambda f: sum(us[k] for k in fam[f]))
            group = {hip.MAIN_CONV3X3: "conv2d3x3"}.get(main, f"main{main}")
            t = sum(bracketed(ctx, prep, fam[main], repeats))
            if brackets is not None:
                brackets.append({"tag": "decoder", "group": group, "kernels": len(fam[main]), "repeats": repeats})
            flops = sum(kernel_flops(prep.program.kernel(k)) for k in fam[main])
            nbytes = sum(kernel_bytes(prep.program.kernel(k), 2 if dtype == hip.F16 else 4) for k in fam[main])
            peak = PEAK_TFLOPS["f16"] if dtype == hip.F16 else PEAK_TFLOPS["bf16"] / 3.0
            a = flops / t / 1e6
            math_name = "f16" if dtype == hip.F16 else "bf16x3"
            hbm = read_traffic("depth-anything-v2-small", math_name).get(("decoder", group))
            out["decoder_roofline"] = {
                "kernel": {hip.MAIN_CONV3X3: "conv2d3x3 (all fusions)"}.get(main, str(main)), "launches": len(fam[main]),
                "bound": "mfma", "achieved": round(a, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
                "frac": round(a / peak, 4), "us": round(t, 1), "algorithmic_flop": int(flops),
                "algorithmic_bytes_per_launch": int(nbytes / len(fam[main])),
                "traffic": int(hbm) if hbm is not None else None,
                "traffic_unit": "HBM bytes per launch (mean over the family's launches)"}
        prep.close()
    return out


def cpu_baseline(cfg, tokens, threads):
    """The reference's WGSL kernels' arithmetic (oracle, f32, same summation
    order) for ONE block of this workload on the host cores: 1 warm-up, median
    of 5."""
    import oracle

    width, heads = cfg["width"], cfg["heads"]
    mlp = 4 * width
    rng = np.random.default_rng(7)
    w = {
        "norm1_g": 1 + 0.1 * rng.normal(0, 1, width), "norm1_b": 0.1 * rng.normal(0, 1, width),
        "qkv_w": xavier(1, width, 3 * width, np.float32), "qkv_b": rng.uniform(-0.1, 0.1, 3 * width),
        "proj_w": xavier(2, width, width, np.float32), "proj_b": rng.uniform(-0.1, 0.1, width),
        "ls1": rng.uniform(0.1, 1, width), "norm2_g": 1 + 0.1 * rng.normal(0, 1, width),
        "norm2_b": 0.1 * rng.normal(0, 1, width), "fc1_w": xavier(3, width, mlp, np.float32),
        "fc1_b": rng.uniform(-0.1, 0.1, mlp), "fc2_w": xavier(4, mlp, width, np.float32),
        "fc2_b": rng.uniform(-0.1, 0.1, width), "ls2": rng.uniform(0.1, 1, width),
    }
    block = oracle.WgBlock(w, tokens, heads, width // heads, mlp, EPS, threads)
    x = rng.normal(0, 1, tokens * width).astype(np.float32)
    block(x)
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        block(x)
        times.append(time.perf_counter() - t0)
    return statistics.median(times) * 1e6


def oracle_encoder_output(cfg, emb, block_ids, tokens, vals, frames_input=None):
    """The oracle's encoder (patch embedding, class token and positions, the
    blocks) over the values the GPU was given, f32 (f16 values widened)."""
    import oracle

    f = {k: np.asarray(v, np.float32) for k, v in vals.items()}
    if frames_input is not None:
        f[emb.image] = np.asarray(frames_input, np.float32)
    grid, width, heads = cfg["grid"], cfg["width"], cfg["heads"]
    x = oracle.patch_embed(f[emb.image], f[emb.patch_w], f[emb.patch_b], grid, grid, PATCH, 3, width)
    x = oracle.add(oracle.prepend_token(f[emb.cls], x, grid * grid, width), f[emb.pos])
    for ids in block_ids:
        w = {name: f[getattr(ids, name)] for name in ir.BLOCK_WEIGHTS}
        x = oracle.vit_block(x, w, tokens, heads, width // heads, 4 * width, EPS, attention_rounded=cfg["dtype"] == "f32")
    return x


def frame_image(cfg, frame: int, np_dtype):
    """Frame `frame`'s image: U[0,1] normalised, its own seed per frame."""
    side = cfg["grid"] * PATCH
    rng = np.random.default_rng(700 + frame)
    mean = np.array([0.485, 0.456, 0.406], np.float32)
    std = np.array([0.229, 0.224, 0.225], np.float32)
    return (((rng.uniform(0, 1, (side, side, 3)).astype(np.float32) - mean) / std).ravel()).astype(np_dtype)


def measure_encoder(ctx, name: str, steps: int, warmup: int, repeats: int, f32_math: str, check: bool):
    """One encoder workload: `frames` frames a step, each through its own job
    slot (one binding set per frame, as the reference's Net slots), timed over
    `steps` steps after `warmup`; per-launch kernel times; the attention group
    against the matrix cores' peak; the output against the oracle."""
    cfg = CONFIGS[name]
    dtype = hip.F16 if cfg["dtype"] == "f16" else hip.F32
    np_dtype = np.float16 if dtype == hip.F16 else np.float32
    elt = 2 if dtype == hip.F16 else 4
    frames = cfg["frames"]
    g, emb, block_ids, tokens = build_encoder(cfg)
    allocs0, bytes0 = ctx.allocations(), ctx.device_bytes()
    prep = ir.prepare(ctx, g, dtype=dtype, slots=frames)
    device_memory = {
        "allocations": ctx.allocations() - allocs0, "bytes": ctx.device_bytes() - bytes0,
        "arena_bytes": prep.plan.total_bytes(), "workspace_bytes": prep.kernels.workspace_bytes(),
    }
    vals = synthetic_values(cfg, emb, block_ids, tokens, np_dtype)
    for tid, v in vals.items():
        prep.write(tid, v)
    if frames > 1:
        for f in range(frames):
            prep.write(emb.image, frame_image(cfg, f, np_dtype), slot=f)

    def step():
        for f in range(frames):
            prep.run(f)

    for _ in range(warmup):
        step()
    ctx.synchronize()
    allocs_before = ctx.allocations()
    packs_before = prep.kernels.packs_made()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    assert ctx.allocations() == allocs_before, "the frame loop allocated device memory"
    assert prep.kernels.packs_made() == packs_before, "the frame loop repacked weights"
    outs = [prep.read(block_ids[-1].output, slot=f).astype(np.float32) for f in range(frames)]
    assert all(np.isfinite(o).all() for o in outs), "non-finite encoder output"

    ms_per_step = elapsed * 1e3 / steps
    us_per_block = ms_per_step * 1e3 / (cfg["blocks"] * frames)
    # The spread over single steps (after the timed region, which stays the
    # K steps between synchronisations).
    spread = step_distribution(ctx, step, max(steps, 100) if frames == 1 else steps)
    n_kernels = len(prep.kernels)
    # GPU launches per frame: the kernel nodes of the graph a frame replays
    # (none when graphs are off, e.g. under a profiler).
    try:
        launches = prep.kernels.range_launches(0, n_kernels, 0)
    except Exception:
        launches = None
    per_launch = [prep.kernels.time(k, repeats) for k in range(n_kernels)]
    infos = [prep.program.kernel(k) for k in range(n_kernels)]
    groups: dict[str, list[int]] = {}
    for k in range(n_kernels):
        groups.setdefault(prep.program.name(k), []).append(k)
    math_name = "f16" if dtype == hip.F16 else ("bf16x3" if f32_math == "split" else "f32")
    # An f32 product on bf16 matrix cores is three bf16 MFMAs.
    mfma_peak = PEAK_TFLOPS["f16"] if dtype == hip.F16 else (
        PEAK_TFLOPS["bf16"] / 3.0 if f32_math == "split" else PEAK_TFLOPS["f32"])
    out = {
        "workload": f"{name}: patch embed + {cfg['blocks']} pre-LN ViT blocks, {tokens} tokens, width {cfg['width']}, "
                    f"{cfg['heads']} heads x 64, MLP {4 * cfg['width']}, {frames} frame(s) per step "
                    f"(one job slot each), {cfg['dtype']}",
        "tokens": tokens, "blocks": cfg["blocks"], "frames": frames, "dtype": cfg["dtype"], "matrix_math": math_name,
        "value": round(us_per_block, 2), "unit": "us/block", "ms_per_step": round(ms_per_step, 4),
        "kernels_per_frame": launches, "ir_kernels_per_frame": n_kernels, "device_memory": device_memory,
        "step_us": spread,
        "per_kernel_us": {g: round(statistics.mean(per_launch[k] for k in ks), 2) for g, ks in groups.items()},
        "kernel_sum_us_per_block": round(sum(per_launch) / cfg["blocks"], 2),
    }
    if check:
        want = oracle_encoder_output(cfg, emb, block_ids, tokens, vals)
        err = float(np.max(np.abs(outs[0].astype(np.float64) - want)))
        tol = 2e-2 if dtype == hip.F16 else 1e-4
        out["parity"] = {"max_abs_error": float(f"{err:.3e}"), "tolerance": tol, "within": err <= tol,
                         "checked": "the timed output (frame 0) against the oracle's encoder over the same values"}
    return prep, infos, groups, per_launch, mfma_peak, elt, out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="vit-s-518", choices=sorted(CONFIGS))
    ap.add_argument("--f32-math", default="split", choices=["split", "mfma"])
    ap.add_argument("--no-f32-mfma-line", dest="f32_mfma_line", action="store_false",
                    help="skip timing an f32 workload on the f32 matrix cores beside its bf16x3 line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-check", action="store_true", help="skip comparing the timed output with the oracle")
    ap.add_argument("--kernel-repeats", type=int, default=20)
    ap.add_argument("--roofline-group", default=None,
                    help="bracket this kernel group as the roofline one (counter profiles, whose timings differ)")
    ap.add_argument("--pmc-summary", metavar="DIR", help="write the counter summary of a profile directory and exit")
    ap.add_argument("--pmc-kernels", metavar="DIR", nargs="+",
                    help="write the per-kernel counter summary of rocprofv3 --pmc runs and exit")
    ap.add_argument("--trace-summary", metavar="DIR", help="write the kernel statistics of a kernel trace and exit")
    ap.add_argument("--counter-table", metavar="DIR", nargs="+",
                    help="write every counter of rocprofv3 --pmc runs per kernel and exit")
    ap.add_argument("--attention-only", metavar="T,H,DTYPE", nargs="+",
                    help="time the flash attention spec alone for each case (e.g. 5477,6,f16) and exit")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run 256 MiB device copies (the traffic counters' calibration) and exit")
    ap.add_argument("--other-configs", default="vit-b-518,vit-l-518x4,vit-s-1036",
                    help="comma-separated configurations also measured into `configs` ('' for none)")
    ap.add_argument("--frame-loop-frames", type=int, default=120)
    ap.add_argument("--depth-runs", type=int, default=20, help="runs of the whole depth model per side (0 skips it)")
    ap.add_argument("--layernorm-rows", type=int, default=262144)
    ap.add_argument("--render-us", type=int, default=8000)
    ap.add_argument("--max-dispatch-us", type=int, default=frameloop.DEFAULT_MAX_DISPATCH_US)
    args = ap.parse_args()
    if args.pmc_summary:
        sys.stdout.write(pmc_summary(args.pmc_summary))
        return 0
    if args.pmc_kernels:
        sys.stdout.write(pmc_kernels(args.pmc_kernels))
        return 0
    if args.trace_summary:
        sys.stdout.write(trace_summary(args.trace_summary))
        return 0
    if args.counter_table:
        sys.stdout.write(counter_table(args.counter_table))
        return 0
    if args.copy_calibration:
        copy_calibration()
        return 0
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
            "run with --gpus 1",
            file=sys.stderr,
        )
        return 2

    ctx = hip.Context(0)
    if args.f32_math == "mfma":
        ctx.set_f32_math(hip.F32_MATH_MFMA_F32)
    if args.attention_only:
        for r in attention_only(ctx, args.attention_only, args.kernel_repeats):
            print(json.dumps(r), flush=True)
        return 0
    cfg = CONFIGS[args.config]
    prep, infos, groups, per_launch, mfma_peak, elt, main_line = measure_encoder(
        ctx, args.config, args.steps, args.warmup, args.kernel_repeats, args.f32_math,
        check=not args.no_check and args.config != "vit-l-518x4")
    totals = {g: sum(per_launch[k] for k in ks) for g, ks in groups.items()}
    dominant = args.roofline_group if args.roofline_group in totals else max(totals, key=totals.get)
    traffic = read_traffic(args.config, main_line["matrix_math"])
    brackets = []

    def roof(prep, infos, groups, mfma_peak, elt, group, tag, traffic):
        """The group's launches re-timed between two zero-length spin launches,
        which mark the span in a counter profile; achieved = algorithmic work of
        one launch of each kernel over their summed per-launch time."""
        ks = groups[group]
        us = bracketed(ctx, prep, ks, args.kernel_repeats)
        brackets.append({"tag": tag, "group": group, "kernels": len(ks), "repeats": args.kernel_repeats})
        t = sum(us)
        flops = sum(kernel_flops(infos[k]) for k in ks)
        nbytes = sum(kernel_bytes(infos[k], elt) for k in ks)
        hbm = traffic.get((tag, group))
        if hbm is None:  # the same group measured under another tag
            hbm = next((v for (_, g), v in traffic.items() if g == group), None)
        common = {"kernel": group, "launches": len(ks), "us_per_launch": round(t / len(ks), 2),
                  "algorithmic_bytes_per_launch": int(nbytes / len(ks)),
                  "traffic": int(hbm) if hbm is not None else None}
        if flops > 0:
            a = flops / t / 1e6
            return {"bound": "mfma", "achieved": round(a, 2), "peak": round(mfma_peak, 1), "unit": "TFLOP/s",
                    "frac": round(a / mfma_peak, 4), **common,
                    "algorithmic_flop_per_launch": int(flops / len(ks))}
        a = nbytes / t / 1e3
        return {"bound": "hbm", "achieved": round(a, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(a / PEAK_HBM_GBS, 4), **common}

    roofline = roof(prep, infos, groups, mfma_peak, elt, dominant, "roofline", traffic)
    attn = (roof(prep, infos, groups, mfma_peak, elt, "flash_attention", "attention", traffic)
            if "flash_attention" in groups else None)
    prep.close()
    result = {
        "metric": METRIC,
        "value": main_line["value"],
        "unit": "us/block",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_line["ms_per_step"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded image U[0,1] normalised, random Xavier weights)",
        "config": {
            "workload": main_line["workload"],
            "tokens": main_line["tokens"],
            "blocks": main_line["blocks"],
            "frames": main_line["frames"],
            "matrix_math": main_line["matrix_math"],
            "kernels_per_frame": main_line["kernels_per_frame"],
            "ir_kernels_per_frame": main_line["ir_kernels_per_frame"],
        },
        "roofline": roofline,
        "attention": attn,
        "per_kernel_us": main_line["per_kernel_us"],
        "kernel_sum_us_per_block": main_line["kernel_sum_us_per_block"],
        "device_memory": main_line["device_memory"],
        "step_us": main_line["step_us"],
    }
    if "parity" in main_line:
        result["parity"] = main_line["parity"]
    if attn:
        result["attention_tflops"] = attn["achieved"]
        result["attention_frac_of_mfma_peak"] = attn["frac"]

    # An f32 workload with bf16x3 math: the same workload on the f32 matrix
    # cores (v_mfma_f32_16x16x4_f32, 157.3 TFLOP/s dense) beside it, with its
    # own dominant group against that peak.
    if args.f32_mfma_line and cfg["dtype"] == "f32" and args.f32_math == "split":
        ctx.set_f32_math(hip.F32_MATH_MFMA_F32)
        p2, infos2, groups2, per2, peak2, elt2, line = measure_encoder(
            ctx, args.config, max(5, args.steps // 4), max(2, args.warmup // 2), args.kernel_repeats, "mfma",
            check=not args.no_check)
        totals2 = {g: sum(per2[k] for k in ks) for g, ks in groups2.items()}
        traffic2 = read_traffic(args.config, line["matrix_math"])
        dominant2 = max(totals2, key=totals2.get)
        line["roofline"] = roof(p2, infos2, groups2, peak2, elt2, dominant2, "roofline_f32", traffic2)
        if "flash_attention" in groups2:
            line["attention"] = roof(p2, infos2, groups2, peak2, elt2, "flash_attention", "attention_f32", traffic2)
        p2.close()
        ctx.set_f32_math(hip.F32_MATH_SPLIT_BF16)
        result["f32_mfma"] = line

    # The other configurations: their own µs/block, and their attention
    # against the f16 matrix cores' peak (2.5 PFLOP/s dense).
    others = [c for c in args.other_configs.split(",") if c and c != args.config]
    if others:
        result["configs"] = {}
    for name in others:
        p2, infos2, groups2, per2, peak2, elt2, line = measure_encoder(
            ctx, name, max(5, args.steps // 4), max(2, args.warmup // 2), args.kernel_repeats, args.f32_math,
            check=not args.no_check and name == "vit-b-518")
        if "flash_attention" in groups2:
            line["attention"] = roof(p2, infos2, groups2, peak2, elt2, "flash_attention", f"attention_{name}",
                                     read_traffic(name, line["matrix_math"]))
        p2.close()
        result["configs"][name] = line

    if args.layernorm_rows > 0:
        ln = layernorm_hbm(ctx, args.layernorm_rows, 384, args.kernel_repeats)
        group = f"layernorm_{args.layernorm_rows}x384"
        brackets.append({"tag": "layernorm", "group": group, "kernels": 1, "repeats": args.kernel_repeats})
        hbm = traffic.get(("layernorm", group))
        ln["traffic"] = int(hbm) if hbm is not None else None
        result["layernorm_hbm"] = ln

    if args.frame_loop_frames > 0:
        hi = CONFIGS["vit-s-1036"]
        g5, emb5, ids5, tokens5 = build_encoder(hi)
        vals5 = synthetic_values(hi, emb5, ids5, tokens5, np.float16)
        loop = frameloop.run(ctx, g5, vals5, ids5[-1].output, hip.F16, frames=args.frame_loop_frames,
                             render_us=args.render_us, bound_us=args.max_dispatch_us)
        loop["workload"] = (f"vit-s-1036: patch embed + {hi['blocks']} pre-LN ViT blocks, {tokens5} tokens, "
                            f"width 384, 6 heads x 64, f16, as " + loop["workload"])
        result["frame_loop"] = loop

    if args.depth_runs > 0:
        result["depth_model"] = depth_model_runs(ctx, args.depth_runs, args.kernel_repeats, brackets=brackets)
        result["depth_model"]["f16_ms_per_run_at_518"] = depth_model_f16_ms(ctx, args.depth_runs)
        result["depth_model"]["checkpoint_load"] = checkpoint_load()
        if not args.no_cpu_baseline:
            threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
            result["depth_model"]["cpu_baseline"] = depth_decoder_cpu(threads)

    if not args.no_cpu_baseline:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
        cpu_us = cpu_baseline(cfg, main_line["tokens"], threads)
        result["cpu_baseline"] = {
            "value": round(cpu_us, 1),
            "unit": "us/block",
            "cores": threads,
            "kind": "port",
            "sample": f"one f32 block ({main_line['tokens']} tokens) of the reference's WGSL kernels restated in C "
            "(oracle, same summation order), OpenMP over rows; 1 warm-up, median of 5",
        }
    result["brackets"] = brackets
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
