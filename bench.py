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

The same line carries `frame_loop`: the high-resolution encoder (ViT-S/14 at
1036 x 1036, 5477 tokens, 12 blocks, f16) run as frame-budget slices at 60
frames per second beside a render load spinning the GPU for 8 ms a frame,
after calibration: slices per frame, the delivery latency k the calibrated
costs call for, deliveries and misses (--frame-loop-frames 0 skips it).
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
    return 0.0


def time_kernels(prep, frames: int, warmup: int = 3):
    """Median per-kernel µs over `frames` frames, from the slice timer's
    hipEvent pairs on the backend's stream."""
    n = len(prep.kernels)
    timer = hip.Timer(prep.ctx, n)
    per = [[] for _ in range(n)]
    for f in range(warmup + frames):
        timer.begin_frame(f)
        for k in range(n):
            prep.kernels.encode(k, 0, timer, k)
        r = timer.resolve()
        timer.submitted(r)
        prep.ctx.synchronize()
        for frame, slices in timer.collect():
            if frame >= warmup:
                for tag, us in slices:
                    per[tag].append(us)
    timer.close()
    return [statistics.median(p) if p else float("nan") for p in per]


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="vit-s-518", choices=sorted(CONFIGS))
    ap.add_argument("--f32-math", default="split", choices=["split", "mfma"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-frames", type=int, default=20)
    ap.add_argument("--frame-loop-frames", type=int, default=120)
    ap.add_argument("--render-us", type=int, default=8000)
    ap.add_argument("--max-dispatch-us", type=int, default=frameloop.DEFAULT_MAX_DISPATCH_US)
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (every box has one GPU); "
            "run with --gpus 1",
            file=sys.stderr,
        )
        return 2

    cfg = CONFIGS[args.config]
    dtype = hip.F16 if cfg["dtype"] == "f16" else hip.F32
    np_dtype = np.float16 if dtype == hip.F16 else np.float32
    elt = 2 if dtype == hip.F16 else 4

    ctx = hip.Context(0)
    if args.f32_math == "mfma":
        ctx.set_f32_math(hip.F32_MATH_MFMA_F32)
    g, emb, block_ids, tokens = build_encoder(cfg)
    prep = ir.prepare(ctx, g, dtype=dtype)
    vals = synthetic_values(cfg, emb, block_ids, tokens, np_dtype)
    for tid, v in vals.items():
        prep.write(tid, v)

    frames = cfg["frames"]

    def step():
        for _ in range(frames):
            prep.run()

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    allocs_before = ctx.allocations()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    assert ctx.allocations() == allocs_before, "the frame loop allocated device memory"
    out = prep.read(block_ids[-1].output)
    assert np.isfinite(out.astype(np.float32)).all(), "non-finite encoder output"

    ms_per_step = elapsed * 1e3 / args.steps
    blocks_per_step = cfg["blocks"] * frames
    us_per_block = ms_per_step * 1e3 / blocks_per_step

    # Per-kernel times from hipEvent pairs, for the roofline.
    med = time_kernels(prep, args.profile_frames)
    infos = [prep.program.kernel(k) for k in range(len(prep.program))]
    labels = [prep.kernels.label(k) for k in range(len(prep.kernels))]
    by_kind: dict[str, list[float]] = {}
    flops_kind: dict[str, float] = {}
    bytes_kind: dict[str, float] = {}
    for k, info in enumerate(infos):
        name = prep.program.name(k)
        by_kind.setdefault(name, []).append(med[k])
        flops_kind[name] = kernel_flops(info)
        bytes_kind[name] = kernel_bytes(info, elt)
    totals = {n: sum(v) for n, v in by_kind.items()}
    dominant = max(totals, key=totals.get)
    avg_us = statistics.mean(by_kind[dominant])

    math_name = "f16" if dtype == hip.F16 else ("bf16x3" if args.f32_math == "split" else "f32")
    # An f32 product on bf16 matrix cores is three bf16 MFMAs.
    mfma_peak = PEAK_TFLOPS["f16"] if dtype == hip.F16 else (
        PEAK_TFLOPS["bf16"] / 3.0 if args.f32_math == "split" else PEAK_TFLOPS["f32"]
    )

    def roof(name):
        us = statistics.mean(by_kind[name])
        if flops_kind[name] > 0:
            a = flops_kind[name] / us / 1e6
            return {"bound": "mfma", "achieved": round(a, 2), "peak": round(mfma_peak, 1), "unit": "TFLOP/s",
                    "frac": round(a / mfma_peak, 4), "traffic": None, "kernel": name, "us_per_launch": round(us, 2)}
        a = bytes_kind[name] / us / 1e3
        return {"bound": "hbm", "achieved": round(a, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(a / PEAK_HBM_GBS, 4), "traffic": None, "kernel": name, "us_per_launch": round(us, 2)}

    attn = roof("flash_attention") if "flash_attention" in by_kind else None
    result = {
        "metric": METRIC,
        "value": round(us_per_block, 2),
        "unit": "us/block",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded image U[0,1] normalised, random Xavier weights)",
        "config": {
            "workload": f"{args.config}: patch embed + {cfg['blocks']} pre-LN ViT blocks, {tokens} tokens, "
            f"width {cfg['width']}, {cfg['heads']} heads x 64, MLP {4 * cfg['width']}, "
            f"{frames} frame(s) per step, {cfg['dtype']}",
            "tokens": tokens,
            "blocks": cfg["blocks"],
            "frames": frames,
            "matrix_math": math_name,
            "kernels_per_frame": len(prep.kernels),
        },
        "roofline": roof(dominant),
        "attention": attn,
        "per_kernel_us": {n: round(statistics.mean(v), 2) for n, v in by_kind.items()},
        "kernel_sum_us_per_block": round(sum(med) / cfg["blocks"], 2),
    }
    if attn:
        result["attention_tflops"] = attn["achieved"]
        result["attention_frac_of_mfma_peak"] = attn["frac"]

    if args.frame_loop_frames > 0:
        hi = CONFIGS["vit-s-1036"]
        g5, emb5, ids5, tokens5 = build_encoder(hi)
        vals5 = synthetic_values(hi, emb5, ids5, tokens5, np.float16)
        loop = frameloop.run(ctx, g5, vals5, ids5[-1].output, hip.F16, frames=args.frame_loop_frames,
                             render_us=args.render_us, bound_us=args.max_dispatch_us)
        loop["workload"] = (f"vit-s-1036: patch embed + {hi['blocks']} pre-LN ViT blocks, {tokens5} tokens, "
                            f"width 384, 6 heads x 64, f16, as " + loop["workload"])
        result["frame_loop"] = loop

    if not args.no_cpu_baseline:
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, os.cpu_count() or 1)
        cpu_us = cpu_baseline(cfg, tokens, threads)
        result["cpu_baseline"] = {
            "value": round(cpu_us, 1),
            "unit": "us/block",
            "cores": threads,
            "kind": "port",
            "sample": f"one f32 block ({tokens} tokens) of the reference's WGSL kernels restated in C "
            "(oracle, same summation order), OpenMP over rows; 1 warm-up, median of 5",
        }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
