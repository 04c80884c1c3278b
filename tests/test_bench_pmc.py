"""bench.py's counter summary over synthetic rocprofv3 --pmc output: the
dispatches between two marker launches are the bracketed group's (repeats + 1
launches of each of its kernels); set-up launches in the span (kernels
launched a number of times that is not a multiple of repeats + 1, such as a
flash kernel's projections run again) are listed but not counted, and each
counter is scaled by what it reads for a 256 MiB copy."""

import csv
import json
import os

import bench

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Value"]


def write_rows(path, rows):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, FIELDS)
        w.writeheader()
        for i, (name, value) in enumerate(rows):
            w.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Value": value})


def test_the_summary_counts_the_groups_launches_and_not_set_up_launches(tmp_path):
    d = str(tmp_path)
    # The copy reads 2 x (256 MiB / 1024) "KiB" of fetches and 1 x of writes:
    # scales 0.5 and 1.0.
    kib = (256 << 20) / 1024
    write_rows(os.path.join(d, "copy_FETCH_SIZE"), [("__amd_rocclr_copyBuffer", 2 * kib)] * 3)
    write_rows(os.path.join(d, "copy_WRITE_SIZE"), [("__amd_rocclr_copyBuffer", kib)] * 3)
    repeats = 2
    attn = "void bl::(anonymous namespace)::attn_kernel<(bl::Math)1>(bl::FlashArgs)"
    qkv = "void bl::(anonymous namespace)::gemm_pipe_kernel<(bl::Math)1, 64, 64>(bl::GemmArgs)"
    spin = "bl::(anonymous namespace)::spin_kernel(unsigned long)"
    for c, per_attn, per_qkv in (("FETCH_SIZE", 1000.0, 7000.0), ("WRITE_SIZE", 300.0, 5000.0)):
        rows = [("before", 1e9), (spin, 0.0)]
        for _ in range(2):  # two kernels in the group, each preceded by a set-up projection
            rows.append((qkv, per_qkv))
            rows += [(attn, per_attn)] * (repeats + 1)
        rows += [(spin, 0.0), ("after", 1e9)]
        write_rows(os.path.join(d, f"pmc_{c}"), rows)
    line = {"metric": "m", "brackets": [{"tag": "attention", "group": "flash_attention", "kernels": 2, "repeats": repeats}]}
    with open(os.path.join(d, "pmc_FETCH_SIZE.log"), "w") as f:
        f.write("progress\n" + json.dumps(line) + "\n")
    out = bench.pmc_summary(d)
    traffic = [l for l in out.splitlines() if l.startswith("traffic ")]
    # Per launch: 1000 KiB x 1024 x 0.5 fetched + 300 KiB x 1024 x 1.0 written.
    assert traffic == [f"traffic attention flash_attention {1000 * 1024 * 0.5 + 300 * 1024:.0f}"], out
    assert "(set-up, not counted)" in out and out.count("(set-up, not counted)") == 2, out


def test_without_set_up_launches_every_dispatch_in_the_span_counts(tmp_path):
    d = str(tmp_path)
    kib = (256 << 20) / 1024
    write_rows(os.path.join(d, "copy_FETCH_SIZE"), [("__amd_rocclr_copyBuffer", kib)])
    write_rows(os.path.join(d, "copy_WRITE_SIZE"), [("__amd_rocclr_copyBuffer", kib)])
    spin = "spin_kernel"
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        # Two kernels of the group, 3 launches each (repeats 2), different names.
        write_rows(os.path.join(d, f"pmc_{c}"), [(spin, 0.0)] + [("k1", 10.0)] * 3 + [("k2", 30.0)] * 3 + [(spin, 0.0)])
    line = {"metric": "m", "brackets": [{"tag": "roofline", "group": "g", "kernels": 2, "repeats": 2}]}
    with open(os.path.join(d, "pmc_FETCH_SIZE.log"), "w") as f:
        f.write(json.dumps(line) + "\n")
    out = bench.pmc_summary(d)
    assert f"traffic roofline g {2 * (120 / 6) * 1024:.0f}" in out.splitlines(), out
    assert "not counted" not in out
