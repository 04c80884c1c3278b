"""bench.py's host-side pieces, on the CPU: the refusal of more than one GPU,
the full-size checkpoint measurement, and the decoder's FLOP accounting the
roofline uses."""

import subprocess
import sys

import pytest

import bench
from beatlm_amd import hip, ir


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True, timeout=300,
                       cwd=bench.ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_the_checkpoint_measurement_reads_the_whole_small_model():
    out = bench.checkpoint_load()
    assert out["parameters"] == 24_785_089
    assert out["file_bytes"] > 24_785_089 * 4
    assert out["read_and_parse_ms"] > 0 and out["convert_ms"] > 0


def test_convolution_flops_count_every_tap_and_channel():
    g = ir.Graph()
    g.tensor(0, ir.INPUT, 37 * 37 * 384)
    g.tensor(1, ir.WEIGHT, 9 * 384 * 384)
    g.tensor(2, ir.OUTPUT, 19 * 19 * 384)
    g.push(ir.op(ir.OP_CONV3X3, [0, 1, ir.NONE], [37, 37, 384, 384, 2]), 2)
    info = g.lower().kernel(0)
    assert info.main == hip.MAIN_CONV3X3
    assert bench.kernel_flops(info) == pytest.approx(2.0 * 19 * 19 * 9 * 384 * 384)
