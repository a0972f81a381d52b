"""CPU bounds check of the decode launch plans: tests/plan_check.cpp, built with g++ and the
address and undefined-behaviour sanitizers, plans every BASELINE decode shape (C1-C5 at their
configured sizes, including C5's global layers with the wide split plan and its sliding-window
ring layers) and extreme tuning settings with the runtime's own planner, then walks every
workgroup's partial-buffer, counter and tile indexing with the kernels' own index functions. It
also checks the K tile layout (k_index is a bijection, and the decode and prefill K loads address
the elements it places there, each decode operand load one contiguous 1 KB run), and that a split
prefill launch's work items cover every stripe's (or stripe pair's) kv tiles exactly once."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_decode_plans_stay_in_bounds(tmp_path):
    exe = tmp_path / "plan_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "models_amd", "csrc"),
           os.path.join(ROOT, "tests", "plan_check.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().endswith("ok"), run.stdout
    assert "C5 global d256 4/1 @32767" in run.stdout and "separate" in run.stdout
    assert "K layout: bijective" in run.stdout
    assert "split prefill items: every unit covered once" in run.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_projection_launches_stay_in_bounds(tmp_path):
    """tests/qmat_check.cpp: the quantized-projection launches of decode- and prefill-sized
    grouped calls (biases, residuals, mixed formats, the 200-row grouped shape, 2048-row prefill
    batches, 16 matrices, rows of 14336 inputs) planned with the runtime's planner, every
    workgroup's weight, activation, LDS, output and addend index walked under ASan/UBSan, every
    output written exactly once."""
    exe = tmp_path / "qmat_check"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-I", os.path.join(ROOT, "models_amd", "csrc"),
           os.path.join(ROOT, "tests", "qmat_check.cpp"), "-o", str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.strip().endswith("ok"), run.stdout
    assert "grouped 2048 rows, biases" in run.stdout and "product" in run.stdout
