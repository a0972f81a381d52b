"""The library's host runtime and the benchmark's drivers on the CPU, under AddressSanitizer and
UndefinedBehaviorSanitizer, against a host-memory simulation of the HIP runtime
(tests/hostsim/hip_sim.cpp, built as libamdhip64.so.7) with launch stubs in place of the kernels
(tests/hostsim/launch_stubs.cpp). Every launch names the device ranges its kernel would touch; the
simulation checks them against the live allocations when the launch executes, which for a
captured launch is every graph replay, so a buffer freed while a graph still names it, or smaller
than a launch assumes, fails the run. The bench legs run as they do on the GPU box: C5's 26
layers with 64 per-token graphs (the leg during which one profiled run once ended in a
segmentation fault), and the default bench line with every other leg. Kernels do not run, so no
figure here means anything; the test is about host code and lifetimes."""

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _runtime(name):
    out = subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


@pytest.fixture(scope="module")
def sim(tmp_path_factory):
    if shutil.which("g++") is None or _runtime("libasan.so") is None:
        pytest.skip("needs g++ with AddressSanitizer")
    d = tmp_path_factory.mktemp("hostsim")
    flags = ["-std=c++17", "-O1", "-g", "-fPIC", "-shared", "-fno-omit-frame-pointer",
             "-I", os.path.join(ROOT, "tests", "hostsim")]
    runtime = d / "libamdhip64.so.7"
    build = subprocess.run(["g++", *flags, "-fsanitize=address",
                            os.path.join(ROOT, "tests", "hostsim", "hip_sim.cpp"),
                            "-Wl,-soname,libamdhip64.so.7", "-o", str(runtime)],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    lib = d / "libjmodels_attn_hostsim.so"
    build = subprocess.run(["g++", *flags, "-fsanitize=address,undefined",
                            "-I", os.path.join(ROOT, "include"),
                            "-I", os.path.join(ROOT, "models_amd", "csrc"),
                            os.path.join(ROOT, "models_amd", "csrc", "jma_runtime.cpp"),
                            os.path.join(ROOT, "tests", "hostsim", "launch_stubs.cpp"),
                            f"-L{d}", "-l:libamdhip64.so.7", f"-Wl,-rpath,{d}", "-o", str(lib)],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    env = dict(os.environ)
    env.update({
        "LD_LIBRARY_PATH": str(d),
        "LD_PRELOAD": " ".join(p for p in (_runtime("libasan.so"), _runtime("libubsan.so")) if p),
        "ASAN_OPTIONS": "detect_leaks=0",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "MODELS_HIP_ATTENTION_LIBRARY": str(lib),
        "PYTHONUNBUFFERED": "1",
    })
    return env


def _bench(env, *args, timeout=900):
    run = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], cwd=ROOT, env=env,
                         capture_output=True, text=True, timeout=timeout)
    out = run.stdout + run.stderr
    assert run.returncode == 0, out[-4000:]
    assert "hipsim:" in out and " 0 errors" in out, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    return run.stdout


def test_c5_leg_lifetimes(sim):
    """bench.py --c5-only: the cache filled layer by layer, 64 eager tokens, 64 per-token graphs
    (30 launches each: 22 sliding layers, 4 global layers with their reduce launch) replayed after
    warm-up, then graphs destroyed, buffers freed and the cache closed, as on the GPU box."""
    out = _bench(sim, "--c5-only")
    assert '"c5_us_per_token"' in out


def test_default_bench_line(sim):
    """The default bench line (every leg but the CPU baseline, 2 timed steps): C2, C1, C3, the
    other prefills and decode layers, C4, C5 and the projections, ending in the JSON line."""
    out = _bench(sim, "--steps", "2", "--warmup", "1", "--no-cpu", timeout=1500)
    assert '"metric"' in out and '"roofline"' in out
