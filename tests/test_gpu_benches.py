"""The benchmark harnesses that mirror the reference's (cpp_benchmarks/ and the
plugin-root scripts benchmark_scaled_mm_hip_configs.py, benchmark_scaled_mm_hip.py,
benchmark_convert.py, profile_scaled_mm_hip.py) run and report: the libtorch C++
bench with its float64 check of the output, the per-config sweep over every
compatible tuple, the square-size and cast sweeps, and the profiling workload."""

import re
import subprocess
import sys

import pytest

from conftest import REPO

pytestmark = pytest.mark.gpu
PKG = REPO / "comfyui-featherops_amd"


def _run(cmd, cwd=REPO):
    print("run", " ".join(map(str, cmd)), flush=True)
    out = subprocess.run([str(c) for c in cmd], cwd=cwd, capture_output=True, text=True, timeout=240)
    assert out.returncode == 0, out.stdout + out.stderr
    return out.stdout


@pytest.mark.parametrize("shape,cfg,out", [((512, 1024, 1024), (2, 4, 4, 8, 4), "fp16"),
                                           ((48, 3072, 2048), (1, 1, 2, 1, 2), "bf16"),
                                           ((4096, 3072, 3072), (2, 4, 4, 8, 3), "bf16")])
def test_libtorch_bench_runs_and_checks(shape, cfg, out):
    exe = PKG / "cpp_benchmarks" / "build" / "benchmark_scaled_mm_hip_libtorch"
    m, n, k = shape
    text = _run([exe, "--m", m, "--n", n, "--k", k, "--iters", 3, "--warmup", 1, "--warps_m", cfg[0], "--warps_n",
                 cfg[1], "--unroll", cfg[2], "--repeat_m", cfg[3], "--repeat_n", cfg[4], "--out", out, "--check"])
    assert "scaled_mm libtorch benchmark" in text and re.search(r"avg TFLOP/s: [0-9.]+", text)
    assert "check:" in text and " ok" in text


def test_config_sweep_script():
    text = _run([sys.executable, "benchmark_scaled_mm_hip_configs.py", "--shapes", "256,512,512;64,1024,1024",
                 "--rep", "3", "--warmup", "1"], cwd=PKG)
    lines = [ln for ln in text.splitlines() if "avg_TFLOPS=" in ln]
    assert len(lines) >= 20, text
    assert any(ln.strip().startswith("any_m pick=") for ln in lines)
    for ln in lines:
        assert float(re.search(r"avg_TFLOPS=([0-9.]+)", ln).group(1)) > 0


@pytest.mark.parametrize("args,title", [
    (["--convert", "rtz", "--n", 1024, "--rotate", 4], "bf16_to_fp16 benchmark"),
    (["--convert", "rne", "--n", 2048, "--rotate", 2], "bf16_to_fp16_rne benchmark"),
    (["--dequant", "--n", 1024, "--k", 2048, "--rotate", 2], "dequantize_e5m2 benchmark"),
    (["--quant", "--n", 1024, "--k", 2048, "--rotate", 2], "quantize_prepack_e5m2 benchmark"),
    (["--m", 16, "--n", 1024, "--k", 1024, "--rotate", 4, "--warps_m", 1, "--warps_n", 1, "--unroll", 2,
      "--repeat_m", 1, "--repeat_n", 2], "scaled_mm benchmark"),
])
def test_cpp_bench_modes(args, title):
    """The C++ bench's auxiliary modes (the casts and the dequantize, the quantize) and the GEMM's
    back-to-back and HIP-graph replay timings run and report a positive rate."""
    exe = PKG / "cpp_benchmarks" / "build" / "benchmark_scaled_mm_hip"
    text = _run([exe, *args, "--warmup", 2, "--iters", 8])
    assert title in text, text
    assert re.search(r"back-to-back (us|ms): [0-9.]*[1-9]", text), text
    if title == "scaled_mm benchmark":
        assert re.search(r"graph-replay us: [0-9.]*[1-9]", text), text


def test_hbm_copy_floor_both_launch_methods():
    exe = PKG / "cpp_benchmarks" / "build" / "benchmark_hbm_copy"
    plain = _run([exe, "--read-bytes", 4 << 20])
    graph = _run([exe, "--read-bytes", 4 << 20, "--graph"])
    assert re.search(r"us/call", plain) and "(graph replay)" in graph


def test_square_sweep_script():
    text = _run([sys.executable, "benchmark_scaled_mm_hip.py", "--sizes", "128,512", "--rep", "3", "--warmup", "1"],
                cwd=PKG)
    rows = [ln.split() for ln in text.splitlines() if re.match(r"^\s+\d+\s+[0-9.]+\s+[0-9.]+\s*$", ln)]
    assert [int(r[0]) for r in rows] == [128, 512], text
    assert all(float(v) > 0 for r in rows for v in r[1:]), text


def test_convert_sweep_script():
    text = _run([sys.executable, "benchmark_convert.py", "--sizes", "1024,2048", "--rep", "3", "--warmup", "1"],
                cwd=PKG)
    rows = [ln.split() for ln in text.splitlines() if re.match(r"^\s+\d+(\s+[0-9.]+){3}\s*$", ln)]
    assert [int(r[0]) for r in rows] == [1024, 2048], text
    assert all(float(v) > 0 for r in rows for v in r[1:]), text


def test_profile_script():
    text = _run([sys.executable, "profile_scaled_mm_hip.py", "-N", "512", "--iters", "2"], cwd=PKG)
    assert "runs kernel" in text and text.rstrip().endswith("Done"), text
    text = _run([sys.executable, "profile_scaled_mm_hip.py", "-N", "256", "--iters", "1", "--config", "2,4,4,8,4",
                 "--no-scale", "--no-bias"], cwd=PKG)
    assert text.rstrip().endswith("Done"), text
