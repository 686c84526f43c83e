"""Build recipe for libfeatherops_amd.so (gfx950), the torch op library and the
C++ bench harnesses.

Plain hipcc invocations: every `csrc/*.hip` file is compiled to an object in
`_build/`, then linked into `lib/libfeatherops_amd.so` (no torch involved).
`csrc/torch_op.cpp` (host C++ only) is compiled with g++ against torch's
headers into `lib/libfeather_torch_ops.so`, which registers
torch.ops.feather_ops.scaled_mm and links the library above.
The C++ benches in `cpp_benchmarks/` link against libfeatherops_amd.so
(mirroring the reference's cpp_benchmarks/build_benchmark_scaled_mm_hip.sh,
which links the kernel's extern "C" ABI directly).

    python build.py            # library + benches
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libfeatherops_amd.so"
OPS_LIB_PATH = LIB_DIR / "libfeather_torch_ops.so"
BENCH_DIR = PKG_DIR / "cpp_benchmarks"
BENCH_BIN_DIR = BENCH_DIR / "build"

ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from forming v_pk_*_f32 instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only feature flag; drop that noise
    err = "\n".join(line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build_library(jobs: int = 8) -> Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = [BUILD_DIR / (s.stem + ".o") for s in sources]
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(sources)))) as ex:
        list(ex.map(lambda so: _run([hipcc, *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])]), zip(sources, objects)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_torch_ops() -> Path:
    """lib/libfeather_torch_ops.so from csrc/torch_op.cpp (needs libfeatherops_amd.so)."""
    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd += [f"-I{rocm}/include", f"-I{INCLUDE}", str(CSRC / "torch_op.cpp"),
            f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
            f"-L{LIB_DIR}", "-lfeatherops_amd", "-Wl,-rpath,$ORIGIN"]
    tmp = OPS_LIB_PATH.with_suffix(".so.tmp")
    _run([*cmd, "-o", str(tmp)])
    os.replace(tmp, OPS_LIB_PATH)
    return OPS_LIB_PATH


def _torch_host_flags() -> tuple[list[str], list[str]]:
    """g++ compile flags and link flags for host code against the installed torch (ROCm)."""
    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
              f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}"]
    cflags += [f"-I{p}" for p in cpp_extension.include_paths()] + [f"-I{rocm}/include", f"-I{INCLUDE}"]
    # --no-as-needed: nothing references libtorch_hip directly, but loading it registers the
    # GPU backend of the ATen ops
    lflags = [f"-L{torch_lib}", "-Wl,--no-as-needed", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch",
              "-Wl,--as-needed",
              f"-Wl,-rpath,{torch_lib}", f"-L{rocm}/lib", "-lamdhip64"]
    return cflags, lflags


def build_libtorch_bench() -> Path:
    """cpp_benchmarks/build/benchmark_scaled_mm_hip_libtorch: host C++ on ATen tensors, calling the C ABI."""
    BENCH_BIN_DIR.mkdir(exist_ok=True)
    cflags, lflags = _torch_host_flags()
    exe = BENCH_BIN_DIR / "benchmark_scaled_mm_hip_libtorch"
    _run([os.environ.get("CXX", "g++"), *cflags, str(BENCH_DIR / "benchmark_scaled_mm_hip_libtorch.cpp"), *lflags,
          f"-L{LIB_DIR}", "-lfeatherops_amd", f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)])
    return exe


def build_benches() -> list[Path]:
    hipcc = _hipcc()
    BENCH_BIN_DIR.mkdir(exist_ok=True)
    out = []
    for src in sorted(BENCH_DIR.glob("*.cpp")):
        if src.stem.endswith("_libtorch"):
            continue  # host C++ against torch: build_libtorch_bench
        exe = BENCH_BIN_DIR / src.stem
        _run([hipcc, "-x", "hip", *HIP_FLAGS, str(src), f"-L{LIB_DIR}", "-lfeatherops_amd",
              f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)])
        out.append(exe)
    return out


def build_all() -> None:
    build_library()
    with ThreadPoolExecutor(max_workers=3) as ex:
        jobs = [ex.submit(build_torch_ops), ex.submit(build_benches), ex.submit(build_libtorch_bench)]
        for j in jobs:
            j.result()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB_PATH} and {OPS_LIB_PATH}")
