"""Build recipe for libfeatherops_amd.so (gfx950) and the C++ bench harnesses.

Plain hipcc invocations, no torch involved: every `csrc/*.hip` file is
compiled to an object in `_build/`, then linked into `lib/libfeatherops_amd.so`.
The C++ benches in `cpp_benchmarks/` link against that library (mirroring the
reference's cpp_benchmarks/build_benchmark_scaled_mm_hip.sh, which links the
kernel's extern "C" ABI directly).

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


def build_benches() -> list[Path]:
    hipcc = _hipcc()
    BENCH_BIN_DIR.mkdir(exist_ok=True)
    out = []
    for src in sorted(BENCH_DIR.glob("*.cpp")):
        exe = BENCH_BIN_DIR / src.stem
        _run([hipcc, "-x", "hip", *HIP_FLAGS, str(src), f"-L{LIB_DIR}", "-lfeatherops_amd",
              f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)])
        out.append(exe)
    return out


def build_all() -> None:
    build_library()
    build_benches()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB_PATH}")
