"""Build the gfx950 sampling library in-tree.

``python voidinfer_amd/build.py`` (or ``build()``) compiles every HIP source
under ``voidinfer_amd/csrc`` with hipcc for gfx950 and links
``voidinfer_amd/libvoidinfer_sampling.so``.  Objects go to ``_build/``.  Run it as a
script (not ``-m``): importing the package loads the library this builds.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "libvoidinfer_sampling.so"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation (some of their forms have
# given wrong results on these GPUs).  -ffp-contract=off: every float operation is
# rounded as written, as in the CPU reference (fused multiply-adds only where the
# source calls fmaf).
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    "-I", str(ROOT / "include"),
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    build_launcher_test(verbose)
    return LIB


# The compiled GPU test of the C++ launchers (tests/cpp/test_launchers_gpu.cpp):
# host code over the HIP runtime and this library, run by a -m gpu test.
LAUNCHER_TEST = ROOT / "tests" / "cpp" / "test_launchers_gpu"


def build_launcher_test(verbose: bool = False) -> Path:
    rocm = Path(HIPCC).resolve().parent.parent
    src = LAUNCHER_TEST.with_suffix(".cpp")
    cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include", "-I",
           str(ROOT / "include"), str(src), "-o", str(LAUNCHER_TEST), "-L", str(LIB.parent), "-lvoidinfer_sampling",
           f"-L{rocm}/lib", "-lamdhip64", f"-Wl,-rpath,$ORIGIN/../../voidinfer_amd:{rocm}/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"launcher test build failed:\n{res.stderr}")
    if verbose:
        print(f"built {LAUNCHER_TEST}")
    return LAUNCHER_TEST


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
