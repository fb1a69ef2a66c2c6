"""Builds libcellm_hip.so (HIP kernels + C ABI) for gfx950, in-tree.

    python -m cellm_amd.build          # or cellm_amd.build.build_library()

Every HIP source is compiled with hipcc --offload-arch=gfx950 and with the
packed-FP32 target feature disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops); the library is linked next to this file so it travels with
the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libcellm_hip.so"
STEP_LIB_PATH = PKG_DIR / "libcellm_llama_step.so"
PROBES_LIB_PATH = PKG_DIR / "libcellm_probes.so"
REPO_ROOT = PKG_DIR.parent

SOURCES = ["qgemv.hip", "qgemv_mfma.hip", "qgemv_f32x_mfma.hip", "qgemm.hip", "dequant.hip", "decode.hip", "lowbit.hip", "capi.cpp", "cellm_file.cpp"]
HEADERS = ["common.hpp", "kernels.hpp"]
ARCH = os.environ.get("CELLM_HIP_ARCH", "gfx950")


def _hipcc() -> str:
    env = os.environ.get("HIPCC")
    if env:
        return env
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc") or ""):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{REPO_ROOT / 'include'}",
    ]


def _compile_one(src: str, verbose: bool) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [_hipcc(), *_flags(), "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    return obj


def build_library(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source and link libcellm_hip.so; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile_one(s, verbose), SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stderr)
    os.replace(tmp, LIB_PATH)
    build_step_library(verbose)
    build_probes_library(verbose)
    return LIB_PATH


def build_probes_library(verbose: bool = False) -> Path:
    """bench.py's measurement probes (measured MFMA and streaming-read ceilings): a
    separate library the hot path never loads."""
    tmp = PROBES_LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), *_flags(), "-shared", "-x", "hip", str(CSRC / "probes.hip"), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        raise RuntimeError("probe library build failed:\n" + "\n".join(noise))
    os.replace(tmp, PROBES_LIB_PATH)
    return PROBES_LIB_PATH


def build_step_library(verbose: bool = False) -> Path:
    """The host-side decode-step runners over libcellm_hip.so (C++; the CPU
    parts compiled without FP contraction so they round as the reference; the
    device runner also calls the HIP runtime for its own buffers)."""
    cxx = os.environ.get("CXX", "g++")
    tmp = STEP_LIB_PATH.with_suffix(".so.tmp")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = [cxx, "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fno-math-errno",
           "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{rocm}/include", "-o", str(tmp), str(CSRC / "llama_step.cpp"),
           str(CSRC / "llama_device.cpp"), f"-L{PKG_DIR}", "-lcellm_hip", f"-L{rocm}/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{rocm}/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("decode-step library build failed:\n" + res.stderr)
    os.replace(tmp, STEP_LIB_PATH)
    return STEP_LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
