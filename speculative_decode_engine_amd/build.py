"""Builds libsde_paged.so (HIP, gfx950) in-tree with hipcc.

The library is the product: the C-ABI of include/sde_paged_kv.h over
hand-written HIP kernels.  It is compiled for gfx950 only, with packed FP32
instructions disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libsde_paged.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = "gfx950"

SOURCES = ["kv_cache.hip", "paged_attention.hip", "attention_generic.hip", "spec_accept.hip", "matvec.hip",
           "model_loader.hip", "spec_loop.hip"]

# Measurement kernels for bench.py (a streaming read and the attention's
# load skeleton): a library of their own, not part of the product.
MEASURE_SRC = CSRC / "measure.hip"
MEASURE_LIB = PKG_DIR / "libsde_measure.so"

# Test infrastructure: kernels that call the device-side API of
# include/sde/attention_device.hpp from inside a caller's kernel.
DEVICE_TEST_SRC = REPO_ROOT / "tests" / "device" / "device_api_test.hip"
DEVICE_TEST_LIB = REPO_ROOT / "tests" / "device" / "libsde_device_test.so"

HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libsde_paged)")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    lines = [
        ln for ln in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in ln
    ]
    if proc.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compiles every HIP source and links the shared library (always)."""
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([cc, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    workers = min(len(cmds), max(1, (os.cpu_count() or 2) // 2))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    build_measure(verbose)
    build_device_tests(verbose)
    return LIB_PATH


def build_measure(verbose: bool = False) -> Path:
    """Compiles bench.py's measurement kernels into libsde_measure.so."""
    tmp = MEASURE_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-shared", str(MEASURE_SRC), "-o", str(tmp),
          f"-L{PKG_DIR}", "-lsde_paged", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, MEASURE_LIB)
    if verbose:
        print(f"built {MEASURE_LIB}")
    return MEASURE_LIB


def build_device_tests(verbose: bool = False) -> Path:
    """Compiles the device-API test kernels into their own library."""
    tmp = DEVICE_TEST_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-shared", str(DEVICE_TEST_SRC), "-o", str(tmp),
          f"-L{PKG_DIR}", "-lsde_paged", "-Wl,-rpath,$ORIGIN/../../speculative_decode_engine_amd"])
    os.replace(tmp, DEVICE_TEST_LIB)
    if verbose:
        print(f"built {DEVICE_TEST_LIB}")
    return DEVICE_TEST_LIB


if __name__ == "__main__":
    build(verbose=True)
