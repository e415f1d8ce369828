"""Ahead-of-time build of the package's native parts.

* libfrisk_hip.so, the C-ABI of include/frisk_hip.h: every .hip file under
  csrc/ compiled for gfx950 with hipcc and linked into one shared library.
* frisk_ffi (Python extension), the tile-IR builder: the C++ sources under
  ir/ compiled with g++ against pybind11 (host code only).

Both land next to this file, so they travel with the source tree.  Invoked
by __graft_entry__.build() and by `python -m frisk_amd.build`.
"""
from __future__ import annotations

import os
import shlex
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
IRSRC = HERE / "ir"
LIB = HERE / "libfrisk_hip.so"
FFI = HERE / ("frisk_ffi" + sysconfig.get_config_var("EXT_SUFFIX"))
ARCH = "gfx950"
CXX = os.environ.get("CXX", "g++")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-fp32 VALU forms are kept out of generated code on this platform.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# MFMA accumulators in VGPRs: the softmax rescale and epilogue read them
# with VALU ops, which would otherwise copy AGPRs back and forth.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
# Files whose MFMA accumulators live in AGPRs: their kernels hold 256
# accumulator registers per lane and read them only in the epilogue.
AGPR_ACC_PREFIX = "gemm_w4_"


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(verbose: bool = False, extra: list[str] | None = None) -> Path:
    objdir = HERE / "_build"
    objdir.mkdir(exist_ok=True)
    flags = COMMON + (extra or [])

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        form = [] if src.name.startswith(AGPR_ACC_PREFIX) else VGPR_FORM
        cmd = [HIPCC, *flags, *form, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(shlex.quote(c) for c in cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, sources()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    write_build_info()
    return LIB


def source_digest() -> str:
    """sha256 (first 16 hex digits) over the kernel sources and the C-ABI
    header, in name order: the same digest bench.py reports."""
    import hashlib
    h = hashlib.sha256()
    files = sorted(list(CSRC.glob("*")) + list((HERE.parent / "include").glob("*.h")))
    for f in sorted(files, key=lambda f: f.name):
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def write_build_info() -> None:
    """frisk_amd/BUILD_INFO.json: the git commit the library was built from
    (with a '+dirty' mark for uncommitted changes) and the source digest,
    so that a run on a machine without the repository history can name
    what it measured."""
    import json
    commit = None
    try:
        root = HERE.parent
        r = subprocess.run(["git", "-C", str(root), "rev-parse", "HEAD"], capture_output=True,
                           text=True, timeout=10)
        if r.returncode == 0:
            commit = r.stdout.strip()
            d = subprocess.run(["git", "-C", str(root), "status", "--porcelain", "--",
                                "frisk_amd/csrc", "include"], capture_output=True, text=True,
                               timeout=10)
            if d.returncode == 0 and d.stdout.strip():
                commit += "+dirty"
    except (OSError, subprocess.SubprocessError):
        commit = None
    (HERE / "BUILD_INFO.json").write_text(
        json.dumps({"git_commit": commit, "source_sha256_16": source_digest()}) + "\n")


def build_ffi(verbose: bool = False) -> Path:
    """Compile the pybind11 tile-IR module (host C++ only)."""
    import pybind11
    objdir = HERE / "_build" / "ir"
    objdir.mkdir(parents=True, exist_ok=True)
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-fvisibility=hidden",
             f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}"]

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [CXX, *flags, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(shlex.quote(c) for c in cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"{CXX} failed on {src.name}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, sorted(IRSRC.glob("*.cpp"))))
    tmp = FFI.with_name(FFI.name + ".tmp")
    r = subprocess.run([CXX, "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of frisk_ffi failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, FFI)
    return FFI


def build_all(verbose: bool = False) -> list[Path]:
    return [build(verbose), build_ffi(verbose)]


if __name__ == "__main__":
    if "--ffi" in sys.argv:
        print(build_ffi(verbose="-v" in sys.argv))
    else:
        print(build_all(verbose="-v" in sys.argv))
