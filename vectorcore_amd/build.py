"""In-tree build of the native parts of vectorcore_amd.

  libvc_hip.so   HIP kernels + the C ABI of include/vc_hip.h, for gfx950
  _vectorcore*.so  the C++20 tensor/autograd runtime and its pybind11 module,
                 linked against libvc_hip.so (rpath $ORIGIN)

Run `python vectorcore_amd/build.py` (or __graft_entry__.build()). Every call
recompiles; objects go to vectorcore_amd/_build/, libraries next to this file.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_SOURCES = ["runtime.hip", "elementwise.hip", "reduce.hip", "xent.hip", "gemm.hip"]
CORE_SOURCES = ["shape.cpp", "storage.cpp", "tensor.cpp", "autograd.cpp", "ops.cpp", "nn.cpp",
                "cpu/parallel.cpp", "cpu/cpu_backend.cpp", "hip/hip_backend.cpp", "python/bindings.cpp"]

# hipcc flags. Packed FP32 instructions are disabled (they are not trusted on
# this hardware pool); floating-point contraction is off so elementwise
# results round exactly like the reference CPU path.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", str(ROOT / "include"), "-I", str(CSRC / "hip")]


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r.stderr


def _parallel(fn, items):
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        return list(pool.map(fn, items))


def build_hip(verbose: bool = False) -> Path:
    """Compile the HIP kernels and the C ABI into libvc_hip.so."""
    OBJ.mkdir(exist_ok=True)

    def compile_one(src: str) -> Path:
        obj = OBJ / (Path(src).stem + ".hip.o")
        log = _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / "hip" / src), "-o", str(obj)])
        if verbose and log:
            print(log, file=sys.stderr)
        return obj

    objs = _parallel(compile_one, HIP_SOURCES)
    out = PKG / "libvc_hip.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    tmp.replace(out)
    return out


def _python_includes() -> list[str]:
    import pybind11
    return ["-I", sysconfig.get_paths()["include"], "-I", pybind11.get_include()]


def build_core(verbose: bool = False) -> Path:
    """Compile the C++ runtime + bindings into the _vectorcore extension module."""
    OBJ.mkdir(exist_ok=True)
    (OBJ / "cpu").mkdir(exist_ok=True)
    (OBJ / "hip").mkdir(exist_ok=True)
    (OBJ / "python").mkdir(exist_ok=True)
    flags = ["g++", "-std=c++20", "-O3", "-DNDEBUG", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra",
             "-I", str(CSRC / "core" / "include"), "-I", str(ROOT / "include"), *_python_includes()]

    def compile_one(src: str) -> Path:
        obj = OBJ / (src.replace(".cpp", ".o"))
        log = _run(flags + ["-c", str(CSRC / "core" / src), "-o", str(obj)])
        if verbose and log:
            print(log, file=sys.stderr)
        return obj

    objs = _parallel(compile_one, CORE_SOURCES)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / f"_vectorcore{suffix}"
    tmp = out.with_name(out.name + ".tmp")
    _run(["g++", "-shared", "-o", str(tmp), *map(str, objs), "-L", str(PKG), "-lvc_hip",
          "-Wl,-rpath,$ORIGIN", "-lpthread"])
    tmp.replace(out)
    return out


def build_all(verbose: bool = False) -> None:
    build_hip(verbose)
    build_core(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", PKG / "libvc_hip.so")
