"""ORACLE build recipe — test infrastructure only.

Builds the two CPU oracles:
  * oracle/liboracle.so  — the C restatement (vc_oracle.c) of the reference's
    CPU kernels, with gcc.
  * oracle/_ref/libvc_ref.so — the reference VectorCore C++ library compiled
    straight from its own source files where they lie (REFERENCE_ROOT, the
    read-only checkout; its CMake build is not used), plus ref_harness.cpp.
    Compiled with the reference's Release flags (-O3 -DNDEBUG, C++20, no
    -march; src/metal/metal_backend_stub.cpp is the reference's own non-Apple
    backend). Only built where the reference checkout exists.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REFERENCE_ROOT = Path(os.environ.get("VC_REFERENCE_ROOT", "/root/reference"))
REF_OUT = HERE / "_ref"

# Reference translation units for the CPU path (CMakeLists.txt:14-22 + the
# non-Apple backend stub selected at CMakeLists.txt:34-35).
REF_SOURCES = [
    "src/autograd.cpp", "src/nn.cpp", "src/ops.cpp", "src/shape.cpp", "src/storage.cpp",
    "src/tensor.cpp", "src/cpu/cpu_backend.cpp", "src/cpu/parallel.cpp",
    "src/metal/metal_backend_stub.cpp",
]


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{result.stdout}\n{result.stderr}")


def build_oracle() -> Path:
    out = HERE / "liboracle.so"
    _run(["gcc", "-std=c11", "-O2", "-fopenmp", "-ffp-contract=off", "-fPIC", "-shared",
          "-o", str(out), str(HERE / "vc_oracle.c"), "-lm"])
    return out


def reference_available() -> bool:
    return (REFERENCE_ROOT / "src" / "cpu" / "cpu_backend.cpp").is_file()


def build_ref() -> Path | None:
    if not reference_available():
        return None
    obj_dir = REF_OUT / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    flags = ["g++", "-std=c++20", "-O3", "-DNDEBUG", "-fPIC", "-I", str(REFERENCE_ROOT / "include")]
    units = [REFERENCE_ROOT / s for s in REF_SOURCES] + [HERE / "ref_harness.cpp"]
    objects = []

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.parent.name + "_" + src.stem + ".o")
        _run(flags + ["-c", str(src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objects = list(pool.map(compile_one, units))
    out = REF_OUT / "libvc_ref.so"
    _run(["g++", "-shared", "-o", str(out)] + [str(o) for o in objects] + ["-lpthread"])
    return out


if __name__ == "__main__":
    print(build_oracle())
    print(build_ref() or "reference checkout absent: oracle/_ref not built")
    sys.exit(0)
