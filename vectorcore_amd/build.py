"""In-tree build of the native parts of vectorcore_amd.

  libvc_hip.so      HIP kernels + the C ABI of include/vc_hip.h, for gfx950
  libvectorcore.so  the C++20 tensor/autograd runtime (the reference's C++
                    API with the hip device), linked against libvc_hip.so
  _vectorcore*.so   the pybind11 module over libvectorcore.so (rpath $ORIGIN)
  _build/bin/test_vectorcore, _build/asan/..., _build/tsan/...
                    the C++ suite (tests/cpp), linked against the library and,
                    for the sanitizer builds, compiled together with the
                    runtime's sources under ASan+UBSan or TSan

Run `python vectorcore_amd/build.py` (or __graft_entry__.build()). Every call
recompiles; objects go to vectorcore_amd/_build/, libraries next to this file.
"""

from __future__ import annotations

import os
import re
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

HIP_SOURCES = ["runtime.hip", "elementwise.hip", "reduce.hip", "xent.hip", "gemm.hip", "fused_map.hip"]
# Sources compiled once per define set: the fused-map interpreters, one object
# per input count, so that they compile in parallel.
HIP_VARIANT_SOURCES = {"fused_map_inputs.hip": [[f"-DVC_MAP_NIN={k}"] for k in range(1, 9)]}
LIB_SOURCES = ["shape.cpp", "storage.cpp", "tensor.cpp", "autograd.cpp", "ops.cpp", "nn.cpp",
               "cpu/parallel.cpp", "cpu/cpu_backend.cpp", "hip/hip_backend.cpp"]
BINDINGS = "python/bindings.cpp"
CPP_TEST = ROOT / "tests" / "cpp" / "test_vectorcore.cpp"
ORACLE_C = ROOT / "oracle" / "vc_oracle.c"
# Sanitizer variants of the C++ suite: (directory under _build, compile and link flags).
SANITIZERS = {"asan": ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"],
              "tsan": ["-fsanitize=thread"]}

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


def _scratch_kernels(log: str) -> list[tuple[str, int]]:
    """Kernels that the compiler's resource report (-Rpass-analysis=
    kernel-resource-usage) gives a nonzero ScratchSize: register spills to
    memory, which every kernel here is written to avoid."""
    spills, name = [], None
    for line in log.splitlines():
        m = re.search(r"remark:\s*Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"remark:\s*ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0:
            spills.append((name, int(m.group(1))))
    return spills


def build_hip(verbose: bool = False) -> Path:
    """Compile the HIP kernels and the C ABI into libvc_hip.so. Fails when any
    kernel spills registers to scratch memory."""
    OBJ.mkdir(exist_ok=True)

    def compile_one(job) -> Path:
        src, defines, tag = job
        obj = OBJ / (Path(src).stem + tag + ".hip.o")
        log = _run([HIPCC, *HIP_FLAGS, *defines, "-Rpass-analysis=kernel-resource-usage", "-c",
                    str(CSRC / "hip" / src), "-o", str(obj)])
        spills = _scratch_kernels(log)
        if spills:
            raise RuntimeError(f"{src} {' '.join(defines)}: kernels spill to scratch memory "
                               f"(bytes per lane): {spills}")
        if verbose:
            print("\n".join(l for l in log.splitlines() if "remark:" not in l), file=sys.stderr)
        return obj

    jobs = [(src, [], "") for src in HIP_SOURCES]
    for src, define_sets in HIP_VARIANT_SOURCES.items():
        jobs += [(src, d, "_" + "_".join(x.split("=")[-1] for x in d)) for d in define_sets]
    # The slowest compiles (the interpreters) first.
    jobs.sort(key=lambda j: 0 if j[0] in HIP_VARIANT_SOURCES else 1)
    objs = _parallel(compile_one, jobs)
    out = PKG / "libvc_hip.so"
    tmp = out.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    tmp.replace(out)
    return out


def _python_includes() -> list[str]:
    import pybind11
    return ["-I", sysconfig.get_paths()["include"], "-I", pybind11.get_include()]


def _core_flags() -> list[str]:
    return ["-std=c++20", "-fPIC", "-Wall", "-Wextra", "-I", str(CSRC / "core" / "include"), "-I", str(ROOT / "include")]


def build_core(verbose: bool = False) -> Path:
    """Compile the C++ runtime into libvectorcore.so and its bindings into the _vectorcore module."""
    for sub in ("cpu", "hip", "python"):
        (OBJ / sub).mkdir(parents=True, exist_ok=True)
    flags = ["g++", "-O3", "-DNDEBUG", *_core_flags()]

    def compile_one(src: str) -> Path:
        obj = OBJ / (src.replace(".cpp", ".o"))
        extra = ["-fvisibility=hidden", *_python_includes()] if src == BINDINGS else []
        log = _run(flags + extra + ["-c", str(CSRC / "core" / src), "-o", str(obj)])
        if verbose and log:
            print(log, file=sys.stderr)
        return obj

    objs = _parallel(compile_one, LIB_SOURCES + [BINDINGS])
    lib = PKG / "libvectorcore.so"
    tmp = lib.with_suffix(".so.tmp")
    _run(["g++", "-shared", "-o", str(tmp), *map(str, objs[:-1]), "-L", str(PKG), "-lvc_hip", "-Wl,-rpath,$ORIGIN",
          "-lpthread"])
    tmp.replace(lib)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG / f"_vectorcore{suffix}"
    tmp = out.with_name(out.name + ".tmp")
    _run(["g++", "-shared", "-o", str(tmp), str(objs[-1]), "-L", str(PKG), "-lvectorcore", "-lvc_hip",
          "-Wl,-rpath,$ORIGIN", "-lpthread"])
    tmp.replace(out)
    return out


def build_cpp_tests(sanitizers: bool = True) -> list[Path]:
    """The C++ suite against libvectorcore.so, and (sanitizers=True) its ASan+UBSan and TSan builds,
    which compile the runtime's sources and the oracle's C kernels with the sanitizer."""
    built = []
    bindir = OBJ / "bin"
    bindir.mkdir(parents=True, exist_ok=True)
    oracle_obj = bindir / "vc_oracle.o"
    # The oracle's C kernels, serial (no OpenMP), as the suite's cross-check.
    _run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-c", str(ORACLE_C), "-o", str(oracle_obj)])
    exe = bindir / "test_vectorcore"
    _run(["g++", "-O2", *_core_flags(), "-I", str(ORACLE_C.parent), str(CPP_TEST), str(oracle_obj), "-o", str(exe),
          "-L", str(PKG), "-lvectorcore", "-lvc_hip", "-Wl,-rpath,$ORIGIN/../..", "-lpthread", "-lm"])
    built.append(exe)
    if not sanitizers:
        return built

    def compile_variant(item: tuple[str, str]) -> Path:
        name, src = item
        obj = OBJ / name / src.replace(".cpp", ".o").replace(".c", ".o")
        obj.parent.mkdir(parents=True, exist_ok=True)
        if src.endswith(".c"):
            _run(["gcc", "-std=c11", "-O1", "-g", *SANITIZERS[name], "-ffp-contract=off", "-c", str(ORACLE_C),
                  "-o", str(obj)])
        else:
            _run(["g++", "-O1", "-g", *SANITIZERS[name], *_core_flags(), "-c", str(CSRC / "core" / src), "-o", str(obj)])
        return obj

    jobs = [(name, src) for name in SANITIZERS for src in LIB_SOURCES + ["vc_oracle.c"]]
    objs = dict(zip(jobs, _parallel(compile_variant, jobs)))
    for name, san in SANITIZERS.items():
        out = OBJ / name / "test_vectorcore"
        _run(["g++", "-O1", "-g", *san, *_core_flags(), "-I", str(ORACLE_C.parent), str(CPP_TEST),
              *[str(objs[(name, src)]) for src in LIB_SOURCES + ["vc_oracle.c"]], "-o", str(out), "-L", str(PKG),
              "-lvc_hip", "-Wl,-rpath,$ORIGIN/../..", "-lpthread", "-lm"])
        built.append(out)
    return built


def build_all(verbose: bool = False, cpp_tests: bool = True) -> None:
    build_hip(verbose)
    build_core(verbose)
    if cpp_tests:
        build_cpp_tests()


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
    print("built", PKG / "libvc_hip.so")
