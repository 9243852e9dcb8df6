"""The C ABI library loads and exports every function include/vc_hip.h
declares; without a GPU every compute entry point reports "unavailable"
through its status instead of throwing or crashing. No device work here."""

import ctypes
import re
from pathlib import Path

import pytest

from vectorcore_amd import cabi as C

HEADER = Path(__file__).resolve().parents[1] / "include" / "vc_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vc_hip_\w+)\s*\(", text)))


def test_header_declares_the_device_interface():
    names = declared_functions()
    for required in ("vc_hip_alloc", "vc_hip_upload", "vc_hip_download", "vc_hip_binary", "vc_hip_unary",
                     "vc_hip_matmul", "vc_hip_transpose_last2", "vc_hip_reduce_sum", "vc_hip_reduce_axis",
                     "vc_hip_scatter_axis", "vc_hip_axpy", "vc_hip_synchronize", "vc_hip_xent_forward",
                     "vc_hip_xent_backward", "vc_hip_relu_backward", "vc_hip_sigmoid_backward"):
        assert required in names


def test_library_exports_every_declared_function():
    lib = C.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers the whole header
    assert set(declared_functions()) == set(C.EXPORTED)


def test_status_codes_match_the_header():
    text = HEADER.read_text()
    codes = dict(re.findall(r"#define (VC_HIP_\w+) (\d+)", text))
    assert codes["VC_HIP_OK"] == "0"
    assert {int(v) for k, v in codes.items() if k.startswith("VC_HIP_ERR")} == set(C.ERRORS)
    ops = dict(re.findall(r"#define (VC_(?:BINARY|UNARY|REDUCE)_\w+) (\d+)", text))
    assert int(ops["VC_BINARY_DIVIDE"]) == C.DIV and int(ops["VC_UNARY_LOG"]) == C.LOG
    assert int(ops["VC_REDUCE_ARGMAX"]) == C.ARGMAX


def test_unavailable_device_is_reported_by_status():
    if C.available():
        pytest.skip("a GPU is present; covered by the gpu tests")
    lib = C.lib()
    assert lib.vc_hip_gemm_kernel() == b"unavailable"
    assert b"no HIP device" in lib.vc_hip_last_error() or b"gfx950" in lib.vc_hip_last_error()
    ptr = ctypes.c_void_p()
    assert lib.vc_hip_alloc(16, ctypes.byref(ptr)) == 5  # VC_HIP_ERR_UNAVAILABLE
    assert lib.vc_hip_unary(None, None, 4, 0) == 5
    assert lib.vc_hip_matmul(None, None, None, 2, 2, 2, C.sizes([0]), C.sizes([0]), 1, 0, 0) == 5
    assert lib.vc_hip_synchronize() == 0  # a no-op without a device, as in the reference
    with pytest.raises(RuntimeError, match="unavailable"):
        C.check(lib.vc_hip_fill(None, 4, ctypes.c_float(1.0)))


def test_a_c_program_compiles_and_links_against_the_header(tmp_path):
    # The boundary is plain C: a C99 translation unit that calls every group of
    # entry points compiles warning-free with the header alone and links
    # against the built library (nothing runs: no device here).
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "uses_abi.c"
    src.write_text(
        '#include "vc_hip.h"\n'
        "int main(void) {\n"
        "    vc_hip_map_program program = {0};\n"
        "    void* p = 0;\n"
        "    size_t off = 0;\n"
        "    int status = vc_hip_available() ? 0 : 1;\n"
        "    status |= vc_hip_alloc(16, &p);\n"
        "    status |= vc_hip_matmul(0, 0, 0, 1, 1, 1, &off, &off, 1, 0, 0);\n"
        "    status |= vc_hip_reduce_axis_noalloc(0, 0, 1, 1, 1, VC_REDUCE_SUM);\n"
        "    status |= vc_hip_map(&program);\n"
        "    status |= vc_hip_xent_forward(0, 0, 1, 1, 0, 0);\n"
        "    return status;\n"
        "}\n")
    lib = Path(C.LIB_PATH)
    out = tmp_path / "uses_abi"
    r = subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror", "-I", str(HEADER.parent),
                        str(src), "-o", str(out), "-L", str(lib.parent), "-lvc_hip", f"-Wl,-rpath,{lib.parent}"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
