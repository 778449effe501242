"""CPU tests of the C ABI boundary: libllmi_hip.so loads, exports every
function include/llmi_hip.h declares, and rejects calls made before
llmi_hip_init without touching a GPU."""

import ctypes as C
import os
import re
import subprocess

import llmi_hip as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llmi_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llmi_hip_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("llmi_hip_quantize", "llmi_hip_dequantize_row", "llmi_hip_matmul", "llmi_hip_weight_upload"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = H.load()
    names = declared()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    out = subprocess.run(["nm", "-D", "--defined-only", H.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (llmi_hip_\w+)", out))
    assert set(names) <= exported


def test_binding_covers_the_header():
    assert set(declared()) == set(H.SIGNATURES)


def test_calls_before_init_fail_cleanly():
    lib = H.load()
    assert lib.llmi_hip_version().startswith(b"llmi_hip")
    assert lib.llmi_hip_row_bytes(33, H.Q4_0) == 17
    assert lib.llmi_hip_row_bytes(33, H.Q8_0) == 33
    y = (C.c_float * 4)()
    rc = lib.llmi_hip_matmul(None, None, 1, 4, 4, None, y)
    assert rc == 3  # LLMI_ERR_STATE
    assert b"init" in lib.llmi_hip_last_error()
    assert lib.llmi_hip_weight_free(None) == 0


def test_library_is_gfx950_code():
    out = subprocess.run(["/opt/rocm/bin/roc-obj-ls", H.LIB_PATH], capture_output=True, text=True)
    if out.returncode == 0 and out.stdout:
        assert "gfx950" in out.stdout
