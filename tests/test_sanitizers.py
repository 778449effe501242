"""AddressSanitizer + UndefinedBehaviorSanitizer on the CPU code, as the
reference's CI runs its tests under both (CMakeLists.txt:30-33,
.github/workflows/ci.yml:27):

* the oracle and the compiled reference rebuilt with
  -fsanitize=address,undefined (make -C oracle sanitize), loaded into a python
  with libasan preloaded, run the oracle test modules (the 32 s baseline-shape
  sweep left out: the smaller shapes cover the same code);
* a planted out-of-bounds write through the sanitized oracle is reported, so
  the sanitizer is known to be live in that setup;
* the host layer (host/src/*.cpp) built with the same flags runs its
  GPU-free paths (tests/native/host_cpu_checks.cpp), leak checking on.

Skipped where the compiler has no sanitizer runtime."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-inference-cpp_amd")
ORACLE = os.path.join(ROOT, "oracle")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]


def libasan():
    p = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


pytestmark = pytest.mark.skipif(libasan() is None, reason="no libasan for g++")


def asan_env(**extra):
    env = dict(os.environ)
    prev = env.get("LD_PRELOAD")
    env["LD_PRELOAD"] = libasan() + (":" + prev if prev else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    env["LLMI_ORACLE_SANITIZED"] = "1"
    env.update(extra)
    return env


@pytest.fixture(scope="module")
def sanitized_oracle():
    subprocess.run(["make", "-C", ORACLE, "sanitize", "-j", "8"], check=True, capture_output=True)
    assert os.path.exists(os.path.join(ORACLE, "_asan", "liboracle.so"))


def test_oracle_tests_pass_under_asan_and_ubsan(sanitized_oracle):
    mods = [os.path.join(ROOT, "tests", m) for m in ("test_oracle.py", "test_oracle_sampling.py", "test_oracle_gguf.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider", "-k",
                        "not test_baseline_shapes_match_reference", *mods], capture_output=True, text=True,
                       env=asan_env(), timeout=900, cwd=ROOT)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-3000:]


def test_a_planted_overflow_is_reported(sanitized_oracle):
    """Oracle-side mistake on purpose: dequantize a 64-column row into a
    one-float buffer."""
    code = (
        "import ctypes as C, numpy as np, sys\n"
        f"sys.path.insert(0, {ORACLE!r})\n"
        "import oracle as O\n"
        "assert '_asan' in O.ORACLE_SO\n"
        "lib = O.oracle().lib\n"
        "data = np.zeros(64, np.uint8); scales = np.ones(2, np.float32); dst = np.zeros(1, np.float32)\n"
        "lib.oracle_dequantize_row(data.ctypes.data_as(C.c_void_p), scales.ctypes.data_as(C.c_void_p),"
        " C.c_size_t(64), C.c_int(1), C.c_size_t(0), dst.ctypes.data_as(C.c_void_p))\n"
    )
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=asan_env(), timeout=120)
    assert r.returncode != 0
    assert "heap-buffer-overflow" in r.stderr, r.stderr[-2000:]


def test_host_layer_gpu_free_paths_under_asan_and_ubsan(tmp_path):
    exe = str(tmp_path / "host_cpu_checks")
    srcs = [os.path.join(PKG, "host", "src", f) for f in sorted(os.listdir(os.path.join(PKG, "host", "src")))]
    subprocess.run(["g++", "-std=c++20", *SAN, "-Wall", "-I" + os.path.join(PKG, "host", "include"),
                    "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "tests", "native"), "-o", exe,
                    os.path.join(ROOT, "tests", "native", "host_cpu_checks.cpp"), *srcs, "-L" + PKG, "-lllmi_hip",
                    "-Wl,-rpath," + PKG, "-pthread"], check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout
