"""The C++ host layer (llm-inference-cpp_amd/host: llmi::quant, llmi::Weight,
llmi::Transformer, llmi::sample with the reference's interface): the
programs tests/native/host_*_diff.cpp drive it through tables of cases and
compare every output with the CPU oracle bit for bit.  Building them needs
no GPU; running them does."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-inference-cpp_amd")
NATIVE = os.path.join(ROOT, "tests", "native")
TESTS = ["host_quant_diff", "host_model_diff", "host_sampling_diff"]


SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g", "-O1"]


def build(name, out_dir, sanitize=False):
    """The test program against libllmi_gpu.so; with sanitize, the host
    layer's sources are compiled into it with AddressSanitizer and UBSan
    (host code only: the HIP library and its kernels are the ordinary ones)."""
    exe = os.path.join(out_dir, name + ("_san" if sanitize else ""))
    host = [os.path.join(PKG, "host", "src", f) for f in sorted(os.listdir(os.path.join(PKG, "host", "src")))]
    subprocess.run(["g++", "-std=c++20", *(SAN if sanitize else ["-O2"]), "-ffp-contract=off", "-Wall",
                    "-I" + os.path.join(PKG, "host", "include"), "-I" + os.path.join(ROOT, "include"), "-I" + NATIVE,
                    "-o", exe, os.path.join(NATIVE, name + ".cpp"), *(host if sanitize else ["-L" + PKG, "-lllmi_gpu"]),
                    "-L" + PKG, "-lllmi_hip", "-L" + os.path.join(ROOT, "oracle"), "-loracle",
                    "-Wl,-rpath," + PKG + ":" + os.path.join(ROOT, "oracle"), "-pthread"], check=True)
    return exe


@pytest.mark.parametrize("name", TESTS)
def test_native_tests_build(name, tmp_path):
    assert os.path.exists(build(name, str(tmp_path)))


@pytest.mark.parametrize("name", TESTS)
def test_native_tests_build_with_sanitizers(name, tmp_path):
    assert os.path.exists(build(name, str(tmp_path), sanitize=True))


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_native_tests_pass_on_gpu_with_sanitized_host_code(name, tmp_path):
    """The same programs with the host layer under AddressSanitizer + UBSan
    (leak checking off: the HIP runtime keeps its allocations to exit)."""
    exe = build(name, str(tmp_path), sanitize=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:protect_shadow_gap=0", UBSAN_OPTIONS="print_stacktrace=1")
    out = subprocess.run([exe], capture_output=True, text=True, timeout=600, env=env)
    print(out.stdout)
    assert out.returncode == 0, out.stdout[-3000:] + out.stderr[-3000:]
    assert "AddressSanitizer" not in out.stderr and "runtime error:" not in out.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_native_tests_pass_on_gpu(name, tmp_path):
    exe = build(name, str(tmp_path))
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
