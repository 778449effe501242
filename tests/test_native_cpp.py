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


def build(name, out_dir):
    exe = os.path.join(out_dir, name)
    subprocess.run(["g++", "-std=c++20", "-O2", "-ffp-contract=off", "-Wall", "-I" + os.path.join(PKG, "host", "include"),
                    "-I" + os.path.join(ROOT, "include"), "-I" + NATIVE, "-o", exe, os.path.join(NATIVE, name + ".cpp"),
                    "-L" + PKG, "-lllmi_gpu", "-lllmi_hip", "-L" + os.path.join(ROOT, "oracle"), "-loracle",
                    "-Wl,-rpath," + PKG + ":" + os.path.join(ROOT, "oracle"), "-pthread"], check=True)
    return exe


@pytest.mark.parametrize("name", TESTS)
def test_native_tests_build(name, tmp_path):
    assert os.path.exists(build(name, str(tmp_path)))


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_native_tests_pass_on_gpu(name, tmp_path):
    exe = build(name, str(tmp_path))
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
