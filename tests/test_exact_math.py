"""CPU test: the device expf restatement (csrc/exact_math.hpp) equals the
host libm's expf -- the function the reference's softmax and SiLU call
(src/model/kernels.cpp:141, :148) -- on every float input."""

import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_equals_host_libm_on_all_floats(tmp_path):
    exe = tmp_path / "expf_exhaustive"
    subprocess.run(["g++", "-O2", "-std=c++20", "-ffp-contract=off", "-mfma", "-pthread", "-o", str(exe),
                    os.path.join(ROOT, "tests", "native", "expf_exhaustive.cpp")], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("mismatches 0"), out.stdout
