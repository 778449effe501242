"""CPU test: the C++ layer builds inside the reference engine -- with the
reference's own headers (ModelConfig, Model, SafetensorsFile, TokenId) and
the reference's Transformer::load(const Model&, quant::Type) signature --
the way a maintainer adds it to the reference's build, and the reference's
own callers of Transformer and sample() (the server, the grammar constraint,
llmi-chat) compile unchanged against it.  Skipped where the reference is not
present."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-inference-cpp_amd")
REF = "/root/reference"


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "include", "llmi")), reason="reference sources not present")
def test_host_layer_compiles_against_the_reference_headers():
    srcs = [os.path.join(PKG, "host", "src", f) for f in ("quant.cpp", "weight.cpp", "transformer.cpp", "sampling.cpp")]
    srcs.append(os.path.join(PKG, "host", "integration", "load_from_model.cpp"))
    for src in srcs:
        subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-DLLMI_GPU_WITH_REFERENCE_MODEL",
                        "-I" + os.path.join(PKG, "host", "include"), "-I" + os.path.join(REF, "include"),
                        "-I" + os.path.join(ROOT, "include"), src], check=True)


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "include", "llmi")), reason="reference sources not present")
@pytest.mark.parametrize("caller", ["src/server/server.cpp", "src/grammar/constraint.cpp", "apps/llmi-chat/main.cpp"])
def test_reference_callers_compile_against_the_gpu_headers(caller):
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-w", "-DLLMI_GPU_WITH_REFERENCE_MODEL",
                    "-I" + os.path.join(PKG, "host", "include"), "-I" + os.path.join(REF, "include"),
                    "-I" + os.path.join(REF, "third_party", "cpp-httplib"), "-I" + os.path.join(ROOT, "include"),
                    os.path.join(REF, caller)], check=True)
