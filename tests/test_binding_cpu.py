"""The reference-side binding compiles: tests/binding/hip_ops.h (the C++ shim
over include/ghassan_hip.h) and tests/binding/ops_dispatch.cpp (the GAI_HIP
dispatch of core/ops.cpp:28-40 as out-of-line definitions of the reference's
core/ops.h / core/device.h functions) are syntax-checked with g++ against the
reference's own headers. A qualified definition must match the reference's
declaration exactly, so this proves that every wrapped call site's argument
list is the reference's and that it type-checks against the C ABI. Skipped
where the reference tree is absent (the GPU box)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
SRC = os.path.join(ROOT, "tests", "binding", "ops_dispatch.cpp")

pytestmark = pytest.mark.skipif(not os.path.isfile(os.path.join(REF, "core", "ops.h")),
                                reason="reference headers not present")


def _compile(source_text):
    cmd = ["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", f"-I{REF}",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROOT, 'tests', 'binding')}", "-x", "c++", "-"]
    return subprocess.run(cmd, input=source_text, capture_output=True, text=True)


def test_dispatch_binding_type_checks():
    r = _compile(open(SRC).read())
    assert r.returncode == 0, r.stderr


@pytest.mark.parametrize("old,new", [
    ("int M, int K, int N, int kind) {\n    GAI_HIP_ONLY(dev, linear_forward_q4", "int M, int K, int N, long kind) {\n"
     "    GAI_HIP_ONLY(dev, linear_forward_q4"),
    ("float scale, float* scratch, int window) {\n    GAI_DISPATCH(dev, attention_decode_ring_fp16",
     "float scale, int window) {\n    GAI_DISPATCH(dev, attention_decode_ring_fp16"),
])
def test_mismatched_argument_list_is_rejected(old, new):
    """The check has teeth: a definition whose argument list differs from the
    reference's declaration does not compile."""
    src = open(SRC).read()
    assert old in src
    r = _compile(src.replace(old, new))
    assert r.returncode != 0
