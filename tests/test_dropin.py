"""The drop-in claim, checked against the reference's own interface headers where the reference tree is present (this
build container; the GPU box has no reference tree, so these are skipped there):

- the HIP backend (xpu-serve_amd/host/hip_backend.cpp) compiles against the reference's src/backend/backend.h,
  graph/graph.h, tensor/tensor.h and util/error.h instead of the restatement it builds against standalone;
- the C++ launcher surface (include/xs_hip_kernels.hpp) compiles with its error type derived from the reference's
  xs::Error (XS_HIP_ERROR_BASE), so a refused launch is the exception every caller of a backend already handles.

Compile-only (g++ -fsyntax-only): nothing of the reference is linked or run."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="the reference tree is not present here")


def syntax_check(path, extra=()):
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-Werror=return-type", f"-I{REF_SRC}",
           "-I/root/reference/third_party", f"-I{os.path.join(ROOT, 'include')}", *extra, path]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]


def test_backend_compiles_against_the_reference_interface():
    syntax_check(os.path.join(ROOT, "xpu-serve_amd", "host", "hip_backend.cpp"))


def test_launchers_throw_the_reference_error_type():
    src = """#include "util/error.h"
#define XS_HIP_ERROR_BASE ::xs::Error
#include "xs_hip_kernels.hpp"
#include <type_traits>
static_assert(std::is_base_of_v<::xs::Error, ::xs::hip_be::Error>, "a refused launch is an xs::Error");
int main() { return 0; }
"""
    with tempfile.NamedTemporaryFile("w", suffix=".cpp", delete=False) as f:
        f.write(src)
        path = f.name
    try:
        syntax_check(path)
    finally:
        os.unlink(path)
