"""The drop-in claim, compiled: tests/dropin/caller.cpp calls the library
with the reference's own syntax (find_kernel(id)->fn(...), gemm() with its
default stream argument, batched_gemm, the flash entry points and _cfg
variants, the GPT & overloads of gpt.h) and is built against include/*.h and
lib/libbmb.so with the host C++ compiler, as a maintainer swapping the
library in would build src/bench.cu, tools/test_gemm.cu and src/gpt.cu's
callers. The CPU test proves it compiles and links; the GPU test runs it
(every call checked against a double-precision or unfused reference inside
the program)."""
import os
import subprocess

import pytest

import bmb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "dropin", "caller.cpp")
INC = os.path.join(ROOT, "include")


def _build(out):
    libdir = os.path.dirname(bmb.LIB_PATH)
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I" + INC, "-I/opt/rocm/include", SRC, "-o", out,
           "-L" + libdir, "-lbmb", "-Wl,-rpath," + libdir,
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def test_reference_shaped_caller_builds(tmp_path):
    exe = _build(str(tmp_path / "caller"))
    assert os.path.exists(exe)


@pytest.mark.gpu
def test_reference_shaped_caller_runs(gpu, tmp_path):
    exe = _build(str(tmp_path / "caller"))
    print("running the reference-shaped C++ caller", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("dropin: OK")
