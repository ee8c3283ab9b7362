"""The C++ header shims in include/rdna4/ keep the reference's rdna4:: API
(kv.h:58-169, attn.cuh:56-1049, attn_fa2.cuh:173-207, nn.cuh:414): a caller
written against that API compiles with g++, links librdna4attn and gets the
reference's table values and false-on-bad-arguments behaviour (host only)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_reference_api_caller_builds_and_runs(rd4, tmp_path):
    lib = rd4.LIB_PATH
    exe = str(tmp_path / "shim_caller")
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
           os.path.join(ROOT, "tests", "shim_caller.cpp"), "-o", exe, lib,
           "-Wl,-rpath," + os.path.dirname(lib)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr
