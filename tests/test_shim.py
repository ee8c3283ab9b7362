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


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not installed")
def test_unknown_kv_type_aborts(rd4, tmp_path):
    """kv_unreachable (kv.h:58-69, checked by check_kvtype.hip:55-75,249-263 with
    a forked child): a KvType outside the enum kills the caller with SIGABRT
    instead of returning a guess."""
    import signal
    lib = rd4.LIB_PATH
    exe = str(tmp_path / "shim_caller")
    cmd = ["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include"),
           os.path.join(ROOT, "tests", "shim_caller.cpp"), "-o", exe, lib,
           "-Wl,-rpath," + os.path.dirname(lib)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    r = subprocess.run([exe, "abort"], capture_output=True, text=True, timeout=60)
    assert r.returncode == -signal.SIGABRT, (r.returncode, r.stdout, r.stderr)
    assert "unknown KvType" in r.stderr and "no abort" not in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("hd", [256, 96])
def test_shim_device_readers_bit_exact(orc, dev, hd):
    """rdna4::kv_load<> and kv_load8<> of the shim (built into tests/libshimkv.so)
    return the oracle's dequant bits (kv.h:174-368) for every type."""
    import ctypes

    import numpy as np
    import torch

    so = os.path.join(ROOT, "tests", "libshimkv.so")
    if not os.path.exists(so):
        pytest.fail("tests/libshimkv.so is not built: run __graft_entry__.build()")
    L = ctypes.CDLL(so)
    L.shim_kv_read_rows.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    n_rows = 64
    x = orc.randn(n_rows * hd, 77) * 2
    x[5::hd] *= 8
    x[: 2 * hd] = 0.0
    for t in range(6):
        b = orc.store_rows(t, x)
        want = orc.load_rows(t, b, x.size)
        bd = torch.from_numpy(b).to(dev)
        for use8 in (0, 1):
            out = torch.full((n_rows * hd,), float("nan"), dtype=torch.float32, device=dev)
            rc = L.shim_kv_read_rows(t, bd.data_ptr(), out.data_ptr(), n_rows, hd, use8,
                                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            assert rc == 0
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (t, use8)
