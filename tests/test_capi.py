"""C-ABI library checks that need no GPU: it loads, exports every entry point
include/rdna4attn.h declares, and its host-side tables and argument checks
behave like the reference's (kv.h:100-169, attn.cuh:665, attn.cuh:895)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "rdna4attn.h")).read()
    return sorted(set(re.findall(r"\b(rd4_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(rd4):
    L = rd4.lib()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(L, n), n
        assert n in rd4.SIGNATURES, n
    out = subprocess.run(["nm", "-D", "--defined-only", rd4.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (rd4_\w+)", out))
    assert set(names) <= exported


def test_type_names_and_parse(rd4):
    for t, name in enumerate(rd4.TYPE_NAMES):
        assert rd4.kv_type_name(t) == name
        assert rd4.kv_type_parse(name) == t
    assert rd4.kv_type_name(99) == "<unknown-kv-type>"
    for bad in ("q9_9", "q5_1", ""):
        with pytest.raises(ValueError, match="kv type must be one of"):
            rd4.kv_type_parse(bad)


def test_row_bytes_and_bytes_per_elem(rd4, orc):
    assert [rd4.kv_row_bytes(t, 256) for t in range(6)] == [1024, 512, 272, 144, 176, 160]
    assert [rd4.kv_bytes_per_elem(t) for t in range(6)] == [4.0, 2.0, 34 / 32, 18 / 32, 22 / 32, 20 / 32]
    assert rd4.kv_row_bytes(99, 256) == -1 and rd4.kv_bytes_per_elem(99) == 0.0
    for t in range(6):
        for hd in (32, 96, 256, 512):
            assert rd4.kv_row_bytes(t, hd) == orc.row_bytes(t, hd)


def test_kv_budget_131k(rd4):
    # check_kvtype.hip:146-158: 16 layers x 4 kv heads x 256 dims per side per token
    def budget(k, v):
        return int(131072 * 16 * 4 * 256 * (rd4.kv_bytes_per_elem(k) + rd4.kv_bytes_per_elem(v)))
    assert budget(1, 1) == 8589934592
    assert budget(2, 2) == 4563402752
    assert budget(3, 3) == 2415919104
    assert budget(4, 5) == 2818572288


def test_partial_bytes_and_wpb_policy(rd4):
    L = rd4.lib()
    assert L.rd4_attn_partial_bytes(24, 256, 16) == 24 * 16 * 258 * 4
    assert [L.rd4_attn_split_wpb(s) for s in (1, 4, 5, 15, 16, 32)] == [16, 16, 8, 8, 16, 16]


def test_argument_errors_without_gpu(rd4):
    """Rejected before any HIP call, like the reference's `return false` paths."""
    L = rd4.lib()
    nul = ctypes.c_void_p(0)
    assert L.rd4_kv_store_row_launch(99, nul, nul, 32, nul) == rd4.ETYPE
    assert L.rd4_kv_store_row_launch(2, nul, nul, 33, nul) == rd4.EINVAL
    assert L.rd4_kv_fill_launch(7, nul, 1, 256, 1, nul) == rd4.ETYPE
    # head_dim % 32 != 0, head_dim > 512, bad GQA ratio, unknown type, n_splits < 1
    assert L.rd4_attn_launch(nul, nul, nul, nul, 0, 24, 4, 100, 1.0, 1, 1, nul) == rd4.EINVAL
    assert L.rd4_attn_launch(nul, nul, nul, nul, 0, 24, 4, 544, 1.0, 1, 1, nul) == rd4.EINVAL
    assert L.rd4_attn_launch(nul, nul, nul, nul, 0, 24, 5, 256, 1.0, 1, 1, nul) == rd4.EINVAL
    assert L.rd4_attn_launch(nul, nul, nul, nul, 0, 24, 4, 256, 1.0, 6, 1, nul) == rd4.ETYPE
    assert L.rd4_attn_launch_split(nul, nul, nul, nul, nul, 0, 24, 4, 256, 1.0, 1, 1, 0, nul) == rd4.EINVAL
    assert L.rd4_attn_launch_split_wpb(nul, nul, nul, nul, nul, 0, 24, 4, 256, 1.0, 1, 1, 4, 12, nul) == rd4.EINVAL
    assert b"wpb" in L.rd4_last_error()


def test_fa2_usable_admission(rd4, monkeypatch):
    L = rd4.lib()
    assert L.rd4_fa2_prefill_usable(1, 1, 512, 2048, 24, 4, 256) == 1
    assert L.rd4_fa2_prefill_usable(2, 2, 512, 2048, 24, 4, 256) == 0  # f16/f16 only
    monkeypatch.setenv("RD_GFX12_FA2_PREFILL", "0")
    assert L.rd4_fa2_prefill_usable(1, 1, 512, 2048, 24, 4, 256) == 0


def test_split_count_beyond_scratch_is_refused(rd4):
    """A requested split count whose records do not fit the library scratch is an
    error (RD4_EINVAL), not a silently smaller split; nothing is launched, so this
    runs without a GPU. Neither is a count above the kernels' maximum (256)."""
    L = rd4.lib()
    fake = ctypes.c_void_p(0x10000)
    # 256 heads x 256 splits: one token's records alone exceed the 64 MiB
    # scratch (more tokens than fit are run as consecutive token chunks instead)
    rc = L.rd4_attn_split_batch_launch(fake, fake, fake, fake, None, fake, 4, 256, 4, 256,
                                       ctypes.c_float(1 / 16), 2, 2, 256, None)
    assert rc == rd4.EINVAL
    assert b"exceed the library scratch" in L.rd4_last_error()
    rc = L.rd4_attn_launch_split(fake, fake, fake, fake, None, 100, 24, 4, 256, ctypes.c_float(1 / 16),
                                 2, 2, 300, None)
    assert rc == rd4.EINVAL and b"maximum" in L.rd4_last_error()
