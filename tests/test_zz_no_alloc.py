"""The allocation-free decode entry point (rd4_attn_decode_append_noalloc)
against the entry point it mirrors (rd4_attn_decode_append): same kernels, its
split records in the library's fixed device array. Two calls in a row, the
second on a smaller input, each checked against the allocating entry point on
identical inputs and against the f64 oracle. Both entry points run the same
split kernel and the same merge launch, so at an explicit, equal split count
their outputs are bit-identical; with automatic counts the allocation-free one
may run fewer splits (its array is smaller), so the bar there is the attention
tolerance."""
import numpy as np
import pytest

from gpu_util import check_close, to_dev

pytestmark = pytest.mark.gpu
NH, NKV, HD = 24, 4, 256


def _case(rd4, orc, dev, kt, vt, n, seed, n_splits=0):
    import torch
    k = orc.store_rows(kt, orc.randn(n * NKV * HD, seed))
    v = orc.store_rows(vt, orc.randn(n * NKV * HD, seed + 1))
    q = orc.randn(NH * HD, seed + 2)
    g = orc.randn(NH * HD, seed + 3)
    kn, vn = orc.randn(NKV * HD, seed + 4), orc.randn(NKV * HD, seed + 5)
    res = []
    for fn in (rd4.attn_decode_append, rd4.attn_decode_append_noalloc):
        kd, vd = to_dev(k, torch, dev), to_dev(v, torch, dev)
        out = torch.full((NH * HD,), float("nan"), device=dev)
        gd = to_dev(g, torch, dev)
        fn(to_dev(q, torch, dev), to_dev(kn, torch, dev), to_dev(vn, torch, dev), kd, vd, out, n - 1, NH,
           NKV, HD, 1 / 16, kt, vt, gate=gd, n_splits=n_splits)
        torch.cuda.synchronize()
        res.append((out.cpu().numpy(), gd.cpu().numpy(), kd.cpu().numpy(), vd.cpu().numpy()))
    (o0, g0, k0, v0), (o1, g1, k1, v1) = res
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)  # the same appended rows
    check_close(o1, o0, "noalloc vs decode_append")
    if n_splits > 0:
        assert np.array_equal(o1, o0), "same kernels at the same split count: bit-identical"
    assert np.array_equal(g1, g0)
    # and against the oracle, on the caches with the appended row
    _, want = orc.sigmoid_gate(g, orc.attn_decode(q, k1, v1, n - 1, NH, NKV, HD, 1 / 16, kt, vt).ravel())
    check_close(o1, want, "noalloc vs oracle")
    return o0, o1


def test_noalloc_two_calls_second_smaller(rd4, orc, dev):
    import torch
    # a fresh stream: the allocating entry point would create that stream's
    # scratch on first use; the allocation-free one allocates nothing
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        _case(rd4, orc, dev, 2, 2, 8192, 300)                   # q8_0, 64 splits
        _case(rd4, orc, dev, 2, 2, 8192, 305, n_splits=32)      # the same split count on both
        _case(rd4, orc, dev, 1, 3, 700, 310)                    # smaller: f16 K / q4_0 V, 11 splits
        _case(rd4, orc, dev, 1, 3, 700, 315, n_splits=4)
        _case(rd4, orc, dev, 0, 0, 300, 320)                    # generic kernel, one split
        torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    s2 = torch.cuda.Stream()
    with torch.cuda.stream(s2):
        k = torch.zeros(2048 * NKV * 272, dtype=torch.uint8, device=dev)
        v = torch.zeros_like(k)
        q = torch.zeros(NH * HD, device=dev)
        out = torch.full_like(q, float("nan"))  # unwritten elements stay NaN
        kn = torch.zeros(NKV * HD, device=dev)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        rd4.attn_decode_append_noalloc(q, kn, kn, k, v, out, 2047, NH, NKV, HD, 1 / 16, 2, 2)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0


def test_noalloc_rejects_records_beyond_the_array(rd4, orc, dev):
    import torch
    k = torch.zeros(4096 * NKV * 272, dtype=torch.uint8, device=dev)
    q = torch.zeros(NH * HD, device=dev)
    kn = torch.zeros(NKV * HD, device=dev)
    out = torch.full_like(q, float("nan"))  # unwritten elements stay NaN
    # 24 heads x 256 splits x 258 floats > 1M floats
    with pytest.raises(rd4.Rd4Error, match="fixed scratch"):
        rd4.attn_decode_append_noalloc(q, kn, kn, k, k.clone(), out, 4095, NH, NKV, HD, 1 / 16, 2, 2,
                                       n_splits=256)
