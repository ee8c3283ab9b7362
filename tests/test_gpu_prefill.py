"""Causal prefill on the GPU vs the f64 CPU oracle (reference attn_fa2.cuh and
the batched path of graph.cuh:1473-1535)."""
import numpy as np
import pytest

from gpu_util import check_close, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("q_f16", [False, True])
def test_prefill_small(rd4, orc, dev, q_f16):
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 300, 200
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 1))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 2))
    q = orc.randn(nq * nh * hd, 3).reshape(nq, nh, hd)
    g = orc.randn(nq * nh * hd, 4)
    if q_f16:
        q = q.astype(np.float16).astype(np.float32)
    pos = np.arange(pos0, n, dtype=np.int32)
    att = orc.attn_batch(q, k, v, pos, nh, nkv, hd, 1 / 16, 1, 1)
    gs, want = orc.sigmoid_gate(g, att.ravel())
    qd = to_dev(q.astype(np.float16) if q_f16 else q, torch, dev)
    out = torch.empty(nq * nh * hd, dtype=torch.float32, device=dev)
    gd = to_dev(g, torch, dev)
    rd4.prefill(qd, to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv, hd, 1 / 16,
                1, 1, gate=gd)
    check_close(out.cpu().numpy(), want, "prefill")


def test_fa2_entry_point(rd4, orc, dev):
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 100, 64
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 5))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 6))
    q = orc.randn(nq * nh * hd, 7).reshape(nq, nh, hd)
    pos = np.arange(pos0, n, dtype=np.int32)
    want = orc.attn_batch(q, k, v, pos, nh, nkv, hd, 1 / 16, 1, 1)
    qd = to_dev(q, torch, dev)
    rd4.fa2_prefill(qd, to_dev(k, torch, dev), to_dev(v, torch, dev), qd, to_dev(pos, torch, dev),
                    n - 1, n, nh, nkv, hd, 1 / 16)
    check_close(qd.cpu().numpy(), want, "fa2 in-place")
