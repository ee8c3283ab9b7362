"""Seeded sweep over shapes the fixed-case tests do not name: decode over random
(K, V) pairs, GQA groups, context lengths, split counts and gates, and prefill
over random GQA groups, chunk positions and sizes, each against the f64 oracle
(tolerance max-abs 2e-3, mean-rel 1e-3). The cases are fixed by the seed, so a
failure names a reproducible case."""
import numpy as np
import pytest

from gpu_util import check_close, to_dev
from test_gpu_attn import make_cache, run_decode

pytestmark = pytest.mark.gpu

GQA = [(24, 4), (16, 2), (8, 8), (12, 3), (32, 8), (6, 1)]


def _decode_cases(n=12, seed=2024):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        nh, nkv = GQA[r.integers(len(GQA))]
        out.append((i, nh, nkv, int(r.integers(0, 6)), int(r.integers(0, 6)), int(r.integers(1, 9000)),
                    int(r.choice([0, 1, 2, 7, 33, 64])), bool(r.integers(2))))
    return out


@pytest.mark.parametrize("i,nh,nkv,kt,vt,n,splits,gated", _decode_cases())
def test_decode_sweep(rd4, orc, dev, i, nh, nkv, kt, vt, n, splits, gated):
    import torch
    hd = 256
    k = make_cache(orc, kt, n, nkv, hd, 700 + 3 * i)
    v = make_cache(orc, vt, n, nkv, hd, 701 + 3 * i)
    q = orc.randn(nh * hd, 702 + 3 * i)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, vt, threads=8)
    g = orc.randn(nh * hd, 900 + i) if gated else None
    got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, vt, gate=g, n_splits=splits)
    if gated:
        _, want = orc.sigmoid_gate(g, want.ravel())
    check_close(got.ravel(), np.asarray(want).ravel(), "decode case %d" % i)


def _prefill_cases(n=8, seed=77):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        nh, nkv = GQA[r.integers(len(GQA))]
        out.append((i, nh, nkv, int(r.integers(0, 3000)), int(r.integers(1, 700)), bool(r.integers(2)),
                    bool(r.integers(2))))
    return out


@pytest.mark.parametrize("i,nh,nkv,pos0,nq,q_f16,gated", _prefill_cases())
def test_prefill_sweep(rd4, orc, dev, i, nh, nkv, pos0, nq, q_f16, gated):
    import torch
    hd = 256
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 800 + 4 * i))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 801 + 4 * i))
    q = orc.randn(nq * nh * hd, 802 + 4 * i).reshape(nq, nh, hd)
    if q_f16:
        q = q.astype(np.float16).astype(np.float32)
    # every row when the chunk is small, else a stratified sample
    rows = np.arange(nq, dtype=np.int32) if nq <= 96 else np.unique(np.linspace(0, nq - 1, 96).astype(np.int32))
    want = orc.attn_batch(q[rows], k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1, threads=8)
    g = orc.randn(nq * nh * hd, 803 + 4 * i).reshape(nq, nh, hd)
    if gated:
        _, want = orc.sigmoid_gate(g[rows], want)
    qd = to_dev(q.astype(np.float16) if q_f16 else q, torch, dev)
    out = torch.empty((nq, nh, hd), dtype=torch.float32, device=dev)
    rd4.prefill(qd, to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv, hd, 1 / 16, 1, 1,
                gate=to_dev(g, torch, dev) if gated else None)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy()[rows].ravel(), np.asarray(want).ravel(), "prefill case %d" % i)
