"""Multi-token decode: the MTP verify step (N = D+1 drafted tokens through
attn_split_batch_launch, graph.cuh:1494-1527) and the draft loop (append one row
then attend, mtp.cuh:578-604), on the GPU vs the f64 oracle and vs per-token
decode.

The reference's batched split kernel is bit-identical to its per-token split
kernel (same key assignment and merge order, graph.cuh:1486-1493). The same
holds here: rd4_attn_split_batch_launch and rd4_attn_decode_tokens with a given
split count give each token exactly the bytes of a single-token rd4_attn_decode
with that split count.
"""
import numpy as np
import pytest

from gpu_util import check_close, to_dev
from test_gpu_attn import make_cache

pytestmark = pytest.mark.gpu
NH, NKV, HD = 24, 4, 256


def _caches(orc, torch, dev, kt, vt, n, seed):
    k = make_cache(orc, kt, n, NKV, HD, seed, outlier=(kt == 2))
    v = make_cache(orc, vt, n, NKV, HD, seed + 1)
    return k, v, to_dev(k, torch, dev), to_dev(v, torch, dev)


def _per_token(rd4, torch, dev, qd, kd, vd, t0, n_tok, kt, vt, splits):
    outs = []
    for i in range(n_tok):
        qi = qd[i * NH * HD:(i + 1) * NH * HD].clone()
        oi = torch.empty_like(qi)
        rd4.attn_decode(qi, kd, vd, oi, t0 + i, NH, NKV, HD, 1 / 16, kt, vt, n_splits=splits)
        outs.append(oi)
    torch.cuda.synchronize()
    return torch.cat(outs).cpu().numpy()


@pytest.mark.parametrize("kt,vt", [(2, 2), (1, 1), (4, 5), (3, 3), (0, 2)])
@pytest.mark.parametrize("n_tok", [2, 4])
def test_tokens_bit_identical_to_per_token(rd4, orc, dev, kt, vt, n_tok):
    import torch
    print("mtp bit-identity kt=%d vt=%d n_tok=%d" % (kt, vt, n_tok), flush=True)
    n = 3000
    k, v, kd, vd = _caches(orc, torch, dev, kt, vt, n, 300 + kt)
    t0 = n - n_tok
    q = orc.randn(n_tok * NH * HD, 310)
    qd = to_dev(q, torch, dev)
    splits = 6
    want = _per_token(rd4, torch, dev, qd, kd, vd, t0, n_tok, kt, vt, splits)
    out = torch.empty_like(qd)
    rd4.attn_decode_tokens(qd, kd, vd, out, t0, n_tok, NH, NKV, HD, 1 / 16, kt, vt, n_splits=splits)
    pos = to_dev(np.arange(t0, n, dtype=np.int32), torch, dev)
    out2 = torch.empty_like(qd)
    rd4.attn_split_batch(qd, kd, vd, out2, pos, NH, NKV, HD, 1 / 16, kt, vt, splits)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), want)
    assert np.array_equal(out2.cpu().numpy(), want)
    # and the automatic split count against the oracle
    rd4.attn_decode_tokens(qd, kd, vd, out, t0, n_tok, NH, NKV, HD, 1 / 16, kt, vt)
    torch.cuda.synchronize()
    ref = orc.attn_batch(q.reshape(n_tok, NH, HD), k, v, np.arange(t0, n, dtype=np.int32), NH, NKV,
                         HD, 1 / 16, kt, vt, threads=8)
    check_close(out.cpu().numpy(), ref, "tokens auto")


@pytest.mark.parametrize("kt,vt", [(2, 2), (4, 5)])
def test_draft_then_verify(rd4, orc, dev, kt, vt):
    """D = 3 draft tokens, each appended then attended (gated) one at a time, then
    the verify step over the D + 1 positions in one launch; every output vs the
    oracle on the cache the appends produced."""
    import torch
    D, n0 = 3, 2500
    n = n0 + D + 1
    k, v, kd, vd = _caches(orc, torch, dev, kt, vt, n, 320)
    krb, vrb = orc.row_bytes(kt, HD), orc.row_bytes(vt, HD)
    k_ref, v_ref = k.copy(), v.copy()
    for i in range(D + 1):  # rows the drafts and the verify's last token append
        kn, vn = orc.randn(NKV * HD, 330 + i), orc.randn(NKV * HD, 340 + i)
        r = n0 + i
        k_ref[r * NKV * krb:(r + 1) * NKV * krb] = orc.store_rows(kt, kn)
        v_ref[r * NKV * vrb:(r + 1) * NKV * vrb] = orc.store_rows(vt, vn)
        if i < D:
            q = orc.randn(NH * HD, 350 + i)
            g = orc.randn(NH * HD, 360 + i)
            out = torch.empty(NH * HD, device=dev)
            gd = to_dev(g, torch, dev)
            rd4.attn_decode_append(to_dev(q, torch, dev), to_dev(kn, torch, dev), to_dev(vn, torch, dev),
                                   kd, vd, out, r, NH, NKV, HD, 1 / 16, kt, vt, gate=gd)
            torch.cuda.synchronize()
            _, want = orc.sigmoid_gate(g, orc.attn_decode(q, k_ref, v_ref, r, NH, NKV, HD, 1 / 16, kt, vt,
                                                          threads=8).ravel())
            check_close(out.cpu().numpy(), want, "draft %d" % i)
        else:
            rd4.kv_store_rows(kt, to_dev(kn, torch, dev), kd[r * NKV * krb:])
            rd4.kv_store_rows(vt, to_dev(vn, torch, dev), vd[r * NKV * vrb:])
    assert np.array_equal(kd.cpu().numpy(), k_ref) and np.array_equal(vd.cpu().numpy(), v_ref)
    q = orc.randn((D + 1) * NH * HD, 370)
    g = orc.randn((D + 1) * NH * HD, 371)
    out = torch.empty((D + 1) * NH * HD, device=dev)
    gd = to_dev(g, torch, dev)
    rd4.attn_decode_tokens(to_dev(q, torch, dev), kd, vd, out, n0, D + 1, NH, NKV, HD, 1 / 16, kt, vt,
                           gate=gd)
    torch.cuda.synchronize()
    att = orc.attn_batch(q.reshape(D + 1, NH, HD), k_ref, v_ref, np.arange(n0, n, dtype=np.int32),
                         NH, NKV, HD, 1 / 16, kt, vt, threads=8)
    gs, want = orc.sigmoid_gate(g, att.ravel())
    check_close(out.cpu().numpy(), want, "verify")
    assert np.allclose(gd.cpu().numpy(), gs, rtol=1e-6, atol=1e-7)


def test_verify_full_size_q8_0_32k(rd4, orc, dev):
    """The verify step at the headline shape: 4 tokens ending at key 32767, q8_0."""
    import torch
    n, n_tok = 32768, 4
    k, v, kd, vd = _caches(orc, torch, dev, 2, 2, n, 380)
    q = orc.randn(n_tok * NH * HD, 390)
    out = torch.empty(n_tok * NH * HD, device=dev)
    rd4.attn_decode_tokens(to_dev(q, torch, dev), kd, vd, out, n - n_tok, n_tok, NH, NKV, HD, 1 / 16,
                           2, 2)
    torch.cuda.synchronize()
    ref = orc.attn_batch(q.reshape(n_tok, NH, HD), k, v, np.arange(n - n_tok, n, dtype=np.int32), NH,
                         NKV, HD, 1 / 16, 2, 2, threads=8)
    check_close(out.cpu().numpy(), ref, "verify 32k")


def test_tokens_rejects_bad_arguments(rd4, dev):
    import torch
    x = torch.zeros(NH * HD, device=dev)
    c = torch.zeros(64 * NKV * 512, dtype=torch.uint8, device=dev)
    for t0, n_tok, splits in ((-1, 1, 0), (0, 0, 0), (5, 1, -1)):
        with pytest.raises(rd4.Rd4Error):
            rd4.attn_decode_tokens(x, c, c, x, t0, n_tok, NH, NKV, HD, 1 / 16, 1, 1, n_splits=splits)
