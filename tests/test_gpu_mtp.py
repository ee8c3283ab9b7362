"""Multi-token decode: the MTP verify step (N = D+1 drafted tokens through
attn_split_batch_launch, graph.cuh:1494-1527) and the draft loop (append one row
then attend, mtp.cuh:578-604), on the GPU vs the f64 oracle and vs per-token
decode.

The reference's batched split kernel is bit-identical to its per-token split
kernel (same key assignment and merge order, graph.cuh:1486-1493). The same
holds here for rd4_attn_split_batch_launch: with a given split count each token
gets exactly the bytes of a single-token rd4_attn_decode. rd4_attn_decode_tokens
reads each K/V tile once for two tokens (f16 queries) and is held to the
attention tolerance.
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
        oi = torch.full_like(qi, float("nan"))  # unwritten elements stay NaN
        rd4.attn_decode(qi, kd, vd, oi, t0 + i, NH, NKV, HD, 1 / 16, kt, vt, n_splits=splits)
        outs.append(oi)
    torch.cuda.synchronize()
    return torch.cat(outs).cpu().numpy()


@pytest.mark.parametrize("kt,vt", [(2, 2), (1, 1), (4, 5), (3, 3), (0, 2)])
@pytest.mark.parametrize("n_tok", [2, 3, 4])
def test_tokens_vs_per_token_and_oracle(rd4, orc, dev, kt, vt, n_tok):
    """Split-batch (the reference entry) is bit-identical to per-token decode at
    the same split count. rd4_attn_decode_tokens may put two tokens in one CTA
    with f16 queries (pair mode), so it is held to the tolerance instead, against
    per-token decode and the oracle; odd n_tok leaves the last pair half full."""
    import torch
    print("mtp kt=%d vt=%d n_tok=%d" % (kt, vt, n_tok), flush=True)
    n = 3000
    k, v, kd, vd = _caches(orc, torch, dev, kt, vt, n, 300 + kt)
    t0 = n - n_tok
    q = orc.randn(n_tok * NH * HD, 310)
    qd = to_dev(q, torch, dev)
    splits = 6
    want = _per_token(rd4, torch, dev, qd, kd, vd, t0, n_tok, kt, vt, splits)
    pos = to_dev(np.arange(t0, n, dtype=np.int32), torch, dev)
    out2 = torch.full_like(qd, float("nan"))  # unwritten elements stay NaN
    rd4.attn_split_batch(qd, kd, vd, out2, pos, NH, NKV, HD, 1 / 16, kt, vt, splits)
    out = torch.full_like(qd, float("nan"))  # unwritten elements stay NaN
    rd4.attn_decode_tokens(qd, kd, vd, out, t0, n_tok, NH, NKV, HD, 1 / 16, kt, vt, n_splits=splits)
    torch.cuda.synchronize()
    assert np.array_equal(out2.cpu().numpy(), want)
    check_close(out.cpu().numpy(), want, "tokens vs per-token")
    ref = orc.attn_batch(q.reshape(n_tok, NH, HD), k, v, np.arange(t0, n, dtype=np.int32), NH, NKV,
                         HD, 1 / 16, kt, vt, threads=8)
    check_close(out.cpu().numpy(), ref, "tokens forced splits")
    rd4.attn_decode_tokens(qd, kd, vd, out, t0, n_tok, NH, NKV, HD, 1 / 16, kt, vt)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), ref, "tokens auto")


@pytest.mark.parametrize("kt,vt", [(2, 2), (1, 1)])
def test_tokens_split_with_only_the_last_key(rd4, orc, dev, kt, vt):
    """3009 keys in 189 splits of 16: the last split holds key 3008 only, which
    the first token of the pair (position 3007) must not see: its rows in that
    split have no key at all and must merge as empty."""
    import torch
    n, n_tok = 3009, 2
    k, v, kd, vd = _caches(orc, torch, dev, kt, vt, n, 320 + kt)
    q = orc.randn(n_tok * NH * HD, 330)
    out = torch.full((n_tok * NH * HD,), float("nan"), device=dev)
    rd4.attn_decode_tokens(to_dev(q, torch, dev), kd, vd, out, n - n_tok, n_tok, NH, NKV, HD, 1 / 16,
                           kt, vt, n_splits=189)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    ref = orc.attn_batch(q.reshape(n_tok, NH, HD), k, v, np.arange(n - n_tok, n, dtype=np.int32), NH,
                         NKV, HD, 1 / 16, kt, vt, threads=8)
    check_close(got, ref, "last-key split")


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
            out = torch.full((NH * HD,), float("nan"), device=dev)
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
    out = torch.full(((D + 1) * NH * HD,), float("nan"), device=dev)
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
    out = torch.full((n_tok * NH * HD,), float("nan"), device=dev)
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


@pytest.mark.parametrize("kt,vt", [(2, 2), (4, 5)])
def test_layer_verify_step_epilogue_then_tokens(rd4, orc, dev, kt, vt):
    """One full-attention layer of an MTP verify step, as graph.cuh:1444-1535
    runs it for a chunk: the fused epilogue writes q, the gate and the chunk's K/V
    rows, then the multi-token decode attends and gates. Checked against the
    oracle doing the same steps (deinterleave, RMSNorm, RoPE, quantize, f64
    attention, gate)."""
    import torch
    n0, n_tok, n_rot, eps, base = 1500, 4, 64, 1e-6, 10000000.0
    n = n0 + n_tok
    k, v, kd, vd = _caches(orc, torch, dev, kt, vt, n, 400)
    krb, vrb = orc.row_bytes(kt, HD), orc.row_bytes(vt, HD)
    qg = (orc.randn(n_tok * NH * 2 * HD, 410) * 2).astype(np.float32)
    kn = (orc.randn(n_tok * NKV * HD, 411) * 2).astype(np.float32)
    vn = orc.randn(n_tok * NKV * HD, 412).astype(np.float32)
    qw = (1 + 0.1 * orc.randn(HD, 413)).astype(np.float32)
    kw = (1 + 0.1 * orc.randn(HD, 414)).astype(np.float32)
    pos = np.arange(n0, n, dtype=np.int32)
    q_out = torch.empty(n_tok * NH * HD, device=dev)
    g_out = torch.empty_like(q_out)
    k_out = torch.empty(n_tok * NKV * HD, device=dev)
    rd4.qk_norm_rope_append(to_dev(qg, torch, dev), to_dev(kn, torch, dev), to_dev(vn, torch, dev),
                            to_dev(qw, torch, dev), to_dev(kw, torch, dev), eps, n_rot, base,
                            to_dev(pos, torch, dev), n_tok, NH, NKV, HD, q_out, kd, vd, kt, vt,
                            gate_out=g_out, k_out=k_out)
    out = torch.full_like(q_out, float("nan"))  # unwritten elements stay NaN
    rd4.attn_decode_tokens(q_out, kd, vd, out, n0, n_tok, NH, NKV, HD, 1 / 16, kt, vt, gate=g_out)
    torch.cuda.synchronize()
    # oracle pipeline on the host
    q3 = qg.reshape(n_tok, NH, 2, HD)
    q_ref = orc.rope(orc.rms_norm(q3[:, :, 0].ravel(), qw, HD, eps), n_tok, NH, HD, n_rot, base, pos)
    k_ref = orc.rope(orc.rms_norm(kn, kw, HD, eps), n_tok, NKV, HD, n_rot, base, pos).ravel()
    kc, vc = k.copy(), v.copy()
    kc[n0 * NKV * krb:] = orc.store_rows(kt, k_out.cpu().numpy())  # the GPU's own rows (bit-checked elsewhere)
    vc[n0 * NKV * vrb:] = orc.store_rows(vt, vn)
    assert np.array_equal(kd.cpu().numpy(), kc) and np.array_equal(vd.cpu().numpy(), vc)
    assert np.abs(k_out.cpu().numpy() - k_ref).max() < 1e-3
    att = orc.attn_batch(q_ref.reshape(n_tok, NH, HD), kc, vc, pos, NH, NKV, HD, 1 / 16, kt, vt, threads=8)
    _, want = orc.sigmoid_gate(q3[:, :, 1].ravel(), att.ravel())
    check_close(out.cpu().numpy(), want, "layer verify step")


def test_tokens_wide_group_takes_per_token_ctas(rd4, orc, dev):
    """GQA group 16 (two head chunks per kv head) cannot pair tokens in one
    16-row tile; the multi-token entry then runs one token per CTA and stays
    bit-identical to per-token decode at the same split count."""
    import torch
    nh, nkv, n, n_tok = 32, 2, 1200, 3
    k = make_cache(orc, 3, n, nkv, HD, 700)
    v = make_cache(orc, 3, n, nkv, HD, 701)
    kd, vd = to_dev(k, torch, dev), to_dev(v, torch, dev)
    q = orc.randn(n_tok * nh * HD, 702)
    qd = to_dev(q, torch, dev)
    out = torch.full_like(qd, float("nan"))  # unwritten elements stay NaN
    rd4.attn_decode_tokens(qd, kd, vd, out, n - n_tok, n_tok, nh, nkv, HD, 1 / 16, 3, 3, n_splits=5)
    per = []
    for i in range(n_tok):
        o = torch.full((nh * HD,), float("nan"), device=dev)
        rd4.attn_decode(qd[i * nh * HD:(i + 1) * nh * HD].clone(), kd, vd, o, n - n_tok + i, nh, nkv, HD,
                        1 / 16, 3, 3, n_splits=5)
        per.append(o)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), torch.cat(per).cpu().numpy())
    ref = orc.attn_batch(q.reshape(n_tok, nh, HD), k, v, np.arange(n - n_tok, n, dtype=np.int32), nh, nkv,
                         HD, 1 / 16, 3, 3, threads=8)
    check_close(out.cpu().numpy(), ref, "wide group")
