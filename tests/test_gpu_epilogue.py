"""Pre-attention epilogue on the GPU: rms_norm (nn.cuh:24-63,239) and the fused
deinterleave + q/k RMSNorm + RoPE + K/V append (graph.cuh:914-954, 1444-1462).

Two bars:
  - bit-exact against the unfused sequence of this library's own launches (the
    reference's six launches: torch slicing stands in for deinterleave, which only
    moves floats), for q, gate, k and every cache byte;
  - against the CPU oracle: rms_norm within 4 ulp (the device rsqrtf is within
    1 ulp of the oracle's correctly rounded 1/sqrt), rotated q/k pairs within two
    ulp of their f32 angle (powf's last bit), and cache bytes equal to the oracle's
    quantization of the GPU's own k/v rows.
"""
import numpy as np
import pytest

from gpu_util import to_dev

pytestmark = pytest.mark.gpu


def _ulps(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    return np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))


@pytest.mark.parametrize("rows,ncols,use_w", [(24, 256, True), (4, 256, False), (3, 64, True),
                                              (2, 512, True), (5, 1000, True), (1, 5120, True),
                                              (7, 300, False)])
def test_rms_norm_kernel(rd4, orc, dev, rows, ncols, use_w):
    import torch
    print("rms_norm rows=%d ncols=%d w=%d" % (rows, ncols, use_w), flush=True)
    x = (orc.randn(rows * ncols, 11 * ncols + rows) * 3).astype(np.float32)
    w = orc.randn(ncols, ncols + 5) if use_w else None
    want = orc.rms_norm(x, w, ncols, 1e-6)
    xd = to_dev(x, torch, dev)
    wd = to_dev(w, torch, dev) if use_w else None
    yd = torch.empty_like(xd)
    rd4.rms_norm(xd, wd, yd, rows, ncols, 1e-6)
    rd4.rms_norm(xd, wd, xd, rows, ncols, 1e-6)  # in place, like graph.cuh:918
    torch.cuda.synchronize()
    got = yd.cpu().numpy()
    assert np.array_equal(got, xd.cpu().numpy())
    # y = (x * scale) * w: a 1-ulp scale plus two roundings, each measured in the
    # result's own binade, stays within 4 ulp of the oracle
    assert _ulps(got, want).max() <= 4


def test_rms_norm_tree_order_gpu(rd4, orc, dev):
    """The crafted row whose sum depends on the reference's fmaf chains and halving
    tree (see the oracle test): the GPU's scale lands within 1 ulp of the oracle's
    and 10+ ulp away from the 128-partial and sequential orders."""
    import torch
    n = 5120
    x = np.ones(n, np.float32)
    x[0] = 4096.0
    xd = to_dev(x, torch, dev)
    rd4.rms_norm(xd, None, xd, 1, n, 0.0)
    got = xd.cpu().numpy()
    assert _ulps(got[1:2], orc.rms_norm(x, None, n, 0.0)[1:2]).max() <= 1


CASES = [
    # (kt, vt, head_dim, n_head, n_head_kv, n_rot, n_tok, pos0)
    (1, 1, 256, 24, 4, 64, 1, 300),       # decode, Qwen3.5 shape, f16 cache
    (2, 2, 256, 24, 4, 64, 1, 4095),      # decode, q8_0
    (2, 2, 256, 24, 4, 64, 7, 1000),      # chunk of 7 tokens
    (3, 3, 256, 16, 2, 256, 3, 17),       # q4_0, full rotary
    (4, 5, 128, 8, 2, 128, 5, 64),        # q5_0 / q4_1
    (0, 2, 512, 4, 1, 64, 2, 9),          # f32 K, head_dim 512
    (5, 4, 64, 8, 8, 32, 4, 0),           # MHA, head_dim 64
    (2, 3, 256, 24, 4, 0, 2, 50),         # n_rot 0: no rotation
]


def _inputs(orc, kt, vt, hd, nh, nkv, n_tok, seed):
    qg = orc.randn(n_tok * nh * 2 * hd, seed) * 2
    k = orc.randn(n_tok * nkv * hd, seed + 1) * 2
    v = orc.randn(n_tok * nkv * hd, seed + 2)
    qw = 1.0 + 0.1 * orc.randn(hd, seed + 3)
    kw = 1.0 + 0.1 * orc.randn(hd, seed + 4)
    return [a.astype(np.float32) for a in (qg, k, v, qw, kw)]


def _check_normed_rotated(got, want, hd, n_rot, pos, base):
    """Dims past n_rot are only normed: within 4 ulp (rsqrtf). A rotated pair carries
    the f32 angle pos * powf(base, -2p/n_rot), whose last bit may differ between the
    device and host powf: the pair's error is bounded by its norm times two ulp of
    that angle, plus 1e-6 for the norm, cos and sin roundings."""
    got = got.reshape(len(pos), -1, hd).astype(np.float64)
    want = want.reshape(len(pos), -1, hd).astype(np.float64)
    if n_rot < hd:
        assert _ulps(got[..., n_rot:].astype(np.float32), want[..., n_rot:].astype(np.float32)).max() <= 4
    half = n_rot // 2
    if not half:
        return
    p = np.arange(half)
    theta = np.float32(pos)[:, None] * np.float32(base) ** (-2.0 * p / n_rot)
    tol = 2 * np.spacing(np.abs(theta).astype(np.float32)).astype(np.float64) + 1e-6  # [tok][p]
    err = np.hypot(got[..., :half] - want[..., :half], got[..., half:n_rot] - want[..., half:n_rot])
    norm = np.hypot(want[..., :half], want[..., half:n_rot])
    assert np.all(err <= tol[:, None, :] * norm + 1e-6)


@pytest.mark.parametrize("case", CASES)
def test_epilogue_matches_unfused_and_oracle(rd4, orc, dev, case):
    import torch
    kt, vt, hd, nh, nkv, n_rot, n_tok, pos0 = case
    print("epilogue case %s" % (case,), flush=True)
    eps, base = 1e-6, 10000000.0
    qg, k, v, qw, kw = _inputs(orc, kt, vt, hd, nh, nkv, n_tok, 97 + hd + n_tok)
    pos = np.arange(pos0, pos0 + n_tok, dtype=np.int32)
    n_rows = (pos0 + n_tok + 3) * nkv
    krb, vrb = orc.row_bytes(kt, hd), orc.row_bytes(vt, hd)
    fill = np.random.default_rng(5).integers(0, 256, n_rows * max(krb, vrb), dtype=np.uint8)

    qgd, kd, vd, qwd, kwd, posd = (to_dev(a, torch, dev) for a in (qg, k, v, qw, kw, pos))
    # fused
    kc = to_dev(fill[:n_rows * krb], torch, dev)
    vc = to_dev(fill[:n_rows * vrb], torch, dev)
    q_out = torch.empty(n_tok * nh * hd, dtype=torch.float32, device=dev)
    g_out = torch.empty_like(q_out)
    k_out = torch.empty_like(kd)
    rd4.qk_norm_rope_append(qgd, kd, vd, qwd, kwd, eps, n_rot, base, posd, n_tok, nh, nkv, hd,
                            q_out, kc, vc, kt, vt, gate_out=g_out, k_out=k_out)
    # unfused: deinterleave, rms_norm x2, rope x2, kv_store x2 (graph.cuh:914-954)
    kc2 = to_dev(fill[:n_rows * krb], torch, dev)
    vc2 = to_dev(fill[:n_rows * vrb], torch, dev)
    qg3 = qgd.view(n_tok, nh, 2, hd)
    q2 = qg3[:, :, 0].contiguous().view(-1)
    g2 = qg3[:, :, 1].contiguous().view(-1)
    k2 = kd.clone()
    rd4.rms_norm(q2, qwd, q2, n_tok * nh, hd, eps)
    rd4.rms_norm(k2, kwd, k2, n_tok * nkv, hd, eps)
    if n_rot:
        rd4.rope(q2, n_tok, nh, hd, n_rot, base, posd)
        rd4.rope(k2, n_tok, nkv, hd, n_rot, base, posd)
    w = n_tok * nkv * hd
    rd4.kv_store_rows(kt, k2, kc2[pos0 * nkv * krb:], w)
    rd4.kv_store_rows(vt, vd, vc2[pos0 * nkv * vrb:], w)
    torch.cuda.synchronize()

    got = {n: t.cpu().numpy() for n, t in (("q", q_out), ("gate", g_out), ("k", k_out),
                                            ("kc", kc), ("vc", vc))}
    ref = {n: t.cpu().numpy() for n, t in (("q", q2), ("gate", g2), ("k", k2), ("kc", kc2),
                                            ("vc", vc2))}
    for n in got:
        bad = np.nonzero(got[n].view(np.uint8) != ref[n].view(np.uint8))[0]
        assert bad.size == 0, "%s: %d bytes differ from the unfused sequence" % (n, bad.size)

    # oracle: deinterleave, rms_norm, rope in f32/f64
    q3 = qg.reshape(n_tok, nh, 2, hd)
    q_want = orc.rms_norm(q3[:, :, 0].ravel(), qw, hd, eps)
    k_want = orc.rms_norm(k, kw, hd, eps)
    if n_rot:
        q_want = orc.rope(q_want, n_tok, nh, hd, n_rot, base, pos).ravel()
        k_want = orc.rope(k_want, n_tok, nkv, hd, n_rot, base, pos).ravel()
    assert np.array_equal(got["gate"], q3[:, :, 1].ravel())
    _check_normed_rotated(got["q"], q_want, hd, n_rot, pos, base)
    _check_normed_rotated(got["k"], k_want, hd, n_rot, pos, base)
    # cache bytes: rows pos0.. hold the oracle's quantization of the GPU's k and v;
    # every other row keeps its old bytes
    a, b = pos0 * nkv, (pos0 + n_tok) * nkv
    assert np.array_equal(got["kc"][a * krb:b * krb], orc.store_rows(kt, got["k"]))
    assert np.array_equal(got["vc"][a * vrb:b * vrb], orc.store_rows(vt, v))
    assert np.array_equal(got["kc"][:a * krb], fill[:a * krb])
    assert np.array_equal(got["kc"][b * krb:], fill[b * krb:n_rows * krb])
    assert np.array_equal(got["vc"][b * vrb:], fill[b * vrb:n_rows * vrb])


def test_epilogue_in_place_k_no_weights(rd4, orc, dev):
    """k_out == k_new (in place), no norm weights, no gate output."""
    import torch
    hd, nh, nkv, n_tok = 256, 24, 4, 2
    qg, k, v, _, _ = _inputs(orc, 2, 2, hd, nh, nkv, n_tok, 5)
    pos = np.int32([40, 41])
    qgd, kd, vd, posd = (to_dev(a, torch, dev) for a in (qg, k, v, pos))
    rb = orc.row_bytes(2, hd)
    kc = torch.zeros(50 * nkv * rb, dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    q_out = torch.empty(n_tok * nh * hd, dtype=torch.float32, device=dev)
    rd4.qk_norm_rope_append(qgd, kd, vd, None, None, 1e-6, 64, 10000.0, posd, n_tok, nh, nkv, hd,
                            q_out, kc, vc, 2, 2, k_out=kd)
    torch.cuda.synchronize()
    k_want = orc.rope(orc.rms_norm(k, None, hd, 1e-6), n_tok, nkv, hd, 64, 10000.0, pos).ravel()
    got_k = kd.cpu().numpy()
    _check_normed_rotated(got_k, k_want, hd, 64, pos, 10000.0)
    assert np.array_equal(kc.cpu().numpy()[40 * nkv * rb:42 * nkv * rb], orc.store_rows(2, got_k))


def test_epilogue_rejects_bad_shapes(rd4, dev):
    import torch
    x = torch.zeros(4096, dtype=torch.float32, device=dev)
    c = torch.zeros(4096, dtype=torch.uint8, device=dev)
    p = torch.zeros(1, dtype=torch.int32, device=dev)
    for hd, n_rot, kt in ((96, 64, 2), (256, 63, 2), (256, 512, 2), (256, 64, 9)):
        with pytest.raises(rd4.Rd4Error):
            rd4.qk_norm_rope_append(x, x, x, None, None, 1e-6, n_rot, 1e4, p, 1, 2, 1, hd, x, c,
                                    c, kt, 2)
    with pytest.raises(rd4.Rd4Error):  # misaligned f32 buffer
        rd4.qk_norm_rope_append(x[1:], x, x, None, None, 1e-6, 64, 1e4, p, 1, 2, 1, 256, x, c, c,
                                2, 2)
