"""The decode and epilogue entry points captured in a HIP graph (the way a
serving loop replays one step) give the eager results on every replay.

rd4_init() creates the library scratch before capture, so nothing is allocated
inside it, and no entry point records a memset. Replays are separated by eager
work (resetting the gate logits, a copy) and synchronizations, and each one is
compared with the eager launch on the same inputs.
"""
import numpy as np
import pytest

from gpu_util import to_dev
from test_gpu_attn import make_cache

pytestmark = pytest.mark.gpu
NH, NKV, HD = 24, 4, 256


def _eager_vs_graph(torch, run, outs, reset, replays=4):
    """run() enqueues the step on the current stream; reset() restores the inputs
    the step modifies; outs are the tensors compared."""
    reset()
    run()
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        reset()
        run()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        run()
    for i in range(replays):
        for o in outs:
            o.fill_(float("nan") if o.is_floating_point() else 0)
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w), "replay %d differs from the eager launch" % i


@pytest.mark.parametrize("kt", [2, 4])
def test_decode_append_in_graph(rd4, orc, dev, kt):
    import torch
    assert rd4.lib().rd4_init() == 0
    n = 4096
    vt = 5 if kt == 4 else kt
    kc = to_dev(make_cache(orc, kt, n, NKV, HD, 600), torch, dev)
    vc = to_dev(make_cache(orc, vt, n, NKV, HD, 601), torch, dev)
    q = to_dev(orc.randn(NH * HD, 602), torch, dev)
    g0 = to_dev(orc.randn(NH * HD, 603), torch, dev)
    gate = g0.clone()
    kn, vn = to_dev(orc.randn(NKV * HD, 604), torch, dev), to_dev(orc.randn(NKV * HD, 605), torch, dev)
    out = torch.full((NH * HD,), float("nan"), device=dev)

    def run():
        rd4.attn_decode_append(q, kn, vn, kc, vc, out, n - 1, NH, NKV, HD, 1 / 16, kt, vt, gate=gate)

    _eager_vs_graph(torch, run, [out, gate], lambda: gate.copy_(g0))


def test_decode_tokens_in_graph(rd4, orc, dev):
    import torch
    assert rd4.lib().rd4_init() == 0
    n, n_tok = 3000, 3
    kc = to_dev(make_cache(orc, 2, n, NKV, HD, 610), torch, dev)
    vc = to_dev(make_cache(orc, 2, n, NKV, HD, 611), torch, dev)
    q = to_dev(orc.randn(n_tok * NH * HD, 612), torch, dev)
    g0 = to_dev(orc.randn(n_tok * NH * HD, 613), torch, dev)
    gate = g0.clone()
    out = torch.full((n_tok * NH * HD,), float("nan"), device=dev)

    def run():
        rd4.attn_decode_tokens(q, kc, vc, out, n - n_tok, n_tok, NH, NKV, HD, 1 / 16, 2, 2, gate=gate)

    _eager_vs_graph(torch, run, [out, gate], lambda: gate.copy_(g0))


def test_epilogue_then_decode_in_graph(rd4, orc, dev):
    """One decode layer step as a serving loop would capture it: the fused
    epilogue (q/k norm, RoPE, append) then the gated decode over keys 0..t."""
    import torch
    assert rd4.lib().rd4_init() == 0
    n = 2048
    t = n - 1
    kc = to_dev(make_cache(orc, 2, n, NKV, HD, 620), torch, dev)
    vc = to_dev(make_cache(orc, 2, n, NKV, HD, 621), torch, dev)
    qg = to_dev(orc.randn(NH * 2 * HD, 622), torch, dev)
    kn, vn = to_dev(orc.randn(NKV * HD, 623), torch, dev), to_dev(orc.randn(NKV * HD, 624), torch, dev)
    qw = to_dev((1 + 0.1 * orc.randn(HD, 625)).astype(np.float32), torch, dev)
    kw = to_dev((1 + 0.1 * orc.randn(HD, 626)).astype(np.float32), torch, dev)
    pos = to_dev(np.int32([t]), torch, dev)
    q = torch.empty(NH * HD, device=dev)
    gate = torch.empty_like(q)
    out = torch.full_like(q, float("nan"))  # unwritten elements stay NaN

    def run():
        rd4.qk_norm_rope_append(qg, kn, vn, qw, kw, 1e-6, 64, 1e7, pos, 1, NH, NKV, HD, q, kc, vc, 2, 2,
                                gate_out=gate)
        rd4.attn_decode(q, kc, vc, out, t, NH, NKV, HD, 1 / 16, 2, 2, gate=gate)

    _eager_vs_graph(torch, run, [out, gate, q], lambda: None)


def test_prefill_key_splits_in_graph(rd4, orc, dev):
    """A 512-query prefill_append call (key splits + merge launch, records in the
    stream's library scratch) captured on a stream given its scratch by
    rd4_stream_init: every replay equals the eager call on that stream."""
    import ctypes
    import torch
    nh, nkv, hd, pos0, nq = NH, NKV, HD, 4096, 512
    n = pos0 + nq
    k = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 701)), torch, dev)
    v = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 702)), torch, dev)
    q = to_dev(orc.randn(nq * nh * hd, 703).reshape(nq, nh, hd).astype(np.float16), torch, dev)
    g0 = to_dev(orc.randn(nq * nh * hd, 704).reshape(nq, nh, hd), torch, dev)
    kn = to_dev(orc.randn(nq * nkv * hd, 705).reshape(nq, nkv, hd), torch, dev)
    vn = to_dev(orc.randn(nq * nkv * hd, 706).reshape(nq, nkv, hd), torch, dev)
    rb = rd4.kv_row_bytes(2, hd)
    kq8 = torch.zeros(nq * nkv * rb, dtype=torch.uint8, device=dev)
    vq8 = torch.zeros_like(kq8)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    gate = g0.clone()
    s = torch.cuda.Stream()
    assert rd4.lib().rd4_stream_init(ctypes.c_void_p(s.cuda_stream)) == 0

    def run():
        rd4.prefill_append(q, k, v, out, pos0, nh, nkv, hd, 1 / 16, 1, 1, kn, vn, kq8, vq8, 2, gate=gate)

    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gate.copy_(g0)
        run()
    s.synchronize()
    want = [out.clone(), gate.clone(), kq8.clone(), vq8.clone()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run()
    for i in range(3):
        out.fill_(float("nan"))
        kq8.zero_()
        vq8.zero_()
        gate.copy_(g0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip((out, gate, kq8, vq8), want):
            assert torch.equal(o, w), "replay %d differs from the eager call" % i
