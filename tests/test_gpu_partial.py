"""Caller-owned split records and per-stream scratch (attn.cuh:593-608,
665-667; graph.cuh:771-778): a caller that gives two streams two `partial`
buffers, or runs the native entry points on two streams, gets race-free
results."""
import numpy as np
import pytest

from gpu_util import check_close, to_dev

pytestmark = pytest.mark.gpu

NH, NKV, HD = 24, 4, 256


def problem(orc, kt, n, seed):
    k = orc.store_rows(kt, orc.randn(n * NKV * HD, seed))
    v = orc.store_rows(kt, orc.randn(n * NKV * HD, seed + 1))
    q = orc.randn(NH * HD, seed + 2)
    return q, k, v, orc.attn_decode(q, k, v, n - 1, NH, NKV, HD, 1 / 16, kt, kt).ravel()


def test_caller_partial_receives_the_records(rd4, orc, dev):
    """With n_splits at least the library's own count (64 at 4096 keys), the split
    records land in the caller's partial: its first n_head * S * (2 + hd) floats
    are overwritten, the rest of it is left alone."""
    import torch
    n, S = 4096, 64
    q, k, v, want = problem(orc, 2, n, 40)
    nbytes = rd4.attn_partial_bytes(NH, HD, S)
    assert nbytes == NH * S * (2 + HD) * 4
    part = torch.full((nbytes // 4 + 64,), float("nan"), dtype=torch.float32, device=dev)
    out = torch.full((NH * HD,), float("nan"), dtype=torch.float32, device=dev)
    rd4.attn_launch_split(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out, part,
                          n - 1, NH, NKV, HD, 1 / 16, 2, 2, S)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), want, "caller partial")
    p = part.cpu().numpy()
    assert np.isfinite(p[: NH * S * HD]).all()        # acc records
    ml = p[NH * S * HD: NH * S * (HD + 2)].reshape(NH, S, 2)
    assert np.isfinite(ml).all() and (ml[:, :, 1] > 0).all()  # every split holds 64 keys
    assert np.isnan(p[nbytes // 4:]).all()            # nothing past attn_partial_bytes


@pytest.mark.parametrize("mode", ["caller_partial", "library_scratch", "native"])
def test_two_streams_race_free(rd4, orc, dev, mode):
    """Two different decodes launched alternately on two streams, 12 times each
    with no synchronisation between them; every output matches its oracle."""
    import torch
    n = 4096
    probs = [problem(orc, 2, n, 50), problem(orc, 3, n, 60)]
    types = [2, 3]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    dq = [(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev)) for q, k, v, _ in probs]
    # caller_partial: n_splits 64 (records fit the caller's buffer); library_scratch:
    # n_splits 2 (the library runs 64, so each stream's own scratch holds them)
    S = 64 if mode == "caller_partial" else 2
    parts = [torch.empty(rd4.attn_partial_bytes(NH, HD, S) // 4, device=dev) for _ in range(2)]
    outs = [[torch.full((NH * HD,), float("nan"), device=dev) for _ in range(12)] for _ in range(2)]
    torch.cuda.synchronize()
    for it in range(12):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                q, k, v = dq[i]
                if mode == "native":
                    rd4.attn_decode(q, k, v, outs[i][it], n - 1, NH, NKV, HD, 1 / 16, types[i], types[i])
                else:
                    rd4.attn_launch_split(q, k, v, outs[i][it], parts[i], n - 1, NH, NKV, HD, 1 / 16,
                                          types[i], types[i], S)
    torch.cuda.synchronize()
    for i in range(2):
        for it in range(12):
            check_close(outs[i][it].cpu().numpy(), probs[i][3], "%s stream %d iter %d" % (mode, i, it))


def test_split_batch_caller_partial(rd4, orc, dev):
    """attn_split_batch_launch with the caller's [n_tok] x attn_partial_bytes buffer."""
    import torch
    n, ntok, S = 600, 5, 4
    k = orc.store_rows(1, orc.randn(n * NKV * HD, 70))
    v = orc.store_rows(1, orc.randn(n * NKV * HD, 71))
    q = orc.randn(ntok * NH * HD, 72).reshape(ntok, NH, HD)
    pos = np.int32([100, 250, 400, 598, 599])
    want = orc.attn_batch(q, k, v, pos, NH, NKV, HD, 1 / 16, 1, 1)
    part = torch.full((ntok * rd4.attn_partial_bytes(NH, HD, S) // 4,), float("nan"), device=dev)
    out = torch.full((ntok * NH * HD,), float("nan"), device=dev)
    rd4.attn_split_batch(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out,
                         to_dev(pos, torch, dev), NH, NKV, HD, 1 / 16, 1, 1, S, partial=part)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), want, "split batch, caller partial")
    assert np.isfinite(part.cpu().numpy()).all()


@pytest.mark.parametrize("kt", [0, 2])
def test_split_batch_token_chunks(rd4, orc, dev, kt):
    """40 tokens x 256 splits: the records of all tokens exceed the stream's
    64 MiB scratch, so the library runs consecutive token chunks; every token
    still matches the oracle (f32 caches take the generic kernel, q8_0 the MFMA
    one)."""
    import torch
    n, ntok, S = 600, 40, 256
    k = orc.store_rows(kt, orc.randn(n * NKV * HD, 90))
    v = orc.store_rows(kt, orc.randn(n * NKV * HD, 91))
    q = orc.randn(ntok * NH * HD, 92).reshape(ntok, NH, HD)
    pos = np.int32(np.random.default_rng(3).integers(100, n, ntok))
    want = orc.attn_batch(q, k, v, pos, NH, NKV, HD, 1 / 16, kt, kt, threads=8)
    out = torch.full((ntok * NH * HD,), float("nan"), device=dev)
    rd4.attn_split_batch(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out,
                         to_dev(pos, torch, dev), NH, NKV, HD, 1 / 16, kt, kt, S)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), want, "token chunks")
