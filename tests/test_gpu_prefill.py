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
    out = torch.full((nq * nh * hd,), float("nan"), dtype=torch.float32, device=dev)
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


def test_fa2_entry_point_reference_chunk(rd4, orc, dev):
    """fa2_prefill_launch as graph.cuh calls it (n_q = 512, device positions,
    q == out) at 2048 + 512 keys: the call takes the key-split path (64 row-block
    CTAs on 256 CUs); sampled rows against the oracle, including the first and
    last row of each 192-row CTA of kv head 0 and the chunk's last rows."""
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 2048, 512
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 15))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 16))
    q = orc.randn(nq * nh * hd, 17).reshape(nq, nh, hd)
    pos = np.arange(pos0, n, dtype=np.int32)
    qd = to_dev(q, torch, dev)
    rd4.fa2_prefill(qd, to_dev(k, torch, dev), to_dev(v, torch, dev), qd, to_dev(pos, torch, dev),
                    n - 1, n, nh, nkv, hd, 1 / 16)
    torch.cuda.synchronize()
    got = qd.cpu().numpy()
    grp = nh // nkv
    rows = sorted({0, 1, nq - 2, nq - 1} | {min(nq - 1, (192 * c) // grp) for c in range(16)} |
                  {min(nq - 1, (192 * c + 191) // grp) for c in range(16)})
    rows = np.int32(rows)
    want = orc.attn_batch(q[rows], k, v, pos[rows], nh, nkv, hd, 1 / 16, 1, 1, threads=8)
    check_close(got[rows].ravel(), want, "fa2 512-query chunk (key splits) vs oracle")


@pytest.mark.parametrize("nh,nkv,pos0,nq,q_f16,gated", [
    (24, 4, 0, 37, True, True),      # first chunk, ragged row count
    (16, 2, 50, 129, False, False),  # group 8, f32 queries, no gate
    (4, 4, 7, 65, True, True),       # group 1 (MHA)
    (24, 4, 1000, 512, True, False), # the reference's chunk size
    (6, 3, 40, 300, True, True),     # 3 kv heads (the CTA order without the XCD map)
    (16, 8, 5, 97, False, True),     # 8 kv heads, group 2
])
def test_prefill_shapes(rd4, orc, dev, nh, nkv, pos0, nq, q_f16, gated):
    import torch
    hd = 256
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 11))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 12))
    q = orc.randn(nq * nh * hd, 13).reshape(nq, nh, hd)
    if q_f16:
        q = q.astype(np.float16).astype(np.float32)
    pos = np.arange(pos0, n, dtype=np.int32)
    want = orc.attn_batch(q, k, v, pos, nh, nkv, hd, 1 / 16, 1, 1, threads=8).ravel()
    g = orc.randn(nq * nh * hd, 14)
    if gated:
        _, want = orc.sigmoid_gate(g, want)
    qd = to_dev(q.astype(np.float16) if q_f16 else q, torch, dev)
    out = torch.full((nq * nh * hd,), float("nan"), dtype=torch.float32, device=dev)
    rd4.prefill(qd, to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv, hd, 1 / 16, 1, 1,
                gate=to_dev(g, torch, dev) if gated else None)
    check_close(out.cpu().numpy(), want, "prefill %d/%d pos0 %d n %d" % (nh, nkv, pos0, nq))


def test_prefill_config5_sampled_rows(rd4, orc, dev):
    """4096 f16 queries at 4096..8191 over 8192 f16 keys,
    causal, gated; every output row of a sample of tokens vs the oracle."""
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 4096, 4096
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 21))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 22))
    q = orc.randn(nq * nh * hd, 23).reshape(nq, nh, hd).astype(np.float16)
    g = orc.randn(nq * nh * hd, 24).reshape(nq, nh, hd)
    out = torch.full((nq, nh, hd), float("nan"), dtype=torch.float32, device=dev)
    gd = to_dev(g, torch, dev)
    rd4.prefill(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv,
                hd, 1 / 16, 1, 1, gate=gd)
    got = out.cpu().numpy()
    rows = np.int32([0, 1, 2, 63, 64, 127, 1000, 2047, 2048, 3333, 4094, 4095])
    want = orc.attn_batch(q[rows].astype(np.float32), k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1,
                          threads=8)
    _, want = orc.sigmoid_gate(g[rows], want)
    check_close(got[rows].ravel(), want, "config 5 rows")
    assert np.all(np.isfinite(got))


def test_prefill_mfma_matches_generic(rd4, orc, dev, monkeypatch):
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 333, 300
    n = pos0 + nq
    k = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 31)), torch, dev)
    v = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 32)), torch, dev)
    q = to_dev(orc.randn(nq * nh * hd, 33).reshape(nq, nh, hd).astype(np.float16), torch, dev)
    a = torch.empty(nq * nh * hd, device=dev)
    b = torch.empty_like(a)
    rd4.prefill(q, k, v, a, pos0, nh, nkv, hd, 1 / 16, 1, 1)
    monkeypatch.setenv("RD4_PREFILL_GENERIC", "1")
    rd4.prefill(q, k, v, b, pos0, nh, nkv, hd, 1 / 16, 1, 1)
    check_close(a.cpu().numpy(), b.cpu().numpy(), "mfma vs generic")


@pytest.mark.parametrize("dst_type,q_f16", [(2, True), (3, False), (1, True), (4, True), (5, True), (0, True)])
def test_prefill_append_fused(rd4, orc, dev, dst_type, q_f16):
    """rd4_prefill_append: the chunk's K/V rows quantized into a second cache in
    the same launch. The attention output and gate equal rd4_prefill's bit for bit;
    the appended bytes equal the oracle's quantization of the same rows."""
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 200, 300
    n = pos0 + nq
    k = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 21)), torch, dev)
    v = to_dev(orc.store_rows(1, orc.randn(n * nkv * hd, 22)), torch, dev)
    q = orc.randn(nq * nh * hd, 23).reshape(nq, nh, hd)
    qd = to_dev(q.astype(np.float16) if q_f16 else q, torch, dev)
    g = orc.randn(nq * nh * hd, 24)
    knew = orc.randn(nq * nkv * hd, 25)
    vnew = orc.randn(nq * nkv * hd, 26)
    knew[7 * hd + 3] = 0.0
    vnew[: hd] *= 40.0  # a wide row
    rb = rd4.kv_row_bytes(dst_type, hd)
    kdst = torch.zeros(n * nkv * rb, dtype=torch.uint8, device=dev)
    vdst = torch.zeros(n * nkv * rb, dtype=torch.uint8, device=dev)
    off = pos0 * nkv * rb
    out1 = torch.empty(nq * nh * hd, dtype=torch.float32, device=dev)
    g1 = to_dev(g, torch, dev)
    rd4.prefill_append(qd, k, v, out1, pos0, nh, nkv, hd, 1 / 16, 1, 1, to_dev(knew, torch, dev),
                       to_dev(vnew, torch, dev), kdst[off:], vdst[off:], dst_type, gate=g1)
    out0 = torch.empty_like(out1)
    g0 = to_dev(g, torch, dev)
    rd4.prefill(qd, k, v, out0, pos0, nh, nkv, hd, 1 / 16, 1, 1, gate=g0)
    torch.cuda.synchronize()
    assert torch.equal(out1, out0) and torch.equal(g1, g0)
    assert np.array_equal(kdst[off:].cpu().numpy(), orc.store_rows(dst_type, knew))
    assert np.array_equal(vdst[off:].cpu().numpy(), orc.store_rows(dst_type, vnew))
    assert not kdst[:off].any() and not vdst[:off].any()


def test_prefill_append_rejects_overlap(rd4, orc, dev):
    """Appending into the rows the same launch attends is refused (the reference
    stores first, then attends; one pass cannot order that)."""
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 64, 32
    n = pos0 + nq
    rb = rd4.kv_row_bytes(1, hd)
    k = torch.zeros(n * nkv * rb, dtype=torch.uint8, device=dev)
    v = torch.zeros_like(k)
    q = torch.zeros(nq * nh * hd, dtype=torch.float16, device=dev).reshape(nq, nh, hd)
    out = torch.full((nq * nh * hd,), float("nan"), dtype=torch.float32, device=dev)
    src = torch.zeros(nq * nkv * hd, dtype=torch.float32, device=dev)
    with pytest.raises(rd4.Rd4Error):
        rd4.prefill_append(q, k, v, out, pos0, nh, nkv, hd, 1 / 16, 1, 1, src, src,
                           k[pos0 * nkv * rb:], v[pos0 * nkv * rb:], 1)


def test_prefill_append_config5_full(rd4, orc, dev, monkeypatch):
    """The launch bench.py times for configs[4] (rd4_prefill_append: 4096 f16
    queries at 4096..8191 over 8192 f16 keys, causal, gated, the chunk's K/V rows
    appended as q8_0), at full size (graph.cuh:1462 store + 1479-1535):
    - all 4096 x 24 output rows against the generic (VALU) kernel on the same inputs;
    - the first and last query row of every eighth 192-row (and 128-row) CTA
      block, plus the chunk's first and last rows, against the f64 oracle;
    - the 4096 appended q8_0 rows of each cache byte-for-byte against the oracle's
      quantization of the same f32 rows."""
    import torch
    nh, nkv, hd, pos0, nq = 24, 4, 256, 4096, 4096
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 81))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 82))
    q = orc.randn(nq * nh * hd, 83).reshape(nq, nh, hd).astype(np.float16)
    g = orc.randn(nq * nh * hd, 84).reshape(nq, nh, hd)
    knew = orc.randn(nq * nkv * hd, 85)
    vnew = orc.randn(nq * nkv * hd, 86)
    knew.reshape(nq, nkv, hd)[:, :, 7] *= 8  # the outlier channel of configs[2]
    rb = rd4.kv_row_bytes(2, hd)
    kq8 = torch.zeros(n * nkv * rb, dtype=torch.uint8, device=dev)
    vq8 = torch.zeros_like(kq8)
    qd, kd, vd = to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev)
    out = torch.full((nq, nh, hd), float("nan"), dtype=torch.float32, device=dev)
    gd = to_dev(g, torch, dev)
    off = pos0 * nkv * rb
    rd4.prefill_append(qd, kd, vd, out, pos0, nh, nkv, hd, 1 / 16, 1, 1, to_dev(knew, torch, dev),
                       to_dev(vnew, torch, dev), kq8[off:], vq8[off:], 2, gate=gd)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    sig = gd.cpu().numpy()
    assert np.array_equal(kq8[off:].cpu().numpy(), orc.store_rows(2, knew))
    assert np.array_equal(vq8[off:].cpu().numpy(), orc.store_rows(2, vnew))
    assert not kq8[:off].any() and not vq8[:off].any()
    # every row against the generic kernel
    monkeypatch.setenv("RD4_PREFILL_GENERIC", "1")
    ref = torch.empty_like(out)
    gd2 = to_dev(g, torch, dev)
    rd4.prefill(qd, kd, vd, ref, pos0, nh, nkv, hd, 1 / 16, 1, 1, gate=gd2)
    torch.cuda.synchronize()
    check_close(got.ravel(), ref.cpu().numpy().ravel(), "config 5 mfma vs generic, all rows")
    assert np.array_equal(sig, gd2.cpu().numpy())
    # CTA-boundary rows against the oracle: a CTA holds 192 (query, head) rows
    # (12 waves of 16; 128 in the 8-wave shape)
    grp = nh // nkv
    rows = {0, nq - 1}
    for bm in (192, 128):
        blocks = range(0, (nq * grp + bm - 1) // bm, 8)
        rows |= {min(nq - 1, bm * c // grp) for c in blocks} | {min(nq - 1, (bm * c + bm - 1) // grp) for c in blocks}
    rows = sorted(rows)
    rows = np.int32(rows)
    want = orc.attn_batch(q[rows].astype(np.float32), k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1,
                          threads=8)
    _, want = orc.sigmoid_gate(g[rows], want)
    check_close(got[rows].ravel(), want, "config 5 rows vs oracle (%d rows)" % len(rows))


@pytest.mark.parametrize("shape", ["1", "2", "3"])
def test_prefill_shape_variants(shape):
    """The kernel's other CTA shapes (RD4_PREFILL_SHAPE: 1 = 4 waves x 32 rows,
    2 = 8 waves x 32 rows, 3 = 8 waves x 16 rows; the default is 12 x 16) on a
    GQA chunk with a masked last block, against the f64 oracle on every query
    row. Run in a child process, since the library reads the variable once."""
    import os
    import subprocess
    import sys
    code = r'''
import sys
sys.path.insert(0, "tests"); sys.path.insert(0, "oracle")
import numpy as np, torch
from conftest import load_package
import oracle as orc
from gpu_util import to_dev, check_close
rd4 = load_package(); dev = torch.device("cuda:0")
nh, nkv, hd, pos0, nq = 24, 4, 256, 333, 301
n = pos0 + nq
k = orc.store_rows(1, orc.randn(n * nkv * hd, 41))
v = orc.store_rows(1, orc.randn(n * nkv * hd, 42))
q = orc.randn(nq * nh * hd, 43).reshape(nq, nh, hd).astype(np.float16)
g = orc.randn(nq * nh * hd, 44).reshape(nq, nh, hd)
out = torch.full((nq, nh, hd), float("nan"), dtype=torch.float32, device=dev)
gd = to_dev(g, torch, dev)
rd4.prefill(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv, hd,
            1 / 16, 1, 1, gate=gd)
torch.cuda.synchronize()
rows = np.arange(nq, dtype=np.int32)
want = orc.attn_batch(q.astype(np.float32), k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1, threads=8)
_, want = orc.sigmoid_gate(g, want)
check_close(out.cpu().numpy().ravel(), want, "shape " + sys.argv[1])
print("ok")
'''
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, RD4_PREFILL_SHAPE=shape)
    r = subprocess.run([sys.executable, "-c", code, shape], cwd=root, env=env, capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.parametrize("split", ["8x512", "1+3+4"])
def test_prefill_chunked_equals_one_call(rd4, orc, dev, split):
    """Chunked prefill against one call over the whole chunk: the reference
    requires chunks 1+3+4 to equal one pass (check_kvctx_gpu.hip:109-163), and
    its engine sends a 4096-token prompt as 8 calls of 512 queries
    (graph.cuh:1890-1939, fa2_prefill_usable's n_q == 512, attn_fa2.cuh:192-207).
    Without key splits each query row's arithmetic depends only on its own keys
    (blocks past a row's causal limit are masked to exact zeros), so 1+3+4 and
    one call match bit for bit. A 512-query call fills only a quarter of the
    CUs with row blocks, so it splits the keys (4 splits, merged by a second
    launch) while the 4096-query call does not: there P is rounded to f16
    against each split's own running max, so the outputs agree to the f16
    rounding of P (the attention tolerance), and the chunked sequence repeated
    gives the same bits again. Gate and appended q8_0 bytes match bit for bit."""
    import torch
    nh, nkv, hd = 24, 4, 256
    if split == "8x512":
        pos0, sizes = 4096, [512] * 8
    else:
        pos0, sizes = 1000, [1, 3, 4]
    nq = sum(sizes)
    n = pos0 + nq
    k = orc.store_rows(1, orc.randn(n * nkv * hd, 91))
    v = orc.store_rows(1, orc.randn(n * nkv * hd, 92))
    q = orc.randn(nq * nh * hd, 93).reshape(nq, nh, hd).astype(np.float16)
    g = orc.randn(nq * nh * hd, 94).reshape(nq, nh, hd)
    knew = orc.randn(nq * nkv * hd, 95).reshape(nq, nkv, hd)
    vnew = orc.randn(nq * nkv * hd, 96).reshape(nq, nkv, hd)
    rb = rd4.kv_row_bytes(2, hd)
    qd, kd, vd = to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev)
    kn, vn = to_dev(knew, torch, dev), to_dev(vnew, torch, dev)
    res = []
    for chunks in ([nq], sizes, sizes):
        out = torch.full((nq, nh, hd), float("nan"), dtype=torch.float32, device=dev)
        gd = to_dev(g, torch, dev)
        kq8 = torch.zeros(nq * nkv * rb, dtype=torch.uint8, device=dev)
        vq8 = torch.zeros_like(kq8)
        r0 = 0
        for c in chunks:
            rd4.prefill_append(qd[r0:r0 + c], kd, vd, out[r0:r0 + c], pos0 + r0, nh, nkv, hd, 1 / 16, 1, 1,
                               kn[r0:r0 + c], vn[r0:r0 + c], kq8[r0 * nkv * rb:], vq8[r0 * nkv * rb:], 2,
                               gate=gd[r0:r0 + c])
            r0 += c
        torch.cuda.synchronize()
        res.append([t.cpu().numpy() for t in (out, gd, kq8, vq8)])
    for a, b, what in zip(res[0], res[1], ("out", "gate", "k q8_0", "v q8_0")):
        if what == "out" and split == "8x512":
            check_close(b, a, "chunked 8x512 (key splits) vs one call")
        else:
            assert np.array_equal(a, b), "%s: chunked %s differs from one call" % (what, split)
    for a, b, what in zip(res[1], res[2], ("out", "gate", "k q8_0", "v q8_0")):
        assert np.array_equal(a, b), "%s: chunked %s repeated differs" % (what, split)
    # and the one-call result itself against the oracle on its last rows
    rows = np.int32(sorted({nq - 1, nq - 2, 0, nq // 2, min(nq - 1, 511), min(nq - 1, 512)}))
    want = orc.attn_batch(q[rows].astype(np.float32), k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1, threads=8)
    _, want = orc.sigmoid_gate(g[rows], want)
    check_close(res[0][0][rows].ravel(), want, "one-call prefill rows vs oracle")
    check_close(res[1][0][rows].ravel(), want, "chunked prefill rows vs oracle")


@pytest.mark.parametrize("splits", ["2", "5", "16"])
def test_prefill_forced_key_splits(splits):
    """The key-split path (RD4_PREFILL_KSPLIT forces the count) on a GQA chunk
    whose CTAs reach different last keys (so some splits of some CTAs hold no
    key of a row, or none at all): every query row against the f64 oracle, the
    gate, and the q8_0 bytes appended by the first split's CTAs. Run in a child
    process, since the library reads the variable once."""
    import os
    import subprocess
    import sys
    code = r'''
import sys
sys.path.insert(0, "tests"); sys.path.insert(0, "oracle")
import numpy as np, torch
from conftest import load_package
import oracle as orc
from gpu_util import to_dev, check_close
rd4 = load_package(); dev = torch.device("cuda:0")
nh, nkv, hd, pos0, nq = 24, 4, 256, 333, 301
n = pos0 + nq
k = orc.store_rows(1, orc.randn(n * nkv * hd, 51))
v = orc.store_rows(1, orc.randn(n * nkv * hd, 52))
q = orc.randn(nq * nh * hd, 53).reshape(nq, nh, hd).astype(np.float16)
g = orc.randn(nq * nh * hd, 54).reshape(nq, nh, hd)
knew = orc.randn(nq * nkv * hd, 55).reshape(nq, nkv, hd)
vnew = orc.randn(nq * nkv * hd, 56).reshape(nq, nkv, hd)
rb = rd4.kv_row_bytes(2, hd)
kq8 = torch.zeros(nq * nkv * rb, dtype=torch.uint8, device=dev)
vq8 = torch.zeros_like(kq8)
out = torch.full((nq, nh, hd), float("nan"), dtype=torch.float32, device=dev)
gd = to_dev(g, torch, dev)
rd4.prefill_append(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out, pos0, nh, nkv,
                   hd, 1 / 16, 1, 1, to_dev(knew, torch, dev), to_dev(vnew, torch, dev), kq8, vq8, 2, gate=gd)
torch.cuda.synchronize()
rows = np.arange(nq, dtype=np.int32)
want = orc.attn_batch(q.astype(np.float32), k, v, pos0 + rows, nh, nkv, hd, 1 / 16, 1, 1, threads=8)
sig, want = orc.sigmoid_gate(g, want)
check_close(out.cpu().numpy().ravel(), want, "key splits " + sys.argv[1])
assert np.allclose(gd.cpu().numpy(), sig.reshape(gd.shape), rtol=2e-7, atol=0)  # device vs host expf
assert np.array_equal(kq8.cpu().numpy(), orc.store_rows(2, knew))
assert np.array_equal(vq8.cpu().numpy(), orc.store_rows(2, vnew))
print("ok")
'''
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, RD4_PREFILL_KSPLIT=splits)
    r = subprocess.run([sys.executable, "-c", code, splits], cwd=root, env=env, capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr
