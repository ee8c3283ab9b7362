"""KV append/quantize, fill and dequant on the GPU vs the CPU oracle: bit-exact
(reference kv.h:386-694; llama.cpp's quantize_row_*_ref semantics)."""
import numpy as np
import pytest

from gpu_util import to_dev

pytestmark = pytest.mark.gpu
TYPES = range(6)


def hostile_rows(orc, n_rows=64, hd=256):
    """check_kvquant_gpu.hip:101-137 patterns plus ties, exact .5 cases, outliers."""
    x = (orc.randn(n_rows * hd, 42) * 2).reshape(n_rows, hd)
    x[1] = 0.0
    x[2] = 0.5
    x[3, :] = np.where(np.arange(hd) & 1, -1.0, 1.0)
    x[4] *= 100
    x[5, 7] = 8.0 * np.abs(x[5]).max()  # outlier channel
    x[6, ::32] = 3.0; x[6, 5::32] = -3.0  # |v| ties, first occurrence wins
    x[7] = np.round(x[7] * 4) / 4 * 127 / 4  # many exact .5 multiples of d
    x[8] = np.abs(x[8])
    x[9, :] = -x[9, 0]
    x[10] = 1e-30 * x[10]  # subnormal scales
    return x.astype(np.float32).ravel()


@pytest.mark.parametrize("t", TYPES)
def test_store_bit_exact(rd4, orc, dev, t):
    import torch
    x = hostile_rows(orc)
    want = orc.store_rows(t, x)
    src = to_dev(x, torch, dev)
    dst = torch.full((want.size,), 0xAB, dtype=torch.uint8, device=dev)
    rd4.kv_store_rows(t, src, dst)
    got = dst.cpu().numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, "type %s: %d bytes differ, first at %d" % (orc.TYPE_NAMES[t], bad.size, bad[0])


@pytest.mark.parametrize("t", TYPES)
def test_store_decode_append_one_token(rd4, orc, dev, t):
    """Decode append (graph.cuh:1011-1031): 4 kv heads x 256 written at row pos."""
    import torch
    hd, nkv, ctx, pos = 256, 4, 8, 5
    rb = orc.row_bytes(t, hd)
    cache = torch.zeros(ctx * nkv * rb, dtype=torch.uint8, device=dev)
    x = orc.randn(nkv * hd, 3)
    rd4.kv_store_rows(t, to_dev(x, torch, dev), cache[pos * nkv * rb:])
    got = cache.cpu().numpy()
    assert np.array_equal(got[pos * nkv * rb:(pos + 1) * nkv * rb], orc.store_rows(t, x))
    assert not got[: pos * nkv * rb].any() and not got[(pos + 1) * nkv * rb:].any()


@pytest.mark.parametrize("t", TYPES)
def test_fill_bit_exact(rd4, orc, dev, t):
    import torch
    rows, hd, seed = 37, 256, 1234
    want = orc.fill(t, rows, hd, seed)
    cache = torch.zeros(want.size, dtype=torch.uint8, device=dev)
    rd4.kv_fill(t, cache, rows, hd, seed)
    assert np.array_equal(cache.cpu().numpy(), want)


@pytest.mark.parametrize("t", TYPES)
def test_dequant_bit_exact(rd4, orc, dev, t):
    import torch
    x = hostile_rows(orc)
    raw = orc.store_rows(t, x)
    want = orc.load_rows(t, raw, x.size)
    out = torch.empty(x.size, dtype=torch.float32, device=dev)
    rd4.kv_load_rows(t, to_dev(raw, torch, dev), out, x.size)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_store_width_is_block_local(rd4, orc, dev):
    """A prefill chunk's n_tok*NKV*hd values in one launch equal per-row stores."""
    import torch
    n = 4096 * 4 * 256 // 64
    x = orc.randn(n, 9)
    dst = torch.empty(n // 32 * 34, dtype=torch.uint8, device=dev)
    rd4.kv_store_rows(2, to_dev(x, torch, dev), dst)
    assert np.array_equal(dst.cpu().numpy(), orc.store_rows(2, x))


def test_store_rounding_order_pins(rd4, orc, dev):
    """The GPU quantizer on the rounding-order blocks of tests/quant_pins.py
    (x*(1/d) and a separate offset add, as the reference): the same codes as
    the exact derivation."""
    import torch
    import quant_pins as qp
    for kind, vals, t in (("q8_0", qp.Q8_0_BLOCK, orc.Q8_0), ("q4_0", qp.Q4_0_BLOCK, orc.Q4_0),
                          ("q5_0", qp.Q5_0_BLOCK, orc.Q5_0), ("q4_1", qp.Q4_1_BLOCK, orc.Q4_1)):
        x = qp.block(vals)
        want = qp.q8_0_codes(x)[0] if kind == "q8_0" else qp.nib_codes(kind, x)[0]
        nb = orc.row_bytes(t, 32)
        dst = torch.full((nb,), 0xAB, dtype=torch.uint8, device=dev)
        rd4.kv_store_rows(t, to_dev(x, torch, dev), dst)
        assert qp.decode_codes(kind, dst.cpu().numpy()) == want, kind
