"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the oracle's own formulas: numpy's float16 casts,
the reference's own fp16/table code compiled from its sources (oracle/_ref),
hand-derived known-answer blocks, closed forms of attention (one key, equal
keys, no keys), numpy softmax on small cases, and the committed golden vectors.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- fp16 --------

def test_f16_decode_all_finite_patterns(orc):
    h = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.load_rows(orc.F16, h.view(np.uint8), h.size)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isinf(got[np.isinf(ref)])) and np.all(np.isnan(got[np.isnan(ref)]))


def test_f16_encode_matches_numpy_rne(orc):
    rng = np.random.default_rng(7)
    # random bit patterns over the whole f32 range + every f16 halfway point
    bits = rng.integers(0, 1 << 32, size=200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    halves = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids, np.float32([65504, 65519.99, 65520, 1e-8, 2.98e-8, 0.0, -0.0])])
    x = x[~np.isnan(x)]
    got = orc.store_rows(orc.F16, x).view(np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16_nan_becomes_inf_like_reference(orc):
    # fp16.h:54: exponent >= 31 (which includes NaN inputs) returns a signed inf
    got = orc.store_rows(orc.F16, np.float32([np.nan, -np.nan, np.inf, -np.inf])).view(np.uint16)
    assert list(got) == [0x7C00, 0xFC00, 0x7C00, 0xFC00]


def test_f16_encode_matches_reference_source(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(11)
    x = rng.integers(0, 1 << 32, size=20000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    got = orc.store_rows(orc.F16, x).view(np.uint16)
    want = np.array([ref.ref_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


def test_tables_match_reference_source(orc):
    ref = orc.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    for t in range(6):
        for hd in (32, 64, 128, 256, 512):
            assert orc.row_bytes(t, hd) == ref.ref_row_bytes(t, hd)
        assert orc.lib().orc_bytes_per_elem(t) == ref.ref_bytes_per_elem(t)
        assert ref.ref_type_parse(orc.TYPE_NAMES[t].encode()) == t


def test_row_bytes_known_values(orc):
    # check_kvtype.hip:77-89 and the survey's table for head_dim 256
    assert [orc.row_bytes(t, 256) for t in range(6)] == [1024, 512, 272, 144, 176, 160]
    assert orc.row_bytes(99, 256) == -1


# ---------------------------------------------------- quantizer known answers --

def _block(vals):
    x = np.zeros(32, np.float32)
    x[: len(vals)] = vals
    return x


def test_q8_0_known_answer(orc):
    # amax = 127 -> d = 1.0 exactly, so q = round-half-away-from-zero(x)
    x = _block([127.0, 2.5, -2.5, 0.5, -0.5, 1.49, -126.6, 3.5])
    b = orc.store_rows(orc.Q8_0, x)
    assert b[:2].view(np.uint16)[0] == 0x3C00
    q = b[2:].view(np.int8)
    assert list(q[:8]) == [127, 3, -3, 1, -1, 1, -127, 4]
    assert np.all(q[8:] == 0)


def test_q8_0_zero_block(orc):
    b = orc.store_rows(orc.Q8_0, np.zeros(32, np.float32))
    assert np.all(b == 0)


def test_q4_0_known_answer(orc):
    # signed max -8 -> d = -8/-8 = 1.0; q = trunc(x*1 + 8.5) clamped to [0, 15]
    x = _block([-8.0, 7.0, 0.4, -0.6, 6.6, 7.9])
    b = orc.store_rows(orc.Q4_0, x)
    assert b[:2].view(np.uint16)[0] == 0x3C00
    qs = b[2:18]
    lo = qs & 15
    hi = qs >> 4
    assert list(lo[:6]) == [0, 15, 8, 7, 15, 15]  # 6.6+8.5=15.1->15, 7.9+8.5=16.4->16->15
    assert np.all(lo[6:] == 8) and np.all(hi == 8)  # zeros -> 8


def test_q4_0_tie_first_occurrence_wins(orc):
    # |8| == |-8|: the first one (+8) is the signed max -> d = -1
    x = _block([8.0, -8.0])
    b = orc.store_rows(orc.Q4_0, x)
    assert b[:2].view(np.uint16)[0] == 0xBC00  # -1.0
    assert b[2] & 15 == 0 and b[3] & 15 == 15  # -8+8.5 -> 0; 8+8.5=16.5 -> 16 -> clamp 15
    x2 = _block([-8.0, 8.0])
    assert orc.store_rows(orc.Q4_0, x2)[:2].view(np.uint16)[0] == 0x3C00


def test_q4_0_zero_block_sign(orc):
    # amax stays 0, vmax = +0 -> d = +0/-8 = -0.0 -> f16 0x8000, every nibble 8
    b = orc.store_rows(orc.Q4_0, np.zeros(32, np.float32))
    assert b[:2].view(np.uint16)[0] == 0x8000
    assert np.all(b[2:] == 0x88)


def test_q5_0_known_answer(orc):
    # signed max -16 -> d = 1; q = trunc(x + 16.5) in [0,31]; element 1 = 15 -> 31
    x = _block([-16.0, 15.0, 0.0, 1.0])
    x[20] = 3.0  # element 20 -> 19 (bit 4 set, low nibble 3), high half of byte 4
    b = orc.store_rows(orc.Q5_0, x)
    assert b[:2].view(np.uint16)[0] == 0x3C00
    qh = int(b[2]) | int(b[3]) << 8 | int(b[4]) << 16 | int(b[5]) << 24
    qs = b[6:22]
    q = np.concatenate([qs & 15, qs >> 4]).astype(int) | np.array([(qh >> e) & 1 for e in range(32)]) << 4
    want = np.full(32, 16)
    want[:4] = [0, 31, 16, 17]
    want[20] = 19
    assert list(q) == list(want)


def test_q4_1_known_answer(orc):
    # min 0, max 15 -> d = 1, m = 0; q = trunc(x + 0.5)
    x = _block([0.0, 15.0, 2.49, 2.5, 7.0])
    x[5:] = 1.0
    b = orc.store_rows(orc.Q4_1, x)
    assert b[:2].view(np.uint16)[0] == 0x3C00 and b[2:4].view(np.uint16)[0] == 0
    q = np.concatenate([b[4:20] & 15, b[4:20] >> 4])
    assert list(q[:5]) == [0, 15, 2, 3, 7] and np.all(q[5:] == 1)


def _kvquant_patterns(rows_per=4, hd=256, seed=5):
    """The 8 row shapes of check_kvquant_gpu.hip:101-137 (uniform, positive,
    one outlier, constant 0.5, zeros, alternating +-1, gaussian-ish, wide), drawn
    from numpy instead of the reference's frand."""
    rng = np.random.default_rng(seed)
    out = []
    for p in range(8):
        u = rng.uniform(-1, 1, size=(rows_per, hd)).astype(np.float32)
        d = np.arange(hd)
        x = {0: u, 1: 0.5 * (u + 1), 2: np.where(d == 7, 1.0, 1e-3 * u),
             3: np.full_like(u, 0.5), 4: np.zeros_like(u),
             5: np.broadcast_to(np.where(d & 1, -1.0, 1.0), u.shape),
             6: 0.25 * (u + rng.uniform(-1, 1, size=u.shape) * 3), 7: 100 * u}[p]
        out.append(np.ascontiguousarray(x, np.float32))
    return out


def test_kvquant_patterns_q8_0_invariants(orc):
    # Per block: d = f16(amax/127) (IEEE divide, then RNE to f16); the element
    # holding amax maps to +-127; every code is round(x/d) up to the f16
    # rounding of d (|x*id - q| <= 0.5 + 127*2^-11); sign(q) = sign(x) or q == 0.
    for p, x in enumerate(_kvquant_patterns()):
        b = orc.store_rows(orc.Q8_0, x.ravel()).reshape(-1, 34)
        xb = x.reshape(-1, 32)
        amax = np.abs(xb).max(1)
        d16 = b[:, :2].copy().view(np.float16).ravel()
        want = (amax / np.float32(127)).astype(np.float32).astype(np.float16)
        assert np.array_equal(d16.view(np.uint16), want.view(np.uint16)), p
        q = b[:, 2:].view(np.int8).astype(np.int32)
        nz = amax > 0
        arg = np.abs(xb).argmax(1)
        assert np.all(np.abs(q[np.arange(len(q)), arg][nz]) == 127), p
        assert np.all(q[~nz] == 0), p
        dd = (amax / np.float32(127)).astype(np.float64)[:, None]
        r = np.where(nz[:, None], xb / np.where(dd > 0, dd, 1), 0)
        assert np.all(np.abs(r - q) <= 0.5 + 1e-6), p
        assert np.all((q == 0) | (np.sign(q) == np.sign(xb))), p
        if p == 3:  # constant 0.5: every code 127
            assert np.all(q == 127)
        if p == 5:  # alternating: +-127
            assert np.all(np.abs(q) == 127)


def test_kvquant_patterns_q4_0_invariants(orc):
    # Per block: the signed max v (first of equal magnitudes) gives d = v/-8, so
    # v itself codes to nibble 0 (dequant -8d = v exactly); nibbles in [0,15];
    # dequant error <= one step |d| (the +8.5 truncation rounds half up, and the
    # clamp at 15 costs at most one step on the side opposite to v).
    for p, x in enumerate(_kvquant_patterns()):
        flat = x.ravel()
        b = orc.store_rows(orc.Q4_0, flat).reshape(-1, 18)
        xb = flat.reshape(-1, 32)
        arg = np.abs(xb).argmax(1)  # numpy argmax: first occurrence
        v = xb[np.arange(len(xb)), arg]
        d16 = b[:, :2].copy().view(np.float16).astype(np.float32).ravel()
        want = (v / np.float32(-8)).astype(np.float32).astype(np.float16).astype(np.float32)
        assert np.array_equal(d16, want), p
        nib = np.concatenate([b[:, 2:] & 15, b[:, 2:] >> 4], 1).astype(np.int32)
        nz = v != 0
        assert np.all(nib[np.arange(len(nib)), arg][nz] == 0), p
        assert np.all(nib[~nz] == 8), p
        y = orc.load_rows(orc.Q4_0, b.ravel(), flat.size).reshape(-1, 32)
        step = np.abs(d16)[:, None]
        assert np.all(np.abs(y - xb) <= step * (1 + 2.0 ** -10) + 1e-6), p
        if p == 3:  # constant 0.5: d = -1/16, every x*id = -8 -> nibble 0
            assert np.all(nib == 0) and np.all(d16 == -0.0625)
        if p == 5:  # +1 first -> d = -1/8: +1 -> 0, -1 -> 16.5 -> clamp 15
            assert np.all(nib[:, 0::2] == 0) and np.all(nib[:, 1::2] == 15)


@pytest.mark.parametrize("t", [2, 3, 4, 5])
def test_quant_roundtrip_error_bound(orc, t):
    # dequant(quant(x)) is within one quantization step d (q4_1: d) of x, per block
    x = orc.randn(256 * 64, 3) * 3
    x[7::256] *= 8  # outlier channel
    b = orc.store_rows(t, x)
    y = orc.load_rows(t, b, x.size)
    bb = orc.BLOCK_BYTES[t]
    d = np.abs(b.reshape(-1, bb)[:, :2].copy().view(np.float16).astype(np.float32)).repeat(32)
    err = np.abs(y - x)
    # q8_0: half a step plus the f16 rounding of d over |q| <= 127 (127 * 2^-11 of a step)
    assert np.all(err <= d * (0.5 + 127 * 2.0 ** -11 if t == 2 else 1.0) * 1.01 + 1e-6)


def test_dequant_closed_forms(orc):
    # one block per type with chosen bytes, decoded by hand
    b = np.zeros(34, np.uint8)
    b[:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    b[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    assert np.array_equal(orc.load_rows(orc.Q8_0, b, 32), 0.5 * np.arange(-16, 16, dtype=np.float32))
    b = np.zeros(18, np.uint8)
    b[:2] = np.frombuffer(np.float16(-2.0).tobytes(), np.uint8)
    b[2:] = (np.arange(16) | (np.arange(16)[::-1] << 4)).astype(np.uint8)
    want = -2.0 * (np.concatenate([np.arange(16), np.arange(16)[::-1]]) - 8)
    assert np.array_equal(orc.load_rows(orc.Q4_0, b, 32), want.astype(np.float32))
    b = np.zeros(20, np.uint8)
    b[:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(-1.0).tobytes(), np.uint8)
    b[4:] = 0xF3
    want = np.float32([0.25 * 3 - 1.0] * 16 + [0.25 * 15 - 1.0] * 16)
    assert np.array_equal(orc.load_rows(orc.Q4_1, b, 32), want)


# ----------------------------------------------------------------- fill -------

def test_kv_rand_closed_form(orc):
    # kv.h:508-513 evaluated by hand for idx 0, seed 0: h = 0 -> -1.0
    assert orc.kv_rand(0, 0) == -1.0
    idx, seed = 12345, 777
    h = ((idx * 2654435761) ^ (seed * 2246822519)) & 0xFFFFFFFF
    h ^= h >> 13
    h = (h * 1274126177) & 0xFFFFFFFF
    assert orc.kv_rand(idx, seed) == np.float32((h >> 8) / 8388608.0 - 1.0)


def test_fill_equals_store_of_hash(orc):
    for t in range(6):
        rows, hd, seed = 5, 64, 99
        x = np.array([orc.kv_rand(i, seed) for i in range(rows * hd)], np.float32)
        assert np.array_equal(orc.fill(t, rows, hd, seed), orc.store_rows(t, x))


# ------------------------------------------------------------- attention ------

def _np_attention(q, kd, vd, pos, n_head, n_kv, scale):
    """numpy float64 softmax attention over dequantized K/V [n][n_kv][hd]."""
    grp = n_head // n_kv
    out = np.zeros(q.shape, np.float64)
    for i, t in enumerate(pos):
        for h in range(n_head):
            k = kd[: t + 1, h // grp].astype(np.float64)
            v = vd[: t + 1, h // grp].astype(np.float64)
            s = k @ q[i, h].astype(np.float64) * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ v
    return out


@pytest.mark.parametrize("kt,vt", [(1, 1), (2, 2), (3, 3), (0, 4), (5, 2)])
def test_attention_vs_numpy(orc, kt, vt):
    n_head, n_kv, hd, n = 8, 2, 64, 40
    kx = orc.randn(n * n_kv * hd, 21)
    vx = orc.randn(n * n_kv * hd, 22)
    k = orc.store_rows(kt, kx)
    v = orc.store_rows(vt, vx)
    kd = orc.load_rows(kt, k, kx.size).reshape(n, n_kv, hd)
    vd = orc.load_rows(vt, v, vx.size).reshape(n, n_kv, hd)
    pos = [0, 5, 39, 17]
    q = orc.randn(len(pos) * n_head * hd, 23).reshape(len(pos), n_head, hd)
    got = orc.attn_batch(q, k, v, pos, n_head, n_kv, hd, 0.125, kt, vt)
    want = _np_attention(q, kd, vd, pos, n_head, n_kv, 0.125)
    assert np.abs(got - want).max() < 1e-6


def test_attention_closed_forms(orc):
    n_head, n_kv, hd = 6, 1, 32
    q = orc.randn(n_head * hd, 5)
    # one key: output is the (dequantized) V row
    k = orc.store_rows(orc.F32, orc.randn(hd, 6))
    v = orc.store_rows(orc.Q8_0, orc.randn(hd, 7))
    got = orc.attn_decode(q, k, v, 0, n_head, n_kv, hd, 1.0, orc.F32, orc.Q8_0)
    assert np.array_equal(got, np.tile(orc.load_rows(orc.Q8_0, v, hd), (n_head, 1)))
    # identical keys: uniform softmax -> mean of V
    n = 10
    kk = np.tile(orc.randn(hd, 8), n)
    vv = orc.randn(n * hd, 9)
    got = orc.attn_decode(q, orc.store_rows(0, kk), orc.store_rows(0, vv), n - 1, n_head, n_kv, hd,
                          0.3, 0, 0)
    assert np.allclose(got, vv.reshape(n, hd).mean(0), atol=1e-6)
    # no keys: zeros
    got = orc.attn_decode(q, k, v, -1, n_head, n_kv, hd, 1.0, 0, 2)
    assert np.all(got == 0)


def test_merge_equals_unsplit(orc):
    # splitting the keys into partial (m, l, acc) records and merging reproduces attention
    hd, n = 32, 50
    q = orc.randn(hd, 1).astype(np.float64)
    k = orc.randn(n * hd, 2).reshape(n, hd).astype(np.float64)
    v = orc.randn(n * hd, 3).reshape(n, hd).astype(np.float64)
    s = k @ q
    bounds = [0, 0, 7, 30, 50, 50]  # includes empty splits
    recs = []
    for a, b in zip(bounds[:-1], bounds[1:]):
        if a == b:
            recs.append(np.concatenate([[-np.inf, 0.0], np.zeros(hd)]))
            continue
        m = s[a:b].max()
        p = np.exp(s[a:b] - m)
        recs.append(np.concatenate([[m + 20 * (a == 7) * 0, p.sum()], p @ v[a:b]]))
    got = orc.merge(np.array(recs, np.float32), 1, hd, len(recs))[0]
    want = (np.exp(s - s.max()) / np.exp(s - s.max()).sum()) @ v
    assert np.abs(got - want).max() < 1e-5
    allempty = np.array([[-np.inf, 0.0] + [np.nan] * hd] * 3, np.float32)
    assert np.all(orc.merge(allempty, 1, hd, 3) == 0)


def test_sigmoid_gate_closed_form(orc):
    g = np.float32([0.0, 1.0, -3.0, 30.0, -30.0])
    y = np.float32([2.0, 1.0, 1.0, 5.0, 7.0])
    gs, ys = orc.sigmoid_gate(g, y)
    want = 1.0 / (1.0 + np.exp(-g.astype(np.float64)))
    assert np.allclose(gs, want, rtol=2e-7, atol=0) and gs[0] == 0.5
    assert np.allclose(ys, y * want, rtol=3e-7)


def test_rope_closed_form(orc):
    # position 0: identity; a pair rotated by theta = pos * base^(-2p/n_rot)
    x = orc.randn(2 * 64, 4).reshape(1, 2, 64)
    assert np.allclose(orc.rope(x, 1, 2, 64, 64, 10000.0, [0]), x)
    got = orc.rope(x, 1, 2, 64, 32, 10000.0, [3])
    th = 3 * 10000.0 ** (-2 * 5 / 32)
    x0, x1 = x[0, 1, 5], x[0, 1, 21]
    assert np.isclose(got[0, 1, 5], x0 * np.cos(th) - x1 * np.sin(th), atol=1e-6)
    assert np.array_equal(got[0, 1, 32:], x[0, 1, 32:])


# --------------------------------------------------------------- golden -------

def test_golden_vectors(orc):
    """tests/golden/kv_golden.npz: quantized bytes and attention outputs of fixed
    inputs (written by tests/golden/make_golden.py); guards the oracle against
    silent change."""
    path = os.path.join(GOLDEN, "kv_golden.npz")
    z = np.load(path)
    meta = json.loads(str(z["meta"]))
    for t in range(6):
        assert np.array_equal(orc.store_rows(t, z["x"]), z["bytes_%d" % t]), orc.TYPE_NAMES[t]
        assert np.array_equal(orc.load_rows(t, z["bytes_%d" % t], z["x"].size), z["deq_%d" % t])
    got = orc.attn_batch(z["q"], z["k"], z["v"], z["pos"], meta["n_head"], meta["n_kv"],
                         meta["hd"], meta["scale"], meta["kt"], meta["vt"])
    assert np.abs(got - z["attn"]).max() <= 1e-6


def test_rms_norm_power_of_two_rows_exact(orc):
    # |x| = 2^k everywhere: mean(x^2) = 4^k and the scale 2^-k are exact, so y = sign(x) * w
    for ncols, k in ((64, 3), (256, -2), (512, 5), (1000, 1)):
        sign = np.where(orc.randn(ncols, ncols) > 0, 1.0, -1.0).astype(np.float32)
        x = (sign * 2.0 ** k).astype(np.float32)
        w = orc.randn(ncols, 7 + ncols)
        assert np.array_equal(orc.rms_norm(x, w, ncols, 0.0), sign * w)
        assert np.array_equal(orc.rms_norm(x, None, ncols, 0.0), sign)


def test_rms_norm_tree_order(orc):
    """One large element among ones, 5120 columns (nn.cuh:37-59): thread 0's fmaf chain
    2^24 + 1 + ... rounds every +1 away, each other thread's chain sums 20 ones, and the
    halving tree adds those 255 partials exactly: sum = 2^24 + 5100. A sequential sum
    (2^24), a 128-partial tree (2^24 + 5080) or the exact sum (2^24 + 5119) give other
    scales."""
    n = 5120
    x = np.ones(n, np.float32)
    x[0] = 4096.0
    y = orc.rms_norm(x, None, n, 0.0)

    def scale_of(total):
        mean = np.float32(np.float32(total) / np.float32(n))
        return np.float32(1.0 / np.sqrt(np.float64(mean)))

    want = scale_of(2.0 ** 24 + 5100)
    assert y[1] == want and y[0] == np.float32(4096.0 * np.float64(want))
    for other in (2.0 ** 24, 2.0 ** 24 + 5080, 2.0 ** 24 + 5119):
        assert scale_of(other) != want


def test_rms_norm_matches_f64(orc):
    for rows, ncols, eps in ((24, 256, 1e-6), (3, 1000, 1e-5), (2, 5120, 1e-6), (4, 64, 0.1)):
        x = orc.randn(rows * ncols, rows + ncols).reshape(rows, ncols)
        w = orc.randn(ncols, 3 * ncols)
        got = orc.rms_norm(x, w, ncols, eps)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps) * w
        assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


# ------------------------------------------ rounding-order pins (x*(1/d), separate add) --

def test_quantizer_rounding_order_pins(orc):
    """Blocks where the reference's order (id = 1/d, x*id rounded, then the
    offset added and rounded) gives other codes than x/d or a fused add: the
    oracle must produce the codes of the reference order, derived by exact
    rational arithmetic in tests/quant_pins.py."""
    import quant_pins as qp
    x8 = qp.block(qp.Q8_0_BLOCK)
    ref, div = qp.q8_0_codes(x8)
    assert ref[1:5] == [-19, -61, 64, 96]            # worked out exactly, see quant_pins
    assert ref != div                                 # x/d would change codes here
    assert qp.decode_codes("q8_0", orc.store_rows(orc.Q8_0, x8)) == ref
    for kind, vals, t in (("q4_0", qp.Q4_0_BLOCK, orc.Q4_0), ("q5_0", qp.Q5_0_BLOCK, orc.Q5_0),
                          ("q4_1", qp.Q4_1_BLOCK, orc.Q4_1)):
        x = qp.block(vals)
        ref, fused, div = qp.nib_codes(kind, x)
        assert ref != fused and ref != div, kind      # both alternatives are caught
        assert qp.decode_codes(kind, orc.store_rows(t, x)) == ref, kind
    # the literal codes of the discriminating elements
    assert qp.nib_codes("q4_0", qp.block(qp.Q4_0_BLOCK))[0][1:4] == [12, 8, 11]
    assert qp.nib_codes("q5_0", qp.block(qp.Q5_0_BLOCK))[0][1:5] == [14, 23, 30, 18]
    assert qp.nib_codes("q4_1", qp.block(qp.Q4_1_BLOCK))[0][2:6] == [1, 11, 7, 8]
