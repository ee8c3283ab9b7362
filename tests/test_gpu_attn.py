"""Decode / batched attention on the GPU vs the f64 CPU oracle (reference
attn.cuh:95-1049 semantics; tolerance max-abs 2e-3, mean-rel 1e-3)."""
import numpy as np
import pytest

from gpu_util import check_close, to_dev

pytestmark = pytest.mark.gpu


def make_cache(orc, t, n, nkv, hd, seed, outlier=False):
    x = orc.randn(n * nkv * hd, seed)
    if outlier:
        x = x.reshape(n, nkv, hd)
        x[:, :, 7] *= 8
        x = x.ravel()
    return orc.store_rows(t, x)


def run_decode(rd4, torch, dev, q, k, v, t, nh, nkv, hd, kt, vt, gate=None, n_splits=0):
    out = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=dev)
    g = None if gate is None else to_dev(gate, torch, dev)
    rd4.attn_decode(to_dev(q, torch, dev), to_dev(k, torch, dev), to_dev(v, torch, dev), out, t,
                    nh, nkv, hd, 1.0 / np.sqrt(hd), kt, vt, gate=g, n_splits=n_splits)
    torch.cuda.synchronize()
    return out.cpu().numpy().reshape(nh, hd), (None if g is None else g.cpu().numpy())


def test_config1_cpu_reference_case(rd4, orc, dev):
    """16 q heads / 2 kv heads, hd 256, f16 K/V x 512, no gate."""
    import torch
    nh, nkv, hd, n = 16, 2, 256, 512
    k = make_cache(orc, 1, n, nkv, hd, 1)
    v = make_cache(orc, 1, n, nkv, hd, 2)
    q = orc.randn(nh * hd, 3)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, 1, 1)
    got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, 1, 1)
    check_close(got, want, "cfg1")


PAIRS = [(kt, vt) for kt in range(6) for vt in range(6)]


@pytest.mark.parametrize("kt,vt", PAIRS)
def test_all_36_pairs(rd4, orc, dev, kt, vt):
    """Every (K, V) storage pair dispatches (attn.cuh:203-246) and matches."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 300
    k = make_cache(orc, kt, n, nkv, hd, 10 + kt)
    v = make_cache(orc, vt, n, nkv, hd, 20 + vt)
    q = orc.randn(nh * hd, 30)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, vt)
    got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, vt, n_splits=3)
    check_close(got, want, "pair %d/%d" % (kt, vt))


@pytest.mark.parametrize("kt,vt", [(2, 2), (2, 3), (3, 3), (1, 1), (5, 4)])
def test_query_outlier_dims(rd4, orc, dev, kt, vt):
    """Queries with a wide dynamic range: one dim x100 in every head, one head of
    values ~1e-3 with a single dim of 50, one all-zero head. The q8_0 K path
    carries the f32 query as int8 hi/lo parts with a scale pair per 32-dim block,
    so a large dim coarsens only its own block."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 700
    k = make_cache(orc, kt, n, nkv, hd, 50 + kt, outlier=True)
    v = make_cache(orc, vt, n, nkv, hd, 60 + vt)
    q = orc.randn(nh * hd, 61).reshape(nh, hd)
    q[:, 7] *= 100.0
    q[3] *= 1e-3
    q[3, 200] = 50.0
    q[5] = 0.0
    q = np.ascontiguousarray(q.ravel())
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, vt)
    for splits in (1, 0):
        got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, vt, n_splits=splits)
        check_close(got, want, "outlier q %d/%d splits %d" % (kt, vt, splits))


@pytest.mark.parametrize("splits", [1, 2, 7, 16, 17, 64, 256])
def test_split_invariance_and_merge_tree(rd4, orc, dev, splits):
    """Any split count (one-level merge <= 16, two-level above) gives the same
    attention, including splits with no keys (t+1 < splits*32)."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 1000
    k = make_cache(orc, 2, n, nkv, hd, 40, outlier=True)
    v = make_cache(orc, 2, n, nkv, hd, 41, outlier=True)
    q = orc.randn(nh * hd, 42)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, 2, 2)
    got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, 2, 2, n_splits=splits)
    check_close(got, want, "splits %d" % splits)
    # repeated launches reuse the self-resetting merge counters
    got2, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, 2, 2, n_splits=splits)
    assert np.array_equal(got, got2)


def test_more_splits_than_keys_and_no_keys(rd4, orc, dev):
    import torch
    nh, nkv, hd = 8, 2, 128
    k = make_cache(orc, 1, 4, nkv, hd, 50)
    v = make_cache(orc, 1, 4, nkv, hd, 51)
    q = orc.randn(nh * hd, 52)
    got, _ = run_decode(rd4, torch, dev, q, k, v, 0, nh, nkv, hd, 1, 1, n_splits=200)
    want = np.tile(orc.load_rows(1, v, 4 * nkv * hd).reshape(4, nkv, hd)[0], (1, 4)).reshape(nkv, 4, hd)
    check_close(got, np.repeat(orc.load_rows(1, v, 4 * nkv * hd).reshape(4, nkv, hd)[0], 4, 0), "1 key")
    got, _ = run_decode(rd4, torch, dev, q, k, v, -1, nh, nkv, hd, 1, 1, n_splits=5)
    assert np.all(got == 0)


def test_gate_fused(rd4, orc, dev):
    """rd4_attn_decode with a gate == attention then sigmoid_gate (graph.cuh:958-981)."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 2048
    k = make_cache(orc, 2, n, nkv, hd, 60)
    v = make_cache(orc, 2, n, nkv, hd, 61)
    q = orc.randn(nh * hd, 62)
    g = orc.randn(nh * hd, 63)
    att = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, 2, 2)
    gs, want = orc.sigmoid_gate(g, att.ravel())
    got, gg = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, 2, 2, gate=g)
    check_close(got.ravel(), want, "gated")
    assert np.allclose(gg, gs, rtol=1e-6, atol=1e-7)


def test_reference_entry_points_in_place(rd4, orc, dev):
    """attn_launch / attn_launch_split with q == out (graph.cuh:964-969)."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 700
    k = make_cache(orc, 3, n, nkv, hd, 70)
    v = make_cache(orc, 3, n, nkv, hd, 71)
    q = orc.randn(nh * hd, 72)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, 3, 3)
    kd, vd = to_dev(k, torch, dev), to_dev(v, torch, dev)
    for fn in ("launch", "split"):
        buf = to_dev(q, torch, dev)
        if fn == "launch":
            rd4.attn_launch(buf, kd, vd, buf, n - 1, nh, nkv, hd, 1 / 16, 3, 3)
        else:
            part = torch.empty(nh * 16 * (hd + 2), dtype=torch.float32, device=dev)
            rd4.attn_launch_split(buf, kd, vd, buf, part, n - 1, nh, nkv, hd, 1 / 16, 3, 3, 4)
        check_close(buf.cpu().numpy().reshape(nh, hd), want, fn)


@pytest.mark.parametrize("split", [False, True])
def test_batched(rd4, orc, dev, split):
    """attn_batch_launch / attn_split_batch_launch: token i attends keys 0..pos[i]."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 1500
    k = make_cache(orc, 2, n, nkv, hd, 80)
    v = make_cache(orc, 1, n, nkv, hd, 81)
    pos = np.int32([0, 1, 31, 32, 511, 512, 1200, 1499])
    q = orc.randn(pos.size * nh * hd, 82).reshape(pos.size, nh, hd)
    want = orc.attn_batch(q, k, v, pos, nh, nkv, hd, 1 / 16, 2, 1)
    qd = to_dev(q, torch, dev)
    out = torch.full_like(qd, float("nan"))  # unwritten elements stay NaN
    args = (qd, to_dev(k, torch, dev), to_dev(v, torch, dev), out, to_dev(pos, torch, dev), nh, nkv,
            hd, 1 / 16, 2, 1)
    if split:
        rd4.attn_split_batch(*args, 6)
    else:
        rd4.attn_batch(*args)
    check_close(out.cpu().numpy(), want, "batch")


def test_sigmoid_gate_kernel(rd4, orc, dev):
    import torch
    g = orc.randn(24 * 256 + 3, 90) * 4
    y = orc.randn(g.size, 91)
    gs, ys = orc.sigmoid_gate(g, y)
    gd, yd = to_dev(g, torch, dev), to_dev(y, torch, dev)
    rd4.sigmoid_gate(gd, yd)
    assert np.allclose(gd.cpu().numpy(), gs, rtol=2e-6, atol=1e-7)
    assert np.allclose(yd.cpu().numpy(), ys, rtol=3e-6, atol=1e-7)


def test_rope_kernel(rd4, orc, dev):
    import torch
    nt, nh, hd, nrot = 5, 4, 256, 64
    x = orc.randn(nt * nh * hd, 92).reshape(nt, nh, hd)
    pos = np.int32([0, 1, 7, 4096, 131000])
    want = orc.rope(x, nt, nh, hd, nrot, 1e7, pos)
    xd = to_dev(x, torch, dev)
    rd4.rope(xd, nt, nh, hd, nrot, 1e7, to_dev(pos, torch, dev))
    got = xd.cpu().numpy()
    # positions <= 4096: tight; at 131000 one ulp of the f32 angle (from powf's last
    # bit on either side) is ~8e-3 rad, so only a loose bound is meaningful there
    rel = np.linalg.norm(got[:4] - want[:4]) / np.linalg.norm(want[:4])
    assert rel < 1e-5  # device cosf/sinf and powf last-bit differences at angles up to 4096 rad
    assert np.linalg.norm(got[4] - want[4]) / np.linalg.norm(want[4]) < 2e-2


@pytest.mark.parametrize("t,vt", [(1, 1), (2, 2), (3, 3), (4, 4), (4, 5), (5, 5), (5, 2)])
def test_decode_append_fused(rd4, orc, dev, t, vt):
    """rd4_attn_decode_append == kv_store of the new row + gated decode."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 777
    rb, vrb = orc.row_bytes(t, hd), orc.row_bytes(vt, hd)
    k = make_cache(orc, t, n, nkv, hd, 100)
    v = make_cache(orc, vt, n, nkv, hd, 101)
    kn, vn = orc.randn(nkv * hd, 102), orc.randn(nkv * hd, 103)
    k_ref, v_ref = k.copy(), v.copy()
    k_ref[(n - 1) * nkv * rb:] = orc.store_rows(t, kn)
    v_ref[(n - 1) * nkv * vrb:] = orc.store_rows(vt, vn)
    k[(n - 1) * nkv * rb:] = 0x5A  # stale row content must be replaced
    v[(n - 1) * nkv * vrb:] = 0xA5
    q, g = orc.randn(nh * hd, 104), orc.randn(nh * hd, 105)
    gs, want = orc.sigmoid_gate(g, orc.attn_decode(q, k_ref, v_ref, n - 1, nh, nkv, hd, 1 / 16, t, vt).ravel())
    kd, vd, gd = to_dev(k, torch, dev), to_dev(v, torch, dev), to_dev(g, torch, dev)
    out = torch.full((nh * hd,), float("nan"), device=dev)
    rd4.attn_decode_append(to_dev(q, torch, dev), to_dev(kn, torch, dev), to_dev(vn, torch, dev), kd, vd,
                           out, n - 1, nh, nkv, hd, 1 / 16, t, vt, gate=gd)
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), k_ref) and np.array_equal(vd.cpu().numpy(), v_ref)
    check_close(out.cpu().numpy(), want, "append %d/%d" % (t, vt))


@pytest.mark.parametrize("kt,vt", [(1, 1), (2, 2), (3, 3), (2, 3), (1, 2), (4, 5), (5, 5), (4, 2),
                                   (5, 3), (1, 5), (2, 5), (4, 1), (4, 4), (5, 4), (1, 4)])
def test_mfma_path_matches_generic_path(rd4, orc, dev, kt, vt, monkeypatch):
    """The MFMA decode kernel and the all-types kernel agree (both vs the oracle)."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 3000
    k = make_cache(orc, kt, n, nkv, hd, 110, outlier=True)
    v = make_cache(orc, vt, n, nkv, hd, 111)
    q = orc.randn(nh * hd, 112)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, vt, threads=8)
    got_fast, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, vt)
    monkeypatch.setenv("RD4_DECODE_GENERIC", "1")
    got_gen, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, vt)
    check_close(got_fast, want, "mfma")
    check_close(got_gen, want, "generic")


@pytest.mark.parametrize("cfg", ["f16_32k_gate", "q8_0_32k_append", "q4_0_131k", "q5_0_q4_1_131k"])
def test_baseline_decode_configs_full_size(rd4, orc, dev, cfg):
    """BASELINE configs[1..3] at their real shapes vs the f64 oracle, and the
    reference's 131K default pair (K q5_0, V q4_1) at the same shape."""
    import torch
    nh, nkv, hd = 24, 4, 256
    kt, vt = {"f16_32k_gate": (1, 1), "q8_0_32k_append": (2, 2), "q4_0_131k": (3, 3),
              "q5_0_q4_1_131k": (4, 5)}[cfg]
    n = 131001 if kt >= 3 else 32768
    k = make_cache(orc, kt, n, nkv, hd, 120, outlier=(kt == 2))
    v = make_cache(orc, vt, n, nkv, hd, 121, outlier=(kt == 2))
    q, g = orc.randn(nh * hd, 122), orc.randn(nh * hd, 123)
    kd, vd = to_dev(k, torch, dev), to_dev(v, torch, dev)
    out = torch.full((nh * hd,), float("nan"), device=dev)
    gd = to_dev(g, torch, dev)
    if kt == 2:
        kn, vn = orc.randn(nkv * hd, 124), orc.randn(nkv * hd, 125)
        rb = orc.row_bytes(kt, hd)
        k[(n - 1) * nkv * rb:] = orc.store_rows(kt, kn)
        v[(n - 1) * nkv * rb:] = orc.store_rows(kt, vn)
        rd4.attn_decode_append(to_dev(q, torch, dev), to_dev(kn, torch, dev), to_dev(vn, torch, dev), kd,
                               vd, out, n - 1, nh, nkv, hd, 1 / 16, kt, kt, gate=gd)
    else:
        rd4.attn_decode(to_dev(q, torch, dev), kd, vd, out, n - 1, nh, nkv, hd, 1 / 16, kt, vt, gate=gd)
    torch.cuda.synchronize()
    _, want = orc.sigmoid_gate(g, orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, vt, threads=8).ravel())
    check_close(out.cpu().numpy(), want, cfg)


def test_rd_attn_splits_env_forces_the_count():
    """RD_ATTN_SPLITS=N (graph.cuh:509-519) forces N splits on the launches that
    pick their own count: attn_launch / attn_launch_split then equal a forced
    rd4_attn_decode(n_splits=N) bit for bit. Run in a child process, since the
    library reads the variable once."""
    import subprocess
    import sys
    code = r'''
import sys
sys.path.insert(0, "tests"); sys.path.insert(0, "oracle")
import numpy as np, torch
from conftest import load_package
import oracle as orc
from test_gpu_attn import make_cache
from gpu_util import to_dev
rd4 = load_package(); dev = torch.device("cuda:0")
nh, nkv, hd, n = 24, 4, 256, 5000
k = to_dev(make_cache(orc, 2, n, nkv, hd, 500), torch, dev)
v = to_dev(make_cache(orc, 2, n, nkv, hd, 501), torch, dev)
q = to_dev(orc.randn(nh * hd, 502), torch, dev)
outs = []
for f in ("launch", "split", "forced"):
    o = torch.full((nh * hd,), float("nan"), device=dev)
    if f == "launch":
        rd4.attn_launch(q, k, v, o, n - 1, nh, nkv, hd, 1 / 16, 2, 2)
    elif f == "split":
        rd4.attn_launch_split(q, k, v, o, o, n - 1, nh, nkv, hd, 1 / 16, 2, 2, 4)
    else:
        rd4.attn_decode(q, k, v, o, n - 1, nh, nkv, hd, 1 / 16, 2, 2, n_splits=int(sys.argv[1]))
    torch.cuda.synchronize()
    outs.append(o.cpu().numpy())
assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[1], outs[2]), "env count not used"
print("ok")
'''
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    for count in ("1", "3"):
        env = dict(os.environ, RD_ATTN_SPLITS=count)
        r = subprocess.run([sys.executable, "-c", code, count], cwd=root, env=env,
                           capture_output=True, text=True, timeout=180)
        assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


def test_in_kernel_merge_generic():
    """RD4_DECODE_GENERIC=1 sends every pair to the all-types kernel, whose split
    records are folded inside the launch by a counter tree (the MFMA decode uses
    the merge launch). It must match the oracle at 16 and 64 splits and repeat
    bit for bit (the tree's counters reset themselves). Child process: the
    library reads the variable once."""
    import subprocess
    import sys
    import os
    code = r'''
import sys
sys.path.insert(0, "tests"); sys.path.insert(0, "oracle")
import numpy as np, torch
from conftest import load_package
import oracle as orc
from test_gpu_attn import make_cache
from gpu_util import to_dev, check_close
rd4 = load_package(); dev = torch.device("cuda:0")
nh, nkv, hd, n = 24, 4, 256, 3000
for kt, vt in ((2, 2), (3, 3), (1, 1)):
    kh = make_cache(orc, kt, n, nkv, hd, 700 + kt, outlier=True)
    vh = make_cache(orc, vt, n, nkv, hd, 710 + vt)
    qh = orc.randn(nh * hd, 720)
    want = orc.attn_decode(qh, kh, vh, n - 1, nh, nkv, hd, 1 / 16, kt, vt)
    k, v, q = to_dev(kh, torch, dev), to_dev(vh, torch, dev), to_dev(qh, torch, dev)
    for splits in (16, 64):
        outs = []
        for rep in range(2):
            o = torch.full((nh * hd,), float("nan"), device=dev)
            rd4.attn_decode(q, k, v, o, n - 1, nh, nkv, hd, 1 / 16, kt, vt, n_splits=splits)
            torch.cuda.synchronize()
            outs.append(o.cpu().numpy())
        check_close(outs[0], want, "merge %d/%d splits %d" % (kt, vt, splits))
        assert np.array_equal(outs[0], outs[1]), "repeat differs"
print("ok")
'''
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, RD4_DECODE_GENERIC="1")
    r = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True, text=True,
                       timeout=180)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.parametrize("kt", [1, 2])
@pytest.mark.parametrize("shift", [20.0, -20.0])
def test_merge_with_lse_spread(rd4, orc, dev, kt, shift):
    """The merge audit of bench_attn_gpu.hip:1161-1428: split records whose
    log-sum-exp maxima differ by about +-20. All heads share one query direction
    u, and the first 64 keys lean along u, so their scores sit about `shift`
    above (or below) the other keys'. Forced split counts put those keys in
    one split or spread them out."""
    import torch
    nh, nkv, hd, n = 24, 4, 256, 4096
    u = orc.randn(hd, 800)
    u = (u / np.linalg.norm(u)).astype(np.float32)
    q = np.tile(u * 16.0, nh).astype(np.float32)  # |q| = 16: a unit key along u scores 1.0
    kx = orc.randn(n * nkv * hd, 801).reshape(n, nkv, hd) * 0.2
    kx[:64] += (shift * u)[None, None, :]
    k = orc.store_rows(kt, kx.astype(np.float32).ravel())
    v = make_cache(orc, kt, n, nkv, hd, 802)
    want = orc.attn_decode(q, k, v, n - 1, nh, nkv, hd, 1 / 16, kt, kt, threads=8)
    for splits in (1, 4, 64):
        got, _ = run_decode(rd4, torch, dev, q, k, v, n - 1, nh, nkv, hd, kt, kt, n_splits=splits)
        check_close(got, want, "shift %g splits %d" % (shift, splits))
        assert np.all(np.isfinite(got))
