"""Writes tests/golden/kv_golden.npz from the CPU oracle.

Inputs: the eight hostile row patterns of the reference's
tests/check_kvquant_gpu.hip:101-137 (uniform, positive, one outlier, constant
0.5, zeros, alternating +-1, gaussian-ish, wide range x100), built from this
repo's seeded generator, plus a small GQA attention case (q8_0 K / q4_0 V).
Run: python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as orc  # noqa: E402


def patterns(hd=256):
    rows = []
    u = orc.randn(8 * hd * 4, 0x5EED1234).reshape(8, 4, hd)
    u = np.tanh(u)  # (-1, 1)
    for p in range(8):
        x = np.zeros(hd, np.float32)
        if p == 0: x = u[p, 0]
        elif p == 1: x = 0.5 * (u[p, 0] + 1)
        elif p == 2: x = 1e-3 * u[p, 0]; x[7] = 1.0
        elif p == 3: x[:] = 0.5
        elif p == 4: pass
        elif p == 5: x = np.where(np.arange(hd) & 1, -1.0, 1.0)
        elif p == 6: x = 0.25 * u[p].sum(0)
        else: x = 100 * u[p, 0]
        rows.append(np.asarray(x, np.float32))
    return np.concatenate(rows)


def main():
    out = {}
    x = patterns()
    out["x"] = x
    for t in range(6):
        b = orc.store_rows(t, x)
        out["bytes_%d" % t] = b
        out["deq_%d" % t] = orc.load_rows(t, b, x.size)
    meta = dict(n_head=6, n_kv=2, hd=64, scale=0.125, kt=orc.Q8_0, vt=orc.Q4_0, n=33)
    n, kv, hd = meta["n"], meta["n_kv"], meta["hd"]
    out["k"] = orc.store_rows(meta["kt"], orc.randn(n * kv * hd, 101))
    out["v"] = orc.store_rows(meta["vt"], orc.randn(n * kv * hd, 102))
    out["pos"] = np.int32([0, 1, 16, 32])
    out["q"] = orc.randn(4 * meta["n_head"] * hd, 103).reshape(4, meta["n_head"], hd)
    out["attn"] = orc.attn_batch(out["q"], out["k"], out["v"], out["pos"], meta["n_head"], kv, hd,
                                 meta["scale"], meta["kt"], meta["vt"])
    out["meta"] = np.array(json.dumps(meta))
    np.savez_compressed(os.path.join(HERE, "kv_golden.npz"), **out)


if __name__ == "__main__":
    main()
