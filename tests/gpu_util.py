"""Helpers for the GPU parity tests (device buffers from the oracle's seeded inputs)."""
import numpy as np

MAX_ABS = 2e-3   # attention output tolerance vs the f64-accumulating oracle
MEAN_REL = 1e-3  # sum|got - ref| / sum|ref|


def to_dev(a, torch, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def check_close(got, ref, what=""):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    assert np.all(np.isfinite(got)), what + ": non-finite output"
    err = np.abs(got - ref)
    mx = float(err.max()) if err.size else 0.0
    mr = float(err.sum() / max(np.abs(ref).sum(), 1e-30))
    assert mx <= MAX_ABS and mr <= MEAN_REL, "%s: max-abs %.3e mean-rel %.3e" % (what, mx, mr)
    return mx, mr
