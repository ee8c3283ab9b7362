"""numpy front-end of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker. Each wrapper names the reference code it restates
(file:line into Vmarcelo49/rdna4-infer).

Parity pinning of each function: see the header of oracle/oracle.c.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

F32, F16, Q8_0, Q4_0, Q5_0, Q4_1 = range(6)
TYPE_NAMES = ["f32", "f16", "q8_0", "q4_0", "q5_0", "q4_1"]
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, Q5_0: 22, Q4_1: 20}

_lib = None


def build(force=False):
    """Compile liboracle.so (and oracle/_ref when the reference tree is mounted)."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if os.path.isdir("/root/reference/include/rdna4"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, I64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = F
        L.orc_f32_to_f16.argtypes = [F]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_row_bytes.argtypes = [I, I]
        L.orc_row_bytes.restype = I64
        L.orc_bytes_per_elem.argtypes = [I]
        L.orc_bytes_per_elem.restype = ctypes.c_double
        L.orc_store_rows.argtypes = [I, P, P, I64]
        L.orc_load_rows.argtypes = [I, P, P, I64]
        L.orc_kv_rand.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        L.orc_kv_rand.restype = F
        L.orc_fill.argtypes = [I, P, I64, I, ctypes.c_uint32]
        L.orc_attn_decode.argtypes = [P, P, P, P, I, I, I, I, F, I, I, I]
        L.orc_attn_batch.argtypes = [P, P, P, P, P, I, I, I, I, F, I, I, I]
        L.orc_merge.argtypes = [P, P, I, I, I]
        L.orc_merge.restype = None
        L.orc_sigmoid_gate.argtypes = [P, P, I64]
        L.orc_sigmoid_gate.restype = None
        L.orc_rope.argtypes = [P, I, I, I, I, F, P]
        L.orc_rope.restype = None
        L.orc_rms_norm.argtypes = [P, P, P, I64, I64, F]
        L.orc_rms_norm.restype = None
        L.orc_randn.argtypes = [P, I64, ctypes.c_uint64]
        L.orc_randn.restype = None
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def row_bytes(t, head_dim):
    return int(lib().orc_row_bytes(t, head_dim))


def randn(n, seed):
    """Seeded N(0,1) float32 vector (splitmix64 + Box-Muller)."""
    out = np.empty(int(n), np.float32)
    lib().orc_randn(_p(out), out.size, seed)
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    return np.array([lib().orc_f32_to_f16(float(v)) for v in x], np.uint16)


def store_rows(t, x):
    """kv_store_row_kernel semantics (include/rdna4/kv.h:386-501): f32 -> bytes."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    nbytes = row_bytes(t, x.size) if t in (F32, F16) else x.size // 32 * BLOCK_BYTES[t]
    out = np.zeros(nbytes, np.uint8)
    if lib().orc_store_rows(t, _p(x), _p(out), x.size) != 0:
        raise ValueError("orc_store_rows rejected type %d width %d" % (t, x.size))
    return out


def load_rows(t, raw, width):
    """kv_load semantics (include/rdna4/kv.h:174-229): bytes -> f32."""
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(int(width), np.float32)
    if lib().orc_load_rows(t, _p(raw), _p(out), int(width)) != 0:
        raise ValueError("orc_load_rows rejected type %d" % t)
    return out


def kv_rand(idx, seed):
    return lib().orc_kv_rand(idx & 0xFFFFFFFF, seed & 0xFFFFFFFF)


def fill(t, n_rows, head_dim, seed):
    """kv_fill (kv.h:508-513, 632): element e of row r = store(kv_rand(r*hd+e, seed))."""
    out = np.zeros(n_rows * row_bytes(t, head_dim), np.uint8)
    if lib().orc_fill(t, _p(out), n_rows, head_dim, seed) != 0:
        raise ValueError("orc_fill rejected")
    return out


def attn_batch(q, k, v, pos, n_head, n_head_kv, head_dim, scale, kt, vt, threads=1):
    """f64 GQA attention per token over keys 0..pos[i] (check_rope_gpu.hip:103-130)."""
    q = np.ascontiguousarray(q, np.float32)
    pos = np.ascontiguousarray(pos, np.int32)
    out = np.zeros((pos.size, n_head, head_dim), np.float32)
    k = np.ascontiguousarray(k, np.uint8)
    v = np.ascontiguousarray(v, np.uint8)
    rc = lib().orc_attn_batch(_p(q), _p(k), _p(v), _p(out), _p(pos), pos.size, n_head, n_head_kv,
                              head_dim, scale, kt, vt, threads)
    if rc != 0:
        raise ValueError("orc_attn_batch rejected the shape")
    return out


def attn_decode(q, k, v, t, n_head, n_head_kv, head_dim, scale, kt, vt, threads=1):
    return attn_batch(q, k, v, [t], n_head, n_head_kv, head_dim, scale, kt, vt, threads)[0]


def merge(partial, n_rows, head_dim, n_splits):
    partial = np.ascontiguousarray(partial, np.float32)
    out = np.zeros((n_rows, head_dim), np.float32)
    lib().orc_merge(_p(partial), _p(out), n_rows, head_dim, n_splits)
    return out


def sigmoid_gate(g, y):
    g = np.array(g, np.float32, copy=True)
    y = np.array(y, np.float32, copy=True)
    lib().orc_sigmoid_gate(_p(g), _p(y), g.size)
    return g, y


def rope(x, n_tokens, n_heads, head_dim, n_rot, freq_base, pos):
    x = np.array(x, np.float32, copy=True)
    pos = np.ascontiguousarray(pos, np.int32)
    lib().orc_rope(_p(x), n_tokens, n_heads, head_dim, n_rot, freq_base, _p(pos))
    return x


def rms_norm(x, w, ncols, eps):
    """Row RMSNorm in the reference's f32 order (nn.cuh:24-63); w may be None."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    wp = None
    if w is not None:
        w = np.ascontiguousarray(w, np.float32)
        wp = _p(w)
    lib().orc_rms_norm(_p(x), wp, _p(y), x.size // ncols, ncols, eps)
    return y


def ref_lib():
    """The reference's own host fp16/table code, if oracle/_ref was built."""
    if not os.path.exists(REF_PATH):
        return None
    L = ctypes.CDLL(REF_PATH)
    L.ref_f32_to_f16.argtypes = [ctypes.c_float]
    L.ref_f32_to_f16.restype = ctypes.c_uint16
    L.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.ref_f16_to_f32.restype = ctypes.c_float
    L.ref_row_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    L.ref_row_bytes.restype = ctypes.c_longlong
    L.ref_bytes_per_elem.argtypes = [ctypes.c_int]
    L.ref_bytes_per_elem.restype = ctypes.c_double
    L.ref_type_parse.argtypes = [ctypes.c_char_p]
    L.ref_type_name.argtypes = [ctypes.c_int]
    L.ref_type_name.restype = ctypes.c_char_p
    return L
