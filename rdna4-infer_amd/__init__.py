"""Python host side of the gfx950 full-attention library.

Thin ctypes mirror of the C ABI in include/rdna4attn.h, which itself mirrors the
reference's operator API (include/rdna4/attn.cuh, attn_fa2.cuh, kv.h, nn.cuh of
Vmarcelo49/rdna4-infer). Functions take torch tensors on the GPU for device
memory and streams; every call runs the HIP kernels of librdna4attn.so. There is
no CPU fallback: when the library is missing, loading fails with an error.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("RD4_LIB") or os.path.join(HERE, "librdna4attn.so")

F32, F16, Q8_0, Q4_0, Q5_0, Q4_1 = range(6)
TYPE_NAMES = ("f32", "f16", "q8_0", "q4_0", "q5_0", "q4_1")
OK, EINVAL, ETYPE, ELAUNCH, ENOMEM = 0, -1, -2, -3, -4

# exported symbol -> (argtypes, restype); the C-ABI test checks include/ against this
_P, _I, _I64, _F, _U32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_uint32
SIGNATURES = {
    "rd4_kv_cache_bytes": ([ctypes.c_uint64, ctypes.c_int, ctypes.c_int], ctypes.c_uint64),
    "rd4_kv_cache_bytes_shape": ([ctypes.c_uint64] + [ctypes.c_int] * 5, ctypes.c_uint64),
    "rd4_kv_max_ctx": ([ctypes.c_uint64, ctypes.c_uint64] + [ctypes.c_int] * 5, ctypes.c_uint64),
    "rd4_version": ([], ctypes.c_char_p),
    "rd4_init": ([], _I),
    "rd4_stream_init": ([_P], _I),
    "rd4_last_error": ([], ctypes.c_char_p),
    "rd4_kv_type_name": ([_I], ctypes.c_char_p),
    "rd4_kv_type_parse": ([ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)], ctypes.c_char_p),
    "rd4_kv_bytes_per_elem": ([_I], ctypes.c_double),
    "rd4_kv_row_bytes": ([_I, _I], _I64),
    "rd4_kv_store_row_launch": ([_I, _P, _P, _I64, _P], _I),
    "rd4_kv_fill_launch": ([_I, _P, _I64, _I, _U32, _P], _I),
    "rd4_kv_load_rows_launch": ([_I, _P, _P, _I64, _P], _I),
    "rd4_attn_launch": ([_P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P], _I),
    "rd4_attn_launch_split": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_attn_launch_split_wpb": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _I, _P], _I),
    "rd4_attn_partial_bytes": ([_I, _I, _I], ctypes.c_size_t),
    "rd4_attn_split_wpb": ([_I], _I),
    "rd4_attn_decode": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_attn_decode_append": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_attn_decode_append_noalloc": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_attn_batch_launch": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P], _I),
    "rd4_attn_split_batch_launch": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_fa2_prefill_launch": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P], _I),
    "rd4_fa2_prefill_usable": ([_I, _I, _I, _I, _I, _I, _I], _I),
    "rd4_prefill": ([_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P], _I),
    "rd4_prefill_append": ([_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P, _P, _I,
                            _P], _I),
    "rd4_sigmoid_gate_launch": ([_P, _P, _I64, _P], _I),
    "rd4_rope_launch": ([_P, _I, _I, _I, _I, _F, _P, _P], _I),
    "rd4_attn_decode_tokens": ([_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I, _P], _I),
    "rd4_read_probe": ([_P, _I64, _P, _P], _I),
    "rd4_rms_norm_launch": ([_P, _P, _P, _I64, _I64, _F, _P], _I),
    "rd4_qk_norm_rope_append": ([_P, _P, _P, _P, _P, _F, _I, _F, _P, _I, _I, _I, _I, _P, _P, _P,
                                 _P, _P, _I, _I, _P], _I),
}

_lib = None


class Rd4Error(RuntimeError):
    pass


def lib():
    """Load librdna4attn.so (built by rdna4-infer_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Rd4Error("librdna4attn.so is not built: run rdna4-infer_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _build_module():
    from importlib import util
    spec = util.spec_from_file_location("_rd4_build", os.path.join(HERE, "build.py"))
    mod = util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def build():
    return _build_module().build(verbose=False)


def build_shim_check():
    """Build the test-only device check of the include/rdna4 C++ shims."""
    return _build_module().build_shim_check()


def _check(rc, what):
    if rc != OK:
        msg = lib().rd4_last_error().decode()
        raise Rd4Error("%s failed (%d): %s" % (what, rc, msg))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# ---- KV tables (kv.h:100-169) ------------------------------------------------

def kv_type_name(t):
    return lib().rd4_kv_type_name(t).decode()


def kv_type_parse(name):
    """Returns the KvType value; raises ValueError with the reference's message."""
    out = ctypes.c_int(-1)
    err = lib().rd4_kv_type_parse(name.encode(), ctypes.byref(out))
    if err is not None:
        raise ValueError(err.decode())
    return out.value


def kv_row_bytes(t, head_dim):
    return int(lib().rd4_kv_row_bytes(t, head_dim))


def kv_bytes_per_elem(t):
    return float(lib().rd4_kv_bytes_per_elem(t))


# ---- KV append / fill / dequant (kv.h:386-694) --------------------------------

def kv_store_rows(t, src, dst, width=None):
    """kv_store_row_launch: quantize f32 `src` into uint8 tensor `dst`."""
    width = src.numel() if width is None else width
    _check(lib().rd4_kv_store_row_launch(t, _ptr(src), _ptr(dst), width, _stream()), "kv_store")


def kv_fill(t, cache, n_rows, head_dim, seed):
    _check(lib().rd4_kv_fill_launch(t, _ptr(cache), n_rows, head_dim, seed & 0xFFFFFFFF, _stream()),
           "kv_fill")


def kv_load_rows(t, src, dst, width):
    _check(lib().rd4_kv_load_rows_launch(t, _ptr(src), _ptr(dst), width, _stream()), "kv_load")


# ---- attention -----------------------------------------------------------------

def attn_decode(q, k, v, out, t, n_head, n_head_kv, head_dim, scale, kt, vt, gate=None, n_splits=0):
    _check(lib().rd4_attn_decode(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(gate), t, n_head,
                                 n_head_kv, head_dim, scale, kt, vt, n_splits, _stream()),
           "attn_decode")


def attn_decode_append(q, k_new, v_new, k, v, out, t, n_head, n_head_kv, head_dim, scale, kt, vt,
                       gate=None, n_splits=0):
    """Append the token's K/V rows at position t, then gated decode over keys 0..t."""
    _check(lib().rd4_attn_decode_append(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k), _ptr(v), _ptr(out),
                                        _ptr(gate), t, n_head, n_head_kv, head_dim, scale, kt, vt,
                                        n_splits, _stream()), "attn_decode_append")


def attn_decode_append_noalloc(q, k_new, v_new, k, v, out, t, n_head, n_head_kv, head_dim, scale, kt,
                               vt, gate=None, n_splits=0):
    """attn_decode_append through the allocation-free entry point (fixed
    library scratch; calls overlapping on one GPU race)."""
    _check(lib().rd4_attn_decode_append_noalloc(_ptr(q), _ptr(k_new), _ptr(v_new), _ptr(k), _ptr(v),
                                                _ptr(out), _ptr(gate), t, n_head, n_head_kv, head_dim,
                                                scale, kt, vt, n_splits, _stream()),
           "attn_decode_append_noalloc")


def attn_decode_tokens(q, k, v, out, t0, n_tok, n_head, n_head_kv, head_dim, scale, kt, vt,
                       gate=None, n_splits=0):
    """Multi-token decode: token i at position t0 + i attends keys 0..t0+i."""
    _check(lib().rd4_attn_decode_tokens(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(gate), t0, n_tok,
                                        n_head, n_head_kv, head_dim, scale, kt, vt, n_splits,
                                        _stream()), "attn_decode_tokens")


def attn_launch(q, k, v, out, t, n_head, n_head_kv, head_dim, scale, kt, vt):
    _check(lib().rd4_attn_launch(_ptr(q), _ptr(k), _ptr(v), _ptr(out), t, n_head, n_head_kv,
                                 head_dim, scale, kt, vt, _stream()), "attn_launch")


def attn_launch_split(q, k, v, out, partial, t, n_head, n_head_kv, head_dim, scale, kt, vt, n_splits):
    _check(lib().rd4_attn_launch_split(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(partial), t,
                                       n_head, n_head_kv, head_dim, scale, kt, vt, n_splits,
                                       _stream()), "attn_launch_split")


def attn_batch(q, k, v, out, pos, n_head, n_head_kv, head_dim, scale, kt, vt):
    _check(lib().rd4_attn_batch_launch(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(pos), pos.numel(),
                                       n_head, n_head_kv, head_dim, scale, kt, vt, _stream()),
           "attn_batch")


def attn_split_batch(q, k, v, out, pos, n_head, n_head_kv, head_dim, scale, kt, vt, n_splits,
                     partial=None):
    _check(lib().rd4_attn_split_batch_launch(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(partial), _ptr(pos),
                                             pos.numel(), n_head, n_head_kv, head_dim, scale, kt,
                                             vt, n_splits, _stream()), "attn_split_batch")


def prefill(q, k, v, out, pos0, n_head, n_head_kv, head_dim, scale, kt, vt, gate=None):
    """Causal prefill of q.shape[0] tokens at positions pos0.. (f16 or f32 q)."""
    import torch
    q_f16 = 1 if q.dtype == torch.float16 else 0
    _check(lib().rd4_prefill(_ptr(q), q_f16, _ptr(k), _ptr(v), _ptr(out), _ptr(gate), pos0,
                             q.shape[0], n_head, n_head_kv, head_dim, scale, kt, vt, _stream()),
           "prefill")


def prefill_append(q, k, v, out, pos0, n_head, n_head_kv, head_dim, scale, kt, vt, k_new, v_new,
                   k_dst, v_dst, dst_type, gate=None):
    """prefill() with the chunk's new K/V rows (f32 [n_q][n_head_kv][hd]) quantized to
    dst_type into k_dst / v_dst in the same launch (graph.cuh:1462 store + 1479-1535)."""
    import torch
    q_f16 = 1 if q.dtype == torch.float16 else 0
    _check(lib().rd4_prefill_append(_ptr(q), q_f16, _ptr(k), _ptr(v), _ptr(out), _ptr(gate), pos0,
                                    q.shape[0], n_head, n_head_kv, head_dim, scale, kt, vt,
                                    _ptr(k_new), _ptr(v_new), _ptr(k_dst), _ptr(v_dst), dst_type,
                                    _stream()), "prefill_append")


def fa2_prefill(q, k, v, out, pos, kmax, keys_total, n_head, n_head_kv, head_dim, scale):
    _check(lib().rd4_fa2_prefill_launch(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(pos), pos.numel(),
                                        kmax, keys_total, n_head, n_head_kv, head_dim, scale,
                                        _stream()), "fa2_prefill")


def sigmoid_gate(g, y):
    _check(lib().rd4_sigmoid_gate_launch(_ptr(g), _ptr(y), g.numel(), _stream()), "sigmoid_gate")


def rope(x, n_tokens, n_heads, head_dim, n_rot, freq_base, pos):
    _check(lib().rd4_rope_launch(_ptr(x), n_tokens, n_heads, head_dim, n_rot, freq_base, _ptr(pos),
                                 _stream()), "rope")


def rms_norm(x, w, y, nrows, ncols, eps):
    """rms_norm_launch (nn.cuh:239): y <- x * rsqrt(mean(x^2) + eps) * w per row."""
    _check(lib().rd4_rms_norm_launch(_ptr(x), _ptr(w), _ptr(y), nrows, ncols, eps, _stream()),
           "rms_norm")


def qk_norm_rope_append(qg, k_new, v_new, q_norm, k_norm, eps, n_rot, freq_base, pos, n_tok,
                        n_head, n_head_kv, head_dim, q_out, k_cache, v_cache, kt, vt,
                        gate_out=None, k_out=None):
    """Fused deinterleave + q/k RMSNorm + RoPE + K/V cache append
    (graph.cuh:914-954): one launch for the six of the reference."""
    _check(lib().rd4_qk_norm_rope_append(
        _ptr(qg), _ptr(k_new), _ptr(v_new), _ptr(q_norm), _ptr(k_norm), eps, n_rot, freq_base,
        _ptr(pos), n_tok, n_head, n_head_kv, head_dim, _ptr(q_out), _ptr(gate_out), _ptr(k_out),
        _ptr(k_cache), _ptr(v_cache), kt, vt, _stream()), "qk_norm_rope_append")


def kv_cache_bytes(ctx_size, kt, vt, n_layers=None, n_head_kv=None, head_dim=None):
    """KV cache bytes at ctx_size tokens (device.h:176): the reference model
    shape by default, or n_layers x n_head_kv x head_dim per side."""
    if n_layers is None:
        return lib().rd4_kv_cache_bytes(ctx_size, kt, vt)
    return lib().rd4_kv_cache_bytes_shape(ctx_size, n_layers, n_head_kv, head_dim, kt, vt)


def kv_max_ctx(budget_bytes, reserved_bytes, n_layers, n_head_kv, head_dim, kt, vt):
    """Largest context whose KV caches fit in budget_bytes - reserved_bytes."""
    return lib().rd4_kv_max_ctx(budget_bytes, reserved_bytes, n_layers, n_head_kv, head_dim, kt, vt)


def init():
    """rd4_init: create the null stream's library scratch on the current device."""
    _check(lib().rd4_init(), "init")


def stream_init(stream=None):
    """rd4_stream_init: create the library scratch of `stream` (a torch stream,
    default the current one) now instead of at its first split launch."""
    import torch
    st = stream if stream is not None else torch.cuda.current_stream()
    _check(lib().rd4_stream_init(ctypes.c_void_p(st.cuda_stream)), "stream_init")


def attn_partial_bytes(n_head, head_dim, n_splits):
    return int(lib().rd4_attn_partial_bytes(n_head, head_dim, n_splits))


def read_probe(buf, sink):
    """rd4_read_probe: one streaming-read launch over the bytes of `buf` (bench calibration)."""
    _check(lib().rd4_read_probe(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink), _stream()),
           "read_probe")
