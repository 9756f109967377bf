"""numpy wrappers over liboracle_kv.so (TEST INFRASTRUCTURE, see __init__.py).

fp16 arrays are numpy ``float16`` (IEEE binary16), passed to C as their bit
patterns. Every wrapper returns new arrays and leaves its inputs untouched
unless it says "in place".
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_kv.so")
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_I64 = ctypes.c_int64


def build(force=False):
    """Compiles liboracle_kv.so with the committed Makefile."""
    args = ["make", "-C", _HERE]
    if force:
        args.append("-B")
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "ok_f32_to_f16": (ctypes.c_uint16, [_F]),
            "ok_f16_to_f32": (_F, [ctypes.c_uint16]),
            "ok_f32_to_f16_array": (None, [_P, _P, _SZ]),
            "ok_f16_to_f32_array": (None, [_P, _P, _SZ]),
            "ok_rope_table": (None, [_P, _P, _I, _I, _F]),
            "ok_rope": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
            "ok_write_kv_cache": (None, [_P, _P, _P, _I, _I, _I]),
            "ok_rope_append": (None, [_P, _P, _P, _P, _P, _I, _I, _I, _I]),
            "ok_cached_attention": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
            "ok_cached_attention_f64": (None, [_P, _P, _P, _P, _I, _I, _I, _I]),
            "ok_cached_attention_mt": (None, [_P, _P, _P, _P, _I, _I, _I, _I, _I]),
            "ok_e4m3_decode": (_F, [ctypes.c_uint8]),
            "ok_e4m3_encode": (ctypes.c_uint8, [_F]),
            "ok_fp8_quantize_f16": (None, [_P, _P, _SZ, _F]),
            "ok_paged_gather": (None, [_P, _P, _I, _I, _I, _I, _P]),
            "ok_paged_attention_f16": (None, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _I]),
            "ok_paged_attention_fp8": (None, [_P, _P, _P, _P, _P, _P, _I, _I, _P, _I, _I, _I]),
            "ok_paged_write_f16": (None, [_P, _P, _P, _P, _I64, _I]),
            "ok_paged_write_fp8": (None, [_P, _P, _P, _P, _I64, _I, _I, _P, _P]),
            "ok_w8a16_gemv": (None, [_P, _P, _P, _P, _I, _I, _I]),
            "ok_w8a16_gemv_f64": (None, [_P, _P, _P, _P, _I, _I, _I]),
            "ok_prefill_attention": (None, [_P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I]),
            "ok_prefill_attention_f64": (None, [_P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
            "ok_prefill_rope_append": (None, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- fp16 -----------------------------------------------------------------
def f32_to_f16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().ok_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f16_to_f32(h):
    h = _c(h, np.float16).view(np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ok_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


# ---- a1 / a2 / a3 -----------------------------------------------------------
def rope_table(max_seq, head_dim, base=500000.0):
    cos = np.empty((max_seq, head_dim // 2), np.float32)
    sin = np.empty((max_seq, head_dim // 2), np.float32)
    lib().ok_rope_table(_ptr(cos), _ptr(sin), max_seq, head_dim, base)
    return cos, sin


def rope(q, k, cos_rows, sin_rows, n_q_heads, n_kv_heads, head_dim):
    """launch_rope on q [seq, nq*hd], k [seq, nkv*hd]; returns rotated copies."""
    q = _c(q, np.float16).copy()
    k = _c(k, np.float16).copy()
    seq = q.shape[0] if q.ndim > 1 else 1
    cos_rows = _c(cos_rows, np.float32)
    sin_rows = _c(sin_rows, np.float32)
    lib().ok_rope(_ptr(q), _ptr(k), _ptr(cos_rows), _ptr(sin_rows), seq, n_kv_heads, n_q_heads,
                  head_dim)
    return q, k


def write_kv_cache(qkv_out, k_cache, v_cache, pos, q_dim, kv_dim):
    """In place on k_cache / v_cache (fp16 arrays)."""
    qkv_out = _c(qkv_out, np.float16)
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    lib().ok_write_kv_cache(_ptr(qkv_out), _ptr(k_cache), _ptr(v_cache), pos, q_dim, kv_dim)


def rope_append(qkv_out, k_cache, v_cache, cos, sin, pos, n_q_heads, n_kv_heads, head_dim):
    """Returns the rotated qkv_out copy; k_cache / v_cache are updated in place."""
    qkv = _c(qkv_out, np.float16).copy()
    assert k_cache.dtype == np.float16 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float16 and v_cache.flags.c_contiguous
    cos = _c(cos, np.float32)
    sin = _c(sin, np.float32)
    lib().ok_rope_append(_ptr(qkv), _ptr(k_cache), _ptr(v_cache), _ptr(cos), _ptr(sin), pos,
                         n_q_heads, n_kv_heads, head_dim)
    return qkv


# ---- a5 -------------------------------------------------------------------
def cached_attention(q, k_cache, v_cache, seq_len, n_q_heads, n_kv_heads, head_dim, threads=1):
    q = _c(q, np.float16)
    k_cache = _c(k_cache, np.float16)
    v_cache = _c(v_cache, np.float16)
    out = np.empty(n_q_heads * head_dim, np.float16)
    if threads > 1:
        lib().ok_cached_attention_mt(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len,
                                     head_dim, n_q_heads, n_kv_heads, threads)
    else:
        lib().ok_cached_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len,
                                  head_dim, n_q_heads, n_kv_heads)
    return out


def cached_attention_f64(q, k_cache, v_cache, seq_len, n_q_heads, n_kv_heads, head_dim):
    q = _c(q, np.float16)
    k_cache = _c(k_cache, np.float16)
    v_cache = _c(v_cache, np.float16)
    out = np.empty(n_q_heads * head_dim, np.float64)
    lib().ok_cached_attention_f64(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), seq_len,
                                  head_dim, n_q_heads, n_kv_heads)
    return out


# ---- b2: prefill -------------------------------------------------------------
def prefill_attention(q, k_cache, v_cache, p0, n, kv_len, n_q_heads, n_kv_heads, head_dim,
                      threads=1):
    """q: [n, q_stride] fp16 (Q heads in the first n_q_heads*head_dim columns)."""
    q = _c(q, np.float16)
    k_cache = _c(k_cache, np.float16)
    v_cache = _c(v_cache, np.float16)
    q_dim = n_q_heads * head_dim
    out = np.empty((n, q_dim), np.float16)
    lib().ok_prefill_attention(_ptr(q), q.shape[-1], _ptr(k_cache), _ptr(v_cache), _ptr(out),
                               q_dim, p0, n, kv_len, head_dim, n_q_heads, n_kv_heads, threads)
    return out


def prefill_attention_f64(q, k_cache, v_cache, p0, n, kv_len, n_q_heads, n_kv_heads, head_dim):
    q = _c(q, np.float16)
    k_cache = _c(k_cache, np.float16)
    v_cache = _c(v_cache, np.float16)
    out = np.empty((n, n_q_heads * head_dim), np.float64)
    lib().ok_prefill_attention_f64(_ptr(q), q.shape[-1], _ptr(k_cache), _ptr(v_cache),
                                   _ptr(out), p0, n, kv_len, head_dim, n_q_heads, n_kv_heads)
    return out


def prefill_rope_append(qkv, k_cache, v_cache, cos, sin, p0, n_q_heads, n_kv_heads, head_dim):
    """Returns the rotated qkv rows; k_cache / v_cache (C-contiguous fp16) are updated."""
    qkv = np.array(qkv, np.float16, order="C", copy=True)
    assert k_cache.dtype == np.float16 and k_cache.flags.c_contiguous
    assert v_cache.dtype == np.float16 and v_cache.flags.c_contiguous
    cos = _c(cos, np.float32)
    sin = _c(sin, np.float32)
    lib().ok_prefill_rope_append(_ptr(qkv), qkv.shape[0], _ptr(k_cache), _ptr(v_cache),
                                 _ptr(cos), _ptr(sin), p0, n_q_heads, n_kv_heads, head_dim)
    return qkv


# ---- a8 -------------------------------------------------------------------
def e4m3_decode_table():
    return np.array([lib().ok_e4m3_decode(c) for c in range(256)], np.float32)


def e4m3_encode(x):
    x = _c(x, np.float32).ravel()
    return np.array([lib().ok_e4m3_encode(float(v)) for v in x], np.uint8)


def fp8_quantize(x_f16, scale):
    x = _c(x_f16, np.float16)
    out = np.empty(x.shape, np.uint8)
    lib().ok_fp8_quantize_f16(_ptr(x), _ptr(out), x.size, scale)
    return out


# ---- a7 -------------------------------------------------------------------
def paged_gather(slab, block_table, seq_len, block_size, kv_dim):
    slab = np.ascontiguousarray(slab)
    table = _c(block_table, np.int32)
    out = np.empty((seq_len, kv_dim), slab.dtype)
    lib().ok_paged_gather(_ptr(slab), _ptr(table), seq_len, block_size, kv_dim,
                          slab.dtype.itemsize, _ptr(out))
    return out


def paged_attention_f16(q, k_slab, v_slab, block_table, seq_len, block_size, n_q_heads,
                        n_kv_heads, head_dim):
    q = _c(q, np.float16)
    k_slab = _c(k_slab, np.float16)
    v_slab = _c(v_slab, np.float16)
    table = _c(block_table, np.int32)
    out = np.empty(n_q_heads * head_dim, np.float16)
    lib().ok_paged_attention_f16(_ptr(q), _ptr(k_slab), _ptr(v_slab), _ptr(table), seq_len,
                                 block_size, _ptr(out), head_dim, n_q_heads, n_kv_heads)
    return out


def paged_attention_fp8(q, k_slab, v_slab, k_scales, v_scales, block_table, seq_len, block_size,
                        n_q_heads, n_kv_heads, head_dim):
    q = _c(q, np.float16)
    k_slab = _c(k_slab, np.uint8)
    v_slab = _c(v_slab, np.uint8)
    ks = _c(k_scales, np.float32)
    vs = _c(v_scales, np.float32)
    table = _c(block_table, np.int32)
    out = np.empty(n_q_heads * head_dim, np.float16)
    lib().ok_paged_attention_fp8(_ptr(q), _ptr(k_slab), _ptr(v_slab), _ptr(ks), _ptr(vs),
                                 _ptr(table), seq_len, block_size, _ptr(out), head_dim, n_q_heads,
                                 n_kv_heads)
    return out


def paged_write_f16(k_row, v_row, k_slab, v_slab, slot, kv_dim):
    """In place on the slabs."""
    k_row = _c(k_row, np.float16)
    v_row = _c(v_row, np.float16)
    lib().ok_paged_write_f16(_ptr(k_row), _ptr(v_row), _ptr(k_slab), _ptr(v_slab), slot, kv_dim)


def paged_write_fp8(k_row, v_row, k_slab, v_slab, slot, kv_dim, head_dim, k_scales, v_scales):
    """In place on the uint8 slabs."""
    k_row = _c(k_row, np.float16)
    v_row = _c(v_row, np.float16)
    ks = _c(k_scales, np.float32)
    vs = _c(v_scales, np.float32)
    lib().ok_paged_write_fp8(_ptr(k_row), _ptr(v_row), _ptr(k_slab), _ptr(v_slab), slot, kv_dim,
                             head_dim, _ptr(ks), _ptr(vs))


def w8a16_gemv(w, x, scales, group_size=128):
    """y[n] = sum_k e4m3(w[n,k]) * scales[n, k/group_size] * x[k] in the reference
    kernel's fp32 summation order, rounded to fp16 (qkv_gemm.cu:32-110).
    w: uint8 [n, k] E4M3 codes, x: float16 [k], scales: float16 [n, k/group_size]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float16)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    n, k = w.shape
    assert x.shape == (k,) and scales.shape == (n, k // group_size)
    y = np.empty(n, dtype=np.float16)
    lib().ok_w8a16_gemv(w.ctypes.data, x.ctypes.data, scales.ctypes.data, y.ctypes.data, n, k, group_size)
    return y


def w8a16_gemv_f64(w, x, scales, group_size=128):
    """The same products summed in float64 (an order-free reference)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float16)
    scales = np.ascontiguousarray(scales, dtype=np.float16)
    n, k = w.shape
    y = np.empty(n, dtype=np.float64)
    lib().ok_w8a16_gemv_f64(w.ctypes.data, x.ctypes.data, scales.ctypes.data, y.ctypes.data, n, k, group_size)
    return y
