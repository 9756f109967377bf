"""Seeded synthetic inputs shared by the tests (numpy PCG64, N(0,1) -> fp16 RNE).

Seed convention: 0xA70F10 + n for BASELINE config n (1-based), plus a small
offset per tensor.
"""
import numpy as np

NQ, NKV, HD = 24, 8, 128          # Llama-3.2-3B attention shape
Q_DIM, KV_DIM = NQ * HD, NKV * HD
QKV = Q_DIM + 2 * KV_DIM
THETA = 500000.0
SEED_BASE = 0xA70F10


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def randn_f16(shape, seed, scale=1.0):
    return (rng(seed).standard_normal(shape) * scale).astype(np.float16)


def contiguous_case(max_seq, filled, seed, nq=NQ, nkv=NKV, hd=HD):
    """qkv row + caches with rows [0, filled) ~ N(0,1), the rest zero."""
    kv_dim = nkv * hd
    qkv = randn_f16((nq + 2 * nkv) * hd, seed)
    k = np.zeros((max_seq, kv_dim), np.float16)
    v = np.zeros((max_seq, kv_dim), np.float16)
    k[:filled] = randn_f16((filled, kv_dim), seed + 1)
    v[:filled] = randn_f16((filled, kv_dim), seed + 2)
    return qkv, k, v


# Attention tolerance: fp16 KV within max-abs 2e-3 /
# rel 1e-2, FP8 KV within 5e-2. Two separate bounds, both enforced literally:
#   max |got - ref|                       <= atol  (2e-3 fp16 KV, 5e-2 FP8 KV)
#   ||got - ref||_2 / ||ref||_2           <= rtol  (1e-2)
# The relative bound is norm-wise: an elementwise ratio is unbounded where the
# reference is near zero, and there the absolute bound already holds the error.
ATOL_F16, RTOL_F16 = 2e-3, 1e-2
ATOL_FP8, RTOL_FP8 = 5e-2, 1e-2


def assert_attn_close(got, ref, atol=ATOL_F16, rtol=RTOL_F16, what=""):
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    assert g.shape == r.shape or g.size == r.size, (what, g.shape, r.shape)
    g, r = g.ravel(), r.ravel()
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    err = np.abs(g - r)
    max_abs = float(err.max()) if err.size else 0.0
    norm_ref = float(np.linalg.norm(r))
    rel = float(np.linalg.norm(g - r)) / norm_ref if norm_ref > 0 else max_abs
    print(f"[err] {what}: max abs {max_abs:.3e} (bar {atol:g}), rel {rel:.3e} (bar {rtol:g})",
          flush=True)
    assert max_abs <= atol, (f"{what}: max abs err {max_abs:.3e} > {atol:g} at element "
                             f"{int(err.argmax())} (got {g[err.argmax()]:.6f}, "
                             f"ref {r[err.argmax()]:.6f})")
    assert rel <= rtol, f"{what}: relative err {rel:.3e} > {rtol:g}"
    return max_abs


# ---- W8A16 GEMV inputs (FP8 E4M3 weights with fp16 group scales) ------------
_E4M3_POS = None


def _e4m3_positive_values():
    """Finite positive E4M3FN values, indexed by code 0..126 (0x7F is NaN)."""
    global _E4M3_POS
    if _E4M3_POS is None:
        vals = []
        for c in range(127):
            e, m = c >> 3, c & 7
            vals.append(m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10))
        _E4M3_POS = np.array(vals, np.float64)
    return _E4M3_POS


def e4m3_encode_np(x):
    """Round-to-nearest-even E4M3FN codes of float values already within +-448."""
    vals = _e4m3_positive_values()
    a = np.abs(np.asarray(x, np.float64))
    hi = np.clip(np.searchsorted(vals, a), 1, 126)
    lo = hi - 1
    d_lo, d_hi = a - vals[lo], vals[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    return code | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)


def gemv_case(n, k, seed, group=128, wscale=0.05):
    """Weights ~ N(0, wscale) quantised per (row, group) with scale = absmax / 448
    (1 for an all-zero group) in fp16 and RNE E4M3 codes (the convention of
    tools/quantize_weights.py:249-260); activation ~ N(0, 1) fp16."""
    r = rng(seed)
    wf = r.standard_normal((n, k)) * wscale
    g = wf.reshape(n, k // group, group)
    absmax = np.abs(g).max(axis=2)
    scales = np.where(absmax > 0, absmax / 448.0, 1.0).astype(np.float16)
    q = np.clip(g / scales.astype(np.float64)[..., None], -448.0, 448.0)
    codes = e4m3_encode_np(q).reshape(n, k)
    x = r.standard_normal(k).astype(np.float16)
    return codes, x, scales


def gemv_abs_terms(codes, x, scales, group=128):
    """sum_k |e4m3(w) * s * x| per row (float64), the scale of fp32 summation error."""
    vals = np.concatenate([_e4m3_positive_values(), [np.nan]])
    mag = vals[codes & 0x7f]
    n, k = codes.shape
    s = np.repeat(np.abs(scales.astype(np.float64)), group, axis=1)
    return (mag * s * np.abs(x.astype(np.float64))[None, :]).sum(axis=1)


def fp16_ulp(v):
    """Spacing of fp16 values at |v| (2^-24 below the normal range)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)
