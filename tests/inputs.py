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
# rel 1e-2, FP8 KV within 5e-2, read elementwise as |got - ref| <= atol + rtol*|ref|.
ATOL_F16, RTOL_F16 = 2e-3, 1e-2
ATOL_FP8, RTOL_FP8 = 5e-2, 1e-2


def assert_attn_close(got, ref, atol=ATOL_F16, rtol=RTOL_F16, what=""):
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    assert np.all(np.isfinite(g)), f"{what}: non-finite output"
    err = np.abs(g - r)
    bad = err > atol + rtol * np.abs(r)
    assert not bad.any(), (f"{what}: {bad.sum()} elements outside atol={atol} rtol={rtol}; "
                           f"max abs err {err.max():.3e} at {int(err.argmax())}")
    return float(err.max())
