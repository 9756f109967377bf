"""The allocation-free attention entry point (af_cached_attention_noalloc)
against af_cached_attention, through the C ABI, on two calls in a row (the
second with a smaller input), to the attention bar, and against the fp64
oracle."""
import ctypes

import numpy as np
import pytest

import atomflow_amd
import oracle
from atomflow_amd import device as dev
from inputs import HD, KV_DIM, NKV, NQ, Q_DIM, assert_attn_close, contiguous_case

pytestmark = pytest.mark.gpu


def _attend(fn, q, k, v, seq_len, nq, nkv, hd):
    d_q, d_k, d_v = (dev.DeviceBuffer.from_array(a) for a in (q, k, v))
    d_out = dev.DeviceBuffer(nq * hd * 2)
    st = fn(ctypes.c_void_p(d_q.ptr), ctypes.c_void_p(d_k.ptr), ctypes.c_void_p(d_v.ptr),
            ctypes.c_void_p(d_out.ptr), seq_len, hd, nq, nkv, None)
    assert st == 0, atomflow_amd.lib().af_status_string(st)
    dev.synchronize()
    return d_out.download(np.float16)


def test_noalloc_attention_matches_allocating_entry_point(gpu):
    lib = atomflow_amd.lib()
    assert lib.af_cached_attention_noalloc_max_bytes() == 4 * 1024 * 1024 + 128 * 1024
    # two calls in a row: the second with a smaller input (shorter sequence,
    # fewer heads), so it reuses the scratch left behind by the first
    cases = [(8193, NQ, NKV, 8192 + 64, 0xA70F10 + 41), (777, 8, 2, 1024, 0xA70F10 + 42)]
    for seq_len, nq, nkv, max_seq, seed in cases:
        print(f"[case] noalloc seq_len={seq_len} nq={nq} nkv={nkv}", flush=True)
        qkv, k, v = contiguous_case(max_seq, seq_len, seed, nq=nq, nkv=nkv)
        q = qkv[: nq * HD].copy()
        kk, vv = k[:seq_len].copy(), v[:seq_len].copy()
        got = _attend(lib.af_cached_attention_noalloc, q, kk, vv, seq_len, nq, nkv, HD)
        ref = _attend(lib.af_cached_attention, q, kk, vv, seq_len, nq, nkv, HD)
        err = assert_attn_close(got.astype(np.float32), ref.astype(np.float32),
                                what="noalloc vs af_cached_attention")
        # same split count and kernel: the outputs are the same bits
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
        ref64 = oracle.cached_attention_f64(q, kk, vv, seq_len, nq, nkv, HD)
        err64 = assert_attn_close(got.astype(np.float64), ref64, what="noalloc vs fp64 oracle")
        print(f"[case] max abs err vs af_cached_attention {err:.2e}, vs fp64 oracle {err64:.2e}",
              flush=True)


def test_noalloc_rejects_shapes_beyond_the_scratch(gpu):
    lib = atomflow_amd.lib()
    # 128 Q heads x head_dim 128 over 2 KV heads at 200k tokens: 128 splits (more
    # than the combiner form takes, so no CUs are held back for combiners), an
    # 8.2 MiB workspace, more than the array holds. Rejected before any launch,
    # so the (small) buffers are never read.
    assert lib.af_attention_default_splits(200000, 1, 2) == 128
    assert (lib.af_attention_workspace_size(1, 128, 2, 128, 128)
            > lib.af_cached_attention_noalloc_max_bytes())
    d = dev.DeviceBuffer(4096)
    p = ctypes.c_void_p(d.ptr)
    assert lib.af_cached_attention_noalloc(p, p, p, p, 200000, 128, 128, 2, None) == -6
