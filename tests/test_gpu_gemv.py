"""GPU parity of the W8A16 GEMV and the fused decode QKV projection + RoPE + append.

GEMV: within half an fp16 ulp plus the fp32 summation bound of the float64
oracle, and within one ulp plus that bound of the reference-order fp32 oracle
(qkv_gemm.cu:32-110). Fused kernel: bit for bit af_w8a16_gemv followed by
af_rope_append, whole caches compared (untouched rows included).
"""
import numpy as np
import pytest

import atomflow_amd
import oracle
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import HD, KV_DIM, NKV, NQ, QKV, THETA, fp16_ulp, gemv_abs_terms, gemv_case

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def gemv_gpu(w, x, s, group=128):
    n, k = w.shape
    y = dev.DeviceBuffer(n * 2)
    kv.launch_w8a16_gemv(up(x), up(w), up(s), y, n, k, group)
    return y.download(np.float16, (n,))


@pytest.mark.parametrize("n,k", [(QKV, 3072), (3072, 3072), (3072, 8192), (13, 3072), (37, 1040)])
def test_gemv_parity(gpu, n, k):
    say(f"gemv n={n} k={k}")
    group = 128 if k % 128 == 0 else 16
    w, x, s = gemv_case(n, k, 0xA70F10 + 7 * n + k, group=group)
    got = gemv_gpu(w, x, s, group).astype(np.float64)
    y64 = oracle.w8a16_gemv_f64(w, x, s, group)
    bound = k * 2.0 ** -24 * gemv_abs_terms(w, x, s, group)
    assert np.all(np.isfinite(got))
    err = np.abs(got - y64)
    assert np.all(err <= 0.5 * fp16_ulp(y64) + bound), f"max err {err.max():.3e}"
    ref = oracle.w8a16_gemv(w, x, s, group).astype(np.float64)
    assert np.all(np.abs(got - ref) <= fp16_ulp(y64) + 2 * bound)


@pytest.mark.parametrize("n0,n1,k", [(8192, 8192, 3072), (37, 5120, 1040), (3072, 13, 8192)])
def test_gemv_pair_equals_two_gemvs(gpu, n0, n1, k):
    """af_w8a16_gemv_pair (gate and up in one launch): each output bit for bit the
    single af_w8a16_gemv of its matrix, and within the oracle bound."""
    say(f"gemv pair n0={n0} n1={n1} k={k}")
    group = 128 if k % 128 == 0 else 16
    w0, x, s0 = gemv_case(n0, k, 0xA70F20 + n0, group=group)
    w1, _, s1 = gemv_case(n1, k, 0xA70F21 + n1, group=group)
    y0, y1 = dev.DeviceBuffer(n0 * 2), dev.DeviceBuffer(n1 * 2)
    kv.launch_w8a16_gemv_pair(up(x), up(w0), up(s0), y0, n0, up(w1), up(s1), y1, n1, k, group)
    got0 = y0.download(np.float16, (n0,))
    got1 = y1.download(np.float16, (n1,))
    assert np.array_equal(got0.view(np.uint16), gemv_gpu(w0, x, s0, group).view(np.uint16))
    assert np.array_equal(got1.view(np.uint16), gemv_gpu(w1, x, s1, group).view(np.uint16))
    for w, s, got in ((w0, s0, got0), (w1, s1, got1)):
        y64 = oracle.w8a16_gemv_f64(w, x, s, group)
        bound = k * 2.0 ** -24 * gemv_abs_terms(w, x, s, group)
        assert np.all(np.abs(got.astype(np.float64) - y64) <= 0.5 * fp16_ulp(y64) + bound)


def test_gemv_identity_and_nan_codes(gpu):
    say("gemv identity weights, NaN code propagates to its row only")
    n = k = 1024
    w = np.zeros((n, k), np.uint8)
    w[np.arange(n), np.arange(n)] = 0x38
    x = np.random.default_rng(3).standard_normal(k).astype(np.float16)
    s = np.ones((n, k // 128), np.float16)
    assert np.array_equal(gemv_gpu(w, x, s).view(np.uint16), x.view(np.uint16))
    w[5, 900] = 0x7F  # E4M3FN NaN
    y = gemv_gpu(w, x, s)
    assert np.isnan(y[5]) and np.array_equal(np.delete(y, 5).view(np.uint16),
                                             np.delete(x, 5).view(np.uint16))


def test_gemv_rejects_bad_shapes(gpu):
    say("gemv argument checks")
    w, x, s = gemv_case(16, 1024, 5)
    y = dev.DeviceBuffer(32)
    lib = atomflow_amd.lib()
    assert lib.af_w8a16_gemv(up(x).ptr, up(w).ptr, up(s).ptr, y.ptr, 16, 1000, 128, None) < 0
    assert lib.af_w8a16_gemv(up(x).ptr, up(w).ptr, up(s).ptr, y.ptr, 16, 1024, 100, None) < 0
    assert lib.af_w8a16_gemv(up(x).ptr, up(w).ptr, up(s).ptr, y.ptr, 0, 1024, 128, None) < 0


def _qkv_case(seed, max_seq=64, filled=20):
    w, x, s = gemv_case(QKV, 3072, seed)
    r = np.random.default_rng(seed + 1)
    k_cache = r.standard_normal((max_seq, KV_DIM)).astype(np.float16)
    v_cache = r.standard_normal((max_seq, KV_DIM)).astype(np.float16)
    k_cache[filled:] = np.float16(7.0)  # canaries
    v_cache[filled:] = np.float16(-7.0)
    return w, x, s, k_cache, v_cache


@pytest.mark.parametrize("pos", [0, 19, 63])
def test_qkv_rope_append_equals_gemv_then_rope_append(gpu, pos):
    say(f"fused qkv+rope+append pos={pos}")
    max_seq = 64
    w, x, s, kc, vc = _qkv_case(0xA70F11 + pos, max_seq)
    d_cos, d_sin = dev.DeviceBuffer(max_seq * 64 * 4), dev.DeviceBuffer(max_seq * 64 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA)
    dw, dx, ds = up(w), up(x), up(s)
    # fused
    qkv_f, kc_f, vc_f = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    kv.launch_qkv_rope_append(dx, dw, ds, 3072, qkv_f, kc_f, vc_f, d_cos, d_sin, pos, max_seq,
                              NQ, NKV, HD)
    # two-call sequence
    qkv_u, kc_u, vc_u = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    kv.launch_w8a16_gemv(dx, dw, ds, qkv_u, QKV, 3072)
    y = qkv_u.download(np.float16, (QKV,))
    kv.launch_rope_append(qkv_u, kc_u, vc_u, d_cos, d_sin, pos, max_seq, NQ, NKV, HD)
    for a, b in [(qkv_f, qkv_u), (kc_f, kc_u), (vc_f, vc_u)]:
        assert np.array_equal(a.download(np.uint16), b.download(np.uint16))
    # and the rotation on the projection equals the oracle's rope_append
    cos, sin = oracle.rope_table(max_seq, HD, THETA)
    kc_o, vc_o = kc.copy(), vc.copy()
    qkv_o = oracle.rope_append(y, kc_o, vc_o, cos, sin, pos, NQ, NKV, HD)
    assert np.array_equal(qkv_f.download(np.uint16), qkv_o.view(np.uint16))
    assert np.array_equal(kc_f.download(np.uint16, kc.shape), kc_o.view(np.uint16))
    assert np.array_equal(vc_f.download(np.uint16, vc.shape), vc_o.view(np.uint16))


def test_qkv_rope_append_device_position_and_range(gpu):
    say("fused qkv: device position, out-of-range writes nothing")
    max_seq = 32
    w, x, s, kc, vc = _qkv_case(0xA70F19, max_seq, filled=10)
    d_cos, d_sin = dev.DeviceBuffer(max_seq * 64 * 4), dev.DeviceBuffer(max_seq * 64 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA)
    dw, dx, ds = up(w), up(x), up(s)
    ref_q, ref_k, ref_v = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    kv.launch_qkv_rope_append(dx, dw, ds, 3072, ref_q, ref_k, ref_v, d_cos, d_sin, 10, max_seq,
                              NQ, NKV, HD)
    d_pos = up(np.array([10], np.int32))
    q1, k1, v1 = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    kv.launch_qkv_rope_append(dx, dw, ds, 3072, q1, k1, v1, d_cos, d_sin, 0, max_seq, NQ, NKV, HD,
                              d_pos=d_pos)
    for a, b in [(q1, ref_q), (k1, ref_k), (v1, ref_v)]:
        assert np.array_equal(a.download(np.uint16), b.download(np.uint16))
    bad = up(np.array([max_seq], np.int32))
    status = up(np.zeros(1, np.int32))
    q2 = up(np.zeros(QKV, np.float16))
    k2, v2 = up(kc), up(vc)
    kv.launch_qkv_rope_append(dx, dw, ds, 3072, q2, k2, v2, d_cos, d_sin, 0, max_seq, NQ, NKV, HD,
                              d_pos=bad, d_status=status)
    assert status.download(np.int32)[0] == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert not q2.download(np.uint16).any()
    assert np.array_equal(k2.download(np.uint16, kc.shape), kc.view(np.uint16))
    assert np.array_equal(v2.download(np.uint16, vc.shape), vc.view(np.uint16))


def test_qkv_step_graph_replay(gpu):
    say("graph: [qkv+rope+append(d_pos), pos += 1] x 3 replays == 3 eager steps")
    max_seq = 32
    w, x, s, kc, vc = _qkv_case(0xA70F1A, max_seq, filled=4)
    d_cos, d_sin = dev.DeviceBuffer(max_seq * 64 * 4), dev.DeviceBuffer(max_seq * 64 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA)
    dw, dx, ds = up(w), up(x), up(s)
    stream = dev.Stream()
    e_q, e_k, e_v = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    for p in (4, 5, 6):
        kv.launch_qkv_rope_append(dx, dw, ds, 3072, e_q, e_k, e_v, d_cos, d_sin, p, max_seq, NQ,
                                  NKV, HD, stream=stream)
    g_q, g_k, g_v = dev.DeviceBuffer(QKV * 2), up(kc), up(vc)
    d_pos = up(np.array([4], np.int32))
    stream.sync()

    def body():
        kv.launch_qkv_rope_append(dx, dw, ds, 3072, g_q, g_k, g_v, d_cos, d_sin, 0, max_seq, NQ,
                                  NKV, HD, d_pos=d_pos, stream=stream)
        dev.add_i32(d_pos.ptr, 1, 1, stream)

    graph = dev.Graph.capture(stream, body)
    for _ in range(3):
        graph.launch(stream)
        stream.sync()
    graph.destroy()
    assert d_pos.download(np.int32)[0] == 7
    for a, b in [(g_q, e_q), (g_k, e_k), (g_v, e_v)]:
        assert np.array_equal(a.download(np.uint16), b.download(np.uint16))
