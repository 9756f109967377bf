"""GPU parity of the batched W8A16 projection (af_w8a16_gemm_batched) and the
paged serving step's fused QKV projection + RoPE + paged append
(af_paged_qkv_rope_append).

Batched projection: every token row within half an fp16 ulp plus the fp32
summation bound of the float64 oracle (the reference's per-token GEMV,
qkv_gemm.cu:32-110), the same bar as af_w8a16_gemv. Fused kernel: bit for bit
the batched projection followed by af_paged_rope_append, whole pool compared.
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


def batched_gpu(w, xs, s, group=128, x_stride=None):
    n, k = w.shape
    m = xs.shape[0]
    stride = x_stride or k
    xb = np.zeros((max(m, 1), stride), np.float16)
    xb[:m, :k] = xs
    y = dev.DeviceBuffer(max(m, 1) * n * 2)
    kv.launch_w8a16_gemm_batched(up(xb), stride, m, up(w), up(s), y, n, n, k, group)
    return y.download(np.float16, (max(m, 1), n))[:m]


@pytest.mark.parametrize("n,k,m,group", [(QKV, 3072, 32, 128), (QKV, 3072, 1, 128),
                                         (3072, 3072, 7, 128), (8192, 3072, 45, 128),
                                         (3072, 8192, 16, 128), (100, 1024, 33, 128),
                                         (512, 1024, 20, 32), (256, 768, 5, 96), (272, 640, 3, 64)])
def test_gemm_batched_parity(gpu, n, k, m, group):
    """Group sizes 32 and 96 take the 32-k chunk path (8 weight bytes per MFMA),
    the others the 64-k path with the activations staged through LDS."""
    say(f"batched gemm n={n} k={k} m={m} group={group}")
    w, _, s = gemv_case(n, k, 0xA70F30 + n + k, group=group)
    xs = np.random.default_rng(m + n).standard_normal((m, k)).astype(np.float16)
    got = batched_gpu(w, xs, s, group, x_stride=k + (8 if m % 2 else 0)).astype(np.float64)
    assert np.all(np.isfinite(got))
    for i in range(m):
        y64 = oracle.w8a16_gemv_f64(w, xs[i], s, group)
        bound = k * 2.0 ** -24 * gemv_abs_terms(w, xs[i], s, group)
        err = np.abs(got[i] - y64)
        assert np.all(err <= 0.5 * fp16_ulp(y64) + bound), f"token {i}: max err {err.max():.3e}"


def test_gemm_batched_rejects_bad_shapes(gpu):
    say("batched gemm argument checks")
    w, x, s = gemv_case(64, 1024, 5)
    lib = atomflow_amd.lib()
    y = dev.DeviceBuffer(64 * 2)
    dx, dw, ds = up(x), up(w), up(s)
    call = lib.af_w8a16_gemm_batched
    assert call(dx.ptr, 1024, 1, dw.ptr, ds.ptr, y.ptr, 64, 64, 1000, 128,
                None) == atomflow_amd.AF_ERR_UNSUPPORTED
    assert call(dx.ptr, 1000, 1, dw.ptr, ds.ptr, y.ptr, 64, 64, 1024, 128,
                None) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(dx.ptr, 1024, 1, dw.ptr, ds.ptr, y.ptr, 32, 64, 1024, 128,
                None) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(dx.ptr, 1024, 0, dw.ptr, ds.ptr, y.ptr, 64, 64, 1024, 128, None) == 0


@pytest.mark.parametrize("fp8,group,m,bad", [(False, 128, 19, 5), (True, 128, 19, 5),
                                              (False, 32, 19, 5), (False, 128, 1, None),
                                              (True, 128, 1, None), (True, 128, 1, "pos"),
                                              (False, 128, 1, "slot")])
def test_paged_qkv_rope_append_equals_unfused(gpu, fp8, group, m, bad):
    """m = 1 takes the single-token GEMV form; it must still equal the batched
    projection (itself the GEMV at m = 1) followed by the paged append."""
    say(f"paged qkv rope append, fp8 {fp8}, group {group}, m {m}, out of range {bad}")
    k_in, bs, total, max_pos = 3072, 16, 96, 700
    w, _, s = gemv_case(QKV, k_in, 0xA70F31, group=group)
    xs = np.random.default_rng(3).standard_normal((m, k_in)).astype(np.float16)
    r = np.random.default_rng(4)
    slots = r.permutation(total * bs)[:m].astype(np.int64)
    positions = r.integers(0, max_pos, m).astype(np.int32)
    # an out-of-range token: its projection stays unrotated, nothing is appended
    bad_row = None
    if bad == "pos" or isinstance(bad, int):
        bad_row = bad if isinstance(bad, int) else 0
        positions[bad_row] = max_pos
    elif bad == "slot":
        bad_row = 0
        slots[0] = total * bs
    esz = 1 if fp8 else 2
    pool_bytes = 2 * 2 * total * bs * KV_DIM * esz  # two layers
    init = r.integers(0, 256, pool_bytes, dtype=np.uint8)
    scales = up(np.full((2, 2, NKV), 0.04, np.float32)) if fp8 else None
    dtype = atomflow_amd.AF_KV_FP8_E4M3 if fp8 else atomflow_amd.AF_KV_FP16
    pools = []
    for _ in range(2):
        buf = up(init)
        pools.append((buf, kv.make_pool(buf, dtype, bs, 2, NKV, HD, total, scales)))
    c, sn = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(sn)
    dx, dw, ds = up(xs), up(w), up(s)
    d_slots, d_pos = up(slots), up(positions)
    # fused
    q1 = dev.DeviceBuffer(m * QKV * 2)
    st = up(np.zeros(1, np.int32))
    kv.launch_paged_qkv_rope_append(dx, k_in, m, dw, ds, k_in, q1, pools[0][1], 1, d_slots,
                                    d_pos, d_c, d_s, max_pos, NQ, d_status=st, group_size=group)
    # unfused: batched projection, then the paged append
    q2 = dev.DeviceBuffer(m * QKV * 2)
    kv.launch_w8a16_gemm_batched(dx, k_in, m, dw, ds, q2, QKV, QKV, k_in, group)
    kv.launch_paged_rope_append(q2, m, pools[1][1], 1, d_slots, d_pos, d_c, d_s, max_pos, NQ)
    assert np.array_equal(q1.download(np.uint16, (m, QKV)), q2.download(np.uint16, (m, QKV)))
    p1 = pools[0][0].download(np.uint8, (pool_bytes,))
    p2 = pools[1][0].download(np.uint8, (pool_bytes,))
    assert np.array_equal(p1, p2)
    plain = batched_gpu(w, xs, s, group)
    if m == 1:  # the batched projection of one token is the GEMV, bit for bit
        y = dev.DeviceBuffer(QKV * 2)
        kv.launch_w8a16_gemv(dx, dw, ds, y, QKV, k_in, group)
        assert np.array_equal(plain[0].view(np.uint16), y.download(np.uint16, (QKV,)))
    status = st.download(np.int32, (1,))[0]
    if bad_row is None:
        assert status == 0
        assert not np.array_equal(p1, init)  # something was appended
        # the appended row matches the oracle's append of the rotated projection
        if m == 1:
            host = init.reshape(2, 2, total * bs, KV_DIM * esz).copy()
            rq = oracle.rope_append(plain[0], np.zeros((1, KV_DIM), np.float16),
                                    np.zeros((1, KV_DIM), np.float16), c[positions[0]:],
                                    sn[positions[0]:], 0, NQ, NKV, HD)
            assert np.array_equal(q1.download(np.uint16, (QKV,)), rq.view(np.uint16))
            kr, vr = rq[NQ * HD:NQ * HD + KV_DIM], rq[NQ * HD + KV_DIM:]
            if fp8:
                hk = host[1, 0].reshape(-1, KV_DIM)
                hv = host[1, 1].reshape(-1, KV_DIM)
                oracle.paged_write_fp8(kr, vr, hk, hv, int(slots[0]), KV_DIM, HD,
                                       np.full(NKV, 0.04, np.float32),
                                       np.full(NKV, 0.04, np.float32))
            else:
                host[1, 0, slots[0]] = kr.view(np.uint8)
                host[1, 1, slots[0]] = vr.view(np.uint8)
            assert np.array_equal(p1, host.reshape(-1))
    else:
        assert status == atomflow_amd.AF_ERR_OUT_OF_RANGE
        assert np.array_equal(q1.download(np.uint16, (m, QKV))[bad_row],
                              plain[bad_row].view(np.uint16))
        if m == 1:
            assert np.array_equal(p1, init)  # nothing appended


def test_paged_qkv_rope_append_graph_replays(gpu):
    """Captured in a hipGraph and replayed three times (device positions advanced
    between replays by the eager side): every replay equals the eager launch."""
    say("paged qkv rope append under graph replay")
    k_in, m, bs, total, max_pos = 3072, 8, 16, 64, 256
    w, _, s = gemv_case(QKV, k_in, 0xA70F32, group=128)
    xs = np.random.default_rng(6).standard_normal((m, k_in)).astype(np.float16)
    slots = np.arange(m, dtype=np.int64) * 5
    c, sn = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(sn)
    dx, dw, ds = up(xs), up(w), up(s)
    pool_bytes = 2 * total * bs * KV_DIM * 2
    bufs = [dev.DeviceBuffer(pool_bytes) for _ in range(2)]
    for b in bufs:
        b.fill_u32(0, None)
    dev.synchronize()
    pools = [kv.make_pool(b, atomflow_amd.AF_KV_FP16, bs, 1, NKV, HD, total) for b in bufs]
    outs = [dev.DeviceBuffer(m * QKV * 2) for _ in range(2)]
    d_slots = up(slots)
    d_pos = [up(np.zeros(m, np.int32)) for _ in range(2)]
    stream = dev.Stream()
    run = lambda i: kv.launch_paged_qkv_rope_append(dx, k_in, m, dw, ds, k_in, outs[i], pools[i],
                                                    0, d_slots, d_pos[i], d_c, d_s, max_pos, NQ,
                                                    stream=stream)
    graph = dev.Graph.capture(stream, lambda: run(1))
    for step in range(3):
        pos = (np.arange(m) * 7 + 11 * step).astype(np.int32)
        for dp in d_pos:
            dp.upload(pos)
        run(0)
        graph.launch(stream)
        stream.sync()
        assert np.array_equal(outs[0].download(np.uint16, (m, QKV)),
                              outs[1].download(np.uint16, (m, QKV))), f"replay {step}"
        assert np.array_equal(bufs[0].download(np.uint8, (pool_bytes,)),
                              bufs[1].download(np.uint8, (pool_bytes,))), f"replay {step}"
    graph.destroy()
