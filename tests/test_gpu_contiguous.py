"""GPU parity of the contiguous KV path (libatomflow_kv.so vs the CPU oracle).

Bit-exact: RoPE table, RoPE, KV write, fused RoPE+append (whole caches are
compared, so untouched rows are checked too). Attention: within the fp16 bar of
both the fp32 oracle and the fp64 oracle. Graph replay: byte-identical to the
same number of eager steps.
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_ERR_TIMEOUT
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import (HD, KV_DIM, NKV, NQ, Q_DIM, SEED_BASE, THETA, assert_attn_close,
                    contiguous_case, randn_f16)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def test_rope_table_device_equals_oracle(gpu):
    say("rope table 8192 x 64")
    max_seq = 8192
    d_cos, d_sin = dev.DeviceBuffer(max_seq * 64 * 4), dev.DeviceBuffer(max_seq * 64 * 4)
    kv.build_rope_cache(d_cos, d_sin, max_seq, HD, THETA)
    c, s = oracle.rope_table(max_seq, HD, THETA)
    assert np.array_equal(d_cos.download(np.float32).view(np.uint32), c.ravel().view(np.uint32))
    assert np.array_equal(d_sin.download(np.float32).view(np.uint32), s.ravel().view(np.uint32))


@pytest.mark.parametrize("seq_len", [1, 3])
def test_launch_rope_reference_shape(gpu, seq_len):
    say(f"launch_rope seq_len={seq_len}")
    c, s = oracle.rope_table(64, HD, THETA)
    q = randn_f16((seq_len, Q_DIM), 101 + seq_len)
    k = randn_f16((seq_len, KV_DIM), 102 + seq_len)
    d_q, d_k, d_c, d_s = up(q), up(k), up(c), up(s)
    row = 17 * (HD // 2) * 4  # table rows start at position 17
    kv.launch_rope(d_q, d_k, d_c.ptr + row, d_s.ptr + row, seq_len, NKV, NQ, HD)
    rq, rk = oracle.rope(q, k, c[17:17 + seq_len], s[17:17 + seq_len], NQ, NKV, HD)
    assert np.array_equal(bits(d_q.download(np.float16)), bits(rq).ravel())
    assert np.array_equal(bits(d_k.download(np.float16)), bits(rk).ravel())


def test_write_kv_cache_bit_exact(gpu):
    say("write_kv_cache pos 37")
    qkv, k, v = contiguous_case(128, 37, 111)
    d_qkv, d_k, d_v = up(qkv), up(k), up(v)
    kv.launch_write_kv_cache(d_qkv, d_k, d_v, 37, Q_DIM, KV_DIM, 128)
    oracle.write_kv_cache(qkv, k, v, 37, Q_DIM, KV_DIM)
    assert np.array_equal(bits(d_k.download(np.float16)), bits(k).ravel())
    assert np.array_equal(bits(d_v.download(np.float16)), bits(v).ravel())


def test_write_kv_cache_rejects_out_of_range(gpu):
    qkv, k, v = contiguous_case(16, 0, 112)
    d_qkv, d_k, d_v = up(qkv), up(k), up(v)
    with pytest.raises(Exception):
        kv.launch_write_kv_cache(d_qkv, d_k, d_v, 16, Q_DIM, KV_DIM, 16)


@pytest.mark.parametrize("pos", [0, 1, 511, 512, 4095])
def test_rope_append_bit_exact(gpu, pos):
    say(f"rope_append pos={pos}")
    max_seq = 4096
    c, s = oracle.rope_table(max_seq, HD, THETA)
    qkv, k, v = contiguous_case(max_seq, pos, SEED_BASE + 1 + pos)
    d_qkv, d_k, d_v, d_c, d_s = up(qkv), up(k), up(v), up(c), up(s)
    kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, pos, max_seq, NQ, NKV, HD)
    rq = oracle.rope_append(qkv, k, v, c, s, pos, NQ, NKV, HD)
    assert np.array_equal(bits(d_qkv.download(np.float16)), bits(rq))
    assert np.array_equal(bits(d_k.download(np.float16)), bits(k).ravel())
    assert np.array_equal(bits(d_v.download(np.float16)), bits(v).ravel())


def test_rope_append_device_pos_and_status(gpu):
    say("rope_append device pos + out-of-range status")
    max_seq = 64
    c, s = oracle.rope_table(max_seq, HD, THETA)
    qkv, k, v = contiguous_case(max_seq, 20, 121)
    d_qkv, d_k, d_v, d_c, d_s = up(qkv), up(k), up(v), up(c), up(s)
    d_pos = up(np.array([20], np.int32))
    d_st = up(np.array([0], np.int32))
    kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, -1, max_seq, NQ, NKV, HD, d_pos=d_pos,
                          d_status=d_st)
    rq = oracle.rope_append(qkv, k, v, c, s, 20, NQ, NKV, HD)
    assert np.array_equal(bits(d_qkv.download(np.float16)), bits(rq))
    assert np.array_equal(bits(d_k.download(np.float16)), bits(k).ravel())
    assert d_st.download(np.int32)[0] == 0
    # a device position at capacity writes nothing and reports AF_ERR_OUT_OF_RANGE
    d_pos.upload(np.array([max_seq], np.int32))
    before = d_k.download(np.float16)
    kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, -1, max_seq, NQ, NKV, HD, d_pos=d_pos,
                          d_status=d_st)
    assert d_st.download(np.int32)[0] == -4
    assert np.array_equal(bits(d_k.download(np.float16)), bits(before))


def _attention_case(L, max_seq, nq, nkv, hd, seed):
    kvd = nkv * hd
    q = randn_f16(nq * hd, seed)
    k = np.zeros((max_seq, kvd), np.float16)
    v = np.zeros((max_seq, kvd), np.float16)
    k[:L] = randn_f16((L, kvd), seed + 1)
    v[:L] = randn_f16((L, kvd), seed + 2)
    return q, k, v


@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 63, 64, 65, 127, 513, 1025, 4097, 8193])
def test_cached_attention_llama_shape(gpu, L):
    say(f"cached_attention L={L}")
    max_seq = L + 7
    q, k, v = _attention_case(L, max_seq, NQ, NKV, HD, 200 + L)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_cached_attention(d_q, d_k, d_v, d_o, L, HD, NQ, NKV)
    got = d_o.download(np.float16)
    ref32 = oracle.cached_attention(q, k, v, L, NQ, NKV, HD)
    ref64 = oracle.cached_attention_f64(q, k, v, L, NQ, NKV, HD)
    assert_attn_close(got, ref64, what=f"L={L} vs fp64")
    assert_attn_close(got, ref32, what=f"L={L} vs fp32 oracle")
    if L == 1:  # softmax of one score is exactly 1: out = V row
        assert np.array_equal(bits(got), bits(ref32))


@pytest.mark.parametrize("shape", [(8, 8, 128), (16, 4, 128), (8, 1, 128), (32, 8, 128),
                                   (16, 8, 64), (4, 2, 64)])
@pytest.mark.parametrize("L", [1, 100, 1500])
def test_cached_attention_gqa_ratios(gpu, shape, L):
    nq, nkv, hd = shape
    say(f"cached_attention nq={nq} nkv={nkv} hd={hd} L={L}")
    q, k, v = _attention_case(L, L, nq, nkv, hd, 300 + L + nq)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = dev.DeviceBuffer(nq * hd * 2)
    kv.launch_cached_attention(d_q, d_k, d_v, d_o, L, hd, nq, nkv)
    got = d_o.download(np.float16)
    assert_attn_close(got, oracle.cached_attention_f64(q, k, v, L, nq, nkv, hd),
                      what=f"{shape} L={L}")


@pytest.mark.parametrize("splits", [1, 2, 7, 33, 64])
def test_cached_attention_split_counts_agree(gpu, splits):
    L = 3001
    say(f"cached_attention_ex splits={splits} L={L}")
    q, k, v = _attention_case(L, L, NQ, NKV, HD, 401)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, splits)
    kv.launch_cached_attention_ex(d_q, d_k, d_v, d_o, L, L, HD, NQ, NKV, ws, num_splits=splits)
    got = d_o.download(np.float16)
    assert_attn_close(got, oracle.cached_attention_f64(q, k, v, L, NQ, NKV, HD),
                      what=f"splits={splits}")
    # counters are re-armed: a second launch gives identical bits
    kv.launch_cached_attention_ex(d_q, d_k, d_v, d_o, L, L, HD, NQ, NKV, ws, num_splits=splits)
    assert np.array_equal(bits(d_o.download(np.float16)), bits(got))


def test_cached_attention_rejects_too_many_splits(gpu):
    q, k, v = _attention_case(100, 100, NQ, NKV, HD, 404)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 0)  # sized for the largest split count
    with pytest.raises(Exception, match="invalid argument"):
        kv.launch_cached_attention_ex(d_q, d_k, d_v, d_o, 100, 100, HD, NQ, NKV, ws,
                                      num_splits=100000)


def test_cached_attention_device_length_equals_host_length(gpu):
    L, max_seq = 5000, 8192
    say("cached_attention_ex device seq_len")
    q, k, v = _attention_case(max_seq, max_seq, NQ, NKV, HD, 402)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_a, d_b = dev.DeviceBuffer(Q_DIM * 2), dev.DeviceBuffer(Q_DIM * 2)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 64)
    d_len = up(np.array([L], np.int32))
    kv.launch_cached_attention_ex(d_q, d_k, d_v, d_a, L, max_seq, HD, NQ, NKV, ws, num_splits=64)
    kv.launch_cached_attention_ex(d_q, d_k, d_v, d_b, 0, max_seq, HD, NQ, NKV, ws, num_splits=64,
                                  d_seq_len=d_len)
    a, b = d_a.download(np.float16), d_b.download(np.float16)
    assert np.array_equal(bits(a), bits(b))
    assert_attn_close(a, oracle.cached_attention_f64(q, k, v, L, NQ, NKV, HD), what="L=5000")


def test_cached_attention_ignores_rows_past_length(gpu):
    """Rows >= L hold NaN: they must not leak into the output."""
    L, max_seq = 700, 1024
    say("cached_attention NaN canaries past L")
    q, k, v = _attention_case(L, max_seq, NQ, NKV, HD, 403)
    k[L:] = np.float16(np.nan)
    v[L:] = np.float16(np.nan)
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_cached_attention(d_q, d_k, d_v, d_o, L, HD, NQ, NKV)
    assert_attn_close(d_o.download(np.float16),
                      oracle.cached_attention_f64(q, k, v, L, NQ, NKV, HD), what="canaries")


def test_config1_decode_step(gpu):
    """append at pos 512 then attention over 513 tokens."""
    say("config 1 decode step")
    max_seq, pos = 4096, 512
    c, s = oracle.rope_table(max_seq, HD, THETA)
    qkv, k, v = contiguous_case(max_seq, pos, SEED_BASE + 1)
    d_qkv, d_k, d_v = up(qkv), up(k), up(v)
    d_c, d_s = dev.DeviceBuffer(c.nbytes), dev.DeviceBuffer(s.nbytes)
    kv.build_rope_cache(d_c, d_s, max_seq, HD, THETA)
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, pos, max_seq, NQ, NKV, HD)
    kv.launch_cached_attention(d_qkv, d_k, d_v, d_o, pos + 1, HD, NQ, NKV)
    rq = oracle.rope_append(qkv, k, v, c, s, pos, NQ, NKV, HD)
    ref = oracle.cached_attention(rq[:Q_DIM], k, v, pos + 1, NQ, NKV, HD)
    assert np.array_equal(bits(d_qkv.download(np.float16)), bits(rq))
    assert np.array_equal(bits(d_k.download(np.float16)), bits(k).ravel())
    assert_attn_close(d_o.download(np.float16), ref, what="config 1")


def _decode_step(layers, bufs, d_c, d_s, max_seq, ws, splits, pos, d_state, stream):
    """One decode step over all layers: rope_append + attention per layer."""
    for l in range(layers):
        d_qkv, d_k, d_v, d_o = bufs[l]
        if d_state is None:
            kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, pos, max_seq, NQ, NKV, HD,
                                  stream=stream)
            kv.launch_cached_attention_ex(d_qkv, d_k, d_v, d_o, pos + 1, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, stream=stream)
        else:
            kv.launch_rope_append(d_qkv, d_k, d_v, d_c, d_s, -1, max_seq, NQ, NKV, HD,
                                  d_pos=d_state.ptr, stream=stream)
            kv.launch_cached_attention_ex(d_qkv, d_k, d_v, d_o, 0, max_seq, HD, NQ, NKV, ws,
                                          num_splits=splits, d_seq_len=d_state.ptr + 4,
                                          stream=stream)
    if d_state is not None:
        dev.add_i32(d_state.ptr, 2, 1, stream)


def test_graph_replay_equals_eager_steps(gpu):
    """hipGraph of a 4-layer decode step replayed N times == N eager steps, bit for bit."""
    layers, max_seq, pos0, steps, splits = 4, 2048, 1000, 5, 32
    say("graph replay vs eager")
    c, s = oracle.rope_table(max_seq, HD, THETA)
    d_c, d_s = up(c), up(s)
    host = [contiguous_case(max_seq, pos0, 500 + l) for l in range(layers)]

    def make():
        return [(up(q), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)) for (q, k, v) in host]

    eager, graphed = make(), make()
    stream = dev.Stream()
    ws_e = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    ws_g = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    d_state = up(np.array([pos0, pos0 + 1], np.int32))
    graph = dev.Graph.capture(stream, lambda: _decode_step(layers, graphed, d_c, d_s, max_seq,
                                                           ws_g, splits, 0, d_state, stream))
    for step in range(steps):
        _decode_step(layers, eager, d_c, d_s, max_seq, ws_e, splits, pos0 + step, None, stream)
        graph.launch(stream)
        stream.sync()
        for l in range(layers):
            for a, b in zip(eager[l], graphed[l]):
                assert np.array_equal(a.download(np.uint16), b.download(np.uint16)), (step, l)
    assert list(d_state.download(np.int32)) == [pos0 + steps, pos0 + steps + 1]
    graph.destroy()
    stream.destroy()


@pytest.mark.parametrize("pos", [0, 1, 17, 512, 8192])
@pytest.mark.parametrize("splits", [0, 1, 5, 64])
def test_fused_decode_equals_append_then_attention(gpu, pos, splits):
    """af_decode_attention_fused == af_rope_append + af_cached_attention_ex, bit for bit."""
    say(f"fused decode pos={pos} splits={splits}")
    max_seq = pos + 33
    c, s = oracle.rope_table(max_seq, HD, THETA)
    qkv, k, v = contiguous_case(max_seq, pos, 600 + pos)
    k[pos + 1:] = np.float16(np.nan)  # rows past the new token must never be read
    v[pos + 1:] = np.float16(np.nan)
    d_c, d_s = up(c), up(s)
    a_qkv, a_k, a_v, a_o = up(qkv), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)
    b_qkv, b_k, b_v, b_o = up(qkv), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 64)
    kv.launch_rope_append(a_qkv, a_k, a_v, d_c, d_s, pos, max_seq, NQ, NKV, HD)
    kv.launch_cached_attention_ex(a_qkv, a_k, a_v, a_o, pos + 1, max_seq, HD, NQ, NKV, ws,
                                  num_splits=splits)
    kv.launch_decode_attention_fused(b_qkv, b_k, b_v, d_c, d_s, pos, max_seq, b_o, NQ, NKV, HD,
                                     ws, num_splits=splits)
    for x, y in ((a_qkv, b_qkv), (a_k, b_k), (a_v, b_v), (a_o, b_o)):
        assert np.array_equal(x.download(np.uint16), y.download(np.uint16))
    rq = oracle.rope_append(qkv, k, v, c, s, pos, NQ, NKV, HD)
    assert_attn_close(b_o.download(np.float16),
                      oracle.cached_attention_f64(rq[:Q_DIM], k, v, pos + 1, NQ, NKV, HD),
                      what=f"fused pos={pos}")


def test_fused_graph_replay_advances_position(gpu):
    """A captured fused step with a device position, replayed N times == N eager two-call steps."""
    layers, max_seq, pos0, steps, splits = 3, 4096, 2000, 4, 48
    say("fused graph replay")
    c, s = oracle.rope_table(max_seq, HD, THETA)
    d_c, d_s = up(c), up(s)
    host = [contiguous_case(max_seq, pos0, 800 + l) for l in range(layers)]
    eager = [(up(q), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)) for (q, k, v) in host]
    fused = [(up(q), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)) for (q, k, v) in host]
    stream = dev.Stream()
    ws_e = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    ws_f = kv.AttentionWorkspace(1, NQ, NKV, HD, splits, stream)
    d_pos = up(np.array([pos0], np.int32))
    d_st = up(np.array([0], np.int32))

    def step():
        for (qkv, k, v, o) in fused:
            kv.launch_decode_attention_fused(qkv, k, v, d_c, d_s, -1, max_seq, o, NQ, NKV, HD,
                                             ws_f, num_splits=splits, d_pos=d_pos,
                                             d_status=d_st, stream=stream)
        dev.add_i32(d_pos.ptr, 1, 1, stream)

    graph = dev.Graph.capture(stream, step)
    for i in range(steps):
        for (qkv, k, v, o) in eager:
            kv.launch_rope_append(qkv, k, v, d_c, d_s, pos0 + i, max_seq, NQ, NKV, HD,
                                  stream=stream)
            kv.launch_cached_attention_ex(qkv, k, v, o, pos0 + i + 1, max_seq, HD, NQ, NKV, ws_e,
                                          num_splits=splits, stream=stream)
        graph.launch(stream)
        stream.sync()
        for l in range(layers):
            for a, b in zip(eager[l], fused[l]):
                assert np.array_equal(a.download(np.uint16), b.download(np.uint16)), (i, l)
    assert d_pos.download(np.int32)[0] == pos0 + steps and d_st.download(np.int32)[0] == 0
    graph.destroy()
    stream.destroy()


# Counter word a combiner that timed out sets (kFlagBase + kCombMaxGroups * kCombSplits).
POISON_BYTE = (8192 + 16 * 32) * 4


def test_poisoned_workspace_writes_nan_and_status(gpu):
    """A combiner that gives up poisons its workspace. The host sets that word here (no kernel
    is made to wait): every later dedicated-combiner launch on the workspace writes NaN and
    AF_ERR_TIMEOUT while the splits' append still lands, and af_attention_workspace_init
    brings back the same bits as before."""
    pos, max_seq = 4000, 4096
    splits = kv.default_splits(pos + 1, 1, NKV)
    assert 2 <= splits <= 32  # the dedicated-combiner form
    say(f"poisoned workspace pos={pos} splits={splits}")
    c, s = oracle.rope_table(max_seq, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv, k, v = contiguous_case(max_seq, pos, 901)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 0)

    def fused():
        d_qkv, d_k, d_v, d_o = up(qkv), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)
        d_st = up(np.array([0], np.int32))
        kv.launch_decode_attention_fused(d_qkv, d_k, d_v, d_c, d_s, pos, max_seq, d_o, NQ, NKV,
                                         HD, ws, d_status=d_st)
        dev.synchronize()
        return d_o.download(np.uint16), d_k.download(np.uint16), int(d_st.download(np.int32)[0])

    def attention():
        d_o = dev.DeviceBuffer(Q_DIM * 2)
        kv.launch_cached_attention_ex(up(qkv), up(k), up(v), d_o, pos, max_seq, HD, NQ, NKV, ws)
        dev.synchronize()
        return d_o.download(np.uint16)

    o0, k0, st0 = fused()
    a0 = attention()
    assert st0 == 0 and np.all(np.isfinite(o0.view(np.float16)))
    assert np.all(np.isfinite(a0.view(np.float16)))
    ws.buf.upload(np.array([1], np.uint32), offset=POISON_BYTE)
    for _ in range(2):  # it stays poisoned
        o1, k1, st1 = fused()
        assert st1 == AF_ERR_TIMEOUT
        assert np.all(np.isnan(o1.view(np.float16)))
        assert np.array_equal(k1, k0)  # the append is the splits' work
        assert np.all(np.isnan(attention().view(np.float16)))
    ws.reset()
    o2, k2, st2 = fused()
    assert st2 == 0 and np.array_equal(o2, o0) and np.array_equal(k2, k0)
    assert np.array_equal(attention(), a0)
