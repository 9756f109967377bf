"""GPU parity of the persistent form of batched paged decode attention.

Batches of FP8 pools with the default split count (batch * KV heads * 2 >= CUs)
run as one persistent grid whose workgroups claim items (big row ranges, then
small ones) from a device counter. Checked here against the CPU oracle
(paged_attention_fp8, src/kernel/tiled_attention.cu:196-269 over a block table)
at the FP8 bar (5e-2) and the fp16 bar, on ragged batches with empty, one-row
and block-boundary sequences; fused decode (RoPE + append + attention) equals
the unfused kernel on the appended pool bit for bit; graph replays (the claim
counters re-armed by each launch) equal the eager launch bit for bit.
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_KV_FP8_E4M3
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import (ATOL_FP8, HD, KV_DIM, NKV, NQ, Q_DIM, QKV, RTOL_FP8, THETA,
                    assert_attn_close, randn_f16, rng)
from test_gpu_paged import Pool, _sequences

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def _batch(lengths, seed, layers=2, bs=32):
    """BlockManager over a permuted free list, FP8 pool, block tables of `lengths`."""
    total = sum((n + 1 + bs - 1) // bs for n in lengths) + 4
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP8_E4M3)
    ids = [bm.allocate_block() for _ in range(total)]
    for b in rng(seed).permutation(ids):
        bm.free_block(int(b))
    seqs = _sequences(bm, lengths)
    P = Pool(layers, total, bs, True, seed + 1)
    return bm, seqs, P


def _lengths(seed, B):
    r = rng(seed)
    lengths = list(r.integers(1, 6000, B))
    lengths[:6] = [0, 1, 31, 32, 33, 64]  # empty, single-row and block-boundary sequences
    return [int(n) for n in lengths]


@pytest.mark.parametrize("B", [24, 64])
def test_persistent_fp8_vs_oracle(gpu, B):
    lengths = _lengths(900 + B, B)
    say(f"persistent fp8 B={B} rows={sum(lengths)}")
    assert B * NKV * 2 >= dev.device_info()["compute_units"]  # the batched (persistent) regime
    bm, seqs, P = _batch(lengths, 910 + B)
    bs = P.bs
    max_len = max(lengths)
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, Q_DIM), 920 + B)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * Q_DIM * 2)
    d_o.upload(np.full((B, Q_DIM), 7.0, np.float16))  # empty sequences must come back zero
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    sample = list(range(6)) + list(rng(930 + B).choice(np.arange(6, B), 6, replace=False))
    for layer in range(P.layers):
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B, max_len,
                                  d_o, Q_DIM, NQ, ws)
        got = d_o.download(np.float16, (B, Q_DIM))
        for b in sample:
            if lengths[b] == 0:
                assert not np.any(bits(got[b])), f"seq {b}: empty sequence not zero"
                continue
            ref = oracle.paged_attention_fp8(q[b], P.slab(layer, 0), P.slab(layer, 1),
                                             P.scales[layer, 0], P.scales[layer, 1], tables[b],
                                             lengths[b], bs, NQ, NKV, HD)
            assert_attn_close(got[b], ref, ATOL_FP8, RTOL_FP8, what=f"layer {layer} seq {b}")
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} (fp16 bar)")
    bm.close()


def test_persistent_fused_equals_unfused_and_appends(gpu):
    """Fused decode (RoPE + append + attention) == append, then the unfused kernel."""
    B = 96  # several items per workgroup, so item set-up overlaps the previous tail
    lengths = _lengths(940, B)
    lengths[0] = 5  # fused decode appends to every sequence
    say(f"persistent fused vs unfused B={B}")
    bm, seqs, P = _batch(lengths, 941)
    bs = P.bs
    plan = bm.plan_decode(seqs)
    assert not isinstance(plan, int), plan
    slots, positions, copies = plan
    assert len(copies) == 0
    max_len = max(lengths) + 1
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    max_pos = max_len + 1
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((B, QKV), 942)
    d_qkv, d_t, d_l = up(qkv), up(tables), up(lens)
    d_sl, d_p = up(slots), up(positions)
    d_o1, d_o2 = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    layer = 1
    kv.launch_paged_decode_fused(d_qkv, B, P.desc, layer, d_sl, d_p, d_c, d_s, max_pos, d_t,
                                 max_blocks, max_len, d_o1, Q_DIM, NQ, ws)
    kv.launch_paged_attention(d_qkv, QKV, P.desc, layer, d_t, max_blocks, d_l, B, max_len, d_o2,
                              Q_DIM, NQ, ws)
    dev.synchronize()
    assert np.array_equal(bits(d_o1.download(np.float16)), bits(d_o2.download(np.float16)))
    # the appended rows and the rotated queries match the oracle's append, byte for byte
    host = P.host.copy()
    rq = np.empty_like(qkv)
    for b in range(B):
        pos = int(positions[b])
        rq[b] = oracle.rope_append(qkv[b], np.zeros((1, KV_DIM), np.float16),
                                   np.zeros((1, KV_DIM), np.float16), c[pos:], s[pos:], 0, NQ,
                                   NKV, HD)
        oracle.paged_write_fp8(rq[b, Q_DIM:Q_DIM + KV_DIM], rq[b, Q_DIM + KV_DIM:],
                               host[layer, 0], host[layer, 1], int(slots[b]), KV_DIM, HD,
                               P.scales[layer, 0], P.scales[layer, 1])
    assert np.array_equal(P.download().view(np.uint8), host.view(np.uint8))
    assert np.array_equal(bits(d_qkv.download(np.float16, (B, QKV))), bits(rq))
    bm.close()


def test_persistent_graph_replays(gpu):
    """Replays of a captured persistent launch equal the eager launch (counters re-armed)."""
    B = 32
    lengths = _lengths(950, B)
    say(f"persistent graph replays B={B}")
    bm, seqs, P = _batch(lengths, 951)
    bs = P.bs
    max_len = max(lengths)
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    d_q, d_t, d_l = up(randn_f16((B, Q_DIM), 952)), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    stream = dev.Stream()

    def launch():
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, 0, d_t, max_blocks, d_l, B, max_len, d_o,
                                  Q_DIM, NQ, ws, stream=stream)

    launch()
    stream.sync()
    ref = d_o.download(np.float16).copy()
    g = dev.Graph.capture(stream, launch)
    try:
        for i in range(4):
            d_o.upload(np.zeros(B * Q_DIM, np.float16))
            g.launch(stream)
            stream.sync()
            assert np.array_equal(bits(d_o.download(np.float16)), bits(ref)), f"replay {i}"
            launch()  # eager work between replays
            stream.sync()
            assert np.array_equal(bits(d_o.download(np.float16)), bits(ref)), f"eager after {i}"
    finally:
        g.destroy()
    bm.close()
