"""GPU parity of batched fp16 paged decode attention in the grid form.

Batches with batch * KV heads * 2 >= CUs and the default split count split
every sequence into ~512-row ranges; the grid is sized for the longest one and
its workgroups map onto the splits that exist (shorter sequences need fewer).
Checked here against the CPU oracle (paged_attention_f16: the decode attention
of src/kernel/tiled_attention.cu:196-269 over a block table) at the fp16 bar on
ragged batches: empty, one-row and block-boundary sequences and long ones; an
empty sequence's output is zero; the fused step (RoPE + append + attention)
equals the unfused pair bit for bit, including a sequence whose position is
out of range (nothing written for it).
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_KV_FP16
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import HD, NKV, NQ, Q_DIM, QKV, THETA, assert_attn_close, randn_f16, rng
from test_gpu_paged import Pool, _sequences

pytestmark = pytest.mark.gpu

EDGE = [0, 1, 15, 16, 17, 511, 512, 513, 1024, 1025]  # empty, one row, block / span boundaries


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def _lengths(seed, B, hi):
    r = rng(seed)
    lengths = [int(n) for n in r.integers(1, hi, B)]
    lengths[: len(EDGE)] = EDGE
    return lengths


def _batch(lengths, seed, layers=2, bs=16, extra=1):
    total = sum((n + extra + bs - 1) // bs for n in lengths) + 4
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total)]
    for blk in rng(seed).permutation(ids):  # permuted free list: scattered tables
        bm.free_block(int(blk))
    seqs = _sequences(bm, lengths)
    return bm, seqs, Pool(layers, total, bs, False, seed + 1)


@pytest.mark.parametrize("B,hi", [(32, 6000), (48, 2500)])
def test_batched_fp16_vs_oracle(gpu, B, hi):
    lengths = _lengths(960 + B, B, hi)
    assert B * NKV * 2 >= dev.device_info()["compute_units"]  # the batched regime
    splits = kv.default_splits(max(lengths), B, NKV)
    say(f"batched fp16 grid form B={B} rows={sum(lengths)} splits {splits}")
    bm, seqs, P = _batch(lengths, 970 + B)
    bs = P.bs
    max_len = max(lengths)
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, Q_DIM), 980 + B)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * Q_DIM * 2)
    d_o.upload(np.full((B, Q_DIM), 7.0, np.float16))  # empty sequences must come back zero
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    sample = list(range(len(EDGE))) + list(rng(990 + B).choice(np.arange(len(EDGE), B), 8,
                                                                replace=False))
    for layer in range(P.layers):
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B, max_len,
                                  d_o, Q_DIM, NQ, ws)
        got = d_o.download(np.float16, (B, Q_DIM))
        for b in sample:
            if lengths[b] == 0:
                assert not np.any(bits(got[b])), f"seq {b}: empty sequence not zero"
                continue
            ref = oracle.paged_attention_f16(q[b], P.slab(layer, 0), P.slab(layer, 1), tables[b],
                                             lengths[b], bs, NQ, NKV, HD)
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} L={lengths[b]}")
    bm.close()


def test_batched_fp16_fused_equals_unfused(gpu):
    """Fused step == paged append, then the unfused kernel, bit for bit; one
    sequence's position is out of range (nothing is appended or attended for it)."""
    B = 40
    lengths = _lengths(1000, B, 4000)
    lengths[0] = 3  # the fused step appends to every sequence
    say(f"batched fp16 fused vs unfused B={B}")
    bm, seqs, P = _batch(lengths, 1001)
    bs = P.bs
    plan = bm.plan_decode(seqs)
    assert not isinstance(plan, int), plan
    slots, positions, copies = plan
    assert len(copies) == 0
    max_pos = max(lengths) + 2
    bad = 7
    positions = positions.copy()
    positions[bad] = max_pos  # out of range: nothing written, status set
    max_len = max(lengths) + 1
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((B, QKV), 1002)
    d_t = up(tables)
    d_sl, d_p = up(slots), up(positions)
    init = P.download().copy()
    # fused on one copy of the pool and qkv
    q1 = up(qkv)
    o1 = dev.DeviceBuffer(B * Q_DIM * 2)
    o1.upload(np.full((B, Q_DIM), 7.0, np.float16))
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    kv.launch_paged_decode_fused(q1, B, P.desc, 1, d_sl, d_p, d_c, d_s, max_pos, d_t, max_blocks,
                                 max_len, o1, Q_DIM, NQ, ws)
    dev.synchronize()
    fused_pool = P.download().copy()
    fused_q = q1.download(np.uint16, (B, QKV)).copy()
    fused_o = o1.download(np.uint16, (B, Q_DIM)).copy()
    # unfused on a fresh copy: append the in-range tokens, then attention
    P.buf.upload(init)
    ok = np.array([b != bad for b in range(B)])
    idx = np.nonzero(ok)[0]
    q2 = up(qkv)
    sub = dev.DeviceBuffer(int(ok.sum()) * QKV * 2)
    sub.upload(qkv[idx])
    kv.launch_paged_rope_append(sub, int(ok.sum()), P.desc, 1, up(slots[idx]), up(positions[idx]),
                                d_c, d_s, max_pos, NQ)
    rot = sub.download(np.float16, (int(ok.sum()), QKV))
    full = qkv.copy()
    full[idx] = rot
    q2.upload(full)
    lens2 = lens.copy()
    o2 = dev.DeviceBuffer(B * Q_DIM * 2)
    o2.upload(np.full((B, Q_DIM), 7.0, np.float16))
    kv.launch_paged_attention(q2, QKV, P.desc, 1, d_t, max_blocks, up(lens2), B, max_len, o2,
                              Q_DIM, NQ, ws)
    dev.synchronize()
    got_o = o2.download(np.uint16, (B, Q_DIM))
    assert np.array_equal(P.download().view(np.uint8), fused_pool.view(np.uint8))
    assert np.array_equal(fused_q[ok], q2.download(np.uint16, (B, QKV))[ok])
    assert np.array_equal(fused_q[bad], bits(qkv[bad]))  # untouched
    assert np.array_equal(fused_o[ok], got_o[ok])
    assert np.all(fused_o[bad] == np.float16(7.0).view(np.uint16))  # nothing written
    bm.close()
