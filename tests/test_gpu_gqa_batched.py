"""GPU parity of the batched paged decode forms over every GQA ratio.

Batches with batch * KV heads * 2 >= CUs take the batched forms: fp16 pools the
compact grid (workgroups mapped onto the ~512-row splits each sequence needs),
FP8 pools the persistent grid (workgroups claiming row ranges from a counter;
KV heads in pairs when their count is even, single heads when it is odd). Each
(query heads, KV heads) shape below runs both: sampled sequences (empty,
one-row, block and span boundaries, long) against the CPU oracle
(paged_attention_f16 / paged_attention_fp8: the decode attention of
src/kernel/tiled_attention.cu:196-269 over a block table) at the dtype's bar,
and the fused step (RoPE + append + attention) against the paged append then
the unfused kernel, bit for bit, with one sequence whose position is out of
range (nothing is appended, rotated or attended for it).
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_KV_FP16, AF_KV_FP8_E4M3
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import ATOL_FP8, HD, RTOL_FP8, THETA, assert_attn_close, randn_f16, rng
from test_gpu_paged import _sequences

pytestmark = pytest.mark.gpu

EDGE = [0, 1, 31, 32, 33, 511, 512, 513]


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def _setup(nq, nkv, fp8, seed, hi=2500):
    """A batch just inside the batched regime, its BlockManager over a permuted free
    list and a random pool of `nkv` KV heads."""
    cus = dev.device_info()["compute_units"]
    B = max(16, -(-cus // (2 * nkv)))
    assert B * nkv * 2 >= cus and B <= 256
    r = rng(seed)
    lengths = [int(n) for n in r.integers(1, hi, B)]
    lengths[: len(EDGE)] = EDGE
    lengths[len(EDGE)] = hi + 700  # one long sequence: several splits / items
    bs, layers = (32 if fp8 else 16), 2
    total = sum((n + 1 + bs - 1) // bs for n in lengths) + 4
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total)]
    for blk in r.permutation(ids):
        bm.free_block(int(blk))
    seqs = _sequences(bm, lengths)
    shape = (layers, 2, total * bs, nkv * HD)
    if fp8:
        host = r.integers(0, 256, shape, dtype=np.uint8)
        host[(host & 0x7F) == 0x7F] = 0x00  # keep NaN codes out
        scales = r.uniform(0.004, 0.02, (layers, 2, nkv)).astype(np.float32)
        d_sc = up(scales)
    else:
        host = randn_f16(shape, seed + 1)
        scales, d_sc = None, None
    buf = up(host)
    desc = kv.make_pool(buf, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16, bs, layers, nkv, HD, total,
                        d_sc)
    return B, lengths, bm, seqs, bs, host, scales, buf, desc, d_sc


def _ref(q, host, scales, layer, table, n, bs, nq, nkv):
    if scales is None:
        return oracle.paged_attention_f16(q, host[layer, 0], host[layer, 1], table, n, bs, nq, nkv,
                                          HD)
    return oracle.paged_attention_fp8(q, host[layer, 0], host[layer, 1], scales[layer, 0],
                                      scales[layer, 1], table, n, bs, nq, nkv, HD)


SHAPES = [(8, 1), (9, 3), (16, 8), (64, 8)]


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("nq,nkv", SHAPES)
def test_batched_gqa_vs_oracle(gpu, nq, nkv, fp8):
    B, lengths, bm, seqs, bs, host, scales, buf, desc, d_sc = _setup(nq, nkv, fp8,
                                                                     1100 + nq + nkv + 7 * fp8)
    q_dim = nq * HD
    say(f"batched gqa nq={nq} nkv={nkv} fp8={fp8} B={B} rows={sum(lengths)}")
    max_len = max(lengths)
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, q_dim), 1110 + nq)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * q_dim * 2)
    d_o.upload(np.full((B, q_dim), 7.0, np.float16))  # empty sequences must come back zero
    ws = kv.AttentionWorkspace(B, nq, nkv, HD, 0)
    sample = list(range(len(EDGE) + 1)) + list(
        rng(1120 + nq).choice(np.arange(len(EDGE) + 1, B), 6, replace=False))
    atol, rtol = (ATOL_FP8, RTOL_FP8) if fp8 else (2e-3, 1e-2)
    for layer in range(2):
        kv.launch_paged_attention(d_q, q_dim, desc, layer, d_t, max_blocks, d_l, B, max_len, d_o,
                                  q_dim, nq, ws)
        got = d_o.download(np.float16, (B, q_dim))
        for b in sample:
            if lengths[b] == 0:
                assert not np.any(bits(got[b])), f"seq {b}: empty sequence not zero"
                continue
            ref = _ref(q[b], host, scales, layer, tables[b], lengths[b], bs, nq, nkv)
            assert_attn_close(got[b], ref, atol, rtol, what=f"layer {layer} seq {b} L={lengths[b]}")
    bm.close()


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("nq,nkv", SHAPES)
def test_batched_gqa_fused_equals_unfused(gpu, nq, nkv, fp8):
    B, _, bm, seqs, bs, host, scales, buf, desc, d_sc = _setup(nq, nkv, fp8,
                                                               1200 + nq + nkv + 7 * fp8)
    q_dim, kv_dim = nq * HD, nkv * HD
    qkv_w = q_dim + 2 * kv_dim
    say(f"batched gqa fused nq={nq} nkv={nkv} fp8={fp8} B={B}")
    plan = bm.plan_decode(seqs)
    assert not isinstance(plan, int), plan
    slots, positions, copies = plan
    assert len(copies) == 0
    lengths = [int(p) for p in positions]
    max_pos = max(lengths) + 2
    bad = len(EDGE) + 2
    positions = positions.copy()
    positions[bad] = max_pos  # out of range: nothing written for this sequence
    max_len = max(lengths) + 1
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((B, qkv_w), 1210 + nq)
    d_t, d_sl, d_p = up(tables), up(slots), up(positions)
    ws = kv.AttentionWorkspace(B, nq, nkv, HD, 0)
    init = host.copy()
    # fused
    q1 = up(qkv)
    o1 = dev.DeviceBuffer(B * q_dim * 2)
    o1.upload(np.full((B, q_dim), 7.0, np.float16))
    kv.launch_paged_decode_fused(q1, B, desc, 1, d_sl, d_p, d_c, d_s, max_pos, d_t, max_blocks,
                                 max_len, o1, q_dim, nq, ws)
    dev.synchronize()
    fused_pool = buf.download(init.dtype, init.shape).copy()
    fused_q = q1.download(np.uint16, (B, qkv_w)).copy()
    fused_o = o1.download(np.uint16, (B, q_dim)).copy()
    # unfused on a fresh copy: append the in-range tokens, then attention
    buf.upload(init)
    idx = np.array([b for b in range(B) if b != bad])
    sub = dev.DeviceBuffer(len(idx) * qkv_w * 2)
    sub.upload(qkv[idx])
    kv.launch_paged_rope_append(sub, len(idx), desc, 1, up(slots[idx]), up(positions[idx]), d_c,
                                d_s, max_pos, nq)
    full = qkv.copy()
    full[idx] = sub.download(np.float16, (len(idx), qkv_w))
    o2 = dev.DeviceBuffer(B * q_dim * 2)
    o2.upload(np.full((B, q_dim), 7.0, np.float16))
    lens2 = lens.copy()
    lens2[bad] = 0
    kv.launch_paged_attention(up(full), qkv_w, desc, 1, d_t, max_blocks, up(lens2), B, max_len,
                              o2, q_dim, nq, ws)
    dev.synchronize()
    unfused_pool = buf.download(init.dtype, init.shape)
    unfused_o = o2.download(np.uint16, (B, q_dim))
    # pool: bit-identical appends, nothing for the out-of-range sequence
    assert np.array_equal(fused_pool.view(np.uint8), unfused_pool.view(np.uint8))
    # queries and keys rotated in place for the in-range sequences only
    assert np.array_equal(fused_q[idx], bits(full[idx]))
    assert np.array_equal(fused_q[bad], bits(qkv[bad])), "out-of-range row was rotated"
    # attention: bit-identical for every in-range sequence; nothing written for the other
    assert np.array_equal(fused_o[idx], unfused_o[idx])
    assert np.all(fused_o[bad] == np.float16(7.0).view(np.uint16)), "out-of-range output written"
    # and one in-range sequence against the oracle on the appended pool
    b = len(EDGE) + 1
    ref = _ref(full[b, :q_dim], unfused_pool, scales, 1, tables[b], lengths[b] + 1, bs, nq, nkv)
    atol, rtol = (ATOL_FP8, RTOL_FP8) if fp8 else (2e-3, 1e-2)
    assert_attn_close(fused_o[b].view(np.float16), ref, atol, rtol, what=f"fused seq {b}")
    bm.close()


@pytest.mark.parametrize("fp8", [False, True])
def test_shared_blocks_policy_gives_the_same_bits(gpu, fp8):
    """AF_KV_POOL_SHARED_BLOCKS selects the kernels that read KV rows with the ordinary cache
    policy instead of non-temporal loads; only the load policy differs, so a batch whose odd
    sequences map the same blocks as their even neighbours (forks) gets the same bits either
    way, unfused and fused, and matches the oracle."""
    from atomflow_amd import AF_KV_POOL_SHARED_BLOCKS
    nq, nkv = 24, 8
    B, lengths, bm, seqs, bs, host, scales, buf, desc, d_sc = _setup(nq, nkv, fp8, 1300 + 7 * fp8)
    shared = kv.make_pool(buf, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16, bs, 2, nkv, HD,
                          desc.total_blocks, d_sc, flags=AF_KV_POOL_SHARED_BLOCKS)
    say(f"shared-blocks policy fp8={fp8} B={B}")
    q_dim = nq * HD
    max_len = max(lengths)
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    tables[1::2], lens[1::2] = tables[0::2][: B // 2], lens[0::2][: B // 2]  # forks
    lengths = [int(n) for n in lens]
    q = randn_f16((B, q_dim), 1310)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    ws = kv.AttentionWorkspace(B, nq, nkv, HD, 0)
    outs = []
    for pool in (desc, shared):
        d_o = dev.DeviceBuffer(B * q_dim * 2)
        kv.launch_paged_attention(d_q, q_dim, pool, 1, d_t, max_blocks, d_l, B, max_len, d_o,
                                  q_dim, nq, ws)
        outs.append(d_o.download(np.float16, (B, q_dim)))
    assert np.array_equal(bits(outs[0]), bits(outs[1]))
    atol, rtol = (ATOL_FP8, RTOL_FP8) if fp8 else (2e-3, 1e-2)
    for b in (1, 9, 10, B - 1):
        if lengths[b]:
            ref = _ref(q[b], host, scales, 1, tables[b], lengths[b], bs, nq, nkv)
            assert_attn_close(outs[1][b], ref, atol, rtol, what=f"seq {b} L={lengths[b]}")
    # fused step (RoPE + append + attention) on the unshared sequences, both policies
    plan = bm.plan_decode(seqs)
    assert not isinstance(plan, int), plan
    slots, positions, _ = plan
    max_pos = int(positions.max()) + 2
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    ftables, flens = bm.export_tables(seqs, (int(positions.max()) + 1 + bs - 1) // bs)
    qkv = randn_f16((B, q_dim + 2 * nkv * HD), 1320)
    res = []
    for pool in (desc, shared):
        buf.upload(host)
        d_qkv, d_o = up(qkv), dev.DeviceBuffer(B * q_dim * 2)
        kv.launch_paged_decode_fused(d_qkv, B, pool, 0, up(slots), up(positions), d_c, d_s,
                                     max_pos, up(ftables), ftables.shape[1],
                                     int(positions.max()) + 1, d_o, q_dim, nq, ws)
        res.append((d_o.download(np.uint16), buf.download(np.uint8)))
    assert np.array_equal(res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1])
    bm.close()
