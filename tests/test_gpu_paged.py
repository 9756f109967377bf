"""GPU parity of the paged KV path (libatomflow_kv.so vs the CPU oracle).

Bit-exact: block-table gather, paged RoPE+append (fp16 copy and FP8
quantisation) into BlockManager slots, copy-on-write block copies (whole pool
compared). Attention: fp16 within 2e-3 / 1e-2 and FP8 within 5e-2 / 1e-2 of the
oracle run on the same bytes; the paged kernel also equals the contiguous
kernel on the gathered rows bit for bit.
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_KV_FP8_E4M3, AF_KV_FP16
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import (ATOL_FP8, HD, KV_DIM, NKV, NQ, Q_DIM, QKV, RTOL_FP8, THETA,
                    assert_attn_close, randn_f16, rng)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def u16(a):
    return np.ascontiguousarray(a).view(np.uint16)


class Pool:
    """Host mirror + device copy of a paged pool [layers][K,V][blocks*bs][kv_dim]."""

    def __init__(self, layers, blocks, bs, fp8, seed):
        self.layers, self.blocks, self.bs, self.fp8 = layers, blocks, bs, fp8
        shape = (layers, 2, blocks * bs, KV_DIM)
        r = rng(seed)
        if fp8:
            h = r.integers(0, 256, shape, dtype=np.uint8)
            h[(h & 0x7F) == 0x7F] = 0x00  # keep NaN codes out
            self.scales = r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32)
            self.d_scales = up(self.scales)
        else:
            h = randn_f16(shape, seed)
            self.scales, self.d_scales = None, None
        self.host = h
        self.buf = up(h)
        self.desc = kv.make_pool(self.buf, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16, bs, layers, NKV,
                                 HD, blocks, self.d_scales)

    def download(self):
        return self.buf.download(self.host.dtype, self.host.shape)

    def slab(self, layer, which, arr=None):
        a = self.host if arr is None else arr
        return a[layer, which]


def _sequences(bm, lengths):
    seqs = []
    for n in lengths:
        s = bm.seq_create()
        r = bm.seq_extend(s, int(n))
        assert not isinstance(r, int), r
        seqs.append(s)
    return seqs


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_gather_bit_exact(gpu, fp8):
    say(f"paged_gather fp8={fp8}")
    bs, blocks = 16, 300
    P = Pool(2, blocks, bs, fp8, 700)
    table = rng(701).permutation(blocks).astype(np.int32)
    L = 2000
    d_table = up(table)
    esz = 1 if fp8 else 2
    k_dst, v_dst = dev.DeviceBuffer(L * KV_DIM * esz), dev.DeviceBuffer(L * KV_DIM * esz)
    for layer in range(2):
        kv.paged_gather(P.desc, layer, d_table, L, k_dst, v_dst)
        dt = P.host.dtype
        for which, dst in ((0, k_dst), (1, v_dst)):
            ref = oracle.paged_gather(P.slab(layer, which), table, L, bs, KV_DIM)
            assert np.array_equal(dst.download(dt, (L, KV_DIM)).view(np.uint8),
                                  ref.view(np.uint8)), (layer, which)


@pytest.mark.parametrize("bs", [16, 32])
def test_paged_attention_fp16_vs_oracle(gpu, bs):
    say(f"paged_attention fp16 bs={bs}")
    B, layers = 12, 2
    lengths = [1, 2, 15, 16, 17, 100, 129, 700, 1024, 1500, 2049, 3001]
    total = sum((n + bs - 1) // bs for n in lengths) + 5
    bm = kv.BlockManager(total, bs, layers)
    # scramble the free list so tables are non-contiguous
    ids = [bm.allocate_block() for _ in range(total)]
    for b in rng(702).permutation(ids):
        bm.free_block(int(b))
    seqs = _sequences(bm, lengths)
    P = Pool(layers, total, bs, False, 703)
    bm.attach_pool(P.buf.ptr)
    max_blocks = max((n + bs - 1) // bs for n in lengths)
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, Q_DIM), 704)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * Q_DIM * 2)
    max_len = max(lengths)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    for layer in range(layers):
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B, max_len,
                                  d_o, Q_DIM, NQ, ws)
        got = d_o.download(np.float16, (B, Q_DIM))
        for b in range(B):
            ref = oracle.paged_attention_f16(q[b], P.slab(layer, 0), P.slab(layer, 1), tables[b],
                                             lengths[b], bs, NQ, NKV, HD)
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} L={lengths[b]}")


def test_paged_equals_contiguous_kernel_bitwise(gpu):
    say("paged vs contiguous kernel on gathered rows")
    bs, blocks, L, splits = 16, 400, 5000, 40
    P = Pool(1, blocks, bs, False, 710)
    table = rng(711).permutation(blocks).astype(np.int32)
    q = randn_f16(Q_DIM, 712)
    d_q, d_table, d_len = up(q), up(table[None, :]), up(np.array([L], np.int32))
    k_dst, v_dst = dev.DeviceBuffer(L * KV_DIM * 2), dev.DeviceBuffer(L * KV_DIM * 2)
    kv.paged_gather(P.desc, 0, d_table, L, k_dst, v_dst)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, splits)
    a, b = dev.DeviceBuffer(Q_DIM * 2), dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_paged_attention(d_q, Q_DIM, P.desc, 0, d_table, blocks, d_len, 1, L, a, Q_DIM, NQ,
                              ws, num_splits=splits)
    kv.launch_cached_attention_ex(d_q, k_dst, v_dst, b, L, L, HD, NQ, NKV, ws, num_splits=splits)
    assert np.array_equal(u16(a.download(np.float16)), u16(b.download(np.float16)))


def test_paged_attention_fp8_vs_oracle(gpu):
    say("paged_attention fp8 bs=32")
    bs, layers = 32, 2
    lengths = [1, 31, 32, 33, 500, 2000, 4097, 777]
    B = len(lengths)
    total = sum((n + bs - 1) // bs for n in lengths) + 3
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP8_E4M3)
    ids = [bm.allocate_block() for _ in range(total)]
    for b in rng(720).permutation(ids):
        bm.free_block(int(b))
    seqs = _sequences(bm, lengths)
    P = Pool(layers, total, bs, True, 721)
    max_blocks = max((n + bs - 1) // bs for n in lengths)
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, Q_DIM), 722)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    for layer in range(layers):
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B,
                                  max(lengths), d_o, Q_DIM, NQ, ws)
        got = d_o.download(np.float16, (B, Q_DIM))
        for b in range(B):
            ref = oracle.paged_attention_fp8(q[b], P.slab(layer, 0), P.slab(layer, 1),
                                             P.scales[layer, 0], P.scales[layer, 1], tables[b],
                                             lengths[b], bs, NQ, NKV, HD)
            assert_attn_close(got[b], ref, ATOL_FP8, RTOL_FP8, what=f"fp8 layer {layer} seq {b}")
            assert_attn_close(got[b], ref, what=f"fp8 layer {layer} seq {b} (fp16 bar)")


def test_fp8_decode_exhaustive_through_attention(gpu):
    """L = 1: out = dequant(V row) * v_scale exactly, over every finite E4M3 code."""
    say("fp8 decode of all codes")
    bs = 32
    P = Pool(1, 2, bs, True, 730)
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    row = np.resize(codes, KV_DIM)
    host = P.host.copy()
    host[0, 1, 0] = row  # V row 0 of block 0
    P.host = host
    P.buf.upload(host)
    scales = np.ones((1, 2, NKV), np.float32)
    P.d_scales.upload(scales)
    q = randn_f16(Q_DIM, 731)
    d_q, d_t, d_l = up(q), up(np.array([[0]], np.int32)), up(np.array([1], np.int32))
    d_o = dev.DeviceBuffer(Q_DIM * 2)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 0)
    kv.launch_paged_attention(d_q, Q_DIM, P.desc, 0, d_t, 1, d_l, 1, 1, d_o, Q_DIM, NQ, ws)
    got = d_o.download(np.float16)
    lut = oracle.e4m3_decode_table()
    exp = np.concatenate([lut[row[(h // 3) * HD:(h // 3 + 1) * HD]] for h in range(NQ)])
    assert np.array_equal(got.astype(np.float32), exp.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_rope_append_bit_exact(gpu, fp8):
    say(f"paged_rope_append fp8={fp8}")
    bs, layers, B = 16, 2, 9
    lengths = [0, 1, 15, 16, 17, 31, 32, 300, 1000]
    total = sum(n // bs + 1 for n in lengths) + 4
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16)
    seqs = _sequences(bm, lengths)
    slots, positions, copies = bm.plan_decode(seqs)
    assert len(copies) == 0 and list(positions) == lengths
    P = Pool(layers, total, bs, fp8, 740)
    max_pos = 2048
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((layers, B, QKV), 741)
    d_qkv = up(qkv)
    d_slots, d_pos = up(slots), up(positions)
    ref_pool = P.host.copy()
    for layer in range(layers):
        kv.launch_paged_rope_append(d_qkv.ptr + layer * B * QKV * 2, B, P.desc, layer, d_slots,
                                    d_pos, d_c, d_s, max_pos, NQ)
        for b in range(B):
            rq = oracle.rope_append(qkv[layer, b], np.zeros((1, KV_DIM), np.float16),
                                    np.zeros((1, KV_DIM), np.float16), c[positions[b]:],
                                    s[positions[b]:], 0, NQ, NKV, HD)
            krow, vrow = rq[Q_DIM:Q_DIM + KV_DIM], rq[Q_DIM + KV_DIM:]
            qkv[layer, b] = rq
            if fp8:
                oracle.paged_write_fp8(krow, vrow, ref_pool[layer, 0], ref_pool[layer, 1],
                                       int(slots[b]), KV_DIM, HD, P.scales[layer, 0],
                                       P.scales[layer, 1])
            else:
                oracle.paged_write_f16(krow, vrow, ref_pool[layer, 0], ref_pool[layer, 1],
                                       int(slots[b]), KV_DIM)
    assert np.array_equal(u16(d_qkv.download(np.float16, qkv.shape)), u16(qkv))
    assert np.array_equal(P.download().view(np.uint8), ref_pool.view(np.uint8))


def test_cow_copy_blocks_bit_exact(gpu):
    """64 sequences share a prefix ending mid-block (BASELINE configs[3] pattern)."""
    say("copy-on-write block copies")
    bs, layers = 16, 3
    bm = kv.BlockManager(400, bs, layers)
    root = bm.seq_create()
    bm.seq_extend(root, 2048 + 8)
    seqs = [root] + [bm.seq_fork(root) for _ in range(63)]
    slots, positions, copies = bm.plan_decode(seqs, max_copies=64)
    assert len(copies) == 63
    P = Pool(layers, 400, bs, False, 750)
    ref = P.host.copy()
    for (src, dst, rows) in copies:
        for layer in range(layers):
            for which in range(2):
                ref[layer, which, dst * bs:dst * bs + rows] = ref[layer, which,
                                                                  src * bs:src * bs + rows]
    d_copies = up(np.ascontiguousarray(copies, np.int32))
    d_count = up(np.array([len(copies)], np.int32))
    kv.kv_copy_blocks(P.desc, d_copies, d_count, 64)
    assert np.array_equal(u16(P.download()), u16(ref))


def test_cow_decode_step_end_to_end(gpu):
    """Forked sequences: plan (CoW) -> copy blocks -> paged append -> attention, 2 layers,
    checked against the oracle on each sequence's logical rows."""
    say("CoW decode step end to end")
    bs, layers, prefix = 16, 2, 200 + 5
    bm = kv.BlockManager(200, bs, layers)
    root = bm.seq_create()
    bm.seq_extend(root, prefix)
    seqs = [root] + [bm.seq_fork(root) for _ in range(7)]
    for i, s in enumerate(seqs[1:]):  # independent suffixes
        r = bm.seq_extend(s, 3 * i + 1)
        assert not isinstance(r, int)
    P = Pool(layers, 200, bs, False, 760)
    slots, positions, copies = bm.plan_decode(seqs, max_copies=16)
    B = len(seqs)
    max_pos = 1024
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((layers, B, QKV), 761)
    d_qkv = up(qkv)
    d_copies = up(np.ascontiguousarray(copies, np.int32).reshape(-1, 3) if len(copies) else
                  np.zeros((1, 3), np.int32))
    d_count = up(np.array([len(copies)], np.int32))
    max_blocks = 32
    tables, lens = bm.export_tables(seqs, max_blocks)
    d_t, d_l, d_slots, d_pos = up(tables), up(lens), up(slots), up(positions)
    d_o = dev.DeviceBuffer(layers * B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    kv.kv_copy_blocks(P.desc, d_copies, d_count, 16)
    for layer in range(layers):
        q_ptr = d_qkv.ptr + layer * B * QKV * 2
        kv.launch_paged_rope_append(q_ptr, B, P.desc, layer, d_slots, d_pos, d_c, d_s, max_pos, NQ)
        kv.launch_paged_attention(q_ptr, QKV, P.desc, layer, d_t, max_blocks, d_l, B, int(lens.max()),
                                  d_o.ptr + layer * B * Q_DIM * 2, Q_DIM, NQ, ws)
    got = d_o.download(np.float16, (layers, B, Q_DIM))
    # oracle: apply the copies, then per sequence append + attention on its logical rows
    ref = P.host.copy()
    for (src, dst, rows) in copies:
        ref[:, :, dst * bs:dst * bs + rows] = ref[:, :, src * bs:src * bs + rows]
    for layer in range(layers):
        for b in range(B):
            rq = oracle.rope_append(qkv[layer, b], np.zeros((1, KV_DIM), np.float16),
                                    np.zeros((1, KV_DIM), np.float16), c[positions[b]:],
                                    s[positions[b]:], 0, NQ, NKV, HD)
            oracle.paged_write_f16(rq[Q_DIM:Q_DIM + KV_DIM], rq[Q_DIM + KV_DIM:], ref[layer, 0],
                                   ref[layer, 1], int(slots[b]), KV_DIM)
            out = oracle.paged_attention_f16(rq[:Q_DIM], ref[layer, 0], ref[layer, 1], tables[b],
                                             int(lens[b]), bs, NQ, NKV, HD)
            assert_attn_close(got[layer, b], out, what=f"layer {layer} seq {b}")
    assert np.array_equal(u16(P.download()), u16(ref))


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_fused_equals_append_then_attention(gpu, fp8):
    """af_paged_decode_fused == af_paged_rope_append + af_paged_attention, bit for bit.
    Lengths 64 and 128 (L = 65, 129 after the append, 8 splits) give a last split
    that starts at the appended row itself: its only row comes from LDS and the
    rows it reads stay inside its staged block-table window."""
    say(f"paged fused fp8={fp8}")
    bs, layers = (32 if fp8 else 16), 2
    lengths = [0, 1, 15, 16, 31, 64, 128, 200, 1000, 2500]
    B = len(lengths)
    total = sum(n // bs + 2 for n in lengths) + 4
    dt = AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16
    bm = kv.BlockManager(total, bs, layers, dtype=dt)
    ids = [bm.allocate_block() for _ in range(total)]
    for blk in rng(770).permutation(ids):
        bm.free_block(int(blk))
    seqs = _sequences(bm, lengths)
    slots, positions, _ = bm.plan_decode(seqs)
    max_blocks = max((n + 1 + bs - 1) // bs for n in lengths)
    tables, lens = bm.export_tables(seqs, max_blocks)
    assert list(lens) == [n + 1 for n in lengths]
    max_pos = 4096
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((B, QKV), 771)
    P1 = Pool(layers, total, bs, fp8, 772)
    P2 = Pool(layers, total, bs, fp8, 772)
    q1, q2 = up(qkv), up(qkv)
    d_t, d_l, d_sl, d_p = up(tables), up(lens), up(slots), up(positions)
    o1, o2 = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    max_len = int(lens.max())
    for layer in range(layers):
        kv.launch_paged_rope_append(q1, B, P1.desc, layer, d_sl, d_p, d_c, d_s, max_pos, NQ)
        kv.launch_paged_attention(q1, QKV, P1.desc, layer, d_t, max_blocks, d_l, B, max_len, o1,
                                  Q_DIM, NQ, ws, num_splits=8)
        kv.launch_paged_decode_fused(q2, B, P2.desc, layer, d_sl, d_p, d_c, d_s, max_pos, d_t,
                                     max_blocks, max_len, o2, Q_DIM, NQ, ws, num_splits=8)
        assert np.array_equal(o1.download(np.uint16), o2.download(np.uint16)), layer
    assert np.array_equal(q1.download(np.uint16), q2.download(np.uint16))
    assert np.array_equal(P1.download().view(np.uint8), P2.download().view(np.uint8))


@pytest.mark.parametrize("nq,nkv", [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (6, 2), (9, 3),
                                    (8, 1)])
def test_paged_fp8_gqa_shapes(gpu, nq, nkv):
    """FP8 attention over every supported GQA ratio (1, 2, 3, 4, 8): even KV-head counts run
    the KV-head-pair kernel (GQ = 2 x GROUP query heads per workgroup), odd ones the single
    head kernel. Each sequence against the oracle at the FP8 and the fp16 bar, and the
    fused RoPE + append + attention kernel against append then attention bit for bit."""
    say(f"paged fp8 gqa nq={nq} nkv={nkv}")
    bs, layers = 32, 2
    kv_dim, q_dim = nkv * HD, nq * HD
    qkv_w = q_dim + 2 * kv_dim
    lengths = [1, 32, 33, 200, 1500, 4000]
    B = len(lengths)
    total = sum(n // bs + 2 for n in lengths) + 3
    bm = kv.BlockManager(total, bs, layers, dtype=AF_KV_FP8_E4M3)
    ids = [bm.allocate_block() for _ in range(total)]
    for blk in rng(790 + nq + nkv).permutation(ids):
        bm.free_block(int(blk))
    seqs = _sequences(bm, lengths)
    r = rng(791 + nq)
    shape = (layers, 2, total * bs, kv_dim)
    host = r.integers(0, 256, shape, dtype=np.uint8)
    host[(host & 0x7F) == 0x7F] = 0x00
    scales = r.uniform(0.004, 0.02, (layers, 2, nkv)).astype(np.float32)
    d_sc = up(scales)
    bufs = [up(host), up(host)]
    descs = [kv.make_pool(b, AF_KV_FP8_E4M3, bs, layers, nkv, HD, total, d_sc) for b in bufs]
    max_blocks = max((n + 1 + bs - 1) // bs for n in lengths)
    # attention over the current lengths, against the oracle
    tables, lens = bm.export_tables(seqs, max_blocks)
    q = randn_f16((B, q_dim), 792 + nkv)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_o = dev.DeviceBuffer(B * q_dim * 2)
    ws = kv.AttentionWorkspace(B, nq, nkv, HD, 0)
    for layer in range(layers):
        kv.launch_paged_attention(d_q, q_dim, descs[0], layer, d_t, max_blocks, d_l, B,
                                  int(lens.max()), d_o, q_dim, nq, ws)
        got = d_o.download(np.float16, (B, q_dim))
        for b in range(B):
            ref = oracle.paged_attention_fp8(q[b], host[layer, 0], host[layer, 1],
                                             scales[layer, 0], scales[layer, 1], tables[b],
                                             int(lens[b]), bs, nq, nkv, HD)
            assert_attn_close(got[b], ref, ATOL_FP8, RTOL_FP8, what=f"layer {layer} seq {b}")
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} (fp16 bar)")
    # one decode step: fused == paged append + attention, bit for bit
    slots, positions, _ = bm.plan_decode(seqs)
    tables, lens = bm.export_tables(seqs, max_blocks)
    max_pos = 4096
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((B, qkv_w), 793 + nq)
    q1, q2 = up(qkv), up(qkv)
    d_t, d_l, d_sl, d_p = up(tables), up(lens), up(slots), up(positions)
    o1, o2 = dev.DeviceBuffer(B * q_dim * 2), dev.DeviceBuffer(B * q_dim * 2)
    for layer in range(layers):
        kv.launch_paged_rope_append(q1, B, descs[0], layer, d_sl, d_p, d_c, d_s, max_pos, nq)
        kv.launch_paged_attention(q1, qkv_w, descs[0], layer, d_t, max_blocks, d_l, B,
                                  int(lens.max()), o1, q_dim, nq, ws)
        kv.launch_paged_decode_fused(q2, B, descs[1], layer, d_sl, d_p, d_c, d_s, max_pos, d_t,
                                     max_blocks, int(lens.max()), o2, q_dim, nq, ws)
        assert np.array_equal(o1.download(np.uint16), o2.download(np.uint16)), layer
    assert np.array_equal(q1.download(np.uint16), q2.download(np.uint16))
    assert np.array_equal(bufs[0].download(np.uint8), bufs[1].download(np.uint8))
