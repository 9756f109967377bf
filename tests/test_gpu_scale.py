"""GPU parity at BASELINE config points that the smaller tests do not reach.

* configs[1] at ctx 32768: one decode step at position 32768 (L = 32769 rows,
  the library's default split count), fused and as the two separate launches,
  against the float64 and float32 oracles (the decode attention of
  src/kernel/tiled_attention.cu:196-269; RoPE + append of rope.cu:11-46 and
  helpers.cu:126-139). The reference itself cannot run here: its shared-memory
  score buffer fails above about 12 160 rows (tiled_attention.cu:275-296).
* configs[4] at its stated scale: an FP8-E4M3 paged pool of 28 layers and
  32-token blocks (about 93 GiB), 128 sequences with contexts uniform in
  [8192, 16384], permuted block tables. The fused paged decode step runs at
  layer 0 and at layer 27, whose slabs start about 96 GB into the pool (byte
  offsets far above 2^32). Eight sequences (the longest, the shortest, and
  those holding the highest block ids among them) are checked against the
  oracle: the rotated query and the appended K/V codes bit for bit, attention
  within the FP8 bar and the fp16 bar. The unfused paged attention over the
  updated pool must equal the fused output bit for bit.
* configs[2] at its stated scale: an fp16 paged pool of 28 layers and
  16-token blocks (about 16 GiB, sized like bench.py's: the blocks the batch
  needs plus 10 %), 32 sequences with contexts uniform in [128, 8192],
  permuted block tables. The fused paged decode step (the compact batched
  grid) runs at layer 0 and at layer 27, whose slabs start past 2^32 bytes.
  Sampled sequences are checked against the oracle (the rotated query and the
  appended K/V rows bit for bit, attention at the fp16 bar), and the unfused
  kernel over the updated pool must equal the fused output bit for bit.
* configs[1] as bench.py times it: the 28-layer contiguous stack at ctx 8192,
  every layer's fused step in one captured hipGraph, each layer against the
  oracle.
"""
import numpy as np
import pytest

import oracle
from atomflow_amd import AF_KV_FP16, AF_KV_FP8_E4M3
from atomflow_amd import check as af_check
from atomflow_amd import device as dev
from atomflow_amd import kv
from atomflow_amd import lib as af_lib
from inputs import (ATOL_FP8, HD, KV_DIM, NKV, NQ, Q_DIM, QKV, RTOL_FP8, SEED_BASE, THETA,
                    assert_attn_close, contiguous_case)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def test_config2_ctx32k_fused_and_unfused(gpu):
    """BASELINE configs[1] at ctx 32768: append at pos 32768, attention over 32769 rows."""
    pos = 32768
    L = pos + 1
    max_seq = L + 127
    say(f"configs[1] ctx 32768: pos {pos}, L {L}, default splits "
        f"{kv.default_splits(max_seq, 1, NKV)}")
    c, s = oracle.rope_table(max_seq, HD, THETA)
    qkv, k, v = contiguous_case(max_seq, pos, SEED_BASE + 2)
    k[L:] = np.float16(np.nan)  # rows past the new token are never read
    v[L:] = np.float16(np.nan)
    d_c, d_s = up(c), up(s)
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 0)
    # two launches: RoPE + append, then attention (default splits)
    a_qkv, a_k, a_v, a_o = up(qkv), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_rope_append(a_qkv, a_k, a_v, d_c, d_s, pos, max_seq, NQ, NKV, HD)
    kv.launch_cached_attention_ex(a_qkv, a_k, a_v, a_o, L, max_seq, HD, NQ, NKV, ws, num_splits=0)
    # one fused launch on a second copy
    b_qkv, b_k, b_v, b_o = up(qkv), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2)
    kv.launch_decode_attention_fused(b_qkv, b_k, b_v, d_c, d_s, pos, max_seq, b_o, NQ, NKV, HD,
                                     ws, num_splits=0)
    dev.synchronize()
    for x, y, what in ((a_qkv, b_qkv, "qkv"), (a_k, b_k, "K"), (a_v, b_v, "V"),
                       (a_o, b_o, "attention")):
        assert np.array_equal(x.download(np.uint16), y.download(np.uint16)), what
    rq = oracle.rope_append(qkv, k, v, c, s, pos, NQ, NKV, HD)  # writes row pos of k, v
    assert np.array_equal(bits(b_qkv.download(np.float16)), bits(rq))
    assert np.array_equal(b_k.download(np.uint16, k.shape), bits(k))
    assert np.array_equal(b_v.download(np.uint16, v.shape), bits(v))
    got = b_o.download(np.float16)
    ref64 = oracle.cached_attention_f64(rq[:Q_DIM], k, v, L, NQ, NKV, HD)
    ref32 = oracle.cached_attention(rq[:Q_DIM], k, v, L, NQ, NKV, HD, threads=8)
    assert_attn_close(got, ref64, what="ctx 32768 vs fp64 oracle")
    assert_attn_close(got, ref32, what="ctx 32768 vs fp32 oracle")


def test_config2_28_layer_graph_ctx8k_vs_oracle(gpu):
    """BASELINE configs[1] as bench.py times it: 28 contiguous layers, ctx 8192, one
    fused RoPE + append + attention launch per layer (default split count) and the
    position advance captured in one hipGraph. Two replays (positions 8192 and
    8193), fresh QKV rows uploaded before each: every layer's rotated QKV row and
    appended K/V row bit for bit, its attention output within the fp16 bar of the
    float64 oracle (tiled_attention.cu:196-269 over the reference's per-layer
    [MAX_SEQ_LEN, KV_DIM] slabs, engine.cu:187-215)."""
    layers, pos0, steps = 28, 8192, 2
    max_seq = pos0 + 128
    say(f"configs[1] 28-layer graph: ctx {pos0}, max_seq {max_seq}, default splits "
        f"{kv.default_splits(max_seq, 1, NKV)}")
    c, s = oracle.rope_table(max_seq, HD, THETA)
    d_c, d_s = up(c), up(s)
    host = [contiguous_case(max_seq, pos0, SEED_BASE + 100 + 3 * l) for l in range(layers)]
    dev_l = [(dev.DeviceBuffer(QKV * 2), up(k), up(v), dev.DeviceBuffer(Q_DIM * 2))
             for (_, k, v) in host]
    ws = kv.AttentionWorkspace(1, NQ, NKV, HD, 0)
    d_pos = up(np.array([pos0], np.int32))
    d_st = up(np.array([0], np.int32))
    stream = dev.Stream()

    def step():
        for (qkv, k, v, o) in dev_l:
            kv.launch_decode_attention_fused(qkv, k, v, d_c, d_s, -1, max_seq, o, NQ, NKV, HD, ws,
                                             num_splits=0, d_pos=d_pos, d_status=d_st,
                                             stream=stream)
        dev.add_i32(d_pos.ptr, 1, 1, stream)

    graph = dev.Graph.capture(stream, step)
    try:
        for i in range(steps):
            pos = pos0 + i
            rows = [np.random.default_rng(SEED_BASE + 1000 * i + l).standard_normal(QKV)
                    .astype(np.float16) for l in range(layers)]
            for l in range(layers):
                dev_l[l][0].upload(rows[l])
            graph.launch(stream)
            stream.sync()
            for l in range(layers):
                _, k, v = host[l]
                rq = oracle.rope_append(rows[l], k, v, c, s, pos, NQ, NKV, HD)  # row pos of k, v
                qkv_d, k_d, v_d, o_d = dev_l[l]
                assert np.array_equal(bits(qkv_d.download(np.float16)), bits(rq)), (i, l)
                for d_cache, h_cache in ((k_d, k), (v_d, v)):
                    got_row = d_cache.download(np.uint16, (max_seq, KV_DIM))[pos]
                    assert np.array_equal(got_row, bits(h_cache[pos])), (i, l)
                ref = oracle.cached_attention_f64(rq[:Q_DIM], k, v, pos + 1, NQ, NKV, HD)
                assert_attn_close(o_d.download(np.float16), ref, what=f"step {i} layer {l}")
        assert d_pos.download(np.int32)[0] == pos0 + steps and d_st.download(np.int32)[0] == 0
    finally:
        graph.destroy()
        stream.destroy()


def _sample(rng_, tables, lens, k):
    """Longest, shortest, those with the highest block ids, then random ones."""
    order = [int(np.argmax(lens)), int(np.argmin(lens))]
    top = np.argsort([-t[: (n + 31) // 32].max() for t, n in zip(tables, lens)])
    for b in list(top) + list(rng_.permutation(len(lens))):
        if len(order) >= k:
            break
        if int(b) not in order:
            order.append(int(b))
    return order


def test_config5_fp8_paged_at_scale(gpu):
    """FP8 paged pool of ~93 GiB, B = 128, L in [8192, 16384]."""
    bs, layers, B = 32, 28, 128
    r = np.random.Generator(np.random.PCG64(SEED_BASE + 5))
    ctx = r.integers(8192, 16385, B)
    lens_after = ctx + 1
    need = int(sum((int(n) + bs - 1) // bs for n in lens_after))
    total = int(need * 1.1) + 8
    bm = kv.BlockManager(total, bs, layers, NKV, HD, AF_KV_FP8_E4M3)
    ids = [bm.allocate_block() for _ in range(total)]
    for b in r.permutation(ids):
        bm.free_block(int(b))
    seqs = []
    for n in ctx:
        sq = bm.seq_create()
        assert not isinstance(bm.seq_extend(sq, int(n)), int)
        seqs.append(sq)
    slots, positions, copies = bm.plan_decode(seqs)
    assert len(copies) == 0 and np.array_equal(positions, ctx)
    max_len = int(lens_after.max())
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    desc = bm.pool()
    nbytes = kv.pool_bytes(desc)
    slab_bytes = total * bs * KV_DIM
    say(f"configs[4] at scale: {total} blocks, pool {nbytes / 2**30:.1f} GiB, layer 27 K slab at "
        f"byte {54 * slab_bytes}, max block id in use {int(tables.max())}")
    assert nbytes > 2**36 and 54 * slab_bytes > 2**32
    lib = af_lib()
    pool = dev.DeviceBuffer(nbytes)
    scales = r.uniform(0.008, 0.014, (layers, 2, NKV)).astype(np.float32)
    d_scales = up(scales)
    af_check(lib.af_rt_fill_randn_fp8(pool.ptr, nbytes, 7, 448.0 / 5.0, None), "fill pool")
    bm.attach_pool(pool.ptr, d_scales.ptr)
    desc = bm.pool()
    max_pos = max_len + 1
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    d_tables, d_lens = up(tables), up(lens)
    d_slots, d_pos = up(slots), up(positions)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    sample = _sample(r, tables, lens, 8)
    for layer in (0, layers - 1):
        qkv = (r.standard_normal((B, QKV))).astype(np.float16)
        d_qkv = up(qkv)
        d_out = dev.DeviceBuffer(B * Q_DIM * 2)
        d_out2 = dev.DeviceBuffer(B * Q_DIM * 2)
        say(f"layer {layer}: fused paged decode over {B} sequences, {int(lens.sum())} rows")
        kv.launch_paged_decode_fused(d_qkv, B, desc, layer, d_slots, d_pos, d_c, d_s, max_pos,
                                     d_tables, max_blocks, max_len, d_out, Q_DIM, NQ, ws)
        # the unfused kernel over the updated pool and the rotated queries
        kv.launch_paged_attention(d_qkv, QKV, desc, layer, d_tables, max_blocks, d_lens, B,
                                  max_len, d_out2, Q_DIM, NQ, ws)
        dev.synchronize()
        got = d_out.download(np.float16, (B, Q_DIM))
        assert np.array_equal(bits(got), bits(d_out2.download(np.float16, (B, Q_DIM))))
        got_qkv = d_qkv.download(np.float16, (B, QKV))
        base_k = (2 * layer) * slab_bytes
        base_v = (2 * layer + 1) * slab_bytes
        for b in sample:
            n_blk = (int(lens[b]) + bs - 1) // bs
            blk = tables[b, :n_blk]
            # this sequence's blocks of the layer, downloaded into a compact slab
            kslab = np.empty((n_blk * bs, KV_DIM), np.uint8)
            vslab = np.empty((n_blk * bs, KV_DIM), np.uint8)
            for i, bid in enumerate(blk):
                off = int(bid) * bs * KV_DIM
                kslab[i * bs:(i + 1) * bs] = pool.download(np.uint8, (bs, KV_DIM),
                                                           offset=base_k + off)
                vslab[i * bs:(i + 1) * bs] = pool.download(np.uint8, (bs, KV_DIM),
                                                           offset=base_v + off)
            pos = int(positions[b])
            row = pos  # the compact slab's row of the new token
            got_k, got_v = kslab[row].copy(), vslab[row].copy()
            # oracle: RoPE of Q and K at pos, FP8 append of the new K/V row
            rq = oracle.rope_append(qkv[b], np.zeros((1, KV_DIM), np.float16),
                                    np.zeros((1, KV_DIM), np.float16), c[pos:], s[pos:], 0, NQ,
                                    NKV, HD)
            assert np.array_equal(bits(got_qkv[b]), bits(rq)), f"rotated qkv, sequence {b}"
            ref_k, ref_v = kslab.copy(), vslab.copy()
            oracle.paged_write_fp8(rq[Q_DIM:Q_DIM + KV_DIM], rq[Q_DIM + KV_DIM:], ref_k, ref_v,
                                   row, KV_DIM, HD, scales[layer, 0], scales[layer, 1])
            assert np.array_equal(got_k, ref_k[row]), f"appended K codes, sequence {b}"
            assert np.array_equal(got_v, ref_v[row]), f"appended V codes, sequence {b}"
            ref = oracle.paged_attention_fp8(rq[:Q_DIM], ref_k, ref_v, scales[layer, 0],
                                             scales[layer, 1], np.arange(n_blk, dtype=np.int32),
                                             int(lens[b]), bs, NQ, NKV, HD)
            what = f"configs[4] layer {layer} seq {b} L={int(lens[b])}"
            assert_attn_close(got[b], ref, ATOL_FP8, RTOL_FP8, what=what + " (fp8 bar)")
            assert_attn_close(got[b], ref, what=what + " (fp16 bar)")
        del d_qkv, d_out, d_out2
    pool.free()
    bm.close()


def test_config3_fp16_paged_at_scale(gpu):
    """fp16 paged pool of ~16 GiB, B = 32, L in [128, 8192]."""
    bs, layers, B = 16, 28, 32
    r = np.random.Generator(np.random.PCG64(SEED_BASE + 3))
    ctx = r.integers(128, 8193, B)
    lens_after = ctx + 1
    need = int(sum((int(n) + bs - 1) // bs for n in lens_after))
    total = int(need * 1.1) + 8  # bench.py's sizing: 10 % free-list headroom
    bm = kv.BlockManager(total, bs, layers, NKV, HD, AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(total)]
    for b in r.permutation(ids):
        bm.free_block(int(b))
    seqs = []
    for n in ctx:
        sq = bm.seq_create()
        assert not isinstance(bm.seq_extend(sq, int(n)), int)
        seqs.append(sq)
    slots, positions, copies = bm.plan_decode(seqs)
    assert len(copies) == 0 and np.array_equal(positions, ctx)
    max_len = int(lens_after.max())
    max_blocks = (max_len + bs - 1) // bs
    tables, lens = bm.export_tables(seqs, max_blocks)
    desc = bm.pool()
    nbytes = kv.pool_bytes(desc)
    slab_bytes = total * bs * KV_DIM * 2
    say(f"configs[2] at scale: {total} blocks, pool {nbytes / 2**30:.1f} GiB, layer 27 K slab at "
        f"byte {54 * slab_bytes}, max block id in use {int(tables.max())}")
    assert nbytes > 2**33 and 54 * slab_bytes > 2**32
    assert B * NKV * 2 >= dev.device_info()["compute_units"]  # the batched (compact grid) form
    lib = af_lib()
    pool = dev.DeviceBuffer(nbytes)
    af_check(lib.af_rt_fill_randn_f16(pool.ptr, nbytes // 2, 7, 1.0, None), "fill pool")
    bm.attach_pool(pool.ptr, None)
    desc = bm.pool()
    max_pos = max_len + 1
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    d_tables, d_lens = up(tables), up(lens)
    d_slots, d_pos = up(slots), up(positions)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    sample = _sample(r, tables, lens, 6)
    for layer in (0, layers - 1):
        qkv = (r.standard_normal((B, QKV))).astype(np.float16)
        d_qkv = up(qkv)
        d_out = dev.DeviceBuffer(B * Q_DIM * 2)
        d_out2 = dev.DeviceBuffer(B * Q_DIM * 2)
        say(f"layer {layer}: fused paged decode over {B} sequences, {int(lens.sum())} rows")
        kv.launch_paged_decode_fused(d_qkv, B, desc, layer, d_slots, d_pos, d_c, d_s, max_pos,
                                     d_tables, max_blocks, max_len, d_out, Q_DIM, NQ, ws)
        kv.launch_paged_attention(d_qkv, QKV, desc, layer, d_tables, max_blocks, d_lens, B,
                                  max_len, d_out2, Q_DIM, NQ, ws)
        dev.synchronize()
        got = d_out.download(np.float16, (B, Q_DIM))
        assert np.array_equal(bits(got), bits(d_out2.download(np.float16, (B, Q_DIM))))
        got_qkv = d_qkv.download(np.float16, (B, QKV))
        base_k = (2 * layer) * slab_bytes
        base_v = (2 * layer + 1) * slab_bytes
        row_bytes = KV_DIM * 2
        for b in sample:
            n_blk = (int(lens[b]) + bs - 1) // bs
            blk = tables[b, :n_blk]
            kslab = np.empty((n_blk * bs, KV_DIM), np.float16)
            vslab = np.empty((n_blk * bs, KV_DIM), np.float16)
            for i, bid in enumerate(blk):
                off = int(bid) * bs * row_bytes
                kslab[i * bs:(i + 1) * bs] = pool.download(np.float16, (bs, KV_DIM),
                                                           offset=base_k + off)
                vslab[i * bs:(i + 1) * bs] = pool.download(np.float16, (bs, KV_DIM),
                                                           offset=base_v + off)
            pos = int(positions[b])
            got_k, got_v = kslab[pos].copy(), vslab[pos].copy()
            rq = oracle.rope_append(qkv[b], np.zeros((1, KV_DIM), np.float16),
                                    np.zeros((1, KV_DIM), np.float16), c[pos:], s[pos:], 0, NQ,
                                    NKV, HD)
            assert np.array_equal(bits(got_qkv[b]), bits(rq)), f"rotated qkv, sequence {b}"
            assert np.array_equal(bits(got_k), bits(rq[Q_DIM:Q_DIM + KV_DIM])), f"K row, seq {b}"
            assert np.array_equal(bits(got_v), bits(rq[Q_DIM + KV_DIM:])), f"V row, seq {b}"
            ref = oracle.paged_attention_f16(rq[:Q_DIM], kslab, vslab,
                                             np.arange(n_blk, dtype=np.int32), int(lens[b]), bs,
                                             NQ, NKV, HD)
            assert_attn_close(got[b], ref, what=f"configs[2] layer {layer} seq {b} L={int(lens[b])}")
        del d_qkv, d_out, d_out2
    pool.free()
    bm.close()
