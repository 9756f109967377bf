"""GPU parity of the shared-prefix ("cascade") paged attention
(af_paged_attention_shared_prefix, af_paged_decode_fused_shared_prefix).

Forks of one prompt share its blocks under copy-on-write (the sandbox's
BlockManager, src/experimental/server_arch/paged_kv_manager.h:51,61). The
cascade attends the shared rows once for the batch on the matrix cores and the
rest per sequence, merging both in the split-K combine. Its result is the same
attention as af_paged_attention: every sequence is checked against the oracle on
its own block table and length (fp16 within 2e-3 / 1e-2, FP8 within 5e-2), and
against af_paged_attention on the same inputs to the same bar. The fused form
leaves qkv_out and the pool bit for bit as af_paged_decode_fused does.
"""
import numpy as np
import pytest

import atomflow_amd
import oracle
from atomflow_amd import AF_KV_FP8_E4M3, AF_KV_FP16, AF_KV_POOL_SHARED_BLOCKS
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import (ATOL_FP8, HD, KV_DIM, NKV, NQ, Q_DIM, QKV, RTOL_FP8, THETA,
                    assert_attn_close, randn_f16, rng)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


class Pool:
    """Host mirror + device copy of a paged pool [layers][K,V][blocks*bs][kv_dim]."""

    def __init__(self, layers, blocks, bs, fp8, seed):
        shape = (layers, 2, blocks * bs, KV_DIM)
        r = rng(seed)
        if fp8:
            h = r.integers(0, 256, shape, dtype=np.uint8)
            h[(h & 0x7F) == 0x7F] = 0x00  # no NaN codes
            self.scales = r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32)
            self.d_scales = up(self.scales)
        else:
            h = randn_f16(shape, seed)
            self.scales, self.d_scales = None, None
        self.host, self.bs, self.fp8 = h, bs, fp8
        self.buf = up(h)
        self.desc = kv.make_pool(self.buf, AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16, bs, layers, NKV,
                                 HD, blocks, self.d_scales)

    def copy_rows(self, src, dst, rows):
        """A copy-on-write copy (rows [0, rows) of block src into dst, every layer)."""
        b = self.bs
        self.host[:, :, dst * b:dst * b + rows] = self.host[:, :, src * b:src * b + rows]

    def sync(self):
        self.buf.upload(self.host)

    def download(self):
        return self.buf.download(self.host.dtype, self.host.shape)

    def reference(self, q, layer, table, L, host=None):
        h = self.host if host is None else host
        if self.fp8:
            return oracle.paged_attention_fp8(q, h[layer, 0], h[layer, 1], self.scales[layer, 0],
                                              self.scales[layer, 1], table, L, self.bs, NQ, NKV,
                                              HD)
        return oracle.paged_attention_f16(q, h[layer, 0], h[layer, 1], table, L, self.bs, NQ,
                                          NKV, HD)


def forked_batch(prefix, suffixes, bs, layers, fp8, seed, extra_blocks=8):
    """A root of `prefix` rows and len(suffixes)-1 forks, sequence i extended by
    suffixes[i] rows (the copy-on-write copies of a shared partial block applied
    to the pool). Returns (pool, bm, seqs, tables, lens, max_blocks)."""
    need = (prefix + bs - 1) // bs + sum((n + bs) // bs + 1 for n in suffixes) + extra_blocks
    bm = kv.BlockManager(need, bs, layers, dtype=AF_KV_FP8_E4M3 if fp8 else AF_KV_FP16)
    ids = [bm.allocate_block() for _ in range(need)]
    for b in rng(seed).permutation(ids):
        bm.free_block(int(b))
    P = Pool(layers, need, bs, fp8, seed + 1)
    root = bm.seq_create()
    assert not isinstance(bm.seq_extend(root, prefix), int)
    seqs = [root] + [bm.seq_fork(root) for _ in suffixes[1:]]
    for s, n in zip(seqs, suffixes):
        if n:
            r = bm.seq_extend(s, int(n))
            assert not isinstance(r, int), r
            src, dst, rows = r[1]
            if rows:
                P.copy_rows(src, dst, rows)
    P.sync()
    lens_all = [prefix + n for n in suffixes]
    max_blocks = (max(lens_all) + 1 + bs - 1) // bs + 1
    tables, lens = bm.export_tables(seqs, max_blocks)
    assert list(lens) == lens_all
    return P, bm, seqs, tables, lens, max_blocks


@pytest.mark.parametrize("prefix,bs,splits,psplits", [
    (2048, 16, 0, 0), (205, 16, 0, 0), (64, 16, 0, 0), (1, 16, 0, 0), (1000, 32, 0, 0),
    (2048, 16, 5, 1), (2048, 16, 3, 32), (777, 16, 1, 7)])
def test_shared_prefix_fp16_vs_oracle(gpu, prefix, bs, splits, psplits):
    say(f"shared prefix fp16 prefix={prefix} bs={bs} splits={splits} prefix_splits={psplits}")
    suffixes = [0, 1, 2, 15, 64, 65, 700, 1100, 3]
    layers = 2
    P, bm, seqs, tables, lens, max_blocks = forked_batch(prefix, suffixes, bs, layers, False,
                                                         0x5A00 + prefix)
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x5A01 + prefix)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    d_root = up(tables[0])
    o_c, o_p = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    max_len = int(lens.max())
    for layer in range(layers):
        kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, P.desc, layer, d_root, prefix, d_t,
                                                max_blocks, d_l, B, max_len, o_c, Q_DIM, NQ, ws,
                                                num_splits=splits, prefix_splits=psplits)
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B, max_len,
                                  o_p, Q_DIM, NQ, ws)
        got = o_c.download(np.float16, (B, Q_DIM))
        plain = o_p.download(np.float16, (B, Q_DIM))
        for b in range(B):
            ref = P.reference(q[b], layer, tables[b], int(lens[b]))
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} L={lens[b]}")
            assert_attn_close(got[b], plain[b].astype(np.float64),
                              what=f"vs af_paged_attention, layer {layer} seq {b}")


def test_shared_prefix_fp8_vs_oracle(gpu):
    say("shared prefix fp8 prefix=1500 bs=32")
    prefix, bs, layers = 1500, 32, 2
    suffixes = [0, 1, 31, 32, 33, 500, 2000, 7]
    P, bm, seqs, tables, lens, max_blocks = forked_batch(prefix, suffixes, bs, layers, True, 0x5B00)
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x5B01)
    d_q, d_t, d_l, d_root = up(q), up(tables), up(lens), up(tables[0])
    o = dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    for layer in range(layers):
        kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, P.desc, layer, d_root, prefix, d_t,
                                                max_blocks, d_l, B, int(lens.max()), o, Q_DIM, NQ,
                                                ws)
        got = o.download(np.float16, (B, Q_DIM))
        for b in range(B):
            ref = P.reference(q[b], layer, tables[b], int(lens[b]))
            assert_attn_close(got[b], ref, ATOL_FP8, RTOL_FP8, what=f"fp8 layer {layer} seq {b}")


def test_shared_prefix_zero_equals_paged_bitwise(gpu):
    """prefix_len 0 is af_paged_attention itself: same bits."""
    say("shared prefix 0 == paged attention")
    P, bm, seqs, tables, lens, max_blocks = forked_batch(300, [5, 50, 500], 16, 1, False, 0x5C00)
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x5C01)
    d_q, d_t, d_l = up(q), up(tables), up(lens)
    a, b = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, P.desc, 0, d_t, 0, d_t, max_blocks, d_l,
                                            B, int(lens.max()), a, Q_DIM, NQ, ws)
    kv.launch_paged_attention(d_q, Q_DIM, P.desc, 0, d_t, max_blocks, d_l, B, int(lens.max()), b,
                              Q_DIM, NQ, ws)
    assert np.array_equal(a.download(np.uint16), b.download(np.uint16))


@pytest.mark.parametrize("fp8", [False, True])
def test_shared_prefix_fused_step(gpu, fp8):
    """af_paged_decode_fused_shared_prefix: qkv_out and the pool equal
    af_paged_decode_fused's bit for bit (the copy-on-write copy of the shared tail
    applied first), attention within tolerance of it and of the oracle."""
    say(f"shared prefix fused step fp8={fp8}")
    bs = 32 if fp8 else 16
    prefix, layers = 1000 + bs // 2, 2  # a shared partial tail block
    suffixes = [0, 0, 1, 9, 40, 300, 1200]
    P1, bm, seqs, tables0, _, _ = forked_batch(prefix, suffixes, bs, layers, fp8, 0x5D00 + fp8)
    slots, positions, copies = bm.plan_decode(seqs, max_copies=len(seqs))
    for src, dst, rows in copies:  # forks still sharing the partial tail copy it now
        P1.copy_rows(src, dst, rows)
    P1.sync()
    host0 = P1.host.copy()
    max_blocks = (prefix + max(suffixes) + 2 + bs - 1) // bs + 1
    tables, lens = bm.export_tables(seqs, max_blocks)
    assert list(lens) == [prefix + n + 1 for n in suffixes]
    B = len(seqs)
    P2 = Pool(layers, P1.host.shape[2] // bs, bs, fp8, 0)
    P2.host[...] = host0
    P2.sync()
    if fp8:
        P2.scales = P1.scales
        P2.d_scales.upload(P1.scales)
    max_pos = 4096
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    qkv = randn_f16((layers, B, QKV), 0x5D10 + fp8)
    q1, q2 = up(qkv), up(qkv)
    d_t, d_sl, d_p = up(tables), up(slots), up(positions)
    # the shared rows through the root's table as it was before this step
    d_root = up(tables0[0])
    o1, o2 = dev.DeviceBuffer(layers * B * Q_DIM * 2), dev.DeviceBuffer(layers * B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    max_len = int(lens.max())
    for layer in range(layers):
        qo, oo = layer * B * QKV * 2, layer * B * Q_DIM * 2
        kv.launch_paged_decode_fused_shared_prefix(q1.ptr + qo, B, P1.desc, layer, d_sl, d_p, d_c,
                                                   d_s, max_pos, d_root, prefix, d_t, max_blocks,
                                                   max_len, o1.ptr + oo, Q_DIM, NQ, ws)
        kv.launch_paged_decode_fused(q2.ptr + qo, B, P2.desc, layer, d_sl, d_p, d_c, d_s, max_pos,
                                     d_t, max_blocks, max_len, o2.ptr + oo, Q_DIM, NQ, ws)
    assert np.array_equal(q1.download(np.uint16), q2.download(np.uint16))
    pool_after = P1.download()
    assert np.array_equal(pool_after.view(np.uint8), P2.download().view(np.uint8))
    got = o1.download(np.float16, (layers, B, Q_DIM))
    plain = o2.download(np.float16, (layers, B, Q_DIM))
    roped = q1.download(np.float16, (layers, B, QKV))
    atol, rtol = (ATOL_FP8, RTOL_FP8) if fp8 else (2e-3, 1e-2)
    for layer in range(layers):
        for b in range(B):
            ref = P1.reference(roped[layer, b, :Q_DIM], layer, tables[b], int(lens[b]),
                               host=pool_after)
            assert_attn_close(got[layer, b], ref, atol, rtol, what=f"layer {layer} seq {b}")
            assert_attn_close(got[layer, b], plain[layer, b].astype(np.float64), atol, rtol,
                              what=f"vs fused paged, layer {layer} seq {b}")


def test_shared_prefix_configs3_shape(gpu):
    """BASELINE configs[3]'s shape (64 forks of a 2048-row prefix, suffixes 1..1024)
    against af_paged_attention and, for a sample of sequences, the oracle."""
    say("shared prefix configs[3] shape")
    r = np.random.Generator(np.random.PCG64(0xA70F14))
    suffixes = [int(n) for n in r.integers(1, 1025, 64)]
    P, bm, seqs, tables, lens, max_blocks = forked_batch(2048, suffixes, 16, 1, False, 0x5E00)
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x5E01)
    d_q, d_t, d_l, d_root = up(q), up(tables), up(lens), up(tables[0])
    a, b = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    max_len = int(lens.max())
    kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, P.desc, 0, d_root, 2048, d_t, max_blocks,
                                            d_l, B, max_len, a, Q_DIM, NQ, ws)
    kv.launch_paged_attention(d_q, Q_DIM, P.desc, 0, d_t, max_blocks, d_l, B, max_len, b, Q_DIM,
                              NQ, ws)
    got = a.download(np.float16, (B, Q_DIM))
    plain = b.download(np.float16, (B, Q_DIM))
    assert_attn_close(got, plain.astype(np.float64), what="vs af_paged_attention")
    for i in range(0, B, 9):
        ref = P.reference(q[i], 0, tables[i], int(lens[i]))
        assert_attn_close(got[i], ref, what=f"seq {i} L={lens[i]}")
    # the forks map the prefix blocks: with AF_KV_POOL_SHARED_BLOCKS both paths take the
    # kernels with the default load policy, and give the same bits as above
    shared = kv.make_pool(P.buf, AF_KV_FP16, 16, 1, NKV, HD, P.desc.total_blocks,
                          flags=AF_KV_POOL_SHARED_BLOCKS)
    kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, shared, 0, d_root, 2048, d_t, max_blocks,
                                            d_l, B, max_len, a, Q_DIM, NQ, ws)
    kv.launch_paged_attention(d_q, Q_DIM, shared, 0, d_t, max_blocks, d_l, B, max_len, b, Q_DIM,
                              NQ, ws)
    assert np.array_equal(a.download(np.uint16), got.view(np.uint16).ravel())
    assert np.array_equal(b.download(np.uint16), plain.view(np.uint16).ravel())


@pytest.mark.parametrize("fp8,splits", [(False, 0), (False, 1), (False, 3), (True, 0)])
def test_shared_prefix_lengths_below_prefix(gpu, fp8, splits):
    """Sequences no longer than prefix_len (a stale or too-long prefix_len): one
    with L < prefix_len attends its own rows [0, L) and leaves the prefix records
    out; L == prefix_len attends the prefix records alone. Each equals the oracle
    on its table and length, and af_paged_attention on the same inputs."""
    say(f"shared prefix, lengths below the prefix, fp8={fp8} splits={splits}")
    prefix = 640
    P, bm, seqs, tables, lens_all, max_blocks = forked_batch(
        prefix, [0, 5, 100, 400, 0, 1, 2, 3, 4], 16, 2, fp8, 0x6100 + splits)
    lens = np.array([1, 645, 17, 1040, 639, 640, 300, 64, 65], np.int32)
    assert np.all(lens <= lens_all)  # every row attended is mapped by the table
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x6101 + splits)
    d_q, d_t, d_l, d_root = up(q), up(tables), up(lens), up(tables[0])
    o_c, o_p = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    max_len = int(lens.max())
    kw = {"atol": ATOL_FP8, "rtol": RTOL_FP8} if fp8 else {}  # the oracle bar for FP8 KV
    for layer in range(2):
        kv.launch_paged_attention_shared_prefix(d_q, Q_DIM, P.desc, layer, d_root, prefix, d_t,
                                                max_blocks, d_l, B, max_len, o_c, Q_DIM, NQ, ws,
                                                num_splits=splits)
        kv.launch_paged_attention(d_q, Q_DIM, P.desc, layer, d_t, max_blocks, d_l, B, max_len,
                                  o_p, Q_DIM, NQ, ws)
        got = o_c.download(np.float16, (B, Q_DIM))
        plain = o_p.download(np.float16, (B, Q_DIM))
        for b in range(B):
            ref = P.reference(q[b], layer, tables[b], int(lens[b]))
            assert_attn_close(got[b], ref, what=f"layer {layer} seq {b} L={lens[b]}", **kw)
            assert_attn_close(got[b], plain[b].astype(np.float64),
                              what=f"vs af_paged_attention, layer {layer} seq {b}")


def test_shared_prefix_graph_replays(gpu):
    """Both launches captured in one hipGraph: three replays equal the eager call."""
    say("shared prefix under graph replay")
    P, bm, seqs, tables, lens, max_blocks = forked_batch(640, [3, 100, 900, 17], 16, 1, False,
                                                         0x5F00)
    B = len(seqs)
    q = randn_f16((B, Q_DIM), 0x5F01)
    d_q, d_t, d_l, d_root = up(q), up(tables), up(lens), up(tables[0])
    eager, replay = dev.DeviceBuffer(B * Q_DIM * 2), dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    stream = dev.Stream()
    run = lambda out: kv.launch_paged_attention_shared_prefix(
        d_q, Q_DIM, P.desc, 0, d_root, 640, d_t, max_blocks, d_l, B, int(lens.max()), out, Q_DIM,
        NQ, ws, stream=stream)
    graph = dev.Graph.capture(stream, lambda: run(replay))
    for i in range(3):
        run(eager)
        replay.fill_u32(0, stream)
        graph.launch(stream)
        stream.sync()
        assert np.array_equal(eager.download(np.uint16), replay.download(np.uint16)), f"replay {i}"
    graph.destroy()


def test_shared_prefix_rejects_bad_arguments(gpu):
    say("shared prefix argument checks")
    P, bm, seqs, tables, lens, max_blocks = forked_batch(200, [1, 2], 16, 1, False, 0x6000)
    B = len(seqs)
    d_q, d_t, d_l = up(randn_f16((B, Q_DIM), 1)), up(tables), up(lens)
    out = dev.DeviceBuffer(B * Q_DIM * 2)
    ws = kv.AttentionWorkspace(B, NQ, NKV, HD, 0)
    lib = atomflow_amd.lib()
    import ctypes

    def call(prefix_table, prefix, psplits, max_len=int(lens.max()), ws_bytes=ws.nbytes):
        return lib.af_paged_attention_shared_prefix(
            d_q.ptr, Q_DIM, ctypes.byref(P.desc), 0, prefix_table, prefix, psplits, d_t.ptr,
            max_blocks, d_l.ptr, B, max_len, out.ptr, Q_DIM, NQ, 0, ws.ptr, ws_bytes, None)

    assert call(d_t.ptr, -1, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(None, 200, 0) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(d_t.ptr, 200, 5) == atomflow_amd.AF_ERR_INVALID_ARG  # > ceil(200 / 64) splits
    assert call(d_t.ptr, 200, -1) == atomflow_amd.AF_ERR_INVALID_ARG
    assert call(d_t.ptr, max_blocks * 16 + 1, 0) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert call(d_t.ptr, 200, 0, ws_bytes=1024) == atomflow_amd.AF_ERR_WORKSPACE
    pool64 = kv.make_pool(P.buf, AF_KV_FP16, 16, 1, NKV, 64, P.host.shape[2] // 16)
    assert lib.af_paged_attention_shared_prefix(
        d_q.ptr, Q_DIM, ctypes.byref(pool64), 0, d_t.ptr, 200, 0, d_t.ptr, max_blocks, d_l.ptr,
        B, int(lens.max()), out.ptr, Q_DIM, NQ, 0, ws.ptr, ws.nbytes,
        None) == atomflow_amd.AF_ERR_UNSUPPORTED
    assert call(d_t.ptr, 200, 4) == 0
    dev.synchronize()
