"""GPU parity of the prefill path: multi-token RoPE + append and causal attention
over a prompt chunk (libatomflow_kv.so vs the CPU oracle).

Append: bit-exact, whole caches compared (untouched rows included). Attention:
within the fp16 bar (max-abs 2e-3, rel 1e-2) of the float64 oracle and of the
fp32 oracle of the reference's causal kernel (tiled_attention.cu:34-130); query
rows whose softmax has a single key are compared bit for bit (out = V row).
"""
import numpy as np
import pytest

import atomflow_amd
import oracle
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import (HD, KV_DIM, NKV, NQ, Q_DIM, QKV, THETA, assert_attn_close, randn_f16, rng)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def rope_tables(max_seq):
    c, s = oracle.rope_table(max_seq, HD, THETA)
    return c, s, up(c), up(s)


def caches(max_seq, filled, seed):
    k = randn_f16((max_seq, KV_DIM), seed)
    v = randn_f16((max_seq, KV_DIM), seed + 1)
    k[filled:] = np.float16(7.0)  # canaries
    v[filled:] = np.float16(-7.0)
    return k, v


# ---- multi-token append ------------------------------------------------------
@pytest.mark.parametrize("p0,n", [(0, 1), (0, 37), (100, 300), (4000, 96)])
def test_prefill_rope_append_bit_exact(gpu, p0, n):
    say(f"prefill_rope_append p0={p0} n={n}")
    max_seq = 4096
    c, s, d_c, d_s = rope_tables(max_seq)
    qkv = randn_f16((n, QKV), 0xA70F30 + n)
    k, v = caches(max_seq, p0, 0xA70F31 + p0)
    d_qkv, d_k, d_v = up(qkv), up(k), up(v)
    kv.launch_prefill_rope_append(d_qkv, n, d_k, d_v, d_c, d_s, p0, max_seq, NQ, NKV, HD)
    ref = oracle.prefill_rope_append(qkv, k, v, c, s, p0, NQ, NKV, HD)
    assert np.array_equal(bits(d_qkv.download(np.float16, qkv.shape)), bits(ref))
    assert np.array_equal(bits(d_k.download(np.float16, k.shape)), bits(k))
    assert np.array_equal(bits(d_v.download(np.float16, v.shape)), bits(v))


def test_prefill_rope_append_range_checks(gpu):
    say("prefill_rope_append: host range error, device start skips rows past max_seq")
    max_seq = 64
    c, s, d_c, d_s = rope_tables(max_seq)
    qkv = randn_f16((10, QKV), 0xA70F32)
    k, v = caches(max_seq, 60, 0xA70F33)
    d_qkv, d_k, d_v = up(qkv), up(k), up(v)
    with pytest.raises(RuntimeError):
        kv.launch_prefill_rope_append(d_qkv, 10, d_k, d_v, d_c, d_s, 55, max_seq, NQ, NKV, HD)
    assert np.array_equal(bits(d_k.download(np.float16, k.shape)), bits(k))
    # device start 58: rows 58..63 written, rows for positions 64..67 skipped + status
    d_p0 = up(np.array([58], np.int32))
    status = up(np.zeros(1, np.int32))
    kv.launch_prefill_rope_append(d_qkv, 10, d_k, d_v, d_c, d_s, 0, max_seq, NQ, NKV, HD,
                                  d_p0=d_p0, d_status=status)
    assert status.download(np.int32)[0] == atomflow_amd.AF_ERR_OUT_OF_RANGE
    ref = oracle.prefill_rope_append(qkv[:6], k, v, c, s, 58, NQ, NKV, HD)
    got = d_qkv.download(np.float16, qkv.shape)
    assert np.array_equal(bits(got[:6]), bits(ref))
    assert np.array_equal(bits(got[6:]), bits(qkv[6:]))  # skipped rows untouched
    assert np.array_equal(bits(d_k.download(np.float16, k.shape)), bits(k))
    assert np.array_equal(bits(d_v.download(np.float16, v.shape)), bits(v))


# ---- causal attention ----------------------------------------------------------
def run_prefill(q, k, v, p0, n, kv_len, q_stride, out_stride=Q_DIM):
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = up(np.full((n, out_stride), np.float16(3.0)))
    kv.launch_prefill_attention(d_q, q_stride, d_k, d_v, d_o, out_stride, p0, n, kv_len,
                                k.shape[0], NQ, NKV, HD)
    return d_o.download(np.float16, (n, out_stride))


@pytest.mark.parametrize("p0,n,kv_len", [
    (0, 1, 1), (0, 17, 17), (0, 64, 64), (0, 200, 200), (0, 300, 300),
    (100, 77, 177), (1000, 129, 1129), (37, 250, 287), (0, 50, 30), (5, 40, 20)])
def test_prefill_attention_vs_oracle(gpu, p0, n, kv_len):
    say(f"prefill_attention p0={p0} n={n} kv_len={kv_len}")
    max_seq = max(kv_len, p0 + n) + 5
    q = randn_f16((n, QKV), 0xA70F40 + 3 * n + p0)  # Q heads in the first Q_DIM columns
    k, v = caches(max_seq, kv_len, 0xA70F41 + kv_len)
    got = run_prefill(q, k, v, p0, n, kv_len, QKV, out_stride=Q_DIM + 64)
    assert np.all(got[:, Q_DIM:] == np.float16(3.0))  # nothing past the row's heads
    got = got[:, :Q_DIM]
    ref64 = oracle.prefill_attention_f64(q, k, v, p0, n, kv_len, NQ, NKV, HD)
    assert_attn_close(got, ref64, what="vs fp64")
    ref32 = oracle.prefill_attention(q, k, v, p0, n, kv_len, NQ, NKV, HD, threads=8)
    assert_attn_close(got, ref32, what="vs fp32 oracle")
    single = [i for i in range(n) if min(p0 + i + 1, kv_len) == 1]
    for i in single:  # one key: softmax weight exactly 1, out = V row 0
        assert np.array_equal(bits(got[i]), bits(ref32[i])), i


def test_prefill_attention_long_chunk_sampled_rows(gpu):
    say("prefill_attention p0=0 n=2048 (sampled rows vs decode oracle)")
    n = 2048
    q = randn_f16((n, Q_DIM), 0xA70F50)
    k, v = caches(n, n, 0xA70F51)
    got = run_prefill(q, k, v, 0, n, n, Q_DIM)
    rows = sorted(set(rng(7).choice(n, 24, replace=False).tolist()) | {0, 127, 128, n - 1})
    for i in rows:
        ref = oracle.cached_attention_f64(q[i], k, v, i + 1, NQ, NKV, HD)
        assert_attn_close(got[i], ref, what=f"row {i}")


@pytest.mark.parametrize("p0,n,kv_len", [(0, 6000, 6000), (3000, 5500, 8500), (0, 5600, 4100)])
def test_prefill_attention_long_chunks(gpu, p0, n, kv_len):
    """Long chunks (thousands of workgroups, many LDS tiles per workgroup); sampled
    rows against the float64 decode oracle over min(p0+i+1, kv_len) rows."""
    say(f"prefill_attention p0={p0} n={n} kv_len={kv_len} (sampled rows)")
    max_seq = max(kv_len, p0 + n)
    q = randn_f16((n, Q_DIM), 0xA70F58 + n)
    k, v = caches(max_seq, kv_len, 0xA70F59 + p0)
    got = run_prefill(q, k, v, p0, n, kv_len, Q_DIM)
    edge = {0, 31, 32, 63, 64, 255, 256, 257, n - 257, n - 256, n - 1, max(0, kv_len - p0 - 1)}
    rows = sorted(set(rng(p0 + n).choice(n, 20, replace=False).tolist()) | {i for i in edge if 0 <= i < n})
    for i in rows:
        L = min(p0 + i + 1, kv_len)
        ref = oracle.cached_attention_f64(q[i], k, v, L, NQ, NKV, HD)
        assert_attn_close(got[i], ref, what=f"row {i} (L={L})")


# ---- key pieces: heavy query tiles cut into key ranges, merged by the last ------
def run_prefill_ws(q, k, v, p0, n, kv_len, q_stride, key_pieces, ws=None, out_stride=Q_DIM):
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = up(np.full((n, out_stride), np.float16(3.0)))
    if ws is None:
        ws = kv.PrefillWorkspace(p0, n, kv_len, NQ, key_pieces)
    kv.launch_prefill_attention_ws(d_q, q_stride, d_k, d_v, d_o, out_stride, p0, n, kv_len,
                                   k.shape[0], NQ, NKV, HD, ws, key_pieces=key_pieces)
    return d_o.download(np.float16, (n, out_stride)), ws


@pytest.mark.parametrize("p0,n,kv_len,key_pieces", [
    (0, 2048, 2048, 0),      # a 2k prompt: tiles cut into up to 3 pieces
    (3000, 300, 3300, 0),    # a chunk late in a prompt: 4 pieces per tile
    (0, 700, 700, 2),        # 2 pieces, a partial last tile
    (2000, 333, 2200, 3),    # queries past kv_len, a partial last wave
    (0, 200, 200, 0)])       # too little work to cut: the plain launch
def test_prefill_attention_key_pieces_vs_oracle(gpu, p0, n, kv_len, key_pieces):
    """Every row against the float64 decode oracle over min(p0+i+1, kv_len) rows
    (sampled for the 2k prompt); a second launch on the same workspace (its
    counters re-zeroed by the first) gives the same bits."""
    say(f"prefill key pieces p0={p0} n={n} kv_len={kv_len} key_pieces={key_pieces}")
    max_seq = max(kv_len, p0 + n) + 3
    q = randn_f16((n, QKV), 0xA70F90 + n + p0)
    k, v = caches(max_seq, kv_len, 0xA70F91 + kv_len)
    got, ws = run_prefill_ws(q, k, v, p0, n, kv_len, QKV, key_pieces, out_stride=Q_DIM + 64)
    assert np.all(got[:, Q_DIM:] == np.float16(3.0))  # nothing past the row's heads
    got = got[:, :Q_DIM]
    edge = {0, 127, 128, 1000, n - 129, n - 1}
    rows = range(n) if n <= 400 else sorted(
        set(rng(n).choice(n, 40, replace=False).tolist()) | {i for i in edge if 0 <= i < n})
    for i in rows:
        L = min(p0 + i + 1, kv_len)
        ref = oracle.cached_attention_f64(q[i, :Q_DIM], k, v, L, NQ, NKV, HD)
        assert_attn_close(got[i], ref, what=f"row {i} (L={L})")
    again, _ = run_prefill_ws(q, k, v, p0, n, kv_len, QKV, key_pieces, ws=ws,
                              out_stride=Q_DIM + 64)
    assert np.array_equal(bits(again[:, :Q_DIM]), bits(got))


def test_prefill_attention_one_piece_equals_plain(gpu):
    say("prefill key_pieces=1 == af_prefill_attention bit for bit; workspace checks")
    p0, n, kv_len = 0, 1024, 1024
    q = randn_f16((n, Q_DIM), 0xA70F95)
    k, v = caches(kv_len, kv_len, 0xA70F96)
    plain = run_prefill(q, k, v, p0, n, kv_len, Q_DIM)
    one, _ = run_prefill_ws(q, k, v, p0, n, kv_len, Q_DIM, 1)
    assert np.array_equal(bits(one), bits(plain))
    lib = atomflow_amd.lib()
    assert lib.af_prefill_workspace_size(p0, n, kv_len, NQ, 1) == 64 * 1024
    big = lib.af_prefill_workspace_size(p0, n, kv_len, NQ, 0)
    assert big > 64 * 1024
    d_q, d_k, d_v = up(q), up(k), up(v)
    d_o = up(np.zeros((n, Q_DIM), np.float16))
    small = kv.PrefillWorkspace(p0, n, kv_len, NQ, 1)  # counters only
    with pytest.raises(atomflow_amd.AfError) as e:
        kv.launch_prefill_attention_ws(d_q, Q_DIM, d_k, d_v, d_o, Q_DIM, p0, n, kv_len, kv_len,
                                       NQ, NKV, HD, small, key_pieces=0)
    assert e.value.status == atomflow_amd.AF_ERR_WORKSPACE
    with pytest.raises(atomflow_amd.AfError):
        kv.launch_prefill_attention_ws(d_q, Q_DIM, d_k, d_v, d_o, Q_DIM, p0, n, kv_len, kv_len,
                                       NQ, NKV, HD, None, key_pieces=0)
    with pytest.raises(atomflow_amd.AfError):
        kv.launch_prefill_attention_ws(d_q, Q_DIM, d_k, d_v, d_o, Q_DIM, p0, n, kv_len, kv_len,
                                       NQ, NKV, HD, small, key_pieces=5)


def test_prefill_attention_large_scores(gpu):
    say("prefill_attention: scaled inputs (scores up to ~100), lazy rescale path")
    p0, n, kv_len = 0, 160, 160
    q = randn_f16((n, Q_DIM), 0xA70F52, scale=3.0)
    k = randn_f16((kv_len, KV_DIM), 0xA70F53, scale=3.0)
    v = randn_f16((kv_len, KV_DIM), 0xA70F54)
    got = run_prefill(q, k, v, p0, n, kv_len, Q_DIM)
    assert_attn_close(got, oracle.prefill_attention_f64(q, k, v, p0, n, kv_len, NQ, NKV, HD))


def test_tiled_attention_reference_form(gpu):
    say("launch_tiled_attention_kernel: seq_q 70 / seq_kv 70, seq_kv 1, seq_kv 0")
    n = 70
    q = randn_f16((n, Q_DIM), 0xA70F55)
    k = randn_f16((n, KV_DIM), 0xA70F56)
    v = randn_f16((n, KV_DIM), 0xA70F57)
    d_q, d_k, d_v, d_o = up(q), up(k), up(v), up(np.zeros((n, Q_DIM), np.float16))
    kv.launch_tiled_attention_kernel(d_q, d_k, d_v, d_o, n, n, HD, NQ, NKV)
    ref = oracle.prefill_attention(q, k, v, 0, n, n, NQ, NKV, HD)
    assert_attn_close(d_o.download(np.float16, (n, Q_DIM)), ref)
    # seq_kv = 1: every query's output is V row 0 (tiled_attention.cu:57-63), exactly
    kv.launch_tiled_attention_kernel(d_q, d_k, d_v, d_o, n, 1, HD, NQ, NKV)
    got = d_o.download(np.float16, (n, Q_DIM))
    vrow = np.concatenate([v[0, (h * NKV // NQ) * HD:(h * NKV // NQ + 1) * HD] for h in range(NQ)])
    assert np.array_equal(bits(got), np.tile(bits(vrow), (n, 1)))
    kv.launch_tiled_attention_kernel(d_q, d_k, d_v, d_o, n, 0, HD, NQ, NKV)
    assert not d_o.download(np.uint16).any()


def test_prefill_attention_rejects_bad_arguments(gpu):
    say("prefill_attention argument checks")
    lib = atomflow_amd.lib()
    b = up(np.zeros((8, QKV), np.float16))
    assert lib.af_prefill_attention(b.ptr, QKV, b.ptr, b.ptr, b.ptr, Q_DIM, 0, 4, 4, 8, NQ, NKV,
                                    64, None) == atomflow_amd.AF_ERR_UNSUPPORTED
    assert lib.af_prefill_attention(b.ptr, QKV, b.ptr, b.ptr, b.ptr, Q_DIM, 0, 4, 9, 8, NQ, NKV,
                                    HD, None) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert lib.af_prefill_attention(b.ptr, QKV, b.ptr, b.ptr, b.ptr, Q_DIM, 0, 4, 0, 8, NQ, NKV,
                                    HD, None) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert lib.af_prefill_attention(b.ptr, 100, b.ptr, b.ptr, b.ptr, Q_DIM, 0, 4, 4, 8, NQ, NKV,
                                    HD, None) == atomflow_amd.AF_ERR_INVALID_ARG
    assert lib.af_prefill_attention(b.ptr, QKV, b.ptr, b.ptr, b.ptr, Q_DIM, 0, 0, 0, 8, NQ, NKV,
                                    HD, None) == atomflow_amd.AF_OK


# ---- chunked prefill then decode ------------------------------------------------
def test_chunked_prefill_then_decode_step(gpu):
    say("prefill 2 chunks (p0 0 / 300) via append+attention, then one decode step")
    max_seq, chunks = 1024, [(0, 300), (300, 213)]
    c, s, d_c, d_s = rope_tables(max_seq)
    k = np.zeros((max_seq, KV_DIM), np.float16)
    v = np.zeros((max_seq, KV_DIM), np.float16)
    d_k, d_v = up(k), up(v)
    for p0, n in chunks:
        qkv = randn_f16((n, QKV), 0xA70F60 + p0)
        d_qkv = up(qkv)
        kv.launch_prefill_rope_append(d_qkv, n, d_k, d_v, d_c, d_s, p0, max_seq, NQ, NKV, HD)
        d_o = up(np.zeros((n, Q_DIM), np.float16))
        kv.launch_prefill_attention(d_qkv, QKV, d_k, d_v, d_o, Q_DIM, p0, n, p0 + n, max_seq, NQ,
                                    NKV, HD)
        ref_qkv = oracle.prefill_rope_append(qkv, k, v, c, s, p0, NQ, NKV, HD)
        assert np.array_equal(bits(d_qkv.download(np.float16, qkv.shape)), bits(ref_qkv))
        ref = oracle.prefill_attention_f64(ref_qkv, k, v, p0, n, p0 + n, NQ, NKV, HD)
        assert_attn_close(d_o.download(np.float16, (n, Q_DIM)), ref, what=f"chunk p0={p0}")
    assert np.array_equal(bits(d_k.download(np.float16, k.shape)), bits(k))
    assert np.array_equal(bits(d_v.download(np.float16, v.shape)), bits(v))
    pos = 513
    qkv1 = randn_f16(QKV, 0xA70F62)
    d_qkv1, d_o1 = up(qkv1), up(np.zeros(Q_DIM, np.float16))
    kv.launch_rope_append(d_qkv1, d_k, d_v, d_c, d_s, pos, max_seq, NQ, NKV, HD)
    kv.launch_cached_attention(d_qkv1, d_k, d_v, d_o1, pos + 1, HD, NQ, NKV)
    r1 = oracle.rope_append(qkv1, k, v, c, s, pos, NQ, NKV, HD)
    assert_attn_close(d_o1.download(np.float16),
                      oracle.cached_attention_f64(r1[:Q_DIM], k, v, pos + 1, NQ, NKV, HD))


def test_paged_chunk_append_whole_blocks(gpu):
    say("paged pool: a 48-token chunk appended row by row into 3 whole blocks")
    bs, nblocks, n, p0 = 16, 12, 48, 32
    pool_bytes = 2 * nblocks * bs * KV_DIM * 2
    base = dev.DeviceBuffer(pool_bytes)
    base.fill_u32(0x47004700)  # 7.0 canaries
    pool = kv.make_pool(base, atomflow_amd.AF_KV_FP16, bs, 1, NKV, HD, nblocks)
    table = np.array([7, 2, 9, 4, 0], np.int32)  # positions 0..79 -> blocks
    pos = np.arange(p0, p0 + n, dtype=np.int32)
    slots = (table[pos // bs].astype(np.int64) * bs + pos % bs)
    c, s, d_c, d_s = rope_tables(128)
    qkv = randn_f16((n, QKV), 0xA70F63)
    d_qkv = up(qkv)
    kv.launch_paged_rope_append(d_qkv, n, pool, 0, up(slots), up(pos), d_c, d_s, 128, NQ)
    slab = base.download(np.float16).reshape(2, nblocks * bs, KV_DIM)
    ks = np.full((nblocks * bs, KV_DIM), np.float16(7.0))
    vs = ks.copy()
    ref = np.empty_like(qkv)
    for i in range(n):
        kk = np.zeros((128, KV_DIM), np.float16)
        vv = np.zeros((128, KV_DIM), np.float16)
        ref[i] = oracle.rope_append(qkv[i], kk, vv, c, s, p0 + i, NQ, NKV, HD)
        oracle.paged_write_f16(kk[p0 + i], vv[p0 + i], ks, vs, int(slots[i]), KV_DIM)
    assert np.array_equal(bits(d_qkv.download(np.float16, qkv.shape)), bits(ref))
    assert np.array_equal(bits(slab[0]), bits(ks))
    assert np.array_equal(bits(slab[1]), bits(vs))


# ---- paged pool: causal chunk attention through a block table -----------------
def _paged_pool(bs, nblocks, layers, seed):
    host = randn_f16((layers, 2, nblocks * bs, KV_DIM), seed)
    buf = up(host)
    pool = kv.make_pool(buf, atomflow_amd.AF_KV_FP16, bs, layers, NKV, HD, nblocks)
    return host, buf, pool


@pytest.mark.parametrize("bs,p0,n,kv_len", [(16, 0, 200, 200), (16, 300, 129, 429),
                                             (32, 1000, 300, 1300), (64, 0, 50, 37)])
def test_paged_prefill_attention_vs_oracle(gpu, bs, p0, n, kv_len):
    say(f"paged prefill bs={bs} p0={p0} n={n} kv_len={kv_len}")
    layers, layer = 2, 1
    max_blocks = (kv_len + bs - 1) // bs + 1
    nblocks = max_blocks + 7
    host, buf, pool = _paged_pool(bs, nblocks, layers, 0xA70F70 + bs + p0)
    table = rng(bs + n).permutation(nblocks)[:max_blocks].astype(np.int32)
    q = randn_f16((n, QKV), 0xA70F71 + n)
    d_o = up(np.full((n, Q_DIM), np.float16(3.0)))
    kv.launch_paged_prefill_attention(up(q), QKV, pool, layer, up(table), max_blocks, p0, n, kv_len,
                                      d_o, Q_DIM, NQ)
    got = d_o.download(np.float16, (n, Q_DIM))
    kc = oracle.paged_gather(host[layer, 0], table, kv_len, bs, KV_DIM)
    vc = oracle.paged_gather(host[layer, 1], table, kv_len, bs, KV_DIM)
    assert_attn_close(got, oracle.prefill_attention_f64(q, kc, vc, p0, n, kv_len, NQ, NKV, HD),
                      what="vs fp64")
    assert_attn_close(got, oracle.prefill_attention(q, kc, vc, p0, n, kv_len, NQ, NKV, HD,
                                                    threads=8), what="vs fp32 oracle")


def test_paged_prefill_rejects_bad_arguments(gpu):
    say("paged prefill argument checks")
    lib = atomflow_amd.lib()
    host, buf, pool = _paged_pool(16, 8, 1, 0xA70F72)
    b = up(np.zeros((8, QKV), np.float16))
    t = up(np.arange(4, dtype=np.int32))
    import ctypes
    args = lambda kv_len, max_blocks=4: (b.ptr, QKV, ctypes.byref(pool), 0, t.ptr, max_blocks, 0,
                                         4, kv_len, b.ptr, Q_DIM, NQ, None)
    assert lib.af_paged_prefill_attention(*args(65)) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert lib.af_paged_prefill_attention(*args(0)) == atomflow_amd.AF_ERR_OUT_OF_RANGE
    assert lib.af_paged_prefill_attention(*args(64)) == atomflow_amd.AF_OK
    fp8 = kv.make_pool(buf, atomflow_amd.AF_KV_FP8_E4M3, 16, 1, NKV, HD, 8)  # no scales
    assert lib.af_paged_prefill_attention(b.ptr, QKV, ctypes.byref(fp8), 0, t.ptr, 4, 0, 4, 10,
                                          b.ptr, Q_DIM, NQ, None) == atomflow_amd.AF_ERR_INVALID_ARG
    hd64 = kv.make_pool(buf, atomflow_amd.AF_KV_FP16, 16, 1, NKV, 64, 8)
    assert lib.af_paged_prefill_attention(b.ptr, QKV, ctypes.byref(hd64), 0, t.ptr, 4, 0, 4, 10,
                                          b.ptr, Q_DIM, NQ, None) == atomflow_amd.AF_ERR_UNSUPPORTED


def test_chunked_prefill_into_paged_pool_with_block_manager(gpu):
    say("BlockManager: two prefill chunks (300, 213 tokens) appended + attended through the pool")
    bs, nblocks = 16, 64
    bm = kv.BlockManager(nblocks, bs, 1, NKV, HD, atomflow_amd.AF_KV_FP16, allocate_pool=True)
    pool = bm.pool()
    max_seq = 1024
    c, s, d_c, d_s = rope_tables(max_seq)
    filler = [bm.seq_create() for _ in range(3)]  # interleave other sequences' blocks
    seq = bm.seq_create()
    k_ref = np.zeros((max_seq, KV_DIM), np.float16)
    v_ref = np.zeros((max_seq, KV_DIM), np.float16)
    for p0, n in [(0, 300), (300, 213)]:
        for f in filler:
            bm.seq_extend(f, 20)
        r = bm.seq_extend(seq, n)
        assert not isinstance(r, int), r
        pos = np.arange(p0, p0 + n, dtype=np.int32)
        slots = np.array([bm.seq_slot(seq, int(p)) for p in pos], np.int64)
        qkv = randn_f16((n, QKV), 0xA70F73 + p0)
        d_qkv = up(qkv)
        kv.launch_paged_rope_append(d_qkv, n, pool, 0, up(slots), up(pos), d_c, d_s, max_seq, NQ)
        tables, lens = bm.export_tables([seq], 64)
        assert lens[0] == p0 + n
        d_o = up(np.zeros((n, Q_DIM), np.float16))
        kv.launch_paged_prefill_attention(d_qkv, QKV, pool, 0, up(tables[0]), 64, p0, n, p0 + n,
                                          d_o, Q_DIM, NQ)
        ref_qkv = oracle.prefill_rope_append(qkv, k_ref, v_ref, c, s, p0, NQ, NKV, HD)
        assert np.array_equal(bits(d_qkv.download(np.float16, qkv.shape)), bits(ref_qkv))
        ref = oracle.prefill_attention_f64(ref_qkv, k_ref, v_ref, p0, n, p0 + n, NQ, NKV, HD)
        assert_attn_close(d_o.download(np.float16, (n, Q_DIM)), ref, what=f"chunk p0={p0}")
    bm.close()


@pytest.mark.parametrize("bs,p0,n,kv_len", [(32, 0, 150, 150), (16, 700, 200, 900)])
def test_paged_prefill_attention_fp8_pool(gpu, bs, p0, n, kv_len):
    """FP8-E4M3 pool with per-(layer, K/V, KV-head) fp32 scales: every row against the
    FP8 decode oracle over min(p0+i+1, kv_len) rows (ok_paged_attention_fp8), and
    sampled rows against a float64 numpy dequantise + softmax."""
    say(f"paged prefill fp8 bs={bs} p0={p0} n={n} kv_len={kv_len}")
    from inputs import ATOL_FP8, RTOL_FP8
    layers, layer = 2, 1
    max_blocks = (kv_len + bs - 1) // bs
    nblocks = max_blocks + 5
    r = rng(0xA70F75 + bs)
    host = r.integers(0, 256, (layers, 2, nblocks * bs, KV_DIM), dtype=np.uint8)
    host[(host & 0x7F) == 0x7F] = 0  # no NaN codes
    scales = r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32)
    buf = up(host)
    d_scales = up(scales)  # the pool descriptor holds its address: keep it alive
    pool = kv.make_pool(buf, atomflow_amd.AF_KV_FP8_E4M3, bs, layers, NKV, HD, nblocks, d_scales)
    table = r.permutation(nblocks)[:max_blocks].astype(np.int32)
    q = randn_f16((n, QKV), 0xA70F76 + n)
    d_o = up(np.zeros((n, Q_DIM), np.float16))
    kv.launch_paged_prefill_attention(up(q), QKV, pool, layer, up(table), max_blocks, p0, n,
                                      kv_len, d_o, Q_DIM, NQ)
    got = d_o.download(np.float16, (n, Q_DIM))
    ks, vs = scales[layer, 0], scales[layer, 1]
    for i in range(n):
        L = min(p0 + i + 1, kv_len)
        ref = oracle.paged_attention_fp8(q[i, :Q_DIM], host[layer, 0], host[layer, 1], ks, vs,
                                         table, L, bs, NQ, NKV, HD)
        assert_attn_close(got[i], ref, ATOL_FP8, RTOL_FP8, what=f"row {i}")
    lut = oracle.e4m3_decode_table().astype(np.float64)
    kc = oracle.paged_gather(host[layer, 0], table, kv_len, bs, KV_DIM)
    vc = oracle.paged_gather(host[layer, 1], table, kv_len, bs, KV_DIM)
    kf = lut[kc].reshape(kv_len, NKV, HD) * ks[None, :, None]
    vf = lut[vc].reshape(kv_len, NKV, HD) * vs[None, :, None]
    for i in sorted({0, n // 2, n - 1}):
        L = min(p0 + i + 1, kv_len)
        qi = q[i, :Q_DIM].astype(np.float64).reshape(NQ, HD)
        out = np.empty((NQ, HD))
        for h in range(NQ):
            g = h * NKV // NQ
            sc = kf[:L, g] @ qi[h] / np.sqrt(HD)
            p = np.exp(sc - sc.max())
            out[h] = p @ vf[:L, g] / p.sum()
        assert_attn_close(got[i], out.ravel(), ATOL_FP8, RTOL_FP8, what=f"row {i} vs float64")


@pytest.mark.parametrize("fp8", [False, True])
def test_paged_prefill_key_pieces_vs_oracle(gpu, fp8):
    """Paged fp16 / FP8 pool, a chunk late in the prompt (4 pieces per tile):
    every row against the paged decode oracle over min(p0+i+1, kv_len) rows."""
    from inputs import ATOL_FP8, RTOL_FP8
    bs, p0, n, kv_len = 16, 3000, 260, 3260
    say(f"paged prefill key pieces fp8={fp8} bs={bs} p0={p0} n={n}")
    layers, layer = 2, 1
    max_blocks = (kv_len + bs - 1) // bs
    nblocks = max_blocks + 5
    r = rng(0xA70F98 + fp8)
    table = r.permutation(nblocks)[:max_blocks].astype(np.int32)
    q = randn_f16((n, QKV), 0xA70F99)
    if fp8:
        host = r.integers(0, 256, (layers, 2, nblocks * bs, KV_DIM), dtype=np.uint8)
        host[(host & 0x7F) == 0x7F] = 0  # no NaN codes
        scales = r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32)
        buf, d_scales = up(host), up(scales)
        pool = kv.make_pool(buf, atomflow_amd.AF_KV_FP8_E4M3, bs, layers, NKV, HD, nblocks, d_scales)
    else:
        host, buf, pool = _paged_pool(bs, nblocks, layers, 0xA70F9A)
    ws = kv.PrefillWorkspace(p0, n, kv_len, NQ, 0)
    assert ws.nbytes > 64 * 1024  # the planner cuts this chunk
    d_o = up(np.zeros((n, Q_DIM), np.float16))
    kv.launch_paged_prefill_attention_ws(up(q), QKV, pool, layer, up(table), max_blocks, p0, n,
                                         kv_len, d_o, Q_DIM, NQ, ws)
    got = d_o.download(np.float16, (n, Q_DIM))
    for i in range(n):
        L = min(p0 + i + 1, kv_len)
        if fp8:
            ref = oracle.paged_attention_fp8(q[i, :Q_DIM], host[layer, 0], host[layer, 1],
                                             scales[layer, 0], scales[layer, 1], table, L, bs, NQ,
                                             NKV, HD)
            assert_attn_close(got[i], ref, ATOL_FP8, RTOL_FP8, what=f"row {i}")
        else:
            ref = oracle.paged_attention_f16(q[i, :Q_DIM], host[layer, 0], host[layer, 1], table,
                                             L, bs, NQ, NKV, HD)
            assert_attn_close(got[i], ref, what=f"row {i}")


@pytest.mark.parametrize("fp8", [False, True])
def test_batched_paged_prefill_equals_per_chunk_launches(gpu, fp8):
    """One launch over the chunks of several sequences == one launch per chunk,
    bit for bit (each workgroup's arithmetic does not depend on the grid)."""
    say(f"batched paged prefill fp8={fp8}")
    bs, layers, layer = 16, 1, 0
    chunks = [(0, 300, 300), (1000, 100, 1100), (0, 1, 1), (64, 200, 200), (500, 129, 629)]
    max_blocks = max((kvl + bs - 1) // bs for _, _, kvl in chunks)
    nblocks = sum((kvl + bs - 1) // bs for _, _, kvl in chunks) + 4
    r = rng(0xA70F77 + fp8)
    if fp8:
        host = r.integers(0, 256, (layers, 2, nblocks * bs, KV_DIM), dtype=np.uint8)
        host[(host & 0x7F) == 0x7F] = 0
        scales = up(r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32))
        buf = up(host)
        pool = kv.make_pool(buf, atomflow_amd.AF_KV_FP8_E4M3, bs, layers, NKV, HD, nblocks, scales)
    else:
        host, buf, pool = _paged_pool(bs, nblocks, layers, 0xA70F78)
    perm = r.permutation(nblocks).astype(np.int32)
    tables = np.zeros((len(chunks), max_blocks), np.int32)
    at = 0
    for c, (_, _, kvl) in enumerate(chunks):
        nb = (kvl + bs - 1) // bs
        tables[c, :nb] = perm[at:at + nb]
        at += nb
    rows = sum(n for _, n, _ in chunks)
    q = randn_f16((rows, QKV), 0xA70F79)
    desc, row0 = [], 0
    for p0, n, kvl in chunks:
        desc.append((p0, n, kvl, row0))
        row0 += n
    tmap = kv.prefill_tile_map(desc)
    d_q = up(q)
    d_o = up(np.zeros((rows, Q_DIM), np.float16))
    kv.launch_paged_prefill_attention_batched(d_q, QKV, pool, layer, up(tables), max_blocks,
                                              up(np.array(desc, np.int32)), up(tmap), len(tmap),
                                              d_o, Q_DIM, NQ)
    got = d_o.download(np.float16, (rows, Q_DIM))
    for c, (p0, n, kvl, r0) in enumerate(desc):
        one = up(np.zeros((n, Q_DIM), np.float16))
        kv.launch_paged_prefill_attention(d_q.ptr + r0 * QKV * 2, QKV, pool, layer,
                                          up(tables[c]), max_blocks, p0, n, kvl, one, Q_DIM, NQ)
        assert np.array_equal(bits(got[r0:r0 + n]), bits(one.download(np.float16, (n, Q_DIM)))), c
    if not fp8:
        for c, (p0, n, kvl, r0) in enumerate(desc):
            kc = oracle.paged_gather(host[layer, 0], tables[c], kvl, bs, KV_DIM)
            vc = oracle.paged_gather(host[layer, 1], tables[c], kvl, bs, KV_DIM)
            assert_attn_close(got[r0:r0 + n],
                              oracle.prefill_attention_f64(q[r0:r0 + n], kc, vc, p0, n, kvl, NQ,
                                                           NKV, HD), what=f"chunk {c}")


@pytest.mark.parametrize("fp8", [False, True])
def test_batched_paged_prefill_key_pieces(gpu, fp8):
    """The batched launch over a key-piece map: with key_pieces=1 it equals the
    plain batched launch bit for bit; cut (heavy tiles in up to 4 pieces) it
    matches the oracle per chunk, and a second launch on the same workspace gives
    the same bits."""
    from inputs import ATOL_FP8, RTOL_FP8
    say(f"batched paged prefill key pieces fp8={fp8}")
    bs, layers, layer = 16, 1, 0
    chunks = [(3000, 300, 3300), (0, 300, 300), (1000, 100, 1100), (0, 1, 1), (2000, 200, 2150)]
    max_blocks = max((kvl + bs - 1) // bs for _, _, kvl in chunks)
    nblocks = sum((kvl + bs - 1) // bs for _, _, kvl in chunks) + 4
    r = rng(0xA70F9C + fp8)
    if fp8:
        host = r.integers(0, 256, (layers, 2, nblocks * bs, KV_DIM), dtype=np.uint8)
        host[(host & 0x7F) == 0x7F] = 0
        scales = r.uniform(0.004, 0.02, (layers, 2, NKV)).astype(np.float32)
        d_scales, buf = up(scales), up(host)
        pool = kv.make_pool(buf, atomflow_amd.AF_KV_FP8_E4M3, bs, layers, NKV, HD, nblocks, d_scales)
    else:
        host, buf, pool = _paged_pool(bs, nblocks, layers, 0xA70F9D)
    perm = r.permutation(nblocks).astype(np.int32)
    tables = np.zeros((len(chunks), max_blocks), np.int32)
    at = 0
    for c, (_, _, kvl) in enumerate(chunks):
        nb = (kvl + bs - 1) // bs
        tables[c, :nb] = perm[at:at + nb]
        at += nb
    rows = sum(n for _, n, _ in chunks)
    q = randn_f16((rows, QKV), 0xA70F9E)
    desc, row0 = [], 0
    for p0, n, kvl in chunks:
        desc.append((p0, n, kvl, row0))
        row0 += n
    d_q, d_t, d_c = up(q), up(tables), up(np.array(desc, np.int32))

    def run(key_pieces, ws=None):
        pmap, groups, most, nbytes = kv.prefill_piece_map(desc, NQ, key_pieces)
        ws = ws or kv.RecordWorkspace(nbytes)
        d_o = up(np.zeros((rows, Q_DIM), np.float16))
        kv.launch_paged_prefill_attention_batched_ws(d_q, QKV, pool, layer, d_t, max_blocks, d_c,
                                                     up(pmap), len(pmap), groups, most, d_o, Q_DIM,
                                                     NQ, ws)
        return d_o.download(np.float16, (rows, Q_DIM)), pmap, most, ws

    tmap = kv.prefill_tile_map(desc)
    d_o = up(np.zeros((rows, Q_DIM), np.float16))
    kv.launch_paged_prefill_attention_batched(d_q, QKV, pool, layer, d_t, max_blocks, d_c, up(tmap),
                                              len(tmap), d_o, Q_DIM, NQ)
    plain = d_o.download(np.float16, (rows, Q_DIM))
    one, pmap1, most1, _ = run(1)
    assert most1 == 1 and len(pmap1) == len(tmap)
    assert np.array_equal(bits(one), bits(plain))
    got, pmap, most, ws = run(0)
    assert most > 1  # 10 tiles x 24 heads: the planner cuts the heavy tiles
    seen = {(int(c), int(t), int(pp) & 0xff) for c, t, pp, _ in pmap}
    assert len(seen) == len(pmap)  # every (chunk, tile, piece) once
    for c, t, pp, g in pmap:
        assert (int(pp) & 0xff) < (int(pp) >> 8) <= 4
    again, _, _, _ = run(0, ws)
    assert np.array_equal(bits(again), bits(got))
    for c, (p0, n, kvl, r0) in enumerate(desc):
        sample = range(n) if n <= 100 else sorted(set(rng(c).choice(n, 40, replace=False).tolist())
                                                   | {0, 127, 128, n - 1})
        for i in sample:
            L = min(p0 + i + 1, kvl)
            if fp8:
                ref = oracle.paged_attention_fp8(q[r0 + i, :Q_DIM], host[layer, 0], host[layer, 1],
                                                 scales[layer, 0], scales[layer, 1], tables[c], L,
                                                 bs, NQ, NKV, HD)
                assert_attn_close(got[r0 + i], ref, ATOL_FP8, RTOL_FP8, what=f"chunk {c} row {i}")
            else:
                ref = oracle.paged_attention_f16(q[r0 + i, :Q_DIM], host[layer, 0], host[layer, 1],
                                                 tables[c], L, bs, NQ, NKV, HD)
                assert_attn_close(got[r0 + i], ref, what=f"chunk {c} row {i}")
