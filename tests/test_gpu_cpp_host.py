"""The C++ operator and memory API driven from a C++ host (tests/cpp/engine_step,
built with the library): one contiguous decode step the way the reference
engine issues it (launch_rope, launch_write_kv_cache, launch_cached_attention;
src/core/engine.cu:326-370) and the sandbox's paged step (BlockManager fork +
copy-on-write, launch_kv_copy_blocks, launch_paged_rope_append,
launch_paged_attention), plus launch_paged_attention_shared_prefix over the
forked pair. The program checks in itself that launch_rope_append equals the
three-launch sequence bit for bit and that the shared-prefix form agrees with
the paged attention of the forked pair; here its outputs are checked
against the oracle: append and copies bit-exact, attention within the
north-star tolerance of the float64 oracle."""
import os
import subprocess

import numpy as np
import pytest

import oracle
from inputs import HD, KV_DIM, NKV, NQ, Q_DIM, QKV, THETA, assert_attn_close

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "engine_step")
MAX_SEQ, POS = 1024, 300


def load(d, name, dtype, shape=None):
    a = np.fromfile(os.path.join(d, name + ".bin"), dtype)
    return a.reshape(shape) if shape is not None else a


def test_cpp_host_decode_steps(gpu, tmp_path):
    print("[case] C++ host: contiguous and paged decode step", flush=True)
    assert os.path.exists(EXE), "tests/cpp/engine_step is built by the library's Makefile"
    r = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
    d = str(tmp_path)

    # contiguous: the engine's three launches at position POS
    c, s = oracle.rope_table(MAX_SEQ, HD, THETA)
    qkv = load(d, "c_qkv_in", np.float16)
    k = load(d, "c_k_in", np.float16, (MAX_SEQ, KV_DIM)).copy()
    v = load(d, "c_v_in", np.float16, (MAX_SEQ, KV_DIM)).copy()
    roped = oracle.rope_append(qkv, k, v, c, s, POS, NQ, NKV, HD)
    assert np.array_equal(load(d, "c_qkv_out", np.uint16), roped.view(np.uint16))
    assert np.array_equal(load(d, "c_k_out", np.uint16, (MAX_SEQ, KV_DIM)), k.view(np.uint16))
    assert np.array_equal(load(d, "c_v_out", np.uint16, (MAX_SEQ, KV_DIM)), v.view(np.uint16))
    ref = oracle.cached_attention_f64(roped[:Q_DIM], k, v, POS + 1, NQ, NKV, HD)
    assert_attn_close(load(d, "c_attn", np.float16), ref, what="C++ host contiguous step")

    # paged: pool [K, V][blocks][16][kv_dim] for one layer
    bs, total, max_pos = 16, 64, 512
    pool = load(d, "p_pool_in", np.float16, (2, total * bs, KV_DIM)).copy()
    copies = load(d, "p_copies", np.int32, (-1, 3))
    assert len(copies) == 1
    for src, dst, rows in copies:
        pool[:, dst * bs:dst * bs + rows] = pool[:, src * bs:src * bs + rows]
    tables = load(d, "p_tables", np.int32, (3, -1))
    lens = load(d, "p_lens", np.int32)
    slots = load(d, "p_slots", np.int64)
    positions = load(d, "p_positions", np.int32)
    qkv = load(d, "p_qkv_in", np.float16, (3, QKV))
    c, s = oracle.rope_table(max_pos, HD, THETA)
    got_attn = load(d, "p_attn", np.float16, (3, Q_DIM))
    roped_rows = []
    for b in range(3):
        L, pos = int(lens[b]), int(positions[b])
        assert L == pos + 1
        rows = np.array([tables[b][t // bs] * bs + t % bs for t in range(L)])
        assert rows[pos] == slots[b]
        kseq = np.zeros((max_pos, KV_DIM), np.float16)
        vseq = np.zeros((max_pos, KV_DIM), np.float16)
        kseq[:pos] = pool[0, rows[:pos]]
        vseq[:pos] = pool[1, rows[:pos]]
        roped = oracle.rope_append(qkv[b], kseq, vseq, c, s, pos, NQ, NKV, HD)
        roped_rows.append(roped)
        ref = oracle.cached_attention_f64(roped[:Q_DIM], kseq, vseq, L, NQ, NKV, HD)
        assert_attn_close(got_attn[b], ref, what=f"C++ host paged step, sequence {b}")
        pool[0, slots[b]] = kseq[pos]
        pool[1, slots[b]] = vseq[pos]
    assert np.array_equal(load(d, "p_qkv_out", np.uint16, (3, QKV)),
                          np.stack(roped_rows).view(np.uint16))
    assert np.array_equal(load(d, "p_pool_out", np.uint16, (2, total * bs, KV_DIM)),
                          pool.view(np.uint16))


def test_cpp_host_pooled_layers(gpu, tmp_path):
    """Row a4: the engine's one-arena KV pool [L0_K | L0_V | L1_K | ...] of
    MAX_SEQ x KV_DIM fp16 slabs (engine.cu:187-215, model_state.h:56-64) carved
    by ArenaAllocator into Views; four layers' fused decode steps at pos 700.
    Rows [700, MAX_SEQ) of every slab hold NaN. The whole pool after the step
    must equal the oracle's (each layer's row 700 appended, nothing else
    touched, canaries included); each layer's attention must meet the bar."""
    print("[case] C++ host: pooled 4-layer decode step", flush=True)
    r = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
    d = str(tmp_path)
    NL, pos = 4, 700
    pool = load(d, "pl_pool_in", np.float16, (NL, 2, MAX_SEQ, KV_DIM)).copy()
    assert np.isnan(pool[:, :, pos:].astype(np.float32)).all()
    qkv = load(d, "pl_qkv_in", np.float16, (NL, QKV))
    c, s = oracle.rope_table(MAX_SEQ, HD, THETA)
    got_qkv = load(d, "pl_qkv_out", np.uint16, (NL, QKV))
    got_attn = load(d, "pl_attn", np.float16, (NL, Q_DIM))
    for layer in range(NL):
        k, v = pool[layer, 0], pool[layer, 1]  # views: rope_append writes row pos in place
        roped = oracle.rope_append(qkv[layer], k, v, c, s, pos, NQ, NKV, HD)
        assert np.array_equal(got_qkv[layer], roped.view(np.uint16)), layer
        ref = oracle.cached_attention_f64(roped[:Q_DIM], k, v, pos + 1, NQ, NKV, HD)
        assert_attn_close(got_attn[layer], ref, what=f"pooled layer {layer}")
    got_pool = load(d, "pl_pool_out", np.uint16, (NL, 2, MAX_SEQ, KV_DIM))
    assert np.array_equal(got_pool, pool.view(np.uint16))


def test_cpp_host_prefill_key_pieces(gpu, tmp_path):
    """launch_prefill_attention_ws from the C++ host: a 300-token chunk at p0 700
    (kv_len 1000) with its query tiles cut into key pieces (the workspace the
    library sized is larger than the counter region) against the float64
    oracle on every row, beside launch_prefill_attention on the same inputs."""
    print("[case] C++ host: prefill chunk with key pieces", flush=True)
    r = subprocess.run([EXE, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)
    d = str(tmp_path)
    p0, n, kv_len = 700, 300, 1000
    assert load(d, "f_ws_bytes", np.uint64)[0] > 64 * 1024  # the chunk was cut
    q = load(d, "f_q", np.float16, (n, Q_DIM))
    k = load(d, "f_k", np.float16, (MAX_SEQ, KV_DIM))
    v = load(d, "f_v", np.float16, (MAX_SEQ, KV_DIM))
    got = load(d, "f_attn", np.float16, (n, Q_DIM))
    plain = load(d, "f_attn_plain", np.float16, (n, Q_DIM))
    for i in range(n):
        L = min(p0 + i + 1, kv_len)
        ref = oracle.cached_attention_f64(q[i], k, v, L, NQ, NKV, HD)
        assert_attn_close(got[i], ref, what=f"pieces row {i}")
        assert_attn_close(plain[i], ref, what=f"plain row {i}")
