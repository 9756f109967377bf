"""Continuous batching end to end on the GPU: the Scheduler's plans drive the
paged kernels (af_paged_rope_append, af_paged_attention, af_paged_prefill_attention)
over a BlockManager-owned pool, and every attention row of every step is checked
against a contiguous per-request mirror built by the oracle (RoPE + append of the
same rows, float64 attention). Token data are a deterministic function of
(request, position), so a preempted request's recomputed prefill writes the same
rows again."""
import numpy as np
import pytest

import atomflow_amd
import oracle
from atomflow_amd import device as dev
from atomflow_amd import kv
from inputs import HD, KV_DIM, NKV, NQ, Q_DIM, QKV, THETA, assert_attn_close

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)


def up(a):
    return dev.DeviceBuffer.from_array(a)


def token_qkv(rid, pos):
    r = np.random.default_rng(0xA70F80 * 1009 + rid * 100003 + pos)
    return r.standard_normal(QKV).astype(np.float16)


def prefix_qkv(key, pos):
    r = np.random.default_rng(0xA70F90 * 1013 + key * 100019 + pos)
    return r.standard_normal(QKV).astype(np.float16)


@pytest.mark.parametrize("total_blocks,max_running,budget,chunk,max_new", [
    (96, 6, 160, 64, 25),    # roomy pool
    (24, 4, 96, 48, 150)])   # tight pool: decode growth forces preemption and recompute
def test_scheduler_drives_paged_kernels(gpu, total_blocks, max_running, budget, chunk, max_new):
    say(f"serving loop: {total_blocks} blocks, running<={max_running}, budget {budget}, chunk {chunk}")
    bs = 16
    max_pos = 1024
    bm = kv.BlockManager(total_blocks, bs, 1, NKV, HD, atomflow_amd.AF_KV_FP16, allocate_pool=True)
    pool = bm.pool()
    sched = kv.Scheduler(bm, max_running, budget, chunk, 1)
    c, s = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s)
    rr = np.random.default_rng(total_blocks)
    reqs = {i: (int(rr.integers(10, 170)), int(rr.integers(3, max_new))) for i in range(10)}
    for i, (pl, mn) in reqs.items():
        assert sched.add_request(i, pl, mn)
    mirror = {}  # rid -> (k [max_pos, KV_DIM], v)
    max_blocks = total_blocks
    ws = kv.AttentionWorkspace(max_running, NQ, NKV, HD, 0)
    steps, rows_checked, preempted = 0, 0, 0
    while True:
        p = sched.step()
        preempted += len(p["preempted"])
        if not p["decode"] and not p["prefill"]:
            assert p["running"] == 0 and p["waiting"] == 0
            break
        assert not p["copies"]  # no forks here: copy-on-write never fires
        # decode batch
        if p["decode"]:
            nd = len(p["decode"])
            qkv = np.stack([token_qkv(rid, pos) for rid, _, _, pos in p["decode"]])
            d_qkv = up(qkv)
            a = p["arrays"]
            kv.launch_paged_rope_append(d_qkv, nd, pool, 0, up(a["decode_slots"]),
                                        up(a["decode_positions"]), d_c, d_s, max_pos, NQ)
            tables, lens = bm.export_tables(a["decode_seqs"], max_blocks)
            assert np.array_equal(lens, a["decode_positions"] + 1)
            d_o = dev.DeviceBuffer(nd * Q_DIM * 2)
            kv.launch_paged_attention(d_qkv, QKV, pool, 0, up(tables), max_blocks, up(lens), nd,
                                      int(lens.max()), d_o, Q_DIM, NQ, ws)
            got = d_o.download(np.float16, (nd, Q_DIM))
            for b, (rid, seq, slot, pos) in enumerate(p["decode"]):
                k, v = mirror[rid]
                roped = oracle.rope_append(qkv[b], k, v, c, s, pos, NQ, NKV, HD)
                ref = oracle.cached_attention_f64(roped[:Q_DIM], k, v, pos + 1, NQ, NKV, HD)
                assert_attn_close(got[b], ref, what=f"step {steps} decode rid {rid} pos {pos}")
                rows_checked += 1
        # prefill chunks
        for rid, seq, p0, n, last, slots in p["prefill"]:
            if p0 == 0:
                mirror[rid] = (np.zeros((max_pos, KV_DIM), np.float16),
                               np.zeros((max_pos, KV_DIM), np.float16))
            k, v = mirror[rid]
            qkv = np.stack([token_qkv(rid, p0 + i) for i in range(n)])
            d_qkv = up(qkv)
            kv.launch_paged_rope_append(d_qkv, n, pool, 0, up(np.array(slots, np.int64)),
                                        up(np.arange(p0, p0 + n, dtype=np.int32)), d_c, d_s,
                                        max_pos, NQ)
            tables, lens = bm.export_tables([seq], max_blocks)
            assert lens[0] == p0 + n
            d_o = dev.DeviceBuffer(n * Q_DIM * 2)
            kv.launch_paged_prefill_attention(d_qkv, QKV, pool, 0, up(tables[0]), max_blocks, p0,
                                              n, p0 + n, d_o, Q_DIM, NQ)
            roped = oracle.prefill_rope_append(qkv, k, v, c, s, p0, NQ, NKV, HD)
            ref = oracle.prefill_attention_f64(roped, k, v, p0, n, p0 + n, NQ, NKV, HD)
            assert_attn_close(d_o.download(np.float16, (n, Q_DIM)), ref,
                              what=f"step {steps} prefill rid {rid} p0 {p0} n {n}")
            rows_checked += n
        steps += 1
        assert steps < 5000
    say(f"{steps} steps, {rows_checked} attention rows checked, {preempted} preemptions")
    if total_blocks < 32:
        assert preempted > 0
    assert bm.num_free_blocks() == total_blocks
    sched.close()
    bm.close()


def test_scheduler_prefix_cache_drives_paged_kernels(gpu):
    """Requests sharing prompt prefixes: the scheduler forks cached prefixes, the
    plan's copy-on-write copies run on the device (af_kv_copy_blocks) before the
    step's appends, and every attention row still matches the oracle over each
    request's own logical sequence (shared prefix rows + its own rows). Each decode
    batch is also attended grouped by the plan's share groups, every group through
    af_paged_attention_shared_prefix with its first member's table as the prefix
    table, to the same tolerance."""
    say("serving loop with a prefix cache: 40 blocks, 2 prefix keys, cache of 2")
    bs, total_blocks, max_pos = 16, 40, 512
    bm = kv.BlockManager(total_blocks, bs, 1, NKV, HD, atomflow_amd.AF_KV_FP16,
                         allocate_pool=True)
    pool = bm.pool()
    sched = kv.Scheduler(bm, 6, 96, 40, 0, max_cached_prefixes=2)
    c, s_ = oracle.rope_table(max_pos, HD, THETA)
    d_c, d_s = up(c), up(s_)
    rr = np.random.default_rng(5)
    plens = {0: 45, 1: 32}  # a partial and a block-aligned prefix
    reqs = {}
    for i in range(14):
        key = int(rr.integers(-1, 2))
        plen = plens.get(key, 0)
        reqs[i] = (plen + int(rr.integers(3, 60)), int(rr.integers(2, 40)), key, plen)
        assert sched.add_request(i, reqs[i][0], reqs[i][1], key if plen else -1, plen)

    def tok(rid, pos):
        _, _, key, plen = reqs[rid]
        return prefix_qkv(key, pos) if pos < plen else token_qkv(rid, pos)

    prefix_mirror = {}
    for key, plen in plens.items():
        k = np.zeros((max_pos, KV_DIM), np.float16)
        v = np.zeros((max_pos, KV_DIM), np.float16)
        oracle.prefill_rope_append(np.stack([prefix_qkv(key, p) for p in range(plen)]), k, v, c,
                                   s_, 0, NQ, NKV, HD)
        prefix_mirror[key] = (k, v)
    mirror = {}
    ws = kv.AttentionWorkspace(6, NQ, NKV, HD, 0)
    steps = rows = hits = copies = grouped = 0
    while True:
        p = sched.step()
        if not p["decode"] and not p["prefill"]:
            assert p["running"] == 0 and p["waiting"] == 0
            break
        hits += len(p["prefix_hits"])
        if p["copies"]:
            cp = np.ascontiguousarray(p["copies"], np.int32)
            kv.kv_copy_blocks(pool, up(cp), up(np.array([len(cp)], np.int32)), len(cp))
            copies += len(cp)
        if p["decode"]:
            nd = len(p["decode"])
            qkv = np.stack([tok(rid, pos) for rid, _, _, pos in p["decode"]])
            d_qkv = up(qkv)
            a = p["arrays"]
            kv.launch_paged_rope_append(d_qkv, nd, pool, 0, up(a["decode_slots"]),
                                        up(a["decode_positions"]), d_c, d_s, max_pos, NQ)
            tables, lens = bm.export_tables(a["decode_seqs"], total_blocks)
            d_o = dev.DeviceBuffer(nd * Q_DIM * 2)
            kv.launch_paged_attention(d_qkv, QKV, pool, 0, up(tables), total_blocks, up(lens), nd,
                                      int(lens.max()), d_o, Q_DIM, NQ, ws)
            got = d_o.download(np.float16, (nd, Q_DIM))
            # the same batch grouped by the plan's share groups: each group's prefix
            # through the shared-prefix entry (lone members too on odd steps)
            order, segs = kv.decode_share_segments(a["decode_share_groups"],
                                                   a["decode_share_rows"], 1 + steps % 2,
                                                   min_saved_rows=0)
            q_perm = up(d_qkv.download(np.float16, (nd, QKV))[order])
            t_perm, l_perm = up(tables[order]), up(lens[order])
            d_g = dev.DeviceBuffer(nd * Q_DIM * 2)
            for s0, sn, prefix in segs:
                args = (t_perm.ptr + s0 * total_blocks * 4, total_blocks, l_perm.ptr + s0 * 4, sn,
                        int(lens[order][s0:s0 + sn].max()), d_g.ptr + s0 * Q_DIM * 2, Q_DIM, NQ,
                        ws)
                if prefix:
                    kv.launch_paged_attention_shared_prefix(q_perm.ptr + s0 * QKV * 2, QKV, pool,
                                                            0, args[0], prefix, *args)
                    grouped += sn
                else:
                    kv.launch_paged_attention(q_perm.ptr + s0 * QKV * 2, QKV, pool, 0, *args)
            got_g = np.empty_like(got)
            got_g[order] = d_g.download(np.float16, (nd, Q_DIM))
            for b, (rid, seq, slot, pos) in enumerate(p["decode"]):
                k, v = mirror[rid]
                roped = oracle.rope_append(qkv[b], k, v, c, s_, pos, NQ, NKV, HD)
                ref = oracle.cached_attention_f64(roped[:Q_DIM], k, v, pos + 1, NQ, NKV, HD)
                assert_attn_close(got[b], ref, what=f"step {steps} decode rid {rid} pos {pos}")
                assert_attn_close(got_g[b], ref,
                                  what=f"step {steps} grouped decode rid {rid} pos {pos}")
                rows += 1
        for rid, seq, p0, n, last, slots in p["prefill"]:
            if rid in p["prefix_hits"]:
                pk, pv = prefix_mirror[reqs[rid][2]]
                mirror[rid] = (pk.copy(), pv.copy())
                assert p0 == reqs[rid][3]
            elif p0 == 0:
                mirror[rid] = (np.zeros((max_pos, KV_DIM), np.float16),
                               np.zeros((max_pos, KV_DIM), np.float16))
            k, v = mirror[rid]
            qkv = np.stack([tok(rid, p0 + i) for i in range(n)])
            d_qkv = up(qkv)
            kv.launch_paged_rope_append(d_qkv, n, pool, 0, up(np.array(slots, np.int64)),
                                        up(np.arange(p0, p0 + n, dtype=np.int32)), d_c, d_s,
                                        max_pos, NQ)
            tables, lens = bm.export_tables([seq], total_blocks)
            assert lens[0] == p0 + n
            d_o = dev.DeviceBuffer(n * Q_DIM * 2)
            kv.launch_paged_prefill_attention(d_qkv, QKV, pool, 0, up(tables[0]), total_blocks,
                                              p0, n, p0 + n, d_o, Q_DIM, NQ)
            roped = oracle.prefill_rope_append(qkv, k, v, c, s_, p0, NQ, NKV, HD)
            ref = oracle.prefill_attention_f64(roped, k, v, p0, n, p0 + n, NQ, NKV, HD)
            assert_attn_close(d_o.download(np.float16, (n, Q_DIM)), ref,
                              what=f"step {steps} prefill rid {rid} p0 {p0} n {n}")
            rows += n
        steps += 1
        assert steps < 5000
    say(f"{steps} steps, {rows} attention rows, {hits} prefix hits, {copies} CoW copies, "
        f"{grouped} decode rows attended through a shared prefix")
    assert hits > 0 and copies > 0 and grouped > 0
    sched.clear_prefix_cache()
    assert bm.num_free_blocks() == total_blocks
    sched.close()
    bm.close()
