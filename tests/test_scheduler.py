"""Continuous-batching scheduler (af_sched_*): the C++ Scheduler against the
Python model of its rules (oracle/sched_model.py) decision for decision on
random request traces, plus the invariants the rules promise."""
import numpy as np
import pytest

import atomflow_amd
from atomflow_amd import kv
from oracle.block_model import BlockModel
from oracle.sched_model import SchedModel


def _same(a, b, step):
    for key in ("finished", "preempted", "decode", "copies", "prefix_hits", "cached", "evicted",
                "decode_shared"):
        assert [tuple(x) if isinstance(x, (list, tuple)) else x for x in a[key]] == \
               [tuple(x) if isinstance(x, (list, tuple)) else x for x in b[key]], (step, key)
    assert len(a["prefill"]) == len(b["prefill"]), step
    for x, y in zip(a["prefill"], b["prefill"]):
        assert tuple(x[:5]) == tuple(y[:5]) and list(x[5]) == list(y[5]), (step, x[:5], y[:5])


def run_trace(seed, total_blocks, bs, max_running, max_step_tokens, chunk, watermark, n_req,
              max_prompt, max_new, arrivals_per_step, n_prefixes=0, max_cached=0):
    """Random trace; with n_prefixes > 0 about half the requests share one of
    n_prefixes prompt prefixes (lengths drawn per key) and the prefix cache holds
    max_cached entries."""
    r = np.random.default_rng(seed)
    bm = kv.BlockManager(total_blocks, bs, 1, 8, 128)
    sched = kv.Scheduler(bm, max_running, max_step_tokens, chunk, watermark, max_cached)
    model = SchedModel(BlockModel(total_blocks, bs), max_running, max_step_tokens, chunk,
                       watermark, max_cached)
    plens = [int(r.integers(1, max_prompt)) for _ in range(n_prefixes)]
    reqs = []
    for i in range(n_req):
        pl, mn = int(r.integers(1, max_prompt + 1)), int(r.integers(1, max_new + 1))
        key, plen = -1, 0
        if n_prefixes and r.random() < 0.5:
            key = int(r.integers(0, n_prefixes))
            plen = plens[key]
            pl = plen + int(r.integers(1, max(2, max_prompt - plen + 1)))
        reqs.append((i, pl, mn, key, plen))
    generated = {q[0]: 0 for q in reqs}
    max_blocks = -(-max(q[1] + q[2] for q in reqs) // bs) + 1
    finished = []
    pending = list(reqs)
    steps = hits = 0
    while pending or not model.idle():
        for _ in range(int(r.integers(0, arrivals_per_step + 1))):
            if pending:
                rid, pl, mn, key, plen = pending.pop(0)
                assert sched.add_request(rid, pl, mn, key, plen) == \
                    model.add_request(rid, pl, mn, key, plen)
        a = sched.step()
        b = model.step()
        _same(a, b, steps)
        # a share group's members map the group's full shared blocks to the same blocks
        groups = {}
        for (rid, seq, slot, pos), (g, rows) in zip(a["decode"], a["decode_shared"]):
            if g >= 0:
                assert 0 < rows <= pos
                groups.setdefault(g, []).append((seq, rows))
        for g, members in groups.items():
            assert len({rows for _, rows in members}) == 1, g
            full = members[0][1] // bs
            tables, _ = bm.export_tables([seq for seq, _ in members], max_blocks)
            assert (tables[:, :full] == tables[0, :full]).all(), g
        # invariants
        # copies run together in one launch before the step's appends: a block is
        # never both a source and a destination, and destinations are unique
        srcs = [c[0] for c in a["copies"]]
        dsts = [c[1] for c in a["copies"]]
        assert not set(srcs) & set(dsts), (steps, a["copies"])
        assert len(set(dsts)) == len(dsts), (steps, a["copies"])
        # ... no row written this step is a row a copy reads
        written = {int(sl) for _, _, sl, _ in a["decode"]}
        for c in a["prefill"]:
            written |= {int(sl) for sl in c[5]}
        read = {src * bs + j for src, _, rows in a["copies"] for j in range(rows)}
        assert not written & read, (steps, a["copies"])
        # ... and the holds are gone once the plan is returned
        assert model.bm.holds == [] and bm.num_free_blocks() == model.bm.num_free_blocks()
        toks = len(a["decode"]) + sum(c[3] for c in a["prefill"])
        assert toks <= max_step_tokens
        assert a["running"] <= max_running
        for rid, seq, slot, pos in a["decode"]:
            generated[rid] += 1
        for rid, seq, p0, n, last, slots in a["prefill"]:
            assert len(slots) == n
            if last:
                generated[rid] += 1
        assert a["cache_entries"] == len(model.cache) <= max(max_cached, 0)
        hits += len(a["prefix_hits"])
        finished += a["finished"]
        steps += 1
        assert steps < 20000, "no progress"
    assert sorted(finished) == sorted(q[0] for q in reqs)
    for rid, pl, mn, _, _ in reqs:
        assert generated[rid] == mn, (rid, generated[rid], mn)
    sched.clear_prefix_cache()
    model.clear_prefix_cache()
    assert bm.num_free_blocks() == total_blocks
    sched.close()
    bm.close()
    return steps, hits


@pytest.mark.parametrize("seed", range(6))
def test_scheduler_matches_model_roomy_pool(seed):
    run_trace(seed, total_blocks=400, bs=16, max_running=16, max_step_tokens=256, chunk=64,
              watermark=4, n_req=40, max_prompt=300, max_new=40, arrivals_per_step=3)


@pytest.mark.parametrize("seed", range(6))
def test_scheduler_matches_model_tight_pool_with_preemption(seed):
    """A pool far smaller than the offered load: decode preemption (recompute),
    prefill stalls and the liveness rule all fire."""
    run_trace(100 + seed, total_blocks=40, bs=16, max_running=8, max_step_tokens=64, chunk=32,
              watermark=0, n_req=30, max_prompt=200, max_new=120, arrivals_per_step=4)


@pytest.mark.parametrize("seed", range(6))
def test_scheduler_prefix_cache_matches_model(seed):
    """Shared prompt prefixes: forks from the cache, CoW copies of partial shared
    tails, and eviction under pool pressure, decision for decision."""
    steps, hits = run_trace(200 + seed, total_blocks=120, bs=16, max_running=8,
                            max_step_tokens=128, chunk=48, watermark=2, n_req=40,
                            max_prompt=150, max_new=30, arrivals_per_step=3, n_prefixes=3,
                            max_cached=2)
    assert hits > 0


@pytest.mark.parametrize("seed", range(4))
def test_scheduler_prefix_cache_tight_pool(seed):
    run_trace(300 + seed, total_blocks=40, bs=16, max_running=8, max_step_tokens=64, chunk=32,
              watermark=0, n_req=30, max_prompt=200, max_new=60, arrivals_per_step=4,
              n_prefixes=2, max_cached=4)


# Seeds whose traces, without the hold, plan a block as both a copy source and a
# later copy's destination in one step (found by running the model with the hold
# disabled); the remaining seeds are ordinary traces of the same shape.
@pytest.mark.parametrize("seed", [7003, 7064, 7088, 7127, 7184, 7185, 7222, 7247, 7000, 7001])
def test_scheduler_copy_sources_survive_eviction(seed):
    """Tight pool, small blocks, partial shared prefix tails and a two-entry cache:
    evictions inside a step drop the last reference of blocks that earlier copies
    of the same plan still read. Without the copy-source hold the LIFO free list
    handed such a block out as a later copy's destination (e.g. copies
    (27, 17, 4) and (49, 27, 6) in one step)."""
    run_trace(seed, total_blocks=61, bs=8, max_running=7, max_step_tokens=97, chunk=24,
              watermark=2, n_req=30, max_prompt=120, max_new=40, arrivals_per_step=4,
              n_prefixes=2, max_cached=2)


def test_scheduler_prefix_hit_skips_the_prefix():
    """The second request with a cached prefix starts its prefill at prefix_len on
    a fork, and its first append into the shared partial block is a CoW copy."""
    bm = kv.BlockManager(64, 16, 1, 8, 128)
    s = kv.Scheduler(bm, 4, 256, 64, 0, max_cached_prefixes=2)
    assert s.add_request(0, 60, 2, prefix_key=7, prefix_len=40)
    p = s.step()  # request 0: chunk [0, 40) ends at the prefix and caches it
    assert [(c[0], c[2], c[3]) for c in p["prefill"]] == [(0, 0, 40)] and p["cached"] == [7]
    assert s.add_request(1, 50, 2, prefix_key=7, prefix_len=40)
    p = s.step()  # request 0 continues; request 1 forks the (now ready) prefix
    assert p["prefix_hits"] == [1]
    chunks = {c[0]: (c[2], c[3]) for c in p["prefill"]}
    assert chunks == {0: (40, 20), 1: (40, 10)}
    # both append into block 2 of the prefix (rows 32..39 filled, shared by the
    # cache entry, request 0 and request 1): each gets its own copy of 8 rows
    assert sorted(c[2] for c in p["copies"]) == [8, 8]
    p = s.step()  # both prompts are complete: they decode in share group 0 (40 rows)
    assert [d[0] for d in p["decode"]] == [0, 1]
    assert p["decode_shared"] == [(0, 40), (0, 40)]
    assert not s.add_request(2, 40, 2, prefix_key=7, prefix_len=40)  # prefix must be shorter
    assert not s.add_request(3, 50, 2, prefix_key=-1, prefix_len=10)
    while p["running"] or p["waiting"]:
        p = s.step()
    assert p["cache_entries"] == 1
    s.clear_prefix_cache()
    assert bm.num_free_blocks() == 64


def test_scheduler_preempts_in_tight_pool():
    bm = kv.BlockManager(12, 16, 1, 8, 128)
    s = kv.Scheduler(bm, 4, 64, 64, 0)
    for i in range(3):
        assert s.add_request(i, 60, 100)
    preempted = 0
    for _ in range(400):
        p = s.step()
        preempted += len(p["preempted"])
        if p["running"] == 0 and p["waiting"] == 0:
            break
    assert preempted > 0 and bm.num_free_blocks() == 12


def test_scheduler_rejects_requests_that_cannot_fit():
    bm = kv.BlockManager(10, 16, 1, 8, 128)
    s = kv.Scheduler(bm, 4, 64, 32)
    assert not s.add_request(1, 150, 20)   # 170 tokens > 160 rows
    assert s.add_request(2, 150, 10)
    assert not s.add_request(3, 0, 5)
    assert not s.add_request(4, 5, 0)
    lib = atomflow_amd.lib()
    import ctypes
    h = ctypes.c_void_p()
    assert lib.af_sched_create(bm.h, 8, 4, 32, 0, ctypes.byref(h)) == atomflow_amd.AF_ERR_INVALID_ARG


def test_scheduler_chunking_budget_and_fifo():
    """Prompts are split into prefill_chunk pieces, the step budget caps decode +
    prefill tokens, and requests are admitted in arrival order."""
    bm = kv.BlockManager(200, 16, 1, 8, 128)
    s = kv.Scheduler(bm, 4, 48, 32)
    for i, pl in enumerate([70, 10, 10]):
        s.add_request(i, pl, 3)
    p = s.step()  # 32 + 10 + the 6 tokens of budget left
    assert [(c[0], c[2], c[3]) for c in p["prefill"]] == [(0, 0, 32), (1, 0, 10), (2, 0, 6)]
    assert [c[4] for c in p["prefill"]] == [False, True, False]
    p = s.step()  # request 1 decodes at position 10; 0 and 2 continue in admission order
    assert [(d[0], d[3]) for d in p["decode"]] == [(1, 10)]
    assert [(c[0], c[2], c[3]) for c in p["prefill"]] == [(0, 32, 32), (2, 6, 4)]
    p = s.step()  # 1 and 2 decode; 0 gets its last 6 prompt tokens
    assert [(d[0], d[3]) for d in p["decode"]] == [(1, 11), (2, 10)]
    assert [(c[0], c[2], c[3], c[4]) for c in p["prefill"]] == [(0, 64, 6, True)]


def test_prefill_tile_map_orders_heaviest_first():
    chunks = [(0, 300, 300, 0), (1000, 100, 1100, 300), (0, 1, 1, 400), (64, 200, 200, 401)]
    m = kv.prefill_tile_map(chunks)
    # tiles of 128 queries: chunk 0 -> 3, chunk 1 -> 1, chunk 2 -> 1, chunk 3 -> 2 (kv_len caps)
    assert sorted(map(tuple, m)) == sorted([(0, 0), (0, 1), (0, 2), (1, 0), (2, 0), (3, 0), (3, 1)])
    work = {(0, 0): 128, (0, 1): 256, (0, 2): 300, (1, 0): 1100, (2, 0): 1, (3, 0): 192,
            (3, 1): 200}
    w = [work[tuple(x)] for x in m]
    assert w == sorted(w, reverse=True)
    assert kv.prefill_tile_map([]).shape == (0, 2)


def test_decode_share_segments():
    """Decode rows ordered for one attention launch per segment: entries with no
    group or a lone member first (plain attention), then each group together."""
    groups = [-1, 3, 5, 3, -1, 7, 3, 5]
    rows = [0, 40, 100, 40, 0, 9, 40, 100]
    order, segs = kv.decode_share_segments(groups, rows, min_saved_rows=0)
    assert list(order) == [0, 4, 5, 1, 3, 6, 2, 7]
    assert segs == [(0, 3, 0), (3, 3, 40), (6, 2, 100)]
    order, segs = kv.decode_share_segments(groups, rows, min_members=3, min_saved_rows=0)
    assert list(order) == [0, 2, 4, 5, 7, 1, 3, 6] and segs == [(0, 5, 0), (5, 3, 40)]
    order, segs = kv.decode_share_segments([2, 2], [16, 16], min_saved_rows=0)
    assert list(order) == [0, 1] and segs == [(0, 2, 16)]
    # the default threshold keeps small groups in the plain launch
    order, segs = kv.decode_share_segments([2, 2], [16, 16])
    assert list(order) == [0, 1] and segs == [(0, 2, 0)]
    order, segs = kv.decode_share_segments([4] * 64, [4096] * 64)
    assert segs == [(0, 64, 4096)]
    assert kv.SHARE_MIN_SAVED_ROWS == 24576
    assert kv.decode_share_segments([], [])[1] == []
    # only groups that save enough row reads: group 3 saves 2 x 40, group 5 1 x 100
    order, segs = kv.decode_share_segments(groups, rows, min_saved_rows=81)
    assert list(order) == [0, 1, 3, 4, 5, 6, 2, 7] and segs == [(0, 6, 0), (6, 2, 100)]
    with pytest.raises(ValueError):
        kv.decode_share_segments([1, 1], [16, 17])
