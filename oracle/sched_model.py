"""Pure-Python model of the continuous-batching scheduler — TEST INFRASTRUCTURE.

The reference's ServerEngine::step is a stub whose comment lists the intended
iteration (src/experimental/server_arch/server_engine.cu:55-68): take pending
requests from a queue, build a micro-batch, look up each active sequence's
PageTable and run the batched attention, then advance token counts and retire
finished sequences. Admission control follows the BlockManager's
num_free_blocks() (paged_kv_manager.h:115). The rules below fill that in; the C++ Scheduler
(atomflow_amd/csrc/scheduler.cpp) must reproduce them decision for decision.

A request is (id, prompt_len, max_new_tokens). Its sequence holds prompt_eff
tokens after prefill (prompt_eff = prompt_len, or prompt_len + generated after
a preemption: recompute mode); the last prefill chunk yields the first output
token, each decode step one more; a request retires once it has generated
max_new_tokens (its last token is never appended).

step():
 1. retire running entries with generated >= max_new_tokens (free their
    sequences), in admission order;
 2. decode: every running entry whose prefill is complete appends one token
    (BlockManager.plan_decode, all or nothing, admission order). If the pool
    cannot hold the batch, preempt the most recently admitted running entry
    (free its sequence, prompt_eff = prompt_len + generated, prefilled = 0,
    back to the FRONT of the waiting queue) and plan again;
 3. continue prefills in admission order: n = min(remaining, prefill_chunk,
    budget) tokens, budget = max_step_tokens - decode tokens. If the pool cannot
    hold them: when nothing decoded this step and a younger entry is running,
    preempt the youngest and retry; otherwise stop (and admit nothing);
 4. admit from the waiting queue (FIFO) while running < max_running and budget
    remains: the first chunk n = min(prompt_eff, prefill_chunk, budget) needs
    ceil(n / block_size) blocks and leaves at least `watermark` free blocks, or
    admission stops (the head of the queue is never skipped).

Prefix cache (max_cached_prefixes > 0; otherwise prefix fields are ignored). A
request may carry (prefix_key, prefix_len), 0 < prefix_len < prompt_len: its
first prefix_len prompt tokens equal those of every request with that key.
 0. at the start of step(), entries cached by the previous step become ready;
 * prefill chunks of such a request are cut to end exactly at prefix_len; when
   a chunk (step 3 or 4) brings prefilled to prefix_len and no entry (ready or
   not) has this (key, len), the cache evicts its oldest entry if full, then
   appends (key, fork(seq), len, not ready), oldest first;
 * admission of a request with a ready (key, len) entry: base = prefix_len,
   n = min(prompt_eff - base, prefill_chunk, budget), need = ceil((base + n) /
   bs) - floor(base / bs) (the partial shared tail is copied on write); the
   entry moves to the youngest end, seq = fork(entry's seq), prefilled = base,
   extend by n (its CoW copy joins the plan), and the request id is listed in
   prefix_hits. Without a hit, n is also capped at prefix_len;
 * share groups: each new cache entry takes the next group number (from 0),
   which its creator joins; a request admitted on the entry joins it too, with
   shared rows = prefix_len; preemption leaves the group (-1, 0). Each decode
   entry reports (group, rows) in decode_shared;
 * when the decode plan (step 2) or a prefill extend (step 3) finds the pool
   exhausted, the oldest cache entry is evicted (its sequence freed) and the
   same plan is retried; only with an empty cache do the preemption / stall
   rules apply.

Copies: every copy-on-write copy that joins the plan holds its source block
(BlockModel.hold_copy_source) until step() returns, so an eviction or
preemption later in the same step cannot put the source back on the free list
while the plan's copies still read it; within one plan, copy sources and
destinations are disjoint and destinations unique.
"""
from .block_model import POOL_EXHAUSTED


class _Entry:
    __slots__ = ("rid", "prompt_len", "max_new", "seq", "prompt_eff", "prefilled", "generated",
                 "pkey", "plen", "group", "srows")

    def __init__(self, rid, prompt_len, max_new, pkey=-1, plen=0):
        self.rid, self.prompt_len, self.max_new = rid, prompt_len, max_new
        self.seq, self.prompt_eff, self.prefilled, self.generated = -1, prompt_len, 0, 0
        self.pkey, self.plen = pkey, plen
        self.group, self.srows = -1, 0


class SchedModel:
    def __init__(self, bm, max_running, max_step_tokens, prefill_chunk, watermark=0,
                 max_cached_prefixes=0):
        self.bm = bm
        self.max_running, self.max_step_tokens = max_running, max_step_tokens
        self.prefill_chunk, self.watermark = prefill_chunk, watermark
        self.max_cached = max_cached_prefixes
        self.waiting, self.running = [], []
        self.cache = []  # [key, seq, len, ready, group], oldest first
        self.next_group = 0

    def _caching(self, e):
        return self.max_cached > 0 and e.plen > 0

    def _find(self, key, length, ready_only):
        for i, c in enumerate(self.cache):
            if c[0] == key and c[2] == length and (c[3] or not ready_only):
                return i
        return -1

    def _evict_oldest(self, plan):
        if not self.cache:
            return False
        key, seq = self.cache[0][:2]
        self.cache.pop(0)
        self.bm.seq_free(seq)
        plan["evicted"].append(key)
        return True

    def _maybe_cache(self, plan, e):
        if not self._caching(e) or e.prefilled != e.plen or self._find(e.pkey, e.plen, False) >= 0:
            return
        if len(self.cache) >= self.max_cached:
            self._evict_oldest(plan)
        self.cache.append([e.pkey, self.bm.seq_fork(e.seq), e.plen, False, self.next_group])
        e.group, e.srows = self.next_group, e.plen
        self.next_group += 1
        plan["cached"].append(e.pkey)

    def clear_prefix_cache(self):
        for c in self.cache:
            self.bm.seq_free(c[1])
        self.cache = []

    def add_request(self, rid, prompt_len, max_new, prefix_key=-1, prefix_len=0):
        if prompt_len < 1 or max_new < 1:
            return False
        if prefix_len < 0 or prefix_len >= prompt_len or (prefix_len > 0 and prefix_key < 0):
            return False
        if -(-(prompt_len + max_new) // self.bm.bs) > self.bm.total:
            return False  # could never fit alone
        self.waiting.append(_Entry(rid, prompt_len, max_new, prefix_key, prefix_len))
        return True

    def _preempt_youngest(self, plan):
        v = self.running.pop()
        self.bm.seq_free(v.seq)
        v.seq, v.prompt_eff, v.prefilled = -1, v.prompt_len + v.generated, 0
        v.group, v.srows = -1, 0
        self.waiting.insert(0, v)
        plan["preempted"].append(v.rid)

    def _chunk(self, plan, e, first, n):
        slots = [self.bm.seq_slot(e.seq, first + i) for i in range(n)]
        last = e.prefilled + n == e.prompt_eff
        plan["prefill"].append((e.rid, e.seq, first, n, last, slots))
        e.prefilled += n
        if last:
            e.generated += 1

    def _add_copy(self, plan, cow):
        self.bm.hold_copy_source(cow[0])
        plan["copies"].append(cow)

    def step(self):
        plan = self._plan_step()
        self.bm.release_copy_sources()
        return plan

    def _plan_step(self):
        plan = {"finished": [], "preempted": [], "decode": [], "copies": [], "prefill": [],
                "prefix_hits": [], "cached": [], "evicted": [], "decode_shared": []}
        for c in self.cache:
            c[3] = True
        keep = []
        for e in self.running:
            if e.generated >= e.max_new:
                self.bm.seq_free(e.seq)
                plan["finished"].append(e.rid)
            else:
                keep.append(e)
        self.running = keep
        while True:
            dec = [e for e in self.running if e.prefilled == e.prompt_eff]
            if not dec:
                break
            r = self.bm.plan_decode([e.seq for e in dec])
            if r == POOL_EXHAUSTED:
                if not self._evict_oldest(plan):
                    self._preempt_youngest(plan)
                continue
            slots, positions, copies = r
            for e, sl, p in zip(dec, slots, positions):
                plan["decode"].append((e.rid, e.seq, sl, p))
                plan["decode_shared"].append((e.group, e.srows))
                e.generated += 1
            for cow in copies:
                self._add_copy(plan, cow)
            break
        budget = self.max_step_tokens - len(plan["decode"])
        stalled = False
        i = 0
        while i < len(self.running) and budget > 0:
            e = self.running[i]
            if e.prefilled == e.prompt_eff:
                i += 1
                continue
            n = min(e.prompt_eff - e.prefilled, self.prefill_chunk, budget)
            if self._caching(e) and e.prefilled < e.plen:
                n = min(n, e.plen - e.prefilled)
            r = self.bm.seq_extend(e.seq, n)
            if r == POOL_EXHAUSTED:
                if self._evict_oldest(plan):
                    continue
                if not plan["decode"] and i < len(self.running) - 1:
                    self._preempt_youngest(plan)
                    continue
                stalled = True
                break
            first, cow = r
            if cow[0] >= 0:
                self._add_copy(plan, cow)
            self._chunk(plan, e, first, n)
            self._maybe_cache(plan, e)
            budget -= n
            i += 1
        while (not stalled and self.waiting and len(self.running) < self.max_running
               and budget > 0):
            e = self.waiting[0]
            bs = self.bm.bs
            hit = self._find(e.pkey, e.plen, True) if self._caching(e) else -1
            base = e.plen if hit >= 0 else 0
            n = min(e.prompt_eff - base, self.prefill_chunk, budget)
            if hit < 0 and self._caching(e):
                n = min(n, e.plen)
            need = -(-(base + n) // bs) - base // bs
            if self.bm.num_free_blocks() - need < self.watermark:
                break
            self.waiting.pop(0)
            if hit >= 0:
                c = self.cache.pop(hit)
                self.cache.append(c)
                e.seq = self.bm.seq_fork(c[1])
                e.prefilled = base
                e.group, e.srows = c[4], c[2]
                plan["prefix_hits"].append(e.rid)
            else:
                e.seq = self.bm.seq_create()
            r = self.bm.seq_extend(e.seq, n)
            assert r != POOL_EXHAUSTED
            first, cow = r
            if cow[0] >= 0:
                self._add_copy(plan, cow)
            self.running.append(e)
            self._chunk(plan, e, first, n)
            self._maybe_cache(plan, e)
            budget -= n
        return plan

    def idle(self):
        return not self.waiting and not self.running
