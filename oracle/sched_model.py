"""Pure-Python model of the continuous-batching scheduler — TEST INFRASTRUCTURE.

The reference's ServerEngine::step is a stub whose comment lists the intended
iteration (src/experimental/server_arch/server_engine.cu:55-68): take pending
requests from a queue, build a micro-batch, look up each active sequence's
PageTable and run the batched attention, then advance token counts and retire
finished sequences. SURVEY.md names admission control on num_free_blocks()
(paged_kv_manager.h:115). The rules below fill that in; the C++ Scheduler
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
"""
from .block_model import POOL_EXHAUSTED


class _Entry:
    __slots__ = ("rid", "prompt_len", "max_new", "seq", "prompt_eff", "prefilled", "generated")

    def __init__(self, rid, prompt_len, max_new):
        self.rid, self.prompt_len, self.max_new = rid, prompt_len, max_new
        self.seq, self.prompt_eff, self.prefilled, self.generated = -1, prompt_len, 0, 0


class SchedModel:
    def __init__(self, bm, max_running, max_step_tokens, prefill_chunk, watermark=0):
        self.bm = bm
        self.max_running, self.max_step_tokens = max_running, max_step_tokens
        self.prefill_chunk, self.watermark = prefill_chunk, watermark
        self.waiting, self.running = [], []

    def add_request(self, rid, prompt_len, max_new):
        if prompt_len < 1 or max_new < 1:
            return False
        if -(-(prompt_len + max_new) // self.bm.bs) > self.bm.total:
            return False  # could never fit alone
        self.waiting.append(_Entry(rid, prompt_len, max_new))
        return True

    def _preempt_youngest(self, plan):
        v = self.running.pop()
        self.bm.seq_free(v.seq)
        v.seq, v.prompt_eff, v.prefilled = -1, v.prompt_len + v.generated, 0
        self.waiting.insert(0, v)
        plan["preempted"].append(v.rid)

    def _chunk(self, plan, e, first, n):
        slots = [self.bm.seq_slot(e.seq, first + i) for i in range(n)]
        last = e.prefilled + n == e.prompt_eff
        plan["prefill"].append((e.rid, e.seq, first, n, last, slots))
        e.prefilled += n
        if last:
            e.generated += 1

    def step(self):
        plan = {"finished": [], "preempted": [], "decode": [], "copies": [], "prefill": []}
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
                self._preempt_youngest(plan)
                continue
            slots, positions, copies = r
            for e, sl, p in zip(dec, slots, positions):
                plan["decode"].append((e.rid, e.seq, sl, p))
                e.generated += 1
            plan["copies"].extend(copies)
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
            r = self.bm.seq_extend(e.seq, n)
            if r == POOL_EXHAUSTED:
                if not plan["decode"] and i < len(self.running) - 1:
                    self._preempt_youngest(plan)
                    continue
                stalled = True
                break
            first, cow = r
            if cow[0] >= 0:
                plan["copies"].append(cow)
            self._chunk(plan, e, first, n)
            budget -= n
            i += 1
        while (not stalled and self.waiting and len(self.running) < self.max_running
               and budget > 0):
            e = self.waiting[0]
            n = min(e.prompt_eff, self.prefill_chunk, budget)
            need = -(-n // self.bm.bs)
            if self.bm.num_free_blocks() - need < self.watermark:
                break
            self.waiting.pop(0)
            e.seq = self.bm.seq_create()
            r = self.bm.seq_extend(e.seq, n)
            assert r != POOL_EXHAUSTED
            self.running.append(e)
            self._chunk(plan, e, r[0], n)
            budget -= n
        return plan

    def idle(self):
        return not self.waiting and not self.running
