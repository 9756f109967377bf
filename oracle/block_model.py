"""Pure-Python model of the paged BlockManager contract — TEST INFRASTRUCTURE.

The reference declares the contract without defining it
(src/experimental/server_arch/paged_kv_manager.h:90-121, "EMPTY scaffolding"
at :11-12): a pool of ``total_blocks`` blocks handed out from a stack free list
(:119), ``allocate_block() -> id or -1`` (:105-107), ``free_block(id)`` (:111),
``num_free_blocks()`` (:115), PageTable = ordered block ids + last_block_fill
(:68-76), KVBlock.ref_count for copy-on-write (:51) and "fork a PageTable,
bump ref_counts" (:61). The choices this model fixes, and the C++ BlockManager
must reproduce op for op:

* fresh pool: ``allocate_block`` returns 0, 1, 2, ... (stack filled high to low);
  a freed id goes on top of the stack and is the next one handed out (LIFO);
* ``free_block`` drops one reference; the id returns to the stack at zero;
  freeing a free or out-of-range id is an error and changes nothing;
* sequence ids count up from 0 and are never reused;
* ``seq_free`` frees the table's blocks first to last;
* append: full (or missing) tail -> new block; partial tail shared by another
  table (ref > 1) -> copy-on-write: new block, copy ``fill`` rows, old tail
  loses one reference; otherwise write in place;
* a failed append / extend / batched plan changes nothing;
* a copy source can be held until the copies that read it are issued: a held
  block whose last reference is freed stays off the free list until
  ``release_copy_sources`` (holds drop in the order taken); holds are not
  references, so the copy-on-write test is unchanged.
"""

POOL_EXHAUSTED = -1
BAD_BLOCK = -5
BAD_SEQUENCE = -7
INVALID_ARG = -2


class BlockModel:
    def __init__(self, total_blocks, block_size):
        self.total = total_blocks
        self.bs = block_size
        self.ref = [0] * total_blocks
        self.free = list(range(total_blocks - 1, -1, -1))  # top of stack = end
        self.seqs = {}  # id -> [block_ids, fill]
        self.next_seq = 0
        self.held = [0] * total_blocks
        self.holds = []

    # ---- reference contract ---------------------------------------------
    def allocate_block(self):
        if not self.free:
            return POOL_EXHAUSTED
        b = self.free.pop()
        self.ref[b] = 1
        return b

    def free_block(self, b):
        if b < 0 or b >= self.total or self.ref[b] == 0:
            return BAD_BLOCK
        self.ref[b] -= 1
        if self.ref[b] == 0 and self.held[b] == 0:
            self.free.append(b)
        return 0

    def hold_copy_source(self, b):
        if b < 0 or b >= self.total or self.ref[b] == 0:
            return BAD_BLOCK
        self.held[b] += 1
        self.holds.append(b)
        return 0

    def release_copy_sources(self):
        for b in self.holds:
            self.held[b] -= 1
            if self.held[b] == 0 and self.ref[b] == 0:
                self.free.append(b)
        self.holds = []

    def num_free_blocks(self):
        return len(self.free)

    def ref_count(self, b):
        if b < 0 or b >= self.total:
            return BAD_BLOCK
        return self.ref[b]

    # ---- sequences ---------------------------------------------------------
    def seq_create(self):
        s = self.next_seq
        self.next_seq += 1
        self.seqs[s] = [[], 0]
        return s

    def seq_fork(self, src):
        if src not in self.seqs:
            return BAD_SEQUENCE
        ids, fill = self.seqs[src]
        for b in ids:
            self.ref[b] += 1
        s = self.next_seq
        self.next_seq += 1
        self.seqs[s] = [list(ids), fill]
        return s

    def seq_free(self, s):
        if s not in self.seqs:
            return BAD_SEQUENCE
        ids, _ = self.seqs.pop(s)
        for b in ids:
            self.free_block(b)
        return 0

    def seq_len(self, s):
        if s not in self.seqs:
            return BAD_SEQUENCE
        ids, fill = self.seqs[s]
        return 0 if not ids else (len(ids) - 1) * self.bs + fill

    def seq_table(self, s):
        ids, fill = self.seqs[s]
        return list(ids), fill

    def seq_slot(self, s, pos):
        if s not in self.seqs:
            return BAD_SEQUENCE
        if pos < 0 or pos >= self.seq_len(s):
            return -4
        ids, _ = self.seqs[s]
        return ids[pos // self.bs] * self.bs + pos % self.bs

    def _append_one(self, s, undo):
        """One token; returns (pos, slot, cow) or POOL_EXHAUSTED. Records undo ops."""
        ids, fill = self.seqs[s]
        cow = (-1, -1, 0)
        if not ids or fill == self.bs:
            b = self.allocate_block()
            if b < 0:
                return POOL_EXHAUSTED
            undo.append(("alloc", b))
            undo.append(("push", s, fill))
            ids.append(b)
            fill = 0
        elif self.ref[ids[-1]] > 1:
            b = self.allocate_block()
            if b < 0:
                return POOL_EXHAUSTED
            old = ids[-1]
            undo.append(("alloc", b))
            undo.append(("swap", s, old))
            self.ref[old] -= 1
            ids[-1] = b
            cow = (old, b, fill)
        pos = (len(ids) - 1) * self.bs + fill
        slot = ids[-1] * self.bs + fill
        undo.append(("fill", s, fill))
        self.seqs[s][1] = fill + 1
        return pos, slot, cow

    def _undo(self, undo):
        for op in reversed(undo):
            if op[0] == "alloc":
                b = op[1]
                self.ref[b] = 0
                self.free.append(b)
            elif op[0] == "push":
                s, fill = op[1], op[2]
                self.seqs[s][0].pop()
                self.seqs[s][1] = fill
            elif op[0] == "swap":
                s, old = op[1], op[2]
                self.ref[old] += 1
                self.seqs[s][0][-1] = old
            elif op[0] == "fill":
                self.seqs[op[1]][1] = op[2]

    def seq_append(self, s):
        if s not in self.seqs:
            return BAD_SEQUENCE
        undo = []
        r = self._append_one(s, undo)
        if r == POOL_EXHAUSTED:
            self._undo(undo)
        return r

    def seq_extend(self, s, n):
        """Returns (first_pos, cow) or an error code; at most one copy-on-write."""
        if s not in self.seqs:
            return BAD_SEQUENCE
        if n < 0:
            return INVALID_ARG
        first = self.seq_len(s)
        cow = (-1, -1, 0)
        undo = []
        for _ in range(n):
            r = self._append_one(s, undo)
            if r == POOL_EXHAUSTED:
                self._undo(undo)
                return POOL_EXHAUSTED
            if r[2][0] >= 0:
                cow = r[2]
        return first, cow

    def plan_decode(self, seqs):
        """One append per listed sequence, in order; all or nothing."""
        for s in seqs:
            if s not in self.seqs:
                return BAD_SEQUENCE
        undo = []
        slots, positions, copies = [], [], []
        for s in seqs:
            r = self._append_one(s, undo)
            if r == POOL_EXHAUSTED:
                self._undo(undo)
                return POOL_EXHAUSTED
            pos, slot, cow = r
            slots.append(slot)
            positions.append(pos)
            if cow[0] >= 0:
                copies.append(cow)
        return slots, positions, copies

    def export_tables(self, seqs, max_blocks):
        tables, lens = [], []
        for s in seqs:
            ids, _ = self.seqs[s]
            row = list(ids) + [0] * (max_blocks - len(ids))
            tables.append(row[:max_blocks])
            lens.append(self.seq_len(s))
        return tables, lens
