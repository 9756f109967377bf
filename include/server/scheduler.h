#pragma once
// Continuous-batching scheduler over the paged BlockManager.
//
// Fills in ServerEngine::step, a stub in the reference whose comment lists the
// intended iteration (src/experimental/server_arch/server_engine.cu:55-68,
// server_engine.h:46-50): take pending requests from a queue, build a
// micro-batch, resolve each active sequence's PageTable for the batched
// attention, advance token counts and retire finished sequences. Host-side
// bookkeeping only: a StepPlan lists what the step's kernels must do (CoW copies,
// the decode batch's slots and positions, prefill chunks with one slot per
// token); the caller launches af_kv_copy_blocks, af_paged_rope_append,
// af_paged_attention and af_paged_prefill_attention for it. Not thread-safe.
//
// Rules (the reference leaves them open; fixed here):
//  * a request (id, prompt_len, max_new_tokens) is admitted FIFO; its sequence
//    holds prompt_eff tokens after prefill (prompt_len, or prompt_len +
//    generated after a preemption: recompute mode); the last prefill chunk
//    yields the first output token, each decode step one more, and the request
//    retires once it has generated max_new_tokens (its last token is never
//    appended to the cache);
//  * prefix cache (off unless max_cached_prefixes > 0): a request may name a
//    prompt prefix (prefix_key, prefix_len < prompt_len) whose tokens equal
//    every other request's with that key. Its prefill is chunked so that one
//    chunk ends exactly at prefix_len; when a request's prefill reaches it and
//    the key is not cached, the scheduler forks the sequence into the cache
//    (block tables and refcounts only; usable from the next step, after that
//    step's KV writes). A request admitted while its key is cached forks the
//    cached sequence instead of computing the prefix (the first append into a
//    partial shared tail block is a copy-on-write) and prefills the rest.
//    Cached sequences are evicted oldest-first when the cache is full and
//    before any preemption when the pool runs out; a hit makes an entry the
//    youngest. Each cache entry opens a share group: its creator and every
//    request admitted on it hold identical rows [0, prefix_len), so a decode
//    batch can attend them once per group (af_paged_attention_shared_prefix).
//    A preempted request leaves its group;
//  * step(): (0) prefixes cached last step become usable; (1) retire finished
//    entries; (2) decode every fully prefilled
//    entry (plan_decode, all or nothing); if the pool cannot hold the batch,
//    preempt the most recently admitted entry to the front of the queue and
//    plan again; (3) continue partial prefills in admission order with
//    min(remaining, prefill_chunk, budget) tokens, budget = max_step_tokens -
//    decode tokens; a prefill that does not fit preempts the youngest entry
//    when nothing decoded this step, else stops the step's prefill and
//    admission; (4) admit while running < max_running, budget remains and the
//    first chunk leaves at least `watermark_blocks` free blocks.
#include <cstdint>
#include <deque>
#include <vector>

#include "memory/block_manager.h"

namespace atomflow::server {

struct SchedulerConfig {
    int max_running = 256;       // entries admitted (prefilling or decoding)
    int max_step_tokens = 2048;  // decode + prefill tokens per step (>= max_running)
    int prefill_chunk = 512;     // prompt tokens of one request per step
    int watermark_blocks = 0;    // free blocks admission leaves untouched
    int max_cached_prefixes = 0; // prefix-cache entries (0: prefixes are ignored)
};

struct Request {
    int64_t id = 0;
    int prompt_len = 0;
    int max_new_tokens = 0;
    int64_t prefix_key = -1;  // >= 0 when prefix_len > 0
    int prefix_len = 0;       // shared prompt prefix, < prompt_len
};

struct PrefillChunk {
    int64_t request = 0;
    int seq = -1;
    int p0 = 0;         // first position of the chunk
    int n = 0;          // tokens; their slots are StepPlan::prefill_slots[offset .. offset+n)
    int offset = 0;
    bool last = false;  // completes the prompt (yields the first output token)
};

struct StepPlan {
    std::vector<int64_t> finished;   // retired at the start of this step
    std::vector<int64_t> preempted;  // sent back to the queue this step
    std::vector<CowCopy> copies;     // run before the step's appends
    std::vector<int64_t> decode_requests;
    std::vector<int> decode_seqs;
    std::vector<int64_t> decode_slots;
    std::vector<int32_t> decode_positions;  // the new token's position; attends position + 1 rows
    // Share group of each decode entry (-1: none) and the rows [0, share_rows) that
    // every member of the group holds with identical values.
    std::vector<int64_t> decode_share_groups;
    std::vector<int32_t> decode_share_rows;
    std::vector<PrefillChunk> prefill;
    std::vector<int64_t> prefill_slots;
    std::vector<int32_t> prefill_positions;
    std::vector<int64_t> prefix_hits;  // requests admitted onto a cached prefix
    std::vector<int64_t> cached;       // prefix keys cached by this step
    std::vector<int64_t> evicted;      // prefix keys evicted by this step
    int tokens() const { return int(decode_seqs.size() + prefill_slots.size()); }
    void clear();
};

class Scheduler {
public:
    Scheduler(BlockManager& bm, const SchedulerConfig& cfg);
    ~Scheduler();  // frees the cached prefix sequences
    Scheduler(const Scheduler&) = delete;
    Scheduler& operator=(const Scheduler&) = delete;
    // AF_OK, or AF_ERR_INVALID_ARG when the request could never fit the pool alone
    // (ceil((prompt_len + max_new_tokens) / block_size) > total blocks) or its
    // prefix fields are inconsistent.
    int add_request(const Request& r);
    // Frees every cached prefix sequence (blocks shared with running requests
    // stay theirs).
    void clear_prefix_cache();
    // Resizes the prefix cache (0 turns it off), evicting oldest entries first.
    void set_max_cached_prefixes(int n);
    int num_cached_prefixes() const { return int(cache_.size()); }
    // Plans one step into *plan (cleared first). AF_OK or an AF_* error. Within
    // one plan, copy sources and destinations are disjoint and every destination
    // is unique: a copy's source block is held (BlockManager::hold_copy_source)
    // until the plan is final, so no later allocation in the plan reuses it.
    int step(StepPlan* plan);
    int num_waiting() const { return int(waiting_.size()); }
    int num_running() const { return int(running_.size()); }
    bool idle() const { return waiting_.empty() && running_.empty(); }
    const SchedulerConfig& config() const { return cfg_; }

private:
    struct Entry {
        Request req;
        int seq = -1;
        int prompt_eff = 0;
        int prefilled = 0;
        int generated = 0;
        int64_t share_group = -1;  // the cache entry's group this sequence forked from
        int share_rows = 0;
    };
    struct CachedPrefix {
        int64_t key = -1;
        int seq = -1;
        int len = 0;
        bool ready = false;  // false during the step that cached it
        int64_t group = -1;  // shared by the creator and every request that forks it
    };
    int plan_step(StepPlan* plan);
    void add_copy(StepPlan* plan, const CowCopy& c);
    void preempt_youngest(StepPlan* plan);
    void emit_chunk(StepPlan* plan, Entry& e, int first, int n);
    bool caching(const Entry& e) const {
        return cfg_.max_cached_prefixes > 0 && e.req.prefix_len > 0;
    }
    int find_prefix(int64_t key, int len, bool ready_only) const;  // index in cache_ or -1
    bool evict_oldest(StepPlan* plan);
    void maybe_cache(StepPlan* plan, Entry& e);

    BlockManager& bm_;
    SchedulerConfig cfg_;
    std::deque<Entry> waiting_;
    std::vector<Entry> running_;       // admission order
    std::vector<CachedPrefix> cache_;  // oldest first
    int64_t next_group_ = 0;
};

}  // namespace atomflow::server
