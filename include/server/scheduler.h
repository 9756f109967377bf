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
//  * step(): (1) retire finished entries; (2) decode every fully prefilled
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
};

struct Request {
    int64_t id = 0;
    int prompt_len = 0;
    int max_new_tokens = 0;
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
    std::vector<PrefillChunk> prefill;
    std::vector<int64_t> prefill_slots;
    std::vector<int32_t> prefill_positions;
    int tokens() const { return int(decode_seqs.size() + prefill_slots.size()); }
    void clear();
};

class Scheduler {
public:
    Scheduler(BlockManager& bm, const SchedulerConfig& cfg);
    // AF_OK, or AF_ERR_INVALID_ARG when the request could never fit the pool alone
    // (ceil((prompt_len + max_new_tokens) / block_size) > total blocks).
    int add_request(const Request& r);
    // Plans one step into *plan (cleared first). AF_OK or an AF_* error.
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
    };
    void preempt_youngest(StepPlan* plan);
    void emit_chunk(StepPlan* plan, Entry& e, int first, int n);

    BlockManager& bm_;
    SchedulerConfig cfg_;
    std::deque<Entry> waiting_;
    std::vector<Entry> running_;  // admission order
};

}  // namespace atomflow::server
