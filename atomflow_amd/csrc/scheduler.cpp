// scheduler.cpp — continuous-batching scheduler (include/server/scheduler.h)
// and its C ABI (af_sched_*, include/af_kv.h).
#include "server/scheduler.h"

#include <new>

namespace atomflow::server {

void StepPlan::clear() {
    finished.clear();
    preempted.clear();
    copies.clear();
    decode_requests.clear();
    decode_seqs.clear();
    decode_slots.clear();
    decode_positions.clear();
    decode_share_groups.clear();
    decode_share_rows.clear();
    prefill.clear();
    prefill_slots.clear();
    prefill_positions.clear();
    prefix_hits.clear();
    cached.clear();
    evicted.clear();
}

Scheduler::Scheduler(BlockManager& bm, const SchedulerConfig& cfg) : bm_(bm), cfg_(cfg) {}

Scheduler::~Scheduler() { clear_prefix_cache(); }

void Scheduler::clear_prefix_cache() {
    for (const CachedPrefix& c : cache_) (void)bm_.free_sequence(c.seq);
    cache_.clear();
}

void Scheduler::set_max_cached_prefixes(int n) {
    cfg_.max_cached_prefixes = n < 0 ? 0 : n;
    while (int(cache_.size()) > cfg_.max_cached_prefixes) {
        (void)bm_.free_sequence(cache_.front().seq);
        cache_.erase(cache_.begin());
    }
}

int Scheduler::find_prefix(int64_t key, int len, bool ready_only) const {
    for (int i = 0; i < int(cache_.size()); ++i) {
        const CachedPrefix& c = cache_[size_t(i)];
        if (c.key == key && c.len == len && (c.ready || !ready_only)) return i;
    }
    return -1;
}

bool Scheduler::evict_oldest(StepPlan* plan) {
    if (cache_.empty()) return false;
    (void)bm_.free_sequence(cache_.front().seq);
    plan->evicted.push_back(cache_.front().key);
    cache_.erase(cache_.begin());
    return true;
}

// After a chunk: a request whose prefill just reached its prefix caches it
// (a fork of its sequence, which holds exactly the prefix now).
void Scheduler::maybe_cache(StepPlan* plan, Entry& e) {
    if (!caching(e) || e.prefilled != e.req.prefix_len) return;
    if (find_prefix(e.req.prefix_key, e.req.prefix_len, false) >= 0) return;
    if (int(cache_.size()) >= cfg_.max_cached_prefixes) (void)evict_oldest(plan);
    CachedPrefix c;
    c.key = e.req.prefix_key;
    c.seq = bm_.fork_sequence(e.seq);
    c.len = e.req.prefix_len;
    c.group = next_group_++;
    e.share_group = c.group;
    e.share_rows = c.len;
    cache_.push_back(c);
    plan->cached.push_back(c.key);
}

int Scheduler::add_request(const Request& r) {
    if (r.prompt_len < 1 || r.max_new_tokens < 1) return AF_ERR_INVALID_ARG;
    if (r.prefix_len < 0 || r.prefix_len >= r.prompt_len || (r.prefix_len > 0 && r.prefix_key < 0))
        return AF_ERR_INVALID_ARG;
    const int64_t bs = bm_.config().block_size;
    const int64_t need = (int64_t(r.prompt_len) + r.max_new_tokens + bs - 1) / bs;
    if (need > bm_.config().total_blocks) return AF_ERR_INVALID_ARG;
    Entry e;
    e.req = r;
    e.prompt_eff = r.prompt_len;
    waiting_.push_back(e);
    return AF_OK;
}

void Scheduler::preempt_youngest(StepPlan* plan) {
    Entry v = running_.back();
    running_.pop_back();
    (void)bm_.free_sequence(v.seq);
    v.seq = -1;
    v.prompt_eff = v.req.prompt_len + v.generated;
    v.prefilled = 0;
    v.share_group = -1;
    v.share_rows = 0;
    plan->preempted.push_back(v.req.id);
    waiting_.push_front(v);
}

void Scheduler::emit_chunk(StepPlan* plan, Entry& e, int first, int n) {
    PrefillChunk c;
    c.request = e.req.id;
    c.seq = e.seq;
    c.p0 = first;
    c.n = n;
    c.offset = int(plan->prefill_slots.size());
    c.last = e.prefilled + n == e.prompt_eff;
    for (int i = 0; i < n; ++i) {
        plan->prefill_slots.push_back(bm_.slot_of(e.seq, first + i));
        plan->prefill_positions.push_back(first + i);
    }
    plan->prefill.push_back(c);
    e.prefilled += n;
    if (c.last) ++e.generated;
}

// A planned copy's source keeps its rows until the caller has issued the step's
// copies: evictions and preemptions later in the same plan may drop its last
// reference, and the LIFO free list would otherwise hand it out again at once,
// e.g. as the destination of another copy in the same batch of copies.
void Scheduler::add_copy(StepPlan* plan, const CowCopy& c) {
    (void)bm_.hold_copy_source(c.src);
    plan->copies.push_back(c);
}

int Scheduler::step(StepPlan* plan) {
    if (!plan) return AF_ERR_INVALID_ARG;
    const int st = plan_step(plan);
    bm_.release_copy_sources();
    return st;
}

int Scheduler::plan_step(StepPlan* plan) {
    plan->clear();
    // 0. prefixes cached last step are complete in the pool now
    for (CachedPrefix& c : cache_) c.ready = true;
    // 1. retire
    std::vector<Entry> keep;
    keep.reserve(running_.size());
    for (Entry& e : running_) {
        if (e.generated >= e.req.max_new_tokens) {
            (void)bm_.free_sequence(e.seq);
            plan->finished.push_back(e.req.id);
        } else {
            keep.push_back(e);
        }
    }
    running_.swap(keep);
    // 2. decode
    std::vector<int> dec;
    std::vector<AppendSlot> slots;
    for (;;) {
        dec.clear();
        for (int i = 0; i < int(running_.size()); ++i)
            if (running_[size_t(i)].prefilled == running_[size_t(i)].prompt_eff) dec.push_back(i);
        if (dec.empty()) break;
        std::vector<int> seqs(dec.size());
        for (size_t j = 0; j < dec.size(); ++j) seqs[j] = running_[size_t(dec[j])].seq;
        slots.assign(dec.size(), AppendSlot{});
        const int st = bm_.plan_decode(seqs.data(), int(seqs.size()), slots.data());
        if (st == AF_ERR_POOL_EXHAUSTED) {
            if (!evict_oldest(plan)) preempt_youngest(plan);
            continue;
        }
        if (st) return st;
        for (size_t j = 0; j < dec.size(); ++j) {
            Entry& e = running_[size_t(dec[j])];
            plan->decode_requests.push_back(e.req.id);
            plan->decode_seqs.push_back(e.seq);
            plan->decode_slots.push_back(slots[j].slot);
            plan->decode_positions.push_back(slots[j].position);
            plan->decode_share_groups.push_back(e.share_group);
            plan->decode_share_rows.push_back(e.share_rows);
            if (slots[j].cow.src >= 0) add_copy(plan, slots[j].cow);
            ++e.generated;
        }
        break;
    }
    int budget = cfg_.max_step_tokens - int(plan->decode_seqs.size());
    // 3. continue prefills
    bool stalled = false;
    for (size_t i = 0; i < running_.size() && budget > 0;) {
        Entry& e = running_[i];
        if (e.prefilled == e.prompt_eff) {
            ++i;
            continue;
        }
        int n = e.prompt_eff - e.prefilled;
        if (n > cfg_.prefill_chunk) n = cfg_.prefill_chunk;
        if (n > budget) n = budget;
        if (caching(e) && e.prefilled < e.req.prefix_len && n > e.req.prefix_len - e.prefilled)
            n = e.req.prefix_len - e.prefilled;  // a chunk ends at the prefix
        int first = 0;
        CowCopy cow;
        const int st = bm_.extend(e.seq, n, &first, &cow);
        if (st == AF_ERR_POOL_EXHAUSTED) {
            if (evict_oldest(plan)) continue;
            if (plan->decode_seqs.empty() && i + 1 < running_.size()) {
                preempt_youngest(plan);
                continue;
            }
            stalled = true;
            break;
        }
        if (st) return st;
        if (cow.src >= 0) add_copy(plan, cow);
        emit_chunk(plan, e, first, n);
        maybe_cache(plan, e);
        budget -= n;
        ++i;
    }
    // 4. admit
    while (!stalled && !waiting_.empty() && int(running_.size()) < cfg_.max_running &&
           budget > 0) {
        Entry& h = waiting_.front();
        const int bs = bm_.config().block_size;
        const int hit = caching(h) ? find_prefix(h.req.prefix_key, h.req.prefix_len, true) : -1;
        const int base = hit >= 0 ? h.req.prefix_len : 0;  // tokens taken from the cache
        int n = h.prompt_eff - base;
        if (n > cfg_.prefill_chunk) n = cfg_.prefill_chunk;
        if (n > budget) n = budget;
        if (hit < 0 && caching(h) && n > h.req.prefix_len) n = h.req.prefix_len;
        // New blocks: those the chunk touches, the shared partial tail included
        // (copy-on-write).
        const int need = (base + n + bs - 1) / bs - base / bs;
        if (bm_.num_free_blocks() - need < cfg_.watermark_blocks) break;
        Entry e = h;
        waiting_.pop_front();
        CowCopy cow;
        if (hit >= 0) {
            const CachedPrefix c = cache_[size_t(hit)];
            cache_.erase(cache_.begin() + hit);
            cache_.push_back(c);  // youngest
            e.seq = bm_.fork_sequence(c.seq);
            e.prefilled = base;
            e.share_group = c.group;
            e.share_rows = c.len;
            plan->prefix_hits.push_back(e.req.id);
        } else {
            e.seq = bm_.create_sequence();
        }
        int first = 0;
        const int st = bm_.extend(e.seq, n, &first, &cow);
        if (st) return st;  // cannot happen: the blocks were counted above
        if (cow.src >= 0) add_copy(plan, cow);
        running_.push_back(e);
        emit_chunk(plan, running_.back(), first, n);
        maybe_cache(plan, running_.back());
        budget -= n;
    }
    return AF_OK;
}

}  // namespace atomflow::server

// ============================================================================
// C ABI
// ============================================================================
using atomflow::server::Request;
using atomflow::server::Scheduler;
using atomflow::server::SchedulerConfig;
using atomflow::server::StepPlan;

struct af_block_manager;
namespace atomflow::server {
BlockManager* block_manager_of(af_block_manager* h);  // block_manager.cpp
}

struct af_scheduler {
    Scheduler sched;
    StepPlan plan;
    af_scheduler(atomflow::server::BlockManager& bm, const SchedulerConfig& c) : sched(bm, c) {}
};

extern "C" int af_sched_create(af_block_manager* bm, int max_running, int max_step_tokens,
                               int prefill_chunk, int watermark_blocks, af_scheduler** out) {
    if (!bm || !out || max_running < 1 || max_step_tokens < max_running || prefill_chunk < 1 ||
        watermark_blocks < 0)
        return AF_ERR_INVALID_ARG;
    SchedulerConfig c;
    c.max_running = max_running;
    c.max_step_tokens = max_step_tokens;
    c.prefill_chunk = prefill_chunk;
    c.watermark_blocks = watermark_blocks;
    af_scheduler* s = new (std::nothrow) af_scheduler(*atomflow::server::block_manager_of(bm), c);
    if (!s) return AF_ERR_INVALID_ARG;
    *out = s;
    return AF_OK;
}

extern "C" int af_sched_destroy(af_scheduler* s) {
    delete s;
    return AF_OK;
}

extern "C" int af_sched_add_request(af_scheduler* s, int64_t id, int prompt_len,
                                    int max_new_tokens) {
    if (!s) return AF_ERR_INVALID_ARG;
    Request r;
    r.id = id;
    r.prompt_len = prompt_len;
    r.max_new_tokens = max_new_tokens;
    return s->sched.add_request(r);
}

extern "C" int af_sched_add_request_prefix(af_scheduler* s, int64_t id, int prompt_len,
                                           int max_new_tokens, int64_t prefix_key,
                                           int prefix_len) {
    if (!s) return AF_ERR_INVALID_ARG;
    Request r;
    r.id = id;
    r.prompt_len = prompt_len;
    r.max_new_tokens = max_new_tokens;
    r.prefix_key = prefix_key;
    r.prefix_len = prefix_len;
    return s->sched.add_request(r);
}

extern "C" int af_sched_set_prefix_cache(af_scheduler* s, int max_entries) {
    if (!s || max_entries < 0) return AF_ERR_INVALID_ARG;
    s->sched.set_max_cached_prefixes(max_entries);
    return AF_OK;
}

extern "C" int af_sched_clear_prefix_cache(af_scheduler* s) {
    if (!s) return AF_ERR_INVALID_ARG;
    s->sched.clear_prefix_cache();
    return AF_OK;
}

extern "C" int af_sched_plan_prefix(const af_scheduler* s, int32_t* counts, int64_t* hits,
                                    int64_t* cached, int64_t* evicted) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    if (counts) {
        counts[0] = int32_t(p.prefix_hits.size());
        counts[1] = int32_t(p.cached.size());
        counts[2] = int32_t(p.evicted.size());
        counts[3] = s->sched.num_cached_prefixes();
    }
    for (size_t i = 0; hits && i < p.prefix_hits.size(); ++i) hits[i] = p.prefix_hits[i];
    for (size_t i = 0; cached && i < p.cached.size(); ++i) cached[i] = p.cached[i];
    for (size_t i = 0; evicted && i < p.evicted.size(); ++i) evicted[i] = p.evicted[i];
    return AF_OK;
}

extern "C" int af_sched_step(af_scheduler* s, int32_t* counts) {
    if (!s) return AF_ERR_INVALID_ARG;
    const int st = s->sched.step(&s->plan);
    if (st) return st;
    if (counts) {
        const StepPlan& p = s->plan;
        counts[0] = int32_t(p.decode_seqs.size());
        counts[1] = int32_t(p.prefill.size());
        counts[2] = int32_t(p.prefill_slots.size());
        counts[3] = int32_t(p.copies.size());
        counts[4] = int32_t(p.finished.size());
        counts[5] = int32_t(p.preempted.size());
        counts[6] = s->sched.num_running();
        counts[7] = s->sched.num_waiting();
    }
    return AF_OK;
}

extern "C" int af_sched_plan_decode(const af_scheduler* s, int64_t* requests, int32_t* seqs,
                                    int64_t* slots, int32_t* positions) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    for (size_t i = 0; i < p.decode_seqs.size(); ++i) {
        if (requests) requests[i] = p.decode_requests[i];
        if (seqs) seqs[i] = p.decode_seqs[i];
        if (slots) slots[i] = p.decode_slots[i];
        if (positions) positions[i] = p.decode_positions[i];
    }
    return AF_OK;
}

extern "C" int af_sched_plan_decode_shared(const af_scheduler* s, int64_t* groups,
                                           int32_t* rows) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    for (size_t i = 0; i < p.decode_share_groups.size(); ++i) {
        if (groups) groups[i] = p.decode_share_groups[i];
        if (rows) rows[i] = p.decode_share_rows[i];
    }
    return AF_OK;
}

extern "C" int af_sched_plan_prefill(const af_scheduler* s, int64_t* requests, int32_t* chunks,
                                     int64_t* slots, int32_t* positions) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    for (size_t i = 0; i < p.prefill.size(); ++i) {
        const auto& c = p.prefill[i];
        if (requests) requests[i] = c.request;
        if (chunks) {
            chunks[5 * i + 0] = c.seq;
            chunks[5 * i + 1] = c.p0;
            chunks[5 * i + 2] = c.n;
            chunks[5 * i + 3] = c.offset;
            chunks[5 * i + 4] = c.last ? 1 : 0;
        }
    }
    for (size_t i = 0; i < p.prefill_slots.size(); ++i) {
        if (slots) slots[i] = p.prefill_slots[i];
        if (positions) positions[i] = p.prefill_positions[i];
    }
    return AF_OK;
}

extern "C" int af_sched_plan_copies(const af_scheduler* s, int32_t* copies) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    for (size_t i = 0; copies && i < p.copies.size(); ++i) {
        copies[3 * i + 0] = p.copies[i].src;
        copies[3 * i + 1] = p.copies[i].dst;
        copies[3 * i + 2] = p.copies[i].rows;
    }
    return AF_OK;
}

extern "C" int af_sched_plan_events(const af_scheduler* s, int64_t* finished,
                                    int64_t* preempted) {
    if (!s) return AF_ERR_INVALID_ARG;
    const StepPlan& p = s->plan;
    for (size_t i = 0; finished && i < p.finished.size(); ++i) finished[i] = p.finished[i];
    for (size_t i = 0; preempted && i < p.preempted.size(); ++i) preempted[i] = p.preempted[i];
    return AF_OK;
}
