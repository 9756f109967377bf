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
    prefill.clear();
    prefill_slots.clear();
    prefill_positions.clear();
}

Scheduler::Scheduler(BlockManager& bm, const SchedulerConfig& cfg) : bm_(bm), cfg_(cfg) {}

int Scheduler::add_request(const Request& r) {
    if (r.prompt_len < 1 || r.max_new_tokens < 1) return AF_ERR_INVALID_ARG;
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

int Scheduler::step(StepPlan* plan) {
    if (!plan) return AF_ERR_INVALID_ARG;
    plan->clear();
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
            preempt_youngest(plan);
            continue;
        }
        if (st) return st;
        for (size_t j = 0; j < dec.size(); ++j) {
            Entry& e = running_[size_t(dec[j])];
            plan->decode_requests.push_back(e.req.id);
            plan->decode_seqs.push_back(e.seq);
            plan->decode_slots.push_back(slots[j].slot);
            plan->decode_positions.push_back(slots[j].position);
            if (slots[j].cow.src >= 0) plan->copies.push_back(slots[j].cow);
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
        int first = 0;
        CowCopy cow;
        const int st = bm_.extend(e.seq, n, &first, &cow);
        if (st == AF_ERR_POOL_EXHAUSTED) {
            if (plan->decode_seqs.empty() && i + 1 < running_.size()) {
                preempt_youngest(plan);
                continue;
            }
            stalled = true;
            break;
        }
        if (st) return st;
        if (cow.src >= 0) plan->copies.push_back(cow);
        emit_chunk(plan, e, first, n);
        budget -= n;
        ++i;
    }
    // 4. admit
    while (!stalled && !waiting_.empty() && int(running_.size()) < cfg_.max_running &&
           budget > 0) {
        Entry& h = waiting_.front();
        int n = h.prompt_eff;
        if (n > cfg_.prefill_chunk) n = cfg_.prefill_chunk;
        if (n > budget) n = budget;
        const int need = (n + bm_.config().block_size - 1) / bm_.config().block_size;
        if (bm_.num_free_blocks() - need < cfg_.watermark_blocks) break;
        Entry e = h;
        waiting_.pop_front();
        e.seq = bm_.create_sequence();
        int first = 0;
        const int st = bm_.extend(e.seq, n, &first, nullptr);
        if (st) return st;  // cannot happen: the blocks were counted above
        running_.push_back(e);
        emit_chunk(plan, running_.back(), first, n);
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
