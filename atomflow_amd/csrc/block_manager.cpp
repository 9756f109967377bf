// block_manager.cpp — host BlockManager and its af_bm_* C ABI.
#include "memory/block_manager.h"

#include <hip/hip_runtime.h>

#include <new>
#include <string>

namespace atomflow::server {

BlockManager::~BlockManager() {
    if (owns_pool_ && pool_) (void)hipFree(pool_);
}

void BlockManager::initialize(int total_blocks, int kv_dim, int n_layers) {
    PoolConfig c;
    c.total_blocks = total_blocks;
    c.block_size = BLOCK_SIZE;
    c.n_layers = n_layers;
    c.head_dim = 128;
    c.n_kv_heads = kv_dim / 128;
    c.dtype = AF_KV_FP16;
    if (kv_dim <= 0 || kv_dim % 128) throw std::invalid_argument("BlockManager: kv_dim % 128 != 0");
    initialize(c, true);
}

void BlockManager::initialize(const PoolConfig& cfg, bool allocate_pool, void* pool,
                              const float* scales) {
    if (cfg.total_blocks <= 0 || cfg.block_size <= 0 || (cfg.block_size & (cfg.block_size - 1)) ||
        cfg.n_layers <= 0 || cfg.n_kv_heads <= 0 || cfg.head_dim <= 0 ||
        (cfg.dtype != AF_KV_FP16 && cfg.dtype != AF_KV_FP8_E4M3))
        throw std::invalid_argument("BlockManager: bad pool configuration");
    if (owns_pool_ && pool_) (void)hipFree(pool_);
    pool_ = nullptr;
    owns_pool_ = false;
    cfg_ = cfg;
    ref_.assign(size_t(cfg.total_blocks), 0);
    held_.assign(size_t(cfg.total_blocks), 0);
    holds_.clear();
    free_list_.resize(size_t(cfg.total_blocks));
    for (int i = 0; i < cfg.total_blocks; ++i) free_list_[size_t(i)] = cfg.total_blocks - 1 - i;
    tables_.clear();
    live_.clear();
    scales_ = scales;
    if (allocate_pool) {
        af_kv_pool d = pool_desc();
        const size_t bytes = af_kv_pool_bytes(&d);
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess)
            throw std::runtime_error("BlockManager: pool allocation of " + std::to_string(bytes) +
                                     " bytes failed");
        pool_ = p;
        owns_pool_ = true;
    } else {
        pool_ = pool;
    }
}

void BlockManager::attach_pool(void* pool, const float* scales) {
    if (owns_pool_ && pool_) (void)hipFree(pool_);
    owns_pool_ = false;
    pool_ = pool;
    scales_ = scales;
}

int BlockManager::pop_free() {
    if (free_list_.empty()) return AF_ERR_POOL_EXHAUSTED;
    const int b = free_list_.back();
    free_list_.pop_back();
    ref_[size_t(b)] = 1;
    return b;
}

int BlockManager::allocate_block() { return pop_free(); }

int BlockManager::try_free_block(int block_id) {
    if (block_id < 0 || block_id >= cfg_.total_blocks || ref_[size_t(block_id)] == 0)
        return AF_ERR_BAD_BLOCK;
    if (--ref_[size_t(block_id)] == 0 && held_[size_t(block_id)] == 0)
        free_list_.push_back(block_id);
    return AF_OK;
}

int BlockManager::hold_copy_source(int block_id) {
    if (block_id < 0 || block_id >= cfg_.total_blocks || ref_[size_t(block_id)] == 0)
        return AF_ERR_BAD_BLOCK;
    ++held_[size_t(block_id)];
    holds_.push_back(block_id);
    return AF_OK;
}

void BlockManager::release_copy_sources() {
    for (int b : holds_)
        if (--held_[size_t(b)] == 0 && ref_[size_t(b)] == 0) free_list_.push_back(b);
    holds_.clear();
}

void BlockManager::free_block(int block_id) {
    if (try_free_block(block_id) != AF_OK)
        throw std::invalid_argument("BlockManager::free_block: block " + std::to_string(block_id) +
                                    " is not allocated");
}

int BlockManager::ref_count(int block_id) const {
    if (block_id < 0 || block_id >= cfg_.total_blocks) return AF_ERR_BAD_BLOCK;
    return ref_[size_t(block_id)];
}

af_kv_pool BlockManager::pool_desc() const {
    af_kv_pool d{};
    d.base = pool_;
    d.scales = scales_;
    d.dtype = cfg_.dtype;
    d.block_size = cfg_.block_size;
    d.n_layers = cfg_.n_layers;
    d.n_kv_heads = cfg_.n_kv_heads;
    d.head_dim = cfg_.head_dim;
    d.total_blocks = cfg_.total_blocks;
    return d;
}

KVBlock BlockManager::block(int block_id, int layer) const {
    KVBlock kb;
    if (block_id < 0 || block_id >= cfg_.total_blocks || layer < 0 || layer >= cfg_.n_layers)
        return kb;
    kb.block_id = block_id;
    kb.ref_count = ref_[size_t(block_id)];
    if (pool_) {
        const size_t esz = cfg_.dtype == AF_KV_FP8_E4M3 ? 1 : 2;
        const size_t block_bytes = size_t(cfg_.block_size) * cfg_.n_kv_heads * cfg_.head_dim * esz;
        const size_t slab = block_bytes * size_t(cfg_.total_blocks);
        uint8_t* base = static_cast<uint8_t*>(pool_);
        kb.k_data = base + size_t(2 * layer) * slab + size_t(block_id) * block_bytes;
        kb.v_data = base + size_t(2 * layer + 1) * slab + size_t(block_id) * block_bytes;
    }
    return kb;
}

int BlockManager::create_sequence() {
    tables_.emplace_back();
    live_.push_back(1);
    return int(tables_.size()) - 1;
}

bool BlockManager::has_sequence(int seq) const {
    return seq >= 0 && seq < int(tables_.size()) && live_[size_t(seq)];
}

int BlockManager::fork_sequence(int src) {
    if (!has_sequence(src)) return AF_ERR_BAD_SEQUENCE;
    PageTable copy = tables_[size_t(src)];
    for (int b : copy.block_ids) ++ref_[size_t(b)];
    tables_.push_back(std::move(copy));
    live_.push_back(1);
    return int(tables_.size()) - 1;
}

int BlockManager::free_sequence(int seq) {
    if (!has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    PageTable& t = tables_[size_t(seq)];
    for (int b : t.block_ids) (void)try_free_block(b);
    t.block_ids.clear();
    t.block_ids.shrink_to_fit();
    t.last_block_fill = 0;
    live_[size_t(seq)] = 0;
    return AF_OK;
}

const PageTable& BlockManager::table(int seq) const {
    if (!has_sequence(seq)) throw std::out_of_range("BlockManager: unknown sequence");
    return tables_[size_t(seq)];
}

int BlockManager::seq_len(int seq) const {
    if (!has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    const PageTable& t = tables_[size_t(seq)];
    if (t.block_ids.empty()) return 0;
    return int(t.block_ids.size() - 1) * cfg_.block_size + t.last_block_fill;
}

int64_t BlockManager::slot_of(int seq, int pos) const {
    if (!has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    if (pos < 0 || pos >= seq_len(seq)) return AF_ERR_OUT_OF_RANGE;
    const PageTable& t = tables_[size_t(seq)];
    return int64_t(t.block_ids[size_t(pos / cfg_.block_size)]) * cfg_.block_size +
           pos % cfg_.block_size;
}

int BlockManager::append_one(int seq, AppendSlot* out, std::vector<Undo>& undo) {
    PageTable& t = tables_[size_t(seq)];
    CowCopy cow;
    if (t.block_ids.empty() || t.last_block_fill == cfg_.block_size) {
        const int b = pop_free();
        if (b < 0) return AF_ERR_POOL_EXHAUSTED;
        undo.push_back({Undo::kAlloc, b, 0});
        undo.push_back({Undo::kPush, seq, t.last_block_fill});
        t.block_ids.push_back(b);
        t.last_block_fill = 0;
    } else if (ref_[size_t(t.block_ids.back())] > 1) {
        const int b = pop_free();
        if (b < 0) return AF_ERR_POOL_EXHAUSTED;
        const int old = t.block_ids.back();
        undo.push_back({Undo::kAlloc, b, 0});
        undo.push_back({Undo::kSwap, seq, old});
        --ref_[size_t(old)];
        t.block_ids.back() = b;
        cow.src = old;
        cow.dst = b;
        cow.rows = t.last_block_fill;
    }
    out->position = int(t.block_ids.size() - 1) * cfg_.block_size + t.last_block_fill;
    out->slot = int64_t(t.block_ids.back()) * cfg_.block_size + t.last_block_fill;
    out->cow = cow;
    undo.push_back({Undo::kFill, seq, t.last_block_fill});
    ++t.last_block_fill;
    return AF_OK;
}

void BlockManager::rollback(std::vector<Undo>& undo) {
    for (auto it = undo.rbegin(); it != undo.rend(); ++it) {
        switch (it->kind) {
            case Undo::kAlloc:
                ref_[size_t(it->a)] = 0;
                free_list_.push_back(it->a);
                break;
            case Undo::kPush: {
                PageTable& t = tables_[size_t(it->a)];
                t.block_ids.pop_back();
                t.last_block_fill = it->b;
                break;
            }
            case Undo::kSwap: {
                PageTable& t = tables_[size_t(it->a)];
                ++ref_[size_t(it->b)];
                t.block_ids.back() = it->b;
                break;
            }
            case Undo::kFill:
                tables_[size_t(it->a)].last_block_fill = it->b;
                break;
        }
    }
    undo.clear();
}

int BlockManager::append_token(int seq, AppendSlot* out) {
    if (!has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    if (!out) return AF_ERR_INVALID_ARG;
    std::vector<Undo> undo;
    const int st = append_one(seq, out, undo);
    if (st) rollback(undo);
    return st;
}

int BlockManager::extend(int seq, int n_tokens, int* first_pos, CowCopy* cow) {
    if (!has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    if (n_tokens < 0) return AF_ERR_INVALID_ARG;
    const int first = seq_len(seq);
    CowCopy c;
    std::vector<Undo> undo;
    for (int i = 0; i < n_tokens; ++i) {
        AppendSlot s;
        const int st = append_one(seq, &s, undo);
        if (st) {
            rollback(undo);
            return st;
        }
        if (s.cow.src >= 0) c = s.cow;
    }
    if (first_pos) *first_pos = first;
    if (cow) *cow = c;
    return AF_OK;
}

int BlockManager::plan_decode(const int* seqs, int n, AppendSlot* out) {
    if (n < 0 || (n > 0 && (!seqs || !out))) return AF_ERR_INVALID_ARG;
    for (int i = 0; i < n; ++i)
        if (!has_sequence(seqs[i])) return AF_ERR_BAD_SEQUENCE;
    std::vector<Undo> undo;
    for (int i = 0; i < n; ++i) {
        const int st = append_one(seqs[i], &out[i], undo);
        if (st) {
            rollback(undo);
            return st;
        }
    }
    return AF_OK;
}

}  // namespace atomflow::server

// ============================================================================
// C ABI
// ============================================================================
using atomflow::server::AppendSlot;
using atomflow::server::BlockManager;
using atomflow::server::CowCopy;
using atomflow::server::PoolConfig;

struct af_block_manager {
    BlockManager bm;
};

namespace atomflow::server {
BlockManager* block_manager_of(af_block_manager* h) { return h ? &h->bm : nullptr; }
}  // namespace atomflow::server

extern "C" int af_bm_create(int total_blocks, int block_size, int n_layers, int n_kv_heads,
                            int head_dim, int dtype, int allocate_pool, af_block_manager** out) {
    if (!out) return AF_ERR_INVALID_ARG;
    *out = nullptr;
    PoolConfig c;
    c.total_blocks = total_blocks;
    c.block_size = block_size;
    c.n_layers = n_layers;
    c.n_kv_heads = n_kv_heads;
    c.head_dim = head_dim;
    c.dtype = dtype;
    af_block_manager* h = new (std::nothrow) af_block_manager;
    if (!h) return AF_ERR_INVALID_ARG;
    try {
        h->bm.initialize(c, allocate_pool != 0);
    } catch (const std::invalid_argument&) {
        delete h;
        return AF_ERR_INVALID_ARG;
    } catch (const std::exception&) {
        delete h;
        return int(hipErrorOutOfMemory);
    }
    *out = h;
    return AF_OK;
}

extern "C" int af_bm_destroy(af_block_manager* bm) {
    delete bm;
    return AF_OK;
}

extern "C" int af_bm_attach_pool(af_block_manager* bm, void* base, const float* scales) {
    if (!bm) return AF_ERR_INVALID_ARG;
    bm->bm.attach_pool(base, scales);
    return AF_OK;
}

extern "C" int af_bm_pool(const af_block_manager* bm, af_kv_pool* out) {
    if (!bm || !out) return AF_ERR_INVALID_ARG;
    *out = bm->bm.pool_desc();
    return AF_OK;
}

extern "C" int af_bm_allocate_block(af_block_manager* bm) {
    return bm ? bm->bm.allocate_block() : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_free_block(af_block_manager* bm, int block_id) {
    return bm ? bm->bm.try_free_block(block_id) : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_num_free_blocks(const af_block_manager* bm) {
    return bm ? bm->bm.num_free_blocks() : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_ref_count(const af_block_manager* bm, int block_id) {
    return bm ? bm->bm.ref_count(block_id) : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_hold_copy_source(af_block_manager* bm, int block_id) {
    return bm ? bm->bm.hold_copy_source(block_id) : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_release_copy_sources(af_block_manager* bm) {
    if (!bm) return AF_ERR_INVALID_ARG;
    bm->bm.release_copy_sources();
    return AF_OK;
}
extern "C" int af_bm_seq_create(af_block_manager* bm) {
    return bm ? bm->bm.create_sequence() : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_seq_fork(af_block_manager* bm, int src_seq) {
    return bm ? bm->bm.fork_sequence(src_seq) : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_seq_free(af_block_manager* bm, int seq) {
    return bm ? bm->bm.free_sequence(seq) : AF_ERR_INVALID_ARG;
}
extern "C" int af_bm_seq_len(const af_block_manager* bm, int seq) {
    return bm ? bm->bm.seq_len(seq) : AF_ERR_INVALID_ARG;
}

extern "C" int af_bm_seq_table(const af_block_manager* bm, int seq, int32_t* ids, int max_ids,
                               int32_t* last_block_fill) {
    if (!bm || max_ids < 0 || (max_ids > 0 && !ids)) return AF_ERR_INVALID_ARG;
    if (!bm->bm.has_sequence(seq)) return AF_ERR_BAD_SEQUENCE;
    const auto& t = bm->bm.table(seq);
    const int n = int(t.block_ids.size());
    for (int i = 0; i < n && i < max_ids; ++i) ids[i] = t.block_ids[size_t(i)];
    if (last_block_fill) *last_block_fill = t.last_block_fill;
    return n;
}

extern "C" int af_bm_seq_append(af_block_manager* bm, int seq, int64_t* slot, int32_t* cow_src,
                                int32_t* cow_dst, int32_t* cow_rows) {
    if (!bm) return AF_ERR_INVALID_ARG;
    AppendSlot s;
    const int st = bm->bm.append_token(seq, &s);
    if (st) return st;
    if (slot) *slot = s.slot;
    if (cow_src) *cow_src = s.cow.src;
    if (cow_dst) *cow_dst = s.cow.dst;
    if (cow_rows) *cow_rows = s.cow.rows;
    return s.position;
}

extern "C" int af_bm_seq_extend(af_block_manager* bm, int seq, int n_tokens, int32_t* cow_src,
                                int32_t* cow_dst, int32_t* cow_rows) {
    if (!bm) return AF_ERR_INVALID_ARG;
    int first = 0;
    CowCopy c;
    const int st = bm->bm.extend(seq, n_tokens, &first, &c);
    if (st) return st;
    if (cow_src) *cow_src = c.src;
    if (cow_dst) *cow_dst = c.dst;
    if (cow_rows) *cow_rows = c.rows;
    return first;
}

extern "C" int64_t af_bm_seq_slot(const af_block_manager* bm, int seq, int pos) {
    return bm ? bm->bm.slot_of(seq, pos) : int64_t(AF_ERR_INVALID_ARG);
}

extern "C" int af_bm_plan_decode(af_block_manager* bm, const int32_t* seqs, int n, int64_t* slots,
                                 int32_t* positions, int32_t* copies, int max_copies,
                                 int32_t* n_copies) {
    if (!bm || n < 0 || (n > 0 && (!seqs || !slots || !positions)) || !n_copies || max_copies < 0 ||
        (max_copies > 0 && !copies))
        return AF_ERR_INVALID_ARG;
    std::vector<int> s(seqs, seqs + n);
    std::vector<AppendSlot> out(size_t(n > 0 ? n : 0));
    const int st = bm->bm.plan_decode(s.data(), n, out.data());
    if (st) return st;
    int nc = 0;
    for (int i = 0; i < n; ++i) {
        slots[i] = out[size_t(i)].slot;
        positions[i] = out[size_t(i)].position;
        if (out[size_t(i)].cow.src >= 0) {
            if (nc < max_copies) {
                copies[3 * nc] = out[size_t(i)].cow.src;
                copies[3 * nc + 1] = out[size_t(i)].cow.dst;
                copies[3 * nc + 2] = out[size_t(i)].cow.rows;
            }
            ++nc;
        }
    }
    *n_copies = nc;
    return nc > max_copies ? AF_ERR_OUT_OF_RANGE : AF_OK;
}

extern "C" int af_bm_export_tables(const af_block_manager* bm, const int32_t* seqs, int n,
                                   int32_t* tables, int max_blocks, int32_t* seq_lens) {
    if (!bm || n < 0 || max_blocks <= 0 || (n > 0 && (!seqs || !tables))) return AF_ERR_INVALID_ARG;
    for (int i = 0; i < n; ++i)
        if (!bm->bm.has_sequence(seqs[i])) return AF_ERR_BAD_SEQUENCE;
    for (int i = 0; i < n; ++i) {
        const auto& t = bm->bm.table(seqs[i]);
        if (int(t.block_ids.size()) > max_blocks) return AF_ERR_OUT_OF_RANGE;
        int32_t* row = tables + size_t(i) * max_blocks;
        int k = 0;
        for (; k < int(t.block_ids.size()); ++k) row[k] = t.block_ids[size_t(k)];
        for (; k < max_blocks; ++k) row[k] = 0;
        if (seq_lens) seq_lens[i] = bm->bm.seq_len(seqs[i]);
    }
    return AF_OK;
}
