#pragma once
// Paged KV-cache block management.
//
// Fills in the reference's declaration-only contract
// (src/experimental/server_arch/paged_kv_manager.h:26-121; the reference's
// include/memory/block_manager.h is an empty struct): KVBlock, PageTable and a
// BlockManager with one pool allocation at initialize(), a stack free list,
// allocate_block() -> id or -1, free_block(id), num_free_blocks(). Extended with
// reference counts, sequences (PageTables owned by the manager), fork and
// copy-on-write append planning. Host-side bookkeeping only; device copies and
// KV writes are issued by the caller through af_kv_copy_blocks /
// af_paged_rope_append. Not thread-safe.
//
// Rules (the reference leaves them open; fixed here and mirrored op for op by
// the test model):
//  * a fresh pool hands out ids 0, 1, 2, ...; a freed id is reused first (LIFO);
//  * a block id spans every layer: layer l's rows of block b live at
//    pool + ((2l + {0 K, 1 V}) * total_blocks + b) * block_size * kv_dim elements;
//  * free_block drops one reference, the id returns to the stack at zero;
//  * append: full or missing tail -> new block; partial tail with ref > 1 ->
//    copy-on-write (new block, copy `fill` rows, old tail loses a reference);
//    otherwise write in place; a failed append / extend / plan changes nothing;
//  * a copy source can be held (hold_copy_source) until the copies that read it
//    have been issued: a held block whose last reference is freed stays off the
//    free list until release_copy_sources(), so no later allocation in the same
//    plan hands it out as a destination while a planned copy still reads it.
//    Holds do not count as references (the copy-on-write test is unchanged).
#include <cstdint>
#include <stdexcept>
#include <vector>

#include "af_kv.h"

namespace atomflow::server {

// Tokens per block of the reference sandbox (paged_kv_manager.h:34).
static constexpr int BLOCK_SIZE = 16;

// One block of one layer (paged_kv_manager.h:47-52). Pointers are device
// addresses of [block_size, kv_dim] rows; element type per the pool dtype.
struct KVBlock {
    int block_id = -1;
    void* k_data = nullptr;
    void* v_data = nullptr;
    int ref_count = 0;
};

// Logical -> physical mapping of one sequence (paged_kv_manager.h:68-76).
struct PageTable {
    std::vector<int> block_ids;
    int last_block_fill = 0;
};

struct CowCopy {
    int src = -1;
    int dst = -1;
    int rows = 0;
};

struct AppendSlot {
    int position = -1;  // logical index of the new token
    int64_t slot = -1;  // physical row: block * block_size + offset
    CowCopy cow;
};

struct PoolConfig {
    int total_blocks = 0;
    int block_size = BLOCK_SIZE;
    int n_layers = 0;
    int n_kv_heads = 0;
    int head_dim = 0;
    int dtype = AF_KV_FP16;
};

class BlockManager {
public:
    BlockManager() = default;
    ~BlockManager();
    BlockManager(const BlockManager&) = delete;
    BlockManager& operator=(const BlockManager&) = delete;

    // Reference signature (paged_kv_manager.h:103): BLOCK_SIZE-token fp16 blocks,
    // kv_dim split into 128-wide heads, one hipMalloc for the pool. Throws
    // std::runtime_error when the allocation fails.
    void initialize(int total_blocks, int kv_dim, int n_layers);
    // General form. allocate_pool: one hipMalloc owned by the manager; otherwise
    // `pool` (may be null for bookkeeping-only use) is borrowed.
    void initialize(const PoolConfig& cfg, bool allocate_pool, void* pool = nullptr,
                    const float* scales = nullptr);
    void attach_pool(void* pool, const float* scales);

    // Reference contract (paged_kv_manager.h:105-115).
    int allocate_block();          // id, or -1 when the pool is exhausted
    void free_block(int block_id); // throws std::invalid_argument on a free / bad id
    int num_free_blocks() const { return int(free_list_.size()); }

    // Extensions. Status-returning forms use the af_kv.h AF_* codes.
    int try_free_block(int block_id);
    int ref_count(int block_id) const;  // AF_ERR_BAD_BLOCK when out of range
    KVBlock block(int block_id, int layer) const;
    af_kv_pool pool_desc() const;
    const PoolConfig& config() const { return cfg_; }

    int create_sequence();
    int fork_sequence(int src);  // id or AF_ERR_BAD_SEQUENCE
    int free_sequence(int seq);
    bool has_sequence(int seq) const;
    const PageTable& table(int seq) const;  // throws std::out_of_range
    int seq_len(int seq) const;             // tokens, or AF_ERR_BAD_SEQUENCE
    int64_t slot_of(int seq, int pos) const;

    // Copy-source holds (see the rules above). hold: AF_ERR_BAD_BLOCK unless the
    // block is referenced. release: holds drop in the order they were taken; a
    // block with no references left returns to the free list then.
    int hold_copy_source(int block_id);
    void release_copy_sources();
    int num_held_blocks() const { return int(holds_.size()); }

    int append_token(int seq, AppendSlot* out);
    int extend(int seq, int n_tokens, int* first_pos, CowCopy* cow);
    int plan_decode(const int* seqs, int n, AppendSlot* out);

private:
    struct Undo {
        enum Kind { kAlloc, kPush, kSwap, kFill } kind;
        int a;
        int b;
    };
    int append_one(int seq, AppendSlot* out, std::vector<Undo>& undo);
    void rollback(std::vector<Undo>& undo);
    int pop_free();

    PoolConfig cfg_;
    std::vector<int> ref_;
    std::vector<int> free_list_;  // stack: back() is handed out next
    std::vector<int> held_;       // per block: outstanding copy-source holds
    std::vector<int> holds_;      // held block ids, in the order taken
    std::vector<PageTable> tables_;
    std::vector<uint8_t> live_;
    void* pool_ = nullptr;
    const float* scales_ = nullptr;
    bool owns_pool_ = false;
};

}  // namespace atomflow::server
