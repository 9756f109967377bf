#pragma once
// ArenaAllocator: one device allocation, 128-B aligned bump allocation.
// Reference: include/memory/alloc.h:17-29,49-61 — same methods and semantics
// (allocate() throws std::runtime_error when the arena is full,
// reset_workspace() rewinds). Where the reference calls std::exit on a failed
// cudaMalloc (alloc.h:59), the constructor here throws, so a host process can
// report the failure. Sized for a 288 GB HBM3E device: offsets are size_t.
// A second constructor borrows caller-owned memory (a slice of a larger
// allocation, or host memory): it allocates and frees nothing.
#include <cstddef>
#include <stdexcept>

class ArenaAllocator {
public:
    // One hipMalloc of total_size rounded up to 128 B; throws std::runtime_error
    // when the allocation fails.
    explicit ArenaAllocator(size_t total_size);
    // Borrows [base, base + capacity); base must be 128-B aligned.
    ArenaAllocator(void* base, size_t capacity) : base_ptr_(base), capacity_(capacity) {
        if (reinterpret_cast<size_t>(base) & 127)
            throw std::invalid_argument("ArenaAllocator: borrowed base is not 128-B aligned");
    }
    ~ArenaAllocator();
    ArenaAllocator(const ArenaAllocator&) = delete;
    ArenaAllocator& operator=(const ArenaAllocator&) = delete;

    void* allocate(size_t size) {
        size = align_to_128(size);
        if (offset_ + size > capacity_)
            throw std::runtime_error("ArenaAllocator: out of memory! Check max_seq_len.");
        void* ptr = static_cast<char*>(base_ptr_) + offset_;
        offset_ += size;
        return ptr;
    }
    void reset_workspace(size_t new_offset) { offset_ = new_offset; }
    size_t get_capacity() const { return capacity_; }
    size_t get_offset() const { return offset_; }
    void* base() const { return base_ptr_; }

private:
    static constexpr size_t align_to_128(size_t size) { return (size + 127) & ~size_t(127); }
    void* base_ptr_ = nullptr;
    size_t offset_ = 0;
    size_t capacity_ = 0;
    bool owns_ = false;
};
